"""The C ABI driven from a C program (tests/c_abi_smoke.c, built with gcc as
C99): its decode tokens and aligner argmax must equal what the Python binding
and the oracle produce on the same seeded model and inputs, so the C-side
struct layouts, status codes and host-buffer contracts are the ones the
library implements."""
import os
import subprocess

import numpy as np
import pytest

from test_abi import build_c_smoke

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
           vocab=4096, eps=1e-6, theta=1e6)


def test_c_program_matches_python_and_oracle(dev, orc, tmp_path):
    from qwenasr_amd.model import Decoder
    from qwenasr_amd.synth import SynthDecoder, normal_f32
    seed = 1007
    exe = build_c_smoke(tmp_path)
    print("running the C smoke program", flush=True)
    r = subprocess.run([exe, str(seed)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.stdout, r.stderr)
    lines = dict(l.split(":", 1) for l in r.stdout.strip().splitlines() if ":" in l)
    assert r.stdout.strip().endswith("ok")
    c_tokens = [int(t) for t in lines["tokens"].split()]
    c_argmax = [int(t) for t in lines["argmax"].split()]

    w = SynthDecoder(CFG, seed=seed)
    emb = normal_f32((20, CFG["hidden"]), seed, "c_abi_smoke.prefill", std=0.02)
    gpu = Decoder(dev, w, max_seq=128)
    cpu = orc.OracleDecoder(w, max_seq=128)
    try:
        gpu.prefill(emb)
        cpu.prefill(emb)
        tok, py_tokens, or_tokens = 11, [], []
        for _ in range(8):
            tok = gpu.forward(token=tok)
            py_tokens.append(tok)
        tok = 11
        for _ in range(8):
            tok, _ = cpu.forward(cpu.embed(tok))
            or_tokens.append(tok)
        assert c_tokens == py_tokens == or_tokens, (c_tokens, py_tokens, or_tokens)
        gpu.kv_len = 0
        py_argmax = gpu.prefill_argmax(emb, np.array([0, 7, 19], np.int32)).tolist()
        assert c_argmax == py_argmax
    finally:
        gpu.close()
        cpu.close()
