"""BASELINE config 2 at full size through the C ABI: random-init
Qwen3-ASR-0.6B (28-layer int8 decoder, 18-layer encoder), 30 s of synthetic
audio, mel -> encoder -> 404-row prefill -> 200 forced greedy steps
(transcribe.rs:63-247).

- the 200 token ids equal the committed oracle fixture
  (tests/golden/config2_tokens.json, written by make_config2_tokens.py);
- the random-init model settles on one token id, so the token check alone is
  weak: the whole KV cache after the run (every layer, all 604 positions) is
  compared with the oracle's, computed here on the host from the same seeded
  model and audio:
  * the 404 prefill rows of every layer within 1e-5 (f32-class MFMA GEMMs and
    attention against the oracle's f32 sgemm; measured 1e-6);
  * layer 0's 200 decode rows within 1e-5 (identical token embeddings through
    the exact int8 path);
  * deeper decode rows within 5e-2: every decode step re-quantizes its
    activations to int8, so an ulp-level difference can move an element
    across a rounding boundary.  The oracle against itself with its prompt
    rows perturbed by 1e-6 (relative) moves these rows by 0.7-2.1% at layers
    1-27 while its prefill rows move by 1e-6 and its 200 tokens do not change;
    a wrong row, position or layer gives errors of order 1.
"""
import json
import os

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_config2_full_size(dev):
    from oracle import oracle as orc
    from qwenasr_amd.model import Decoder, Encoder, transcribe_forced
    from qwenasr_amd.synth import DEC_0_6B, ENC_0_6B, SynthDecoder, SynthEncoder, audio
    with open(os.path.join(ROOT, "tests", "golden", "config2_tokens.json")) as f:
        golden = json.load(f)
    wd = SynthDecoder(DEC_0_6B, seed=1002)
    we = SynthEncoder(ENC_0_6B, seed=1002)
    x = audio(480000, 1002)
    print("config 2 full size: GPU transcription", flush=True)
    dec = Decoder(dev, wd, max_seq=1024)
    enc = Encoder(dev, we)
    try:
        toks, _ = transcribe_forced(dec, enc, x, 200)
        assert [int(t) for t in toks] == golden["tokens"]
        k_g, v_g = dec.kv_download()
        n = dec.kv_len
    finally:
        dec.close()
        enc.close()
    assert n == golden["prompt_len"] - 1 + 200
    print("config 2 full size: oracle transcription on the host", flush=True)
    orc.set_threads(min(16, os.cpu_count() or 1))
    od, oe = orc.OracleDecoder(wd, max_seq=1024), orc.OracleEncoder(we)
    try:
        res = orc.transcribe_forced(od, oe, x, 200)
        assert [int(t) for t in res["tokens"]] == golden["tokens"]
        k_c, v_c = od.kv()
    finally:
        od.close()
        oe.close()
    P = golden["prompt_len"] - 1                       # prefill rows; decode rows [P, n)
    pre = [max(rel(k_g[l, :, :P], k_c[l, :, :P]), rel(v_g[l, :, :P], v_c[l, :, :P])) for l in range(28)]
    dec = [max(rel(k_g[l, :, P:n], k_c[l, :, P:n]), rel(v_g[l, :, P:n], v_c[l, :, P:n])) for l in range(28)]
    print("per-layer KV relative error, prefill rows:", [f"{e:.2e}" for e in pre], flush=True)
    print("per-layer KV relative error, decode rows:", [f"{e:.2e}" for e in dec], flush=True)
    assert max(pre) < 1e-5, pre
    assert dec[0] < 1e-5, dec[0]
    assert max(dec) < 5e-2, dec
