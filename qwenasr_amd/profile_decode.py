"""Decode-only driver for hardware-counter runs (``rocprofv3 --pmc``).

    QASR_DISABLE_GRAPH=1 rocprofv3 --pmc FETCH_SIZE --kernel-include-regex 'k_qkv_attn|k_attn|k_w8a8|k_oproj|k_argmax|k_copy' \\
        --output-format csv -d <dir> -o run -- python3 -m qwenasr_amd.profile_decode [steps] [calib_mib]

Loads the seeded 0.6B decoder of the headline workload (bench.py, seed 1002),
prefills a `ctx`-row synthetic prompt (494 = the context where bench.py's
per-kernel timing starts: the 404-row config-2 prompt + 90 steps), runs `steps`
greedy decode steps one call at a time, printing each (kernel by kernel when
QASR_DISABLE_GRAPH=1, so the profiler sees every dispatch; a counter run
serialises every dispatch) and finally one device copy of `calib_mib` MiB
with the library's copy kernel, whose counter reading calibrates the others
(``python -m qwenasr_amd.rocprof_summary --pmc``).

With a fourth argument ``1.7b`` it runs config 3's decoder instead: the
seeded Qwen3-1.7B-sized decoder (28 layers, hidden 2048, bf16 KV cache, seed
1003 as bench_configs.config3), its whole KV cache filled with N(0,1) values
and the context set to `ctx` rows (512, 2048 or 4096 in config 3).
"""
import sys

import numpy as np

from . import Device
from .model import Decoder
from .synth import DEC_0_6B, DEC_1_7B, SynthDecoder


def main(steps=20, calib_mib=64, ctx=494, model="0.6b"):
    dev = Device(0)
    if model == "1.7b":
        w = SynthDecoder(DEC_1_7B, seed=1003)
        dec = Decoder(dev, w, max_seq=ctx + steps + 8, kv_bf16=True)
        print("[profile_decode] 1.7B decoder loaded", flush=True)
        rng = np.random.default_rng(1003)
        shape = dec.kv_shape()
        dec.kv_upload(rng.standard_normal(shape, dtype=np.float32), rng.standard_normal(shape, dtype=np.float32))
        dec.kv_len = ctx
        print(f"[profile_decode] bf16 KV filled with N(0,1), context {ctx}", flush=True)
        tok = int(dec.generate(1, first_token=17)[0])
    else:
        w = SynthDecoder(DEC_0_6B, seed=1002)
        dec = Decoder(dev, w, max_seq=1024)
        print("[profile_decode] decoder loaded", flush=True)
        rng = np.random.default_rng(1002)
        prompt = (rng.standard_normal((ctx, DEC_0_6B["hidden"])) * 0.5).astype(np.float32)
        dec.prefill(prompt)
        print("[profile_decode] prompt prefilled", flush=True)
        # one step per call so that a counter run (every dispatch serialised) reports progress
        tok = int(dec.generate(1, first_embed=prompt[-1])[0])
    for s in range(1, steps):
        tok = int(dec.generate(1, first_token=tok)[0])
        print(f"[profile_decode] step {s + 1}/{steps} at context {ctx + s}, token {tok}", flush=True)
    nb = calib_mib << 20
    a, b = dev.empty(nb, np.uint8), dev.empty(nb, np.uint8)
    dev.copy(b, a)
    dev.sync()
    print(f"[profile_decode] calibration copy {calib_mib} MiB done", flush=True)
    dec.close()
    dev.close()


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 20, int(sys.argv[2]) if len(sys.argv) > 2 else 64,
         int(sys.argv[3]) if len(sys.argv) > 3 else 494, sys.argv[4] if len(sys.argv) > 4 else "0.6b")
