"""Multi-stream decode driver for rocprofv3 runs.

    QASR_DISABLE_GRAPH=1 rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- \\
        python3 -u -m qwenasr_amd.profile_batch [steps] [calib_mib] [n_streams]
    QASR_DISABLE_GRAPH=1 rocprofv3 --pmc FETCH_SIZE --kernel-include-regex '_batch|k_quant_rows|k_qk_prep|k_attn|k_embed|k_copy' \\
        --output-format csv -d <dir> -o run -- python3 -u -m qwenasr_amd.profile_batch [steps] [calib_mib] [n_streams]

The config-4 workload of ``bench_configs config4`` (the seeded 0.6B decoder,
32 streams with prefixes of U[100, 1500] positions prefilled from N(0,1)
embeddings, seed 1004) reduced to what a profiler needs: `steps` batched
greedy steps, one call per step with a progress line each (a counter run
serialises every dispatch), no graph capture (QASR_DISABLE_GRAPH=1), no
solo-stream comparison, then one device copy of `calib_mib` MiB with the
library's copy kernel, whose counter reading calibrates the others
(``python -m qwenasr_amd.rocprof_summary --pmc``).
"""
import sys

import numpy as np

from . import Device
from .model import Batch, Decoder
from .synth import DEC_0_6B, SynthDecoder


def main(steps=8, calib_mib=64, n_streams=32):
    cfg = dict(DEC_0_6B)
    w = SynthDecoder(cfg, seed=1004)
    rng = np.random.default_rng(1004)
    lens = rng.integers(100, 1501, n_streams)
    first = rng.integers(0, cfg["vocab"], n_streams)
    dev = Device(0)
    dec = Decoder(dev, w, max_seq=2048)
    bat = Batch(dec, n_streams, 2048, max_steps=1)
    print("[profile_batch] decoder and batch ready", flush=True)
    for i, L in enumerate(lens):
        bat.prefill(i, rng.standard_normal((int(L), cfg["hidden"]), dtype=np.float32))
    dev.sync()
    print(f"[profile_batch] {n_streams} prefixes prefilled ({int(lens.sum())} positions)", flush=True)
    tok = np.asarray(first, np.int32)
    for s in range(steps):
        tok = bat.generate(tok, 1)[:, 0].astype(np.int32)
        print(f"[profile_batch] step {s + 1}/{steps}, stream 0 token {int(tok[0])}", flush=True)
    nb = calib_mib << 20
    a, b = dev.empty(nb, np.uint8), dev.empty(nb, np.uint8)
    dev.copy(b, a)
    dev.sync()
    print(f"[profile_batch] calibration copy {calib_mib} MiB done", flush=True)
    bat.close()
    dec.close()
    dev.close()


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 8, int(sys.argv[2]) if len(sys.argv) > 2 else 64,
         int(sys.argv[3]) if len(sys.argv) > 3 else 32)
