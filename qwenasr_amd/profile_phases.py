"""Phase breakdown of the fused RMSNorm + qkv + attention launch (the decode
step's dominant kernel), from the profiling build's real-time stamps.

    make -C qwenasr_amd/csrc stamps          # builds qwenasr_amd/libqasr_hip_stamps.so
    python -m qwenasr_amd.profile_phases [steps] [ctx]

Loads the seeded 0.6B decoder of the headline workload (bench.py, seed 1002)
into libqasr_hip_stamps.so (the library's sources compiled with QASR_STAMPS),
prefills a `ctx`-row synthetic prompt (494: the context where bench.py's
per-kernel timing starts), and runs `steps` graph-replayed decode steps.  In
every layer's fused launch, lane 0 of one wave per block writes the 100 MHz
real-time counter (10 ns ticks) at the boundaries below; the step's stamps
are read back after each step.

  qkv matvec blocks (wave 0): 0 entry, 1 loads issued, 2 activation in
  registers (the previous launch's residual arrived), 3 RMSNorm + int8
  quantization done, 4 dots + reduce-scatter done (the weights arrived),
  5 tagged rows stored;
  attention blocks (wave 0): 0 entry, 1 K/V loads issued, 2 q/k/v handed over
  by the polling wave, 3 scores, 4 softmax, 5 P V, 6 block merge in LDS,
  7 partial stored; (polling wave) 8 every tag matched.

Per launch, times are taken from the launch's first block entry; a phase's
"last" is its latest stamp over the launch's blocks, "per block" the median
duration inside a block.  Reported as medians over layers 1-27 and the steps
(layer 0 gathers the embedding row instead of reading the residual).
"""
import os
import sys

import numpy as np

from . import _lib

STAMP_SLOTS = 16
TICK_US = 0.01          # s_memrealtime: 100 MHz


def main(steps=20, ctx=494):
    stamps_lib = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqasr_hip_stamps.so")
    if not os.path.exists(stamps_lib):
        raise SystemExit(f"{stamps_lib} is missing: build it with `make -C qwenasr_amd/csrc stamps`")
    _lib.LIB_PATH = stamps_lib
    from . import Device
    from ._lib import check, lib
    from .model import Decoder
    from .synth import DEC_0_6B, SynthDecoder
    cfg = DEC_0_6B
    w = SynthDecoder(cfg, seed=1002)
    dev = Device(0)
    dec = Decoder(dev, w, max_seq=1024)
    nqkv = (cfg["n_heads"] + 2 * cfg["n_kv_heads"]) * cfg["head_dim"]
    n_mv = nqkv // 16
    max_blocks = n_mv + 2 * cfg["n_kv_heads"] * 64
    L = cfg["n_layers"]
    nbytes = L * max_blocks * STAMP_SLOTS * 8
    buf = dev.zeros(nbytes, np.uint8)
    check(lib().qasr_hip_decoder_set_stamps(dec.d, buf.ptr, nbytes))
    print("[profile_phases] decoder loaded (profiling build)", flush=True)
    rng = np.random.default_rng(1002)
    prompt = (rng.standard_normal((ctx, cfg["hidden"])) * 0.5).astype(np.float32)
    dec.prefill(prompt)
    tok = int(dec.generate(1, first_embed=prompt[-1])[0])
    mv_rows, at_rows = [], []
    for s in range(steps):
        pos = dec.kv_len
        buf.copy_from(np.zeros(nbytes, np.uint8))
        dev.sync()
        tok = int(dec.generate(1, first_token=tok)[0])
        raw = buf.numpy().view(np.uint64)
        # this step's bucket: 8 splits up to 1024 positions -> 16 x 8 attention blocks
        cap = min(max(((pos + 1 + 255) // 256) * 256, 256), 1024)
        n_split = 8 if cap <= 1024 else 16
        grid = n_mv + 2 * cfg["n_kv_heads"] * n_split
        st = raw[:L * grid * STAMP_SLOTS].reshape(L, grid, STAMP_SLOTS).astype(np.int64)
        for l in range(1, L):
            t0 = st[l, :, 0].min()
            mv = st[l, :n_mv, :6] - t0
            at = st[l, n_mv:, :9] - t0
            mv_rows.append(mv)
            at_rows.append(at)
        print(f"[profile_phases] step {s + 1}/{steps} at context {pos}", flush=True)
    mv = np.stack(mv_rows) * TICK_US          # [launches][blocks][phase] us from launch start
    at = np.stack(at_rows) * TICK_US
    med = lambda a: float(np.median(a))
    print(f"\nfused launch phases, context {ctx}..{ctx + steps}, {mv.shape[0]} launches (layers 1-27), "
          f"us from the launch's first block entry (medians over launches)")
    print("| block kind | phase | first | median block | last | per block (from previous phase) |")
    print("|---|---|---|---|---|---|")
    names_mv = ["entry", "loads issued", "activation in registers", "RMSNorm + quantization",
                "dots + reduce-scatter", "rows published"]
    for k, n in enumerate(names_mv):
        per = med(mv[:, :, k] - mv[:, :, k - 1]) if k else float("nan")
        print(f"| qkv matvec ({n_mv}) | {k} {n} | {med(mv[:, :, k].min(1)):.2f} | {med(np.median(mv[:, :, k], 1)):.2f} "
              f"| {med(mv[:, :, k].max(1)):.2f} | {per:.2f} |")
    names_at = ["entry", "K/V loads issued", "q/k/v handed over", "scores", "softmax", "P V", "block merge",
                "partial stored"]
    for k, n in enumerate(names_at):
        per = med(at[:, :, k] - at[:, :, k - 1]) if k else float("nan")
        print(f"| attention ({at.shape[1]}) | {k} {n} | {med(at[:, :, k].min(1)):.2f} | "
              f"{med(np.median(at[:, :, k], 1)):.2f} | {med(at[:, :, k].max(1)):.2f} | {per:.2f} |")
    per = med(at[:, :, 8] - at[:, :, 0])
    print(f"| attention poll wave | 8 tags matched | {med(at[:, :, 8].min(1)):.2f} | "
          f"{med(np.median(at[:, :, 8], 1)):.2f} | {med(at[:, :, 8].max(1)):.2f} | {per:.2f} (from entry) |")
    print(f"\nlaunch span (first entry -> last partial stored): {med(at[:, :, 7].max(1)):.2f} us; "
          f"qkv rows published by {med(mv[:, :, 5].max(1)):.2f} us; "
          f"last attention block entered at {med(at[:, :, 0].max(1)):.2f} us")
    check(lib().qasr_hip_decoder_set_stamps(dec.d, None, 0))
    dec.close()
    dev.close()


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 20, int(sys.argv[2]) if len(sys.argv) > 2 else 494)
