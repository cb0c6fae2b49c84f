"""Phase breakdown of the decode step's per-layer launches, from the profiling
build's real-time stamps.

    make -C qwenasr_amd/csrc stamps          # builds qwenasr_amd/libqasr_hip_stamps.so
    python -m qwenasr_amd.profile_phases [steps] [ctx]

Loads the seeded 0.6B decoder of the headline workload (bench.py, seed 1002)
into libqasr_hip_stamps.so (the library's sources compiled with QASR_STAMPS),
prefills a `ctx`-row synthetic prompt (494: the context where bench.py's
per-kernel timing starts), and runs `steps` graph-replayed decode steps.  In
every layer's fused RMSNorm + qkv + attention, o_proj, gate_up and down
launches, lane 0 of one wave per block writes the 100 MHz real-time counter
(10 ns ticks) at the phase boundaries named below; the stamps are read back
after each step.

Per launch, times are taken from the launch's first block entry; for each
phase the table gives its first, median and last stamp over the launch's
blocks and the median time a block spends in it (from the previous phase).
Medians over layers 1-27 and the steps (layer 0's qkv gathers the embedding
row instead of reading the residual).  A phase ends when its last instruction
issues: a wait for memory shows up in the phase whose first instruction uses
the loaded value (the activation of a matvec arrives inside "RMSNorm +
quantization", not at "activation converted", which only renames registers).
"""
import os
import sys

import numpy as np

from . import _lib

STAMP_SLOTS = 16
STAMP_BLOCKS = 2048
TICK_US = 0.01          # s_memrealtime: 100 MHz

MV_PHASES = ["entry", "loads issued", "activation converted", "activation arrived + RMSNorm + quantization",
             "dots + reduce-scatter", "rows stored"]
KINDS = [
    ("qkv matvec blocks of the fused launch", MV_PHASES[:5] + ["tagged rows published"]),
    ("o_proj (split merge in its prologue)", ["entry", "loads issued", "merge weights (exp, LDS)",
                                             "merged attention in LDS", "quantization", "dots + reduce-scatter",
                                             "rows stored"]),
    ("gate_up + SwiGLU", MV_PHASES[:4] + ["dots + reduce-scatter", "SwiGLU rows stored"]),
    ("down", MV_PHASES[:3] + ["activation arrived + quantization", "dots + reduce-scatter", "rows stored"]),
]
ATT_PHASES = ["entry", "K/V loads issued", "q/k/v handed over", "scores", "softmax", "P V", "block merge",
              "partial stored"]


def table(title, st, names):
    """st: [launches][blocks][phases] us from the launch's first entry."""
    med = lambda a: float(np.median(a))
    print(f"\n{title}: {st.shape[1]} blocks, {st.shape[0]} launches")
    print("| phase | first | median block | last | per block |")
    print("|---|---|---|---|---|")
    for k, n in enumerate(names):
        per = f"{med(st[:, :, k] - st[:, :, k - 1]):.2f}" if k else ""
        print(f"| {k} {n} | {med(st[:, :, k].min(1)):.2f} | {med(np.median(st[:, :, k], 1)):.2f} | "
              f"{med(st[:, :, k].max(1)):.2f} | {per} |")


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
    H, I, L = cfg["hidden"], cfg["intermediate"], cfg["n_layers"]
    nqkv = (cfg["n_heads"] + 2 * cfg["n_kv_heads"]) * cfg["head_dim"]
    n_mv = nqkv // 16                                   # 4 rows per wave, 4 waves per block
    blocks = [None, H // 8, 2 * I // 32, H // 4]        # o_proj 2 rows/wave, gate_up 8, down 1
    nbytes = 4 * L * STAMP_BLOCKS * STAMP_SLOTS * 8
    buf = dev.zeros(nbytes, np.uint8)
    check(lib().qasr_hip_decoder_set_stamps(dec.d, buf.ptr, nbytes))
    print("[profile_phases] decoder loaded (profiling build)", flush=True)
    rng = np.random.default_rng(1002)
    prompt = (rng.standard_normal((ctx, H)) * 0.5).astype(np.float32)
    dec.prefill(prompt)
    tok = int(dec.generate(1, first_embed=prompt[-1])[0])
    rows = {k: [] for k in range(4)}
    att_rows = []
    spans = {k: [] for k in range(4)}
    for s in range(steps):
        pos = dec.kv_len
        buf.copy_from(np.zeros(nbytes, np.uint8))
        dev.sync()
        tok = int(dec.generate(1, first_token=tok)[0])
        raw = buf.numpy().view(np.uint64).reshape(4, L, STAMP_BLOCKS, STAMP_SLOTS).astype(np.int64)
        # this step's bucket: 8 splits up to 1024 positions -> 16 x 8 attention blocks
        cap = min(max(((pos + 1 + 255) // 256) * 256, 256), 1024)
        n_att = 2 * cfg["n_kv_heads"] * (8 if cap <= 1024 else 16)
        for l in range(1, L):
            fused = raw[0, l, :n_mv + n_att]
            t0 = fused[:, 0].min()
            rows[0].append(fused[:n_mv, :6] - t0)
            att_rows.append(fused[n_mv:, :9] - t0)
            spans[0].append(fused[n_mv:, 7].max() - t0)
            for k in (1, 2, 3):
                b = raw[k, l, :blocks[k]]
                t0 = b[:, 0].min()
                n = len(KINDS[k][1])
                rows[k].append(b[:, :n] - t0)
                spans[k].append(b[:, n - 1].max() - t0)
        print(f"[profile_phases] step {s + 1}/{steps} at context {pos}", flush=True)
    print(f"\nphase stamps, 0.6B decode, context {ctx}..{ctx + steps}, us from each launch's first block "
          f"entry (medians over layers 1-27 x {steps} steps)")
    for k in range(4):
        table(KINDS[k][0], np.stack(rows[k]) * TICK_US, KINDS[k][1])
        if k == 0:
            at = np.stack(att_rows) * TICK_US
            table("attention blocks of the fused launch", at[:, :, :8], ATT_PHASES)
            print(f"| (polling wave) tags matched | {np.median(at[:, :, 8].min(1)):.2f} | "
                  f"{np.median(np.median(at[:, :, 8], 1)):.2f} | {np.median(at[:, :, 8].max(1)):.2f} | |")
    print("\nspan from the first block entry to the last block's final stamp (us): " +
          ", ".join(f"{KINDS[k][0].split(' (')[0]} {np.median(spans[k]) * TICK_US:.2f}" for k in range(4)))
    check(lib().qasr_hip_decoder_set_stamps(dec.d, None, 0))
    dec.close()
    dev.close()


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 20, int(sys.argv[2]) if len(sys.argv) > 2 else 494)
