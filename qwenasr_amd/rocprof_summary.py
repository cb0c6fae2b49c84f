"""Summarise a rocprofv3 kernel trace (``--kernel-trace --output-format csv``).

    python -m qwenasr_amd.rocprof_summary <dir>/run_kernel_trace.csv [min_batch]
    python -m qwenasr_amd.rocprof_summary --pmc <dir>/run_counter_collection.csv <calib MiB>
    python -m qwenasr_amd.rocprof_summary --traffic <fetch csv> <write csv> <calib MiB> > profiles/hbm_traffic.txt
    python -m qwenasr_amd.rocprof_summary --mfma-config1 <MfmaUtil csv> <MOPS csv> [reps [<FETCH csv> <WRITE csv> <calib MiB>]]

The second form averages each kernel's counter values (``--pmc FETCH_SIZE`` or
``WRITE_SIZE``, KiB per dispatch) and scales them by what the counter read for
the library's copy kernel (``k_copy16``) moving a known number of MiB
(bench.py ``--copy-calib-mb``): bytes per dispatch = value * calib_bytes /
copy_value.

Prints a markdown table of every kernel's calls and average / min / max
duration, and splits the launches of each kernel into those that ran in a
back-to-back batch of at least ``min_batch`` identical launches (the per-kernel
timing batches of ``qasr_hip_decoder_profile``) and the rest (launches inside
real decode steps, prefill, encoder, packing).
"""
import csv
import hashlib
import os
import re
import statistics as st
import sys
from collections import defaultdict

# the device code of the decode kernels (a change of their launch shapes or
# partitions in the host code also calls for a new measurement)
DECODE_SOURCES = ("common.h", "mv_wave.h", "k_attn.hip", "k_int8.hip")

# bench.py's decode kernel labels -> the 0.6B decoder's kernels (rocprofv3 names)
DECODE_LABELS = (("norm+qkv+attention", r"k_qkv_attn<"),
                 ("norm+qkv", r"k_w8a8<1, 4, 0, true, false>"),
                 ("attention", r"k_attn_step<|k_attn_decode<"),
                 ("o_proj+=", r"k_oproj_merge<"),
                 ("norm+gate_up+swiglu", r"k_w8a8<1, 8, 2, true, false>"),
                 ("down+=", r"k_w8a8<3, 1, 1, false, false>"),
                 ("norm+lm_head_argmax", r"k_argmax_w8a8<"),
                 ("argmax_merge", r"k_argmax_finish"))


def decode_sources_hash(root=None):
    """sha256 (16 hex digits) over the decode kernel sources, in DECODE_SOURCES order."""
    root = root or os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc")
    h = hashlib.sha256()
    for f in DECODE_SOURCES:
        with open(os.path.join(root, f), "rb") as fh:
            h.update(f.encode() + b"\0" + fh.read())
    return h.hexdigest()[:16]


def summarise(path, min_batch=20):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    names = [r["Kernel_Name"] for r in rows]
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]
    allk, batch, inline = defaultdict(list), defaultdict(list), defaultdict(list)
    i = 0
    while i < len(rows):
        j = i
        while j + 1 < len(rows) and names[j + 1] == names[i]:
            j += 1
        seg = dur[i:j + 1]
        (batch if len(seg) >= min_batch else inline)[names[i]].extend(seg)
        allk[names[i]].extend(seg)
        i = j + 1
    total = sum(sum(v) for v in allk.values())
    out = ["| kernel | calls | avg us | min us | max us | % time | batch calls | batch avg us | in-step calls | "
           "in-step avg us |", "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, v in sorted(allk.items(), key=lambda kv: -sum(kv[1])):
        b, n = batch.get(name, []), inline.get(name, [])
        short = name.split("(")[0].replace("void ", "")
        out.append(f"| `{short}` | {len(v)} | {st.mean(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                   f"{100 * sum(v) / total:.2f} | {len(b)} | {st.mean(b) if b else 0:.2f} | {len(n)} | "
                   f"{st.mean(n) if n else 0:.2f} |")
    return "\n".join(out)


def summarise_pmc(path, calib_mib):
    rows = list(csv.DictReader(open(path)))
    vals = defaultdict(lambda: defaultdict(list))     # counter -> kernel -> per-dispatch values
    for r in rows:
        name = r["Kernel_Name"].split("(")[0].replace("void ", "")
        vals[r["Counter_Name"]][name].append(float(r["Counter_Value"]))
    out = []
    for counter, per in vals.items():
        copy = [v for k, v in per.items() if "k_copy16" in k]
        ref = st.mean(copy[0]) if copy else None
        # the copy reads and writes calib_mib each
        scale = (calib_mib * 1024.0 / ref) if ref else None
        out.append(f"counter {counter}: copy kernel reads {ref} KiB for {calib_mib} MiB -> scale "
                   f"{scale if scale is None else round(scale, 4)}")
        out.append(f"| kernel | dispatches | avg {counter} KiB | calibrated bytes |")
        out.append("|---|---:|---:|---:|")
        for k, v in sorted(per.items(), key=lambda kv: -st.mean(kv[1])):
            cal = st.mean(v) * 1024.0 * scale if scale else float("nan")
            out.append(f"| `{k}` | {len(v)} | {st.mean(v):.1f} | {cal:.0f} |")
    return "\n".join(out)


def _pmc_bytes(path, calib_mib):
    """kernel -> per-dispatch calibrated bytes of one counter csv (values in
    KiB, scaled so that k_copy16 moved calib_mib MiB)"""
    per = defaultdict(list)
    for r in csv.DictReader(open(path)):
        per[r["Kernel_Name"].split("(")[0].replace("void ", "")].append(float(r["Counter_Value"]))
    copy = [v for k, v in per.items() if "k_copy16" in k][0]
    scale = calib_mib * 1024.0 / st.mean(copy)
    return {k: [x * 1024.0 * scale for x in v] for k, v in per.items()}, scale


def traffic(fetch_csv, write_csv, calib_mib):
    """profiles/hbm_traffic.txt: per bench label, the mean over all its
    dispatches of FETCH_SIZE + WRITE_SIZE bytes (calibrated)."""
    fb, fs = _pmc_bytes(fetch_csv, calib_mib)
    wb, ws = _pmc_bytes(write_csv, calib_mib)
    out = ["# HBM bytes per launch of the config-2 decode kernels: rocprofv3 FETCH_SIZE + WRITE_SIZE (KiB per",
           "# dispatch), each scaled so that the library's copy kernel (k_copy16, %g MiB) reads / writes that" % calib_mib,
           "# much (FETCH_SIZE scale %.4f, WRITE_SIZE scale %.4f); every dispatch of the label's kernels in 20" % (fs, ws),
           "# decode steps at contexts 495-514 (the window of bench.py's per-kernel timing).  Commands (from /tmp,",
           "# TMPDIR=/tmp, PYTHONPATH=$R, QASR_DISABLE_GRAPH=1):",
           "#   timeout -s KILL 150 rocprofv3 --pmc FETCH_SIZE --kernel-include-regex 'k_qkv_attn|k_attn|k_w8a8|k_oproj|k_argmax|k_copy'"
           " --output-format csv -d $R/gpurun_out/pmc_fetch -o run -- python3 -u -m qwenasr_amd.profile_decode 20 64 494",
           "#   (the same with --pmc WRITE_SIZE -d $R/gpurun_out/pmc_write)",
           "#   python -m qwenasr_amd.rocprof_summary --traffic $R/gpurun_out/pmc_fetch/run_counter_collection.csv"
           " $R/gpurun_out/pmc_write/run_counter_collection.csv 64 > profiles/hbm_traffic.txt",
           "# sources_sha256 %s  (qwenasr_amd/csrc/%s; bench.py reports the traffic only for these sources)"
           % (decode_sources_hash(), ", ".join(DECODE_SOURCES)),
           "# columns: bench kernel label, HBM bytes per launch (fetch + write), fetch bytes, write bytes, dispatches"]
    for label, rx in DECODE_LABELS:
        f = [x for k, v in fb.items() if re.search(rx, k) for x in v]
        w = [x for k, v in wb.items() if re.search(rx, k) for x in v]
        if not f or not w:
            continue
        out.append(f"{label} {st.mean(f) + st.mean(w):.0f} {st.mean(f):.0f} {st.mean(w):.0f} {len(f)}")
    return "\n".join(out)


# the shapes of bench_configs.config1, in its order (M outer)
CONFIG1_SHAPES = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
                  ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072), ("lm_head", 151936, 1024)]
BF16_PEAK_TFLOPS = 2500.0


def _gemm_dispatches(path):
    """k_gemm dispatches of one counter csv in dispatch order: (name, {counter: value summed
    over the csv's per-dimension rows}, duration ns)."""
    per = {}
    for r in csv.DictReader(open(path)):
        if "k_gemm" not in r["Kernel_Name"]:
            continue
        d = per.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"].split("(")[0].replace("void ", ""), defaultdict(float),
                                                   int(r["End_Timestamp"]) - int(r["Start_Timestamp"])])
        d[1][r["Counter_Name"]] += float(r["Counter_Value"])
    return [per[k] for k in sorted(per)]


def mfma_config1(util_csv, mops_csv, reps=3, fetch_csv=None, write_csv=None, calib_mib=0.0):
    """The config-1 MFMA table from two counter runs of `bench_configs config1 <reps>`
    (--pmc MfmaUtil; --pmc SQ_INSTS_VALU_MFMA_MOPS_BF16 GRBM_GUI_ACTIVE): per shape the
    median over its reps timed launches (each shape's first launch is its warm-up).
    With the FETCH_SIZE and WRITE_SIZE runs of `bench_configs config1 <reps> <calib MiB>`
    (whose first launch copies calib MiB with k_copy16), also the HBM bytes per launch,
    calibrated on that copy, against the algorithmic bytes (weights, scales, activations
    and the f32 output once)."""
    util, mops = _gemm_dispatches(util_csv), _gemm_dispatches(mops_csv)
    hbm = fetch_csv is not None
    if hbm:
        (_, fs), (_, ws) = _pmc_bytes(fetch_csv, calib_mib), _pmc_bytes(write_csv, calib_mib)
        fetch, write = _gemm_dispatches(fetch_csv), _gemm_dispatches(write_csv)
    per = 1 + reps
    out = ["| M | shape | N x K | kernel | MfmaUtil % | executed GFLOP | 2MNK GFLOP | us | TFLOP/s | % of peak |" +
           (" HBM read MB | HBM write MB | algorithmic MB |" if hbm else ""),
           "|---:|---|---|---|---:|---:|---:|---:|---:|---:|" + ("---:|---:|---:|" if hbm else "")]
    for i, M in enumerate((375, 390, 404)):
        for j, (name, N, K) in enumerate(CONFIG1_SHAPES):
            base = (i * len(CONFIG1_SHAPES) + j) * per
            u = st.median(d[1]["MfmaUtil"] for d in util[base + 1:base + per])
            ex = st.median(d[1]["SQ_INSTS_VALU_MFMA_MOPS_BF16"] for d in mops[base + 1:base + per]) * 512 / 1e9
            us = st.median(d[2] for d in mops[base + 1:base + per]) / 1e3
            kern = re.sub(r"qasr::k_gemm_lds<(.*)>", r"\1", mops[base + 1][0])
            tf = ex * 1e3 / us
            row = (f"| {M} | {name} | {N}x{K} | `{kern}` | {u:.2f} | {ex:.3f} | {2.0 * M * N * K / 1e9:.3f} | "
                   f"{us:.2f} | {tf:.1f} | {100 * tf / BF16_PEAK_TFLOPS:.1f} |")
            if hbm:
                rd = st.median(d[1]["FETCH_SIZE"] for d in fetch[base + 1:base + per]) * 1024 * fs / 1e6
                wr = st.median(d[1]["WRITE_SIZE"] for d in write[base + 1:base + per]) * 1024 * ws / 1e6
                alg = (N * K + 4.0 * N + 2.0 * M * K + 4.0 * M * N) / 1e6
                row += f" {rd:.1f} | {wr:.1f} | {alg:.1f} |"
            out.append(row)
    return "\n".join(out)


if __name__ == "__main__":
    if sys.argv[1] == "--mfma-config1":
        a = sys.argv
        print(mfma_config1(a[2], a[3], int(a[4]) if len(a) > 4 else 3, *(a[5:7] if len(a) > 7 else ()),
                           *((float(a[7]),) if len(a) > 7 else ())))
    elif sys.argv[1] == "--traffic":
        print(traffic(sys.argv[2], sys.argv[3], float(sys.argv[4])))
    elif sys.argv[1] == "--pmc":
        print(summarise_pmc(sys.argv[2], float(sys.argv[3])))
    else:
        print(summarise(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 20))
