"""Summarise a rocprofv3 kernel trace (``--kernel-trace --output-format csv``).

    python -m qwenasr_amd.rocprof_summary <dir>/run_kernel_trace.csv [min_batch]
    python -m qwenasr_amd.rocprof_summary --pmc <dir>/run_counter_collection.csv <calib MiB>

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
import statistics as st
import sys
from collections import defaultdict


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


if __name__ == "__main__":
    if sys.argv[1] == "--pmc":
        print(summarise_pmc(sys.argv[2], float(sys.argv[3])))
    else:
        print(summarise(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 20))
