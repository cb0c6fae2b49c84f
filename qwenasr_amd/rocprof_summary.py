"""Summarise a rocprofv3 kernel trace (``--kernel-trace --output-format csv``).

    python -m qwenasr_amd.rocprof_summary <dir>/run_kernel_trace.csv [min_batch]

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


if __name__ == "__main__":
    print(summarise(sys.argv[1], int(sys.argv[2]) if len(sys.argv) > 2 else 20))
