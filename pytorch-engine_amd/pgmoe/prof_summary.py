"""Summarise a rocprofv3 results database (kernel trace) into a per-kernel table.

    python -m pgmoe.prof_summary gpurun_out/prof/run_results.db

Groups dispatches by kernel name and grid, reporting calls and average / min / max
duration in microseconds plus the kernel's register and LDS use.
"""

import collections
import sqlite3
import sys


def summarise(db: str) -> str:
    c = sqlite3.connect(db)
    rows = c.execute("select name, duration, grid_x, grid_y, workgroup_x, vgpr_count, accum_vgpr_count, "
                     "sgpr_count, lds_size, scratch_size from kernels").fetchall()
    agg = collections.OrderedDict()
    for name, dur, gx, gy, wx, vg, ag, sg, lds, scr in rows:
        key = (name.split("(")[0], gx, gy, wx)
        a = agg.setdefault(key, [0, 0.0, float("inf"), 0.0, (vg, ag, sg, lds, scr)])
        a[0] += 1
        a[1] += dur
        a[2] = min(a[2], dur)
        a[3] = max(a[3], dur)
    out = ["| kernel | grid (threads) | block | calls | avg us | min us | max us | vgpr/agpr/sgpr/lds/scratch |",
           "|---|---|---|---|---|---|---|---|"]
    for (n, gx, gy, wx), (k, tot, mn, mx, res) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| `{n}` | {gx}x{gy} | {wx} | {k} | {tot / k / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} | "
                   f"{'/'.join(str(v) for v in res)} |")
    return "\n".join(out)


if __name__ == "__main__":
    print(summarise(sys.argv[1]))
