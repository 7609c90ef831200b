"""Summarise rocprofv3 results databases.

    python -m pgmoe.prof_summary RUN_results.db                 # kernel trace table
    python -m pgmoe.prof_summary --pmc RUN_results.db [NAME]    # counters per kernel
    python -m pgmoe.prof_summary --traffic FETCH.db WRITE.db NAME  # HBM bytes per launch
    python -m pgmoe.prof_summary --trace-json RUN_results.db [COMMAND]  # per-kernel averages, JSON

The kernel-trace mode groups dispatches by kernel name, grid and block. For each group it
reports the number of calls, the average / min / max duration in microseconds, and the
kernel's register and LDS use.

The counter mode (a `rocprofv3 --pmc ...` database) sums each counter over its instances
within a dispatch (XCDs, channels), then averages over the dispatches of each kernel. The
result is one row per kernel whose name contains NAME; by default these are the pgmoe
kernels and the runtime's copy kernels.
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


def trace_json(db: str, command: str = "") -> dict:
    """{"command": ..., "kernels": {name: {"calls", "avg_us", "min_us", "max_us"}}} of a
    kernel-trace database (dispatches grouped by kernel name and launch shape; the most
    called shape of each name is kept)."""
    c = sqlite3.connect(db)
    rows = c.execute("select name, duration, grid_x, grid_y, workgroup_x from kernels").fetchall()
    agg = collections.defaultdict(list)
    for name, dur, gx, gy, wx in rows:
        agg[(name.split("(")[0], gx, gy, wx)].append(dur)
    best = {}
    for (n, gx, gy, wx), ds in agg.items():
        if n not in best or len(ds) > best[n]["calls"]:
            best[n] = {"calls": len(ds), "avg_us": round(sum(ds) / len(ds) / 1e3, 3),
                       "min_us": round(min(ds) / 1e3, 3), "max_us": round(max(ds) / 1e3, 3),
                       "grid": [gx, gy], "block": wx}
    return {"command": command, "kernels": best}


def pmc_table(db: str, pattern: str = "") -> dict:
    """{kernel: {counter: mean per-dispatch value, "_dispatches": n}}."""
    c = sqlite3.connect(db)
    rows = c.execute("select dispatch_id, name, counter_name, counter_value from pmc_events").fetchall()
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names = {}
    for d, n, cn, cv in rows:
        per[d][cn] += cv
        names[d] = n.split("(")[0]
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for d, cs in per.items():
        n = names[d]
        if pattern and pattern not in n:
            continue
        if not pattern and "pgmoe" not in n and "copy" not in n.lower() and "elementwise" not in n:
            continue
        for cn, v in cs.items():
            agg[n][cn].append(v)
    out = {}
    for n, cs in agg.items():
        out[n] = {cn: sum(vs) / len(vs) for cn, vs in cs.items()}
        out[n]["_dispatches"] = max(len(vs) for vs in cs.values())
    return out


def summarise_pmc(db: str, pattern: str = "") -> str:
    t = pmc_table(db, pattern)
    lines = ["| kernel | dispatches | counters (mean per dispatch) |", "|---|---|---|"]
    for n, cs in sorted(t.items()):
        vals = ", ".join(f"{k}={v:.6g}" for k, v in sorted(cs.items()) if not k.startswith("_"))
        lines.append(f"| `{n}` | {cs['_dispatches']} | {vals} |")
    return "\n".join(lines)


def _dispatch_values(db: str, pattern: str, counter: str) -> list:
    """Per-dispatch totals of `counter` (summed over instances) for kernels whose name
    contains `pattern`."""
    c = sqlite3.connect(db)
    rows = c.execute("select dispatch_id, name, counter_name, counter_value from pmc_events").fetchall()
    per = collections.defaultdict(float)
    for d, n, cn, cv in rows:
        if cn == counter and pattern in n:
            per[d] += cv
    return [per[d] for d in sorted(per)]


def traffic(fetch_db: str, write_db: str, pattern: str, copy_name: str = "copyBuffer") -> dict:
    """HBM bytes per launch of the kernels whose name contains `pattern`, from a
    FETCH_SIZE pass and a WRITE_SIZE pass (KiB per dispatch, summed over instances), each
    scaled by what the same counter reads for the largest runtime device copies in the
    same runs (bytes moved per copy = their WRITE_SIZE, which reports every byte written)."""
    fk = _dispatch_values(fetch_db, pattern, "FETCH_SIZE")
    wk = _dispatch_values(write_db, pattern, "WRITE_SIZE")
    fc = _dispatch_values(fetch_db, copy_name, "FETCH_SIZE")
    wc = _dispatch_values(write_db, copy_name, "WRITE_SIZE")
    big_w = [v for v in wc if v >= 0.5 * max(wc)]
    big_f = sorted(fc)[-len(big_w):]
    moved_kib = sum(big_w) / len(big_w)
    fetch_factor = moved_kib / (sum(big_f) / len(big_f))
    write_factor = 1.0
    f_kib = sum(fk) / len(fk)
    w_kib = sum(wk) / len(wk)
    fetch_b = f_kib * 1024 * fetch_factor
    write_b = w_kib * 1024 * write_factor
    return {"kernel_pattern": pattern, "bytes_per_launch": int(round(fetch_b + write_b)),
            "fetch_bytes": int(round(fetch_b)), "write_bytes": int(round(write_b)),
            "fetch_size_kib_raw": round(f_kib, 3), "write_size_kib_raw": round(w_kib, 3),
            "fetch_factor": round(fetch_factor, 5), "write_factor": write_factor,
            "dispatches": [len(fk), len(wk)],
            "calibration": f"{len(big_w)} device copies ({copy_name}): FETCH_SIZE {sum(big_f) / len(big_f):.1f} KiB, "
                           f"WRITE_SIZE {moved_kib:.1f} KiB per copy"}


if __name__ == "__main__":
    if len(sys.argv) >= 5 and sys.argv[1] == "--traffic":
        import json
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], sys.argv[4]), indent=1))
    elif len(sys.argv) >= 3 and sys.argv[1] == "--trace-json":
        import json
        print(json.dumps(trace_json(sys.argv[2], sys.argv[3] if len(sys.argv) > 3 else ""), indent=1))
    elif len(sys.argv) >= 3 and sys.argv[1] == "--pmc":
        print(summarise_pmc(sys.argv[2], sys.argv[3] if len(sys.argv) > 3 else ""))
    else:
        print(summarise(sys.argv[1]))
