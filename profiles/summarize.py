"""Summarises a rocprofv3 kernel-trace database (rocpd sqlite, `-o run` -> run_results.db) into a short text table:
per libvmk kernel and grid size, the number of dispatches and the average / min / max duration in microseconds.

    python profiles/summarize.py gpurun_out/prof/run_results.db > profiles/<name>.txt
"""
import sqlite3
import sys


def summarize(path, prefix="vmk::"):
    db = sqlite3.connect(path)
    rows = db.execute(
        "select name, grid_x, grid_y, workgroup_x, count(*), avg(duration), min(duration), max(duration), "
        "vgpr_count, accum_vgpr_count, lds_size from kernels where name like ? "
        "group by name, grid_x, grid_y order by name, grid_x", ("%" + prefix + "%",)).fetchall()
    out = [f"{'kernel':32s} {'grid':>14s} {'wg':>5s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s}"
           f" {'vgpr':>5s} {'agpr':>5s} {'lds':>7s}"]
    for name, gx, gy, wgx, n, avg, mn, mx, vg, ag, lds in rows:
        short = name.split("(")[0].replace("void ", "").replace(prefix, "")
        out.append(f"{short:32s} {f'{gx}x{gy}':>14s} {wgx:>5d} {n:>6d} {avg / 1e3:>10.2f} {mn / 1e3:>10.2f} "
                   f"{mx / 1e3:>10.2f} {vg:>5d} {ag:>5d} {lds:>7d}")
    return "\n".join(out)


if __name__ == "__main__":
    print(summarize(sys.argv[1]))
