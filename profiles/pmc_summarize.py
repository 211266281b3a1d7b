"""Summarises the PMC counters of a rocprofv3 `--pmc` run (rocpd sqlite database) per kernel name: the average over
dispatches of each counter's per-dispatch value (summed over the device's instances).

    python profiles/pmc_summarize.py gpurun_out/pmc/run_results.db [kernel-name-substring]
"""
import sqlite3
import sys
from collections import defaultdict


def summarize(path, like="vmk::"):
    db = sqlite3.connect(path)
    rows = db.execute("select kernel_name, dispatch_id, counter_name, sum(value) from counters_collection "
                      "where kernel_name like ? group by kernel_name, dispatch_id, counter_name",
                      (f"%{like}%",)).fetchall()
    acc = defaultdict(lambda: defaultdict(list))
    for name, disp, cname, val in rows:
        acc[name.split("(")[0]][cname].append(val)
    out = []
    for name, cs in sorted(acc.items()):
        n = max(len(v) for v in cs.values())
        out.append(f"{name}  ({n} dispatches)")
        for cname, vals in sorted(cs.items()):
            out.append(f"    {cname:32s} {sum(vals) / len(vals):16.1f}")
    return "\n".join(out)


if __name__ == "__main__":
    print(summarize(sys.argv[1], sys.argv[2] if len(sys.argv) > 2 else "vmk::"))
