"""Short text summaries of rocprofv3 result databases (rocpd sqlite, `-o run` -> run_results.db).

    python -m vmk.rocprof kernels <run_results.db> [name-substring]      per kernel and grid: calls, avg/min/max us
    python -m vmk.rocprof pmc <run_results.db> [name-substring]          per kernel: average counter value per dispatch
    python -m vmk.rocprof traffic <fetch.db> <write.db> <copy_bytes>     HBM bytes per call of the dominant kernels
    python -m vmk.rocprof trafficjson <fetch.db> <write.db> <copy_bytes> <config> <bracket> <algorithmic_bytes>
                          <out.json> <kernel-prefix>...      one configuration's bracket (the kernels whose names
                                                             start with a prefix), as bench.py reads it
    python -m vmk.rocprof mfmajson <sq.db> <config> <bracket> <kernel-prefix> <out.json>
                          MFMA-busy share, co-issue and VALU per MFMA of one kernel from an SQ counter run

`traffic` reads one FETCH_SIZE run and one WRITE_SIZE run of the same command (rocprofv3 collects each in its own
pass).  The command must include a plain streaming kernel that reads `copy_bytes` bytes and writes as many
(bench.py --calibrate-copy runs torch.bitwise_not over int32): the counters' reading for that kernel, divided by its
true bytes, is the calibration factor applied to every kernel.
"""
import sqlite3
import sys
from collections import defaultdict

KERNEL_PREFIX = "vmk"          # matches "vmk::name" and the mangled "_ZN3vmk..." that rocprofv3 leaves for some
                               # template kernels (those with vector-type arguments)

_MANGLED_ARGS = [("Dv8_DF16_", "half8"), ("Dv8_DF16b", "bf16x8"), ("DF16_", "_Float16"), ("DF16b", "__bf16"),
                 ("Lb0E", "false"), ("Lb1E", "true")]


def _demangle_vmk(name):
    """'_ZN3vmk18prefix_rows_kernelILi8ELb1EDv8_DF16_EEvNS_10PrefixArgsE' -> 'prefix_rows_kernel<8, true, half8>'
    (only the argument forms libvmk's kernels use; anything else is returned unchanged)."""
    rest = name[len("_ZN3vmk"):]
    digits = ""
    while rest and rest[0].isdigit():
        digits, rest = digits + rest[0], rest[1:]
    if not digits:
        return name
    base, rest = rest[:int(digits)], rest[int(digits):]
    if not rest.startswith("I"):
        return base
    rest, args = rest[1:], []
    while rest and not rest.startswith("E"):
        if rest.startswith("Li"):
            end = rest.index("E")
            args.append(rest[2:end])
            rest = rest[end + 1:]
            continue
        for code, text in _MANGLED_ARGS:
            if rest.startswith(code):
                args.append(text)
                rest = rest[len(code):]
                break
        else:
            return name
    return f"{base}<{', '.join(args)}>"


def _short(name):
    if name.startswith("_ZN3vmk"):
        return _demangle_vmk(name)
    return name.split("(")[0].replace("void ", "").replace("vmk::", "")


def kernels(path, like=KERNEL_PREFIX):
    db = sqlite3.connect(path)
    rows = db.execute(
        "select name, grid_x, grid_y, workgroup_x, count(*), avg(duration), min(duration), max(duration), "
        "vgpr_count, accum_vgpr_count, lds_size from kernels where name like ? "
        "group by name, grid_x, grid_y order by name, grid_x", (f"%{like}%",)).fetchall()
    out = [f"{'kernel':32s} {'grid':>14s} {'wg':>5s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s}"
           f" {'vgpr':>5s} {'agpr':>5s} {'lds':>7s}"]
    for name, gx, gy, wgx, n, avg, mn, mx, vg, ag, lds in rows:
        out.append(f"{_short(name):32s} {f'{gx}x{gy}':>14s} {wgx:>5d} {n:>6d} {avg / 1e3:>10.2f} {mn / 1e3:>10.2f} "
                   f"{mx / 1e3:>10.2f} {vg:>5d} {ag:>5d} {lds:>7d}")
    return "\n".join(out)


def pmc_table(path, like=""):
    """{kernel short name: {counter: [per-dispatch values]}} (each value summed over the device's instances)."""
    db = sqlite3.connect(path)
    rows = db.execute("select kernel_name, dispatch_id, counter_name, sum(value) from counters_collection "
                      "where kernel_name like ? group by kernel_name, dispatch_id, counter_name",
                      (f"%{like}%",)).fetchall()
    acc = defaultdict(lambda: defaultdict(list))
    for name, _disp, cname, val in rows:
        acc[_short(name)][cname].append(val)
    return acc


def pmc(path, like=KERNEL_PREFIX):
    out = []
    for name, cs in sorted(pmc_table(path, like).items()):
        n = max(len(v) for v in cs.values())
        out.append(f"{name}  ({n} dispatches)")
        for cname, vals in sorted(cs.items()):
            out.append(f"    {cname:32s} {sum(vals) / len(vals):16.1f}")
    return "\n".join(out)


def _copy_kernel(table, counter):
    """The calibration kernel (bench.py --calibrate-copy): the bitwise_not kernel with the largest reading."""
    cands = [k for k in table if "bitwise_not" in k and counter in table[k]]
    if not cands:
        raise SystemExit("no calibration kernel in the run: use bench.py --calibrate-copy")
    return max(cands, key=lambda k: max(table[k][counter]))


def traffic(fetch_db, write_db, copy_bytes):
    """Per vmk kernel: average calibrated HBM read and write bytes per dispatch."""
    f, w = pmc_table(fetch_db), pmc_table(write_db)
    ck = _copy_kernel(f, "FETCH_SIZE")
    fc = max(f[ck]["FETCH_SIZE"]) * 1024.0                  # the largest copy dispatch is the calibration copy
    wc = max(w[_copy_kernel(w, "WRITE_SIZE")]["WRITE_SIZE"]) * 1024.0
    kf, kw = fc / copy_bytes, wc / copy_bytes
    out = [f"calibration: kernel {ck!r} over {copy_bytes} bytes reads FETCH_SIZE x {kf:.3f}, "
           f"WRITE_SIZE x {kw:.3f} of its true bytes", f"{'kernel':32s} {'dispatches':>10s} {'read_MB':>10s} "
           f"{'write_MB':>10s}"]
    res = {}
    for name in sorted(f):
        if name not in w or "FETCH_SIZE" not in f[name] or ck == name:
            continue
        if not any(s in name for s in ("prefix", "spec", "dsa", "proj_", "decode")):
            continue
        fv, wv = f[name]["FETCH_SIZE"], w[name]["WRITE_SIZE"]
        rd = sum(fv) / len(fv) * 1024.0 / kf
        wr = sum(wv) / len(wv) * 1024.0 / kw
        res[name] = dict(read=rd, write=wr, dispatches=len(fv))
        out.append(f"{name:32s} {len(fv):>10d} {rd / 1e6:>10.2f} {wr / 1e6:>10.2f}")
    return "\n".join(out), res, (kf, kw)


def traffic_json(fetch_db, write_db, copy_bytes, config, bracket, algorithmic, prefixes, commands=()):
    """The HBM bytes per call of one configuration's dominant bracket from a FETCH_SIZE and a WRITE_SIZE run of that
    configuration alone: the per-dispatch averages of the bracket's kernels (names starting with one of
    `prefixes`) summed, as the dict bench.py reads from profiles/<config>_traffic.json."""
    _, res, (kf, kw) = traffic(fetch_db, write_db, copy_bytes)
    names = sorted(n for n in res if any(n.startswith(p) for p in prefixes))
    if not names:
        raise SystemExit(f"no kernel of the run starts with {prefixes}")
    rd = sum(res[n]["read"] for n in names)
    wr = sum(res[n]["write"] for n in names)
    return dict(workload=config, kernel=bracket,
                note=f"HBM bytes per call of the {bracket} bracket: {' + '.join(names)}; FETCH_SIZE and WRITE_SIZE "
                     f"scaled by the calibration kernel's reading (read x{kf:.3f}, write x{kw:.3f} of true bytes)",
                read_bytes=int(round(rd, -4)), write_bytes=int(round(wr, -4)), algorithmic_bytes=int(algorithmic),
                ratio=round((rd + wr) / algorithmic, 3), commands=list(commands))


SIMDS = 1024                   # MI355X: 8 XCDs x 32 CUs x 4 SIMDs


def mfma_json(sq_db, config, bracket, prefix):
    """MFMA utilisation of the kernel whose name starts with `prefix`, from one SQ counter run: busy share =
    SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs) (GRBM_GUI_ACTIVE is summed over the 8 XCDs),
    co-issue = SQ_VALU_MFMA_COEXEC_CYCLES / SQ_VALU_MFMA_BUSY_CYCLES, VALU per MFMA = SQ_INSTS_VALU /
    SQ_INSTS_MFMA; per-dispatch averages."""
    t = pmc_table(sq_db)
    names = [n for n in t if n.startswith(prefix)]
    if len(names) != 1:
        raise SystemExit(f"{len(names)} kernels start with {prefix!r}: {names}")
    c = {k: sum(v) / len(v) for k, v in t[names[0]].items()}
    busy = c["SQ_VALU_MFMA_BUSY_CYCLES"]
    return dict(workload=config, kernel=bracket, kernel_name=names[0],
                mfma_busy=round(busy / (c["GRBM_GUI_ACTIVE"] / 8 * SIMDS), 4),
                coexec=round(c["SQ_VALU_MFMA_COEXEC_CYCLES"] / busy, 4) if busy else None,
                valu_per_mfma=round(c["SQ_INSTS_VALU"] / c["SQ_INSTS_MFMA"], 2) if c.get("SQ_INSTS_MFMA") else None,
                counters={k: round(v, 1) for k, v in sorted(c.items())})


if __name__ == "__main__":
    cmd = sys.argv[1] if len(sys.argv) > 1 else ""
    if cmd == "kernels":
        print(kernels(sys.argv[2], sys.argv[3] if len(sys.argv) > 3 else KERNEL_PREFIX))
    elif cmd == "pmc":
        print(pmc(sys.argv[2], sys.argv[3] if len(sys.argv) > 3 else KERNEL_PREFIX))
    elif cmd == "traffic":
        print(traffic(sys.argv[2], sys.argv[3], int(sys.argv[4]))[0])
    elif cmd == "trafficjson":
        import json
        fdb, wdb, cb, config, bracket, algo, out = sys.argv[2:9]
        cmds = [f"cd /tmp && rocprofv3 --pmc {c} -d <dir> -o run -- python3 $R/bench.py --configs {config} --no-cpu "
                f"--ab-rounds 0 --steps 3 --warmup 1 --calibrate-copy {cb} --results ''" for c in ("FETCH_SIZE",
                                                                                                  "WRITE_SIZE")]
        cmds.append(f"PYTHONPATH=$R/verified-metal-kernels_amd python3 -m vmk.rocprof trafficjson <fetch db> "
                    f"<write db> {cb} {config} {bracket} {algo} profiles/{config}_traffic.json {' '.join(sys.argv[9:])}")
        d = traffic_json(fdb, wdb, int(cb), config, bracket, int(algo), sys.argv[9:], cmds)
        with open(out, "w") as f:
            json.dump(d, f, indent=1)
        print(json.dumps(d))
    elif cmd == "mfmajson":
        import json
        d = mfma_json(*sys.argv[2:6])
        with open(sys.argv[6], "w") as f:
            json.dump(d, f, indent=1)
        print(json.dumps(d))
    else:
        raise SystemExit(__doc__)
