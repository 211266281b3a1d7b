"""bench.py's stdout line, built from a stubbed result table of every configuration and a full A/B table: it must
stay a few KB (the driver keeps only the tail of stdout), name the headline configuration and carry the fields of
the driver's contract; the full rows and every A/B sample go to the results files instead."""
import json

import bench

CONFIGS = ["C1", "C2", "C3", "C4", "C5", "D1", "D2", "D3", "P2", "P2n", "D1p", "D2n", "C2b", "DP"]


def stub_row(name, i):
    return dict(op="spec" if name == "C4" else "prefix",
                shape={"B": 2, "k": 64, "L": 65536, "tree": "tree_bd"} if name == "C4" else {"N": 64, "P": 16384},
                dist="randn", us_per_call=100.0 + i, us_spread=dict(p10=99.5, p90=101.25, replays=15),
                gbs=3000.0 + i, pct_peak=37.5, algorithmic_bytes=538969088, tflops=780.5, mfma_pct=31.2,
                eager=dict(us_per_call=120.0, gbs=2900.0),
                dominant=dict(kernel="spec_partial", us=168.79, bytes=537920512, gbs=3186.9, frac=0.3984,
                              tflops=814.0, sq=dict(mfma_busy=0.401, coexec=0.249, valu_per_mfma=4.52),
                              traffic=580000000),
                output_check="ok", distinct_input_sets=4,
                cpu_baseline=dict(value=0.118, unit="GB/s", us_per_call=4567890.1, cores=16, host_cpu_count=128,
                                  blas_threads=[16], runs=3, kind="port",
                                  sample="batch 0 of 2, time scaled x2; median of 3 runs"))


def stub_ab():
    shape = dict(shape={"N": 16, "P": 16384, "S": 1024}, dist="randn", distinct_sets=8, chain=16,
                 median_us={"kernel": 45.0, "torch_naive": 1372.5, "torch_unified": 1942.3},
                 speedup_vs_strongest_ref=30.5, samples_us={"kernel": [45.0] * 30, "torch_naive": [1372.5] * 30})
    return {op: dict(rounds=30, shapes=[dict(shape, config=None) for _ in range(12)], geomean_bench_shapes=20.1,
                     min_bench_shapes=7.0, max_bench_shapes=86.4) for op in ("prefix", "spec", "dsa")}


def test_summary_line_is_short_and_names_the_headline(tmp_path):
    rows = {name: stub_row(name, i) for i, name in enumerate(CONFIGS)}
    ab = stub_ab()
    full = bench.write_results(str(tmp_path), rows, ab, device="AMD Instinct MI355X")
    line = bench.summary_line(rows, ab, steps=20, warmup=5, results=full)
    text = json.dumps(line)
    assert len(text) < 4096, len(text)
    assert "\n" not in text
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in line, k
    assert line["config"]["workload"].startswith("C4:")
    assert line["value"] == rows["C4"]["gbs"]
    assert line["ms_per_step"] == round(rows["C4"]["us_per_call"] / 1e3, 5)
    r = line["roofline"]
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["frac"] == rows["C4"]["dominant"]["frac"] and r["traffic"] == 580000000
    assert r["mfma"]["unit"] == "TFLOP/s" and abs(r["mfma"]["frac"] - 814.0 / 2500.0) < 1e-4
    c = line["cpu_baseline"]
    assert c["kind"] == "port" and c["cores"] == 16 and c["unit"] == "GB/s" and "sample" in c
    assert set(line["ops"]) == set(CONFIGS) and all(len(v) == 3 for v in line["ops"].values())
    assert set(line["ab"]) == {"prefix", "spec", "dsa"}
    # the detail is in the files, not on stdout
    saved = json.load(open(full))
    assert set(saved["ops"]) == set(CONFIGS)
    per_op = json.load(open(tmp_path / "bench_spec.json"))
    assert len(per_op["shapes"][0]["samples_us"]["kernel"]) == 30


def test_summary_line_without_headline_or_ab():
    rows = {"C1": stub_row("C1", 0)}
    rows["C1"].pop("cpu_baseline")
    line = bench.summary_line(rows, None, steps=5, warmup=1)
    assert line["config"]["workload"].startswith("C1:")
    assert line["cpu_baseline"] is None and line["ab"] is None and line["results"] is None
    assert len(json.dumps(line)) < 4096


def test_gate_screens_the_kernel_modules():
    """The A/B leg imports a kernel module only after the verifier's static gate passes it."""
    for op in ("prefix", "spec", "dsa"):
        mod = bench.screened_module(op)
        assert callable(mod.kernel)
