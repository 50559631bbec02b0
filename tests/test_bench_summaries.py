"""The profile summarizers of bench.py on small synthetic rocprofv3 CSVs (CPU only): the kernel
trace's back-to-back / all-dispatch statistics and the counter runs' traffic JSON, whose numbers
bench.py puts in the line's roofline."""

import csv
import json

import bench


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summarize_trace_back_to_back(tmp_path):
    """Dispatches whose neighbours in time are the same kernel count as back-to-back; others only
    in 'all'. Names lose their argument list and namespaces."""
    a = "void (anonymous namespace)::k_a<1, 2>(int, float*)"
    b = "(anonymous namespace)::k_b(int)"
    rows = []
    t = 0
    for name, d in [(a, 1000), (a, 2000), (a, 3000), (a, 4000), (b, 500), (a, 9000)]:
        rows.append((t, t + d, name))
        t += d
    p = tmp_path / "kt.csv"
    _write(p, ["Start_Timestamp", "End_Timestamp", "Kernel_Name"], rows)
    s = bench.summarize_trace(str(p))
    assert set(s) == {"k_a<1, 2>", "k_b"}
    # k_a: dispatches 2 and 3 (of 1..4, then 6) have k_a on both sides
    assert s["k_a<1, 2>"]["b2b"] == {"n": 2, "avg_us": 2.5, "median_us": 3.0}
    assert s["k_a<1, 2>"]["all"]["n"] == 5 and s["k_a<1, 2>"]["all"]["avg_us"] == 3.8
    assert s["k_b"]["b2b"] is None and s["k_b"]["all"]["n"] == 1


def test_summarize_pmc_scales_by_the_copy(tmp_path):
    """Read and written bytes per dispatch are the counters' medians scaled by what they read for
    the 256 MiB calibration copy; one file per M, keyed by projection."""
    copy = "__amd_rocclr_copyBuffer"
    f_rows, w_rows = [], []
    for M, kernels in bench.STEP_KERNELS.items():
        for i, (proj, k) in enumerate(kernels.items()):
            for rep, extra in enumerate((0, 2, 1)):  # three dispatches: median = base + 1
                base = 1000 * (i + 1) + M
                f_rows.append(("FETCH_SIZE", f"void {k}(int)", base + extra))
                w_rows.append(("WRITE_SIZE", f"void {k}(int)", 10 * (i + 1) + extra))
    f_rows.append(("FETCH_SIZE", copy, 131072))   # the copy reads 256 MiB: FETCH_SIZE 0.5x
    w_rows.append(("WRITE_SIZE", copy, 262144))   # WRITE_SIZE 1.0x
    pf, pw = tmp_path / "f.csv", tmp_path / "w.csv"
    _write(pf, ["Counter_Name", "Kernel_Name", "Counter_Value"], f_rows)
    _write(pw, ["Counter_Name", "Kernel_Name", "Counter_Value"], w_rows)
    paths = bench.summarize_pmc(str(pf), str(pw), str(tmp_path))
    assert [p.split("/")[-1] for p in paths] == ["traffic_c2.json", "traffic_c3.json"]
    for M, cfg in ((1, "c2"), (16, "c3")):
        d = json.load(open(tmp_path / f"traffic_{cfg}.json"))
        assert d["M"] == M and abs(d["fetch_scale"] - 0.5) < 1e-12 and d["write_scale"] == 1.0
        for i, (proj, k) in enumerate(bench.STEP_KERNELS[M].items()):
            r = d["projections"][proj]
            assert r["kernel"] == k and r["dispatches"] == 3
            assert r["fetch_kib_median"] == 1000 * (i + 1) + M + 1
            assert r["read_bytes_median"] == (1000 * (i + 1) + M + 1) * 1024 / 0.5
            assert r["write_bytes_median"] == (10 * (i + 1) + 1) * 1024
