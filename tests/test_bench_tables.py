"""
bench.py's profile tables, without a GPU: the HBM-traffic table scales each counter by
what it reads for the calibration copy, and the bench line finds its kernel's row.
"""

import csv

import bench

HEAD = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEAD)
        for i, (name, v) in enumerate(rows):
            w.writerow([i, name, counter, v])


def test_traffic_table_scales_by_the_copy(tmp_path, monkeypatch):
    copy = "void at::native::vectorized_elementwise_kernel<8, at::native::neg_kernel_cuda(x)>(int)"
    fwd = "void nsmoe::expert_fwd_async_kernel<0, 2, 3>(nsmoe::ExpParams)"
    # FETCH_SIZE undercounts by 2 on the copy; WRITE_SIZE is exact
    _write(tmp_path / "f.csv", "FETCH_SIZE", [(copy, bench.COPY_BYTES / 1024 / 2),
                                              (fwd, 100.0), (fwd, 300.0)])
    _write(tmp_path / "w.csv", "WRITE_SIZE", [(copy, bench.COPY_BYTES / 1024),
                                              (fwd, 50.0), (fwd, 50.0)])
    table = bench.pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"))
    row = [l for l in table.splitlines() if l.startswith("| expert_fwd")]
    assert len(row) == 1
    # mean FETCH 200 KiB x 2 + WRITE 50 KiB x 1
    assert row[0].endswith(f"| {200 * 1024 * 2 + 50 * 1024} |")
    md = tmp_path / "traffic.md"
    md.write_text("intro line\n\n" + table + "\n")
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(md))
    assert bench.committed_traffic("expert_fwd") == 200 * 1024 * 2 + 50 * 1024
    assert bench.committed_traffic("expert_bwd") is None


def test_committed_traffic_table_has_the_expert_kernels():
    for k in ("expert_fwd", "expert_bwd", "expert_dx", "dw", "combine", "route_fwd"):
        assert bench.committed_traffic(k) > 0, k


def test_stats_table(tmp_path):
    p = tmp_path / "s.csv"
    with open(p, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs",
                    "MaxNs"])
        w.writerow(["small", 2, 2000, 1000, 10.0, 900, 1100])
        w.writerow(["big", 1, 18000, 18000, 90.0, 18000, 18000])
    lines = bench.stats_summary(str(p)).splitlines()
    assert lines[2].startswith("| big | 1 | 18.00")
    assert lines[3].startswith("| small | 2 | 1.00")
