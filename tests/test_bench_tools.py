"""CPU checks of bench.py's measurement plumbing: roofline.traffic from rocprofv3 counter CSVs
(calibration on the copy probe, per-class dispatch-weighted means) and the source-hash guard
that turns a traffic file taken on other kernel sources into null."""
import csv
import os

import pytest

import bench


def _csv(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, value in rows:
            w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_from_counters_and_hash_guard(tmp_path, monkeypatch):
    monkeypatch.setattr(bench, "TRAFFIC_FILE", str(tmp_path / "traffic.txt"))
    d = lambda n: str(tmp_path / n)   # noqa: E731
    copy = "void at::native::vectorized_elementwise_kernel<4, copy_kernel>(...)"
    # the probe copies 256 MiB: FETCH reads half (131072 KiB), WRITE all (262144 KiB)
    _csv(d("cf"), "FETCH_SIZE", [(copy, 131072.0)] * 5)
    _csv(d("cw"), "WRITE_SIZE", [(copy, 262144.0)] * 5)
    fin = "void fam::final_kernel<2, 8, 4>(fam::GemmArgs)"
    part = "void fam::partial_kernel<2, 2>(fam::PartArgs)"
    _csv(d("f"), "FETCH_SIZE", [(fin, 100.0), (fin, 300.0), (part, 50.0), ("some_torch_kernel", 9.0)])
    _csv(d("w"), "WRITE_SIZE", [(fin, 10.0), (fin, 10.0), (part, 5.0), ("some_torch_kernel", 9.0)])
    bench.traffic_from(d("f"), d("w"), d("cf"), d("cw"))
    # final: mean fetch 200 KiB x2 + write 10 KiB x1; partial: 50 x2 + 5
    assert bench.measured_traffic("gemm_final") == (200 * 2 + 10) * 1024
    assert bench.measured_traffic("gemm_partial") == (50 * 2 + 5) * 1024
    assert bench.measured_traffic("attention") is None
    # a file written for other kernel sources is not used
    text = open(bench.TRAFFIC_FILE).read()
    open(bench.TRAFFIC_FILE, "w").write(text.replace(f"# sources {bench.sources_hash()}", "# sources 0123456789abcdef"))
    assert bench.measured_traffic("gemm_final") is None


def test_kernel_classes():
    assert bench._kernel_class("void fam::big_kernel<7, 8>(fam::GemmArgs, int, int, int)") == "gemm"
    assert bench._kernel_class("void fam::attn_combine_kernel<16>(fam::AttnArgs, long, long)") == "attn_combine"
    assert bench._kernel_class("void fam::attn_long_kernel<128, true>(fam::AttnArgs, int)") == "attention"
    assert bench._kernel_class("fam::sinusoid_kernel(bool const*, bool*, long)") == "sinusoid"
    assert bench._kernel_class("void fam::rowop_vec_kernel<4, 4>(fam::RowArgs)") == "rowop"
    assert bench._kernel_class("__amd_rocclr_copyBuffer") is None


def test_cpu_description_names_the_host():
    s = bench.cpu_description()
    assert "logical CPUs usable" in s and "family" in s
