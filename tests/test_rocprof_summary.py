"""The profile summary tool and bench.py's staleness check of the committed traffic figures
(CPU only: synthetic rocprofv3 CSV files)."""
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from tabinfer_amd import rocprof_summary as RS  # noqa: E402


def _write_pmc(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, vals in rows.items():
            for v in vals:
                w.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": v})


def test_traffic_scales_by_the_copy_calibration(tmp_path):
    copy = "k_copy_u4(uint4 const*, uint4*, unsigned long)"
    gemv = "void k_gemv_q4_q8<64, 1, 1>(signed char const*, float const*)"
    other = "void k_gemv_q4_q8<32, 3, 1>(signed char const*, float const*)"
    # the copy moves 1 MiB each way; FETCH_SIZE reads half of it, WRITE_SIZE all of it; the
    # 4 KiB copies of the same kernel are left out of the calibration
    _write_pmc(str(tmp_path / "f"), "FETCH_SIZE", {copy: [512.0, 2.0, 512.0], gemv: [100.0, 300.0], other: [7.0]})
    _write_pmc(str(tmp_path / "w"), "WRITE_SIZE", {copy: [1024.0, 4.0], gemv: [4.0, 4.0], other: [1.0]})
    src = tmp_path / "k.hip"
    src.write_text("kernel source")
    res = RS.traffic(str(tmp_path / "f"), str(tmp_path / "w"), ("k_copy_u4", 1 << 20), "abc123", [str(src)],
                     [("o_proj", "k_gemv_q4_q8<64")])
    # (mean 200 KiB x 2) read + 4 KiB written
    assert res["families"] == {"o_proj": 400 * 1024 + 4 * 1024}
    assert res["_stamp"]["commit"] == "abc123"
    (path, digest), = res["_stamp"]["sources"].items()
    assert path.endswith("k.hip") and len(digest) == 64


def test_traffic_rejects_an_ambiguous_kernel_name(tmp_path):
    _write_pmc(str(tmp_path / "f"), "FETCH_SIZE", {"k_copy_u4": [1.0], "k_a<1>": [1.0], "k_a<2>": [1.0]})
    _write_pmc(str(tmp_path / "w"), "WRITE_SIZE", {"k_copy_u4": [1.0], "k_a<1>": [1.0], "k_a<2>": [1.0]})
    try:
        RS.traffic(str(tmp_path / "f"), str(tmp_path / "w"), ("k_copy_u4", 1024), "x", [], [("a", "k_a<")])
    except SystemExit as e:
        assert "matches 2 kernels" in str(e)
    else:
        raise AssertionError("an ambiguous --map was accepted")


def test_bench_marks_traffic_measured_on_other_sources(tmp_path, monkeypatch):
    import bench
    src = tmp_path / "csrc" / "k.hip"
    src.parent.mkdir()
    src.write_text("v1")
    (tmp_path / "profiles").mkdir()
    stamp = {"commit": "c0ffee", "sources": {"csrc/k.hip": bench.sha256_file(str(src))}}
    (tmp_path / "profiles" / "traffic.json").write_text(json.dumps(
        {"families": {"qkv": 123}, "_source": "s", "_stamp": stamp}))
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.traffic_record("qkv") == (123, "s", "c0ffee", False)
    src.write_text("v2")
    assert bench.traffic_record("qkv") == (123, "s", "c0ffee", True)
    src.unlink()
    assert bench.traffic_record("qkv")[3] is True


def test_bench_refuses_more_than_one_gpu():
    import subprocess
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], stdout=subprocess.PIPE,
                       stderr=subprocess.PIPE, text=True, timeout=120)
    assert r.returncode == 2 and "single GPU" in r.stderr and not r.stdout
