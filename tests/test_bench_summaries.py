"""CPU tests of bench.py's summaries of rocprofv3 output (the tables under
profiles/ are printed by them): synthetic CSV files in rocprofv3's layout."""
import csv
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP8 = "void mfh::(anonymous namespace)::k_dequant_fp8<4, 2, 128>(unsigned char const*, void*, long, float)"


def write_csv(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def run_bench(*args):
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 0, res.stderr
    return res.stdout


def test_trace_table_takes_the_last_k_dispatches_and_windows_after_the_eager_ones(tmp_path):
    # 3 eager dispatches (one per rotated set), then 40 replayed ones: the
    # first 10 replayed take 2000 ns, the rest 1000 ns, 100 us apart
    sets, k = 3, 20
    trace = [(i * 1_000_000, 5000) for i in range(sets)]
    t0 = 10_000_000
    trace += [(t0 + i * 100_000, 2000 if i < 10 else 1000) for i in range(40)]
    d = tmp_path / "prof"
    write_csv(str(d / "host" / "run_kernel_trace.csv"),
              [{"Kernel_Name": FP8, "Start_Timestamp": s, "End_Timestamp": s + n} for s, n in trace])
    write_csv(str(d / "host" / "run_kernel_stats.csv"),
              [{"Name": FP8, "Calls": len(trace), "AverageNs": 1500.0, "MinNs": 1000, "MaxNs": 5000}])
    bench = {"configs": [{"config": 2, "rotated_sets": sets, "bytes_per_step": 3000, "ms_per_step": 0.0012,
                          "GB_s": 2500.0, "cast_same_mix": {"GB_s": 2600.4}}]}
    (tmp_path / "b.json").write_text("log line\n" + json.dumps(bench) + "\n")
    out = run_bench("--summarize-trace", str(d), "--bench-json", str(tmp_path / "b.json"), "--steps", str(k))
    rows = [l for l in out.splitlines() if l.startswith("| `k_dequant_fp8")]
    assert len(rows) == 2
    # timed avg = last 20 dispatches = 1000 ns; 3000 bytes / 1000 ns = 3 GB/s
    assert rows[0].split(" | ")[5:8] == ["1000", "3000", "3"]
    assert rows[0].endswith("| 1200 | 2500 | 2600 |")
    # the replay starts after the 3 eager dispatches: its first 2 ms hold 20
    # dispatches, mean (10 * 2000 + 10 * 1000) / 20 = 1500 -> +50% against
    # 1000, the next 2 ms the other 20 at 1000; the worst 20 in a row are
    # the first 20
    assert rows[1].split(" | ")[2:4] == ["+50.0% (20)", "+0.0% (20)"]
    assert rows[1].endswith("| +50.0% |")


def test_pmc_summary_scales_by_the_copy_calibration(tmp_path):
    copy = "void mfh::(anonymous namespace)::k_convert_vec<2, 2, 64>(void const*, void*, long)"
    for counter, sub, copy_kib, fp8_kib in (("FETCH_SIZE", "fetch", 32768.0, 28672.0),
                                            ("WRITE_SIZE", "write", 65536.0, 114688.0)):
        rows = []
        for disp, (name, v) in enumerate([(copy, copy_kib), (FP8, fp8_kib), (FP8, fp8_kib)]):
            rows.append({"Dispatch_Id": disp, "Kernel_Name": name, "Counter_Name": counter, "Counter_Value": v})
        write_csv(str(tmp_path / sub / "host" / "run_counter_collection.csv"), rows)
    doc = json.loads(run_bench("--summarize-pmc", str(tmp_path / "fetch"), str(tmp_path / "write")))
    assert doc["calibration"]["read_scale"] == 2.0 and doc["calibration"]["write_scale"] == 1.0
    k = doc["kernels"]["fp8_e4m3_to_bf16"]
    assert k["hbm_read_bytes"] == 28672 * 1024 * 2 and k["hbm_write_bytes"] == 114688 * 1024
    assert k["algorithmic_bytes"] == 176160772
