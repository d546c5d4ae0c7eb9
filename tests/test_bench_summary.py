"""bench.py's rocprofv3 summary (the text under profiles/ and the traffic the
bench line reports): a kernel's full-size dispatches are kept apart from the
short ones (the parity leg runs the decode kernel one layer at a time beside
the whole-step launches), and FETCH_SIZE / WRITE_SIZE of the decode kernel
are scaled by the calibration copy's reading of the same counter."""
import csv
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summary_separates_full_size_dispatches(tmp_path):
    run = tmp_path / "run" / "box"
    run.mkdir(parents=True)
    chain = "void smoe::k_moe_chain<1, 2, 5, 8, 6, 4, 0>(smoe::MoeDims)"
    write_csv(run / "kt_kernel_trace.csv", ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"],
              [[1, chain, 1000, 547000], [2, chain, 0, 14000], [3, chain, 0, 549000],
               [4, "neg_kernel", 0, 100]])
    # two rows of one dispatch are summed; the 12 000 KiB one-layer call is left out of the full-size figure
    write_csv(run / "x_counter_collection.csv", ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"],
              [[1, chain, "FETCH_SIZE", 300000], [1, chain, "FETCH_SIZE", 293000], [2, chain, "FETCH_SIZE", 12000],
               [3, chain, "FETCH_SIZE", 593000], [4, "at::native::neg_kernel_cuda", "FETCH_SIZE", 131072]])
    out = tmp_path / "pmc.json"
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--rocprof-summary", str(tmp_path / "run"),
                        "--pmc-out", str(out), "--calibrate-copy-mib", "256"],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    full = [l for l in lines if "k_moe_chain" in l and l.split()[0] == "2"]
    assert full and float(full[0].split()[1]) == 547.5     # (546 + 549) / 2 us over the two whole-step launches
    data = json.load(open(out))
    ent = data["qwen3-30b-a3b-moe-decode-stack"]["k_moe_chain"]
    assert ent["FETCH_SIZE_kib"] == 593000.0
    assert data["_calibration"]["FETCH_SIZE"]["scale"] == 2.0        # 262144 KiB expected, 131072 read
    assert ent["FETCH_SIZE_bytes_scaled"] == 593000 * 1024 * 2
