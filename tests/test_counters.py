"""tiles_amd/counters.py: the HBM traffic summary bench.py reports as roofline.traffic, built from
synthetic rocprofv3 counter files whose answer is known."""

import csv
import json

from tiles_amd import counters

HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size", "Kernel_Id",
          "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
          "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_run(directory, counter, dispatches):
    directory.mkdir(parents=True)
    with open(directory / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEADER)
        for i, (name, value) in enumerate(dispatches, start=1):
            w.writerow([i, i, "Agent 1", 1, 1, 1, 1, 1, name, 256, 0, 0, 8, 0, 8, counter, value, 0, 1])


def test_summary_calibrates_and_prices_launches(tmp_path):
    mib = 256
    # Reference: FETCH_SIZE counts half of a nontemporal read (131072 KiB for 256 MiB); WRITE_SIZE all.
    write_run(tmp_path / "fref", "FETCH_SIZE", [("__amd_rocclr_fillBufferAligned", 10.0)] +
              [("tiles::stream_read(...)", 131072.0)] * 3)
    write_run(tmp_path / "wref", "WRITE_SIZE", [("__amd_rocclr_fillBufferAligned", 262144.0),
                                                ("tiles::stream_read(...)", 1.0)])
    worker = "void tiles::decoder_worker<true, 4, 8>(Launch<true>)"
    # A prefill, then two generate launches of 64 tokens each: fetch 80 GiB-counted, write 4 GiB.
    write_run(tmp_path / "fetch", "FETCH_SIZE", [(worker, 1.0e6), ("__amd_rocclr_copyBuffer", 5.0),
                                                 (worker, 80.0 * 2**20), (worker, 82.0 * 2**20)])
    write_run(tmp_path / "write", "WRITE_SIZE", [(worker, 7.0e4), (worker, 4.0 * 2**20), (worker, 4.0 * 2**20)])
    s = counters.summarize("ctx1", 1, 64, tmp_path / "fetch", tmp_path / "write", tmp_path / "fref", tmp_path / "wref", mib)
    assert s["calibration"]["fetch_bytes_per_kib"] == 2048.0
    assert s["calibration"]["write_bytes_per_kib"] == 1024.0
    assert len(s["launches"]) == 2
    fetched = (80.0 + 82.0) / 2 * 2**20 * 2048.0
    written = 4.0 * 2**20 * 1024.0
    assert s["traffic_bytes_per_launch"] == fetched + written
    # Algorithmic bytes: positions 1-64 and 65-128, weights once per token and K/V of 0..p.
    first = sum(counters.algorithmic_bytes(p) for p in range(1, 65))
    second = sum(counters.algorithmic_bytes(p) for p in range(65, 129))
    assert s["algorithmic_bytes_per_launch"] == (first + second) / 2
    assert counters.algorithmic_bytes(0) == 2_471_628_800 + 32_768


def test_load_rejects_a_summary_of_other_sources(tmp_path):
    path = tmp_path / "traffic.json"
    entry = {"source_sha256": counters.kernel_source_sha256(), "traffic_bytes_per_launch": 1.0}
    path.write_text(json.dumps({"ctx1": entry, "ctx4096": {**entry, "source_sha256": "0" * 64}}))
    assert counters.load(path, "ctx1") == entry
    assert counters.load(path, "ctx4096") is None
    assert counters.load(path, "ctx32768") is None
    assert counters.load(tmp_path / "missing.json", "ctx1") is None
