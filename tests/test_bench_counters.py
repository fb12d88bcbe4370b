"""bench.py's counter summary (summarize_pmc): per-kernel means over
dispatches, FETCH_SIZE / WRITE_SIZE scaled by the copy probe of the same run,
MFMA flops from the MOPS counters. Runs on synthetic rocprofv3-shaped
databases (no GPU)."""
import json
import os
import sqlite3
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def _db(path, rows):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    con = sqlite3.connect(path)
    con.execute("create table counters_collection (dispatch_id int, kernel_name text, counter_name text, value real,"
                " grid_size_x int, grid_size_y int, grid_size_z int, workgroup_size_x int, workgroup_size_y int,"
                " workgroup_size_z int)")
    con.executemany("insert into counters_collection values (?, ?, ?, ?, 32768, 2, 1, 1024, 1, 1)", rows)
    con.commit()
    con.close()


def test_summarize_pmc(tmp_path):
    import bench
    kib = bench.COPY_PROBE_BYTES / 1024
    # the probe reads half of its bytes in FETCH_SIZE units (factor 2), writes 1:1
    _db(str(tmp_path / "fetch_c1" / "run_results.db"),
        [(1, "qff::dn_chunk_state_kernel(int, float*)", "FETCH_SIZE", 1000.0),
         (2, "qff::dn_chunk_state_kernel(int, float*)", "FETCH_SIZE", 3000.0),
         (3, "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)>(...)", "FETCH_SIZE", kib / 2)])
    _db(str(tmp_path / "write_c1" / "run_results.db"),
        [(1, "qff::dn_chunk_state_kernel(int, float*)", "WRITE_SIZE", 500.0),
         (3, "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)>(...)", "WRITE_SIZE", kib)])
    _db(str(tmp_path / "mfma_c1" / "run_results.db"),
        [(1, "qff::dn_chunk_state_kernel(int, float*)", "SQ_INSTS_VALU_MFMA_MOPS_BF16", 10.0),
         (1, "qff::dn_chunk_state_kernel(int, float*)", "SQ_INSTS_VALU_MFMA_MOPS_F32", 2.0),
         (1, "qff::dn_chunk_state_kernel(int, float*)", "MfmaUtil", 12.5)])
    out = tmp_path / "c.json"
    res = bench.summarize_pmc(str(tmp_path), str(out))
    rec = res["workloads"]["c1"]["dn_chunk_state@32.2.1/1024"]
    assert rec["FETCH_SIZE"] == 2000.0 and rec["dispatches"]["fetch"] == 2
    assert abs(rec["read_bytes"] - 2000.0 * 1024 * 2) < 1e-6
    assert abs(rec["write_bytes"] - 500.0 * 1024) < 1e-6
    assert rec["traffic_bytes"] == rec["read_bytes"] + rec["write_bytes"]
    assert rec["mfma_flops"] == 12.0 * 512 and rec["mfma_util_pct"] == 12.5
    assert json.load(open(out))["workloads"]["c1"]["dn_chunk_state@32.2.1/1024"]["traffic_bytes"] == rec["traffic_bytes"]
