"""The rocprofv3 summaries (pathtile_amd/profiling.py) on hand-made results
databases with the rocpd tables the reports read: the arithmetic of each
report, and that the small correctness-gate dispatches are left out."""

import sqlite3

import pytest

from pathtile_amd import profiling

K_MAIN = "void pt::dwconv_rows_cg_kernel<48, false, 2, 16>(float const*, float*)"
K_IDLE = "void pt::fill_zero_kernel(float*, int)"
COPY = profiling.COPY_KERNEL


def _db(path, counters=(), kernels=()):
    con = sqlite3.connect(path)
    con.execute("create table counters_collection (kernel_name text, dispatch_id int, "
                "grid_size int, counter_name text, value real)")
    con.execute("create table kernels (name text, duration real, grid_x int, grid_y int, "
                "grid_z int, workgroup_x int, workgroup_y int, workgroup_z int, lds_size int, "
                "scratch_size int, vgpr_count int, accum_vgpr_count int, sgpr_count int)")
    con.executemany("insert into counters_collection values (?, ?, ?, ?, ?)", counters)
    con.executemany("insert into kernels values (?, ?, ?, 1, 1, ?, 1, 1, ?, 0, ?, ?, ?)", kernels)
    con.commit()
    con.close()
    return str(path)


def _row(text, name):
    line = next(l for l in text.splitlines() if l.startswith(f"| `{name}`"))
    return [c.strip() for c in line.strip("|").split("|")]


def test_lds_report(tmp_path):
    gui = 8 * 1000.0  # 1000 cycles per XCD
    main = {"SQ_WAVES": 100, "SQ_INSTS_LDS": 500, "SQ_LDS_IDX_ACTIVE": 256 * 1000 * 0.25,
            "SQ_LDS_BANK_CONFLICT": 256 * 1000 * 0.25 * 0.1, "SQ_WAIT_INST_LDS": 40,
            "SQ_WAVE_CYCLES": 800, "GRBM_GUI_ACTIVE": gui}
    rows = []
    for d in range(3):  # three timed dispatches, one small gate dispatch
        rows += [(K_MAIN, d, 4096, c, v) for c, v in main.items()]
    rows += [(K_MAIN, 9, 64, c, 1.0) for c in main]
    # a kernel without LDS instructions is not listed
    rows += [(K_IDLE, 10, 96, c, 0.0 if c == "SQ_INSTS_LDS" else 5.0) for c in main]
    text = profiling.lds_report(_db(tmp_path / "l.db", rows), "cmd")
    r = _row(text, "pt::dwconv_rows_cg_kernel<48, false, 2, 16>")
    assert r[1:] == ["3", "100", "5", "0.250", "0.100", "0.050"]
    assert "fill_zero_kernel" not in text


def test_valu_report(tmp_path):
    gui = 8 * 2400.0  # 2400 cycles per XCD: 1 us at 2400 MHz
    vals = {"SQ_WAVES": 64, "SQ_INSTS_VALU": 6400, "SQ_ACTIVE_INST_VALU": 1024 * 2400 * 0.5 / 4,
            "SQ_BUSY_CYCLES": 1, "GRBM_GUI_ACTIVE": gui, "SQ_WAVE_CYCLES": 1,
            "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 2400 * 0.25}
    rows = [(K_MAIN, 0, 4096, c, v) for c, v in vals.items()]
    fma = int(profiling.PEAK_FP32_VECTOR * 1e-6 / 2 / 4)  # a quarter of the vector peak
    text = profiling.valu_report(_db(tmp_path / "v.db", rows), "cmd",
                                 {"dwconv_rows_cg_kernel<48": fma}, 2400.0)
    r = _row(text, "pt::dwconv_rows_cg_kernel<48, false, 2, 16>")
    assert r[1:7] == ["1", "64", "6400", "100", "0.500", "0.250"]
    assert float(r[8]) == pytest.approx(0.25, abs=1e-3)
    assert float(r[9]) == pytest.approx(0.25 * 78.6 / 157.3, abs=1e-3)


def test_traffic_report_scales_by_the_copy_probe(tmp_path):
    copy_bytes = 1 << 20
    # FETCH_SIZE reads half the bytes a copy loads; WRITE_SIZE reads them exactly
    fetch = [(COPY, 0, 1 << 16, "FETCH_SIZE", copy_bytes / 2 / 1024),
             (K_MAIN, 1, 4096, "FETCH_SIZE", 3000.0), (K_MAIN, 2, 4096, "FETCH_SIZE", 3200.0),
             (K_MAIN, 3, 64, "FETCH_SIZE", 1.0)]
    write = [(COPY, 0, 1 << 16, "WRITE_SIZE", copy_bytes / 1024),
             (K_MAIN, 1, 4096, "WRITE_SIZE", 6000.0), (K_MAIN, 2, 4096, "WRITE_SIZE", 6000.0)]
    text = profiling.traffic_report(_db(tmp_path / "f.db", fetch), _db(tmp_path / "w.db", write),
                                    "dwconv_rows_cg_kernel<48", "fwd", 12_000_000, copy_bytes,
                                    "cmd")
    fetch_b = 3100.0 * 1024 * 2.0
    write_b = 6000.0 * 1024 * 1.0
    assert f"FETCH_BYTES_PER_LAUNCH: {fetch_b:.0f}" in text
    assert f"WRITE_BYTES_PER_LAUNCH: {write_b:.0f}" in text
    assert f"measured/algorithmic = {(fetch_b + write_b) / 12_000_000:.4f}" in text


def test_trace_report_drops_gate_dispatches(tmp_path):
    k = [(K_MAIN, 130_000.0, 4096, 1024, 150000, 80, 40, 30),
         (K_MAIN, 134_000.0, 4096, 1024, 150000, 80, 40, 30),
         (K_MAIN, 9_000.0, 256, 1024, 150000, 80, 40, 30)]
    text = profiling.trace_report(_db(tmp_path / "t.db", kernels=k), "cmd")
    r = _row(text, "pt::dwconv_rows_cg_kernel<48, false, 2, 16>")
    assert r[1:3] == ["2", "132.00"]


def test_mix_report(tmp_path):
    vals = {"SQ_INSTS_VALU": 1000, "SQ_INSTS_VALU_FMA_F32": 400, "SQ_INSTS_VALU_ADD_F32": 100,
            "SQ_INSTS_VALU_MUL_F32": 50, "SQ_INSTS_VALU_INT32": 200, "SQ_INSTS_VALU_CVT": 10,
            "SQ_INSTS_VALU_MFMA_F32": 90, "SQ_INSTS_VALU_MFMA_BF16": 30}
    rows = [(K_MAIN, d, 4096, c, v) for d in range(2) for c, v in vals.items()]
    rows += [(K_MAIN, 5, 64, c, 1.0) for c in vals]
    text = profiling.mix_report(_db(tmp_path / "m.db", rows), "cmd")
    r = _row(text, "pt::dwconv_rows_cg_kernel<48, false, 2, 16>")
    assert r[1:] == ["2", "1000", "0.550", "0.400", "0.100", "0.050", "0.200", "0.010", "0.120"]


def test_stall_report_merges_passes(tmp_path):
    """Occupancy, wait shares, MemUnitStalled, DRAM-credit stall shares and
    the UTCL1 miss rate, from two counter passes of one run (labelled) and
    one counter of another run."""
    gui = 8 * 1000.0  # 1000 cycles per XCD
    pass_a = {"MeanOccupancyPerCU": 6.0, "SQ_WAVE_CYCLES": 1000.0, "SQ_WAIT_ANY": 700.0,
              "SQ_WAIT_INST_ANY": 200.0, "MemUnitStalled": 12.5}
    pass_b = {"GRBM_GUI_ACTIVE": gui,
              "TCC_EA0_RDREQ_DRAM_CREDIT_STALL_sum": 128 * 1000 * 0.25,
              "TCC_EA0_WRREQ_DRAM_CREDIT_STALL_sum": 128 * 1000 * 0.5,
              "TCP_UTCL1_TRANSLATION_MISS_sum": 10.0, "TCP_UTCL1_TRANSLATION_HIT_sum": 990.0}
    rows_a, rows_b = [], []
    for d in range(2):
        rows_a += [(K_MAIN, d, 4096, c, v) for c, v in pass_a.items()]
        rows_b += [(K_MAIN, d, 4096, c, v) for c, v in pass_b.items()]
    rows_a += [(K_MAIN, 9, 64, c, 1.0) for c in pass_a]  # gate dispatch: dropped
    other = [(K_MAIN, 0, 4096, "MeanOccupancyPerCU", 3.0)]
    text = profiling.stall_report(
        [_db(tmp_path / "a.db", rows_a), _db(tmp_path / "b.db", rows_b),
         _db(tmp_path / "c.db", other)], "cmd", labels=["slow", "slow", "fast"])
    lines = [l for l in text.splitlines() if "dwconv_rows_cg_kernel" in l]
    cells = {l.split("|")[1].strip(): [c.strip() for c in l.strip("|").split("|")] for l in lines}
    assert cells["slow"][2:] == ["2", "6.00", "1.50", "0.700", "0.200", "12.5", "0.250",
                                 "0.500", "0.0100"]
    assert cells["fast"][2:] == ["1", "3.00", "0.75", "-", "-", "-", "-", "-", "-"]
