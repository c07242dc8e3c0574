"""bench.py's profile readers on synthetic rocprofv3 databases (no GPU): the kernel-trace
summary and the PMC traffic reduction."""
import sqlite3
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _trace_db(path: Path, rows):
    c = sqlite3.connect(path)
    c.execute("create table kernels (name text, start integer, end integer, grid_x integer, "
              "grid_y integer, workgroup_x integer, vgpr_count integer, accum_vgpr_count "
              "integer, lds_size integer)")
    c.executemany("insert into kernels values (?,?,?,?,?,?,?,?,?)", rows)
    c.commit()
    c.close()


def test_ktrace_summary_runs_and_grouping(tmp_path):
    rows, t = [], 0

    def k(name, us, grid=(1024, 1)):
        nonlocal t
        rows.append((name, t, t + int(us * 1000), grid[0], grid[1], 256, 16, 0, 64))
        t += int(us * 1000) + 500

    # 3 isolated calls at 4 us, then a run of 60 at 2 us, then one torch kernel
    for _ in range(3):
        k("void fhip::rmsnorm_vec_kernel<fhip::TrF16, true, 1>(int)", 4.0)
        k("void at::native::fill_kernel(int)", 1.0)
    for _ in range(60):
        k("void fhip::rmsnorm_vec_kernel<fhip::TrF16, true, 1>(int)", 2.0)
    k("void at::native::fill_kernel(int)", 1.0)
    # one kernel over 6 grid sizes collapses into one row
    for g in range(6):
        k("void fhip::add_vec_kernel<fhip::TrF16>(int)", 3.0, (1000 + g, 1))
    _trace_db(tmp_path / "a_results.db", rows)
    md = bench.ktrace_summary(str(tmp_path)).splitlines()
    body = [line for line in md[2:]]
    assert len(body) == 2, md
    rms = next(line for line in body if "rmsnorm_vec_kernel" in line).split("|")
    cells = [c.strip() for c in rms[1:-1]]
    assert cells[1] == "63"
    assert float(cells[2]) == pytest.approx((3 * 4.0 + 60 * 2.0) / 63, abs=0.01)
    assert float(cells[3]) == pytest.approx(2.0)
    assert cells[12] == "60" and float(cells[13]) == pytest.approx(2.0)
    add = next(line for line in body if "add_vec_kernel" in line).split("|")
    assert add[7].strip() == "6 grids" and add[13].strip() == "0" and add[14].strip() == "-"
    assert not any("at::" in line for line in md)


def test_ktrace_summary_needs_a_database(tmp_path):
    with pytest.raises(SystemExit):
        bench.ktrace_summary(str(tmp_path))


def _pmc_db(path: Path, counter: str, rows):
    c = sqlite3.connect(path)
    c.execute("create table counters_collection (dispatch_id integer, kernel_name text, "
              "counter_name text, value real)")
    c.executemany("insert into counters_collection values (?,?,?,?)",
                  [(i, n, counter, v) for i, (n, v) in enumerate(rows)])
    c.commit()
    c.close()


def test_traffic_from_scales_by_the_calibration_copy(tmp_path):
    keys = [("op_a", 1000), ("op_b", 2000)]
    cal_kib = bench.CAL_BYTES / 1024.0
    for counter, half in (("FETCH_SIZE", 0.5), ("WRITE_SIZE", 1.0)):
        d = tmp_path / counter
        d.mkdir()
        rows = [("__amd_rocclr_copyBuffer", cal_kib * half),   # calibration
                ("__amd_rocclr_copyBuffer", 4 * half),        # marker of op_a
                ("op_a_kernel", 1.0 * half),
                ("op_a_kernel", 0.5 * half),
                ("__amd_rocclr_copyBuffer", 4 * half),        # marker of op_b
                ("op_b_kernel", 3.0 * half),
                ("__amd_rocclr_copyBuffer", 4 * half)]        # end marker
        _pmc_db(d / "pmc_results.db", counter, rows)
    t = bench.traffic_from(str(tmp_path / "FETCH_SIZE"), str(tmp_path / "WRITE_SIZE"), keys)
    assert t["op_a"]["dispatches"] == 2 and t["op_b"]["dispatches"] == 1
    assert t["op_a"]["fetch_size_bytes"] == 1536 and t["op_a"]["write_size_bytes"] == 1536
    assert t["op_b"]["bytes_per_dispatch"] == 2 * 3072
    assert t["op_b"]["traffic_over_algorithmic"] == pytest.approx(3.072)


def test_counters_summary_averages_per_kernel(tmp_path):
    a, b = tmp_path / "a", tmp_path / "b"
    a.mkdir()
    b.mkdir()
    c = sqlite3.connect(a / "pmc_results.db")
    c.execute("create table counters_collection (dispatch_id integer, kernel_name text, "
              "counter_name text, value real)")
    # two dispatches of one kernel, each reported by two hardware instances; a torch kernel
    c.executemany("insert into counters_collection values (?,?,?,?)", [
        (1, "void fhip::k1<4>(int)", "SQ_INSTS_LDS", 10.0),
        (1, "void fhip::k1<4>(int)", "SQ_INSTS_LDS", 5.0),
        (2, "void fhip::k1<4>(int)", "SQ_INSTS_LDS", 20.0),
        (2, "void fhip::k1<4>(int)", "SQ_INSTS_LDS", 5.0),
        (3, "void at::native::fill(int)", "SQ_INSTS_LDS", 99.0)])
    c.commit()
    c.close()
    _pmc_db(b / "pmc_results.db", "SQ_INSTS_MFMA", [("void fhip::k1<4>(int)", 7.0)])
    md = bench.counters_summary([str(a), str(b)]).splitlines()
    assert md[0] == "| kernel | dispatches | SQ_INSTS_LDS | SQ_INSTS_MFMA |"
    assert len(md) == 3 and "at::" not in "".join(md)
    cells = [x.strip() for x in md[2].split("|")[1:-1]]
    assert cells == ["`fhip::k1<4>`", "2", "20", "7"]
