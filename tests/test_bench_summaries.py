"""The profile summaries bench.py writes from rocprofv3 databases (host logic, no GPU): dispatch
selection by kernel, grid and launch-order range, on small synthetic databases with the tables
and columns rocprofv3 writes."""

import sqlite3

import bench


def _trace_db(path, dispatches):
    con = sqlite3.connect(path)
    con.execute("create table kernels (name text, start int, duration int, grid_x int, grid_y int, "
                "grid_z int, workgroup_x int, workgroup_y int, workgroup_z int)")
    for i, (name, wgs, dur) in enumerate(dispatches):
        con.execute("insert into kernels values (?, ?, ?, ?, 1, 1, 512, 1, 1)",
                    (name, i * 1000, dur, wgs * 512))
    con.commit()
    con.close()


def test_grid_sel_parses_grids_and_ranges():
    assert bench._grid_sel("hgemm_kernel<false, 0") == ("hgemm_kernel<false, 0", None, None)
    assert bench._grid_sel("k#240,3072") == ("k", {240, 3072}, None)
    assert bench._grid_sel("k#192[3:6]") == ("k", {192}, (3, 6))


def test_pick_keeps_launch_order_within_the_range():
    rows = {(5, "k", 192, 512): 5.0, (1, "k", 192, 512): 1.0, (3, "k", 256, 512): 3.0,
            (2, "other", 192, 512): 2.0, (4, "k", 192, 512): 4.0}
    assert [v for _, v in bench._pick(rows, "k", {192}, None)] == [1.0, 4.0, 5.0]
    assert [v for _, v in bench._pick(rows, "k", {192}, (1, 3))] == [4.0, 5.0]
    assert [v for _, v in bench._pick(rows, "k", None, (0, 2))] == [1.0, 3.0]


def test_opavg_strided_range_separates_two_operators(tmp_path):
    # two operators alternate on one kernel and grid (o forward, then down forward, per layer),
    # after two untimed dispatches of each
    seq = []
    for layer in range(6):
        seq.append(("dk::hgemm_kernel<false, 0, false>(p)", 192, 17000))
        seq.append(("dk::hgemm_kernel<false, 0, false>(p)", 192, 61000))
    seq.append(("nf4_dequant_kernel(x)", 714, 19000))
    db = str(tmp_path / "t.db")
    _trace_db(db, seq)
    out = bench.summarize_trace(db, ops=[("o", "hgemm_kernel<false, 0, false>", 192, (4, 12, 2)),
                                         ("down", "hgemm_kernel<false, 0, false>", 192, (5, 12, 2)),
                                         ("dq", "nf4_dequant_kernel", 714, None)])
    lines = {l.split(" | ")[0]: l for l in out.splitlines() if l.startswith("OPAVG")}
    assert lines["OPAVG o"].endswith("| 17.00 | 4")
    assert lines["OPAVG down"].endswith("| 61.00 | 4")
    assert lines["OPAVG dq"].endswith("| 19.00 | 1")
