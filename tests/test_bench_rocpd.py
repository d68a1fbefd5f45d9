"""The benchmark's rocprofv3 database summary (bench.py --rocpd-summary) on a
small database built here: kernel rows, counters per dispatch and their
spread over hardware instances, worked by hand."""
import os
import sqlite3
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def make_db(path):
    con = sqlite3.connect(path)
    c = con.cursor()
    c.execute("create table kernels (dispatch_id int, name text, grid_x int, start int, "
              "end int, stream_id int, queue_id int)")
    c.execute("create table pmc_events (dispatch_id int, name text, counter_name text, "
              "counter_value real)")
    c.execute("create table memory_copies (stream_id int, name text, size int, start int, "
              "end int)")
    k = "void kvx::(anonymous namespace)::block_copy_fast_kernel<unsigned int __vector(4)>(P)"
    c.executemany("insert into kernels values (?, ?, ?, ?, ?, ?, ?)",
                  [(1, k, 8388608, 0, 300000, 1, 0), (2, k, 8388608, 400000, 800000, 1, 0)])
    # Dispatch 1: a summed counter (one row) and a per-instance one (4 rows).
    rows = [(1, k, "TCC_EA0_WRREQ_sum", 400.0)]
    rows += [(1, k, "TCC_EA0_WRREQ", v) for v in (100.0, 100.0, 100.0, 100.0)]
    rows += [(2, k, "TCC_EA0_WRREQ", v) for v in (50.0, 150.0, 100.0, 100.0)]
    c.executemany("insert into pmc_events values (?, ?, ?, ?)", rows)
    c.executemany("insert into memory_copies values (?, ?, ?, ?, ?)",
                  [(2, "MEMORY_COPY_HOST_TO_DEVICE", 1000, 0, 100),
                   (3, "MEMORY_COPY_DEVICE_TO_HOST", 1000, 50, 150)])
    con.commit()
    con.close()


def test_summary_per_dispatch_and_instances(tmp_path, capsys):
    db = str(tmp_path / "t_results.db")
    make_db(db)
    bench.rocpd_summary(db)
    out = capsys.readouterr().out
    lines = out.splitlines()
    # Kernel rows: 2 calls of 300 and 400 us.
    krow = [l for l in lines if l.startswith("kvx::") and "8388608" in l and "calls" not in l]
    assert krow and krow[0].split()[-4:] == ["2", "350.00", "300.00", "400.00"], krow
    # Per dispatch: dispatch 1's summed counter is one instance; its
    # per-instance counter sums 400 over 4 equal instances (cv 0); dispatch
    # 2's four instances 50, 150, 100, 100: mean 100, std sqrt(1250), max/mean 1.5.
    per = [l.split() for l in lines
           if l.strip() and l.split()[0] in ("1", "2") and "TCC_" in l]
    got = {(int(t[0]), t[-7]): t[-6:] for t in per}
    assert got[(1, "TCC_EA0_WRREQ_sum")] == ["1", "400", "400", "400", "0.0000", "1.00"]
    assert got[(1, "TCC_EA0_WRREQ")] == ["4", "400", "100", "100", "0.0000", "1.00"]
    assert got[(2, "TCC_EA0_WRREQ")] == ["4", "400", "50", "150", "0.3536", "1.50"]
    # The two copies overlap for 50 of their 150 ns.
    assert "both directions at once" in out and "(33.3%)" in out
