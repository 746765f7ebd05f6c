"""The rocprofv3 summary tool on a small database of its two views."""
import sqlite3

from dwim_amd import rocprof_summary as R


def _db(path):
    c = sqlite3.connect(path)
    c.execute("create table kernels (name text, grid_x int, start int, end int)")
    c.execute("create table counters_collection (kernel_name text, grid_size int, counter_name text, value real, "
              "dispatch_id int)")
    t = 0
    for case, us in enumerate((10, 30)):  # two cases of 3 calls each, then one other kernel
        for _ in range(3):
            c.execute("insert into kernels values (?, ?, ?, ?)", ("k_a(int)", 256, t, t + us * 1000))
            c.execute("insert into counters_collection values (?, ?, ?, ?, ?)", ("k_a(int)", 256, "FETCH_SIZE",
                                                                              100.0 * (case + 1), t))
            t += 100000
    c.execute("insert into kernels values (?, ?, ?, ?)", ("k_b(int)", 64, t, t + 5000))
    c.commit()
    return path


def test_trace_and_pmc_summaries(tmp_path):
    db = _db(str(tmp_path / "run_results.db"))
    out = R.trace(db, 10, None)
    assert "6   " in out.splitlines()[1] and "20.00" in out  # k_a: 6 calls, mean 20 us
    assert "all kernels: 7 dispatches" in out
    split = R.trace(db, 10, "k_a", split=3).splitlines()
    assert "10.00" in split[1] and "[group 0]" in split[1]
    assert "30.00" in split[2] and "[group 1]" in split[2]
    after = R.trace(db, 10, None, after="k_a")
    assert "k_b" in after and "k_a" not in after.splitlines()[1]
    p = R.pmc(db, "k_a", split=3).splitlines()
    assert "100.00" in p[1] and "[group 0]" in p[1]
    assert "200.00" in p[2] and "[group 1]" in p[2]
