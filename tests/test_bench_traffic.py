"""bench.py's HBM-byte measurement harness on the CPU, against stand-in rocprofv3 scripts:
the counter file is parsed per dispatch, a run that overstays its limit is killed with the
program it profiles, and a missing profiler is an error the bench reports instead of
failing."""
import os
import stat
import sys
import textwrap
import time

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _fake_profiler(tmp_path, body):
    d = tmp_path / "bin"
    d.mkdir()
    p = d / "rocprofv3"
    p.write_text("#!/bin/bash\n" + textwrap.dedent(body))
    p.chmod(p.stat().st_mode | stat.S_IEXEC)
    return str(d)


def test_counter_file_parsed_per_dispatch(tmp_path, monkeypatch):
    # writes two dispatches of one counter (the second split over two rows, summed) and one
    # row of another counter, into the directory given after -d
    bindir = _fake_profiler(tmp_path, """
        while [ $# -gt 0 ]; do [ "$1" = "-d" ] && out=$2; shift; done
        mkdir -p "$out"
        {
          echo '"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"'
          echo '7,"k_a","FETCH_SIZE","100.5"'
          echo '9,"k_b","FETCH_SIZE","20"'
          echo '9,"k_b","FETCH_SIZE","22"'
          echo '9,"k_b","WRITE_SIZE","5"'
        } > "$out/p_counter_collection.csv"
        """)
    monkeypatch.setenv("PATH", bindir + os.pathsep + os.environ["PATH"])
    got = bench._pmc_child("FETCH_SIZE", "k_", ["--workload", "copy"], str(tmp_path / "o"))
    assert got == [("k_a", 100.5), ("k_b", 42.0)]


def test_overlong_run_is_killed_with_its_program(tmp_path, monkeypatch):
    pidfile = tmp_path / "child.pid"
    bindir = _fake_profiler(tmp_path, f"""
        sleep 300 &
        echo $! > {pidfile}
        wait
        """)
    monkeypatch.setenv("PATH", bindir + os.pathsep + os.environ["PATH"])
    t0 = time.time()
    with pytest.raises(RuntimeError, match="exceeded"):
        bench._pmc_child("FETCH_SIZE", "x", ["--workload", "copy"], str(tmp_path / "o"),
                         timeout=2)
    assert time.time() - t0 < 30
    pid = int(pidfile.read_text())
    # the profiled program went with the profiler's group: gone, or a zombie awaiting its
    # new parent's reaping
    for _ in range(50):
        try:
            with open(f"/proc/{pid}/status") as f:
                state = next(l for l in f if l.startswith("State:")).split()[1]
        except FileNotFoundError:
            state = "gone"
        if state in ("gone", "Z", "X"):
            break
        time.sleep(0.1)
    assert state in ("gone", "Z", "X"), state


def test_missing_profiler_is_an_error(tmp_path, monkeypatch):
    monkeypatch.setenv("PATH", str(tmp_path))
    with pytest.raises(RuntimeError, match="not on PATH"):
        bench._pmc_child("FETCH_SIZE", "x", ["--workload", "copy"], str(tmp_path / "o"))


def test_run_without_counters_is_an_error(tmp_path, monkeypatch):
    bindir = _fake_profiler(tmp_path, "echo 'error code 38' >&2; exit 3\n")
    monkeypatch.setenv("PATH", bindir + os.pathsep + os.environ["PATH"])
    with pytest.raises(RuntimeError, match="without counters"):
        bench._pmc_child("WRITE_SIZE", "x", ["--workload", "copy"], str(tmp_path / "o"))
