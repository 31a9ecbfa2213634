"""bench.py's JSON line keeps its contract: run in this process (main() with a small
argument list: 2 layers, one step) and check every field the line must carry."""
import json
import os
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEYS = {"metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
        "scaling", "vs_baseline", "dtype", "data", "config"}


def _run(monkeypatch, capsys, *args):
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench
    monkeypatch.setattr(sys, "argv", ["bench.py", *args])
    bench.main()
    out = capsys.readouterr().out.strip().splitlines()
    return json.loads(out[-1])


def test_ef_line(monkeypatch, capsys):
    r = _run(monkeypatch, capsys, "--layers", "2", "--steps", "1", "--warmup", "0",
             "--no-cpu-baseline")
    assert KEYS <= set(r) and r["n_gpus"] == 1 and r["steps"] == 1 and r["warmup"] == 0
    assert r["value"] > 0 and r["higher_is_better"] is True and r["vs_baseline"] is None
    assert "workload" in r["config"] and "model" not in r["config"]
    roof = r["roofline"]
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(roof)
    assert roof["bound"] in ("hbm", "mfma") and 0 < roof["frac"] < 1
    # measured by the bench's own counter runs of the same (2-layer) workload, or null
    # when they could not run; every sweep kernel of the pass is counted
    if roof["traffic"] is not None:
        d = roof["traffic_detail"]
        assert roof["traffic"] > 0
        assert len(d["fetch_bytes_per_launch"]) == len(d["write_bytes_per_launch"]) == 6
    else:
        assert roof.get("traffic_detail") is None or "error" in roof["traffic_detail"]


def test_perm_search_line(monkeypatch, capsys):
    r = _run(monkeypatch, capsys, "--workload", "perm-search", "--layers", "2", "--steps", "1",
             "--warmup", "0", "--no-cpu-baseline")
    assert KEYS <= set(r) and r["value"] > 0
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(r["roofline"])
