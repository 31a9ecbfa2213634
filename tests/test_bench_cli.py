"""bench.py's command-line contract, checked without a GPU: one GPU only (--gpus above 1
exits with status 2 and a JSON line naming the reason, before touching the device), and
the workloads it offers."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"] and line["metric"]
    assert "one GPU" in r.stderr


def test_workloads_listed():
    r = _run("--help")
    assert r.returncode == 0
    for w in ("ef", "single-linear", "tied-output", "llama3-8b-layer", "perm-search",
              "formats", "gguf", "copy", "sweep-pass", "hessian-power"):
        assert w in r.stdout
