"""bench.py's command line on the host: the usual arguments parse, and a request for more than one GPU exits with a JSON line that says
the bench measures one GPU (nothing is launched)."""
from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "3", "--warmup", "1"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 1, r.stderr[-500:]
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_bench_arguments_parse():
    sys.path.insert(0, ROOT)
    import bench

    saved = sys.argv
    try:
        sys.argv = ["bench.py", "--gpus", "1", "--steps", "7", "--warmup", "2", "--no-cpu-baseline", "--no-ref-layer"]
        a = bench.parse()
    finally:
        sys.argv = saved
    assert (a.gpus, a.steps, a.warmup, a.workload) == (1, 7, 2, "pointer")
    assert a.no_cpu_baseline and a.no_ref_layer
