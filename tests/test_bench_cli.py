"""bench.py without a GPU: more than one GPU is refused with an explanation
before anything touches the device, and the default line is the Llama-7B
tree (291 leaves, 6,738,415,616 params)."""

from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_workload_table_and_arguments():
    sys.path.insert(0, ROOT)
    try:
        import bench
    finally:
        sys.path.remove(ROOT)
    assert "llama7b" in bench.WORKLOADS and "llama7b_apply_rne" in bench.WORKLOADS
    # the default line is the Llama-7B fused step
    shapes = bench.llama7b_shapes()
    assert len(shapes) == 291
    assert sum(bench._numel(s) for _, s in shapes) == 6_738_415_616
