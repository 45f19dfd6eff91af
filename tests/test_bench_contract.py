"""CPU: the command-line contract of bench.py that the round-end driver relies on.

- `--gpus N` with N above 1 exits with status 2 and says why (this build runs on one GPU);
- with no GPU visible, bench.py exits with status 2 instead of falling back to the CPU;
- the argument parser accepts every workload the benchmark documents, with its defaults."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run(*args):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", CUDA_VISIBLE_DEVICES="-1")
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=300)


@pytest.mark.parametrize("n", [2, 8])
def test_multi_gpu_request_exits(n):
    r = _run("--gpus", str(n))
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.skipif(Path("/dev/kfd").exists(), reason="checks the behaviour on a host without a GPU driver")
def test_no_gpu_exits_without_fallback():
    r = _run("--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "GPU" in r.stderr and r.stdout == ""


def test_parser_defaults_and_workloads():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
    finally:
        sys.path.remove(str(ROOT))
    argv = sys.argv
    try:
        sys.argv = ["bench.py"]
        a = bench.parse()
        assert a.gpus == 1 and a.steps > 0 and a.warmup >= 0
        assert a.workload == "batched_paged_decode"
        for w in ("batched_paged_decode", "single_decode", "prefill", "multi_depth", "op_b", "pool_build", "d18"):
            sys.argv = ["bench.py", "--workload", w]
            assert bench.parse().workload == w
    finally:
        sys.argv = argv
