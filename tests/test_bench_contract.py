"""bench.py's command-line contract, checked without a GPU: it measures one
GPU only and says so for --gpus N > 1 (exit status 2, nothing on stdout),
and every workload name it accepts is one it can run."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert r.stdout == ""
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr


def test_workload_names():
    sys.path.insert(0, ROOT)
    import bench
    names = set(bench.WORKLOADS) | set(bench.PREFILL) | set(bench.FORK) | set(bench.E2E)
    assert {"qwen3", "qwen25", "qwen3_8b", "qwen3_8b_prefill", "qwen3_fork",
            "qwen3_e2e", "qwen25_e2e"} <= names
    r = _run("--workload", "no_such_workload")
    assert r.returncode != 0 and "invalid choice" in r.stderr
