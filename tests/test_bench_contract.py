"""CPU tests of bench.py's contract with the driver (no GPU: the refusals come before torch is
imported) and of the byte accounting its headline metric rests on."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

import bench  # noqa: E402


def run(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env={**os.environ, "WORLD_SIZE": "1"})


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_invalid_step_counts_are_refused():
    assert run("--steps", "0").returncode == 2
    assert run("--warmup", "-1").returncode == 2


def test_algorithmic_bytes_of_a_linear():
    """Per GEMV: the trellis (k n bits / 8), x and y in fp16 (2 m k, 2 m n), suh and svh (2 k + 2 n)."""
    assert bench.algo_bytes(1, 5120, 1024, 4) == 5120 * 1024 // 2 + 2 * 5120 + 2 * 5120 + 2 * 1024 + 2 * 1024
    assert bench.algo_bytes(2, 256, 128, 3) == 256 * 128 * 3 // 8 + 4 * 256 + 512 + 256 + 4 * 128


def test_config1_step_bytes_and_shapes():
    """The config-1 layer: q / k / v / o / gate / up / down of a Qwen-27B-shaped decoder layer (hidden
    5120, 8 kv heads x 128, intermediate 17408); one step moves 165.6 MB at 4 bpw."""
    assert [(k, n) for _, k, n in bench.LAYER] == [(5120, 5120), (5120, 1024), (5120, 1024), (5120, 5120),
                                                   (5120, 17408), (5120, 17408), (17408, 5120)]
    step = sum(bench.algo_bytes(1, k, n, 4) for _, k, n in bench.LAYER)
    weights = sum(k * n for _, k, n in bench.LAYER)
    assert step == weights // 2 + sum(4 * k + 4 * n for _, k, n in bench.LAYER)
    assert 165.5e6 < step < 165.7e6
