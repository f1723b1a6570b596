"""bench.py's command-line contract, without a GPU.

A benchmark harness runs `python bench.py --gpus N --steps K --warmup W`; bench.py measures one
GPU, so any other N must end with a message and a nonzero status before the GPU is touched.
"""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(REPO, "bench.py")


def run(*args, env=None):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True,
                          timeout=120, env=env, cwd=REPO)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_torchrun_world_size_is_refused():
    env = dict(os.environ, WORLD_SIZE="8")
    r = run("--gpus", "1", env=env)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_help_lists_the_driver_flags():
    r = run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--config"):
        assert flag in r.stdout


def test_flop_count_matches_the_reference_formula():
    # 4 B Hq N^2 D for full attention, half of it under the causal mask.
    sys.path.insert(0, REPO)
    import bench

    assert bench.flops(1, 32, 8192, 128, False) == 4 * 32 * 8192 ** 2 * 128
    assert bench.flops(1, 32, 8192, 128, True) == 2 * 32 * 8192 ** 2 * 128
