"""bench.py's command-line contract on the CPU: one GPU only (a run with more
GPUs, or under a launcher with WORLD_SIZE > 1, stops with a message and exit
code 2 before touching a device), and the refusal to run without a GPU."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, 'bench.py')


def run(*args, env=None):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=300,
                          env={**os.environ, **(env or {})})


def test_more_than_one_gpu_is_refused():
    r = run('--gpus', '2', '--steps', '1', '--warmup', '0')
    assert r.returncode == 2
    assert 'one GPU' in r.stderr
    assert r.stdout == ''


def test_world_size_above_one_is_refused():
    r = run('--steps', '1', env={'WORLD_SIZE': '2'})
    assert r.returncode == 2
    assert 'one GPU' in r.stderr


def test_no_gpu_is_refused():
    # this container has no GPU: the bench stops before any timing
    r = run('--steps', '1', '--warmup', '0', '--no-extras', '--no-cpu-baseline', env={'HIP_VISIBLE_DEVICES': ''})
    assert r.returncode == 2
    assert 'needs a ROCm GPU' in r.stderr
