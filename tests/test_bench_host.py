"""bench.py's command-line contract, on the CPU: more than one GPU is refused
with a message (every box here has one GPU), and the defaults are the headline
run (one GPU, 50 warmup and 100 timed steps, the block-linears workload)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=120)


def test_more_than_one_gpu_is_refused():
    for n in ("2", "8"):
        r = run_bench("--gpus", n, "--steps", "1", "--warmup", "0")
        assert r.returncode == 2
        assert "one GPU" in r.stderr and f"--gpus {n}" in r.stderr
        assert r.stdout == ""                      # no JSON line


def test_defaults_are_the_headline_run():
    r = run_bench("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--cpu-seconds", "--path", "--workload"):
        assert flag in r.stdout
    with open(os.path.join(ROOT, "bench.py")) as f:
        src = f.read()
    assert 'ap.add_argument("--gpus", type=int, default=1)' in src
    assert 'ap.add_argument("--steps", type=int, default=100)' in src
    assert 'ap.add_argument("--warmup", type=int, default=50)' in src
    assert 'default="block-linears"' in src and 'default="bf6"' in src
