"""bench.py's command line on the CPU: the one-GPU contract (a request for
more GPUs exits with status 2 and says why, before touching a device) and
the measurement flags."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line


def test_help_lists_the_protocol_flags():
    r = subprocess.run([sys.executable, BENCH, "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for flag in ("--steps", "--warmup", "--prewarm-ms", "--copies", "--no-cpu-baseline",
                 "--no-long-decode", "--no-short-decode", "--no-stepwise-prefill"):
        assert flag in r.stdout, flag
