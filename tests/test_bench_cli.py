"""bench.py's command line on a host without a GPU: more than one GPU is refused with a message
that says the build measures one GPU (exit 2), and a run without a device fails loudly (exit
1) instead of timing anything."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          env=env, capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "1")
    assert r.returncode == 2, r.stderr
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_no_device_fails_loudly():
    r = _run("--steps", "1", "--warmup", "1")
    assert r.returncode == 1, r.stderr
    assert "needs a GPU" in r.stderr
    assert r.stdout.strip() == ""
