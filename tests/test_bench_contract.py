"""bench.py's command-line contract on the CPU: it measures one GPU and exits
with status 2 and a message for a multi-GPU request or a bad step count,
before touching a device."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          env=e, capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""          # no JSON line


def test_world_size_above_one_is_refused():
    r = _run(env={"WORLD_SIZE": "2"})
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU only" in r.stderr


def test_zero_steps_is_refused():
    r = _run("--steps", "0")
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "--steps" in r.stderr
