"""bench.py's command-line contract on the CPU: a run asked for more than one
GPU (by flag or by a torchrun environment) exits with status 2 and a message
before anything touches torch or the GPU."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _bench(args, env_extra=None):
    env = dict(os.environ)
    env.pop("WORLD_SIZE", None)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args],
                          capture_output=True, text=True, env=env, timeout=60)


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_refused(n):
    out = _bench(["--gpus", str(n), "--steps", "1", "--warmup", "0"])
    assert out.returncode == 2
    assert "one GPU" in out.stderr
    assert out.stdout == ""


def test_torchrun_world_refused():
    out = _bench(["--steps", "1"], {"WORLD_SIZE": "4"})
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_help_lists_phases():
    out = _bench(["--help"])
    assert out.returncode == 0
    for phase in ("roofline", "decode", "counters", "batch"):
        assert phase in out.stdout
