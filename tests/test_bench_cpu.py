"""bench.py's contract on the CPU: more than one GPU is refused before any device work."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

from tests._util import ROOT


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8", "--steps", "5"], {}),
                                      ([], {"WORLD_SIZE": "4"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], cwd=str(ROOT), capture_output=True,
                         text=True, timeout=300, env=dict(os.environ, **env))
    assert res.returncode == 2, res.stderr[-2000:]
    assert "one MI355X" in res.stderr and res.stdout == ""
