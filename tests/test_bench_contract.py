"""bench.py's command-line contract on the CPU: one GPU only (``--gpus N``
above 1, or a multi-rank launch, exits with a message and status 2, before
anything touches a device)."""

import os
import subprocess
import sys

import pytest

from conftest import REPO


@pytest.mark.parametrize("argv, env", [(["--gpus", "2"], {}), (["--gpus", "8", "--steps", "1"], {}),
                                       ([], {"WORLD_SIZE": "2"})])
def test_bench_refuses_more_than_one_gpu(argv, env):
    res = subprocess.run([sys.executable, str(REPO / "bench.py"), *argv], capture_output=True, text=True,
                         env=dict(os.environ, **env), timeout=120, cwd=REPO)
    assert res.returncode == 2, res.stderr
    assert "one GPU only" in res.stderr
    assert res.stdout == ""
