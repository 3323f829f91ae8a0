"""CPU checks of bench.py's command line: more than one GPU is refused with a
message and exit status 2 before anything touches a device."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8", "--steps", "5"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], cwd=ROOT, capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=120)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line
