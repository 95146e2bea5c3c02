"""bench.py's host-side contract, without a GPU: more than one GPU is refused
with a message and exit status 2 before any device work, and the workload
flags the profiles' commands use exist."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    res = _run("--gpus", "2")
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_workload_flags_exist():
    res = _run("--help")
    assert res.returncode == 0
    for flag in ("--attention-workload", "--shapes-workload", "--fused-workload", "--only-train", "--only-stack",
                 "--only-stream", "--copy-calibration", "--no-cpu-baseline"):
        assert flag in res.stdout, flag
