"""bench.py's command line, on the CPU: the driver's contract (one GPU; more exits with a
message before any GPU work) and the workload flags parse."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and r.stdout == ""


def test_workload_flags_parse(monkeypatch):
    cases = [
        (["--workload", "lmstep", "--lm", "3b", "--residuals", "standard,attnres"],
         {"workload": "lmstep", "lm": "3b", "residuals": "standard,attnres", "graph": False}),
        (["--workload", "cfg1btrain", "--graph", "--steps", "4", "--warmup", "1"],
         {"workload": "cfg1btrain", "graph": True, "steps": 4, "warmup": 1}),
        (["--workload", "narrow"], {"workload": "narrow", "gpus": 1}),
        ([], {"workload": "cfg2", "gpus": 1, "steps": 20, "warmup": 3, "pass_": "fwd"}),
    ]
    for argv, want in cases:
        monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
        args = bench.parse_args()
        for k, v in want.items():
            assert getattr(args, k) == v, (argv, k)
    assert {"lmstep", "narrow", "cfg1btrain", "cfg2train", "cfg3train", "segsum"} <= set(bench.WORKLOAD_TEXT)
