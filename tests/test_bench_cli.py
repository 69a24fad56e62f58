"""bench.py's command line on the CPU: more than one GPU is refused with a
message (this build runs on exactly one), and the option set the driver
and the profiles' commands use parses."""

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, timeout=120)
    assert result.returncode == 2
    line = json.loads(result.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_profile_commands_parse():
    sys.path.insert(0, str(ROOT))
    import bench

    argv = sys.argv
    try:
        for args in (["--no-cpu-baseline", "--no-prefill", "--no-mixed", "--no-reference-shape",
                      "--steps", "50", "--warmup", "10"],
                     ["--prefill-only", "--prefill-steps", "2"],
                     ["--mixed-only", "--mixed-steps", "40"]):
            sys.argv = ["bench.py", *args]
            parsed = bench.parse()
            assert parsed.gpus == 1
    finally:
        sys.argv = argv
