"""The reference's run_missstream driver, rebuilt over include/ferry/ferry.hpp,
run end to end on the GPU with the reference's own golden command lines."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "ferry_amd", "run_missstream")


def test_driver_rejects_unknown_flags():
    if not os.path.exists(BIN):
        pytest.skip("run_missstream not built")
    res = subprocess.run([BIN, "--no-such-flag"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "unknown flag" in res.stderr


def _run(args):
    print("[driver]", " ".join(args), flush=True)
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0
    return res.stdout


@pytest.mark.gpu
def test_driver_golden_default_stream():
    # results/wla_7rep_20260930/*.log: selects 589,824, misses 79,550, hit 0.865,
    # refill 1242.97 MB in modes B and C.
    out = _run(["--requests", "48", "--layers", "12", "--steps", "16", "--sel", "64", "--hot", "1"])
    assert "selects=589824 miss=79550 hit_rate=0.865 miss_bytes=1242.97MB" in out
    for mode in ("baseline-B", "ferry-C"):
        row = re.search(mode + r".*refill=\s*(\d+) bytes=\s*([\d.]+)MB status=(-?\d+)", out)
        assert row and row.group(1) == "79550" and row.group(2) == "1242.97" and row.group(3) == "0"


@pytest.mark.gpu
def test_driver_golden_single_gpu_run():
    # 实验设计.txt:494-495: 4 req x 12 layers x 4 steps, sel 128, hot 1024 -> 57.66 MB.
    out = _run(["--requests", "4", "--layers", "12", "--steps", "4", "--sel", "128", "--hot", "4"])
    assert "miss=3690" in out and "miss_bytes=57.66MB" in out
    assert re.search(r"ferry-C .*refill=\s*3690 bytes=\s*57.66MB status=0", out)
