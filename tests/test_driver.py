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


WLA = os.path.join(ROOT, "ferry_amd", "run_wla")


def test_wla_driver_rejects_bad_flags():
    if not os.path.exists(WLA):
        pytest.skip("run_wla not built")
    res = subprocess.run([WLA, "--no-such-flag"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "unknown flag" in res.stderr
    res = subprocess.run([WLA, "--gpus", "0,1"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "one GPU" in res.stderr


def _rows(out):
    rows = {}
    for m in re.finditer(r"^\s+([ABC])\s+makespan=.*refill=\s*(\d+) seg\s+([\d.]+)MB hit=([\d.]+) "
                         r"ticks=(\d+) status=(-?\d+)", out, re.M):
        rows[m.group(1)] = (int(m.group(2)), m.group(3), float(m.group(4)), int(m.group(5)),
                            int(m.group(6)))
    return rows


def _run_wla(args, env=None):
    print("[run_wla]", " ".join(args), flush=True)
    res = subprocess.run([WLA, *args], capture_output=True, text=True, timeout=300,
                         env=dict(os.environ, **(env or {})))
    print(res.stdout[-3000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0
    return res.stdout


@pytest.mark.gpu
def test_wla_slice_default_stream_with_bursty_arrivals():
    # The reference's default stream through the per-GPU tick loop: requests
    # arrive in bursts and run interleaved, but each has its own hot cache, so
    # modes B and C refill exactly the replay's 79,550 misses (1242.97 MB).
    out = _run_wla(["--requests", "48", "--layers", "12", "--steps", "16", "--sel", "64",
                    "--hot", "128", "--arrival", "bursty", "--gap", "0.2"])
    rows = _rows(out)
    for mode in "BC":
        assert rows[mode][0] == 79550 and rows[mode][1] == "1242.97" and rows[mode][4] == 0
        assert round(rows[mode][2], 3) == 0.865
    assert rows["A"][4] == 0 and rows["A"][0] > rows["C"][0]


@pytest.mark.gpu
def test_wla_slice_prefix_groups_match_oracle():
    # C2 prefix groups (wla_multigpu.cuh:355-369): members repeat their head's
    # selections for 8 steps and share the group's LRU, touched member after
    # member within a tick (:2643-2648).  With a virtual clock the tick
    # composition is fixed, and the oracle replays the same ticks.
    import numpy as np

    import ferry_amd as F
    from oracle import pyoracle as O

    R, L, S, SEL, HOT, GRP, PS, GAP, TICK = 12, 3, 10, 16, 40, 4, 8, 0.7, 1.0
    out = _run_wla(["--requests", str(R), "--layers", str(L), "--steps", str(S), "--sel", str(SEL),
                    "--hot", str(HOT), "--arrival", "steady", "--gap", str(GAP),
                    "--prefix-group", str(GRP), "--prefix-steps", str(PS)],
                   env={"FERRY_VIRTUAL_TICK_MS": str(TICK)})
    rows = _rows(out)
    ids = F.refgen_selections(R, L, S, SEL, 42)
    for r in range(R):
        head = (r // GRP) * GRP
        ids[r, :PS] = ids[head, :PS]
    arrive = O.arrivals(0, R, GAP)
    clock = np.arange(0.0, 200.0, TICK)
    table, _, _ = O.sched_run(R, arrive, np.full(R, S), clock, pinned=True)
    g = O.make_geom(n_req=R, group=GRP, n_layers=L, kv_heads=1, k=SEL, cap=HOT,
                    max_blocks=64 + 8 * S, dtype=O.F32, granularity=1)
    ex = O.Executor(g)
    step = np.zeros(R, int)
    misses = ticks = 0
    for t in range(len(clock)):
        live = table[t] >= 0
        if not live.any():
            if t > 0 and (table[:t] >= 0).any() and not (table[t:] >= 0).any():
                break
            continue
        for j in range(GRP):  # member j of every group, in request order (sub-ticks)
            sel = np.full((R, L, 1, SEL), O.NONE, np.uint32)
            for ln in np.nonzero(live)[0]:
                if ln % GRP == j:
                    sel[ln, :, 0] = ids[table[t, ln], step[table[t, ln]]]
            if np.all(sel == O.NONE):
                continue
            _, _, _, c = ex.step(sel)
            misses += int(c[1])
        for ln in np.nonzero(live)[0]:
            step[table[t, ln]] += 1
        ticks += 1
    for mode in "BC":
        assert rows[mode][0] == misses and rows[mode][3] == ticks and rows[mode][4] == 0


def _fnv1a64(data):
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


@pytest.mark.gpu
def test_wla_slice_runs_a_trace(tmp_path):
    # An FMT1 trace drives the tick loop (FERRY_MISS_TRACE): every (request,
    # layer) keeps a 16-slot LRU, so the refills equal the per-touch LRU of
    # each stream (missstream.cuh:137-161) over the trace's dense ids.
    import numpy as np

    from oracle import pyoracle as O
    from test_trace import chained_trace, write_fmt1

    R, S, L, SP, HOT = 6, 5, 3, 4, 24
    recs = chained_trace(R, S, L, SP, groups=2, seed=3)
    path = tmp_path / "t.bin"
    write_fmt1(path, recs, R, S, L, sel_pages=SP)
    out = _run_wla(["--requests", str(R), "--layers", str(L), "--steps", str(S), "--sel", str(SP * 4),
                    "--hot", str(HOT), "--kv-heads", "4", "--head-dim", "128", "--miss-trace",
                    str(path), "--gap", "0.5"])
    assert f"fnv1a64={_fnv1a64(path.read_bytes()):016x}" in out
    _, ids, _, _ = O.trace_load(str(path))
    want = 0
    for r in range(R):
        for l in range(L):
            stream = np.ascontiguousarray(ids[r, :, l].reshape(-1), np.uint32)
            flags = np.zeros(stream.size, np.uint8)
            assert O.lib.ora_deque_lru_run(HOT, stream, stream.size, flags) == 0
            want += int(flags.sum())
    rows = _rows(out)
    for mode in "BC":
        assert rows[mode][0] == want and rows[mode][4] == 0
