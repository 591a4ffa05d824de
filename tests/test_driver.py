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


def _ms_rows(out):
    """run_missstream rows: name -> (refill, MB, status, fetched)."""
    rows = {}
    for m in re.finditer(r"^\s+(baseline-A|baseline-B|ferry-C)\s+makespan=.*refill=\s*(\d+) "
                         r"bytes=\s*([\d.]+)MB status=(-?\d+) fetched=(\d+)", out, re.M):
        rows[m.group(1)] = (int(m.group(2)), m.group(3), int(m.group(4)), int(m.group(5)))
    return rows


@pytest.mark.gpu
def test_driver_golden_default_stream():
    # results/wla_7rep_20260930/*.log: selects 589,824, misses 79,550, hit 0.865.
    # The reference's counts per mode (kv_exec.cuh:108-145, 148-185, 188-292):
    # A copies every selected block (589,824 = 9216.00 MB), B submits every miss
    # (79,550 = 1242.97 MB), C one submit per coalesced run of a request-step's
    # misses under run_missstream's policy (target 8 batches,
    # run_missstream.cu:101), which the oracle's restated planner counts.
    from oracle import pyoracle as O

    out = _run(["--requests", "48", "--layers", "12", "--steps", "16", "--sel", "64", "--hot", "1"])
    assert "selects=589824 miss=79550 hit_rate=0.865 miss_bytes=1242.97MB" in out
    rows = _ms_rows(out)
    blocks, miss, _, nm = O.ref_replay(48, 12, 16, 64, 128)
    assert nm == 79550
    c_runs, c_bytes = O.ref_cmode_runs(48, 12, 16, 64, 128, 16384, blocks, miss, target=8.0)
    assert rows["baseline-A"][:3] == (589824, "9216.00", 0)
    assert rows["baseline-B"][:3] == (79550, "1242.97", 0)
    assert rows["ferry-C"][:3] == (c_runs, "1242.97", 0) and c_bytes == 79550 * 16384
    # the GPU moved each miss once in B and C (A: every distinct block per step)
    assert rows["baseline-B"][3] == rows["ferry-C"][3] == 79550
    assert 79550 < rows["baseline-A"][3] <= 589824
    ratio = re.search(r"refill C/B ([\d.]+)", out).group(1)
    assert ratio == f"{c_runs / 79550:.3f}"
    # each row's interval on the GPU's clock (ferry::HipTimer around the run,
    # which also creates and destroys its executor) covers its host makespan
    spans = re.findall(r"makespan=\s*([\d.]+)ms.* gpu=([\d.]+)ms", out)
    assert len(spans) == 3
    for host_ms, gpu_ms in spans:
        assert 0.0 < float(host_ms) <= float(gpu_ms) * 1.05 + 1.0


@pytest.mark.gpu
def test_driver_golden_single_gpu_run():
    # 实验设计.txt:494-495: 4 req x 12 layers x 4 steps, sel 128, hot 1024 ->
    # 57.66 MB of misses; the C engine's submits drop from 3690 to 1227.
    out = _run(["--requests", "4", "--layers", "12", "--steps", "4", "--sel", "128", "--hot", "4"])
    assert "miss=3690" in out and "miss_bytes=57.66MB" in out
    rows = _ms_rows(out)
    assert rows["baseline-A"][:3] == (24576, "384.00", 0)
    assert rows["baseline-B"][:3] == (3690, "57.66", 0)
    assert rows["ferry-C"][:3] == (1227, "57.66", 0)
    assert rows["baseline-B"][3] == rows["ferry-C"][3] == 3690
    assert "refill C/B 0.333" in out


WLA = os.path.join(ROOT, "ferry_amd", "run_wla")


def test_wla_driver_rejects_bad_flags():
    if not os.path.exists(WLA):
        pytest.skip("run_wla not built")
    res = subprocess.run([WLA, "--no-such-flag"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "unknown flag" in res.stderr
    res = subprocess.run([WLA, "--gpus", "0,1"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "one GPU" in res.stderr


def _rows(out):
    """run_wla rows: mode -> (refill, MB, hit, ticks, status, fetched)."""
    rows = {}
    for m in re.finditer(r"^\s+([ABC])\s+makespan=.*refill=\s*(\d+) seg\s+([\d.]+)MB hit=([\d.]+) "
                         r"ticks=(\d+) status=(-?\d+) fetched=(\d+)", out, re.M):
        rows[m.group(1)] = (int(m.group(2)), m.group(3), float(m.group(4)), int(m.group(5)),
                            int(m.group(6)), int(m.group(7)))
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
    # the refill counts are the reference's golden rows (results/
    # wla_7rep_20260930/*.log l.2-4, default policy target 4): A 589,824
    # selected blocks, B 79,550 misses, C 59,863 coalesced submits, the last
    # two 1242.97 MB; the GPU fetched the 79,550 misses once in B and C.
    out = _run_wla(["--requests", "48", "--layers", "12", "--steps", "16", "--sel", "64",
                    "--hot", "128", "--arrival", "bursty", "--gap", "0.2"])
    rows = _rows(out)
    assert rows["A"][0] == 589824 and rows["A"][1] == "9216.00" and rows["A"][4] == 0
    assert rows["B"][0] == 79550 and rows["C"][0] == 59863
    for mode in "BC":
        assert rows[mode][1] == "1242.97" and rows[mode][4] == 0 and rows[mode][5] == 79550
        assert round(rows[mode][2], 3) == 0.865


@pytest.mark.gpu
@pytest.mark.parametrize("cap_mode", ["group", "perreq"])
def test_wla_slice_prefix_groups_match_oracle(cap_mode):
    # C2 prefix groups (wla_multigpu.cuh:355-369): members repeat their head's
    # selections for 8 steps and share the group's LRU, touched member after
    # member within a tick (:2643-2648).  With a virtual clock the tick
    # composition is fixed, and the oracle replays the same ticks.  Under
    # --cap-mode perreq the group's capacity is hot x resident members: a
    # request joins at its arrival and leaves when it finishes, which trims the
    # group (wla_group_cap, grp_trim, :846-862, 1923-1936).
    import numpy as np

    import ferry_amd as F
    from oracle import pyoracle as O

    R, L, S, SEL, HOT, GRP, PS, GAP, TICK = 12, 3, 10, 16, 40, 4, 8, 0.7, 1.0
    out = _run_wla(["--requests", str(R), "--layers", str(L), "--steps", str(S), "--sel", str(SEL),
                    "--hot", str(HOT), "--arrival", "steady", "--gap", str(GAP),
                    "--prefix-group", str(GRP), "--prefix-steps", str(PS), "--cap-mode", cap_mode],
                   env={"FERRY_VIRTUAL_TICK_MS": str(TICK)})
    rows = _rows(out)
    ids = F.refgen_selections(R, L, S, SEL, 42)
    for r in range(R):
        head = (r // GRP) * GRP
        ids[r, :PS] = ids[head, :PS]
    arrive = O.arrivals(0, R, GAP)
    clock = np.arange(0.0, 200.0, TICK)
    table, _, _ = O.sched_run(R, arrive, np.full(R, S), clock, pinned=True)
    per = cap_mode == "perreq"
    g = O.make_geom(n_req=R, group=GRP, n_layers=L, kv_heads=1, k=SEL,
                    cap=HOT * GRP if per else HOT, max_blocks=64 + 8 * S, dtype=O.F32,
                    granularity=1, cap_mode=1 if per else 0)
    ex = O.Executor(g)
    assert ex.members_leave(list(range(R)))  # members join when they arrive
    step = np.zeros(R, int)
    misses = ticks = runs = 0
    was = np.zeros(R, bool)
    for t in range(len(clock)):
        live = table[t] >= 0
        gone = [int(x) for x in np.nonzero(was & ~live)[0]]
        came = [int(x) for x in np.nonzero(live & ~was)[0]]
        assert (not gone or ex.members_leave(gone)) and (not came or ex.members_join(came))
        was = live
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
            flags = ex.last_flags.reshape(R, L, SEL)
            for ln in np.nonzero(live)[0]:
                if ln % GRP == j:  # this request-step's coalesced submits (target 4)
                    runs += O.ref_cmode_runs(1, L, 1, SEL, HOT, 16384,
                                             sel[ln, :, 0].astype(np.uint64), flags[ln], target=4.0)[0]
        for ln in np.nonzero(live)[0]:
            step[table[t, ln]] += 1
        ticks += 1
    assert rows["B"][0] == misses and rows["C"][0] == runs < misses
    for mode in "BC":
        assert rows[mode][3] == ticks and rows[mode][4] == 0 and rows[mode][5] == misses


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
    miss = np.zeros(ids.shape, np.uint8)  # (r, s, l, k)
    for r in range(R):
        for l in range(L):
            stream = np.ascontiguousarray(ids[r, :, l].reshape(-1), np.uint32)
            flags = np.zeros(stream.size, np.uint8)
            assert O.lib.ora_deque_lru_run(HOT, stream, stream.size, flags) == 0
            miss[r, :, l] = flags.reshape(S, -1)
            want += int(flags.sum())
    # C: the coalesced submits of every request-step (default policy, target 4)
    runs, _ = O.ref_cmode_runs(R, L, S, SP * 4, HOT, 4 * 2 * 4 * 128 * 2,
                               ids.reshape(-1).astype(np.uint64), miss.reshape(-1), target=4.0)
    rows = _rows(out)
    assert rows["B"][0] == want and rows["C"][0] == runs
    for mode in "BC":
        assert rows[mode][4] == 0 and rows[mode][5] == want
