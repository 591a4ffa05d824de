"""Lane turnover on the CPU: empty selection positions, request arrivals, the
tick scheduler and generator admission.  The oracle is pinned by closed forms
(steady/bursty arrivals follow src/runtime/wla_multigpu.cuh:497-501),
statistics (Poisson and Markov-modulated gaps), structural invariants (FIFO,
work conservation, residency for exactly len steps) and compaction identities
(an empty position must behave as if it were absent); the product's host code
is then compared with it bit for bit."""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as O

import ferry_amd as F  # noqa: E402  (host entry points only; no device call)

NONE = O.NONE


def _lru(cap, mb):
    s = O.LRU()
    assert O.lib.ora_lru_init(C.byref(s), cap, mb) == 0
    return s


def _substep(s, x):
    x = np.ascontiguousarray(x, np.uint32)
    n = x.size
    so = np.zeros(max(n, 1), np.uint32)
    mo = np.zeros(max(n, 1), O.MISS_DTYPE)
    fl = np.zeros(max(n, 1), np.uint8)
    nm = C.c_int(0)
    rc = O.lib.ora_lru_substep(C.byref(s), 0, x if n else np.zeros(1, np.uint32), n, so, mo,
                               C.byref(nm), fl.ctypes.data)
    return rc, so[:n].copy(), mo[:nm.value].copy(), fl[:n].copy()


def _state(s):
    cap = s.cap
    return (s.fill, [s.ord[i] for i in range(cap)], [s.tag[i] for i in range(cap)])


@pytest.mark.parametrize("serial", [False, True])
def test_empty_positions_behave_as_absent(serial):
    """A stream with empty positions leaves the same LRU state, misses and
    slots as the same stream with them removed; empties get slot NONE and
    never a miss flag."""
    rng = np.random.default_rng(5)
    cap, mb = 24, 60
    a, b = _lru(cap, mb), _lru(cap, mb)
    for _ in range(40):
        n = int(rng.integers(0, 20))
        x = rng.choice(mb, size=n, replace=False).astype(np.uint32)
        holes = rng.random(n + 8) < 0.3
        full = np.full(n + int(holes.sum()), NONE, np.uint32)
        keep = np.ones(full.size, bool)
        keep[rng.choice(full.size, size=full.size - n, replace=False)] = False
        full[keep] = x
        if serial:
            outs = [_substep(a, full[i:i + 1]) for i in range(full.size)]
            refs = [_substep(b, x[i:i + 1]) for i in range(n)]
            got_slots = np.array([o[1][0] for o in outs], np.uint32)
            got_flags = np.array([o[3][0] for o in outs], np.uint8)
            ref_slots = np.array([r[1][0] for r in refs], np.uint32)
            ref_flags = np.array([r[3][0] for r in refs], np.uint8)
            assert all(o[0] == 0 for o in outs) and all(r[0] == 0 for r in refs)
        else:
            rc, got_slots, gm, got_flags = _substep(a, full)
            rc2, ref_slots, rm, ref_flags = _substep(b, x)
            assert rc == rc2 == 0
            assert np.array_equal(gm, rm)
        assert np.all(got_slots[~keep] == NONE) and np.all(got_flags[~keep] == 0)
        assert np.array_equal(got_slots[keep], ref_slots)
        assert np.array_equal(got_flags[keep], ref_flags)
        assert _state(a) == _state(b)


def _geom(dtype=O.F16, n_req=3, L=2, H=2, Hq=4, k=6, cap=16, mb=40):
    return O.make_geom(n_req=n_req, n_layers=L, kv_heads=H, q_heads=Hq, k=k, cap=cap,
                       max_blocks=mb, dtype=dtype, host_blocks=997)


def test_attention_empty_positions_and_empty_rows():
    """Attention over a row with empty positions equals attention over the
    row's selected blocks alone; a row with nothing selected gives 0."""
    g = _geom()
    rng = np.random.default_rng(2)
    sel = np.stack([rng.choice(40, size=6, replace=False) for _ in range(3 * 2 * 2)]).astype(
        np.uint32)
    q = rng.standard_normal((3, 2, 4, 128)).astype(np.float32)
    holes = sel.copy()
    holes[0, [1, 4]] = NONE          # ragged row
    holes[5, :] = NONE               # empty row (request 1, layer 0, kv head 1)
    out = O.attention_f64(g, holes, q).reshape(3 * 2 * 2, 2, 128)
    # reference: rows 0 and 5 recomputed with a k that matches what is selected
    g4 = _geom(k=4)
    rows4 = np.tile(holes[0, [0, 2, 3, 5]], (12, 1)).astype(np.uint32)
    ref0 = O.attention_f64(g4, rows4, q).reshape(12, 2, 128)[0]
    assert np.allclose(out[0], ref0, rtol=0, atol=1e-12)
    assert np.all(out[5] == 0.0)
    full = O.attention_f64(g, sel, q).reshape(12, 2, 128)
    others = [i for i in range(12) if i not in (0, 5)]
    assert np.array_equal(out[others], full[others])


def test_exec_step_counts_only_selected_positions():
    g = _geom()
    ex = O.Executor(g)
    rng = np.random.default_rng(1)
    sel = np.stack([rng.choice(40, size=6, replace=False) for _ in range(12)]).astype(np.uint32)
    sel[3, 2:] = NONE
    sel[8:12] = NONE  # request 2 not resident
    slots, mc, misses, counts = ex.step(sel)
    assert counts[0] == int((sel != NONE).sum())
    assert np.all(slots.reshape(12, 6)[sel == NONE] == NONE)
    assert counts[1] == int(mc.sum()) == int((sel != NONE).sum())  # cold: every block misses


def test_reset_owner_makes_the_lane_cold():
    g = _geom(n_req=2, L=1, H=1, Hq=1, k=4, cap=8, mb=20)
    ex = O.Executor(g)
    sel = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.uint32)
    ex.step(sel)
    _, mc, _, c = ex.step(sel)
    assert c[1] == 0
    ex.reset_owner(1)
    fill, _, _ = ex.state()
    assert list(fill) == [4, 0]
    _, mc, _, c = ex.step(sel)
    assert list(mc) == [0, 4]


def test_copied_owner_behaves_like_its_source():
    """After an owner's sets are copied into another executor's lane, the same
    future selections give the same hits, slots and evictions there as in the
    source lane (the state a hand-off must carry)."""
    g = _geom(n_req=3, L=2, H=2, Hq=2, k=6, cap=10, mb=40)
    rng = np.random.default_rng(3)
    draw = lambda: np.stack([rng.choice(40, 6, replace=False) for _ in range(12)]).astype(np.uint32)
    x, y = O.Executor(g), O.Executor(g)
    for _ in range(5):
        x.step(draw())
    for _ in range(3):
        y.step(draw())
    y.copy_owner_from(x, 0, 2)
    xf, xo, xt = x.state()
    yf, yo, yt = y.state()
    assert np.array_equal(yf[8:12], xf[0:4]) and np.array_equal(yt[8:12], xt[0:4])
    for _ in range(6):
        s = draw()
        sx = s.copy()
        sy = s.copy()
        sy[8:12] = s[0:4]
        xs, xmc, xm, _ = x.step(sx)
        ys, ymc, ym, _ = y.step(sy)
        # slots are global ids (set * cap + slot): lane 2's sets start 8 sets on
        assert np.array_equal(ys.reshape(12, 6)[8:12] - 80, xs.reshape(12, 6)[0:4])
        assert np.array_equal(ymc[8:12], xmc[0:4])
        for a, b in zip(range(0, 4), range(8, 12)):
            assert np.array_equal(ym[b, :ymc[b]][["block", "slot", "evicted"]],
                                  xm[a, :xmc[a]][["block", "slot", "evicted"]])
    with pytest.raises(ValueError):
        y.copy_owner_from(O.Executor(_geom(n_req=3, L=2, H=2, Hq=2, k=6, cap=11, mb=40)), 0, 0)


# ---------------------------------------------------------------- arrivals
def test_steady_and_bursty_arrivals_closed_form():
    n, gap = 40, 2.5
    steady = O.arrivals(0, n, gap)
    assert np.allclose(steady, gap * np.arange(1, n + 1), rtol=0, atol=1e-9)
    # wla_multigpu.cuh:497-501: t += 40 gap for r % 16 == 0, else 0.1 gap
    incr = np.where(np.arange(n) % 16 == 0, 40.0 * gap, 0.1 * gap)
    assert np.allclose(O.arrivals(1, n, gap), np.cumsum(incr), rtol=0, atol=1e-9)


def test_poisson_arrivals_are_exponential():
    n, gap = 20000, 3.0
    t = O.arrivals(2, n, gap, seed=9)
    d = np.diff(np.concatenate([[0.0], t]))
    assert np.all(d > 0)
    # mean within 4 standard errors; Kolmogorov-Smirnov distance to Exp(gap)
    assert abs(d.mean() - gap) < 4 * gap / np.sqrt(n)
    xs = np.sort(d)
    emp = np.arange(1, n + 1) / n
    ks = np.max(np.abs(emp - (1.0 - np.exp(-xs / gap))))
    assert ks < 1.63 / np.sqrt(n)  # 1% critical value


def test_mmpp_arrivals_rate_and_burstiness():
    gap, period, ratio, n = 4.0, 50.0, 10.0, 40000
    t = O.arrivals(3, n, gap, period, ratio, seed=3)
    assert np.all(np.diff(t) >= 0)
    # equal mean sojourns: half the time at 1/gap, half at ratio/gap
    rate = (1.0 / gap + ratio / gap) / 2
    assert abs(n / t[-1] / rate - 1.0) < 0.1
    # counts in 10 ms windows are over-dispersed (index of dispersion >> 1),
    # unlike a Poisson stream of the same mean rate
    w = 10.0
    cm = np.bincount((t // w).astype(np.int64))
    cp = np.bincount((O.arrivals(2, n, 1.0 / rate, seed=3) // w).astype(np.int64))
    assert cm.var() / cm.mean() > 3.0
    assert 0.8 < cp.var() / cp.mean() < 1.25


@pytest.mark.parametrize("kind", [0, 1, 2, 3])
def test_product_arrivals_equal_oracle(kind):
    for seed in (0, 7, 123456789):
        a = F.arrivals(kind, 3000, 1.7, 50.0, 10.0, seed)
        b = O.arrivals(kind, 3000, 1.7, 50.0, 10.0, seed)
        assert np.array_equal(a, b)


def test_invalid_arrival_parameters_rejected():
    with pytest.raises(F.FerryError):
        F.arrivals(2, 10, 0.0)
    with pytest.raises(F.FerryError):
        F.arrivals(3, 10, 1.0, 0.0, 10.0)
    with pytest.raises(F.FerryError):
        F.arrivals(9, 10, 1.0)


# ---------------------------------------------------------------- scheduler
def _run_sched(lanes, arrive, lens, clock):
    s = F.Sched(lanes, arrive, lens)
    table, adm, ret = [], [], []
    for now in clock:
        r = s.tick(now)
        table.append(r["lane_req"].copy())
        adm.append(list(r["admitted"]))
        ret.append(list(r["retired"]))
    a, d = s.request_ticks()
    return np.array(table), adm, ret, a, d, s


@pytest.mark.parametrize("seed", range(6))
def test_scheduler_matches_oracle_and_invariants(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 60))
    lanes = int(rng.integers(1, 9))
    arrive = np.sort(rng.exponential(3.0, n).cumsum())
    if seed % 2:
        arrive = np.round(arrive)  # ties
    lens = rng.integers(1, 12, n).astype(np.int32)
    ticks = int(lens.sum()) + int(arrive[-1]) + 10
    clock = np.arange(ticks, dtype=np.float64)  # one ms per tick
    table, adm, ret, a, d, s = _run_sched(lanes, arrive, lens, clock)
    otab, oa, od = O.sched_run(lanes, arrive, lens, clock)
    assert np.array_equal(table, otab)
    assert list(a) == oa and list(d) == od
    # every request ran exactly len ticks in one lane, consecutively
    for r in range(n):
        ticks_r, lanes_r = np.nonzero(table == r)
        assert len(ticks_r) == lens[r] and len(set(lanes_r)) == 1
        assert np.array_equal(ticks_r, np.arange(a[r], a[r] + lens[r])) and d[r] == ticks_r[-1]
        assert clock[a[r]] >= arrive[r]
    # FIFO: admission order follows arrival order
    order = sorted(range(n), key=lambda r: (arrive[r], r))
    assert all(a[order[i]] <= a[order[i + 1]] for i in range(n - 1))
    # work conservation: no lane idles while an arrived request waits
    for t, now in enumerate(clock):
        waiting = [r for r in range(n) if arrive[r] <= now and a[r] > t]
        assert not waiting or np.all(table[t] >= 0)
    # admitted/retired lists agree with the table
    for t in range(1, ticks):
        new = [ln for ln in range(lanes) if table[t, ln] >= 0 and table[t, ln] != table[t - 1, ln]]
        gone = [ln for ln in range(lanes) if table[t, ln] < 0 <= table[t - 1, ln]]
        assert adm[t] == new and ret[t] == gone
    assert s.tick(clock[-1] + 1)["done"]


@pytest.mark.parametrize("seed", range(4))
def test_pinned_scheduler_matches_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    n, lanes = int(rng.integers(5, 50)), int(rng.integers(1, 7))
    arrive = np.round(np.sort(rng.exponential(2.0, n).cumsum()))
    lens = rng.integers(1, 9, n).astype(np.int32)
    clock = np.arange(float(lens.sum() + arrive[-1] + 5))
    s = F.Sched(lanes, arrive, lens, pinned=True)
    table = np.array([s.tick(now)["lane_req"] for now in clock])
    otab, oa, od = O.sched_run(lanes, arrive, lens, clock, pinned=True)
    assert np.array_equal(table, otab)
    a, d = s.request_ticks()
    assert list(a) == oa and list(d) == od
    for r in range(n):  # request r only ever runs in lane r % lanes
        assert set(np.nonzero(table == r)[1]) == {r % lanes}
        assert np.count_nonzero(table == r) == lens[r]


def test_scheduler_unbounded_lanes_admits_on_arrival():
    """With at least as many lanes as requests (the reference's unbounded
    residency) a request is admitted at the first tick at or after its arrival."""
    arrive = O.arrivals(1, 33, 0.7)
    lens = np.full(33, 5, np.int32)
    clock = np.arange(0.0, arrive[-1] + 10.0, 0.5)
    _, _, _, a, _, _ = _run_sched(33, arrive, lens, clock)
    assert np.array_equal(a, np.searchsorted(clock, arrive, side="left"))


# ---------------------------------------------------------------- generator admission
def _pair(n_req=4, L=2, H=3, k=8, ctx=(40, 9, 25, 64), **kw):
    ctx = np.array(ctx, np.int32)
    p = F.SelGen(n_req, L, H, k, ctx, **kw)
    o = O.selgen(n_req, L, H, k, ctx, **kw)
    return p, o


def test_selgen_ragged_rows_match_oracle():
    p, o = _pair(dist=1, zipf_s=1.1, reuse=0.5, seed=4)
    for t in range(6):
        a = p.step(t).reshape(-1)
        b = O.selgen_step(o, t)
        assert np.array_equal(a, b)
        rows = a.reshape(4, 2, 3, 8)
        # request 1 has a 9-block context: 8 of 9 selected, no padding
        assert np.all(rows[1] != NONE)
    p2, o2 = _pair(ctx=(40, 5, 25, 3), k=8)
    a = p2.step(0).reshape(4, 2, 3, 8)
    assert np.array_equal(a.reshape(-1), O.selgen_step(o2, 0))
    assert np.all(np.sort(a[1], axis=-1)[..., :5] == np.arange(5)) and np.all(a[1][..., 5:] == NONE)
    assert np.all(a[3][..., 3:] == NONE)


def test_selgen_admission_matches_oracle():
    p, o = _pair(dist=1, zipf_s=1.0, reuse=0.66, seed=11)
    rng = np.random.default_rng(0)
    rid = 100
    for t in range(30):
        if t and t % 4 == 0:
            lane = int(rng.integers(0, 4))
            if rng.random() < 0.3:
                p.retire(lane)
                O.selgen_retire(o, lane)
            else:
                ctx = int(rng.integers(1, 65))
                p.admit(lane, rid, ctx, t)
                O.selgen_admit(o, lane, rid, ctx, t)
                rid += 1
        a = p.step(t).reshape(-1)
        b = O.selgen_step(o, t)
        assert np.array_equal(a, b), t


def test_admitted_request_stream_is_independent_of_its_lane():
    """A request's selections depend on (request id, steps since admission),
    not on the lane or the step it was admitted at."""
    ctx = np.array([50, 50, 50], np.int32)
    p = F.SelGen(3, 2, 2, 6, ctx, reuse=0.66, seed=5)
    q = F.SelGen(3, 2, 2, 6, ctx, reuse=0.66, seed=5)
    p.admit(0, 77, 30, 0)
    for t in range(5):
        q.step(t)
    q.admit(2, 77, 30, 5)
    for i in range(8):
        assert np.array_equal(p.step(i)[0], q.step(5 + i)[2])


def test_admission_rejects_bad_arguments():
    p = F.SelGen(2, 1, 1, 4, np.array([20, 20], np.int32))
    for bad in [(5, 1, 10, 0), (0, 70000, 10, 0), (0, 1, 0, 0), (0, 1, 21, 0)]:
        with pytest.raises(F.FerryError):
            p.admit(*bad)
    p.admit(0, 3, 10, 4)
    with pytest.raises(F.FerryError):
        p.step(2)  # lane 0's request starts at step 4
    g = F.SelGen(4, 1, 1, 4, np.array([20] * 4, np.int32), group=2)
    with pytest.raises(F.FerryError):
        g.admit(0, 9, 10, 0)  # lanes of a prefix group share one permutation


def test_tick_loop_lanes_are_independent_in_the_oracle():
    """Through a tick loop with lane turnover (owner reset on admission), each
    request sees the same hits and misses as when it runs alone from a cold
    cache: the reset removes every trace of the lane's previous occupant."""
    L, H, k, cap, lanes = 2, 2, 6, 14, 3
    arrive = O.arrivals(2, 9, 2.0, seed=1)
    lens = np.array([3, 5, 2, 6, 4, 3, 5, 2, 4], np.int32)
    ctxs = np.array([30, 20, 40, 12, 30, 25, 18, 40, 33], np.int32)
    clock = np.arange(0.0, 80.0, 1.0)
    table, adm_tick, _ = O.sched_run(lanes, arrive, lens, clock)
    g = O.make_geom(n_req=lanes, n_layers=L, kv_heads=H, k=k, cap=cap, max_blocks=40)
    ex = O.Executor(g)
    sg = O.selgen(lanes, L, H, k, np.full(lanes, 40, np.int32), reuse=0.6, seed=2)
    for ln in range(lanes):
        O.selgen_retire(sg, ln)
    flags = {r: [] for r in range(9)}
    prev = [-1] * lanes
    for t in range(len(clock)):
        for ln in range(lanes):
            r = table[t, ln]
            if r != prev[ln]:
                if r >= 0:
                    O.selgen_admit(sg, ln, r, ctxs[r], t)
                    ex.reset_owner(ln)
                else:
                    O.selgen_retire(sg, ln)
            prev[ln] = r
        sel = O.selgen_step(sg, t)
        ex.step(sel)
        for ln in range(lanes):
            if table[t, ln] >= 0:
                flags[table[t, ln]].append(ex.last_flags.reshape(lanes, -1)[ln].copy())
    for r in range(9):
        solo = O.Executor(O.make_geom(n_req=1, n_layers=L, kv_heads=H, k=k, cap=cap,
                                      max_blocks=40))
        sg1 = O.selgen(1, L, H, k, np.array([40], np.int32), reuse=0.6, seed=2)
        O.selgen_admit(sg1, 0, r, ctxs[r], 0)
        for i in range(lens[r]):
            solo.step(O.selgen_step(sg1, i))
            assert np.array_equal(solo.last_flags, flags[r][i]), (r, i)
