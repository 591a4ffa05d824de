"""GPU parity of lane turnover: empty selection positions (ragged rows and
requests that are not resident), per-owner set resets, and the tick loop
driven by request arrivals -- against the CPU oracle, through the C-ABI.

Bookkeeping is bit-exact; attention is within 2e-3 (fp32/fp16/bf16) or 1e-2
(fp8) of the fp64 oracle per (request, layer, head) row, and a row of a
request with nothing selected must be exactly 0.
"""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import TOL, Pair

pytestmark = pytest.mark.gpu

NONE = O.NONE


def _attention(p, sel, seed=0):
    g = p.g
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((g.n_req, g.n_layers, g.q_heads, 128)).astype(np.float32)
    dq = torch.from_numpy(q).cuda()
    out = torch.full_like(dq, float("nan"))
    p.ex.sparse_decode(dq, p.bufs["slots"], out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
    ref = O.attention_f64(g, sel, q).reshape(-1, 128)
    empty = np.all(ref == 0.0, axis=1)
    assert np.all(got[empty] == 0.0)
    rel = np.abs(got[~empty] - ref[~empty]).max(axis=1) / np.abs(ref[~empty]).max(axis=1)
    assert np.all(np.isfinite(got))
    assert rel.max() < TOL[p.dtype], rel.max()
    return int(empty.sum())


@pytest.mark.parametrize("dtype,Hkv,Hq,attn", [
    (F.F16, 4, 4, F.ATTN_AUTO),     # VALU, MHA
    (F.BF16, 2, 8, F.ATTN_AUTO),    # MFMA, GQA-4
    (F.FP8, 2, 8, F.ATTN_AUTO),     # MFMA, fp8 + scales
    (F.BF16, 2, 8, F.ATTN_VALU),    # VALU, GQA-4
    (F.F32, 2, 4, F.ATTN_AUTO),     # VALU, fp32
])
def test_empty_positions_parity(dtype, Hkv, Hq, attn):
    n_req, L, k, cap, mb = 5, 2, 80, 120, 300
    rng = np.random.default_rng(dtype * 10 + Hq)
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, attn=attn)
    ctx = O.ctx_uniform(4, n_req, 100, 300)
    sg = O.selgen(n_req, L, Hkv, k, ctx, reuse=0.66, seed=4)
    for t in range(5):
        sel = O.selgen_step(sg, t).reshape(n_req, L, Hkv, k)
        holes = rng.random(sel.shape) < 0.2
        sel = np.where(holes, np.uint32(NONE), sel)
        sel[t % n_req] = NONE                      # a request that is not resident
        sel[(t + 1) % n_req, 0, 0, 3:] = NONE      # a ragged row
        sel[(t + 2) % n_req, 1, 0, :] = NONE       # one empty row of a resident request
        sel = sel.reshape(-1)
        fetched = p.step(sel)
        p.check_fetched_bytes(fetched)
        p.check_state()
        assert _attention(p, sel, seed=t) >= L * Hq
    st = p.ex.stats()
    assert st["device_error"] == 0


def test_reset_owners_parity():
    n_req, L, Hkv, k, cap, mb = 6, 3, 2, 24, 48, 200
    p = Pair(n_req, L, Hkv, Hkv, k, cap, mb, F.F16)
    ctx = O.ctx_uniform(5, n_req, 60, 200)
    sg = O.selgen(n_req, L, Hkv, k, ctx, reuse=0.5, seed=5)
    for t in range(6):
        if t in (2, 4):
            owners = [1, 4] if t == 2 else [0, 5, 3]
            p.ex.reset_owners(torch.tensor(owners, dtype=torch.int32, device="cuda"))
            for o in owners:
                p.ox.reset_owner(o)
            p.check_state()
        p.check_fetched_bytes(p.step(O.selgen_step(sg, t)))
        p.check_state()
    bad = torch.tensor([n_req], dtype=torch.int32, device="cuda")
    p.ex.reset_owners(bad)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -1  # FERRY_EINVAL latched on the device


@pytest.mark.parametrize("kind", [F.ARRIVAL_POISSON, F.ARRIVAL_MMPP])
def test_tick_loop_with_arrivals_parity(kind):
    """Requests arrive (virtual clock, 1 ms per tick), wait for a lane, decode
    their length and leave.  Every tick: the product's scheduler and
    generator equal the oracle's, the lane of each admitted request is reset
    on both sides, and bookkeeping, fetched bytes and attention match."""
    lanes, L, Hkv, Hq, k, cap = 4, 2, 2, 4, 24, 60
    n = 14
    arrive = F.arrivals(kind, n, 1.5, 6.0, 10.0, seed=2)
    lens = F.ctx_uniform(8, n, 2, 7)
    ctxs = F.ctx_uniform(9, n, 10, 160)
    sched = F.Sched(lanes, arrive, lens)
    ticks = int(lens.sum()) + int(arrive[-1]) + 4
    clock = np.arange(ticks, dtype=np.float64)
    otable, oadmit, olast = O.sched_run(lanes, arrive, lens, clock)
    sg = F.SelGen(lanes, L, Hkv, k, np.full(lanes, 160, np.int32), reuse=0.66, seed=6)
    og = O.selgen(lanes, L, Hkv, k, np.full(lanes, 160, np.int32), reuse=0.66, seed=6)
    p = Pair(lanes, L, Hkv, Hq, k, cap, sg.max_blocks, F.BF16)
    for ln in range(lanes):
        sg.retire(ln)
        O.selgen_retire(og, ln)
    steps = 0
    for t, now in enumerate(clock):
        r = sched.tick(now)
        assert np.array_equal(r["lane_req"], otable[t])
        for ln in r["retired"]:
            sg.retire(ln)
            O.selgen_retire(og, ln)
        if len(r["admitted"]):
            lanes_new = [int(x) for x in r["admitted"]]
            for ln in lanes_new:
                rid = int(r["lane_req"][ln])
                sg.admit(ln, rid, int(ctxs[rid]), t)
                O.selgen_admit(og, ln, rid, int(ctxs[rid]), t)
                p.ox.reset_owner(ln)
            p.ex.reset_owners(torch.tensor(lanes_new, dtype=torch.int32, device="cuda"))
        if r["resident"] == 0:
            if r["done"]:
                break
            continue
        sel = sg.step(t).reshape(-1)
        assert np.array_equal(sel, O.selgen_step(og, t))
        p.check_fetched_bytes(p.step(sel))
        steps += 1
        if steps % 3 == 1:
            p.check_state()
            _attention(p, sel, seed=t)
    assert r["done"]
    a, d = sched.request_ticks()
    assert list(a) == oadmit and list(d) == olast
    st = p.ex.stats()
    assert st["device_error"] == 0 and st["steps"] == steps


def test_reference_stream_through_tick_loop():
    """The reference's default stream (R48 L12 S16 sel64 hot128 seed 42) run by
    the tick loop: requests arrive in bursts (src/runtime/wla_multigpu.cuh:
    497-501), each is resident for its 16 steps, and per-selection LRU gives
    every event the reference's hit/miss flag -- 79,550 misses in all
    (results/wla_7rep_20260930/*.log lines 2-4).  With fewer lanes than
    requests a lane is reused and reset when its next request is admitted, so
    every request starts cold as its own hot cache does in the reference."""
    R, L, S, SEL, HOT = 48, 12, 16, 64, 128
    sels = F.refgen_selections(R, L, S, SEL, 42)  # [R][S][L][sel]
    _, ref_miss, _, ref_total = O.ref_replay(R, L, S, SEL, HOT, 42)
    assert ref_total == 79550
    arrive = F.arrivals(F.ARRIVAL_BURSTY, R, 1.0)
    lanes = 20  # fewer lanes than requests: lanes are reused, so a lane starts cold
    sched = F.Sched(lanes, arrive, np.full(R, S, np.int32))
    ex = F.Executor(lanes, L, 1, SEL, HOT, 64 + 8 * S, q_heads=1, dtype=F.F32,
                    lru_mode=F.LRU_SERIAL, host_blocks=4099, value_std=1.0)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    flags = np.zeros((R, S, L, SEL), np.uint8)
    now, n_admitted = 0.0, 0
    while True:
        r = sched.tick(now)
        if r["done"]:
            break
        if len(r["admitted"]):
            ex.reset_owners(torch.tensor(r["admitted"], dtype=torch.int32, device="cuda"))
            n_admitted += len(r["admitted"])
        if r["resident"]:
            step_sel = np.full((lanes, L, 1, SEL), NONE, np.uint32)
            live = np.nonzero(r["lane_req"] >= 0)[0]
            for ln in live:
                step_sel[ln, :, 0, :] = sels[r["lane_req"][ln], r["lane_step"][ln]]
            dsel = torch.from_numpy(step_sel.view(np.int32)).cuda()
            ex.fetch_step(dsel, bufs)
            f = bufs["miss_flag"].cpu().numpy().reshape(lanes, L, SEL)
            for ln in live:
                flags[r["lane_req"][ln], r["lane_step"][ln]] = f[ln]
        now += 1.0
    a, _ = sched.request_ticks()
    assert n_admitted == R and np.all(a >= 0)
    st = ex.stats()
    assert st["device_error"] == 0
    assert st["misses"] == 79550 and st["selections"] == R * L * S * SEL
    assert np.array_equal(flags.reshape(-1), ref_miss)
