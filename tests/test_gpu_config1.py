"""The CPU-plumbing configuration as stated, on the GPU against the oracle.

1 layer, 8 kv heads MHA, head_dim 128, fp32 KV, 16-token blocks; 4 request
lanes with 2048-token contexts (128 blocks); every step each (request, head)
selects 32 blocks uniformly without replacement; 1000 decode steps with
requests arriving by a Poisson process at 200/s.

Residency: the configuration draws each selected block non-resident with
probability 0.25.  Here residency is the executor's LRU: with selections
uniform over a row's 128 blocks and 96 slots per (request, head) set, an LRU
under independent uniform references holds any given block with probability
96/128 = 0.75 in steady state, so a selected block misses with probability
0.25 -- the test measures it.  (The stated "pools of 512 blocks" cannot hold
one step's 4 x 8 x 32 selections.)

The tick loop runs on a virtual 1 ms clock: 1000 ticks are one second of
arrivals at 200/s, about 200 requests, each decoding U[8, 24] steps in one of
the 4 lanes (served at ~250/s).  Every tick: the scheduler and the selection
generator equal the oracle's, admitted lanes are reset on both sides, and the
slots, miss lists, miss flags and fetched bytes are bit-exact; every 50 ticks
the LRU state and the attention (2e-3 of fp64) too.
"""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import Pair

pytestmark = pytest.mark.gpu

LANES, L, H, K, CTX, C = 4, 1, 8, 32, 128, 96
TICKS, RATE_PER_S = 1000, 200.0


def _attention(p, sel, seed):
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
    assert rel.max() < 2e-3, rel.max()


def test_config1_thousand_steps_with_poisson_arrivals():
    gap_ms = 1000.0 / RATE_PER_S
    n = int(TICKS / gap_ms * 1.2)  # enough arrivals to cover the second
    arrive = F.arrivals(F.ARRIVAL_POISSON, n, gap_ms, seed=11)
    arrive = arrive[arrive < TICKS]
    n = arrive.size
    lens = F.ctx_uniform(12, n, 8, 24)
    print(f"[config1] {n} requests over {TICKS} ticks, lanes {LANES}, C {C}", flush=True)
    sched = F.Sched(LANES, arrive, lens)
    clock = np.arange(TICKS, dtype=np.float64)
    otable, oadmit, olast = O.sched_run(LANES, arrive, lens, clock)
    ctx = np.full(LANES, CTX, np.int32)
    sg = F.SelGen(LANES, L, H, K, ctx, dist=0, reuse=0.0, seed=13)
    og = O.selgen(LANES, L, H, K, ctx, dist=0, reuse=0.0, seed=13)
    p = Pair(LANES, L, H, H, K, C, sg.max_blocks, F.F32, host_blocks=4099)
    for ln in range(LANES):
        sg.retire(ln)
        O.selgen_retire(og, ln)
    steps = sel_total = miss_total = 0
    warm_sel = warm_miss = 0  # requests past their 8th step: the LRU's steady state
    for t, now in enumerate(clock):
        r = sched.tick(now)
        assert np.array_equal(r["lane_req"], otable[t])
        for ln in r["retired"]:
            sg.retire(ln)
            O.selgen_retire(og, ln)
        if len(r["admitted"]):
            new = [int(x) for x in r["admitted"]]
            for ln in new:
                rid = int(r["lane_req"][ln])
                sg.admit(ln, rid, CTX, t)
                O.selgen_admit(og, ln, rid, CTX, t)
                p.ox.reset_owner(ln)
            p.ex.reset_owners(torch.tensor(new, dtype=torch.int32, device="cuda"))
        if r["resident"] == 0:
            continue
        sel = sg.step(t).reshape(-1)
        assert np.array_equal(sel, O.selgen_step(og, t))
        rows = sel.reshape(LANES, L * H * K)
        live = rows[:, 0] != O.NONE
        # uniform without replacement: K distinct ids in [0, CTX) per live row
        for row in sel.reshape(-1, K)[np.repeat(live, L * H)]:
            assert len(np.unique(row)) == K and row.max() < CTX
        p.check_fetched_bytes(p.step(sel))
        steps += 1
        flags = p.bufs["miss_flag"].cpu().numpy().reshape(LANES, L * H * K)
        sel_total += int(live.sum()) * L * H * K
        miss_total += int(flags[live].sum())
        old = live & (r["lane_step"] >= 8)
        warm_sel += int(old.sum()) * L * H * K
        warm_miss += int(flags[old].sum())
        if steps % 50 == 1:
            p.check_state()
            _attention(p, sel, seed=t)
    a, d = sched.request_ticks()
    assert list(a) == oadmit and list(d) == olast
    st = p.ex.stats()
    assert st["device_error"] == 0 and st["steps"] == steps
    assert st["selections"] == sel_total and st["misses"] == miss_total
    warm = warm_miss / warm_sel
    print(f"[config1] {steps} decode steps, {sel_total} selections, miss rate "
          f"{miss_total / sel_total:.4f} (steady {warm:.4f} over {warm_sel} selections)",
          flush=True)
    assert steps >= 900  # the lanes are busy nearly every tick
    assert abs(warm - 0.25) < 0.02
