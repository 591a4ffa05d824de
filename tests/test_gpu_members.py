"""Prefix groups whose members come and go, on the GPU against the oracle.

Requests arrive (Poisson or Markov-modulated, virtual clock) and each runs in
its group's lanes (request r in lane r mod lanes, so a lane stays in one prefix
group): a finishing request leaves its group (ferry_members_leave), an arriving
one joins it (ferry_members_join) with a fresh private id range, and the
group's sets are never reset, so members keep hitting the shared prefix.
With per-member capacity (MissSpec::cap_mode 1, src/workloads/missstream.cuh:
40-47, 91-94) a leave trims the group's sets to one share per remaining member
(grp_trim, src/runtime/wla_multigpu.cuh:1923-1936), moving surviving blocks
into lower slots.  Every tick the slots, miss lists and flags must equal the
oracle's bit for bit, the LRU state and member counts after every change, the
bytes (and fp8 scales) of every resident slot the host tier's, and attention
within the dtype's tolerance of the float64 oracle."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import TOL

pytestmark = pytest.mark.gpu

NONE = O.NONE


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


class GroupPair:
    def __init__(self, lanes, grp, L, Hkv, Hq, k, share, max_blocks, dtype, cap_mode):
        self.C = share * grp
        self.ex = F.Executor(lanes, L, Hkv, k, self.C, max_blocks, q_heads=Hq, group=grp,
                             dtype=dtype, host_blocks=4099, cap_mode=cap_mode)
        self.g = O.make_geom(n_req=lanes, group=grp, n_layers=L, kv_heads=Hkv, q_heads=Hq, k=k,
                             cap=self.C, max_blocks=max_blocks, dtype=dtype, host_blocks=4099,
                             cap_mode=cap_mode)
        self.ox = O.Executor(self.g)
        self.ex.hosttier_fill()
        self.bufs = self.ex.alloc_step_buffers()
        torch.cuda.synchronize()
        host, hsc = self.ex.hosttier_array()
        self.hostb = host.reshape(4099, -1)
        self.hsc = None if hsc is None else hsc.reshape(4099, 2)
        self.dtype = dtype

    def leave(self, lanes):
        self.ex.members_leave(torch.tensor(lanes, dtype=torch.int32, device="cuda"))
        assert self.ox.members_leave(lanes)
        self.check_state()

    def join(self, lanes):
        self.ex.members_join(torch.tensor(lanes, dtype=torch.int32, device="cuda"))
        assert self.ox.members_join(lanes)

    def step(self, sel):
        ex = self.ex
        ex.fetch_step(torch.from_numpy(np.ascontiguousarray(sel).view(np.int32)).cuda(), self.bufs)
        torch.cuda.synchronize()
        st = ex.stats()
        assert st["device_error"] == 0, st
        oslots, omc, oms, _ = self.ox.step(sel)
        assert np.array_equal(_u32(self.bufs["slots"]).reshape(-1), oslots)
        assert np.array_equal(_u32(self.bufs["miss_count"]), omc)
        assert np.array_equal(self.bufs["miss_flag"].cpu().numpy().reshape(-1), self.ox.last_flags)
        oms4 = oms.view(np.uint32).reshape(self.ox.n_sets, -1, 4)
        gms = _u32(self.bufs["misses"]).reshape(self.ox.n_sets, -1, 4)
        live = np.arange(oms4.shape[1])[None, :] < omc[:, None]
        assert np.array_equal(gms[live], oms4[live])
        return int(omc.sum())

    def check_state(self):
        torch.cuda.synchronize()
        assert self.ex.stats()["device_error"] == 0
        fill, ord_, tag = self.ex.sets_state()
        ofill, oord, otag = self.ox.state()
        assert np.array_equal(fill, ofill) and np.array_equal(tag, otag)
        for s in range(len(fill)):
            assert np.array_equal(ord_[s, :fill[s]], oord[s, :fill[s]])
        assert np.array_equal(self.ex.members(), self.ox.members())
        # every resident slot holds its block's bytes (moved ones included)
        sets = np.repeat(np.arange(len(fill)), fill)
        loc = np.concatenate([np.arange(f) for f in fill]) if fill.sum() else np.zeros(0, int)
        if sets.size:
            gslots = sets.astype(np.int64) * self.C + loc
            hidx = (sets.astype(np.int64) * self.g.max_blocks + otag[sets, loc]) % 4099
            assert np.array_equal(self.ex.pool_slots_bytes(gslots), self.hostb[hidx])
            if self.hsc is not None:
                assert np.array_equal(self.ex.pool_slot_scales(gslots), self.hsc[hidx])

    def check_attention(self, sel, seed):
        g = self.g
        q = np.random.default_rng(seed).standard_normal(
            (g.n_req, g.n_layers, g.q_heads, 128)).astype(np.float32)
        dq = torch.from_numpy(q).cuda()
        out = torch.full_like(dq, float("nan"))
        self.ex.sparse_decode(dq, self.bufs["slots"], out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
        ref = O.attention_f64(g, sel, q).reshape(-1, 128)
        empty = np.all(ref == 0.0, axis=1)
        assert np.all(got[empty] == 0.0)
        rel = np.abs(got[~empty] - ref[~empty]).max(axis=1) / np.abs(ref[~empty]).max(axis=1)
        assert rel.max() < TOL[self.dtype], rel.max()


@pytest.mark.parametrize("kind,dtype,cap_mode", [
    (F.ARRIVAL_POISSON, F.BF16, F.CAP_PER_MEMBER),
    (F.ARRIVAL_MMPP, F.FP8, F.CAP_PER_MEMBER),
    (F.ARRIVAL_MMPP, F.F16, F.CAP_GROUP),
])
def test_prefix_groups_turn_over_under_arrivals(kind, dtype, cap_mode):
    lanes, grp, L, Hkv, Hq, k, share, pre = 8, 4, 2, 2, 8, 16, 24, 48
    n = 28
    print(f"[members] kind={kind} dtype={dtype} cap_mode={cap_mode} lanes={lanes} group={grp}",
          flush=True)
    arrive = F.arrivals(kind, n, 0.6, 4.0, 10.0, seed=3)
    arrive[:lanes] = 0.0
    lens = F.ctx_uniform(5, n, 3, 9)
    ctx_req = F.ctx_uniform(6, n, 30, 80) + pre
    sg = F.SelGen(lanes, L, Hkv, k, np.full(lanes, 80 + pre, np.int32), group=grp,
                  prefix_blocks=pre, seed=4)
    og = O.selgen(lanes, L, Hkv, k, np.full(lanes, 80 + pre, np.int32), group=grp,
                  prefix_blocks=pre, seed=4)
    ranges = n // (lanes // grp) + grp
    sg.set_private_ranges(ranges)
    O.selgen_group_turnover(og, ranges)
    assert sg.max_blocks == O.selgen_max_blocks(og)
    p = GroupPair(lanes, grp, L, Hkv, Hq, k, share, sg.max_blocks, dtype, cap_mode)
    # start empty: every lane leaves, then requests join as they are admitted
    p.leave(list(range(lanes)))
    for ln in range(lanes):
        sg.retire(ln)
        O.selgen_retire(og, ln)
    sched = F.Sched(lanes, arrive, lens, pinned=True)
    next_range = [0] * (lanes // grp)
    steps = joins = leaves = trims = 0
    prev_live = np.zeros(lanes, bool)
    for t in range(200):
        r = sched.tick(float(t))
        gone = [int(x) for x in r["retired"]]
        came = [int(x) for x in r["admitted"]]
        # a lane whose request finished and that took the next one in the same
        # tick leaves and joins: the old request leaves first
        out = gone + [ln for ln in came if prev_live[ln]]
        if out:
            before = p.ex.sets_state()[0].copy()
            p.leave(out)
            leaves += len(out)
            trims += int((p.ex.sets_state()[0] < before).any())
        for ln in gone:
            sg.retire(ln)
            O.selgen_retire(og, ln)
        if came:
            p.join(came)
            joins += len(came)
            for ln in came:
                rid, o = int(r["lane_req"][ln]), ln // grp
                sg.admit_member(ln, rid, int(ctx_req[rid]), t, next_range[o])
                O.selgen_admit_member(og, ln, rid, int(ctx_req[rid]), t, next_range[o])
                next_range[o] += 1
        prev_live = r["lane_req"] >= 0
        if r["resident"] == 0:
            if r["done"]:
                break
            continue
        sel = sg.step(t).reshape(-1)
        assert np.array_equal(sel, O.selgen_step(og, t))
        p.step(sel)
        steps += 1
        if steps % 4 == 1:
            p.check_state()
            p.check_attention(sel, seed=t)
    assert r["done"]
    p.check_state()
    assert joins == n and leaves == n
    if cap_mode == F.CAP_PER_MEMBER:
        assert trims > 0
    print(f"[members] {steps} steps, {joins} joins, {leaves} leaves, {trims} trims", flush=True)


def test_members_refusals_latch_einval():
    p = GroupPair(4, 2, 1, 1, 2, 8, 8, 40, F.F16, F.CAP_PER_MEMBER)
    p.ex.members_join(torch.tensor([1], dtype=torch.int32, device="cuda"))  # already resident
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -1
    assert list(p.ex.members()) == [2, 2]
