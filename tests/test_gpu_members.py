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
within the dtype's tolerance of the float64 oracle.  The member masks (own_mask,
src/runtime/wla_multigpu.cuh:1871-1912) must equal the oracle's too, and a
request moved between executors carries only the blocks it alone touched."""
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
        # member masks of the resident slots (own_mask after touches, releases and moves)
        own, oown = self.ex.sets_own(), self.ox.own()
        live = np.arange(self.C)[None, :] < fill[:, None]
        assert np.array_equal(own[live], oown[live])
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


def _image_layout(S, C, dtype):
    """Byte offsets of an owner image: header, fill[S], start[S], ord, tag and
    own [S*C] u32, fp8 scales [S*C][2], data from a 256-byte boundary."""
    N = S * C
    lay = dict(fill=64)
    lay["start"] = lay["fill"] + 4 * S
    lay["ord"] = lay["start"] + 4 * S
    lay["tag"] = lay["ord"] + 4 * N
    lay["own"] = lay["tag"] + 4 * N
    lay["scales"] = lay["own"] + 4 * N
    lay["data"] = (lay["scales"] + (8 * N if dtype == F.FP8 else 0) + 255) // 256 * 256
    return lay


def _u32_at(im, off, n):
    return im[off:off + 4 * n].view(np.uint32)


@pytest.mark.parametrize("dtype,cap_mode", [(F.FP8, F.CAP_PER_MEMBER), (F.BF16, F.CAP_GROUP)])
def test_member_carry_between_executors(dtype, cap_mode):
    """One request of a prefix group moves from executor A to B, carrying only
    the blocks it alone touched (kv_handoff_owned, src/runtime/wla_multigpu.cuh:
    1996-2016): the image must list the oracle's exclusive blocks in LRU order
    with the host tier's bytes; after leave on A and join + merge on B both
    executors' sets, member masks and pool bytes equal the oracle's, and four
    more steps (the request now in B) stay bit-exact."""
    lanes, grp, L, Hkv, Hq, k, share, pre = 8, 4, 2, 2, 8, 16, 24, 48
    mv = 1  # lane of owner 0, member bit 1 << 1
    S = L * Hkv
    print(f"[member carry] dtype={dtype} cap_mode={cap_mode} lane={mv}", flush=True)
    ctx = np.full(lanes, 80 + pre, np.int32)
    sga = F.SelGen(lanes, L, Hkv, k, ctx, group=grp, prefix_blocks=pre, seed=4)
    sgb = F.SelGen(lanes, L, Hkv, k, ctx, group=grp, prefix_blocks=pre, seed=9)
    assert sga.max_blocks == sgb.max_blocks
    mb = sga.max_blocks
    A = GroupPair(lanes, grp, L, Hkv, Hq, k, share, mb, dtype, cap_mode)
    B = GroupPair(lanes, grp, L, Hkv, Hq, k, share, mb, dtype, cap_mode)
    B.leave([mv])  # the lane is free on B until the request arrives
    shape = (lanes, L, Hkv, k)
    for t in range(6):
        A.step(sga.step(t).reshape(-1))
        sb = sgb.step(t).reshape(shape).copy()
        sb[mv] = NONE
        B.step(sb.reshape(-1))
    A.check_state()
    B.check_state()
    img = A.ex.alloc_owner_image()
    A.ex.owner_export_member(mv, img)
    counts, blocks = A.ox.export_member(mv)
    torch.cuda.synchronize()
    assert A.ex.stats()["device_error"] == 0
    im = img.cpu().numpy()
    lay = _image_layout(S, A.C, dtype)
    hdr = im[:64].view(np.uint32)
    assert hdr[0] == 0x4E574F46 and hdr[1] == S and hdr[2] == A.C and hdr[8] == 1 << mv
    assert int(im[24:32].view(np.uint64)[0]) == int(counts.sum())
    assert 0 < counts.sum() < A.ox.state()[0][:S].sum()  # some blocks stay behind
    assert np.array_equal(_u32_at(im, lay["fill"], S), counts)
    start = _u32_at(im, lay["start"], S)
    assert np.array_equal(start, np.concatenate([[0], np.cumsum(counts)[:-1]]))
    afill, aord, atag = A.ex.sets_state()
    n = int(counts.sum())
    itag, iord = _u32_at(im, lay["tag"], n), _u32_at(im, lay["ord"], n)
    assert np.all(_u32_at(im, lay["own"], n) == 1 << mv)
    sets = np.repeat(np.arange(S), counts)
    assert np.array_equal(itag, np.concatenate([blocks[s, :counts[s]] for s in range(S)]))
    assert np.array_equal(atag[sets, iord], itag)  # each slot is where A holds the block
    hidx = (sets.astype(np.int64) * mb + itag) % 4099
    bb = A.ex.block_bytes
    assert np.array_equal(im[lay["data"]:lay["data"] + n * bb].reshape(n, bb), A.hostb[hidx])
    if dtype == F.FP8:
        isc = im[lay["scales"]:lay["scales"] + 8 * n].view(np.float32).reshape(n, 2)
        assert np.array_equal(isc, A.hsc[hidx])
    # the request leaves A and joins B, whose group merges its blocks
    A.leave([mv])
    B.join([mv])
    before = B.ox.state()[0][:S].copy()
    resident = sum(int(np.isin(blocks[s, :counts[s]], B.ox.state()[2][s, :before[s]]).sum())
                   for s in range(S))
    B.ex.owner_import_member(mv, img)
    B.ox.import_member(mv, counts, blocks)
    B.check_state()
    after = B.ox.state()[0][:S]
    evicted = int(before.sum()) + n - resident - int(after.sum())
    print(f"[member carry] {n} blocks carried, {resident} already resident on B, "
          f"{evicted} evicted", flush=True)
    assert resident > 0
    if cap_mode == F.CAP_GROUP:
        assert evicted > 0
    for t in range(6, 10):
        sa = sga.step(t).reshape(shape).copy()
        sb = sgb.step(t).reshape(shape).copy()
        sb[mv] = sa[mv]
        sa[mv] = NONE
        A.step(sa.reshape(-1))
        B.step(sb.reshape(-1))
    A.check_state()
    B.check_state()
    B.check_attention(sb.reshape(-1), seed=11)
    # a whole-owner image carries the member masks too
    whole = B.ex.alloc_owner_image()
    B.ex.owner_export(0, whole)
    C2 = GroupPair(lanes, grp, L, Hkv, Hq, k, share, mb, dtype, cap_mode)
    C2.ex.owner_import(0, whole)
    torch.cuda.synchronize()
    assert C2.ex.stats()["device_error"] == 0
    bf, bo, bt = B.ex.sets_state()
    cf, co, ct = C2.ex.sets_state()
    assert np.array_equal(cf[:S], bf[:S]) and np.array_equal(ct[:S], bt[:S])
    live = np.arange(B.C)[None, :] < bf[:S, None]
    assert np.array_equal(C2.ex.sets_own()[:S][live], B.ex.sets_own()[:S][live])


def test_member_carry_refusals():
    p = GroupPair(4, 2, 1, 1, 2, 8, 8, 40, F.F16, F.CAP_GROUP)
    img = p.ex.alloc_owner_image()
    p.ex.owner_export(1, img)  # a whole-owner image
    p.ex.owner_import_member(0, img)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -1
    q = GroupPair(4, 2, 1, 1, 2, 8, 8, 40, F.F16, F.CAP_GROUP)
    q.ex.owner_export_member(3, img)  # a member image
    q.ex.owner_import(1, img)
    torch.cuda.synchronize()
    assert q.ex.stats()["device_error"] == -1
    with pytest.raises(F.FerryError):
        q.ex.owner_export_member(4, img)  # no such lane
    solo = F.Executor(2, 1, 1, 8, 8, 40, q_heads=1, dtype=F.F16, host_blocks=64)
    with pytest.raises(F.FerryError):
        solo.owner_export_member(0, solo.alloc_owner_image())  # no prefix groups
    with pytest.raises(F.FerryError):
        solo.sets_own()


def test_members_refusals_latch_einval():
    p = GroupPair(4, 2, 1, 1, 2, 8, 8, 40, F.F16, F.CAP_PER_MEMBER)
    p.ex.members_join(torch.tensor([1], dtype=torch.int32, device="cuda"))  # already resident
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -1
    assert list(p.ex.members()) == [2, 2]
