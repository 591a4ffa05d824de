"""Resident members of prefix groups and capacity that follows them, in the
oracle (CPU).  Under per-member capacity (MissSpec::cap_mode 1,
src/workloads/missstream.cuh:40-47, 91-94) an owner's sets hold one share of
slots per resident member; a member leaving trims the group's LRU to the new
capacity, least recent first (grp_trim, src/runtime/wla_multigpu.cuh:
1923-1936), and kv_touch evicts while the set holds its capacity or more
(:1937-1962).

Pins:
  * the executor's set engine, one selection per sub-step, equals a plain
    deque restating kv_touch and grp_trim (ora_deque_lru_run_caps) over random
    streams with members leaving and joining: every hit/miss flag, and the
    final LRU order of blocks;
  * a trim leaves exactly the capacity's most recent blocks in their order,
    in slots [0, capacity): survivors below the capacity keep their slot, the
    ones above move into the freed slots below, in ascending order on both
    sides (the rule the device kernel follows), and the block map agrees;
  * member bookkeeping refuses leaving a lane that is not resident and
    joining one that is."""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as O

NONE = O.NONE


def _blocks_in_order(ox, set_id=0):
    fill, ord_, tag = ox.state()
    return tag[set_id, ord_[set_id, : fill[set_id]]]


@pytest.mark.parametrize("seed", range(12))
def test_serial_engine_with_members_equals_deque(seed):
    rng = np.random.default_rng(seed)
    grp = int(rng.integers(2, 6))
    share = int(rng.integers(2, 9))
    k = int(rng.integers(1, share + 1))  # a step's blocks always fit its members' shares
    nb = int(rng.integers(share + 2, 6 * share * grp))
    g = O.make_geom(n_req=grp, group=grp, n_layers=1, kv_heads=1, k=k, cap=share * grp,
                    max_blocks=nb, dtype=O.F32, granularity=1, cap_mode=1)
    ox = O.Executor(g)
    live = np.ones(grp, bool)
    caps, trims, stream, flags = [], [], [], []
    low = share * grp
    for step in range(60):
        # members come and go between steps (never more than the group); the
        # smallest capacity since the last touch is what the leaves trimmed to
        for ln in range(grp):
            if rng.random() < 0.15:
                if live[ln]:
                    assert ox.members_leave([ln])
                else:
                    assert ox.members_join([ln])
                live[ln] = not live[ln]
                low = min(low, share * max(1, int(live.sum())))
        cap = share * max(1, int(live.sum()))
        assert O.lib.ora_capacity(C.byref(g), int(live.sum())) == cap
        sel = np.full((grp, 1, 1, k), NONE, np.uint32)
        for ln in np.nonzero(live)[0]:
            sel[ln, 0, 0] = rng.integers(0, nb, k)
        ox.step(sel.reshape(-1))
        for ln in range(grp):  # canonical order: member by member
            for j in range(k):
                if sel[ln, 0, 0, j] != NONE:
                    stream.append(int(sel[ln, 0, 0, j]))
                    trims.append(low)
                    low = cap
                    caps.append(cap)
                    flags.append(int(ox.last_flags[ln * k + j]))
    x = np.array(stream, np.uint32)
    ref_flags = np.zeros(len(x), np.uint8)
    final = np.zeros(max(caps) + 1, np.uint32)
    n = O.lib.ora_deque_lru_run_caps(np.array(trims, np.int32), np.array(caps, np.int32), x,
                                     len(x), ref_flags, final)
    assert np.array_equal(np.array(flags, np.uint8), ref_flags)
    assert np.array_equal(_blocks_in_order(ox), final[:n])
    assert (ox.members() == live.sum()).all()


@pytest.mark.parametrize("seed", range(8))
def test_trim_keeps_recent_blocks_and_compacts_slots(seed):
    rng = np.random.default_rng(100 + seed)
    cap, nb = int(rng.integers(8, 60)), 500
    s = O.LRU()
    assert O.lib.ora_lru_init(C.byref(s), cap, nb) == 0
    slot = np.zeros(64, np.uint32)
    miss = np.zeros(64, O.MISS_DTYPE)
    nm = C.c_int()
    for _ in range(30):  # random history, one selection per sub-step
        x = np.array([rng.integers(0, nb)], np.uint32)
        assert O.lib.ora_lru_substep(C.byref(s), 0, x, 1, slot, miss, C.byref(nm), None) == 0
    fill = s.fill
    ord0 = np.ctypeslib.as_array(s.ord, (cap,))[:fill].copy()
    tag0 = np.ctypeslib.as_array(s.tag, (cap,)).copy()
    lim = int(rng.integers(1, fill)) if fill > 1 else 1
    moves = np.zeros(2 * cap, np.uint32)
    n = O.lib.ora_lru_trim(C.byref(s), lim, moves.ctypes.data)
    ordn = np.ctypeslib.as_array(s.ord, (cap,))
    tagn = np.ctypeslib.as_array(s.tag, (cap,))
    mapn = np.ctypeslib.as_array(s.map, (nb,))
    survivors = ord0[fill - lim:]
    # the most recent `lim` blocks, in their order, in slots [0, lim)
    assert s.fill == lim
    assert np.array_equal(tagn[ordn[:lim]], tag0[survivors])
    assert np.array_equal(np.sort(ordn[:lim]), np.arange(lim))
    assert np.all(tagn[lim:] == NONE) and np.all(ordn[lim:] == NONE)
    # survivors below the capacity keep their slot; the others moved, in order
    stay = survivors[survivors < lim]
    assert np.array_equal(tagn[stay], tag0[stay])
    movers = np.sort(survivors[survivors >= lim])
    pairs = moves[: 2 * n].reshape(-1, 2)
    assert np.array_equal(pairs[:, 0], movers)
    assert np.all(np.diff(pairs[:, 1].astype(np.int64)) > 0) and np.all(pairs[:, 1] < lim)
    assert np.array_equal(tagn[pairs[:, 1]], tag0[pairs[:, 0]])
    # the map points every resident block at its slot and forgets the rest
    resident = tagn[:lim]
    assert np.array_equal(mapn[resident], np.arange(lim))
    gone = np.setdiff1d(tag0[ord0], resident)
    assert np.all(mapn[gone] == NONE)
    O.lib.ora_lru_free(C.byref(s))


def test_members_refuse_double_leave_and_join():
    g = O.make_geom(n_req=6, group=3, n_layers=2, kv_heads=1, k=4, cap=12, max_blocks=50,
                    dtype=O.F16, cap_mode=1)
    ox = O.Executor(g)
    assert list(ox.members()) == [3, 3]
    assert ox.members_leave([1, 4])
    assert list(ox.members()) == [2, 2]
    assert not ox.members_leave([1])          # not resident: skipped
    assert not ox.members_join([0])           # resident: skipped
    assert not ox.members_leave([6])          # out of range
    assert list(ox.members()) == [2, 2]
    assert ox.members_join([1])
    assert list(ox.members()) == [3, 2]


def test_group_turnover_selections_match_oracle():
    """Prefix-group lanes turning over: the product's generator and the
    oracle's restatement give the same selections when members retire and new
    requests of the group take their lanes with fresh private id ranges."""
    import ferry_amd as F

    B, grp, L, H, k, pre = 8, 4, 2, 2, 16, 40
    ctx = F.ctx_uniform(3, B, 50, 120) + pre
    mine = F.SelGen(B, L, H, k, ctx, group=grp, prefix_blocks=pre, seed=9)
    ref = O.selgen(B, L, H, k, ctx, group=grp, prefix_blocks=pre, seed=9)
    mine.set_private_ranges(16)
    O.selgen_group_turnover(ref, 16)
    assert mine.max_blocks == O.selgen_max_blocks(ref)
    nperm = [int(ctx[o * grp:(o + 1) * grp].max()) for o in range(B // grp)]
    assert mine.max_blocks == max(pre + 16 * (n - pre) for n in nperm)
    rng = np.random.default_rng(2)
    next_range = [grp, grp]
    rid = B
    for t in range(12):
        if t and t % 3 == 0:
            for ln in rng.choice(B, 3, replace=False):
                ln = int(ln)
                o = ln // grp
                if rng.random() < 0.3:
                    mine.retire(ln)
                    O.selgen_retire(ref, ln)
                    continue
                c = int(rng.integers(pre + 1, nperm[o] + 1))
                mine.admit_member(ln, rid, c, t, next_range[o])
                O.selgen_admit_member(ref, ln, rid, c, t, next_range[o])
                rid += 1
                next_range[o] += 1
        if t == 10:  # every lane re-admitted with a short context: the owners'
            for ln in range(B):  # permutation domains stay their creation values
                o = ln // grp
                mine.admit_member(ln, rid, pre + 3, t, next_range[o])
                O.selgen_admit_member(ref, ln, rid, pre + 3, t, next_range[o])
                rid += 1
                next_range[o] += 1
        got = mine.step(t).reshape(-1)
        assert np.array_equal(got, O.selgen_step(ref, t)), t
        ids = got[got != NONE]
        assert ids.max() < mine.max_blocks
    # refusals: a range past the configured count, a context past the owner's
    with pytest.raises(F.FerryError):
        mine.admit_member(0, rid, pre + 1, 12, 16)
    with pytest.raises(F.FerryError):
        mine.admit_member(0, rid, nperm[0] + 1, 12, 3)


class _RefGroupSet:
    """The reference's state of one (gpu, group, layer) under own_carry,
    restated from its rules with a list and a dict (wla_multigpu.cuh:
    1871-1962): the LRU deque (front = least recent), and the mask of the
    members that touched each resident block (own_mask)."""

    def __init__(self):
        self.dq, self.mask = [], {}

    def touch(self, blk, bit, cap):  # kv_touch + own_mask |= own_bit(r)
        if blk in self.mask:
            self.dq.remove(blk)
            self.dq.append(blk)
        else:
            while len(self.dq) >= cap:  # own_drop with the eviction
                self.mask.pop(self.dq.pop(0))
            self.dq.append(blk)
            self.mask[blk] = 0
        self.mask[blk] |= bit

    def release(self, bit):  # own_release (a zero mask is a dead block, still resident)
        for b in self.mask:
            self.mask[b] &= ~bit

    def trim(self, cap):  # grp_trim
        while len(self.dq) > cap:
            self.mask.pop(self.dq.pop(0))

    def export(self, bit):  # the blocks kv_handoff_owned moves: mask == bit
        return [b for b in self.dq if self.mask[b] == bit]

    def merge(self, blocks, bit, cap):  # kv_handoff_owned at the consumer
        for b in blocks:
            if b in self.mask:
                self.mask[b] |= bit
                continue
            while len(self.dq) >= cap:
                self.mask.pop(self.dq.pop(0))
            self.dq.append(b)
            self.mask[b] = bit


def _compare(ox, model, per):
    fill, ord_, tag = ox.state()
    own = ox.own()
    for s in range(per):
        blocks = tag[s, ord_[s, :fill[s]]]
        assert list(blocks) == model[s].dq, s
        assert [int(own[s, v]) for v in ord_[s, :fill[s]]] == [model[s].mask[b] for b in blocks], s


@pytest.mark.parametrize("seed,cap_mode", [(s, m) for s in range(6) for m in (0, 1)])
def test_member_carry_equals_reference_rules(seed, cap_mode):
    """Serial (kv_touch) bookkeeping with member masks, members leaving and
    joining, and a member's exclusive blocks carried from one executor's group
    into another's: the oracle equals _RefGroupSet after every event."""
    rng = np.random.default_rng(300 + seed)
    grp, L, k = 4, 2, 3
    share = int(rng.integers(k, 3 * k))
    nb = int(rng.integers(2 * share, 8 * share))
    cap_slots = share * grp
    g = O.make_geom(n_req=grp, group=grp, n_layers=L, kv_heads=1, k=k, cap=cap_slots,
                    max_blocks=nb, dtype=O.F32, granularity=1, cap_mode=cap_mode)
    ex = {0: O.Executor(g), 1: O.Executor(g)}
    model = {e: [_RefGroupSet() for _ in range(L)] for e in ex}
    live = {e: np.ones(grp, bool) for e in ex}

    def cap_of(e):
        return share * max(1, int(live[e].sum())) if cap_mode else cap_slots

    def step(e):
        sel = np.full((grp, L, 1, k), NONE, np.uint32)
        for ln in np.nonzero(live[e])[0]:
            sel[ln, :, 0] = rng.integers(0, nb, (L, k))
        ex[e].step(sel.reshape(-1))
        for l in range(L):
            for ln in range(grp):
                for j in range(k):
                    if sel[ln, l, 0, j] != NONE:
                        model[e][l].touch(int(sel[ln, l, 0, j]), 1 << ln, cap_of(e))

    def leave(e, ln):
        assert ex[e].members_leave([ln])
        live[e][ln] = False
        for m in model[e]:
            m.release(1 << ln)
            if cap_mode:
                m.trim(cap_of(e))

    for t in range(40):
        for e in ex:
            for ln in range(grp):
                if rng.random() < 0.1:
                    if live[e][ln]:
                        leave(e, ln)
                    else:
                        assert ex[e].members_join([ln])
                        live[e][ln] = True
            step(e)
            _compare(ex[e], model[e], L)
        if t % 5 == 4:  # a member of executor 0 moves to a free lane of executor 1
            src = [ln for ln in range(grp) if live[0][ln]]
            dst = [ln for ln in range(grp) if not live[1][ln]]
            if not src or not dst:
                continue
            a, b = int(rng.choice(src)), int(rng.choice(dst))
            counts, blocks = ex[0].export_member(a)
            for l in range(L):
                assert list(blocks[l, :counts[l]]) == model[0][l].export(1 << a)
            leave(0, a)
            assert ex[1].members_join([b])
            live[1][b] = True
            ex[1].import_member(b, counts, blocks)
            for l in range(L):
                model[1][l].merge(list(blocks[l, :counts[l]]), 1 << b, cap_of(1))
            for e in ex:
                _compare(ex[e], model[e], L)
