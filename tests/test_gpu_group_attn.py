"""Prefix-group attention on the GPU: one workgroup per (group, layer, kv head)
reads each distinct block of the group's set once and attends every member row
(FERRY_ATTN_GROUP).  Checked against the fp64 oracle (2e-3 relative, 1e-2 for
fp8) and against the per-row MFMA kernel (FERRY_ATTN_MFMA) of a twin executor
that went through the same fetch steps, so its pool holds the same bytes, with
four and with eight wavefronts per workgroup (FERRY_GROUP_WAVES; by default a
launch with no more group sets than CUs runs eight).

Slot tables are also edited by hand: a slot repeated in a row (attended twice),
slots of another group's set, empty positions, rows with nothing selected.
The oracle then attends over the host blocks those slots hold, read from the
pool's own tags (attention_hidx_f64).
"""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import TOL, Pair, _zipf_stream

pytestmark = pytest.mark.gpu

# (dtype, kv heads, q heads, group, requests): query tiles of 16 columns
# (group * G / 16) -> 4, 2, 4, 1, 2, 3
CASES = [
    (F.FP8, 2, 8, 16, 32),   # the shared-prefix fp8 shape: G 4, 64 columns
    (F.BF16, 2, 4, 16, 16),  # G 2, 32 columns
    (F.F16, 1, 8, 8, 16),    # G 8, 64 columns
    (F.FP8, 2, 8, 2, 6),     # G 4, 8 columns (half a tile)
    (F.F16, 2, 8, 5, 13),    # G 4, 20 columns; the last group has 3 members
    (F.BF16, 2, 8, 12, 28),  # G 4, 48 columns; the last group has 4 members
]
# group kernel against the per-row kernel: the same scores, but another
# summation order and other running maxima, so each rounds the fp16 weights
# (2^-11 relative) differently; half the tolerance either has to the oracle
ROW_TOL = {F.F16: 1e-3, F.BF16: 1e-3, F.FP8: 5e-3}


def _twins(dtype, Hkv, Hq, group, n_req, L=2, k=16, prefix=24, steps=3, waves=8):
    # waves: what the group launch runs; every case here fits the wider LDS
    # and launches fewer group sets than the GPU has CUs, so 8 unless forced
    # a set holds every block its members select in one step (at most group * k)
    cap = max(96, group * k + 32)
    print(f"[group-attn] dtype={dtype} Hkv={Hkv} Hq={Hq} group={group} B={n_req} C={cap}",
          flush=True)
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 120, steps, group=group, prefix=prefix)
    grp_pair = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, group=group, attn=F.ATTN_GROUP)
    row_pair = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, group=group, attn=F.ATTN_MFMA)
    assert grp_pair.ex.attn_kernel() == (F.ATTN_GROUP, waves)
    assert row_pair.ex.attn_kernel() == (F.ATTN_MFMA, 4)
    for sel in sels:
        grp_pair.check_fetched_bytes(grp_pair.step(sel))
        row_pair.step(sel)
    return grp_pair, row_pair, sels[-1]


def _decode(p, q, slots):
    out = torch.empty_like(q)
    p.ex.sparse_decode(q, slots, out)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == 0
    return out.cpu().numpy().reshape(-1, 128).astype(np.float64)


def _rel(a, b):
    den = np.maximum(np.abs(b).max(axis=1), 1e-30)
    return np.abs(a - b).max(axis=1) / den


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("dtype,Hkv,Hq,group,n_req", CASES)
def test_group_kernel_matches_oracle_and_row_kernel(dtype, Hkv, Hq, group, n_req, waves,
                                                    monkeypatch):
    monkeypatch.setenv("FERRY_GROUP_WAVES", str(waves))
    gp, rp, sel = _twins(dtype, Hkv, Hq, group, n_req, waves=waves)
    _check_twins(gp, rp, sel, dtype, Hq, n_req, seed=group)


def _check_twins(gp, rp, sel, dtype, Hq, n_req, seed):
    g = gp.g
    rng = np.random.default_rng(seed)
    q = torch.from_numpy(rng.standard_normal((n_req, g.n_layers, Hq, 128)).astype(np.float32)).cuda()
    got = _decode(gp, q, gp.bufs["slots"])
    row = _decode(rp, q, rp.bufs["slots"])
    ref = O.attention_f64(g, sel, q.cpu().numpy()).reshape(-1, 128)
    assert np.all(np.isfinite(got))
    assert _rel(got, ref).max() < TOL[dtype]
    assert _rel(got, row).max() < ROW_TOL[dtype]
    # the list and its order do not depend on the order the atomics ran in
    assert np.array_equal(got, _decode(gp, q, gp.bufs["slots"]))


@pytest.mark.parametrize("waves", [4, 8])
def test_group_kernel_many_repeats_at_large_k(waves, monkeypatch):
    # 256 selections per row drawn with replacement from contexts of 40-120
    # blocks: most of a row repeats, and every repeat is an entry of its own,
    # placed after the earlier members' entries by its member's row alone
    monkeypatch.setenv("FERRY_GROUP_WAVES", str(waves))
    gp, rp, sel = _twins(F.FP8, 2, 8, 4, 8, L=1, k=256, waves=waves)
    rows = sel.reshape(-1, 256)
    repeats = sum(256 - np.unique(r).size for r in rows)
    assert repeats > 100 * rows.shape[0], repeats
    _check_twins(gp, rp, sel, F.FP8, 8, 8, seed=11)


def _hidx_of_slots(p, slots):
    """Host-tier index of the block each pool slot holds (NONE64 for EMPTY)."""
    fill, _, tag = p.ex.sets_state()
    C_ = p.g.cap
    flat = slots.reshape(-1).astype(np.int64)
    out = np.full(flat.size, O.NONE64, np.uint64)
    for i, s in enumerate(flat):
        if s == F.EMPTY:
            continue
        st, loc = divmod(int(s), C_)
        assert loc < fill[st]
        out[i] = O.host_index(p.g, st, int(tag[st, loc]))
    return out.reshape(slots.shape)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("dtype,Hkv,Hq,group,n_req", [CASES[0], CASES[4], CASES[5]])
def test_group_kernel_edited_slot_tables(dtype, Hkv, Hq, group, n_req, waves, monkeypatch):
    monkeypatch.setenv("FERRY_GROUP_WAVES", str(waves))
    gp, rp, _ = _twins(dtype, Hkv, Hq, group, n_req, waves=waves)
    g = gp.g
    k, L = g.k, g.n_layers
    slots = gp.bufs["slots"].cpu().numpy().view(np.uint32).reshape(n_req, L, Hkv, k).copy()
    assert np.array_equal(slots, rp.bufs["slots"].cpu().numpy().view(np.uint32).reshape(slots.shape))
    rng = np.random.default_rng(7)
    n_own = (n_req + group - 1) // group
    for r in range(n_req):
        for l in range(L):
            for h in range(Hkv):
                row = slots[r, l, h]
                kind = (r + 3 * l + h) % 5
                if kind == 0:    # repeats: positions 1..3 repeat position 0
                    row[1:4] = row[0]
                elif kind == 1:  # slots of the next owner's set (another group's blocks)
                    o2 = (r // group + 1) % n_own
                    other = slots[min(o2 * group, n_req - 1), l, h]
                    row[::3] = other[::3]
                elif kind == 2:  # empty positions in the middle and at the end
                    row[rng.choice(k, k // 3, replace=False)] = F.EMPTY
                elif kind == 3 and r % 4 == 1:  # nothing selected
                    row[:] = F.EMPTY
    ds = torch.from_numpy(slots.view(np.int32)).cuda()
    q = torch.from_numpy(rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)).cuda()
    got = _decode(gp, q, ds)
    row = _decode(rp, q, ds)
    ref = O.attention_hidx_f64(g, _hidx_of_slots(gp, slots), q.cpu().numpy()).reshape(-1, 128)
    empty = np.all(slots == F.EMPTY, axis=-1)  # [B][L][Hkv]
    z = np.repeat(empty.reshape(-1), Hq // Hkv)
    assert np.all(got[z] == 0.0) and np.all(row[z] == 0.0)
    assert _rel(got[~z], ref[~z]).max() < TOL[dtype]
    assert _rel(got[~z], row[~z]).max() < ROW_TOL[dtype]


def test_group_kernel_reports_slots_outside_the_pool():
    gp, _, _ = _twins(F.FP8, 2, 8, 4, 8)
    slots = gp.bufs["slots"].cpu().numpy().view(np.uint32).copy()
    slots.reshape(-1)[5] = np.uint32(gp.ex.n_sets * gp.g.cap)  # one past the pool
    q = torch.zeros((8, gp.g.n_layers, 8, 128), device="cuda")
    out = torch.empty_like(q)
    gp.ex.sparse_decode(q, torch.from_numpy(slots.view(np.int32)).cuda(), out)
    torch.cuda.synchronize()
    assert gp.ex.stats()["device_error"] == -3  # FERRY_ERANGE


def test_group_kernel_limits():
    # FERRY_ATTN_GROUP is refused where the kernel cannot run
    with pytest.raises(F.FerryError, match="prefix-group"):
        F.Executor(4, 1, 2, 16, 64, 64, q_heads=8, group=1, dtype=F.FP8, attn=F.ATTN_GROUP)
    with pytest.raises(F.FerryError, match="prefix-group"):  # 16 members x 8 heads > 64 columns
        F.Executor(16, 1, 1, 16, 64, 64, q_heads=8, group=16, dtype=F.F16, attn=F.ATTN_GROUP)
    with pytest.raises(F.FerryError, match="16/8-bit KV"):
        F.Executor(4, 1, 2, 16, 64, 64, q_heads=8, group=4, dtype=F.F32, attn=F.ATTN_GROUP)


def test_auto_picks_the_group_kernel_where_it_fits():
    auto = F.Executor(8, 1, 2, 16, 96, 96, q_heads=8, group=4, dtype=F.FP8)
    assert auto.attn_kernel() == (F.ATTN_GROUP, 8)  # 4 group sets: eight wavefronts
    # 2 groups x 32 layers x 8 kv heads = 512 group sets, more than the CUs: four
    many = F.Executor(8, 32, 8, 16, 96, 96, q_heads=32, group=4, dtype=F.FP8)
    assert many.attn_kernel() == (F.ATTN_GROUP, 4)
    solo = F.Executor(8, 1, 2, 16, 96, 96, q_heads=8, group=1, dtype=F.FP8)
    assert solo.attn_kernel() == (F.ATTN_MFMA, 4)
    wide = F.Executor(16, 1, 1, 16, 96, 96, q_heads=8, group=16, dtype=F.FP8)  # 128 columns
    assert wide.attn_kernel() == (F.ATTN_MFMA, 4)
    mha = F.Executor(8, 1, 2, 16, 96, 96, q_heads=2, group=4, dtype=F.F16)  # G 1: vector ALUs
    assert mha.attn_kernel() == (F.ATTN_VALU, 4)
    mha8 = F.Executor(8, 1, 2, 16, 96, 96, q_heads=2, group=4, dtype=F.FP8)  # fp8 G 1: MFMA
    assert mha8.attn_kernel() == (F.ATTN_MFMA, 4)
