"""The top-k block selection of the oracle (Quest bound,
tools/capture_miss_trace.py:139-159), pinned on the CPU by independent
computations: summaries against a numpy/torch decode of the host-tier block,
the bound against float64 arithmetic and against the true attention scores it
bounds, and the top-k choice against numpy's lexsort with the same tie rule."""
import numpy as np
import pytest
import torch

from oracle import pyoracle as O


def _geom(dtype, n_req=3, L=2, H=2, Hq=4, k=8, mb=64, host_blocks=4099):
    return O.make_geom(n_req=n_req, n_layers=L, kv_heads=H, q_heads=Hq, k=k, cap=k,
                       max_blocks=mb, dtype=dtype, host_blocks=host_blocks, value_std=0.7)


def _decode_block(g, h):
    """K tile [T][D] of host block h as float64, decoded with numpy/torch."""
    raw, sc = O.host_block(g, h)
    T, D = g.block_tokens, g.head_dim
    if g.dtype == O.F32:
        k = raw.view(np.float32)[:T * D].astype(np.float64)
    elif g.dtype == O.F16:
        k = raw.view(np.float16)[:T * D].astype(np.float64)
    elif g.dtype == O.BF16:
        k = (raw.view(np.uint16)[:T * D].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    else:
        k = torch.from_numpy(raw[:T * D].copy()).view(torch.float8_e4m3fn).float().numpy()
        k = k.astype(np.float64)
    return k.reshape(T, D), float(sc[0])


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.BF16, O.FP8])
def test_summary_is_min_and_max_of_the_block(dtype):
    g = _geom(dtype)
    for h in (0, 5, 77, 4098):
        k, _ = _decode_block(g, h)
        kmin, kmax = O.summary(g, h)
        assert np.array_equal(kmin.astype(np.float64), k.min(axis=0))
        assert np.array_equal(kmax.astype(np.float64), k.max(axis=0))


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.BF16, O.FP8])
def test_quest_bound_against_float64_and_true_scores(dtype):
    """Per (request, layer, kv head): score = max over the group's heads of
    sum_d max(q_d kmax_d, q_d kmin_d) (x the K scale for fp8).  It equals the
    float64 formula to fp32 rounding and bounds every token's q.k."""
    g = _geom(dtype, n_req=2, L=1, H=2, Hq=4)
    rng = np.random.default_rng(dtype)
    q = rng.standard_normal((2, 1, 4, 128)).astype(np.float32)
    ctx = np.array([40, 17], np.int32)
    sc = O.quest_scores(g, q, ctx, mode=0)
    G = 2
    for r in range(2):
        for h in range(2):
            row = r * 2 + h
            for b in range(ctx[r]):
                hb = O.host_index(g, (r * 1 + 0) * 2 + h, b)
                k, ks = _decode_block(g, hb)
                kmin, kmax = k.min(axis=0), k.max(axis=0)
                ks = ks if dtype == O.FP8 else 1.0
                want, true = -np.inf, -np.inf
                for gq in range(G):
                    qv = q[r, 0, h * G + gq].astype(np.float64)
                    want = max(want, np.maximum(qv * kmax, qv * kmin).sum() * ks)
                    true = max(true, (k @ qv).max() * ks)
                got = float(sc[row, b])
                assert abs(got - want) <= 1e-5 * (abs(want) + 1.0)
                assert got >= true - 1e-5 * (abs(true) + 1.0)


def _numpy_topk(scores, n, k):
    """Top min(k, n) of scores[:n] by (order-preserving key desc, id asc), sorted by id."""
    s = scores[:n].astype(np.float32)
    u = s.view(np.uint32)
    key = np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint64)
    order = np.lexsort((np.arange(n), -key.astype(np.int64)))
    return np.sort(order[:min(k, n)])


@pytest.mark.parametrize("dtype,host_blocks", [(O.F16, 4099), (O.BF16, 5), (O.FP8, 4099),
                                               (O.F32, 3)])
@pytest.mark.parametrize("mode", [0, 1])
def test_topk_matches_numpy(dtype, host_blocks, mode):
    """Selections against numpy: the k best scores (ties to the lower id, ties
    forced by a host tier of 3-5 blocks that many blocks alias), in ascending
    order, NONE-padded for contexts shorter than k, empty for no context."""
    g = _geom(dtype, n_req=4, L=2, H=2, Hq=4, k=8, mb=64, host_blocks=host_blocks)
    rng = np.random.default_rng(host_blocks + mode)
    q = rng.standard_normal((4, 2, 4, 128)).astype(np.float32)
    ctx = np.array([64, 5, 0, 30], np.int32)
    sel = O.select_topk(g, q, ctx, mode)
    sc = O.quest_scores(g, q, ctx, mode)
    rows_per_rl = 1 if mode else 2
    for r in range(4):
        for l in range(2):
            for h in range(2):
                row = (r * 2 + l) * rows_per_rl + (0 if mode else h)
                want = _numpy_topk(sc[row], ctx[r], 8)
                got = sel[r, l, h]
                assert np.array_equal(got[:len(want)], want)
                assert np.all(got[len(want):] == O.NONE)
    if mode:
        assert np.array_equal(sel[:, :, 0], sel[:, :, 1])
    if host_blocks < 10:  # aliasing produced ties that the id rule had to break
        assert len(np.unique(sc[0, :64])) < 64


def test_layer_mode_with_one_kv_head_equals_per_head():
    g = _geom(O.F16, n_req=2, L=2, H=1, Hq=4)
    q = np.random.default_rng(3).standard_normal((2, 2, 4, 128)).astype(np.float32)
    ctx = np.array([50, 12], np.int32)
    assert np.array_equal(O.select_topk(g, q, ctx, 0), O.select_topk(g, q, ctx, 1))


def test_zero_query_selects_the_first_blocks():
    """q = 0 scores every block 0: all keys tie, so the k lowest ids win."""
    g = _geom(O.BF16, n_req=1, L=1, H=2, Hq=2)
    sel = O.select_topk(g, np.zeros((1, 1, 2, 128), np.float32), np.array([40], np.int32), 0)
    assert np.array_equal(sel[0, 0], np.tile(np.arange(8, dtype=np.uint32), (2, 1)))


# ---------------------------------------------------------------- mass method
def _mass_numpy(g, q, ctx):
    """The capture tool's mass scores (tools/capture_miss_trace.py:147-155) with
    torch.softmax in float64 over K decoded here: [B, L, n]."""
    B, L, Hk, Hq = g.n_req, g.n_layers, g.kv_heads, g.q_heads
    G, T = Hq // Hk, g.block_tokens
    out = np.full((B, L, int(ctx.max())), np.nan)
    for r in range(B):
        n = int(ctx[r])
        for l in range(L):
            score = np.zeros(n)
            for h in range(Hk):
                set_ = (r * L + l) * Hk + h
                K = np.concatenate([(lambda kt: kt[0] * kt[1])(_decode_block(g, O.host_index(g, set_, b)))
                                    for b in range(n)])  # [n*T, D]
                qg = q[r, l, h * G:(h + 1) * G].astype(np.float64)  # [G, D]
                logits = torch.from_numpy(qg @ K.T / np.sqrt(g.head_dim))
                attn = torch.softmax(logits, dim=-1).numpy()
                score += attn.reshape(G, n, T).sum(-1).sum(0)
            out[r, l, :n] = score
    return out


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.BF16, O.FP8])
def test_mass_scores_against_torch_softmax(dtype):
    g = _geom(dtype, n_req=2, L=2, H=2, Hq=4, mb=48, host_blocks=97)
    rng = np.random.default_rng(10 + dtype)
    q = (rng.standard_normal((2, 2, 4, 128)) * 2).astype(np.float32)
    ctx = np.array([30, 11], np.int32)
    got = O.mass_scores(g, q, ctx)
    want = _mass_numpy(g, q, ctx)
    assert np.allclose(np.nan_to_num(got), np.nan_to_num(want), rtol=1e-12, atol=1e-15)
    # every query head's softmax sums to 1: a layer holds Hq of mass
    assert np.allclose(np.nansum(got, axis=2), 4.0, rtol=0, atol=1e-12)


def test_mass_selection_special_cases():
    g = _geom(O.F16, n_req=2, L=1, H=2, Hq=4, k=6, mb=48, host_blocks=97)
    ctx = np.array([20, 4], np.int32)
    # q = 0: every token weighs the same, every block ties: the lowest ids
    sel = O.select_mass(g, np.zeros((2, 1, 4, 128), np.float32), ctx)
    assert np.array_equal(sel[0, 0, 0], np.arange(6, dtype=np.uint32))
    # a context of at most k blocks: all of them, then EMPTY, in every kv head's row
    assert np.array_equal(sel[1, 0, 1], np.array([0, 1, 2, 3, O.NONE, O.NONE], np.uint32))
    # q along one token's key, large: that token's block takes nearly all the mass
    k13, ks = _decode_block(g, O.host_index(g, 0, 13))
    q = np.zeros((2, 1, 4, 128), np.float32)
    q[0, 0, :2] = (k13[5] * ks * 50.0).astype(np.float32)  # both heads of kv head 0
    s = O.mass_scores(g, q, ctx)
    # kv head 0's two heads put (almost) all their mass on block 13; kv head 1's
    # (q = 0) spread theirs evenly, 2/20 per block
    assert int(np.nanargmax(s[0, 0])) == 13 and abs(s[0, 0, 13] - 2.1) < 1e-6
    assert np.allclose(np.delete(s[0, 0], 13), 0.1, atol=1e-6)
    assert 13 in O.select_mass(g, q, ctx)[0, 0, 0]


def test_mass_selection_is_lexsort_of_scores():
    g = _geom(O.BF16, n_req=3, L=2, H=2, Hq=8, k=7, mb=64, host_blocks=131)
    rng = np.random.default_rng(3)
    q = rng.standard_normal((3, 2, 8, 128)).astype(np.float32)
    ctx = np.array([64, 7, 33], np.int32)
    sc = O.mass_scores(g, q, ctx)
    sel = O.select_mass(g, q, ctx)
    for r in range(3):
        for l in range(2):
            n = int(ctx[r])
            order = np.lexsort((np.arange(n), -sc[r, l, :n]))[:min(7, n)]
            want = np.full(7, O.NONE, np.uint32)
            want[:len(order)] = np.sort(order)
            for h in range(2):
                assert np.array_equal(sel[r, l, h], want)
