"""GPU parity of the softmax-mass block selection (the capture tool's "mass"
method): the dense K table bit-exact against the host tier, and each
(request, layer)'s page list against the oracle's float64 scores.

The device scores in float32 (logits on the matrix cores from a 2-3 term
split of the query for 16-bit and fp8 K, on the vector ALUs for fp32 K; each
block's softmax maximum and sum merged over wavefronts in the exp2 domain), so
near-ties may order differently from the float64 oracle.  The bar: every row holds min(k, ctx) distinct ascending ids in
range, the same list in every kv head's row, EMPTY after; a block that the
device takes and the oracle does not (or the reverse) scores within
TOL_MASS x (the row's largest score) of the oracle's k-th score; and at least
90% of the rows match the oracle exactly.  Contexts at or below k, and q = 0
(all blocks tie), have one right answer and are compared exactly."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import Pair

pytestmark = pytest.mark.gpu

TOL_MASS = 2e-4


def _run(p, q, ctx, layers=None):
    B, L, Hkv, k = p.g.n_req, p.g.n_layers, p.g.kv_heads, p.g.k
    sel = torch.full((B, L, Hkv, k), -7, dtype=torch.int32, device="cuda")
    p.ex.select_mass(torch.from_numpy(q).cuda(), torch.from_numpy(ctx).cuda(), sel,
                     layers=layers)
    torch.cuda.synchronize()
    return sel.cpu().numpy().view(np.uint32)


def _check_rows(p, got, q, ctx, rows=None):
    """Compare got [B,L,Hkv,k] with the oracle under the near-tie bar; returns
    the fraction of rows that match exactly."""
    g = p.g
    sc = O.mass_scores(g, q, ctx)
    exact = total = 0
    for r in range(g.n_req):
        for l in range(g.n_layers) if rows is None else rows:
            n = max(int(ctx[r]), 0)
            kk = min(n, g.k)
            row = got[r, l]
            assert np.all(row == row[0]), (r, l)  # one list per layer
            row = row[0]
            assert np.all(row[kk:] == O.NONE), (r, l)
            ids = row[:kk].astype(np.int64)
            assert np.all(ids < n) and np.all(np.diff(ids) > 0), (r, l)
            total += 1
            if n <= g.k:
                assert np.array_equal(ids, np.arange(n)), (r, l)
                exact += 1
                continue
            s = sc[r, l, :n]
            # the oracle's list: highest scores, ties to the lower id, ascending
            # (the same as O.select_mass, which the CPU tests pin to this rule)
            o = np.sort(np.lexsort((np.arange(n), -s))[:kk])
            if np.array_equal(ids, o):
                exact += 1
                continue
            thr = np.sort(s)[::-1][kk - 1]
            tol = TOL_MASS * s.max()
            extra, missed = np.setdiff1d(ids, o), np.setdiff1d(o, ids)
            assert np.all(s[extra] >= thr - tol), (r, l, s[extra], thr)
            assert np.all(s[missed] <= thr + tol), (r, l, s[missed], thr)
    return exact / max(total, 1)


def _table_layout(dtype, hk):
    """Host-tier K halves [n, bytes] in the table's record layout: fp32
    row-major; 16-bit and fp8 lane-transposed, 16-byte word c of token row t
    at word 64 (c // 4) + 16 (c % 4) + t."""
    if dtype == F.F32:
        return hk
    n = hk.shape[0]
    words = hk.reshape(n, 16, -1, 16)  # [record][row][word][16 bytes]
    out = np.empty((n, words.shape[1] * words.shape[2], 16), np.uint8)
    for t in range(16):
        for c in range(words.shape[2]):
            out[:, 64 * (c // 4) + 16 * (c % 4) + t] = words[:, t, c]
    return out.reshape(n, -1)


@pytest.mark.parametrize("dtype", [F.F32, F.F16, F.BF16, F.FP8])
def test_ktiles_bit_exact(dtype):
    hb = 1031
    p = Pair(2, 1, 2, 2, 8, 8, 64, dtype, host_blocks=hb)
    p.ex.ktiles_build(3 * hb)  # three copies of the host tier's records
    torch.cuda.synchronize()
    kt, scales = p.ex.ktiles_array()
    half = p.bb // 2
    assert kt.shape == (3 * hb, half)
    hk = _table_layout(dtype, p.host.reshape(hb, p.bb)[:, :half])
    for c in range(3):
        assert np.array_equal(kt[c * hb:(c + 1) * hb], hk)
    if dtype == F.FP8:
        assert np.array_equal(scales, np.tile(p.hsc.reshape(hb, 2)[:, 0], 3))
    else:
        assert scales is None


@pytest.mark.parametrize("dtype,Hkv,Hq", [
    (F.F16, 2, 2),    # MHA
    (F.BF16, 2, 8),   # GQA-4
    (F.FP8, 2, 8),    # fp8 + K scales
    (F.F32, 1, 2),    # GQA-2, f32
    (F.BF16, 1, 8),   # GQA-8
])
def test_select_mass_parity(dtype, Hkv, Hq):
    n_req, L, k, mb = 6, 2, 16, 300
    p = Pair(n_req, L, Hkv, Hq, k, 64, mb, dtype, host_blocks=4099)
    p.ex.ktiles_build()
    rng = np.random.default_rng(dtype * 7 + Hq)
    ctx = np.array([300, 9, 0, 16, 17, 211], np.int32)  # full, ragged, empty, == k, k + 1
    fracs = []
    for t in range(2):
        q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
        got = _run(p, q, ctx)
        fracs.append(_check_rows(p, got, q, ctx))
    print("[mass] exact rows", fracs, flush=True)
    assert min(fracs) >= 0.9
    assert p.ex.stats()["device_error"] == 0


@pytest.mark.parametrize("dtype,Hkv,Hq", [(F.F16, 2, 2), (F.BF16, 2, 8)])
def test_select_mass_hbm_workspace_parity(dtype, Hkv, Hq, monkeypatch):
    # 16-bit K keeps each block's log-sum in LDS; FERRY_MASS_WS=hbm (read when the
    # K table is built) keeps the (max, sum) pairs in the context's HBM workspace
    monkeypatch.setenv("FERRY_MASS_WS", "hbm")
    n_req, L, k, mb = 6, 2, 16, 300
    print(f"[mass] HBM workspace dtype={dtype} Hkv={Hkv} Hq={Hq}", flush=True)
    p = Pair(n_req, L, Hkv, Hq, k, 64, mb, dtype, host_blocks=4099)
    p.ex.ktiles_build()
    rng = np.random.default_rng(dtype * 11 + Hq)
    ctx = np.array([300, 9, 0, 16, 17, 211], np.int32)
    q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    frac = _check_rows(p, _run(p, q, ctx), q, ctx)
    print("[mass] exact rows", frac, flush=True)
    assert frac >= 0.9
    assert p.ex.stats()["device_error"] == 0


@pytest.mark.parametrize("dtype", [F.F16, F.FP8])
def test_zero_query_takes_the_lowest_ids(dtype):
    """q = 0: every token gets probability 1/(16 ctx), every block the same
    score, and the ties go to the lower ids."""
    n_req, L, Hkv, Hq, k = 3, 2, 2, 4, 24
    p = Pair(n_req, L, Hkv, Hq, k, 64, 500, dtype, host_blocks=1031)
    p.ex.ktiles_build()
    ctx = np.array([500, 25, 7], np.int32)
    got = _run(p, np.zeros((n_req, L, Hq, 128), np.float32), ctx)
    want = O.select_mass(p.g, np.zeros((n_req, L, Hq, 128), np.float32), ctx)
    assert np.array_equal(got, want)
    assert np.array_equal(got[0, 0, 0], np.arange(k, dtype=np.uint32))


def test_layer_ranges_write_only_their_layers():
    n_req, L, Hkv, Hq, k = 2, 4, 1, 4, 8
    p = Pair(n_req, L, Hkv, Hq, k, 32, 120, F.BF16, host_blocks=1031)
    p.ex.ktiles_build()
    rng = np.random.default_rng(5)
    q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    ctx = np.array([120, 40], np.int32)
    got = _run(p, q, ctx, layers=(1, 2))
    assert np.all(got[:, [0, 3]].view(np.int32) == -7)
    _check_rows(p, got, q, ctx, rows=[1, 2])


def test_more_records_give_the_same_selection():
    n_req, L, Hkv, Hq, k, mb, hb = 3, 2, 2, 8, 16, 384, 1031
    p = Pair(n_req, L, Hkv, Hq, k, 64, mb, F.FP8, host_blocks=hb)
    rng = np.random.default_rng(9)
    q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    ctx = np.array([384, 100, 250], np.int32)
    p.ex.ktiles_build()
    a = _run(p, q, ctx)
    p.ex.ktiles_build(2 * hb)
    b = _run(p, q, ctx)
    assert np.array_equal(a, b)


def test_largest_context():
    """max_blocks 15360 (one float score per block in 60 KiB of LDS), k 1024,
    GQA-8; one past it is refused."""
    mb = 15360
    p = Pair(2, 1, 1, 8, 1024, 16, mb, F.F16, host_blocks=4099)
    p.ex.ktiles_build()
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 1, 8, 128)).astype(np.float32)
    ctx = np.array([mb, 1500], np.int32)
    got = _run(p, q, ctx)
    _check_rows(p, got, q, ctx)  # 1024-of-15360 lists: near-ties are likely, the bar holds
    assert p.ex.stats()["device_error"] == 0
    big = Pair(1, 1, 1, 8, 8, 16, mb + 1, F.F16, host_blocks=1031)
    big.ex.ktiles_build()
    with pytest.raises(F.FerryError, match="60 KiB"):
        big.ex.select_mass(torch.zeros((1, 1, 8, 128), device="cuda"),
                           torch.tensor([8], dtype=torch.int32, device="cuda"),
                           torch.empty((1, 1, 1, 8), dtype=torch.int32, device="cuda"))


def test_refusals():
    p = Pair(2, 1, 1, 2, 8, 16, 64, F.F16, host_blocks=257)
    q = torch.zeros((2, 1, 2, 128), device="cuda")
    ctx = torch.tensor([64, 9], dtype=torch.int32, device="cuda")
    sel = torch.empty((2, 1, 1, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(F.FerryError, match="not built"):
        p.ex.select_mass(q, ctx, sel)
    with pytest.raises(F.FerryError, match="multiple"):
        p.ex.ktiles_build(300)
    with pytest.raises(F.FerryError, match="layer range"):
        p.ex.ktiles_build()
        p.ex.select_mass(q, ctx, sel, layers=(0, 2))
    gp = F.Executor(2, 1, 1, 8, 16, 64, q_heads=2, group=2, host_blocks=257)
    gp.ktiles_build()
    with pytest.raises(F.FerryError, match="group 1"):
        gp.select_mass(q, ctx, sel)
    # a context past max_blocks latches FERRY_ERANGE and leaves the row EMPTY
    p.ex.select_mass(q, torch.tensor([65, 9], dtype=torch.int32, device="cuda"), sel)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -3
    assert np.all(sel[0].cpu().numpy().view(np.uint32) == O.NONE)


@pytest.mark.parametrize("dtype", [F.F16, F.FP8, F.F32])
def test_ktable_read_probe(dtype):
    # FERRY_PROBE_KTAB_READ reads the K half of n blocks of every set from the
    # table in the mass selection's order: its bytes, and its refusals
    p = Pair(3, 2, 2, 4, 8, 16, 96, dtype, host_blocks=257)
    with pytest.raises(F.FerryError, match="ktiles_build"):
        p.ex.bw_probe(F.PROBE_KTAB_READ, 10)
    p.ex.ktiles_build()
    b, ms, gbs = p.ex.bw_probe(F.PROBE_KTAB_READ, 96, iters=2)
    assert b == 3 * 2 * 2 * 96 * (p.bb // 2) and ms > 0 and gbs > 0
    b, _, _ = p.ex.bw_probe(F.PROBE_KTAB_READ, 37, iters=1)
    assert b == 3 * 2 * 2 * 37 * (p.bb // 2)
    with pytest.raises(F.FerryError, match="max_blocks"):
        p.ex.bw_probe(F.PROBE_KTAB_READ, 97)
    assert p.ex.stats()["device_error"] == 0


def test_mass_selection_feeds_the_executor():
    """q -> mass selection -> bookkeeping/fetch -> attention over four decode
    steps: the selection under the near-tie bar, everything downstream of it
    (slots, misses, state, fetched bytes, attention) against the oracle fed
    with the device's selection."""
    n_req, L, Hkv, Hq, k, cap, mb = 4, 2, 2, 8, 24, 96, 400
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, F.BF16)
    p.ex.ktiles_build()
    rng = np.random.default_rng(12)
    ctx = np.array([400, 120, 20, 333], np.int32)
    dctx = torch.from_numpy(ctx).cuda()
    base = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    for t in range(4):
        q = (base + 0.3 * rng.standard_normal(base.shape)).astype(np.float32)
        got = _run(p, q, ctx)
        _check_rows(p, got, q, ctx)
        p.check_fetched_bytes(p.step(got.reshape(-1)))
        p.check_state()
    p.check_attention(got.reshape(-1), seed=3)


def _mass_geometry(seed):
    rng = np.random.default_rng(2000 + seed)
    dtype = int(rng.choice([F.F32, F.F16, F.BF16, F.FP8]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    n_req = int(rng.integers(1, 5))
    L = int(rng.integers(1, 4))
    k = int(rng.integers(1, 49))
    mb = int(rng.integers(k + 1, 700))
    hb = int(rng.choice([7, 1031, 4099]))  # 7: records repeat, identical blocks tie exactly
    ctx = rng.integers(0, mb + 1, n_req).astype(np.int32)
    ctx[0] = mb
    return dict(dtype=dtype, Hkv=Hkv, G=G, n_req=n_req, L=L, k=k, mb=mb, hb=hb), ctx


@pytest.mark.parametrize("seed", range(16))
def test_random_geometry_mass(seed):
    c, ctx = _mass_geometry(seed)
    print("[mass geometry]", c, ctx.tolist(), flush=True)
    p = Pair(c["n_req"], c["L"], c["Hkv"], c["Hkv"] * c["G"], c["k"], c["k"], c["mb"],
             c["dtype"], host_blocks=c["hb"])
    p.ex.ktiles_build()
    q = np.random.default_rng(seed).standard_normal(
        (c["n_req"], c["L"], c["Hkv"] * c["G"], 128)).astype(np.float32)
    _check_rows(p, _run(p, q, ctx), q, ctx)
    assert p.ex.stats()["device_error"] == 0
