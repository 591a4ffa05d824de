"""GPU parity of the on-device top-k block selection (Quest bound): block
summaries and selections bit-exact against the oracle, and the selection
feeding the executor (bookkeeping, fetch, attention) end to end."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import TOL, Pair

pytestmark = pytest.mark.gpu


def _decode_summary_bytes(dtype, raw):
    """[n, 2*128*esize] bytes -> float32 [n, 2, 128] (exact)."""
    n = raw.shape[0]
    if dtype == F.F32:
        return raw.view(np.float32).reshape(n, 2, 128)
    if dtype == F.F16:
        return raw.view(np.float16).astype(np.float32).reshape(n, 2, 128)
    if dtype == F.BF16:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(n, 2, 128)
    codes = raw.reshape(-1)
    f = np.array([O.lib.ora_e4m3_to_f32(int(c)) for c in range(256)], np.float32)[codes]
    return f.reshape(n, 2, 128)


@pytest.mark.parametrize("dtype", [F.F32, F.F16, F.BF16, F.FP8])
def test_summaries_bit_exact(dtype):
    p = Pair(2, 1, 2, 2, 8, 8, 64, dtype, host_blocks=1031)
    p.ex.summaries_build()
    torch.cuda.synchronize()
    raw, scales = p.ex.summaries_array()
    got = _decode_summary_bytes(dtype, raw)
    for h in range(1031):
        kmin, kmax = O.summary(p.g, h)
        assert np.array_equal(got[h, 0].view(np.uint32), kmin.view(np.uint32)), h
        assert np.array_equal(got[h, 1].view(np.uint32), kmax.view(np.uint32)), h
    if dtype == F.FP8:
        assert np.array_equal(scales, p.hsc.reshape(-1, 2)[:, 0])


@pytest.mark.parametrize("dtype,Hkv,Hq,host_blocks", [
    (F.F16, 4, 4, 4099),     # MHA
    (F.BF16, 2, 8, 4099),    # GQA-4
    (F.FP8, 2, 8, 4099),     # fp8 + K scales
    (F.F32, 2, 4, 7),        # a tiny host tier: aliased blocks tie
    (F.BF16, 1, 8, 4099),    # GQA-8
])
@pytest.mark.parametrize("mode", [F.TOPK_PER_HEAD, F.TOPK_LAYER_MAX])
def test_select_topk_bit_exact(dtype, Hkv, Hq, host_blocks, mode):
    n_req, L, k, mb = 6, 2, 16, 300
    p = Pair(n_req, L, Hkv, Hq, k, 64, mb, dtype, host_blocks=host_blocks)
    p.ex.summaries_build()
    rng = np.random.default_rng(dtype * 7 + Hq + mode)
    ctx = np.array([300, 9, 0, 16, 17, 211], np.int32)  # full, ragged, empty, == k, k + 1
    for t in range(2):
        q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
        sel = torch.empty((n_req, L, Hkv, k), dtype=torch.int32, device="cuda")
        p.ex.select_topk(torch.from_numpy(q).cuda(), torch.from_numpy(ctx).cuda(), sel, mode)
        torch.cuda.synchronize()
        got = sel.cpu().numpy().view(np.uint32)
        want = O.select_topk(p.g, q, ctx, mode)
        assert np.array_equal(got, want)
    assert p.ex.stats()["device_error"] == 0


def test_one_record_per_block_gives_the_same_selection():
    """A table with a record per (set, block) (3x the host tier here) repeats
    the host-tier records and selects exactly what the small table does."""
    n_req, L, Hkv, Hq, k, mb, hb = 4, 2, 2, 8, 16, 384, 1031
    p = Pair(n_req, L, Hkv, Hq, k, 64, mb, F.FP8, host_blocks=hb)
    q = torch.randn((n_req, L, Hq, 128), device="cuda")
    ctx = torch.tensor([384, 100, 17, 250], dtype=torch.int32, device="cuda")
    a = torch.empty((n_req, L, Hkv, k), dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    p.ex.summaries_build()
    p.ex.select_topk(q, ctx, a)
    torch.cuda.synchronize()
    small, small_sc = p.ex.summaries_array()
    p.ex.summaries_build(3 * hb)
    p.ex.select_topk(q, ctx, b)
    torch.cuda.synchronize()
    big, big_sc = p.ex.summaries_array()
    assert big.shape[0] == 3 * hb
    assert np.array_equal(big, np.tile(small, (3, 1)))
    assert np.array_equal(big_sc, np.tile(small_sc, 3))
    assert torch.equal(a, b)
    with pytest.raises(F.FerryError, match="multiple"):
        p.ex.summaries_build(hb + 1)


def test_select_layers_equals_whole_step():
    n_req, L, Hkv, Hq, k = 3, 4, 2, 4, 12
    p = Pair(n_req, L, Hkv, Hq, k, 48, 200, F.F16)
    p.ex.summaries_build()
    q = torch.randn((n_req, L, Hq, 128), device="cuda")
    ctx = torch.tensor([200, 50, 7], dtype=torch.int32, device="cuda")
    a = torch.empty((n_req, L, Hkv, k), dtype=torch.int32, device="cuda")
    b = torch.full_like(a, -1)
    p.ex.select_topk(q, ctx, a)
    p.ex.select_topk(q, ctx, b, layers=(0, 3))
    p.ex.select_topk(q, ctx, b, layers=(3, 1))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_selection_feeds_the_executor():
    """q -> top-k selection -> bookkeeping/fetch -> attention, over several
    decode steps, against the oracle at every stage."""
    n_req, L, Hkv, Hq, k, cap, mb = 4, 2, 2, 8, 24, 96, 400
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, F.BF16)
    p.ex.summaries_build()
    rng = np.random.default_rng(11)
    ctx = np.array([400, 120, 20, 333], np.int32)
    dctx = torch.from_numpy(ctx).cuda()
    base = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    for t in range(4):
        # slowly drifting queries, so consecutive selections overlap
        q = (base + 0.3 * rng.standard_normal(base.shape)).astype(np.float32)
        dq = torch.from_numpy(q).cuda()
        sel = torch.empty((n_req, L, Hkv, k), dtype=torch.int32, device="cuda")
        p.ex.select_topk(dq, dctx, sel)
        torch.cuda.synchronize()
        s = sel.cpu().numpy().view(np.uint32).reshape(-1)
        assert np.array_equal(s, O.select_topk(p.g, q, ctx, 0).reshape(-1))
        p.check_fetched_bytes(p.step(s))
        p.check_state()
        out = torch.empty_like(dq)
        p.ex.sparse_decode(dq, p.bufs["slots"], out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
        ref = O.attention_f64(p.g, s, q).reshape(-1, 128)
        rel = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
        assert rel.max() < TOL[F.BF16], rel.max()


def test_selection_errors():
    p = Pair(2, 1, 2, 2, 8, 16, 64, F.F16)
    q = torch.zeros((2, 1, 2, 128), device="cuda")
    sel = torch.empty((2, 1, 2, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(F.FerryError, match="summaries not built"):
        p.ex.select_topk(q, torch.tensor([10, 10], dtype=torch.int32, device="cuda"), sel)
    p.ex.summaries_build()
    p.ex.select_topk(q, torch.tensor([65, 10], dtype=torch.int32, device="cuda"), sel)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -3  # FERRY_ERANGE: context longer than max_blocks
    assert np.all(sel.cpu().numpy()[0] == -1)  # that row is left empty


def _const_k_tile(dtype, c):
    """Bytes of a 16 x 128 K tile whose every element is c (exact in dtype)."""
    v = np.full((16, 128), c, np.float32)
    if dtype == F.F16:
        return v.astype(np.float16).view(np.uint8).ravel()
    if dtype == F.BF16:
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).ravel()
    return v.view(np.uint8).ravel()


@pytest.mark.parametrize("mode", [F.TOPK_PER_HEAD, F.TOPK_LAYER_MAX])
@pytest.mark.parametrize("k", [8, 9, 63])
@pytest.mark.parametrize("dtype", [F.F16, F.BF16, F.F32])
def test_select_topk_known_answer(dtype, k, mode):
    """Crafted blocks with a known selection: every K element of block b is
    c_b and q is all ones, so block b's bound is 128 c_b exactly.  Eight blocks
    of each row carry c = 4^j (j = 0..7), the other 56 carry 0.  With k = 8
    the k-th key is alone in its top-byte bin, so the radix search ends at its
    first pass; with k = 9 and 63 the k-th key is one of the 56 equal zeros
    and the ties go to the lower block ids."""
    mb, hb = 64, 128
    big = {0: [3, 10, 17, 24, 31, 38, 45, 52], 1: [60, 50, 40, 30, 20, 10, 5, 0]}
    ex = F.Executor(2, 1, 1, k, 16, mb, q_heads=1, dtype=dtype, host_blocks=hb)
    ex.hosttier_fill()
    torch.cuda.synchronize()  # the fill has landed before the K tiles are rewritten
    host, _ = ex.hosttier_array()
    bb = ex.block_bytes
    kt = 16 * 128 * {F.F16: 2, F.BF16: 2, F.F32: 4}[dtype]
    for r in (0, 1):
        for b in range(mb):
            c = 4.0 ** big[r].index(b) if b in big[r] else 0.0
            h = r * mb + b  # block (set r, b) reads host block r * max_blocks + b
            host[h * bb:h * bb + kt] = _const_k_tile(dtype, c)
    ex.summaries_build()
    q = torch.ones((2, 1, 1, 128), device="cuda")
    sel = torch.empty((2, 1, 1, k), dtype=torch.int32, device="cuda")
    ex.select_topk(q, torch.tensor([mb, mb], dtype=torch.int32, device="cuda"), sel, mode=mode)
    torch.cuda.synchronize()
    got = sel.cpu().numpy().reshape(2, k)
    for r in (0, 1):
        zeros = [b for b in range(mb) if b not in big[r]]
        want = sorted(big[r] + zeros[:k - 8])
        assert got[r].tolist() == want, (r, got[r].tolist(), want)
    assert ex.stats()["device_error"] == 0


@pytest.mark.parametrize("dtype,Hkv,Hq", [(F.F16, 2, 4), (F.BF16, 1, 8), (F.FP8, 2, 8), (F.F32, 2, 2)])
def test_summary_read_probe(dtype, Hkv, Hq):
    # FERRY_PROBE_SUMS_READ reads the min/max record of n blocks of every set
    # from the summary table in the Quest selection's pattern: its bytes, and
    # its refusals
    p = Pair(3, 2, Hkv, Hq, 8, 16, 96, dtype, host_blocks=257)
    rec = 2 * 128 * {F.F32: 4, F.F16: 2, F.BF16: 2, F.FP8: 1}[dtype]
    with pytest.raises(F.FerryError, match="summaries_build"):
        p.ex.bw_probe(F.PROBE_SUMS_READ, 10)
    p.ex.summaries_build()
    b, ms, gbs = p.ex.bw_probe(F.PROBE_SUMS_READ, 96, iters=2)
    assert b == 3 * 2 * Hkv * 96 * rec and ms > 0 and gbs > 0
    b, _, _ = p.ex.bw_probe(F.PROBE_SUMS_READ, 37, iters=1)
    assert b == 3 * 2 * Hkv * 37 * rec
    with pytest.raises(F.FerryError, match="max_blocks"):
        p.ex.bw_probe(F.PROBE_SUMS_READ, 97)
    assert p.ex.stats()["device_error"] == 0


def _topk_geometry(seed):
    rng = np.random.default_rng(3000 + seed)
    dtype = int(rng.choice([F.F32, F.F16, F.BF16, F.FP8]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    mode = int(rng.choice([F.TOPK_PER_HEAD, F.TOPK_LAYER_MAX]))
    n_req = int(rng.integers(1, 5))
    L = int(rng.integers(1, 4))
    k = int(rng.integers(1, 49))
    mb = int(rng.integers(k + 1, 900))
    hb = int(rng.choice([7, 1031, 4099]))  # 7: records repeat, identical blocks tie exactly
    ctx = rng.integers(0, mb + 1, n_req).astype(np.int32)
    ctx[0] = mb
    return dict(dtype=dtype, Hkv=Hkv, G=G, mode=mode, n_req=n_req, L=L, k=k, mb=mb, hb=hb), ctx


@pytest.mark.parametrize("seed", range(16))
def test_random_geometry_topk_bit_exact(seed):
    c, ctx = _topk_geometry(seed)
    print("[topk geometry]", c, ctx.tolist(), flush=True)
    Hq = c["Hkv"] * c["G"]
    p = Pair(c["n_req"], c["L"], c["Hkv"], Hq, c["k"], c["k"], c["mb"], c["dtype"],
             host_blocks=c["hb"])
    p.ex.summaries_build()
    q = np.random.default_rng(seed).standard_normal((c["n_req"], c["L"], Hq, 128)).astype(np.float32)
    sel = torch.full((c["n_req"], c["L"], c["Hkv"], c["k"]), -7, dtype=torch.int32, device="cuda")
    p.ex.select_topk(torch.from_numpy(q).cuda(), torch.from_numpy(ctx).cuda(), sel, c["mode"])
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy().view(np.uint32), O.select_topk(p.g, q, ctx, c["mode"]))
    assert p.ex.stats()["device_error"] == 0
