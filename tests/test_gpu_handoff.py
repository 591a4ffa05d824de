"""GPU parity of the owner hand-off (export / import of one request's
resident KV and LRU state): the importer's sets equal the exporter's bit for
bit, and the moved request then runs in its new lane exactly as the oracle
runs it after the same state copy (kv_handoff with carry,
src/runtime/wla_multigpu.cuh:1970-1994)."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import Pair, _zipf_stream

pytestmark = pytest.mark.gpu


def _owner_rows(arr, owner, L, H):
    """Rows of one owner's sets (group 1: owner = request)."""
    return arr.reshape(-1, L * H, *arr.shape[1:])[owner]


def _move_and_check(dtype, Hkv, Hq, n_req=4, L=3, k=16, cap=40, lo=60, hi=300, seed=4,
                    src=1, dst=2, host_blocks=4099):
    """Four steps in X, two unrelated steps in Y, owner src of X exported into
    lane dst of Y: state, resident bytes, attention and four further steps of
    the moved request compared between the two executors and the oracle."""
    mb, sels = _zipf_stream(n_req, L, Hkv, k, lo, hi, 9, seed=seed)
    X = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, host_blocks=host_blocks)
    Y = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, host_blocks=host_blocks)
    for t in range(4):
        X.step(sels[t])
    for t in range(2):  # Y's lane 2 holds someone else's blocks before the move
        Y.step(sels[8 - t])
    img = X.ex.alloc_owner_image()
    X.ex.owner_export(src, img)
    Y.ex.owner_import(dst, img)
    Y.ox.copy_owner_from(X.ox, src, dst)
    torch.cuda.synchronize()
    assert X.ex.stats()["device_error"] == 0 and Y.ex.stats()["device_error"] == 0
    xf, xo, xt = X.ex.sets_state()
    yf, yo, yt = Y.ex.sets_state()
    S = L * Hkv
    assert np.array_equal(_owner_rows(yf, dst, L, Hkv), _owner_rows(xf, src, L, Hkv))
    assert np.array_equal(_owner_rows(yt, dst, L, Hkv), _owner_rows(xt, src, L, Hkv))
    for s in range(S):
        f = xf[src * S + s]
        assert np.array_equal(yo[dst * S + s, :f], xo[src * S + s, :f])
    Y.check_state()
    # the image header counts the resident blocks
    head = img[:16].cpu().numpy().view(np.uint32)
    assert head[0] == 0x4E574F46 and head[1] == S and head[2] == cap
    assert int(img[24:32].cpu().numpy().view(np.uint64)[0]) == int(xf[src * S:(src + 1) * S].sum())
    # the resident bytes (and fp8 scales) moved with the state
    xs = np.concatenate([src * S * cap + s * cap + np.arange(xf[src * S + s]) for s in range(S)])
    ys = xs + (dst - src) * S * cap
    assert np.array_equal(Y.ex.pool_slots_bytes(ys), X.ex.pool_slots_bytes(xs))
    if dtype == F.FP8:
        assert np.array_equal(Y.ex.pool_slot_scales(ys), X.ex.pool_slot_scales(xs))
    # attention over the moved slots is bit-identical to the exporter's
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)).cuda()
    qy = q.clone()
    qy[dst] = q[src]
    slots_y = Y.bufs["slots"].clone().view(n_req, -1)
    xsl = X.bufs["slots"].view(n_req, -1)[src]
    # slot ids are global (set * C + slot); EMPTY positions stay EMPTY
    slots_y[dst] = torch.where(xsl == -1, xsl, xsl + (dst - src) * S * cap)
    ox, oy = torch.empty_like(q), torch.empty_like(q)
    X.ex.sparse_decode(q, X.bufs["slots"], ox)
    Y.ex.sparse_decode(qy, slots_y, oy)
    torch.cuda.synchronize()
    assert torch.equal(oy[dst], ox[src])
    assert torch.isfinite(ox[src]).all()
    # the moved request keeps running in lane 2 of Y, as in lane 1 of X
    for t in range(4, 8):
        sel = sels[t].reshape(n_req, L, Hkv, k).copy()
        sel[dst] = sel[src]
        sel = sel.reshape(-1)
        x_fetched = X.step(sels[t])
        y_fetched = Y.step(sel)
        xm = x_fetched[x_fetched[:, 3] // S == src]
        ym = y_fetched[y_fetched[:, 3] // S == dst]
        assert np.array_equal(xm[:, :3], ym[:, :3])  # same blocks, slots, evictions
        Y.check_fetched_bytes(y_fetched)
        Y.check_state()


@pytest.mark.parametrize("dtype,Hkv,Hq", [(F.F16, 2, 2), (F.FP8, 2, 8), (F.F32, 1, 2)])
def test_owner_moves_between_executors(dtype, Hkv, Hq):
    _move_and_check(dtype, Hkv, Hq)


@pytest.mark.parametrize("seed", range(12))
def test_owner_moves_random_geometry(seed):
    rng = np.random.default_rng(4000 + seed)
    dtype = int(rng.choice([F.F32, F.F16, F.BF16, F.FP8]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    n_req = int(rng.integers(2, 6))
    L = int(rng.integers(1, 4))
    k = int(rng.integers(4, 33))
    cap = k + int(rng.integers(0, 2 * k + 1))
    lo = int(rng.integers(k, 3 * k + 2))
    src, dst = (int(x) for x in rng.choice(n_req, 2, replace=False))
    print("[handoff geometry]", dict(dtype=dtype, Hkv=Hkv, G=G, n_req=n_req, L=L, k=k, cap=cap,
                                     lo=lo, src=src, dst=dst), flush=True)
    _move_and_check(dtype, Hkv, Hkv * G, n_req=n_req, L=L, k=k, cap=cap, lo=lo,
                    hi=lo + int(rng.integers(0, 300)), seed=seed + 11, src=src, dst=dst,
                    host_blocks=1031)


def test_owner_round_trip_and_refusals():
    n_req, L, Hkv, k, cap = 3, 2, 2, 12, 30
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 200, 4, seed=6)
    X = Pair(n_req, L, Hkv, Hkv, k, cap, mb, F.BF16)
    for t in range(3):
        X.step(sels[t])
    img = X.ex.alloc_owner_image()
    X.ex.owner_export(0, img)
    X.ex.reset_owners(torch.tensor([0], dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert X.ex.sets_state()[0][:L * Hkv].sum() == 0
    X.ex.owner_import(0, img)  # back where it came from: the oracle never moved
    torch.cuda.synchronize()
    assert X.ex.stats()["device_error"] == 0
    X.check_state()
    X.check_fetched_bytes(X.step(sels[3]))  # and carries on as if never moved
    X.check_state()
    # an image of another geometry is refused and leaves the owner empty
    Z = Pair(n_req, L, Hkv, Hkv, k, cap + 2, mb, F.BF16)
    zimg = Z.ex.alloc_owner_image()
    Z.ex.owner_export(0, zimg)
    X.ex.owner_import(1, zimg[:X.ex.owner_image_bytes()])
    torch.cuda.synchronize()
    assert X.ex.stats()["device_error"] == -1
    f, _, _ = X.ex.sets_state()
    assert np.all(f[1 * L * Hkv:2 * L * Hkv] == 0)
    # too small a buffer is refused before any launch
    with pytest.raises(F.FerryError, match="smaller"):
        X.ex.owner_import(0, img[:1024])
    with pytest.raises(F.FerryError, match="out of range"):
        X.ex.owner_export(n_req, img)


def test_corrupted_image_is_refused():
    n_req, L, Hkv, k, cap = 2, 1, 1, 8, 20
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 30, 100, 2, seed=2)
    X = Pair(n_req, L, Hkv, Hkv, k, cap, mb, F.F16)
    for t in range(2):
        X.step(sels[t])
    img = X.ex.alloc_owner_image()
    X.ex.owner_export(0, img)
    torch.cuda.synchronize()
    # the image's LRU order lists one slot twice
    ord_off = 64 + 8 * (L * Hkv)
    o = img[ord_off:ord_off + 8].cpu().numpy().view(np.uint32).copy()
    o[1] = o[0]
    img[ord_off:ord_off + 8] = torch.from_numpy(o.view(np.uint8)).cuda()
    X.ex.owner_import(1, img)
    torch.cuda.synchronize()
    assert X.ex.stats()["device_error"] == -1
    f, _, t = X.ex.sets_state()
    assert f[1] == 0 and np.all(t[1] == O.NONE)
