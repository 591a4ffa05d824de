"""GPU parity at the library's size limits: the largest top-k (1024), the
largest slot count the bookkeeping's 64 KiB LDS budget allows with it (4778
per set: (3 C + 2 k) * 4 bytes per wavefront), prefix-group sets too large for
the bookkeeping to stage their selections in LDS, block ids at the top of the
31-bit range, and the refusals one past each limit."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import Pair, _zipf_stream

pytestmark = pytest.mark.gpu

K_MAX = 1024
C_MAX = (65536 // 4 - 2 * K_MAX) // 3  # 4778


@pytest.mark.parametrize("dtype,Hkv,Hq", [(F.F16, 2, 2), (F.BF16, 2, 8), (F.FP8, 1, 8)])
def test_largest_k_and_slot_count(dtype, Hkv, Hq):
    # 1024 uniform selections per row out of 8192 blocks, 4778 slots per set: the sets
    # fill within a few steps and then evict; attention sums 16384 tokens per
    # row (256 blocks per wavefront)
    mb, sels = _zipf_stream(1, 1, Hkv, K_MAX, 8192, 8192, 14, seed=21, reuse=0.3, dist=0)
    p = Pair(1, 1, Hkv, Hq, K_MAX, C_MAX, mb, dtype)
    evicted = 0
    for sel in sels:
        fetched = p.step(sel)
        p.check_fetched_bytes(fetched)
        evicted += int(np.sum(fetched[:, 2] != O.NONE))
    p.check_state()
    fill, _, _ = p.ex.sets_state()
    assert np.all(fill == C_MAX) and evicted > 0
    p.check_attention(sels[-1], seed=2)


def test_one_past_the_limits_is_refused():
    with pytest.raises(F.FerryError, match="LDS budget"):
        F.Executor(1, 1, 1, K_MAX, C_MAX + 1, 8192)
    with pytest.raises(F.FerryError, match="1024"):
        F.Executor(1, 1, 1, K_MAX + 1, 64, 8192)


def test_group_sets_past_the_staging_budget():
    # 16-member prefix groups with k 64 (1,024 selections per set) and 3,200
    # slots: the set's state fits the bookkeeping's 64 KiB of LDS, but not with
    # its staged selections and slots beside it, so the passes read those from
    # HBM.  Bit-exact against the oracle in both LRU granularities, filling the
    # sets and then evicting.
    n_req, group, L, Hkv, k, C = 16, 16, 1, 1, 64, 3200
    assert (4 * C + 2 * group * k) * 4 <= 65536 < (4 * C + 4 * group * k) * 4
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 300, 600, 8, group=group, prefix=64, seed=5,
                            reuse=0.3, dist=0)
    for lru in (0, 1):
        p = Pair(n_req, L, Hkv, Hkv, k, C, mb, F.F16, group=group, lru=lru)
        evicted = 0
        for sel in sels:
            fetched = p.step(sel)
            p.check_fetched_bytes(fetched)
            evicted += int(np.sum(fetched[:, 2] != O.NONE))
        p.check_state()
        assert evicted > 0
        p.ex.close()


def test_block_ids_at_the_top_of_the_range():
    # max_blocks = 2^31 - 1 (the largest below the map's pending bit): ids
    # just under it are cached and fetched like any other; the id equal to it
    # is out of range
    mb = (1 << 31) - 1
    k, cap = 64, 96
    p = Pair(1, 1, 1, 2, k, cap, mb, F.BF16, host_blocks=1031)
    rng = np.random.default_rng(3)
    top = np.arange(mb - 4 * k, mb, dtype=np.uint64)
    prev = None
    for t in range(4):
        if prev is None:  # the first step includes the largest valid id
            sel = np.sort(np.concatenate([rng.choice(top[:-1], k - 1, replace=False), top[-1:]]))
        else:  # half reused, half new: evictions once the set is full
            keep = rng.choice(prev, k // 2, replace=False)
            fresh = rng.choice(np.setdiff1d(top, prev), k - k // 2, replace=False)
            sel = np.sort(np.concatenate([keep, fresh]))
        sel = sel.astype(np.uint32)
        p.check_fetched_bytes(p.step(sel))
        p.check_state()
        prev = sel.astype(np.uint64)
    p.check_attention(sel, seed=4)
    bad = sel.copy()
    bad[-1] = np.uint32(mb)
    dsel = torch.from_numpy(bad.view(np.int32)).cuda()
    p.ex.fetch_step(dsel, p.bufs)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == -3  # FERRY_ERANGE


@pytest.mark.parametrize("mode,Hkv,Hq", [(F.TOPK_PER_HEAD, 2, 2), (F.TOPK_LAYER_MAX, 2, 8)])
def test_selection_at_its_largest_context(mode, Hkv, Hq):
    # the selection keeps a row's query dims and one key per context block in
    # 64 KiB of LDS: contexts up to 16384 - 128 * (query heads of a row) blocks
    gq = Hq // Hkv if mode == F.TOPK_PER_HEAD else Hq
    mb = 16384 - 128 * gq
    p = Pair(2, 1, Hkv, Hq, K_MAX, 16, mb, F.F16, host_blocks=4099)
    p.ex.summaries_build()
    rng = np.random.default_rng(8)
    q = rng.standard_normal((2, 1, Hq, 128)).astype(np.float32)
    ctx = np.array([mb, mb - 777], np.int32)
    sel = torch.empty((2, 1, Hkv, K_MAX), dtype=torch.int32, device="cuda")
    p.ex.select_topk(torch.from_numpy(q).cuda(), torch.from_numpy(ctx).cuda(), sel, mode)
    torch.cuda.synchronize()
    assert np.array_equal(sel.cpu().numpy().view(np.uint32), O.select_topk(p.g, q, ctx, mode))
    assert p.ex.stats()["device_error"] == 0
    big = Pair(1, 1, Hkv, Hq, 8, 16, mb + 1, F.F16, host_blocks=4099)
    big.ex.summaries_build()
    with pytest.raises(F.FerryError, match="64 KiB"):
        big.ex.select_topk(torch.zeros((1, 1, Hq, 128), device="cuda"),
                           torch.tensor([8], dtype=torch.int32, device="cuda"),
                           torch.empty((1, 1, Hkv, 8), dtype=torch.int32, device="cuda"), mode)


def test_wrong_buffers_are_refused_before_the_call():
    """Host tensors, wrong dtypes, non-contiguous views and buffers smaller
    than the geometry are refused by the Python mirror before a pointer
    reaches a kernel; the executor works normally afterwards."""
    mb, sels = _zipf_stream(2, 2, 2, 8, 30, 60, 1, seed=4)
    p = Pair(2, 2, 2, 4, 8, 16, mb, F.F16, host_blocks=257)
    sel = torch.from_numpy(np.ascontiguousarray(sels[0], np.uint32).view(np.int32)).cuda()
    q = torch.zeros((2, 2, 4, 128), device="cuda")
    with pytest.raises(ValueError, match="CUDA tensor"):
        p.ex.fetch_step(sel.cpu(), p.bufs)
    with pytest.raises(ValueError, match="dtype"):
        p.ex.fetch_step(sel.float(), p.bufs)
    with pytest.raises(ValueError, match="contiguous"):
        p.ex.fetch_step(sel.view(2, 2, 2, 8).transpose(0, 1), p.bufs)
    with pytest.raises(ValueError, match="elements"):
        p.ex.fetch_step(sel[: sel.numel() // 2].contiguous(), p.bufs)
    bad = dict(p.bufs, misses=p.bufs["misses"][:1].contiguous())
    with pytest.raises(ValueError, match="misses"):
        p.ex.fetch_step(sel, bad)
    with pytest.raises(ValueError, match="elements"):
        p.ex.sparse_decode(q[:1].contiguous(), p.bufs["slots"], torch.empty_like(q))
    with pytest.raises(ValueError, match="ctx_blocks"):
        p.ex.summaries_build()
        p.ex.select_topk(q, torch.zeros(1, dtype=torch.int32, device="cuda"), sel)
    p.check_fetched_bytes(p.step(sels[0]))
    assert p.ex.stats()["device_error"] == 0


def test_pageable_memory_is_refused_at_the_c_boundary():
    """The C entry points take bare pointers; one into pageable host memory
    (here numpy's) returns FERRY_EINVAL instead of reaching a kernel."""
    import ctypes as C
    mb, sels = _zipf_stream(2, 1, 1, 8, 20, 40, 1, seed=6)
    p = Pair(2, 1, 1, 2, 8, 16, mb, F.F16, host_blocks=257)
    q_host = np.zeros((2, 1, 2, 128), np.float32)
    out = torch.empty((2, 1, 2, 128), device="cuda")
    rc = F.lib.ferry_sparse_decode(p.ex._h, C.c_void_p(q_host.ctypes.data),
                                   C.c_void_p(p.bufs["slots"].data_ptr()),
                                   C.c_void_p(out.data_ptr()), None)
    assert rc == -1 and b"not device-accessible" in F.lib.ferry_last_error()
    sel_host = np.ascontiguousarray(sels[0], np.uint32)
    rc = F.lib.ferry_fetch_step(p.ex._h, C.c_void_p(sel_host.ctypes.data),
                                *[C.c_void_p(p.bufs[k].data_ptr()) for k in
                                  ("slots", "miss_count", "misses", "miss_flag")], None)
    assert rc == -1 and b"sel" in F.lib.ferry_last_error()
    p.check_fetched_bytes(p.step(sels[0]))  # nothing was launched; the executor works
    assert p.ex.stats()["device_error"] == 0
