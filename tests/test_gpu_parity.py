"""GPU parity: the HIP path through the C-ABI against the CPU oracle.

Bookkeeping (slot of every selection, per-set miss lists with evictions, miss
flags, LRU state) and the fetched bytes must be bit-exact; attention must be
within 2e-3 relative (fp32/fp16/bf16) or 1e-2 (fp8) of the fp64 oracle, where
the relative error of a (request, layer, head) row is
max|out - ref| / max|ref|.
"""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

TOL = {F.F32: 2e-3, F.F16: 2e-3, F.BF16: 2e-3, F.FP8: 1e-2}


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


class Pair:
    """A GPU executor and its oracle twin built from the same geometry."""

    def __init__(self, n_req, L, Hkv, Hq, k, cap, max_blocks, dtype, group=1, lru=0,
                 host_blocks=4099, steal=1, assign=0, workers=0, seed=7, value_std=0.5,
                 attn=F.ATTN_AUTO):
        print(f"[pair] B={n_req} L={L} Hkv={Hkv} Hq={Hq} k={k} C={cap} mb={max_blocks} "
              f"dtype={dtype} group={group} lru={lru} steal={steal} assign={assign} attn={attn}",
              flush=True)
        self.ex = F.Executor(n_req, L, Hkv, k, cap, max_blocks, q_heads=Hq, group=group,
                             dtype=dtype, lru_mode=lru, host_blocks=host_blocks, host_seed=seed,
                             value_std=value_std, fetch_workers=workers, steal=steal,
                             assign=assign, attn=attn)
        self.g = O.make_geom(n_req=n_req, group=group, n_layers=L, kv_heads=Hkv, q_heads=Hq,
                             k=k, cap=cap, max_blocks=max_blocks, dtype=dtype, granularity=lru,
                             host_blocks=host_blocks, seed=seed, value_std=value_std)
        self.ox = O.Executor(self.g)
        self.ex.hosttier_fill()
        torch.cuda.synchronize()
        self.host, self.hsc = self.ex.hosttier_array()
        self.bufs = self.ex.alloc_step_buffers()
        self.dtype = dtype
        self.bb = self.ex.block_bytes

    def step(self, sel):
        ex = self.ex
        dsel = torch.from_numpy(np.ascontiguousarray(sel, np.uint32).view(np.int32)).cuda()
        ex.fetch_step(dsel, self.bufs)
        torch.cuda.synchronize()
        st = ex.stats()
        assert st["device_error"] == 0, st
        oslots, omc, omiss, _ = self.ox.step(sel)
        slots = _u32(self.bufs["slots"]).reshape(-1)
        mc = _u32(self.bufs["miss_count"])
        gm = _u32(self.bufs["misses"]).reshape(ex.n_sets, ex.max_sel, 4)
        flags = self.bufs["miss_flag"].cpu().numpy().reshape(-1)
        assert np.array_equal(slots, oslots)
        assert np.array_equal(mc, omc)
        assert np.array_equal(flags, self.ox.last_flags)
        fetched = []
        for s in np.nonzero(mc)[0]:
            m = gm[s, :mc[s]]
            o = omiss[s, :mc[s]]
            assert np.array_equal(m[:, 0], o["block"])
            assert np.array_equal(m[:, 1], o["slot"])
            assert np.array_equal(m[:, 2], o["evicted"])
            assert np.all(m[:, 3] == s) and np.all(o["set"] == s)
            fetched.append(m)
        assert st["last_misses"] == int(mc.sum())
        return np.concatenate(fetched) if fetched else np.zeros((0, 4), np.uint32)

    def check_state(self):
        fill, ord_, tag = self.ex.sets_state()
        ofill, oord, otag = self.ox.state()
        assert np.array_equal(fill, ofill)
        assert np.array_equal(tag, otag)
        for s in range(len(fill)):
            assert np.array_equal(ord_[s, :fill[s]], oord[s, :fill[s]])

    def check_fetched_bytes(self, fetched, limit=4096):
        if len(fetched) == 0:
            return
        rng = np.random.default_rng(len(fetched))
        pick = fetched if len(fetched) <= limit else fetched[rng.choice(len(fetched), limit, False)]
        gslots = pick[:, 3].astype(np.int64) * self.g.cap + pick[:, 1]
        got = self.ex.pool_slots_bytes(gslots)
        hidx = (pick[:, 3].astype(np.uint64) * np.uint64(self.g.max_blocks)
                + pick[:, 0].astype(np.uint64)) % np.uint64(self.g.host_blocks)
        want = self.host.reshape(-1, self.bb)[hidx.astype(np.int64)]
        assert np.array_equal(got, want)
        if self.dtype == F.FP8:
            gs = self.ex.pool_slot_scales(gslots)
            assert np.array_equal(gs, self.hsc.reshape(-1, 2)[hidx.astype(np.int64)])

    def check_attention(self, sel, seed=0, q_std=1.0):
        g = self.g
        rng = np.random.default_rng(seed)
        q = (rng.standard_normal((g.n_req, g.n_layers, g.q_heads, 128)) * q_std).astype(np.float32)
        dq = torch.from_numpy(q).cuda()
        out = torch.empty_like(dq)
        self.ex.sparse_decode(dq, self.bufs["slots"], out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
        ref = O.attention_f64(g, sel, q).reshape(-1, 128)
        rel = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
        assert np.all(np.isfinite(got))
        assert rel.max() < TOL[self.dtype], rel.max()
        return rel.max()


def _zipf_stream(n_req, L, H, k, lo, hi, steps, seed=3, reuse=0.66, group=1, prefix=0, dist=1,
                 s=1.1):
    ctx = O.ctx_uniform(seed, n_req, lo, hi)
    sg = O.selgen(n_req, L, H, k, ctx, dist=dist, zipf_s=s, reuse=reuse, group=group,
                  prefix_blocks=prefix, seed=seed)
    return O.selgen_max_blocks(sg), [O.selgen_step(sg, t) for t in range(steps)]


def test_hosttier_content_matches_oracle():
    for dtype in (F.F32, F.F16, F.BF16, F.FP8):
        p = Pair(1, 1, 1, 1, 1, 1, 1, dtype, host_blocks=257)
        for h in (0, 1, 17, 128, 256):
            raw, sc = O.host_block(p.g, h)
            assert np.array_equal(p.host.reshape(-1, p.bb)[h], raw)
            if dtype == F.FP8:
                assert np.array_equal(p.hsc.reshape(-1, 2)[h], sc)


@pytest.mark.parametrize("dtype,Hkv,Hq", [(F.F16, 4, 4), (F.BF16, 2, 8), (F.F32, 2, 2)])
def test_step_mode_parity_multistep(dtype, Hkv, Hq):
    n_req, L, k, cap = 4, 2, 16, 40
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 60, 300, 7)
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype)
    for t, sel in enumerate(sels):
        fetched = p.step(sel)
        p.check_fetched_bytes(fetched)
        p.check_state()
        if t in (0, 3, 6):
            p.check_attention(sel, seed=t)


def test_fp8_prefix_groups_dedup_parity():
    # 8 requests in 2 prefix groups; GQA 8/2; concurrent misses on a shared
    # block dedup to one fetch.
    n_req, group, L, Hkv, Hq, k = 8, 4, 2, 2, 8, 16
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 80, 200, 5, group=group, prefix=64)
    p = Pair(n_req, L, Hkv, Hq, k, group * k + 24, mb, F.FP8, group=group)
    for t, sel in enumerate(sels):
        fetched = p.step(sel)
        keys = fetched[:, 3].astype(np.uint64) << np.uint64(32) | fetched[:, 0].astype(np.uint64)
        assert len(np.unique(keys)) == len(keys)  # one fetch per (set, block)
        p.check_fetched_bytes(fetched)
        p.check_state()
        if t in (0, 4):
            p.check_attention(sel, seed=t)


def test_config1_shape_parity():
    # CPU-plumbing workload: 1 layer, 8 heads MHA, fp32, B=4 x 128 blocks,
    # k=32 uniform without replacement.
    mb, sels = _zipf_stream(4, 1, 8, 32, 128, 128, 6, dist=0, reuse=0.5)
    p = Pair(4, 1, 8, 8, 32, 96, mb, F.F32, value_std=1.0)
    for t, sel in enumerate(sels):
        p.check_fetched_bytes(p.step(sel))
        p.check_state()
    p.check_attention(sels[-1], seed=9)


def test_serial_mode_reproduces_reference_golden():
    # replay_miss_stream semantics (per-selection LRU, hot 128 per (r, l)) on
    # the GPU: 79,550 misses of 589,824 selections (results/wla_7rep_20260930).
    R, L, S, sel_n, hot = 48, 12, 16, 64, 128
    sel = F.refgen_selections(R, L, S, sel_n, 42)  # [R, S, L, sel]
    _, ref_miss, _, ref_total = O.ref_replay(R, L, S, sel_n, hot, 42)
    ref_miss = ref_miss.reshape(R, S, L, sel_n)
    ex = F.Executor(R, L, 1, sel_n, hot, 64 + 8 * S, dtype=F.F16, lru_mode=F.LRU_SERIAL,
                    host_blocks=1 << 12)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    total = 0
    for s in range(S):
        step_sel = np.ascontiguousarray(sel[:, s, :, None, :])
        ex.fetch_step(torch.from_numpy(step_sel.view(np.int32)).cuda(), bufs)
        flags = bufs["miss_flag"].cpu().numpy().reshape(R, L, sel_n)
        assert np.array_equal(flags, ref_miss[:, s])
        total += int(_u32(bufs["miss_count"]).sum())
    st = ex.stats()
    assert st["device_error"] == 0
    assert total == ref_total == 79550
    assert st["misses"] == 79550 and st["fetched_bytes"] == 79550 * ex.block_bytes


@pytest.mark.parametrize("mode", [0, 1])
def test_queue_exactly_once(mode):
    # a large ring (65,536 cells): throughput of both reservation modes
    popped, dups, ms = F.queue_selftest(capacity=1 << 16, n_tasks=1 << 20, producers=512,
                                        consumers=512, mode=mode)
    assert popped == 1 << 20 and dups == 0


@pytest.mark.parametrize("mode", [0, 1])
def test_queue_small_ring_partial_pops(mode):
    # 1000 cells (not a multiple of 64) under 256 producers and 1024 consumers:
    # the consumers outnumber what is queued, so wavefront pops often get fewer
    # tickets than lanes asked, and every cell wraps 65 times.
    popped, dups, ms = F.queue_selftest(capacity=1000, n_tasks=1 << 16, producers=256,
                                        consumers=1024, mode=mode)
    assert popped == 1 << 16 and dups == 0


@pytest.mark.parametrize("mode", [0, 1])
def test_queue_more_producers_than_cells(mode):
    # 64 cells under 2048 producers and 512 consumers.  Per-thread
    # reservation (mode 0) can hand lanes of one wavefront tickets a lap or
    # more apart: the later lane's cell is released only after the earlier
    # lane's task is consumed, so each lane must publish as soon as its own
    # cell is free rather than after its siblings' waits.
    popped, dups, ms = F.queue_selftest(capacity=64, n_tasks=1 << 16, producers=2048,
                                        consumers=512, mode=mode)
    assert popped == 1 << 16 and dups == 0
    # fewer cells than a wavefront's lanes: a wave-batched push takes a ticket
    # per lane instead of one batch the ring could never hold
    popped, dups, ms = F.queue_selftest(capacity=16, n_tasks=1 << 14, producers=4096,
                                        consumers=256, mode=mode)
    assert popped == 1 << 14 and dups == 0


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_ticket_probe_counts_every_ticket(kind):
    tickets, ms = F.queue_ticket_probe(threads=512, iters=8, kind=kind)
    assert tickets == 512 * 8 and ms > 0
    with pytest.raises(F.FerryError, match="kind"):
        F.queue_ticket_probe(threads=256, iters=1, kind=3)


def test_steal_and_assignment_do_not_change_results():
    n_req, L, H, k, cap = 6, 2, 4, 16, 48
    mb, sels = _zipf_stream(n_req, L, H, k, 100, 400, 4, seed=11)
    variants = [dict(steal=0, assign=F.ASSIGN_SPREAD, workers=64),
                dict(steal=1, assign=F.ASSIGN_AFFINITY, workers=64),
                dict(steal=0, assign=F.ASSIGN_AFFINITY, workers=3)]
    pools = []
    steals = []
    for v in variants:
        p = Pair(n_req, L, H, H, k, cap, mb, F.F16, **v)
        for sel in sels:
            p.step(sel)
        p.check_state()
        allslots = np.arange(p.ex.pool_slots)
        pools.append(p.ex.pool_slots_bytes(allslots))
        steals.append(p.ex.stats()["steals"])
        p.ex.close()
    assert all(np.array_equal(pools[0], x) for x in pools[1:])
    assert steals[1] > 0  # affinity leaves most workers idle: they steal


def test_missq_push_then_drain():
    p = Pair(2, 1, 2, 2, 4, 8, 32, F.BF16, host_blocks=61)
    rng = np.random.default_rng(1)
    n = 10
    sets = rng.integers(0, p.ex.n_sets, n)
    slots = rng.permutation(p.ex.pool_slots)[:n]  # distinct destinations
    m = np.zeros((n, 4), np.uint32)
    m[:, 0] = rng.integers(0, 32, n)
    m[:, 3] = slots // 8
    m[:, 1] = slots % 8
    m[:, 2] = 0xFFFFFFFF
    dm = torch.from_numpy(m.view(np.int32)).cuda()
    p.ex.missq_push(dm, n)
    p.ex.missq_drain()
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == 0
    p.check_fetched_bytes(m)
    assert sets is not None


def test_capacity_and_range_errors_are_reported():
    p = Pair(1, 1, 1, 1, 8, 4, 16, F.F16)  # 8 distinct blocks per step > 4 slots
    sel = np.arange(8, dtype=np.uint32)
    p.ex.fetch_step(torch.from_numpy(sel.view(np.int32)).cuda(), p.bufs)
    assert p.ex.stats()["device_error"] == -4
    p.ex.stats_reset()
    fill, _, _ = p.ex.sets_state()
    assert fill[0] == 0  # the failed step left the set untouched
    sel = np.array([0, 1, 2, 99, 3, 4, 5, 6], np.uint32)  # 99 >= max_blocks
    p.ex.fetch_step(torch.from_numpy(sel.view(np.int32)).cuda(), p.bufs)
    assert p.ex.stats()["device_error"] == -3


def test_steady_state_properties_at_scale():
    # 7B-like slice: 16 requests x 8 layers x 8 heads, k=64, C=320, contexts
    # 256..2048 blocks; invariants that need no oracle replay.
    n_req, L, H, k, cap = 16, 8, 8, 64, 320
    ctx = F.ctx_uniform(2, n_req, 256, 2048)
    sg = F.SelGen(n_req, L, H, k, ctx, seed=3)
    ex = F.Executor(n_req, L, H, k, cap, sg.max_blocks, dtype=F.F16, host_blocks=1 << 15)
    ex.hosttier_fill()
    host, _ = ex.hosttier_array()
    bufs = ex.alloc_step_buffers()
    for t in range(12):
        sel = sg.step(t)
        ex.fetch_step(torch.from_numpy(sel.view(np.int32)).cuda(), bufs)
    st = ex.stats()
    assert st["device_error"] == 0
    fill, ord_, tag = ex.sets_state()
    slots = _u32(bufs["slots"]).reshape(n_req, L, H, k)
    # every selection's slot holds its block; each set's order is a permutation
    sets = (np.arange(n_req)[:, None, None] * L + np.arange(L)[None, :, None]) * H + \
        np.arange(H)[None, None, :]
    assert np.all(slots // cap == sets[..., None])
    assert np.array_equal(tag.reshape(-1)[slots.reshape(-1)], sel.reshape(-1))
    for s in range(0, ex.n_sets, 37):
        assert sorted(ord_[s, :fill[s]].tolist()) == list(range(fill[s]))
    # fetched bytes of the last step equal the host tier
    mc = _u32(bufs["miss_count"])
    gm = _u32(bufs["misses"]).reshape(ex.n_sets, ex.max_sel, 4)
    m = np.concatenate([gm[s, :mc[s]] for s in np.nonzero(mc)[0]])[:2048]
    got = ex.pool_slots_bytes(m[:, 3].astype(np.int64) * cap + m[:, 1])
    hidx = (m[:, 3].astype(np.int64) * sg.max_blocks + m[:, 0]) % (1 << 15)
    assert np.array_equal(got, host.reshape(-1, ex.block_bytes)[hidx])
    assert 0.02 < st["last_misses"] / (n_req * L * H * k) < 0.3


@pytest.mark.parametrize("chunks", [4, 0])
def test_decode_step_overlap_matches_sequential(chunks):
    # layer-chunked pipeline (fetch of chunk c+1 on a side stream while chunk c
    # attends) must produce exactly the sequential step's slots, pool and output;
    # chunks 0 picks the count from the previous step's fetched bytes
    n_req, L, Hkv, Hq, k, cap = 4, 6, 2, 8, 16, 40
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 60, 300, 5)
    seq = Pair(n_req, L, Hkv, Hq, k, cap, mb, F.BF16)
    ovl = Pair(n_req, L, Hkv, Hq, k, cap, mb, F.BF16)
    if chunks == 0:  # small units, so that these small steps are cut into several chunks
        ovl.ex.set_batch_policy(min_mb=0.01, max_mb=0.05, target_batches=4)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(3)
    for t, sel in enumerate(sels):
        q = torch.from_numpy(rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)).cuda()
        o1, o2 = torch.empty_like(q), torch.empty_like(q)
        d = torch.from_numpy(sel.view(np.int32)).cuda()
        seq.ex.fetch_step(d, seq.bufs)
        seq.ex.sparse_decode(q, seq.bufs["slots"], o1)
        ovl.ex.decode_step(d, q, ovl.bufs, o2, chunks=chunks, side_stream=side)
        torch.cuda.synchronize()
        assert np.array_equal(_u32(seq.bufs["slots"]), _u32(ovl.bufs["slots"]))
        assert torch.equal(o1, o2)
        assert ovl.ex.stats()["device_error"] == 0
    f1, o1_, t1 = seq.ex.sets_state()
    f2, o2_, t2 = ovl.ex.sets_state()
    assert np.array_equal(f1, f2) and np.array_equal(o1_, o2_) and np.array_equal(t1, t2)
    allslots = np.arange(seq.ex.pool_slots)
    assert np.array_equal(seq.ex.pool_slots_bytes(allslots), ovl.ex.pool_slots_bytes(allslots))
    ovl.check_attention(sels[-1], seed=11)


def test_adaptive_chunk_policy_known_answers():
    # AdaptiveBatchPolicy::choose_mb (src/runtime/adaptive_batch.cuh:31-36) in GPU
    # units: g = clamp(pending_MB / 8, 32, 512) MB per chunk, ceil(pending / g)
    # chunks, at least 1 and at most L.  8 KiB blocks: 1 MB = 128 blocks.
    p = Pair(2, 32, 2, 2, 8, 16, 64, F.F16)
    bb = p.ex.block_bytes
    assert bb == 8192
    mb = 1 << 20
    cases = {0: 1, 1: 1, 32 * mb // bb: 1, 33 * mb // bb: 2, 184 * mb // bb: 6,
             1290 * mb // bb: 8, 3440 * mb // bb: 8, 8192 * mb // bb: 16,
             (1 << 40) // bb: 32}
    for blocks, want in cases.items():
        assert p.ex.decode_chunks(blocks) == want, (blocks, want)
    p.ex.set_batch_policy(1.0, 4.0, 4.0)  # the reference's channel defaults
    assert p.ex.decode_chunks(16 * mb // bb) == 4 and p.ex.decode_chunks(2 * mb // bb) == 2
    with pytest.raises(F.FerryError):
        p.ex.set_batch_policy(8.0, 4.0, 4.0)


def test_per_layer_bookkeeping_equals_whole_step():
    n_req, L, H, k, cap = 3, 4, 2, 16, 32
    mb, sels = _zipf_stream(n_req, L, H, k, 60, 200, 4)
    p = Pair(n_req, L, H, H, k, cap, mb, F.F16)
    for sel in sels:
        d = torch.from_numpy(sel.view(np.int32)).cuda()
        for l0 in range(L):
            p.ex.bookkeep_layers(l0, 1, d, p.bufs)
            p.ex.missq_drain()
        torch.cuda.synchronize()
        oslots, omc, _, _ = p.ox.step(sel)
        assert np.array_equal(_u32(p.bufs["slots"]).reshape(-1), oslots)
        assert np.array_equal(_u32(p.bufs["miss_count"]), omc)
    p.check_state()


@pytest.mark.parametrize("dtype", [F.F16, F.BF16, F.FP8])
@pytest.mark.parametrize("G", [2, 4, 8])
def test_mfma_attention_matches_oracle_and_valu(dtype, G):
    # GQA head groups on the matrix cores against the fp64 oracle, and the
    # vector-ALU kernel on the same pool within the same tolerance.  k=13 gives
    # the four wavefronts unequal block counts.
    n_req, L, Hkv, k = 3, 2, 2, 13
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 200, 2, seed=G)
    pm = Pair(n_req, L, Hkv, Hkv * G, k, 32, mb, dtype, attn=F.ATTN_MFMA)
    pv = Pair(n_req, L, Hkv, Hkv * G, k, 32, mb, dtype, attn=F.ATTN_VALU)
    for t, sel in enumerate(sels):
        pm.step(sel)
        pv.step(sel)
    for q_std in (1.0, 4.0):  # 4.0: peaked softmax, scores up to ~30 in log2 units
        pm.check_attention(sels[-1], seed=5, q_std=q_std)
        pv.check_attention(sels[-1], seed=5, q_std=q_std)
    assert pm.ex.stats()["device_error"] == 0


@pytest.mark.parametrize("dtype,G,attn", [(F.F32, 1, F.ATTN_AUTO), (F.F16, 1, F.ATTN_AUTO),
                                           (F.BF16, 4, F.ATTN_VALU), (F.BF16, 4, F.ATTN_MFMA),
                                           (F.FP8, 4, F.ATTN_MFMA), (F.FP8, 2, F.ATTN_VALU),
                                           (F.FP8, 1, F.ATTN_AUTO)])
def test_attention_load_flavours_are_bit_identical(dtype, G, attn, monkeypatch):
    # Non-temporal and temporal K/V loads differ only in cache policy: the
    # outputs must be bit-identical, and both within tolerance of the oracle.
    n_req, L, Hkv, k = 3, 2, 2, 13
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 200, 2, seed=9)
    outs = []
    for flavour in ("nt", "temporal"):
        monkeypatch.setenv("FERRY_ATTN_LOADS", flavour)
        p = Pair(n_req, L, Hkv, Hkv * G, k, 32, mb, dtype, attn=attn)
        for sel in sels:
            p.step(sel)
        p.check_attention(sels[-1], seed=5)
        q = torch.from_numpy(np.random.default_rng(5).standard_normal(
            (n_req, L, Hkv * G, 128)).astype(np.float32)).cuda()
        out = torch.empty_like(q)
        p.ex.sparse_decode(q, p.bufs["slots"], out)
        torch.cuda.synchronize()
        outs.append(out.cpu())
        p.ex.close()
    assert torch.equal(outs[0], outs[1])


def test_fp8_mha_runs_on_the_matrix_cores():
    # fp8 MHA (one query head per kv head): AUTO picks the MFMA kernel with one
    # live column of its 16; it matches the fp64 oracle and the VALU kernel.
    n_req, L, H, k = 3, 2, 4, 13
    mb, sels = _zipf_stream(n_req, L, H, k, 40, 200, 2, seed=11)
    pm = Pair(n_req, L, H, H, k, 32, mb, F.FP8)
    pv = Pair(n_req, L, H, H, k, 32, mb, F.FP8, attn=F.ATTN_VALU)
    assert pm.ex.attn_kernel()[0] == F.ATTN_MFMA and pv.ex.attn_kernel()[0] == F.ATTN_VALU
    for sel in sels:
        pm.step(sel)
        pv.step(sel)
    for q_std in (1.0, 4.0):
        pm.check_attention(sels[-1], seed=3, q_std=q_std)
        pv.check_attention(sels[-1], seed=3, q_std=q_std)
    q = torch.from_numpy(np.random.default_rng(3).standard_normal(
        (n_req, L, H, 128)).astype(np.float32)).cuda()
    om, ov = torch.empty_like(q), torch.empty_like(q)
    pm.ex.sparse_decode(q, pm.bufs["slots"], om)
    pv.ex.sparse_decode(q, pv.bufs["slots"], ov)
    torch.cuda.synchronize()
    rel = ((om - ov).abs().amax(dim=-1) / ov.abs().amax(dim=-1)).max().item()
    assert rel < 5e-3, rel
    assert pm.ex.stats()["device_error"] == 0


def test_mfma_attention_long_selection():
    # k = 300 blocks per kv head: 75 blocks per wavefront, so the slot ids are
    # re-read past the first 64 (one per lane) inside the kernel.
    n_req, L, Hkv, G, k = 2, 1, 2, 4, 300
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 400, 600, 1, seed=4)
    for dtype in (F.BF16, F.FP8):
        p = Pair(n_req, L, Hkv, Hkv * G, k, 320, mb, dtype, host_blocks=1 << 13,
                 attn=F.ATTN_MFMA)
        p.step(sels[0])
        p.check_attention(sels[0], seed=2)
        p.ex.close()


def test_bandwidth_probes_move_the_stated_bytes():
    # ferry_bw_probe: gather of a step's slot table, host reads and DMA copies
    n_req, L, H, k = 4, 2, 2, 16
    mb, sels = _zipf_stream(n_req, L, H, k, 60, 200, 1)
    p = Pair(n_req, L, H, H, k, 32, mb, F.F16)
    p.step(sels[0])
    rows = n_req * L * H
    b, ms, gbs = p.ex.bw_probe(F.PROBE_HBM_GATHER, rows, slots=p.bufs["slots"], iters=2)
    assert b == rows * k * p.bb and ms > 0 and gbs > 0
    for kind in (F.PROBE_HOST_READ, F.PROBE_HOST_DMA):
        b, ms, gbs = p.ex.bw_probe(kind, 512, iters=2)
        assert b == 512 * p.bb and ms > 0 and gbs > 0
    pool = n_req * L * H * 32
    b, ms, gbs = p.ex.bw_probe(F.PROBE_HBM_COPY, pool, iters=2)  # every pool slot, read + written
    assert b == 2 * pool * p.bb and ms > 0 and gbs > 0
    with pytest.raises(F.FerryError):
        p.ex.bw_probe(F.PROBE_HOST_READ, 1 << 40)  # more than the host tier holds
    with pytest.raises(F.FerryError, match="pool"):
        p.ex.bw_probe(F.PROBE_HBM_COPY, pool + 1)
    assert p.ex.stats()["device_error"] == 0
