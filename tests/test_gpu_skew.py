"""The skewed, bursty work-stealing configuration on the GPU, against the
oracle: a 7B-shape slice (8 requests x 32 layers x 32 kv heads, fp16, top-k
64, 320 slots per set), per-request miss counts lognormal(2, 1.2) (each
request re-draws lognormal-many of its 64 blocks per step), Zipf popularity
s in {0.6, 1.0, 1.4}, 304 persistent fetch workgroups with request-affinity
assignment of misses to their deques, stealing off and on.  The reference's
stealing rules are the victim = largest excess over the fair share and the
take min(k, cur - fair, cur/2 + 1) (src/runtime/wla_multigpu.cuh:882-911,
1147-1152, 1518-1534; src/runtime/multigpu.cuh:153-175).

Both executors run the same selections: a steady batch, then ticks of a
Markov-modulated arrival process (rates 1x and 10x) in which finished requests
leave and arrived ones take their lane, which is reset.  Every step, each
executor's slots, per-set miss lists and miss flags must equal the oracle's
bit for bit; at the end of each phase the LRU state too, and the two pools
must be byte-identical over every slot (stealing changes who copies a block,
never what lands where), with sampled fetched blocks equal to the host tier.
With stealing on the drains must have stolen.

The same twins also run the pipelined decode step the benchmark times
(ferry_decode_step with adaptive layer ranges and a side stream, stealing
beside the overlapped attention): slots and miss lists bit-exact every step,
outputs bit-identical between the twins and within 2e-3 of float64, LRU state
and pools at the end.  The whole 64-request batch at Zipf 1.4 with stealing
runs that step from the cold pool with the first two requests replayed in the
oracle (oracle/gate.py)."""
import ctypes as C

import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O
from oracle.gate import OwnerReplay

pytestmark = pytest.mark.gpu

B, L, H, K, CAP, WORKERS = 8, 32, 32, 64, 320, 304
HB = 1 << 16


def _lognormal_reuse(n, k, mu=2.0, sigma=1.2, seed=17):
    z = np.random.default_rng(seed).standard_normal(n)
    return np.clip(1.0 - np.minimum(np.exp(mu + sigma * z), k) / k, 0.0, 1.0)


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


_hip = None


def _pools_equal(ex_a, ex_b, chunk=1 << 30):
    """Byte equality of two executors' whole HBM pools, compared on the
    device: device-to-device copies into torch buffers, chunk by chunk."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    pa, _ = ex_a.pool_ptrs()
    pb, _ = ex_b.pool_ptrs()
    total = ex_a.pool_slots * ex_a.block_bytes
    assert total == ex_b.pool_slots * ex_b.block_bytes
    ba = torch.empty(chunk, dtype=torch.uint8, device="cuda")
    bb = torch.empty(chunk, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    for off in range(0, total, chunk):
        n = min(chunk, total - off)
        assert _hip.hipMemcpy(ba.data_ptr(), pa + off, n, 3) == 0
        assert _hip.hipMemcpy(bb.data_ptr(), pb + off, n, 3) == 0
        if not torch.equal(ba[:n], bb[:n]):
            return False
    return True


class Twin:
    """Two GPU executors (stealing off / on) and one oracle, same geometry."""

    def __init__(self, max_blocks):
        self.ex = {}
        for steal in (0, 1):
            e = F.Executor(B, L, H, K, CAP, max_blocks, dtype=F.F16, host_blocks=HB,
                           fetch_workers=WORKERS, steal=steal, assign=F.ASSIGN_AFFINITY)
            e.hosttier_fill()
            self.ex[steal] = (e, e.alloc_step_buffers())
        self.g = O.make_geom(n_req=B, n_layers=L, kv_heads=H, k=K, cap=CAP,
                             max_blocks=max_blocks, dtype=F.F16, host_blocks=HB)
        self.ox = O.Executor(self.g)
        torch.cuda.synchronize()
        host, _ = self.ex[0][0].hosttier_array()
        self.hostb = host.reshape(HB, -1)
        self.rng = np.random.default_rng(5)

    def reset(self, lanes):
        for e, _ in self.ex.values():
            e.reset_owners(torch.tensor(lanes, dtype=torch.int32, device="cuda"))
        for ln in lanes:
            self.ox.reset_owner(ln)

    def step(self, sel):
        dsel = torch.from_numpy(np.ascontiguousarray(sel, np.uint32).view(np.int32)).cuda()
        for e, bufs in self.ex.values():
            e.fetch_step(dsel, bufs)
        torch.cuda.synchronize()
        oslots, omc, oms, _ = self.ox.step(sel)
        oms4 = oms.view(np.uint32).reshape(self.ox.n_sets, -1, 4)
        live = np.arange(oms4.shape[1])[None, :] < omc[:, None]
        for steal, (e, bufs) in self.ex.items():
            st = e.stats()
            assert st["device_error"] == 0, (steal, st)
            assert np.array_equal(_u32(bufs["slots"]).reshape(-1), oslots), steal
            assert np.array_equal(_u32(bufs["miss_count"]), omc), steal
            assert np.array_equal(bufs["miss_flag"].cpu().numpy().reshape(-1), self.ox.last_flags)
            gms = _u32(bufs["misses"]).reshape(self.ox.n_sets, -1, 4)
            assert np.array_equal(gms[live], oms4[live]), steal
        # sampled fetched blocks of this step against the host tier
        fetched = oms4[live]
        if len(fetched):
            pick = fetched[self.rng.choice(len(fetched), min(2048, len(fetched)), replace=False)]
            gslots = pick[:, 3].astype(np.int64) * CAP + pick[:, 1]
            hidx = (pick[:, 3].astype(np.int64) * self.g.max_blocks + pick[:, 0]) % HB
            for e, _ in self.ex.values():
                assert np.array_equal(e.pool_slots_bytes(gslots), self.hostb[hidx])
        return int(omc.sum())

    def check_state(self):
        ofill, oord, otag = self.ox.state()
        for steal, (e, _) in self.ex.items():
            fill, ord_, tag = e.sets_state()
            assert np.array_equal(fill, ofill) and np.array_equal(tag, otag), steal
            live = np.arange(CAP)[None, :] < ofill[:, None]
            assert np.array_equal(ord_[live], oord[live]), steal
        assert _pools_equal(self.ex[0][0], self.ex[1][0])


@pytest.mark.parametrize("zipf", [0.6, 1.0, 1.4])
def test_skew_stealing_on_off_parity(zipf):
    print(f"[skew] zipf={zipf} B={B} L={L} H={H} k={K} C={CAP} workers={WORKERS}", flush=True)
    n_req = 24
    reuse_req = _lognormal_reuse(n_req, K)
    ctx_req = F.ctx_uniform(7, n_req, 256, 2048)
    sg = F.SelGen(B, L, H, K, np.full(B, 2048, np.int32), dist=1, zipf_s=zipf, reuse=0.66,
                  seed=3)
    tw = Twin(sg.max_blocks)
    # phase 1: steady batch, requests 0..7 in lanes 0..7
    for ln in range(B):
        sg.admit(ln, ln, int(ctx_req[ln]), 0)
    sg.set_reuse(reuse_req[:B])
    misses = []
    for t in range(5):
        misses.append(tw.step(sg.step(t)))
    tw.check_state()
    # phase 2: Markov-modulated arrivals (rates 1x / 10x), requests 8.. take
    # the lanes of finished ones (lane reset), each with its own lognormal reuse
    arrive = 5 + F.arrivals(F.ARRIVAL_MMPP, n_req - B, 1.0, 2.0, 10.0, seed=4)
    lens = np.concatenate([F.ctx_uniform(2, B, 5, 9), F.ctx_uniform(3, n_req - B, 2, 6)])
    sched = F.Sched(B, np.concatenate([np.zeros(B), arrive]), lens)
    lane_reuse = reuse_req[:B].copy()
    ticks = 0
    for t in range(5, 17):
        r = sched.tick(float(t - 5))
        for ln in r["retired"]:
            sg.retire(int(ln))
        new = [int(x) for x in r["admitted"] if t > 5]
        for ln in new:
            rid = int(r["lane_req"][ln])
            sg.admit(ln, rid, int(ctx_req[rid]), t)
            lane_reuse[ln] = reuse_req[rid]
        if new:
            sg.set_reuse(lane_reuse)
            tw.reset(new)
        if r["resident"] == 0:
            continue
        misses.append(tw.step(sg.step(t)))
        ticks += 1
    tw.check_state()
    assert ticks >= 8 and all(m > 0 for m in misses)
    s0, s1 = tw.ex[0][0].stats(), tw.ex[1][0].stats()
    assert s0["steals"] == 0 and s1["steals"] > 0
    assert s0["misses"] == s1["misses"] == sum(misses)
    print(f"[skew] zipf={zipf}: {sum(misses)} misses over {len(misses)} steps, "
          f"{s1['steals']} steals moved {s1['stolen']}", flush=True)


def _attention_layers_f64(g, sel, q, layers):
    """float64 attention of the given layers (the others left empty)."""
    s = np.full_like(sel, O.NONE)
    s[:, layers] = sel[:, layers]
    return O.attention_f64(g, s, q)[:, layers]


@pytest.mark.parametrize("zipf", [0.6, 1.0, 1.4])
def test_skew_pipelined_decode_step_parity(zipf):
    # the step the benchmark times for this configuration: ferry_decode_step
    # with adaptive layer ranges, bookkeeping two ranges ahead and the fetch of
    # each range on a side stream while the range before it attends, with the
    # 304 request-affine workgroups stealing (or not) beside that attention
    print(f"[skew pipelined] zipf={zipf} B={B} L={L} H={H} k={K} C={CAP} workers={WORKERS}",
          flush=True)
    ctx = F.ctx_uniform(2, B, 256, 2048)
    sg = F.SelGen(B, L, H, K, ctx, dist=1, zipf_s=zipf, reuse=0.66, seed=3)
    sg.set_reuse(_lognormal_reuse(B, K))
    tw = Twin(sg.max_blocks)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(8)
    layers = [0, 13, L - 1]
    for t in range(6):
        sel = sg.step(t)
        dsel = torch.from_numpy(np.ascontiguousarray(sel, np.uint32).view(np.int32)).cuda()
        q = torch.from_numpy(rng.standard_normal((B, L, H, 128)).astype(np.float32)).cuda()
        outs = {}
        for steal, (e, bufs) in tw.ex.items():
            outs[steal] = torch.empty_like(q)
            e.decode_step(dsel, q, bufs, outs[steal], chunks=0, side_stream=side)
        torch.cuda.synchronize()
        oslots, omc, oms, _ = tw.ox.step(sel)
        oms4 = oms.view(np.uint32).reshape(tw.ox.n_sets, -1, 4)
        live = np.arange(oms4.shape[1])[None, :] < omc[:, None]
        for steal, (e, bufs) in tw.ex.items():
            st = e.stats()
            assert st["device_error"] == 0, (steal, st)
            assert np.array_equal(_u32(bufs["slots"]).reshape(-1), oslots), (t, steal)
            assert np.array_equal(_u32(bufs["miss_count"]), omc), (t, steal)
            gms = _u32(bufs["misses"]).reshape(tw.ox.n_sets, -1, 4)
            assert np.array_equal(gms[live], oms4[live]), (t, steal)
        # same pool bytes, same kernel: the outputs are bit-identical
        assert torch.equal(outs[0], outs[1]), t
        if t in (0, 5):
            ref = _attention_layers_f64(tw.g, sel.reshape(B, L, H, K), q.cpu().numpy(), layers)
            got = outs[1].cpu().numpy()[:, layers].reshape(-1, 128).astype(np.float64)
            ref = ref.reshape(-1, 128)
            rel = np.abs(got - ref).max(axis=1) / np.abs(ref).max(axis=1)
            assert rel.max() < 2e-3, (t, rel.max())
        print(f"[skew pipelined] zipf={zipf} step {t}: {int(omc.sum())} misses", flush=True)
    tw.check_state()
    s0, s1 = tw.ex[0][0].stats(), tw.ex[1][0].stats()
    assert s0["steals"] == 0 and s1["steals"] > 0
    assert s0["misses"] == s1["misses"] > 0
    print(f"[skew pipelined] zipf={zipf}: {s1['misses']} misses, {s1['steals']} steals moved "
          f"{s1['stolen']}", flush=True)


def test_skew_full_batch_pipelined_owner_replay():
    # the whole config-3 batch (64 requests) at Zipf 1.4 with stealing, through
    # the pipelined step from the cold pool: the first two requests replayed in
    # the oracle every step (slots and miss lists bit-equal; LRU state, fetched
    # and resident bytes and attention at the end), and for all 64 requests the
    # size-independent properties (every slot in its owner's set holding its
    # block, counters adding up)
    Bf = 64
    print(f"[skew full] B={Bf} L={L} H={H} k={K} C={CAP} workers={WORKERS} zipf=1.4", flush=True)
    ctx = F.ctx_uniform(2, Bf, 256, 2048)
    sg = F.SelGen(Bf, L, H, K, ctx, dist=1, zipf_s=1.4, reuse=0.66, seed=3)
    sg.set_reuse(_lognormal_reuse(Bf, K))
    ex = F.Executor(Bf, L, H, K, CAP, sg.max_blocks, dtype=F.F16, host_blocks=HB,
                    fetch_workers=WORKERS, steal=1, assign=F.ASSIGN_AFFINITY)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    side = torch.cuda.Stream()
    replay = OwnerReplay(n_req=Bf, group=1, n_layers=L, kv_heads=H, q_heads=H, k=K,
                         slots_per_set=CAP, max_blocks=sg.max_blocks, dtype=F.F16,
                         host_blocks=HB)
    sets = (np.arange(Bf)[:, None, None] * L + np.arange(L)[None, :, None]) * H + \
        np.arange(H)[None, None, :]
    total = 0
    for t in range(8):
        sel = sg.step(t)
        q = torch.randn((Bf, L, H, 128), device="cuda")
        out = torch.empty_like(q)
        ex.decode_step(torch.from_numpy(sel.view(np.int32)).cuda(), q, bufs, out, chunks=0,
                       side_stream=side)
        torch.cuda.synchronize()
        st = ex.stats()
        assert st["device_error"] == 0, st
        replay.step(sel, bufs)
        total += int(_u32(bufs["miss_count"]).sum())
        assert st["misses"] == total and st["fetched_bytes"] == total * ex.block_bytes
        slots = _u32(bufs["slots"]).reshape(Bf, L, H, K).astype(np.int64)
        assert np.all(slots // CAP == sets[..., None])
        _, _, tag = ex.sets_state()
        assert np.array_equal(tag.reshape(-1)[slots.reshape(-1)], sel.reshape(-1))
        print(f"[skew full] step {t}: {total} misses so far, {st['steals']} steals", flush=True)
    assert ex.stats()["steals"] > 0
    res = replay.final(ex, q, out)
    print(f"[skew full] owner replay: {res}", flush=True)
    assert res["steps"] == 8 and res["misses_compared"] > 0
