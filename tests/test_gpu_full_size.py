"""The benchmark configurations at their full sizes, run through the pipelined
decode step exactly as the benchmark runs them:
  * 7B MHA: 64 requests x 32 layers x 32 kv heads, top-k 64 of 256-2048-block
    contexts, 320 slots per set (a 172 GB pool), fp16;
  * long-context GQA: 16 requests x 32 layers x 8 kv heads of 4 query heads,
    top-k 128 of 8192-block contexts, 128 slots per set, bf16;
  * shared-prefix groups: 8 groups of 16 requests x 32 layers x 8 kv heads of 4
    query heads, a 512-block shared prefix + 32-256 private blocks, top-k 64,
    1536 slots per group set, fp8 E4M3 with per-block K and V scales;
all with Zipf 1.1 popularity, reuse 0.66 and a 1 M-block host tier.  Sets
belong to one owner and draws are keyed per request, so the first owners (two
requests, or one prefix group of 16) evolve exactly as a batch of only them
would: the oracle replays those owners from the same cold start, and every
step their slots and per-set miss lists (block, slot, evicted block) must be
bit-equal; after the last step their LRU state too, the blocks fetched in it
and every resident slot of the first and last layer memcmp-equal to the host
tier, and their attention in three layers within 2e-3 (fp8: 1e-2) of the
float64 oracle (oracle/gate.py).  For the whole batch, whose replay does not
fit a test, the checks are the size-independent properties every step must
keep, plus spot checks of fetched bytes and attention against the host tier:
  * every selection's slot lies in its owner's set and holds its block;
  * each set's LRU order is a permutation of its resident slots;
  * the per-step miss counts add up to the executor's counters, and the
    fetched bytes are misses x block bytes;
  * sampled missed blocks (and fp8 scales) equal the host tier's;
  * sampled rows' attention equals a float64 softmax over the selected blocks'
    keys and values decoded from the host tier (tolerance 2e-3 of the row's
    largest output; 1e-2 for fp8)."""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O
from oracle.gate import OwnerReplay

pytestmark = pytest.mark.gpu

HB = 1 << 20
CONFIGS = {
    "7b": dict(B=64, L=32, Hkv=32, Hq=32, k=64, C=320, lo=256, hi=2048, dtype=F.F16, group=1,
               prefix=0),
    "gqa128k": dict(B=16, L=32, Hkv=8, Hq=32, k=128, C=128, lo=8192, hi=8192, dtype=F.BF16,
                    group=1, prefix=0),
    "prefix_fp8": dict(B=128, L=32, Hkv=8, Hq=32, k=64, C=1536, lo=32, hi=256, dtype=F.FP8,
                       group=16, prefix=512),
}


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


_E4M3 = None


def _decode(dtype, raw):
    """Block bytes [n, bb] -> float64 [n, 2, 16, 128] (K, V), exact."""
    global _E4M3
    n = raw.shape[0]
    if dtype == F.F16:
        return raw.view(np.float16).reshape(n, 2, 16, 128).astype(np.float64)
    if dtype == F.BF16:
        u = raw.view(np.uint16).astype(np.uint32) << 16
        return u.view(np.float32).reshape(n, 2, 16, 128).astype(np.float64)
    if _E4M3 is None:
        _E4M3 = np.array([O.lib.ora_e4m3_to_f32(c) for c in range(256)], np.float64)
    return _E4M3[raw].reshape(n, 2, 16, 128)


@pytest.mark.parametrize("name", list(CONFIGS))
def test_benchmark_shapes_at_full_size(name):
    c = CONFIGS[name]
    B, L, Hkv, Hq, k, C, dtype = c["B"], c["L"], c["Hkv"], c["Hq"], c["k"], c["C"], c["dtype"]
    G = Hq // Hkv
    ctx = F.ctx_uniform(2, B, c["lo"], c["hi"]) + c["prefix"]
    sg = F.SelGen(B, L, Hkv, k, ctx, dist=1, zipf_s=1.1, reuse=0.66, group=c["group"],
                  prefix_blocks=c["prefix"], seed=3)
    mb = sg.max_blocks
    ex = F.Executor(B, L, Hkv, k, C, mb, q_heads=Hq, group=c["group"], dtype=dtype,
                    host_blocks=HB)
    ex.hosttier_fill()
    host, hsc = ex.hosttier_array()
    hostb = host.reshape(HB, ex.block_bytes)
    scales = None if hsc is None else hsc.reshape(HB, 2)
    bufs = ex.alloc_step_buffers()
    side = torch.cuda.Stream()
    rng = np.random.default_rng(9)
    owner = np.arange(B) // c["group"]
    sets = ((owner[:, None, None] * L + np.arange(L)[None, :, None]) * Hkv +
            np.arange(Hkv)[None, None, :])
    total_misses = 0
    tol = 1e-2 if dtype == F.FP8 else 2e-3
    replay = OwnerReplay(n_req=B, group=c["group"], n_layers=L, kv_heads=Hkv, q_heads=Hq, k=k,
                         slots_per_set=C, max_blocks=mb, dtype=dtype, host_blocks=HB)
    for t in range(6):
        sel = sg.step(t)
        q = torch.randn((B, L, Hq, 128), device="cuda")
        out = torch.empty_like(q)
        ex.decode_step(torch.from_numpy(sel.view(np.int32)).cuda(), q, bufs, out, chunks=0,
                       side_stream=side)
        torch.cuda.synchronize()
        st = ex.stats()
        assert st["device_error"] == 0, st
        replay.step(sel, bufs)  # the first owners, bit-exact against the oracle
        mc = _u32(bufs["miss_count"])
        total_misses += int(mc.sum())
        assert st["misses"] == total_misses
        assert st["fetched_bytes"] == total_misses * ex.block_bytes
        if t not in (0, 3, 5):
            continue
        print(f"[full size] {name} step {t}: {int(mc.sum())} misses", flush=True)
        slots = _u32(bufs["slots"]).reshape(B, L, Hkv, k).astype(np.int64)
        sel4 = sel.reshape(B, L, Hkv, k)
        assert np.all(slots // C == sets[..., None])
        fill, ord_, tag = ex.sets_state()
        assert np.array_equal(tag.reshape(-1)[slots.reshape(-1)], sel.reshape(-1))
        for s in rng.choice(ex.n_sets, 256, replace=False):
            assert np.array_equal(np.sort(ord_[s, :fill[s]]), np.arange(fill[s]))
        # missed blocks of this step (and their fp8 scales) against the host tier
        gm = _u32(bufs["misses"]).reshape(ex.n_sets, ex.max_sel, 4)
        owners = np.nonzero(mc)[0]
        pick = rng.choice(owners, min(256, owners.size), replace=False)
        m = np.concatenate([gm[s, :mc[s]] for s in pick])[:2048]
        pslots = m[:, 3].astype(np.int64) * C + m[:, 1]
        hidx = (m[:, 3].astype(np.int64) * mb + m[:, 0]) % HB
        assert np.array_equal(ex.pool_slots_bytes(pslots), hostb[hidx])
        if scales is not None:
            assert np.array_equal(ex.pool_slot_scales(pslots), scales[hidx])
        # attention of sampled rows against a float64 softmax over the host tier
        qn, on = q.cpu().numpy(), out.cpu().numpy()
        for _ in range(6):
            r, l, h = int(rng.integers(B)), int(rng.integers(L)), int(rng.integers(Hkv))
            hid = (sets[r, l, h] * mb + sel4[r, l, h].astype(np.int64)) % HB
            kv = _decode(dtype, hostb[hid])
            if scales is not None:
                kv = kv * scales[hid].astype(np.float64)[:, :, None, None]
            keys, vals = kv[:, 0].reshape(-1, 128), kv[:, 1].reshape(-1, 128)
            for gq in range(G):
                x = keys @ qn[r, l, h * G + gq].astype(np.float64) / np.sqrt(128.0)
                p = np.exp(x - x.max())
                ref = (p / p.sum()) @ vals
                err = np.abs(on[r, l, h * G + gq] - ref).max() / np.abs(ref).max()
                assert err < tol, (name, t, r, l, h, gq, err)
    # after a few steps a minority of the step's selections miss
    assert 0.005 < int(mc.sum()) / (B * L * Hkv * k) < 0.6
    res = replay.final(ex, q, out)
    print(f"[full size] {name} owner replay: {res}", flush=True)
    assert res["steps"] == 6 and res["misses_compared"] > 0
