"""GPU parity over seeded random geometries: dtype, kv heads and head-group
size, prefix groups, LRU granularity, attention kernel, top-k, slots per set
and ragged or short contexts drawn together, so that combinations the
hand-picked cases do not meet are checked against the oracle too."""
import numpy as np
import pytest

import ferry_amd as F

from test_gpu_parity import Pair, _zipf_stream

pytestmark = pytest.mark.gpu


def _geometry(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = int(rng.choice([F.F32, F.F16, F.BF16, F.FP8]))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 1, 2, 4]))
    n_req = group * int(rng.integers(1, 4))
    L = int(rng.integers(1, 4))
    k = int(rng.integers(1, 49))
    lru = int(rng.choice([F.LRU_STEP, F.LRU_STEP, F.LRU_SERIAL]))
    attn = F.ATTN_AUTO if rng.random() < 0.7 else F.ATTN_VALU
    cap = group * k + int(rng.integers(0, 2 * k + 1))
    lo = int(rng.integers(1, 3 * k + 2))  # some contexts shorter than k: ragged rows
    hi = lo + int(rng.integers(0, 200))
    prefix = int(rng.integers(0, 40)) if group > 1 else 0
    return dict(dtype=dtype, Hkv=Hkv, G=G, group=group, n_req=n_req, L=L, k=k, lru=lru,
                attn=attn, cap=cap, lo=lo, hi=hi, prefix=prefix)


@pytest.mark.parametrize("seed", range(32))
def test_random_geometry_parity(seed):
    c = _geometry(seed)
    print("[geometry]", c, flush=True)
    mb, sels = _zipf_stream(c["n_req"], c["L"], c["Hkv"], c["k"], c["lo"], c["hi"], 4,
                            seed=seed + 5, group=c["group"], prefix=c["prefix"],
                            reuse=0.5)
    p = Pair(c["n_req"], c["L"], c["Hkv"], c["Hkv"] * c["G"], c["k"], c["cap"], mb, c["dtype"],
             group=c["group"], lru=c["lru"], attn=c["attn"], host_blocks=1031)
    for sel in sels:
        p.check_fetched_bytes(p.step(sel))
        p.check_state()
    p.check_attention(sels[-1], seed=seed)


@pytest.mark.parametrize("seed", range(16, 32))
def test_random_geometry_pipelined_step(seed):
    """The same draws through ferry_decode_step with a side stream: layer ranges
    booked one range ahead into alternating rings, fetched on the side stream,
    attended on the main stream.  Slots, miss counts, state and attention must
    match the oracle stepping the whole batch at once."""
    import torch

    from oracle import pyoracle as O
    from test_gpu_parity import TOL, _u32

    c = _geometry(seed)
    chunks = int(np.random.default_rng(seed).choice([0, 1, 2, 3, c["L"]]))
    print("[geometry]", c, "chunks", chunks, flush=True)
    mb, sels = _zipf_stream(c["n_req"], c["L"], c["Hkv"], c["k"], c["lo"], c["hi"], 4,
                            seed=seed + 5, group=c["group"], prefix=c["prefix"],
                            reuse=0.5)
    Hq = c["Hkv"] * c["G"]
    p = Pair(c["n_req"], c["L"], c["Hkv"], Hq, c["k"], c["cap"], mb, c["dtype"],
             group=c["group"], lru=c["lru"], attn=c["attn"], host_blocks=1031)
    side = torch.cuda.Stream()
    rng = np.random.default_rng(seed)
    for t, sel in enumerate(sels):
        q = rng.standard_normal((c["n_req"], c["L"], Hq, 128)).astype(np.float32)
        dq = torch.from_numpy(q).cuda()
        out = torch.empty_like(dq)
        dsel = torch.from_numpy(np.ascontiguousarray(sel, np.uint32).view(np.int32)).cuda()
        p.ex.decode_step(dsel, dq, p.bufs, out, chunks=chunks, side_stream=side)
        torch.cuda.synchronize()
        assert p.ex.stats()["device_error"] == 0
        oslots, omc, _, _ = p.ox.step(sel)
        assert np.array_equal(_u32(p.bufs["slots"]).reshape(-1), oslots)
        assert np.array_equal(_u32(p.bufs["miss_count"]), omc)
        p.check_state()
        got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
        ref = O.attention_f64(p.g, sel, q).reshape(-1, 128)
        live = np.abs(ref).max(axis=1) > 0
        rel = np.abs(got - ref).max(axis=1)[live] / np.abs(ref).max(axis=1)[live]
        assert np.all(got[~live] == 0) and (rel.size == 0 or rel.max() < TOL[c["dtype"]]), t
