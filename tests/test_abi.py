"""The C-ABI library without a GPU: it loads, exports every symbol the header
declares, and its host-side code (workload generators, config validation)
agrees with the oracle.  No device compute here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import ferry_amd as F
from oracle import pyoracle as O

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "ferry_amd.h")


def header_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ferry_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert len(names) >= 25
    lib = C.CDLL(F.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_strings():
    assert b"gfx950" in F.lib.ferry_version()
    assert isinstance(F.lib.ferry_last_error(), bytes)


@pytest.mark.parametrize("kw", [
    dict(dist=1, zipf_s=1.1, reuse=0.66, group=1, prefix_blocks=0, n_req=6, L=3, H=4, k=32),
    dict(dist=0, zipf_s=0.0, reuse=0.0, group=1, prefix_blocks=0, n_req=3, L=2, H=8, k=16),
    dict(dist=1, zipf_s=1.4, reuse=0.5, group=4, prefix_blocks=64, n_req=10, L=2, H=2, k=24),
])
def test_selgen_matches_oracle(kw):
    ctx = F.ctx_uniform(11, kw["n_req"], 70, 300)
    assert np.array_equal(ctx, O.ctx_uniform(11, kw["n_req"], 70, 300))
    mine = F.SelGen(kw["n_req"], kw["L"], kw["H"], kw["k"], ctx, dist=kw["dist"],
                    zipf_s=kw["zipf_s"], reuse=kw["reuse"], group=kw["group"],
                    prefix_blocks=kw["prefix_blocks"], seed=5)
    ref = O.selgen(kw["n_req"], kw["L"], kw["H"], kw["k"], ctx, dist=kw["dist"],
                   zipf_s=kw["zipf_s"], reuse=kw["reuse"], group=kw["group"],
                   prefix_blocks=kw["prefix_blocks"], seed=5)
    assert mine.max_blocks == O.selgen_max_blocks(ref)
    for step in range(5):
        assert np.array_equal(mine.step(step).reshape(-1), O.selgen_step(ref, step))


def test_refgen_matches_reference_replay():
    R, L, S, sel = 48, 12, 16, 64
    mine = F.refgen_selections(R, L, S, sel, 42)
    blocks, _, _, _ = O.ref_replay(R, L, S, sel, 128, 42)
    assert np.array_equal(mine.reshape(-1).astype(np.uint64), blocks)


@pytest.mark.parametrize("bad", [
    dict(q_heads=3), dict(head_dim=64), dict(block_tokens=8), dict(dtype=7), dict(lru_mode=3),
    dict(k=0), dict(slots_per_set=0), dict(assign=5), dict(max_blocks=0), dict(attn=3),
    dict(attn=2),  # MFMA kernel needs a GQA group (q_heads/kv_heads >= 2) for 16-bit KV
    dict(attn=3, dtype=3),  # the group kernel needs a GQA group even for fp8
    dict(attn=2, q_heads=4, dtype=0),  # ... and 16/8-bit KV
    dict(cap_mode=2),
    dict(cap_mode=1, group=2, slots_per_set=7),  # per-member shares must divide the slots
])
def test_invalid_config_rejected_before_any_device_call(bad):
    base = dict(n_req=2, group=1, n_layers=1, kv_heads=2, q_heads=2, head_dim=128,
                block_tokens=16, k=4, slots_per_set=8, max_blocks=16, dtype=F.F16, lru_mode=0,
                host_blocks=64, host_seed=1, value_std=0.5, fetch_workers=0, steal=1, assign=0,
                attn=0, cap_mode=0)
    base.update(bad)
    cfg = F.Config(*[base[f] for f, _ in F.Config._fields_])
    h = C.c_void_p()
    assert F.lib.ferry_ctx_create(C.byref(cfg), 0, C.byref(h)) == -1
    assert not h.value
    assert F.lib.ferry_last_error()


def test_selgen_per_request_reuse_matches_oracle():
    B, L, H, k = 5, 2, 3, 16
    ctx = F.ctx_uniform(4, B, 40, 200)
    rr = np.array([0.0, 0.25, 0.66, 0.9, 1.0])
    mine = F.SelGen(B, L, H, k, ctx, reuse=0.5, seed=8)
    mine.set_reuse(rr)
    ref = O.selgen(B, L, H, k, ctx, reuse=0.5, seed=8, reuse_r=rr)
    prev = None
    for step in range(6):
        a = mine.step(step)
        assert np.array_equal(a.reshape(-1), O.selgen_step(ref, step))
        if prev is not None:  # reuse 1.0 keeps the whole selection, 0.0 redraws all of it
            assert np.array_equal(a[4], prev[4])
        prev = a



def test_host_buffers_are_refused_before_the_call():
    """The Python mirror refuses buffers that are not CUDA tensors before any
    pointer reaches the library (the device-side refusals are GPU tests)."""
    import torch
    with pytest.raises(ValueError, match="CUDA tensor"):
        F._dev(torch.zeros(8, dtype=torch.int32), "sel", 8, F._I32, 0)
    with pytest.raises(ValueError, match="CUDA tensor"):
        F._dev(np.zeros(8, np.int32), "sel", 8, F._I32, 0)
