"""fp8 KV whose per-block scales span six orders of magnitude.

A caller registers its own pinned host tier (ferry_hosttier_register) with
fp8 V scales spread log-uniformly over 1e-3..1e3 of the generator's, some V
scales 0 (an all-zero block's amax), some blocks whose V bytes are all zero
under a 1000x scale, and some K scales 0.  Every fp8 attention kernel (the
prefix-group kernel, the per-row matrix-core kernel for GQA and MHA, and the
vector-ALU kernel) must stay finite and within 1e-2 of the float64 oracle
computed over the registered bytes and scales.  The matrix-core kernels keep
their accumulator in units of a reference V scale, so these cases drive
that reference through every move it makes: set by the first nonzero scale,
moved up past 16x and down below 1/64.
"""
import numpy as np
import pytest
import torch

import ferry_amd as F
from oracle import pyoracle as O

from test_gpu_parity import TOL, Pair, _zipf_stream

pytestmark = pytest.mark.gpu

HOST_BLOCKS = 1031

# (kv heads, q heads, group, requests, attention kernel, kernel the executor reports)
CASES = [
    (2, 8, 4, 8, F.ATTN_GROUP, F.ATTN_GROUP),  # prefix groups, G 4: k_attn_group
    (2, 8, 1, 4, F.ATTN_MFMA, F.ATTN_MFMA),    # GQA-4 rows: k_attn_mfma
    (4, 4, 1, 4, F.ATTN_AUTO, F.ATTN_MFMA),    # fp8 MHA: k_attn_mfma with one live column
    (4, 4, 1, 4, F.ATTN_VALU, F.ATTN_VALU),    # fp8 MHA on the vector ALUs: k_attn
]


def _wide_tier(p, seed):
    """The generator's tier with rewritten scales and zero blocks; returns the
    pinned tensors and the per-block class (0 plain, 1 V scale 0, 2 zero V
    bytes at 1000x, 3 K scale 0)."""
    bb = p.bb
    host = torch.empty(p.host.size, dtype=torch.uint8, pin_memory=True)
    scales = torch.empty(p.hsc.size, dtype=torch.float32, pin_memory=True)
    hb = host.numpy().reshape(HOST_BLOCKS, bb)
    sc = scales.numpy().reshape(HOST_BLOCKS, 2)
    hb[:] = p.host.reshape(HOST_BLOCKS, bb)
    sc[:] = p.hsc.reshape(HOST_BLOCKS, 2)
    rng = np.random.default_rng(seed)
    sc[:, 1] *= 10.0 ** rng.uniform(-3.0, 3.0, HOST_BLOCKS)
    cls = rng.choice(4, HOST_BLOCKS, p=[0.82, 0.06, 0.06, 0.06])
    sc[cls == 1, 1] = 0.0
    hb[cls == 2, bb // 2:] = 0
    sc[cls == 2, 1] = 1e3 * p.hsc.reshape(HOST_BLOCKS, 2)[cls == 2, 1]
    sc[cls == 3, 0] = 0.0
    return host, scales, cls


def _hidx(g, sel):
    """Host-tier index of every selection ([B][L][Hkv][k], NONE64 = empty)."""
    B, L, H, k = g.n_req, g.n_layers, g.kv_heads, g.k
    s = np.ascontiguousarray(sel, np.uint32).reshape(B, L, H, k)
    own = (np.arange(B) // g.group)[:, None, None]
    sets = ((own * L + np.arange(L)[None, :, None]) * H + np.arange(H)[None, None, :])
    h = (sets[..., None].astype(np.uint64) * np.uint64(g.max_blocks) + s.astype(np.uint64))
    h %= np.uint64(g.host_blocks)
    return np.where(s == O.NONE, O.NONE64, h)


@pytest.mark.parametrize("Hkv,Hq,group,n_req,attn,kind", CASES)
def test_fp8_attention_with_wide_block_scales(Hkv, Hq, group, n_req, attn, kind):
    L, k = 2, 16
    cap = max(64, group * k + 32)
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 120, 4, group=group, prefix=24 if group > 1 else 0)
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, F.FP8, group=group, host_blocks=HOST_BLOCKS,
             attn=attn)
    assert p.ex.attn_kernel()[0] == kind
    host, scales, cls = _wide_tier(p, seed=Hq + group)
    p.ex.hosttier_register(host, scales)
    p.host, p.hsc = host.numpy(), scales.numpy()
    for sel in sels:  # every fetched block and scale comes from the registered tier
        p.check_fetched_bytes(p.step(sel))
    sel = sels[-1]
    hidx = _hidx(p.g, sel)
    # the cases this test is for occur among the attended blocks, also first in a row
    picked = cls[hidx[hidx != O.NONE64].astype(np.int64)]
    assert all((picked == c).any() for c in (1, 2, 3))
    firsts = hidx.reshape(-1, k)[:, :4].reshape(-1)
    assert (cls[firsts[firsts != O.NONE64].astype(np.int64)] != 0).any()
    rng = np.random.default_rng(5)
    q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    dq = torch.from_numpy(q).cuda()
    out = torch.empty_like(dq)
    p.ex.sparse_decode(dq, p.bufs["slots"], out)
    torch.cuda.synchronize()
    assert p.ex.stats()["device_error"] == 0
    got = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
    ref = O.attention_tier_f64(p.g, hidx, p.host, p.hsc, q).reshape(-1, 128)
    assert np.all(np.isfinite(got))
    den = np.maximum(np.abs(ref).max(axis=1), 1e-30)
    rel = np.abs(got - ref).max(axis=1) / den
    assert rel.max() < TOL[F.FP8], rel.max()
