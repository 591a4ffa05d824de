"""ferry_select_mass_noalloc, the entry point that allocates nothing: the mass
selection with its workspace (per-workgroup (max, sum) slices and, for 16-bit
and fp8 K, the per-kv-head block masses) in the library's static per-GPU array
instead of the context's, through the C-ABI.  Its page lists must equal
ferry_select_mass's bit for bit (same kernels, same arithmetic per (request,
layer, kv head) unit and (request, layer) item, only fewer workgroups sharing
the work and, where the masses of every layer do not fit, layer ranges run one
after the other) on two calls
in a row, the second with smaller inputs, which finds the first call's data
still in the shared array, and on a second, smaller executor on the same
GPU.  It is collected last: it must pass alone in a fresh process and after
every other test."""
import numpy as np
import pytest
import torch

import ferry_amd as F

pytestmark = pytest.mark.gpu


def _exec(B, L, Hkv, Hq, k, max_blocks, dtype):
    ex = F.Executor(B, L, Hkv, k, 8, max_blocks, q_heads=Hq, dtype=dtype, host_blocks=4099)
    ex.hosttier_fill()
    ex.ktiles_build()
    return ex


def _both(ex, q, ctx, shape):
    a = torch.full(shape, -7, dtype=torch.int32, device="cuda")
    b = torch.full(shape, -9, dtype=torch.int32, device="cuda")
    dq, dctx = torch.from_numpy(q).cuda(), torch.from_numpy(ctx).cuda()
    ex.select_mass(dq, dctx, a)
    ex.select_mass_noalloc(dq, dctx, b)
    torch.cuda.synchronize()
    assert ex.stats()["device_error"] == 0
    return a.cpu().numpy(), b.cpu().numpy()


@pytest.mark.parametrize("dtype,Hkv,Hq,ws", [(F.BF16, 4, 16, ""), (F.F16, 2, 4, ""), (F.FP8, 2, 8, ""),
                                             (F.BF16, 2, 8, "hbm"), (F.F32, 2, 4, "")])
def test_noalloc_select_mass_equals_select_mass(dtype, Hkv, Hq, ws, monkeypatch):
    # 16-bit K keeps the blocks' log-sums in LDS (or, with FERRY_MASS_WS=hbm,
    # their max and sum in workspace slices, as fp8 K does); fp32 K runs the
    # one-launch kernel with slices.  The context reads the variable when it
    # first plans a mass selection.
    if ws:
        monkeypatch.setenv("FERRY_MASS_WS", ws)
    else:
        monkeypatch.delenv("FERRY_MASS_WS", raising=False)
    B, L, k, mb = 6, 3, 32, 2000
    print(f"[noalloc] dtype={dtype} B={B} L={L} Hkv={Hkv} Hq={Hq} k={k} max_blocks={mb} ws={ws or 'default'}",
          flush=True)
    ex = _exec(B, L, Hkv, Hq, k, mb, dtype)
    rng = np.random.default_rng(dtype)
    shape = (B, L, Hkv, k)
    # first call: long contexts (up to max_blocks)
    q = rng.standard_normal((B, L, Hq, 128)).astype(np.float32)
    ctx = rng.integers(k + 1, mb + 1, B).astype(np.int32)
    ctx[0] = mb
    a, b = _both(ex, q, ctx, shape)
    assert np.array_equal(a, b)
    assert np.all((a[..., : k] >= 0))
    # second call, smaller: shorter contexts, one at or below k, one empty
    q2 = rng.standard_normal((B, L, Hq, 128)).astype(np.float32)
    ctx2 = rng.integers(k + 1, 300, B).astype(np.int32)
    ctx2[1], ctx2[2] = k - 5, 0
    a2, b2 = _both(ex, q2, ctx2, shape)
    assert np.array_equal(a2, b2)
    ex.close()
    # a second, smaller executor on the same GPU shares the static array
    ex2 = _exec(2, 2, Hkv, Hq, 16, 500, dtype)
    q3 = rng.standard_normal((2, 2, Hq, 128)).astype(np.float32)
    ctx3 = np.array([500, 100], np.int32)
    a3, b3 = _both(ex2, q3, ctx3, (2, 2, Hkv, 16))
    assert np.array_equal(a3, b3)
    ex2.close()


def test_noalloc_select_mass_layer_ranges():
    # the per-kv-head masses of all 12 layers (16 x 12 x 8 x 15360 floats, 94 MB)
    # exceed the 64 MiB array: the call runs layer ranges one after the other
    B, L, Hkv, Hq, k, mb = 16, 12, 8, 16, 32, 15360
    print(f"[noalloc] layer ranges: bf16 B={B} L={L} Hkv={Hkv} Hq={Hq} k={k} max_blocks={mb}",
          flush=True)
    assert B * L * Hkv * mb * 4 > 64 << 20 and B * Hkv * mb * 4 < 64 << 20
    ex = _exec(B, L, Hkv, Hq, k, mb, F.BF16)
    rng = np.random.default_rng(11)
    q = rng.standard_normal((B, L, Hq, 128)).astype(np.float32)
    ctx = rng.integers(k + 1, 1500, B).astype(np.int32)
    ctx[0], ctx[1] = mb, k - 3
    a, b = _both(ex, q, ctx, (B, L, Hkv, k))
    assert np.array_equal(a, b)
    assert np.all(a[2:, ..., :k] >= 0) and np.all(a[1, ..., k - 3:] == -1)
    ex.close()


def test_noalloc_select_mass_refusals():
    ex = F.Executor(2, 2, 2, 8, 8, 300, q_heads=4, dtype=F.BF16, host_blocks=4099)
    q = torch.zeros((2, 2, 4, 128), device="cuda")
    ctx = torch.tensor([100, 100], dtype=torch.int32, device="cuda")
    sel = torch.empty((2, 2, 2, 8), dtype=torch.int32, device="cuda")
    with pytest.raises(F.FerryError, match="K table not built"):
        ex.select_mass_noalloc(q, ctx, sel)
    ex.close()
