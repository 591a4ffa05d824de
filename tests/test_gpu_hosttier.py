"""A caller-owned pinned host tier (ferry_hosttier_register): the executor
fetches from the registered memory, bit-exact against the oracle while it
holds the oracle's content, and from whatever the caller writes there after;
pageable memory and short buffers are refused."""
import numpy as np
import pytest
import torch

import ferry_amd as F

from test_gpu_parity import Pair, _zipf_stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [F.F16, F.FP8])
def test_registered_tier_is_the_fetch_source(dtype):
    n_req, L, Hkv, Hq, k, cap = 3, 2, 2, 4, 12, 30
    mb, sels = _zipf_stream(n_req, L, Hkv, k, 40, 160, 6, seed=13)
    p = Pair(n_req, L, Hkv, Hq, k, cap, mb, dtype, host_blocks=1031)
    own, own_sc = p.host.copy(), None if p.hsc is None else p.hsc.copy()
    host = torch.empty(own.size, dtype=torch.uint8, pin_memory=True)
    host.numpy()[:] = own
    scales = None
    if dtype == F.FP8:
        scales = torch.empty(own_sc.size, dtype=torch.float32, pin_memory=True)
        scales.numpy()[:] = own_sc
    p.ex.hosttier_register(host, scales)
    view, view_sc = p.ex.hosttier_array()
    assert view.ctypes.data == host.data_ptr()
    p.host, p.hsc = host.numpy(), None if scales is None else scales.numpy()
    for t in range(3):  # same content as the oracle's generator: full parity
        p.check_fetched_bytes(p.step(sels[t]))
        p.check_state()
    p.check_attention(sels[2], seed=1)
    # new content in the caller's buffer: later fetches carry it
    rng = np.random.default_rng(4)
    host.numpy()[:] = rng.integers(0, 256, own.size, dtype=np.uint8)
    if scales is not None:
        scales.numpy()[:] = rng.uniform(0.5, 2.0, own_sc.size).astype(np.float32)
    fetched_any = False
    for t in range(3, 6):
        fetched = p.step(sels[t])
        fetched_any |= len(fetched) > 0
        p.check_fetched_bytes(fetched)
    assert fetched_any


def test_register_refusals():
    mb, sels = _zipf_stream(2, 1, 1, 8, 20, 60, 2, seed=2)
    p = Pair(2, 1, 1, 1, 8, 16, mb, F.F16, host_blocks=257)
    need = 257 * p.bb
    with pytest.raises(F.FerryError, match="smaller"):
        p.ex.hosttier_register(torch.empty(need - 1, dtype=torch.uint8, pin_memory=True))
    with pytest.raises(F.FerryError, match="pinned"):
        p.ex.hosttier_register(torch.empty(need, dtype=torch.uint8))  # pageable
    with pytest.raises(F.FerryError, match="fp8"):
        p.ex.hosttier_register(torch.empty(need, dtype=torch.uint8, pin_memory=True),
                               torch.empty(2 * 257, dtype=torch.float32, pin_memory=True))
    # the executor still works on its own tier afterwards
    for sel in sels:
        p.check_fetched_bytes(p.step(sel))
    assert p.ex.stats()["device_error"] == 0
