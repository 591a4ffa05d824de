"""ferry_amd -- MI355X-native per-GPU sparse KV miss-stream executor.

Python mirror of the C-ABI in include/ferry_amd.h, loaded with ctypes.  The
compute path is libferry_amd.so (hand-written gfx950 HIP kernels); there is no
CPU fallback: importing this package without the built library raises.

torch supplies device memory and streams only.  It is imported before the
library so that one HIP runtime serves both.

Reference interfaces mirrored (clearleo126/ferry, paths relative to its tree):
  Executor.fetch_step      run_miss_workload mode C / exec_step C engine
                           (src/workloads/kv_exec.cuh:188-292,
                           src/runtime/wla_multigpu.cuh:2527-2604)
  Executor.sparse_decode   attn_kernel / wla_attn_kernel (real attention here)
  queue_selftest           bench_queue (src/benches/bench_queue.cu:62-123)
  SelGen / refgen_selections  replay_miss_stream (src/workloads/missstream.cuh:104)
  arrivals / Sched         request arrivals and the per-GPU tick loop
                           (src/runtime/wla_multigpu.cuh:497-501, 829-864,
                           2610-2665)
"""
import ctypes as C
import os

import numpy as np
import torch  # noqa: F401  (HIP runtime + device memory; load before the library)

__all__ = [
    "FerryError", "Executor", "SelGen", "Sched", "queue_selftest", "refgen_selections",
    "ctx_uniform", "arrivals", "lib", "LIB_PATH", "F32", "F16", "BF16", "FP8", "LRU_STEP",
    "LRU_SERIAL", "ASSIGN_SPREAD", "ASSIGN_AFFINITY", "ATTN_AUTO", "ATTN_VALU", "ATTN_MFMA",
    "ATTN_GROUP", "MISS_DTYPE", "EMPTY", "ARRIVAL_STEADY", "ARRIVAL_BURSTY", "ARRIVAL_POISSON", "ARRIVAL_MMPP",
    "SCHED_FIFO", "SCHED_PINNED", "trace_load", "TOPK_PER_HEAD", "TOPK_LAYER_MAX", "CAP_GROUP",
    "CAP_PER_MEMBER",
]

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libferry_amd.so")
if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built: run `make -C ferry_amd` "
                      "(or __graft_entry__.build()); there is no fallback path")
lib = C.CDLL(LIB_PATH)

F32, F16, BF16, FP8 = 0, 1, 2, 3
LRU_STEP, LRU_SERIAL = 0, 1
ASSIGN_SPREAD, ASSIGN_AFFINITY = 0, 1
ATTN_AUTO, ATTN_VALU, ATTN_MFMA, ATTN_GROUP = 0, 1, 2, 3
CAP_GROUP, CAP_PER_MEMBER = 0, 1
PROBE_HBM_GATHER, PROBE_HOST_READ, PROBE_HOST_DMA, PROBE_HBM_COPY, PROBE_KTAB_READ = 0, 1, 2, 3, 4
PROBE_SUMS_READ = 5
ARRIVAL_STEADY, ARRIVAL_BURSTY, ARRIVAL_POISSON, ARRIVAL_MMPP = 0, 1, 2, 3
EMPTY = 0xFFFFFFFF  # selection id of an empty position (and its slot)
SCHED_FIFO, SCHED_PINNED = 0, 1
TOPK_PER_HEAD, TOPK_LAYER_MAX = 0, 1
ESIZE = {F32: 4, F16: 2, BF16: 2, FP8: 1}
MISS_DTYPE = np.dtype([("block", "<u4"), ("slot", "<u4"), ("evicted", "<u4"), ("set", "<u4")])

_ERRORS = {-1: "EINVAL", -2: "EHIP", -3: "ERANGE", -4: "ECAPACITY", -5: "ENOMEM",
           -6: "ESPIN", -7: "ESTATE"}


class FerryError(RuntimeError):
    def __init__(self, code, where):
        self.code = code
        msg = lib.ferry_last_error().decode()
        super().__init__(f"{where}: {_ERRORS.get(code, code)} ({code}) {msg}")


class Config(C.Structure):
    _fields_ = [
        ("n_req", C.c_int32), ("group", C.c_int32), ("n_layers", C.c_int32),
        ("kv_heads", C.c_int32), ("q_heads", C.c_int32), ("head_dim", C.c_int32),
        ("block_tokens", C.c_int32), ("k", C.c_int32), ("slots_per_set", C.c_int32),
        ("max_blocks", C.c_int32), ("dtype", C.c_int32), ("lru_mode", C.c_int32),
        ("host_blocks", C.c_uint64), ("host_seed", C.c_uint64), ("value_std", C.c_float),
        ("fetch_workers", C.c_int32), ("steal", C.c_int32), ("assign", C.c_int32),
        ("attn", C.c_int32), ("cap_mode", C.c_int32),
    ]


class Stats(C.Structure):
    _fields_ = [
        ("steps", C.c_uint64), ("selections", C.c_uint64), ("misses", C.c_uint64),
        ("fetched_bytes", C.c_uint64), ("steals", C.c_uint64), ("stolen", C.c_uint64),
        ("last_misses", C.c_uint64), ("device_error", C.c_int32), ("pad", C.c_int32),
    ]


class SelGenConfig(C.Structure):
    _fields_ = [
        ("n_req", C.c_int32), ("group", C.c_int32), ("n_layers", C.c_int32),
        ("kv_heads", C.c_int32), ("k", C.c_int32), ("dist", C.c_int32),
        ("zipf_s", C.c_double), ("reuse", C.c_double), ("prefix_blocks", C.c_int32),
        ("pad", C.c_int32), ("seed", C.c_uint64),
    ]


class TraceInfo(C.Structure):
    _fields_ = [
        ("requests", C.c_uint32), ("steps", C.c_uint32), ("layers", C.c_uint32),
        ("page_tokens", C.c_uint32), ("block_tokens", C.c_uint32), ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("sel_pages", C.c_uint32), ("sel_blocks", C.c_uint32),
        ("short_records", C.c_uint32), ("unique_blocks", C.c_uint64),
        ("max_blocks_per_req", C.c_uint64),
    ]


_vp = C.c_void_p
_i32 = C.c_int32
_PROTOS = {
    "ferry_last_error": (C.c_char_p, []),
    "ferry_version": (C.c_char_p, []),
    "ferry_ctx_create": (C.c_int, [C.POINTER(Config), C.c_int, C.POINTER(_vp)]),
    "ferry_ctx_destroy": (C.c_int, [_vp]),
    "ferry_ctx_config": (C.c_int, [_vp, C.POINTER(Config)]),
    "ferry_ctx_sizes": (C.c_int, [_vp, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                  C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "ferry_hosttier_fill": (C.c_int, [_vp, _vp]),
    "ferry_hosttier_view": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp)]),
    "ferry_hosttier_register": (C.c_int, [_vp, _vp, C.c_uint64, _vp, C.c_uint64]),
    "ferry_pool_view": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp)]),
    "ferry_sets_reset": (C.c_int, [_vp, _vp]),
    "ferry_sets_state": (C.c_int, [_vp, _vp, _vp, _vp]),
    "ferry_sets_reset_owners": (C.c_int, [_vp, _vp, C.c_uint32, _vp]),
    "ferry_members_leave": (C.c_int, [_vp, _vp, C.c_uint32, _vp]),
    "ferry_members_join": (C.c_int, [_vp, _vp, C.c_uint32, _vp]),
    "ferry_members_get": (C.c_int, [_vp, _vp]),
    "ferry_selgen_admit": (C.c_int, [_vp, _i32, _i32, _i32, _i32]),
    "ferry_selgen_retire": (C.c_int, [_vp, _i32]),
    "ferry_arrivals": (C.c_int, [C.c_int, C.c_uint32, C.c_double, C.c_double, C.c_double,
                                 C.c_uint64, _vp]),
    "ferry_sched_create": (C.c_int, [_i32, _i32, C.c_uint32, _vp, _vp, C.POINTER(_vp)]),
    "ferry_trace_load": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(TraceInfo), _vp, C.c_uint64]),
    "ferry_summaries_build": (C.c_int, [_vp, C.c_uint64, _vp]),
    "ferry_set_batch_policy": (C.c_int, [_vp, C.c_double, C.c_double, C.c_double]),
    "ferry_owner_image_bytes": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "ferry_owner_export": (C.c_int, [_vp, C.c_uint32, _vp, C.c_uint64, _vp]),
    "ferry_owner_import": (C.c_int, [_vp, C.c_uint32, _vp, C.c_uint64, _vp]),
    "ferry_owner_export_member": (C.c_int, [_vp, C.c_uint32, _vp, C.c_uint64, _vp]),
    "ferry_owner_import_member": (C.c_int, [_vp, C.c_uint32, _vp, C.c_uint64, _vp]),
    "ferry_sets_own": (C.c_int, [_vp, _vp]),
    "ferry_decode_chunks": (C.c_int, [_vp, C.c_uint64, C.POINTER(_i32)]),
    "ferry_attn_kernel": (C.c_int, [_vp, C.POINTER(_i32), C.POINTER(_i32)]),
    "ferry_summaries_view": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(C.c_uint64)]),
    "ferry_select_topk": (C.c_int, [_vp, _vp, _vp, C.c_int, _vp, _vp]),
    "ferry_select_topk_layers": (C.c_int, [_vp, _i32, _i32, _vp, _vp, C.c_int, _vp, _vp]),
    "ferry_ktiles_build": (C.c_int, [_vp, C.c_uint64, _vp]),
    "ferry_ktiles_view": (C.c_int, [_vp, C.POINTER(_vp), C.POINTER(_vp), C.POINTER(C.c_uint64)]),
    "ferry_select_mass": (C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "ferry_select_mass_layers": (C.c_int, [_vp, _i32, _i32, _vp, _vp, _vp, _vp]),
    "ferry_select_mass_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "ferry_sched_destroy": (C.c_int, [_vp]),
    "ferry_sched_tick": (C.c_int, [_vp, C.c_double, _vp, _vp, _vp, C.POINTER(_i32), _vp,
                                   C.POINTER(_i32), C.POINTER(_i32), C.POINTER(_i32)]),
    "ferry_sched_next_arrival": (C.c_int, [_vp, C.POINTER(C.c_double)]),
    "ferry_sched_request_ticks": (C.c_int, [_vp, _vp, _vp]),
    "ferry_fetch_step": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ferry_bookkeep_step": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ferry_bookkeep_layers": (C.c_int, [_vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ferry_sparse_decode_layers": (C.c_int, [_vp, _i32, _i32, _vp, _vp, _vp, _vp]),
    "ferry_decode_step": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp]),
    "ferry_selgen_set_reuse": (C.c_int, [_vp, _vp]),
    "ferry_missq_push": (C.c_int, [_vp, _vp, C.c_uint32, _vp]),
    "ferry_missq_drain": (C.c_int, [_vp, _vp]),
    "ferry_sparse_decode": (C.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "ferry_stats_get": (C.c_int, [_vp, C.POINTER(Stats)]),
    "ferry_bw_probe": (C.c_int, [_vp, C.c_int, _vp, C.c_uint64, C.c_int,
                                 C.POINTER(C.c_uint64), C.POINTER(C.c_float), _vp]),
    "ferry_stats_reset": (C.c_int, [_vp]),
    "ferry_queue_ticket_probe": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_uint64),
                                          C.POINTER(C.c_float)]),
    "ferry_queue_selftest": (C.c_int, [C.c_int, C.c_uint64, C.c_uint64, C.c_int, C.c_int,
                                       C.c_int, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                       C.POINTER(C.c_float)]),
    "ferry_selgen_create": (C.c_int, [C.POINTER(SelGenConfig), _vp, C.POINTER(_vp)]),
    "ferry_selgen_destroy": (C.c_int, [_vp]),
    "ferry_selgen_max_blocks": (C.c_int, [_vp, C.POINTER(_i32)]),
    "ferry_selgen_set_private_ranges": (C.c_int, [_vp, _i32]),
    "ferry_selgen_admit_member": (C.c_int, [_vp, _i32, _i32, _i32, _i32, _i32]),
    "ferry_selgen_step": (C.c_int, [_vp, _i32, _vp]),
    "ferry_ctx_uniform": (C.c_int, [C.c_uint64, _i32, _i32, _i32, _vp]),
    "ferry_refgen_selections": (C.c_int, [_i32, _i32, _i32, _i32, C.c_uint64, _vp]),
}
for _name, (_res, _args) in _PROTOS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _check(rc, where):
    if rc != 0:
        raise FerryError(rc, where)


def _ptr(t):
    """Device/host pointer of a tensor or ndarray (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return t.data_ptr()
    return t.ctypes.data


def _dev(t, name, numel, dtypes, device):
    """Pointer of a contiguous tensor on CUDA device `device` holding at least
    `numel` elements of one of `dtypes`: the kernels read and write exactly
    that many through the raw pointer, so anything else is refused here
    instead of reaching the device."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name}: expected a CUDA tensor, got {type(t).__name__}"
                         f"{'' if not isinstance(t, torch.Tensor) else ' on ' + str(t.device)}")
    if t.device.index != device:
        raise ValueError(f"{name}: on {t.device}, the executor is on cuda:{device}")
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: dtype {t.dtype}, expected {' or '.join(map(str, dtypes))}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name}: {t.numel()} elements, the geometry needs {numel}")
    return t.data_ptr()


_I32 = (torch.int32,)
_F32 = (torch.float32,)
_U8 = (torch.uint8,)


def _stream(stream):
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


class Executor:
    """One executor (HBM slot pool + LRU sets + miss ring + pinned host tier)."""

    def __init__(self, n_req, n_layers, kv_heads, k, slots_per_set, max_blocks,
                 q_heads=None, group=1, head_dim=128, block_tokens=16, dtype=F16,
                 lru_mode=LRU_STEP, host_blocks=1 << 16, host_seed=7, value_std=0.5,
                 fetch_workers=0, steal=1, assign=ASSIGN_SPREAD, attn=ATTN_AUTO, device=0,
                 cap_mode=CAP_GROUP):
        cfg = Config(n_req, group, n_layers, kv_heads, q_heads or kv_heads, head_dim,
                     block_tokens, k, slots_per_set, max_blocks, dtype, lru_mode,
                     host_blocks, host_seed, value_std, fetch_workers, steal, assign, attn,
                     cap_mode)
        self.device = device
        torch.cuda.set_device(device)
        h = _vp()
        _check(lib.ferry_ctx_create(C.byref(cfg), device, C.byref(h)), "ferry_ctx_create")
        self._h = h
        full = Config()
        _check(lib.ferry_ctx_config(h, C.byref(full)), "ferry_ctx_config")
        self.cfg = full
        ns, ms, bb, ps = C.c_uint32(), C.c_uint32(), C.c_uint64(), C.c_uint64()
        _check(lib.ferry_ctx_sizes(h, C.byref(ns), C.byref(ms), C.byref(bb), C.byref(ps)),
               "ferry_ctx_sizes")
        self.n_sets, self.max_sel = ns.value, ms.value
        self.block_bytes, self.pool_slots = bb.value, ps.value
        self.sel_shape = (n_req, n_layers, kv_heads, k)

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h and lib is not None:
            lib.ferry_ctx_destroy(h)

    def __del__(self):
        self.close()

    # ---- buffers --------------------------------------------------------
    # ---- argument checks (shapes the kernels index) ---------------------------
    def _sel(self, t, name="sel"):
        return _dev(t, name, int(np.prod(self.sel_shape)), _I32, self.device)

    def _q(self, t, name="q"):
        B, L = self.sel_shape[0], self.sel_shape[1]
        return _dev(t, name, B * L * self.cfg.q_heads * self.cfg.head_dim, _F32, self.device)

    def _ctx(self, t):
        return _dev(t, "ctx_blocks", self.sel_shape[0], _I32, self.device)

    def _bufs(self, bufs, flags=True):
        n = int(np.prod(self.sel_shape))
        return (_dev(bufs["slots"], "slots", n, _I32, self.device),
                _dev(bufs["miss_count"], "miss_count", self.n_sets, _I32, self.device),
                _dev(bufs["misses"], "misses", self.n_sets * self.max_sel * 4, _I32, self.device),
                _dev(bufs["miss_flag"], "miss_flag", n, _U8, self.device) if flags else None)

    def alloc_step_buffers(self):
        dev = torch.device("cuda", self.device)
        return dict(
            slots=torch.empty(self.sel_shape, dtype=torch.int32, device=dev),
            miss_count=torch.empty(self.n_sets, dtype=torch.int32, device=dev),
            misses=torch.empty((self.n_sets, self.max_sel, 4), dtype=torch.int32, device=dev),
            miss_flag=torch.empty(self.sel_shape, dtype=torch.uint8, device=dev),
        )

    # ---- path -------------------------------------------------------------
    def hosttier_fill(self, stream=None):
        _check(lib.ferry_hosttier_fill(self._h, _stream(stream)), "ferry_hosttier_fill")

    def fetch_step(self, sel, bufs, stream=None, flags=True):
        _check(lib.ferry_fetch_step(self._h, self._sel(sel), *self._bufs(bufs, flags),
                                    _stream(stream)), "ferry_fetch_step")

    def bookkeep_step(self, sel, bufs, stream=None, flags=True):
        _check(lib.ferry_bookkeep_step(self._h, self._sel(sel), *self._bufs(bufs, flags),
                                       _stream(stream)), "ferry_bookkeep_step")

    def bookkeep_layers(self, l0, nl, sel, bufs, stream=None, flags=True):
        _check(lib.ferry_bookkeep_layers(self._h, l0, nl, self._sel(sel), *self._bufs(bufs, flags),
                                         _stream(stream)), "ferry_bookkeep_layers")

    def sparse_decode_layers(self, l0, nl, q, slots, out, stream=None):
        _check(lib.ferry_sparse_decode_layers(self._h, l0, nl, self._q(q), self._sel(slots, "slots"),
                                              self._q(out, "out"), _stream(stream)),
               "ferry_sparse_decode_layers")

    def owner_image_bytes(self):
        n = C.c_uint64()
        _check(lib.ferry_owner_image_bytes(self._h, C.byref(n)), "ferry_owner_image_bytes")
        return n.value

    def alloc_owner_image(self):
        """A device buffer for one owner image (uint8 tensor)."""
        return torch.empty(self.owner_image_bytes(), dtype=torch.uint8,
                           device=torch.device("cuda", self.device))

    def owner_export(self, owner, image, stream=None):
        _check(lib.ferry_owner_export(self._h, owner, _dev(image, "image", 0, _U8, self.device),
                                      image.numel(), _stream(stream)), "ferry_owner_export")

    def owner_import(self, owner, image, stream=None):
        _check(lib.ferry_owner_import(self._h, owner, _dev(image, "image", 0, _U8, self.device),
                                      image.numel(), _stream(stream)), "ferry_owner_import")

    def owner_export_member(self, lane, image, stream=None):
        """Image of the blocks only `lane`'s member of its prefix group touched
        (kv_handoff_owned's carry, src/runtime/wla_multigpu.cuh:1996-2016)."""
        _check(lib.ferry_owner_export_member(self._h, lane,
                                             _dev(image, "image", 0, _U8, self.device),
                                             image.numel(), _stream(stream)),
               "ferry_owner_export_member")

    def owner_import_member(self, lane, image, stream=None):
        """Merge a member image into `lane`'s owner (join the lane first)."""
        _check(lib.ferry_owner_import_member(self._h, lane,
                                             _dev(image, "image", 0, _U8, self.device),
                                             image.numel(), _stream(stream)),
               "ferry_owner_import_member")

    def set_batch_policy(self, min_mb=32.0, max_mb=512.0, target_batches=8.0):
        _check(lib.ferry_set_batch_policy(self._h, min_mb, max_mb, target_batches),
               "ferry_set_batch_policy")

    def decode_chunks(self, pending_blocks):
        """Layer chunks the adaptive policy picks for a step fetching this many blocks."""
        n = _i32()
        _check(lib.ferry_decode_chunks(self._h, pending_blocks, C.byref(n)), "ferry_decode_chunks")
        return n.value

    def decode_step(self, sel, q, bufs, out, chunks=0, stream=None, side_stream=None):
        """Whole step; fetch of layer chunk c+1 (side stream) overlaps attention
        of chunk c (stream).  side_stream None runs everything on one stream.
        chunks 0 = adaptive (from the last step's fetched bytes)."""
        slots, miss_count, misses, _ = self._bufs(bufs, flags=False)
        _check(lib.ferry_decode_step(self._h, self._sel(sel), self._q(q), slots, self._q(out, "out"),
                                     miss_count, misses, chunks,
                                     _stream(stream),
                                     None if side_stream is None else _stream(side_stream)),
               "ferry_decode_step")

    def missq_push(self, misses, n, stream=None):
        _check(lib.ferry_missq_push(self._h, _dev(misses, "misses", 4 * n, _I32, self.device), n,
                                    _stream(stream)), "ferry_missq_push")

    def missq_drain(self, stream=None):
        _check(lib.ferry_missq_drain(self._h, _stream(stream)), "ferry_missq_drain")

    def attn_kernel(self):
        """(kind, waves) of the attention kernel sparse_decode runs: kind is
        ATTN_VALU, ATTN_MFMA (per request row) or ATTN_GROUP (per group set);
        waves per workgroup of that launch (the group kernel runs 8 on a launch
        of no more group sets than CUs where its LDS allows, else 4)."""
        kind, waves = _i32(), _i32()
        _check(lib.ferry_attn_kernel(self._h, C.byref(kind), C.byref(waves)), "ferry_attn_kernel")
        return kind.value, waves.value

    def sparse_decode(self, q, slots, out, stream=None):
        _check(lib.ferry_sparse_decode(self._h, self._q(q), self._sel(slots, "slots"),
                                       self._q(out, "out"), _stream(stream)), "ferry_sparse_decode")

    def summaries_build(self, n_records=0, stream=None):
        """K min/max summaries for select_topk: n_records records (a multiple of
        the host tier's blocks; 0 = one per host-tier block)."""
        _check(lib.ferry_summaries_build(self._h, n_records, _stream(stream)),
               "ferry_summaries_build")

    def summaries_array(self):
        """Device summaries copied to host: uint8 [records, 2*128*esize] and
        fp8 K scales [records] (or None)."""
        p, sc, n = _vp(), _vp(), C.c_uint64()
        _check(lib.ferry_summaries_view(self._h, C.byref(p), C.byref(sc), C.byref(n)),
               "ferry_summaries_view")
        hb = n.value
        rec = 2 * 128 * ESIZE[self.cfg.dtype]
        sums = _gather_d2h(p.value, hb * rec, [0]).reshape(hb, rec)
        scales = None
        if sc.value:
            scales = _gather_d2h(sc.value, hb * 4, [0]).view(np.float32).reshape(hb)
        return sums, scales

    def select_topk(self, q, ctx_blocks, sel, mode=TOPK_PER_HEAD, stream=None, layers=None):
        """Top-k blocks of every (request, layer, kv head) from q (device
        tensors: q [B,L,Hq,128] fp32, ctx_blocks [B] int32, sel out [B,L,Hkv,k])."""
        if layers is None:
            _check(lib.ferry_select_topk(self._h, self._q(q), self._ctx(ctx_blocks), mode,
                                         self._sel(sel), _stream(stream)), "ferry_select_topk")
        else:
            l0, nl = layers
            _check(lib.ferry_select_topk_layers(self._h, l0, nl, self._q(q), self._ctx(ctx_blocks),
                                                mode, self._sel(sel), _stream(stream)),
                   "ferry_select_topk_layers")

    def ktiles_build(self, n_records=0, stream=None):
        """Dense K table for select_mass: n_records records (a multiple of the
        host tier's blocks; 0 = one per host-tier block)."""
        _check(lib.ferry_ktiles_build(self._h, n_records, _stream(stream)), "ferry_ktiles_build")

    def ktiles_array(self):
        """The K table copied to host: uint8 [records, block_bytes / 2] (fp32
        row-major; 16-bit and fp8 lane-transposed: 16-byte word c of token row
        t at word 64 (c // 4) + 16 (c % 4) + t) and fp8 K scales [records] (or
        None)."""
        p, sc, n = _vp(), _vp(), C.c_uint64()
        _check(lib.ferry_ktiles_view(self._h, C.byref(p), C.byref(sc), C.byref(n)),
               "ferry_ktiles_view")
        rec = self.block_bytes // 2
        kt = _gather_d2h(p.value, n.value * rec, [0]).reshape(n.value, rec)
        scales = None
        if sc.value:
            scales = _gather_d2h(sc.value, n.value * 4, [0]).view(np.float32).reshape(n.value)
        return kt, scales

    def select_mass(self, q, ctx_blocks, sel, stream=None, layers=None):
        """The softmax-mass top-k of every (request, layer), written to every kv
        head's row of sel [B,L,Hkv,k] (device tensors as for select_topk)."""
        if layers is None:
            _check(lib.ferry_select_mass(self._h, self._q(q), self._ctx(ctx_blocks), self._sel(sel),
                                         _stream(stream)), "ferry_select_mass")
        else:
            l0, nl = layers
            _check(lib.ferry_select_mass_layers(self._h, l0, nl, self._q(q), self._ctx(ctx_blocks),
                                                self._sel(sel), _stream(stream)),
                   "ferry_select_mass_layers")

    def select_mass_noalloc(self, q, ctx_blocks, sel, stream=None):
        """select_mass over every layer with the library's static per-GPU
        workspace instead of the context's: allocates nothing.  Calls that
        overlap on one GPU race for that workspace."""
        _check(lib.ferry_select_mass_noalloc(self._h, self._q(q), self._ctx(ctx_blocks),
                                             self._sel(sel), _stream(stream)),
               "ferry_select_mass_noalloc")

    def sets_reset(self, stream=None):
        _check(lib.ferry_sets_reset(self._h, _stream(stream)), "ferry_sets_reset")

    def reset_owners(self, owners, stream=None):
        """Empty the sets of the owners in `owners` (int32 device tensor)."""
        _check(lib.ferry_sets_reset_owners(self._h, _dev(owners, "owners", 0, _I32, self.device),
                                           int(owners.numel()), _stream(stream)),
               "ferry_sets_reset_owners")

    # ---- inspection (synchronous) ---------------------------------------
    def members_leave(self, lanes, stream=None):
        """The requests of these lanes (int32 device tensor) leave their owners;
        under CAP_PER_MEMBER the owners' sets are trimmed to the new capacity."""
        n = int(lanes.numel())
        _check(lib.ferry_members_leave(self._h, _dev(lanes, "lanes", n, _I32, self.device), n,
                                       _stream(stream)), "ferry_members_leave")

    def members_join(self, lanes, stream=None):
        """New requests of the owners' groups take these lanes (resident again)."""
        n = int(lanes.numel())
        _check(lib.ferry_members_join(self._h, _dev(lanes, "lanes", n, _I32, self.device), n,
                                      _stream(stream)), "ferry_members_join")

    def members(self):
        """Resident members of every owner (synchronises)."""
        out = np.zeros((self.sel_shape[0] + self.cfg.group - 1) // self.cfg.group, np.uint32)
        _check(lib.ferry_members_get(self._h, out.ctypes.data), "ferry_members_get")
        return out

    def stats(self):
        s = Stats()
        _check(lib.ferry_stats_get(self._h, C.byref(s)), "ferry_stats_get")
        return {f: getattr(s, f) for f, _ in Stats._fields_ if f != "pad"}

    def bw_probe(self, kind, n, slots=None, iters=5, stream=None):
        """Plain-read bandwidth ceiling (ferry_bw_probe): returns (bytes per
        launch, mean ms per launch, GB/s)."""
        b, ms = C.c_uint64(), C.c_float()
        if kind == PROBE_HBM_GATHER:  # n rows of the slot table
            slots_p = _dev(slots, "slots", n * self.cfg.k, _I32, self.device)
        else:
            slots_p = None
        _check(lib.ferry_bw_probe(self._h, kind, slots_p, n, iters, C.byref(b), C.byref(ms),
                                  _stream(stream)), "ferry_bw_probe")
        return b.value, ms.value, b.value / (ms.value * 1e-3) / 1e9

    def stats_reset(self):
        _check(lib.ferry_stats_reset(self._h), "ferry_stats_reset")

    def sets_state(self):
        cap = self.cfg.slots_per_set
        fill = np.zeros(self.n_sets, np.uint32)
        ord_ = np.zeros((self.n_sets, cap), np.uint32)
        tag = np.zeros((self.n_sets, cap), np.uint32)
        _check(lib.ferry_sets_state(self._h, fill.ctypes.data, ord_.ctypes.data, tag.ctypes.data),
               "ferry_sets_state")
        return fill, ord_, tag

    def sets_own(self):
        """Per-slot member masks [n_sets, slots] of prefix groups (synchronises)."""
        own = np.zeros((self.n_sets, self.cfg.slots_per_set), np.uint32)
        _check(lib.ferry_sets_own(self._h, own.ctypes.data), "ferry_sets_own")
        return own

    def hosttier_register(self, host, scales=None):
        """Use the caller's pinned host memory (a pin_memory uint8 CPU tensor of
        host_blocks * block_bytes, plus float32 scales for fp8) as the host tier.
        The tensors are kept alive by the executor."""
        sb = 0 if scales is None else scales.numel() * scales.element_size()
        _check(lib.ferry_hosttier_register(self._h, _ptr(host), host.numel() * host.element_size(),
                                           _ptr(scales), sb), "ferry_hosttier_register")
        self._registered = (host, scales)

    def hosttier_array(self):
        """numpy view of the pinned host tier (bytes) and fp8 scales (or None)."""
        b, s = _vp(), _vp()
        _check(lib.ferry_hosttier_view(self._h, C.byref(b), C.byref(s)), "ferry_hosttier_view")
        n = self.cfg.host_blocks * self.block_bytes
        arr = np.ctypeslib.as_array(C.cast(b, C.POINTER(C.c_uint8)), shape=(n,))
        sc = None
        if s.value:
            sc = np.ctypeslib.as_array(C.cast(s, C.POINTER(C.c_float)),
                                       shape=(self.cfg.host_blocks * 2,))
        return arr, sc

    def pool_ptrs(self):
        p, s = _vp(), _vp()
        _check(lib.ferry_pool_view(self._h, C.byref(p), C.byref(s)), "ferry_pool_view")
        return p.value, s.value

    def pool_slots_bytes(self, slot_ids):
        """Copy the given pool slots (global ids) to host: [n, block_bytes] uint8."""
        p, _ = self.pool_ptrs()
        return _gather_d2h(p, self.block_bytes, slot_ids)

    def pool_slot_scales(self, slot_ids):
        """fp8 scales (k, v) of the given pool slots, or None."""
        _, s = self.pool_ptrs()
        if not s:
            return None
        return _gather_d2h(s, 8, slot_ids).view(np.float32).reshape(-1, 2)


_hip = None


def _gather_d2h(base, row_bytes, ids):
    """rows base[ids[i] * row_bytes : +row_bytes] of device memory -> host array."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7")  # the runtime already loaded with torch
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipMemcpy.argtypes = [_vp, _vp, C.c_size_t, C.c_int]
        _hip.hipDeviceSynchronize.restype = C.c_int
    ids = np.asarray(ids, np.int64).reshape(-1)
    out = np.zeros((ids.size, row_bytes), np.uint8)
    if _hip.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipDeviceSynchronize failed")
    order = np.argsort(ids, kind="stable")
    i = 0
    while i < ids.size:  # copy runs of consecutive ids in one call
        j = i + 1
        while j < ids.size and ids[order[j]] == ids[order[j - 1]] + 1 and \
                order[j] == order[j - 1] + 1:
            j += 1
        rc = _hip.hipMemcpy(out[order[i]:].ctypes.data, base + int(ids[order[i]]) * row_bytes,
                            (j - i) * row_bytes, 2)
        if rc != 0:
            raise RuntimeError(f"hipMemcpy D2H failed ({rc})")
        i = j
    return out


class SelGen:
    """Synthetic top-k selection stream (host).  Steps must be drawn in order."""

    def __init__(self, n_req, n_layers, kv_heads, k, ctx_blocks, dist=1, zipf_s=1.1,
                 reuse=0.66, group=1, prefix_blocks=0, seed=1):
        self.cfg = SelGenConfig(n_req, group, n_layers, kv_heads, k, dist, zipf_s, reuse,
                                prefix_blocks, 0, seed)
        ctx = np.ascontiguousarray(ctx_blocks, np.int32)
        h = _vp()
        _check(lib.ferry_selgen_create(C.byref(self.cfg), ctx.ctypes.data, C.byref(h)),
               "ferry_selgen_create")
        self._h = h
        mb = _i32()
        _check(lib.ferry_selgen_max_blocks(h, C.byref(mb)), "ferry_selgen_max_blocks")
        self.max_blocks = mb.value
        self.shape = (n_req, n_layers, kv_heads, k)

    def set_reuse(self, reuse):
        """Per-request reuse probabilities (None: the configured one for all)."""
        self._reuse = None if reuse is None else np.ascontiguousarray(reuse, np.float64)
        _check(lib.ferry_selgen_set_reuse(self._h, None if self._reuse is None
                                          else self._reuse.ctypes.data), "ferry_selgen_set_reuse")

    def step(self, step):
        out = np.zeros(self.shape, np.uint32)
        _check(lib.ferry_selgen_step(self._h, step, out.ctypes.data), "ferry_selgen_step")
        return out

    def admit(self, lane, request_id, ctx_blocks, step):
        """Request `request_id` (context ctx_blocks) takes `lane` from `step` on."""
        _check(lib.ferry_selgen_admit(self._h, lane, request_id, ctx_blocks, step),
               "ferry_selgen_admit")

    def retire(self, lane):
        """`lane` produces empty rows until its next admission."""
        _check(lib.ferry_selgen_retire(self._h, lane), "ferry_selgen_retire")

    def set_private_ranges(self, ranges):
        """`ranges` (>= group) private id ranges per prefix-group owner, for
        members that turn over; updates max_blocks."""
        _check(lib.ferry_selgen_set_private_ranges(self._h, ranges),
               "ferry_selgen_set_private_ranges")
        mb = _i32()
        _check(lib.ferry_selgen_max_blocks(self._h, C.byref(mb)), "ferry_selgen_max_blocks")
        self.max_blocks = mb.value

    def admit_member(self, lane, request_id, ctx_blocks, step, private_range):
        """A request of the lane's prefix group takes `lane` from `step` on,
        its private blocks in id range `private_range`."""
        _check(lib.ferry_selgen_admit_member(self._h, lane, request_id, ctx_blocks, step,
                                             private_range), "ferry_selgen_admit_member")

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h and lib is not None:
            lib.ferry_selgen_destroy(h)


def ctx_uniform(seed, n_req, lo, hi):
    out = np.zeros(n_req, np.int32)
    _check(lib.ferry_ctx_uniform(seed, n_req, lo, hi, out.ctypes.data), "ferry_ctx_uniform")
    return out


def arrivals(kind, n, gap_ms, period_ms=50.0, ratio=10.0, seed=0):
    """Arrival times (ms) of n requests (ferry_arrivals)."""
    out = np.zeros(n, np.float64)
    _check(lib.ferry_arrivals(kind, n, gap_ms, period_ms, ratio, seed, out.ctypes.data),
           "ferry_arrivals")
    return out


class Sched:
    """Tick scheduler of one executor (ferry_sched_*): `lanes` batch lanes
    serve requests that arrive at arrive_ms and decode len_steps steps."""

    def __init__(self, lanes, arrive_ms, len_steps, pinned=False):
        self.lanes = lanes
        self._arr = np.ascontiguousarray(arrive_ms, np.float64)
        self._len = np.ascontiguousarray(len_steps, np.int32)
        self.n = self._arr.size
        h = _vp()
        _check(lib.ferry_sched_create(lanes, SCHED_PINNED if pinned else SCHED_FIFO, self.n,
                                      self._arr.ctypes.data, self._len.ctypes.data, C.byref(h)),
               "ferry_sched_create")
        self._h = h

    def tick(self, now_ms):
        """One tick: returns dict(lane_req, lane_step, admitted, retired,
        resident, done)."""
        lr = np.zeros(self.lanes, np.int32)
        ls = np.zeros(self.lanes, np.int32)
        ad = np.zeros(self.lanes, np.int32)
        rt = np.zeros(self.lanes, np.int32)
        na, nr, nres, done = _i32(), _i32(), _i32(), _i32()
        _check(lib.ferry_sched_tick(self._h, now_ms, lr.ctypes.data, ls.ctypes.data,
                                    ad.ctypes.data, C.byref(na), rt.ctypes.data, C.byref(nr),
                                    C.byref(nres), C.byref(done)), "ferry_sched_tick")
        return dict(lane_req=lr, lane_step=ls, admitted=ad[:na.value].copy(),
                    retired=rt[:nr.value].copy(), resident=nres.value, done=bool(done.value))

    def next_arrival(self):
        v = C.c_double()
        _check(lib.ferry_sched_next_arrival(self._h, C.byref(v)), "ferry_sched_next_arrival")
        return v.value

    def request_ticks(self):
        a = np.zeros(self.n, np.int32)
        d = np.zeros(self.n, np.int32)
        _check(lib.ferry_sched_request_ticks(self._h, a.ctypes.data, d.ctypes.data),
               "ferry_sched_request_ticks")
        return a, d

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h and lib is not None:
            lib.ferry_sched_destroy(h)


def trace_load(path, strict=True):
    """Read an FMT1 selection trace: (info dict, dense ids [R, S, L, sel_blocks])."""
    info = TraceInfo()
    p = os.fsencode(path)
    _check(lib.ferry_trace_load(p, int(strict), C.byref(info), None, 0), "ferry_trace_load")
    ids = np.zeros((info.requests, info.steps, info.layers, info.sel_blocks), np.uint32)
    _check(lib.ferry_trace_load(p, int(strict), C.byref(info), ids.ctypes.data, ids.size),
           "ferry_trace_load")
    return {f: getattr(info, f) for f, _ in TraceInfo._fields_}, ids


def refgen_selections(R, L, S, sel, seed=42):
    """replay_miss_stream's selections, (r, s, l, k) order -> array [R, S, L, sel]."""
    out = np.zeros((R, S, L, sel), np.uint32)
    _check(lib.ferry_refgen_selections(R, L, S, sel, seed, out.ctypes.data),
           "ferry_refgen_selections")
    return out


def queue_selftest(capacity=1 << 20, n_tasks=1 << 22, producers=512, consumers=512, mode=1,
                   device=0):
    """Exactly-once run of the device MPMC ring.  Returns (popped, dups, ms)."""
    p, d, ms = C.c_uint64(), C.c_uint64(), C.c_float()
    _check(lib.ferry_queue_selftest(device, capacity, n_tasks, producers, consumers, mode,
                                    C.byref(p), C.byref(d), C.byref(ms)), "ferry_queue_selftest")
    return p.value, d.value, ms.value


def queue_ticket_probe(threads=512, iters=4096, kind=1, device=0):
    """Tickets taken from one shared word by `threads` threads, `iters` each:
    kind 0 fetch-add per thread, kind 1 a load + compare-and-swap retry per
    thread, kind 2 that retry once per wavefront for its 64 lanes.
    Returns (tickets, ms)."""
    t, ms = C.c_uint64(), C.c_float()
    _check(lib.ferry_queue_ticket_probe(device, threads, iters, kind, C.byref(t), C.byref(ms)),
           "ferry_queue_ticket_probe")
    return t.value, ms.value
