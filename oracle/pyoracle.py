"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by the cpu_baseline leg of bench.py, to check the GPU against.  The product never
imports it.
"""
import ctypes as C
import os
import struct
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16, FP8 = 0, 1, 2, 3
NONE = 0xFFFFFFFF


def build():
    """Compile liboracle.so (and oracle/_ref when the reference tree exists)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    if not os.path.exists(_LIB):
        build()
    return C.CDLL(_LIB)


lib = _load()

_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")

MISS_DTYPE = np.dtype([("block", "<u4"), ("slot", "<u4"), ("evicted", "<u4"), ("set", "<u4")])
_missp = np.ctypeslib.ndpointer(MISS_DTYPE, flags="C_CONTIGUOUS")


class Geom(C.Structure):
    _fields_ = [
        ("n_req", C.c_int), ("group", C.c_int), ("n_layers", C.c_int),
        ("kv_heads", C.c_int), ("q_heads", C.c_int), ("head_dim", C.c_int),
        ("block_tokens", C.c_int), ("k", C.c_int), ("cap", C.c_int),
        ("max_blocks", C.c_int), ("dtype", C.c_int), ("granularity", C.c_int),
        ("host_blocks", C.c_uint64), ("seed", C.c_uint64), ("value_std", C.c_float),
        ("cap_mode", C.c_int),
    ]


class SelGen(C.Structure):
    _fields_ = [
        ("n_req", C.c_int), ("group", C.c_int), ("n_layers", C.c_int),
        ("kv_heads", C.c_int), ("k", C.c_int), ("dist", C.c_int),
        ("zipf_s", C.c_double), ("reuse", C.c_double), ("prefix_blocks", C.c_int), ("seed", C.c_uint64),
        ("ctx_blocks", C.POINTER(C.c_int)), ("reuse_r", C.POINTER(C.c_double)),
        ("rid", C.POINTER(C.c_int)), ("start", C.POINTER(C.c_int)),
        ("active", C.POINTER(C.c_uint8)), ("prange", C.POINTER(C.c_int)),
        ("private_ranges", C.c_int), ("nperm", C.POINTER(C.c_int)),
    ]


class MT64(C.Structure):
    _fields_ = [("mt", C.c_uint64 * 312), ("idx", C.c_int)]


class LRU(C.Structure):
    _fields_ = [("cap", C.c_int), ("lim", C.c_int), ("max_blocks", C.c_int), ("fill", C.c_uint32),
                ("ord", C.POINTER(C.c_uint32)), ("tag", C.POINTER(C.c_uint32)),
                ("map", C.POINTER(C.c_uint32)), ("own", C.POINTER(C.c_uint32))]


class TSLRU(C.Structure):
    _fields_ = [("cap", C.c_int), ("max_blocks", C.c_int),
                ("tag", C.POINTER(C.c_uint32)), ("stamp", C.POINTER(C.c_uint64)),
                ("clock", C.c_uint64), ("fill", C.c_uint32)]


def _sig(name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


_sig("ora_mix64", C.c_uint64, C.c_uint64, C.c_uint64)
_sig("ora_f32_to_f16", C.c_uint16, C.c_float)
_sig("ora_f16_to_f32", C.c_float, C.c_uint16)
_sig("ora_f32_to_bf16", C.c_uint16, C.c_float)
_sig("ora_bf16_to_f32", C.c_float, C.c_uint16)
_sig("ora_f32_to_e4m3", C.c_uint8, C.c_float)
_sig("ora_e4m3_to_f32", C.c_float, C.c_uint8)
_sig("ora_mt64_seed", None, C.POINTER(MT64), C.c_uint64)
_sig("ora_mt64_next", C.c_uint64, C.POINTER(MT64))
_sig("ora_ref_replay", C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64,
     C.c_void_p, C.c_void_p, _u64p)
_sig("ora_ref_cmode_runs", C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
     C.c_uint64, C.c_double, C.c_double, C.c_double, _u64p, _u8p, C.POINTER(C.c_uint64))
_sig("ora_lru_init", C.c_int, C.POINTER(LRU), C.c_int, C.c_int)
_sig("ora_lru_free", None, C.POINTER(LRU))
_sig("ora_lru_substep", C.c_int, C.POINTER(LRU), C.c_uint32, _u32p, C.c_int, _u32p, _missp,
     C.POINTER(C.c_int), C.c_void_p)
_sig("ora_deque_lru_run", C.c_int, C.c_int, _u32p, C.c_int, _u8p)
_sig("ora_deque_lru_run_caps", C.c_int, _i32p, _i32p, _u32p, C.c_int, _u8p, _u32p)
_sig("ora_lru_trim", C.c_int, C.POINTER(LRU), C.c_int, C.c_void_p)
_sig("ora_exec_members", C.c_int, C.c_void_p, _u32p, C.c_int, C.c_int)
_sig("ora_exec_members_get", None, C.c_void_p, _u32p)
_sig("ora_exec_own", None, C.c_void_p, _u32p)
_sig("ora_exec_export_member", C.c_int, C.c_void_p, C.c_int, _u32p, _u32p)
_sig("ora_exec_import_member", C.c_int, C.c_void_p, C.c_int, _u32p, _u32p)
_sig("ora_capacity", C.c_int, C.POINTER(Geom), C.c_int)
_sig("ora_tslru_init", C.c_int, C.POINTER(TSLRU), C.c_int, C.c_int)
_sig("ora_tslru_free", None, C.POINTER(TSLRU))
_sig("ora_tslru_step", C.c_int, C.POINTER(TSLRU), _u32p, C.c_int, _u32p, _u32p, _u32p,
     C.POINTER(C.c_int))
_sig("ora_n_sets", C.c_int, C.POINTER(Geom))
_sig("ora_max_sel_per_set", C.c_int, C.POINTER(Geom))
_sig("ora_block_bytes", C.c_uint64, C.POINTER(Geom))
_sig("ora_host_index", C.c_uint64, C.POINTER(Geom), C.c_uint32, C.c_uint32)
_sig("ora_exec_create", C.c_void_p, C.POINTER(Geom))
_sig("ora_exec_destroy", None, C.c_void_p)
_sig("ora_exec_step", C.c_int, C.c_void_p, _u32p, _u32p, _u32p, _missp, _u64p, _u8p)
_sig("ora_exec_state", None, C.c_void_p, _u32p, _u32p, _u32p)
_sig("ora_exec_reset_owner", C.c_int, C.c_void_p, C.c_int)
_sig("ora_exec_copy_owner", C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int)
_sig("ora_arrivals", C.c_int, C.c_int, C.c_uint32, C.c_double, C.c_double, C.c_double,
     C.c_uint64, _f64p)
_sig("ora_ctx_uniform", None, C.c_uint64, C.c_int, C.c_int, C.c_int, _i32p)
_sig("ora_selgen_max_blocks", C.c_int, C.POINTER(SelGen))
_sig("ora_selgen_step", C.c_int, C.POINTER(SelGen), C.c_int, _u32p, _u32p)
_sig("ora_host_elem", C.c_uint32, C.POINTER(Geom), C.c_uint64, C.c_uint32)
_sig("ora_host_scale", C.c_float, C.POINTER(Geom), C.c_uint64, C.c_int)
_sig("ora_host_block", None, C.POINTER(Geom), C.c_uint64, C.c_void_p, C.c_void_p)
_sig("ora_host_fill", None, C.POINTER(Geom), C.c_void_p, C.c_void_p)
_sig("ora_attention_f64", C.c_int, C.POINTER(Geom), _u32p, _f32p, _f64p)
_sig("ora_attention_hidx_f64", C.c_int, C.POINTER(Geom), _u64p, _f32p, _f64p)
_sig("ora_attention_tier_f64", C.c_int, C.POINTER(Geom), _u64p, C.c_void_p, C.c_void_p, _f32p,
     _f64p)
_sig("ora_attention_pool_f32", C.c_int, C.POINTER(Geom), _u32p, C.c_void_p, C.c_void_p,
     _f32p, _f32p)
_sig("ora_summary", None, C.POINTER(Geom), C.c_uint64, _f32p, _f32p)
_sig("ora_quest_scores", C.c_int, C.POINTER(Geom), _f32p, _i32p, C.c_int, C.c_int, _f32p)
_sig("ora_select_topk", C.c_int, C.POINTER(Geom), _f32p, _i32p, C.c_int, _u32p)
_sig("ora_mass_scores", C.c_int, C.POINTER(Geom), _f32p, _i32p, C.c_int,
     np.ctypeslib.ndpointer(np.float64, flags="C"))
_sig("ora_select_mass", C.c_int, C.POINTER(Geom), _f32p, _i32p, _u32p)
_sig("ora_cpu_step", C.c_int, C.c_void_p, _u32p, C.c_void_p, C.c_void_p, C.c_void_p,
     C.c_void_p, _f32p, _f32p, _u32p, _u32p, _missp, _u64p)


def esize(dtype):
    return {F32: 4, F16: 2, BF16: 2, FP8: 1}[dtype]


# ---------------------------------------------------------------- reference replay
def ref_replay(R, L, S, sel, hot, seed=42, events=True):
    """Restated replay_miss_stream; returns (blocks u64, miss u8, selects, misses)."""
    n = R * L * S * sel
    blocks = np.zeros(n, np.uint64) if events else None
    miss = np.zeros(n, np.uint8) if events else None
    counts = np.zeros(2, np.uint64)
    rc = lib.ora_ref_replay(R, L, S, sel, hot, seed,
                            blocks.ctypes.data if events else None,
                            miss.ctypes.data if events else None, counts)
    if rc:
        raise RuntimeError(f"ora_ref_replay rc={rc}")
    return blocks, miss, int(counts[0]), int(counts[1])


def ref_cmode_runs(R, L, S, sel, hot, c4, blocks, miss, min_mb=1.0, max_mb=4.0, target=4.0):
    rb = C.c_uint64(0)
    ev = lib.ora_ref_cmode_runs(R, L, S, sel, hot, c4, min_mb, max_mb, target,
                                np.ascontiguousarray(blocks, np.uint64),
                                np.ascontiguousarray(miss, np.uint8), C.byref(rb))
    return int(ev), int(rb.value)


# ---------------------------------------------------------------- executor
class Executor:
    """Oracle executor: one LRU set per (owner, layer, kv head)."""

    def __init__(self, geom: Geom):
        self.g = geom
        self.ptr = lib.ora_exec_create(C.byref(geom))
        if not self.ptr:
            raise MemoryError("ora_exec_create")
        self.n_sets = lib.ora_n_sets(C.byref(geom))
        self.max_sel = lib.ora_max_sel_per_set(C.byref(geom))

    def __del__(self):
        # at interpreter exit the module globals may already be gone
        if getattr(self, "ptr", None) and lib is not None:
            lib.ora_exec_destroy(self.ptr)
            self.ptr = None

    def step(self, sel):
        g = self.g
        sel = np.ascontiguousarray(sel, np.uint32).reshape(-1)
        slots = np.zeros(sel.size, np.uint32)
        mc = np.zeros(self.n_sets, np.uint32)
        misses = np.zeros(self.n_sets * self.max_sel, MISS_DTYPE)
        counts = np.zeros(3, np.uint64)
        flags = np.zeros(sel.size, np.uint8)
        rc = lib.ora_exec_step(self.ptr, sel, slots, mc, misses, counts, flags)
        if rc:
            raise RuntimeError(f"ora_exec_step rc={rc}")
        self.last_flags = flags
        return slots, mc, misses.reshape(self.n_sets, self.max_sel), counts

    def copy_owner_from(self, src, src_owner, dst_owner):
        if lib.ora_exec_copy_owner(src.ptr, src_owner, self.ptr, dst_owner):
            raise ValueError("geometry or owner mismatch")

    def reset_owner(self, owner):
        if lib.ora_exec_reset_owner(self.ptr, owner):
            raise ValueError(f"owner {owner}")

    def members_leave(self, lanes):
        """Requests of these lanes leave (trim under cap_mode 1); False if a
        lane was out of range or not resident (it is skipped)."""
        return lib.ora_exec_members(self.ptr, np.ascontiguousarray(lanes, np.uint32),
                                    len(lanes), -1) == 0

    def members_join(self, lanes):
        return lib.ora_exec_members(self.ptr, np.ascontiguousarray(lanes, np.uint32),
                                    len(lanes), 1) == 0

    def members(self):
        out = np.zeros((self.g.n_req + self.g.group - 1) // self.g.group, np.uint32)
        lib.ora_exec_members_get(self.ptr, out)
        return out

    def own(self):
        """Member masks [n_sets, cap] (bit m: member m touched the slot's block)."""
        out = np.zeros(self.n_sets * self.g.cap, np.uint32)
        lib.ora_exec_own(self.ptr, out)
        return out.reshape(self.n_sets, self.g.cap)

    def export_member(self, lane):
        """Blocks only lane's member touched, per set of its owner, LRU first:
        (counts [L*Hkv], blocks [L*Hkv, cap])."""
        per = self.g.n_layers * self.g.kv_heads
        counts = np.zeros(per, np.uint32)
        blocks = np.zeros(per * self.g.cap, np.uint32)
        if lib.ora_exec_export_member(self.ptr, lane, counts, blocks):
            raise ValueError(f"lane {lane}")
        return counts, blocks.reshape(per, self.g.cap)

    def import_member(self, lane, counts, blocks):
        if lib.ora_exec_import_member(self.ptr, lane, np.ascontiguousarray(counts, np.uint32),
                                      np.ascontiguousarray(blocks, np.uint32).reshape(-1)):
            raise ValueError("import_member refused")

    def state(self):
        cap = self.g.cap
        fill = np.zeros(self.n_sets, np.uint32)
        ord_ = np.zeros(self.n_sets * cap, np.uint32)
        tag = np.zeros(self.n_sets * cap, np.uint32)
        lib.ora_exec_state(self.ptr, fill, ord_, tag)
        return fill, ord_.reshape(self.n_sets, cap), tag.reshape(self.n_sets, cap)


def make_geom(**kw):
    g = Geom()
    defaults = dict(group=1, q_heads=None, head_dim=128, block_tokens=16, dtype=F16,
                    granularity=0, host_blocks=1 << 16, seed=7, value_std=0.5, cap_mode=0)
    defaults.update(kw)
    if defaults["q_heads"] is None:
        defaults["q_heads"] = defaults["kv_heads"]
    for k, v in defaults.items():
        setattr(g, k, v)
    return g


def selgen(n_req, n_layers, kv_heads, k, ctx_blocks, dist=1, zipf_s=1.1, reuse=0.66,
           group=1, prefix_blocks=0, seed=1, reuse_r=None):
    ctx = np.ascontiguousarray(ctx_blocks, np.int32)
    rr = None if reuse_r is None else np.ascontiguousarray(reuse_r, np.float64)
    s = SelGen(n_req, group, n_layers, kv_heads, k, dist, zipf_s, reuse, prefix_blocks, seed,
               ctx.ctypes.data_as(C.POINTER(C.c_int)),
               rr.ctypes.data_as(C.POINTER(C.c_double)) if rr is not None else None)
    s._ctx = ctx  # keep alive
    s._rr = rr
    s._state = np.zeros(n_req * n_layers * kv_heads * k, np.uint32)
    # lane turnover: request id, admission step and activity of each lane
    s._rid = np.arange(n_req, dtype=np.int32)
    s._start = np.zeros(n_req, np.int32)
    s._active = np.ones(n_req, np.uint8)
    s.rid = s._rid.ctypes.data_as(C.POINTER(C.c_int))
    s.start = s._start.ctypes.data_as(C.POINTER(C.c_int))
    s.active = s._active.ctypes.data_as(C.POINTER(C.c_uint8))
    return s


def selgen_admit(s: SelGen, lane, request_id, ctx_blocks, step):
    """Request `request_id` with context ctx_blocks takes `lane` from `step`."""
    s._rid[lane] = request_id
    s._start[lane] = step
    s._ctx[lane] = ctx_blocks
    s._active[lane] = 1


def selgen_retire(s: SelGen, lane):
    s._active[lane] = 0


def selgen_group_turnover(s: SelGen, private_ranges):
    """Let prefix-group lanes turn over: each owner's permutation domain is
    fixed at its creation value, and `private_ranges` private id ranges per
    owner are available to successive members (selgen_admit_member)."""
    nown = (s.n_req + s.group - 1) // s.group
    s._nperm = np.array([int(s._ctx[o * s.group:(o + 1) * s.group].max()) for o in range(nown)],
                        np.int32)
    s._prange = (np.arange(s.n_req) % s.group).astype(np.int32)
    s.nperm = s._nperm.ctypes.data_as(C.POINTER(C.c_int))
    s.prange = s._prange.ctypes.data_as(C.POINTER(C.c_int))
    s.private_ranges = private_ranges


def selgen_admit_member(s: SelGen, lane, request_id, ctx_blocks, step, private_range):
    """A request of lane's prefix group takes the lane from `step`, with its
    private blocks in id range `private_range`."""
    selgen_admit(s, lane, request_id, ctx_blocks, step)
    s._prange[lane] = private_range


def selgen_step(s: SelGen, step):
    """Selections of `step`; steps must be generated in order (state carries)."""
    out = np.zeros(s.n_req * s.n_layers * s.kv_heads * s.k, np.uint32)
    rc = lib.ora_selgen_step(C.byref(s), step, s._state, out)
    if rc:
        raise RuntimeError(f"ora_selgen_step rc={rc}")
    return out


def selgen_max_blocks(s: SelGen):
    return lib.ora_selgen_max_blocks(C.byref(s))


def ctx_uniform(seed, n_req, lo, hi):
    out = np.zeros(n_req, np.int32)
    lib.ora_ctx_uniform(seed, n_req, lo, hi, out)
    return out


def host_block(g: Geom, h):
    bb = lib.ora_block_bytes(C.byref(g))
    buf = np.zeros(bb, np.uint8)
    sc = np.zeros(2, np.float32)
    lib.ora_host_block(C.byref(g), h, buf.ctypes.data, sc.ctypes.data)
    return buf, sc


def host_fill(g: Geom):
    bb = lib.ora_block_bytes(C.byref(g))
    host = np.zeros(g.host_blocks * bb, np.uint8)
    sc = np.zeros(g.host_blocks * 2, np.float32)
    lib.ora_host_fill(C.byref(g), host.ctypes.data, sc.ctypes.data)
    return host, sc


def attention_f64(g: Geom, sel, q):
    out = np.zeros(q.size, np.float64)
    rc = lib.ora_attention_f64(C.byref(g), np.ascontiguousarray(sel, np.uint32).reshape(-1),
                               np.ascontiguousarray(q, np.float32).reshape(-1), out)
    if rc:
        raise RuntimeError("ora_attention_f64")
    return out.reshape(q.shape)


def attention_hidx_f64(g: Geom, hidx, q):
    """Attention with each row's blocks given as host-tier indices
    ([B][L][Hkv][k] uint64, NONE64 = empty position)."""
    out = np.zeros(q.size, np.float64)
    rc = lib.ora_attention_hidx_f64(C.byref(g), np.ascontiguousarray(hidx, np.uint64).reshape(-1),
                                    np.ascontiguousarray(q, np.float32).reshape(-1), out)
    if rc:
        raise RuntimeError("ora_attention_hidx_f64")
    return out.reshape(q.shape)


def attention_tier_f64(g: Geom, hidx, host, host_scales, q):
    """attention_hidx_f64 over a caller's host tier image (uint8 bytes
    [host_blocks * bb], fp8 scales float32 [host_blocks * 2]) instead of the
    generated content."""
    host = np.ascontiguousarray(host, np.uint8)
    sc = None if host_scales is None else np.ascontiguousarray(host_scales, np.float32)
    out = np.zeros(q.size, np.float64)
    rc = lib.ora_attention_tier_f64(C.byref(g), np.ascontiguousarray(hidx, np.uint64).reshape(-1),
                                    host.ctypes.data, None if sc is None else sc.ctypes.data,
                                    np.ascontiguousarray(q, np.float32).reshape(-1), out)
    if rc:
        raise RuntimeError("ora_attention_tier_f64")
    return out.reshape(q.shape)


NONE64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def host_index(g: Geom, set_id, block):
    return int(lib.ora_host_index(C.byref(g), set_id, block))


def arrivals(kind, n, gap_ms, period_ms=50.0, ratio=10.0, seed=0):
    out = np.zeros(n, np.float64)
    if lib.ora_arrivals(kind, n, gap_ms, period_ms, ratio, seed, out):
        raise ValueError("ora_arrivals")
    return out


def sched_run(lanes, arrive_ms, len_steps, clock_ms, pinned=False):
    """Tick scheduler of one executor, restated for small cases.

    Tick t starts at clock_ms[t].  A request is resident from the tick of its
    admission until it has run len_steps ticks (the reference retires a
    request in tick_end once next_step reaches its length,
    src/runtime/wla_multigpu.cuh:834-857).  Arrived requests queue in arrival
    order (ties by id) and fill free lanes, lowest lane first; `pinned`
    requests only take lane r % lanes.  Returns the
    lane -> request table of every tick ([ticks][lanes], -1 idle) and each
    request's admission and last tick (-1 if never).
    """
    n = len(arrive_ms)
    queue = sorted(range(n), key=lambda r: (arrive_ms[r], r))
    lane_of = [-1] * lanes
    ran = [0] * n
    admit, last = [-1] * n, [-1] * n
    table = []
    qi = 0  # queue[:qi] have been admitted
    for t, now in enumerate(clock_ms):
        for ln in range(lanes):  # the previous tick ran every resident request
            r = lane_of[ln]
            if r >= 0 and t > 0:
                ran[r] += 1
                if ran[r] == len_steps[r]:
                    last[r] = t - 1
                    lane_of[ln] = -1
        if pinned:
            for ln in range(lanes):
                if lane_of[ln] >= 0:
                    continue
                mine = [r for r in queue if r % lanes == ln and admit[r] < 0
                        and arrive_ms[r] <= now]
                if mine:
                    lane_of[ln] = mine[0]
                    admit[mine[0]] = t
        else:
            for ln in range(lanes):
                if lane_of[ln] < 0 and qi < n and arrive_ms[queue[qi]] <= now:
                    lane_of[ln] = queue[qi]
                    admit[queue[qi]] = t
                    qi += 1
        table.append(list(lane_of))
    return np.array(table, np.int32).reshape(len(clock_ms), lanes), admit, last


def trace_load(path, strict=True):
    """FMT1 trace reader restated with numpy (tools/capture_miss_trace.py:27-38
    header, :366-370 records; dense renaming in order of first appearance as
    in src/workloads/miss_trace.cuh:136-145).  Returns (header dict, dense ids
    [R, S, L, sel_blocks] with NONE padding, unique count, max distinct ids of
    one request).  Raises ValueError where the product returns FERRY_EINVAL."""
    raw = open(path, "rb").read()
    if raw[:4] != b"FMT1":
        raise ValueError("magic")
    if len(raw) < 40:
        raise ValueError("header")
    ver, R, S, L, PT, BT, KV, D, SEL = struct.unpack_from("<9I", raw, 4)
    if ver != 1 or BT == 0 or PT == 0 or PT % BT:
        raise ValueError("header")
    nb = SEL * (PT // BT)
    recs, pos = [], 40
    for _ in range(R * S * L):
        if pos + 2 > len(raw):
            raise ValueError("truncated")
        (cnt,) = struct.unpack_from("<H", raw, pos)
        pos += 2
        if cnt > nb or (strict and cnt < nb):
            raise ValueError("count")
        if pos + 4 * cnt > len(raw):
            raise ValueError("truncated")
        recs.append(np.frombuffer(raw, "<u4", cnt, pos))
        pos += 4 * cnt
    flat = np.concatenate(recs) if recs else np.zeros(0, np.uint32)
    uniq, first, inv = np.unique(flat, return_index=True, return_inverse=True)
    rank = np.empty(len(uniq), np.int64)
    rank[np.argsort(first, kind="stable")] = np.arange(len(uniq))
    dense = rank[inv].astype(np.uint32)
    out = np.full((R * S * L, nb), NONE, np.uint32)
    i = 0
    for j, rec in enumerate(recs):
        out[j, :len(rec)] = dense[i:i + len(rec)]
        i += len(rec)
    per_req = [len(np.unique(np.concatenate(recs[r * S * L:(r + 1) * S * L])))
               if S * L else 0 for r in range(R)]
    hdr = dict(requests=R, steps=S, layers=L, page_tokens=PT, block_tokens=BT, kv_heads=KV,
               head_dim=D, sel_pages=SEL, sel_blocks=nb)
    return hdr, out.reshape(R, S, L, nb), len(uniq), max(per_req) if per_req else 0


def summary(g: Geom, h):
    kmin = np.zeros(g.head_dim, np.float32)
    kmax = np.zeros(g.head_dim, np.float32)
    lib.ora_summary(C.byref(g), h, kmin, kmax)
    return kmin, kmax


def quest_scores(g: Geom, q, ctx_blocks, mode=0):
    """Scores [rows, max ctx] (NaN where a row's context ends)."""
    ctx = np.ascontiguousarray(ctx_blocks, np.int32)
    stride = max(1, int(ctx.max()))
    rows = g.n_req * g.n_layers * (1 if mode else g.kv_heads)
    out = np.full(rows * stride, np.nan, np.float32)
    lib.ora_quest_scores(C.byref(g), np.ascontiguousarray(q, np.float32).reshape(-1), ctx, mode,
                         stride, out)
    return out.reshape(rows, stride)


def mass_scores(g: Geom, q, ctx_blocks):
    """Softmax mass per block, double [B, L, max ctx] (NaN past a context)."""
    ctx = np.ascontiguousarray(ctx_blocks, np.int32)
    stride = max(1, int(ctx.max()))
    out = np.full(g.n_req * g.n_layers * stride, np.nan, np.float64)
    if lib.ora_mass_scores(C.byref(g), np.ascontiguousarray(q, np.float32).reshape(-1), ctx,
                           stride, out):
        raise ValueError("context longer than max_blocks")
    return out.reshape(g.n_req, g.n_layers, stride)


def select_mass(g: Geom, q, ctx_blocks):
    sel = np.zeros(g.n_req * g.n_layers * g.kv_heads * g.k, np.uint32)
    if lib.ora_select_mass(C.byref(g), np.ascontiguousarray(q, np.float32).reshape(-1),
                           np.ascontiguousarray(ctx_blocks, np.int32), sel):
        raise ValueError("context longer than max_blocks")
    return sel.reshape(g.n_req, g.n_layers, g.kv_heads, g.k)


def select_topk(g: Geom, q, ctx_blocks, mode=0):
    sel = np.zeros(g.n_req * g.n_layers * g.kv_heads * g.k, np.uint32)
    if lib.ora_select_topk(C.byref(g), np.ascontiguousarray(q, np.float32).reshape(-1),
                           np.ascontiguousarray(ctx_blocks, np.int32), mode, sel):
        raise ValueError("context longer than max_blocks")
    return sel.reshape(g.n_req, g.n_layers, g.kv_heads, g.k)
