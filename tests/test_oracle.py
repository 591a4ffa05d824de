"""The CPU oracle pinned against the reference's golden numbers, a build of the
reference's own generator, and independent restatements (CPU only)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import pyoracle as O

REF_BIN = os.path.join(os.path.dirname(O.__file__), "_ref", "ref_replay")


def test_mt19937_64_known_answer():
    # C++ [rand.predef]: the 10000th output of a default-constructed
    # mt19937_64 (seed 5489) is 9981545732273789042.
    g = O.MT64()
    O.lib.ora_mt64_seed(C.byref(g), 5489)
    for _ in range(9999):
        O.lib.ora_mt64_next(C.byref(g))
    assert O.lib.ora_mt64_next(C.byref(g)) == 9981545732273789042


def test_golden_default_stream():
    # results/wla_7rep_20260930/*.log lines 2-4 (R48 L12 S16 sel64 hot128 seed 42):
    # 589,824 selects, 79,550 misses, hit 0.865, 1242.97 MiB, C-mode 59,863 submits.
    blocks, miss, sel, mis = O.ref_replay(48, 12, 16, 64, 128, 42)
    assert (sel, mis) == (589824, 79550)
    assert round(1.0 - mis / sel, 3) == 0.865
    assert round(mis * 16384 / 2**20, 2) == 1242.97
    ev, rb = O.ref_cmode_runs(48, 12, 16, 64, 128, 16384, blocks, miss, 1.0, 4.0, 4.0)
    assert ev == 59863
    assert rb == mis * 16384  # refill bytes equal across modes B and C


def test_golden_single_gpu_executor():
    # 实验设计.txt:494-495: 57.66 MiB of misses, submits 3690 -> 1227
    # (run_missstream: 4 req x 12 layers x 4 steps, sel 128, hot 8*sel, target 8).
    blocks, miss, sel, mis = O.ref_replay(4, 12, 4, 128, 1024, 42)
    assert mis == 3690
    assert round(mis * 16384 / 2**20, 2) == 57.66
    ev, _ = O.ref_cmode_runs(4, 12, 4, 128, 1024, 16384, blocks, miss, 1.0, 4.0, 8.0)
    assert ev == 1227


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("spec", [(48, 12, 16, 64, 128, 42), (3, 2, 40, 17, 9, 7),
                                  (5, 3, 8, 128, 64, 123456789)])
def test_replay_matches_reference_build(spec, tmp_path):
    R, L, S, sel, hot, seed = spec
    out = tmp_path / "ev.bin"
    res = subprocess.run([REF_BIN, *map(str, spec), str(out)], capture_output=True, text=True,
                         check=True)
    rs, rm = map(int, res.stdout.split())
    raw = out.read_bytes()
    n = R * L * S * sel
    blocks, miss, s, m = O.ref_replay(*spec)
    assert (s, m) == (rs, rm)
    assert np.array_equal(np.frombuffer(raw[:8 * n], np.uint64), blocks)
    assert np.array_equal(np.frombuffer(raw[8 * n:], np.uint8), miss)


def _lru(cap, mb):
    s = O.LRU()
    assert O.lib.ora_lru_init(C.byref(s), cap, mb) == 0
    return s


def _substep(s, x):
    x = np.ascontiguousarray(x, np.uint32)
    n = x.size
    so = np.zeros(max(n, 1), np.uint32)
    mo = np.zeros(max(n, 1), O.MISS_DTYPE)
    nm = C.c_int(0)
    rc = O.lib.ora_lru_substep(C.byref(s), 0, x if n else np.zeros(1, np.uint32), n, so, mo,
                               C.byref(nm), None)
    return rc, so[:n], mo[:nm.value]


def test_serial_lru_equals_deque_lru():
    rng = np.random.default_rng(0)
    for _ in range(150):
        cap, mb, n = int(rng.integers(1, 20)), int(rng.integers(1, 60)), int(rng.integers(1, 300))
        x = rng.integers(0, mb, n).astype(np.uint32)
        ref = np.zeros(n, np.uint8)
        O.lib.ora_deque_lru_run(cap, x, n, ref)
        s = _lru(cap, mb)
        mine = np.array([_substep(s, x[p:p + 1])[2].size for p in range(n)], np.uint8)
        assert np.array_equal(mine, ref)


def test_step_lru_equals_timestamp_lru():
    rng = np.random.default_rng(1)
    for _ in range(200):
        cap, mb = int(rng.integers(1, 40)), int(rng.integers(1, 80))
        s = _lru(cap, mb)
        t = O.TSLRU()
        O.lib.ora_tslru_init(C.byref(t), cap, mb)
        for _ in range(25):
            n = int(rng.integers(0, cap + 3))
            x = rng.integers(0, mb, n).astype(np.uint32)
            rc, so, mo = _substep(s, x)
            if rc == -2:
                break
            so2 = np.zeros(max(n, 1), np.uint32)
            b2 = np.zeros(max(n, 1), np.uint32)
            s2 = np.zeros(max(n, 1), np.uint32)
            nm = C.c_int(0)
            assert O.lib.ora_tslru_step(C.byref(t), x if n else np.zeros(1, np.uint32), n, so2,
                                        b2, s2, C.byref(nm)) == 0
            assert rc == 0 and nm.value == mo.size
            assert np.array_equal(so, so2[:n])
            assert np.array_equal(mo["block"], b2[:nm.value])
            assert np.array_equal(mo["slot"], s2[:nm.value])


def test_step_lru_state_invariants():
    rng = np.random.default_rng(2)
    cap, mb = 24, 100
    s = _lru(cap, mb)
    for _ in range(60):
        x = rng.choice(mb, size=int(rng.integers(1, cap + 1)), replace=False).astype(np.uint32)
        x = np.concatenate([x, x[: len(x) // 3]])  # duplicates hit the in-flight fetch
        rc, so, mo = _substep(s, x)
        assert rc == 0
        # dedup: one fetch per distinct non-resident block, in first-occurrence order
        assert len(set(mo["block"].tolist())) == mo.size
        fill = s.fill
        ordv = np.ctypeslib.as_array(s.ord, shape=(cap,))[:fill]
        tag = np.ctypeslib.as_array(s.tag, shape=(cap,))
        mp = np.ctypeslib.as_array(s.map, shape=(mb,))
        assert sorted(ordv.tolist()) == list(range(fill))
        for v in range(fill):
            assert mp[tag[v]] == v
        assert np.count_nonzero(mp != O.NONE) == fill
        for p, b in enumerate(x):
            assert tag[so[p]] == b
        # the most recently used slots are exactly the ones touched this step
        assert set(ordv[fill - len(set(x.tolist())):].tolist()) == set(so.tolist())


def test_capacity_exceeded_is_an_error():
    s = _lru(4, 50)
    rc, _, _ = _substep(s, np.arange(5, dtype=np.uint32))
    assert rc == -2
    rc, so, mo = _substep(s, np.arange(4, dtype=np.uint32))  # state untouched by the failure
    assert rc == 0 and mo.size == 4


def test_group_dedup_concurrent_misses():
    # 4 requests of one prefix group select the same blocks: one fetch each.
    g = O.make_geom(n_req=4, group=4, n_layers=1, kv_heads=1, k=8, cap=64, max_blocks=64)
    ex = O.Executor(g)
    sel = np.tile(np.arange(8, dtype=np.uint32), 4)
    slots, mc, misses, counts = ex.step(sel)
    assert mc[0] == 8 and counts[1] == 8
    assert np.array_equal(slots.reshape(4, 8), np.tile(slots[:8], (4, 1)))


def test_selgen_properties():
    ctx = O.ctx_uniform(5, 16, 256, 2048)
    sg = O.selgen(16, 2, 4, 64, ctx, dist=1, zipf_s=1.1, reuse=0.66, seed=9)
    prev = None
    kept = []
    for step in range(6):
        sel = O.selgen_step(sg, step).reshape(16, 2, 4, 64)
        assert np.all(np.diff(sel.astype(np.int64), axis=-1) > 0)  # sorted, distinct
        assert np.all(sel < ctx[:, None, None, None])
        if prev is not None:
            kept.append(np.mean([len(np.intersect1d(a, b)) / 64
                                 for a, b in zip(sel.reshape(-1, 64), prev.reshape(-1, 64))]))
        prev = sel
    assert 0.6 < np.mean(kept) < 0.8  # 0.66 kept + fresh draws that hit kept blocks


def test_selgen_zipf_skew_and_uniform():
    ctx = np.full(4, 512, np.int32)
    z = O.selgen(4, 1, 8, 16, ctx, dist=1, zipf_s=1.4, reuse=0.0, seed=2)
    u = O.selgen(4, 1, 8, 16, ctx, dist=0, reuse=0.0, seed=2)
    sz = np.stack([O.selgen_step(z, s).reshape(32, 16) for s in range(40)], 1)  # [row, step, k]
    su = np.stack([O.selgen_step(u, s).reshape(32, 16) for s in range(40)], 1)
    hz = [np.bincount(r.reshape(-1), minlength=512) for r in sz]
    hu = [np.bincount(r.reshape(-1), minlength=512) for r in su]
    # under Zipf the most popular block of a row is drawn nearly every step
    assert np.mean([h.max() for h in hz]) > 35
    assert np.mean([h.max() for h in hu]) < 10
    assert np.mean([np.count_nonzero(h) for h in hu]) > np.mean([np.count_nonzero(h) for h in hz])


def test_selgen_prefix_groups_share_ids():
    ctx = np.array([600, 700, 550, 800], np.int32)
    sg = O.selgen(4, 1, 1, 32, ctx, dist=1, zipf_s=1.0, reuse=0.5, group=4, prefix_blocks=512,
                  seed=4)
    mb = O.selgen_max_blocks(sg)
    assert mb == 512 + 4 * (800 - 512)
    sel = O.selgen_step(sg, 0).reshape(4, 32)
    for m in range(4):
        priv = sel[m][sel[m] >= 512]
        assert np.all((priv >= 512 + m * 288) & (priv < 512 + (m + 1) * 288))
    shared = [set(s[s < 512].tolist()) for s in sel]
    assert len(shared[0] & shared[1] & shared[2] & shared[3]) > 0


def test_codecs_against_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-12, 12, 20000))).astype(np.float32)
    f16 = np.array([O.lib.ora_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(f16, x.astype(np.float16).view(np.uint16))
    bf = np.array([O.lib.ora_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(bf, torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy()
                          .view(np.uint16))
    y = (rng.standard_normal(20000) * 60).astype(np.float32)
    y = y[np.abs(y) < 440]
    e8 = np.array([O.lib.ora_f32_to_e4m3(float(v)) for v in y], np.uint8)
    assert np.array_equal(e8, torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy())
    codes = np.arange(256, dtype=np.uint8)
    dec = np.array([O.lib.ora_e4m3_to_f32(int(c)) for c in codes], np.float32)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(dec[fin], ref[fin]) and np.all(np.isnan(dec[~fin]))


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.BF16, O.FP8])
def test_host_content_statistics(dtype):
    g = O.make_geom(n_req=1, n_layers=1, kv_heads=1, k=1, cap=1, max_blocks=1, dtype=dtype,
                    host_blocks=64, value_std=0.5)
    host, sc = O.host_fill(g)
    bb = O.lib.ora_block_bytes(C.byref(g))
    if dtype == O.F32:
        v = host.view(np.float32).astype(np.float64)
    elif dtype == O.F16:
        v = host.view(np.float16).astype(np.float64)
    elif dtype == O.BF16:
        v = torch.from_numpy(host.view(np.int16).copy()).view(torch.bfloat16).double().numpy()
    else:
        codes = torch.from_numpy(host.copy()).view(torch.float8_e4m3fn).double().numpy()
        per = codes.reshape(64, 2, -1) * sc.reshape(64, 2, 1)
        v = per.reshape(-1)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 0.5) < 0.01
    assert host.size == 64 * bb


def _gather_kv(g, set_id, blocks):
    T, D = g.block_tokens, g.head_dim
    ks, vs = [], []
    for b in blocks:
        h = O.host_index(g, set_id, int(b))
        raw, sc = O.host_block(g, h)
        if g.dtype == O.F16:
            v = raw.view(np.float16).astype(np.float64)
        elif g.dtype == O.F32:
            v = raw.view(np.float32).astype(np.float64)
        elif g.dtype == O.BF16:
            v = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16).double().numpy()
        else:
            v = torch.from_numpy(raw.copy()).view(torch.float8_e4m3fn).double().numpy()
        v = v.reshape(2, T, D)
        ks.append(v[0] * sc[0])
        vs.append(v[1] * sc[1])
    return np.concatenate(ks), np.concatenate(vs)


@pytest.mark.parametrize("dtype,hq,hk", [(O.F16, 2, 2), (O.BF16, 8, 2), (O.FP8, 4, 1), (O.F32, 2, 1)])
def test_attention_f64_against_numpy(dtype, hq, hk):
    B, L, k = 2, 2, 5
    g = O.make_geom(n_req=B, n_layers=L, kv_heads=hk, q_heads=hq, k=k, cap=8, max_blocks=40,
                    dtype=dtype, host_blocks=97)
    rng = np.random.default_rng(4)
    sel = np.stack([rng.choice(40, k, replace=False) for _ in range(B * L * hk)]).astype(np.uint32)
    q = rng.standard_normal((B, L, hq, 128)).astype(np.float32)
    out = O.attention_f64(g, sel, q)
    grp = hq // hk
    for r in range(B):
        for l in range(L):
            for hh in range(hq):
                h = hh // grp
                K, V = _gather_kv(g, (r * L + l) * hk + h, sel[(r * L + l) * hk + h])
                s = K @ q[r, l, hh].astype(np.float64) / np.sqrt(128)
                p = np.exp(s - s.max())
                ref = (p / p.sum()) @ V
                assert np.allclose(out[r, l, hh], ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.FP8])
def test_attention_hidx_rows_against_numpy(dtype):
    # rows that name host blocks directly: a repeated block counts twice, a
    # block of another set is just another block, empty positions are skipped
    B, L, hk, hq, k = 2, 1, 2, 4, 6
    g = O.make_geom(n_req=B, n_layers=L, kv_heads=hk, q_heads=hq, k=k, cap=8, max_blocks=40,
                    dtype=dtype, host_blocks=97)
    rng = np.random.default_rng(11)
    rows = [[(0, 3), (0, 3), (0, 9), (1, 22), None, (0, 9)],
            [None] * k,
            [(1, 5), None, (3, 5), (3, 5), (3, 5), (2, 39)],
            [(2, 0), (0, 0), (1, 0), (3, 0), (2, 0), None]]
    hidx = np.full((B * L * hk, k), O.NONE64, np.uint64)
    for r, row in enumerate(rows):
        for j, e in enumerate(row):
            if e is not None:
                hidx[r, j] = O.host_index(g, *e)
    q = rng.standard_normal((B, L, hq, 128)).astype(np.float32)
    out = O.attention_hidx_f64(g, hidx, q)
    grp = hq // hk
    for r in range(B):
        for hh in range(hq):
            row = rows[r * hk + hh // grp]
            picked = [e for e in row if e is not None]
            if not picked:
                assert np.all(out[r, 0, hh] == 0.0)
                continue
            kv = [_gather_kv(g, s, [b]) for s, b in picked]
            K = np.concatenate([a for a, _ in kv])
            V = np.concatenate([b for _, b in kv])
            s = K @ q[r, 0, hh].astype(np.float64) / np.sqrt(128)
            p = np.exp(s - s.max())
            assert np.allclose(out[r, 0, hh], (p / p.sum()) @ V, rtol=1e-12, atol=1e-12)
    # named through the block ids of the rows' own sets, it is attention_f64
    sel = np.stack([rng.choice(40, k, replace=False) for _ in range(B * L * hk)]).astype(np.uint32)
    sel[1, 2] = O.NONE
    own = np.full_like(hidx, O.NONE64)
    for r in range(B * L * hk):
        for j in range(k):
            if sel[r, j] != O.NONE:
                own[r, j] = O.host_index(g, r, int(sel[r, j]))
    assert np.array_equal(O.attention_hidx_f64(g, own, q), O.attention_f64(g, sel, q))
    # a row that names one block twice attends exactly as one naming it once
    one = np.full_like(hidx, O.NONE64)
    two = np.full_like(hidx, O.NONE64)
    one[:, 0] = own[:, 0]
    two[:, 0] = two[:, 3] = own[:, 0]
    assert np.allclose(O.attention_hidx_f64(g, one, q), O.attention_hidx_f64(g, two, q),
                       rtol=1e-13, atol=1e-13)


def _decode_raw(dtype, raw):
    if dtype == O.F16:
        return raw.view(np.float16).astype(np.float64)
    if dtype == O.F32:
        return raw.view(np.float32).astype(np.float64)
    if dtype == O.BF16:
        return torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16).double().numpy()
    return torch.from_numpy(raw.copy()).view(torch.float8_e4m3fn).double().numpy()


@pytest.mark.parametrize("dtype", [O.F16, O.FP8])
def test_attention_tier_image_against_numpy(dtype):
    # the attention over a caller's tier image: equal to the generated-content
    # attention while the image is ora_host_fill's, and to a numpy softmax over
    # the image's own bytes and scales after they are rewritten (fp8 V scales
    # spread over 1e-3..1e3, some zero, some blocks all zero)
    B, L, hk, hq, k = 2, 1, 2, 4, 6
    g = O.make_geom(n_req=B, n_layers=L, kv_heads=hk, q_heads=hq, k=k, cap=8, max_blocks=40,
                    dtype=dtype, host_blocks=53)
    bb = O.lib.ora_block_bytes(C.byref(g))
    host, sc = O.host_fill(g)
    rng = np.random.default_rng(12)
    hidx = rng.integers(0, 53, (B * L * hk, k)).astype(np.uint64)
    hidx[1, 2] = O.NONE64
    q = rng.standard_normal((B, L, hq, 128)).astype(np.float32)
    assert np.array_equal(O.attention_tier_f64(g, hidx, host, sc if dtype == O.FP8 else None, q),
                          O.attention_hidx_f64(g, hidx, q))
    host = host.copy()
    blocks = host.reshape(53, bb)
    blocks[5] = rng.integers(0, 256, bb, dtype=np.uint8) & 0x77  # finite fp8 codes and f16s
    if dtype == O.FP8:
        sc = sc.copy().reshape(53, 2)
        sc[:, 1] *= 10.0 ** rng.uniform(-3, 3, 53)
        sc[7, 1] = 0.0
        sc[9, 0] = 0.0
        blocks[11, bb // 2:] = 0
        sc[11, 1] = 1e3
        hidx[0, 0], hidx[0, 1], hidx[2, 0], hidx[3, 3] = 11, 7, 9, 5
    else:
        hidx[0, 0] = 5
    out = O.attention_tier_f64(g, hidx, host, sc.reshape(-1) if dtype == O.FP8 else None, q)
    T, D, grp = g.block_tokens, g.head_dim, hq // hk
    for r in range(B):
        for hh in range(hq):
            row = hidx[r * hk + hh // grp]
            picked = [int(b) for b in row if b != O.NONE64]
            kv = [_decode_raw(dtype, blocks[b]).reshape(2, T, D) for b in picked]
            ks = [sc[b, 0] if dtype == O.FP8 else 1.0 for b in picked]
            vs = [sc[b, 1] if dtype == O.FP8 else 1.0 for b in picked]
            K = np.concatenate([a[0] * s for a, s in zip(kv, ks)])
            V = np.concatenate([a[1] * s for a, s in zip(kv, vs)])
            s_ = K @ q[r, 0, hh].astype(np.float64) / np.sqrt(128)
            p = np.exp(s_ - s_.max())
            assert np.allclose(out[r, 0, hh], (p / p.sum()) @ V, rtol=1e-12, atol=1e-12)
    with pytest.raises(RuntimeError):
        if dtype == O.FP8:
            O.attention_tier_f64(g, hidx, host, None, q)  # fp8 needs the scales
        else:
            raise RuntimeError("f16 needs none")


def test_attention_special_cases():
    g = O.make_geom(n_req=1, n_layers=1, kv_heads=1, k=3, cap=4, max_blocks=8, dtype=O.F32,
                    host_blocks=16)
    sel = np.array([1, 4, 6], np.uint32)
    q0 = np.zeros((1, 1, 1, 128), np.float32)
    out = O.attention_f64(g, sel, q0)  # q = 0: uniform weights -> mean of V
    _, V = _gather_kv(g, 0, sel)
    assert np.allclose(out[0, 0, 0], V.mean(0), atol=1e-12)
    # one dominant key: the output tends to that token's value
    K, V = _gather_kv(g, 0, sel)
    qd = (K[17] * 400.0).astype(np.float32).reshape(1, 1, 1, 128)
    out = O.attention_f64(g, sel, qd)
    assert np.allclose(out[0, 0, 0], V[17], atol=1e-6)


def test_cpu_step_matches_f64():
    B, L, H, k = 2, 2, 2, 6
    g = O.make_geom(n_req=B, n_layers=L, kv_heads=H, q_heads=H * 2, k=k, cap=8, max_blocks=30,
                    dtype=O.BF16, host_blocks=200)
    ex = O.Executor(g)
    host, hs = O.host_fill(g)
    bb = O.lib.ora_block_bytes(C.byref(g))
    nslots = ex.n_sets * g.cap
    pool = np.zeros(nslots * bb, np.uint8)
    ps = np.zeros(nslots * 2, np.float32)
    rng = np.random.default_rng(5)
    for step in range(3):
        sel = np.stack([rng.choice(30, k, replace=False) for _ in range(B * L * H)]).astype(np.uint32)
        q = rng.standard_normal((B, L, 2 * H, 128)).astype(np.float32)
        out = np.zeros(q.size, np.float32)
        slots = np.zeros(sel.size, np.uint32)
        mc = np.zeros(ex.n_sets, np.uint32)
        ms = np.zeros(ex.n_sets * ex.max_sel, O.MISS_DTYPE)
        cnt = np.zeros(3, np.uint64)
        rc = O.lib.ora_cpu_step(ex.ptr, sel.reshape(-1), host.ctypes.data, hs.ctypes.data,
                                pool.ctypes.data, ps.ctypes.data, q.reshape(-1), out, slots, mc,
                                ms, cnt)
        assert rc == 0
        ref = O.attention_f64(g, sel, q).reshape(-1, 128)
        o = out.reshape(-1, 128)
        rel = np.abs(o - ref).max(axis=1) / np.abs(ref).max(axis=1)
        assert rel.max() < 1e-4
