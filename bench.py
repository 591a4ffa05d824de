"""Benchmark of the sparse KV miss-stream executor on one MI355X.

One step = one decode step of the whole batch through the executor:
bookkeeping (dedup + LRU slot assignment/eviction, miss-ring push), miss
fetch (persistent workgroups move every missing block from the pinned host
tier into the HBM slot pool over the host link) and block-sparse decode
attention over the selected blocks of every (request, layer, head).

Default workload (the 7B decode shape): 64 requests x 32 layers x 32 heads
(MHA), head_dim 128, fp16 KV, 16-token blocks, contexts uniform in
[4096, 32768] tokens, top-k 64 blocks per head with Zipf(1.1) popularity and
0.66 inter-step reuse, 320 HBM slots per (request, layer, head) set, which
gives ~10% misses in steady state.  Selections and q are generated and
uploaded before the timed region; the host tier is pinned host memory.

The timed steps run ferry_decode_step: layers are cut into --chunks ranges
and the bookkeeping + fetch of range c+1 run on a side stream while range c
attends on the main stream.  By default the count is adaptive: the reference's
batch rule (clamp(pending MB / 8, 32, 512) MB per chunk) on the bytes the
previous step fetched.

Prints ONE JSON line.  `value` is whole-step decode tokens/s (B / step time).
Kernel rates come from HIP events around separate launches of each kernel:
  roofline        attention kernel vs 8 TB/s HBM (algorithmic bytes/launch)
  roofline_fetch  fetch kernel vs the PCIe Gen5 x16 host link (63.0 GB/s)
  roofline_select top-k selection over every context block vs HBM (Quest
                  bound over block summaries)
  roofline_select_mass  the softmax-mass selection over every context token's
                  key vs HBM, where a K table with a record per (set, block)
                  fits in free HBM (gqa128k), else the reason it was skipped
  roofline_handoff export / import of one owner's resident KV vs HBM, with
                  torch's copy and a streaming copy of as many bytes as ceilings
cpu_baseline times the oracle's C restatement of the same step (1 thread) on
2 of the requests (a whole prefix group for grouped workloads), and again on
every usable host core (at most 16) with one replica of those requests per
thread (`cpu_baseline.all_cores`).

Other workloads (--workload): gqa128k (long-context GQA, bf16, ~30% misses),
prefix_fp8 (shared-prefix groups, fp8 + scales, cross-request dedup), skew
(lognormal per-request miss counts; prints a stealing on/off sweep over Zipf
skew with 304 persistent fetch workgroups), small.

Other modes: --arrivals poisson|mmpp (request arrivals and lane turnover
through the tick loop), --queue (the device MPMC ring's push+pop rate, the
reference's bench_queue test, against the ticket rate of one shared word),
--rocprof-summary / --pmc-summary (profile tables).
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "miss-blocks/s + sparse-decode tok/s @7B shape; HBM & host-link GB/s vs peak"
HBM_PEAK_GBS = 8000.0
LINK_PEAK_GBS = 32e9 * 16 * 128 / 130 / 8 / 1e9  # PCIe Gen5 x16, one direction
MMPP_RATIO = 10.0  # fast-state rate / slow-state rate of the Markov-modulated arrivals

WORKLOADS = {
    # 7B-shape steady decode (the headline)
    "7b": dict(B=64, L=32, Hq=32, Hkv=32, k=64, ctx=(256, 2048), C=320, dtype="f16", zipf=1.1,
               reuse=0.66, group=1, prefix=0),
    # long-context GQA, host-tier heavy (~30% misses), bf16
    "gqa128k": dict(B=16, L=32, Hq=32, Hkv=8, k=128, ctx=(8192, 8192), C=128, dtype="bf16",
                    zipf=1.1, reuse=0.66, group=1, prefix=0),
    # shared-prefix agent decode: 8 groups x 16 requests, 8192-token prefix + [512, 4096]
    # private tokens, GQA 32/8, fp8 E4M3 with per-block scales; dedup across the group
    "prefix_fp8": dict(B=128, L=32, Hq=32, Hkv=8, k=64, ctx=(32, 256), C=1536, dtype="fp8",
                       zipf=1.1, reuse=0.66, group=16, prefix=512),
    # skewed per-request miss counts (lognormal(2, 1.2) fresh blocks per step), 7B shape
    "skew": dict(B=64, L=32, Hq=32, Hkv=32, k=64, ctx=(256, 2048), C=320, dtype="f16", zipf=1.0,
                 reuse=0.66, group=1, prefix=0, lognormal=True),
    "small": dict(B=8, L=4, Hq=8, Hkv=8, k=64, ctx=(256, 2048), C=320, dtype="f16", zipf=1.1,
                  reuse=0.66, group=1, prefix=0),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--workload", default="7b", choices=sorted(WORKLOADS))
    ap.add_argument("--host-blocks", type=int, default=1 << 20)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the cpu_baseline leg (the CPU timing and the oracle gate)")
    ap.add_argument("--no-configs", action="store_true",
                    help="7b only: leave out the gqa128k and prefix_fp8 sub-objects")
    ap.add_argument("--cpu-reqs", type=int, default=2)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--steal", type=int, default=1)
    ap.add_argument("--workers", type=int, default=0)
    ap.add_argument("--attn", default="auto", choices=["auto", "valu", "mfma", "group"],
                    help="attention kernel: MFMA for GQA groups of 16/8-bit KV (auto), or forced")
    ap.add_argument("--chunks", type=int, default=0,
                    help="layer chunks of the fetch/attention overlap (1 = no side stream, "
                         "0 = adaptive from the last step's fetched bytes)")
    ap.add_argument("--arrivals", default="none", choices=["none", "poisson", "mmpp"],
                    help="request arrivals instead of a full steady batch: requests wait for a "
                         "lane, decode --len steps and leave (lane reset on admission)")
    ap.add_argument("--len", default="16,48", help="request decode lengths lo,hi (steps)")
    ap.add_argument("--gap-ticks", type=float, default=0.0,
                    help="mean inter-arrival gap in ticks (0: 0.9 of the lanes' service rate)")
    ap.add_argument("--mmpp-period", type=float, default=1.0,
                    help="mean sojourn of each MMPP state, in ticks (rates 1x and 10x)")
    ap.add_argument("--zipf-list", default="0.6,1.0,1.4",
                    help="skew workload: the Zipf exponents swept")
    ap.add_argument("--steal-list", default="0,1", help="skew workload: stealing off/on swept")
    ap.add_argument("--queue", action="store_true",
                    help="the device MPMC ring's push+pop throughput (bench_queue's test) against "
                         "the ticket rate of one shared word")
    ap.add_argument("--rocprof-summary", metavar="DB",
                    help="summarise a rocprofv3 results database instead of benchmarking")
    ap.add_argument("--last", type=int, default=0,
                    help="with --rocprof-summary: also average the last N dispatches per kernel")
    ap.add_argument("--pmc-copy", action="store_true",
                    help="first run a plain 1 GiB device copy (counter calibration)")
    ap.add_argument("--pmc-summary", metavar="CSV",
                    help="summarise a rocprofv3 counter_collection.csv instead of benchmarking")
    return ap.parse_args()


def pmc_summary(csv_path, last):
    """Per-kernel average of each counter over the last N dispatches (markdown)."""
    import csv

    per = {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"].split("(")[0].replace("void ", "")
            key = (name, row["Counter_Name"])
            per.setdefault(key, {})
            did = int(row["Dispatch_Id"])
            per[key][did] = per[key].get(did, 0.0) + float(row["Counter_Value"])
    lines = ["| kernel | counter | dispatches | avg per dispatch (all) | avg (last N) |",
             "|---|---|---|---|---|"]
    for (name, ctr), d in sorted(per.items()):
        vals = [d[k] for k in sorted(d)]
        n = last or len(vals)
        lines.append(f"| `{name}` | {ctr} | {len(vals)} | {np.mean(vals):.1f} | "
                     f"{np.mean(vals[-n:]):.1f} |")
    return "\n".join(lines)


def rocprof_summary(db_path, last):
    """Per-kernel dispatch statistics from a rocprofv3 kernel trace (markdown).

    Two tables: every dispatch of each kernel, and the whole-step dispatches
    only -- those issued after the last k_step_close, i.e. bench.py's
    event-timed steps (bookkeeping, fetch drain and attention of the whole
    batch launched one after the other) and its back-to-back attention
    launches, which are what the bench line's kernel_ms and rooflines are
    computed from.  The pipelined steps before them launch the same kernels
    per layer range."""
    import sqlite3

    if db_path.endswith(".csv"):  # rocprofv3 --output-format csv kernel_trace.csv
        import csv

        with open(db_path) as f:
            rows = sorted(((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]),
                            int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])))
                           for r in csv.DictReader(f)), key=lambda x: x[1])
    else:
        cur = sqlite3.connect(db_path).cursor()
        rows = [(n, a, b, 0) for n, a, b in
                cur.execute("select name, start, end from kernels order by start").fetchall()]

    def short(name):
        return name.split("(")[0].replace("void ", "")

    def table(sel, title, with_last):
        per = {}
        for name, t0, t1, wg in sel:
            per.setdefault((short(name), wg), []).append((t1 - t0) / 1e3)
        lines = [title, "",
                 "| kernel | workgroups | calls | avg us | min us | max us |"
                 + (f" avg us (last {last}) |" if with_last else ""),
                 "|---|---|---|---|---|---|" + ("---|" if with_last else "")]
        for (name, wg), d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            row = (f"| `{name}` | {wg} | {len(d)} | {np.mean(d):.1f} | {min(d):.1f} | "
                   f"{max(d):.1f} |")
            if with_last:
                row += f" {np.mean(d[-last:]):.1f} |"
            lines.append(row)
        return lines

    out = table(rows, "### Every dispatch", bool(last))
    closes = [i for i, r in enumerate(rows) if short(r[0]).endswith("k_step_close")]
    if closes:
        tail = [r for r in rows[closes[-1] + 1:]
                if any(k in short(r[0]) for k in ("k_lru_step", "k_fetch", "k_attn"))]
        # an attention launch right after a fetch drain belongs to an event-timed
        # step; the ones after another attention launch are the back-to-back runs
        timed, b2b = [], []
        for i, r in enumerate(tail):
            if "k_attn" in short(r[0]) and i and "k_attn" in short(tail[i - 1][0]):
                b2b.append(r)
            else:
                timed.append(r)
        out += ["", *table(timed, "### Whole-step dispatches of the event-timed steps (after the "
                                  "last pipelined step; the bench line's kernel_ms)", False)]
        if b2b:
            out += ["", *table(b2b, "### Back-to-back attention launches (kernel_ms."
                                    "attention_back_to_back)", False)]
    return "\n".join(out)


def contexts(F, w):
    """Per-request context lengths (blocks) and the selection generator."""
    lo, hi = w["ctx"]
    ctx = F.ctx_uniform(2, w["B"], lo, hi) + w["prefix"]
    return ctx


def lognormal_reuse(B, k, mu=2.0, sigma=1.2, seed=17):
    """Per-request reuse so that the fresh (re-drawn) blocks of a (request,
    layer, head) per step follow lognormal(mu, sigma), capped at k."""
    z = np.random.default_rng(seed).standard_normal(B)
    fresh = np.minimum(np.exp(mu + sigma * z), k)
    return np.clip(1.0 - fresh / k, 0.0, 1.0)


def cpu_plan(w, ctx, n_req, steps, reuse_r):
    """The sampled requests' selections for a steady cpu_baseline: steps + 1
    steps of the same generator (draws are keyed per request, so requests
    0..n_req-1 draw exactly what they draw in the full batch), no resets."""
    from oracle import pyoracle as O

    sg = O.selgen(n_req, w["L"], w["Hkv"], w["k"], ctx[:n_req], dist=1, zipf_s=w["zipf"],
                  reuse=w["reuse"], group=w["group"], prefix_blocks=w["prefix"], seed=3,
                  reuse_r=None if reuse_r is None else reuse_r[:n_req])
    return [(O.selgen_step(sg, t), ()) for t in range(steps + 1)]


class _CpuRun:
    """One oracle executor with its host pool image, stepping a plan of
    (selections, lanes reset before the step) with ora_cpu_step."""

    def __init__(self, g, host_bytes, host_scales, q):
        from oracle import pyoracle as O

        self.O, self.g, self.q = O, g, q
        self.ex = O.Executor(g)
        bb = O.lib.ora_block_bytes(O.C.byref(g))
        self.host, self.hsc = host_bytes, host_scales
        self.pool = np.zeros(self.ex.n_sets * g.cap * bb, np.uint8)
        self.pscale = (np.zeros(self.ex.n_sets * g.cap * 2, np.float32)
                       if host_scales is not None else None)
        self.out = np.zeros(q.size, np.float32)
        self.slots = np.zeros(g.n_req * g.n_layers * g.kv_heads * g.k, np.uint32)
        self.mc = np.zeros(self.ex.n_sets, np.uint32)
        self.ms = np.zeros(self.ex.n_sets * self.ex.max_sel, O.MISS_DTYPE)
        self.cnt = np.zeros(3, np.uint64)
        self.rc = 0

    def step(self, sel, resets=()):
        for ln in resets:
            self.ex.reset_owner(int(ln))
        rc = self.O.lib.ora_cpu_step(
            self.ex.ptr, sel, self.host.ctypes.data,
            None if self.hsc is None else self.hsc.ctypes.data, self.pool.ctypes.data,
            None if self.pscale is None else self.pscale.ctypes.data, self.q.reshape(-1),
            self.out, self.slots, self.mc, self.ms, self.cnt)
        self.rc = self.rc or rc
        return rc


def cpu_baseline(w, max_blocks, host_bytes, host_scales, host_blocks, n_req, plan, what):
    """The oracle's C step (bookkeeping + memcpy gather + fp32 attention,
    oracle/cpu_step.c) on the first n_req requests of the same workload and
    the same host tier, 1 thread: plan[0] is an untimed cold step, the rest
    are timed.  Then the same on every usable host core (cpu_baseline_threads).
    `what` says what the plan's steps are."""
    from oracle import pyoracle as O

    dt = {"f16": O.F16, "bf16": O.BF16, "fp8": O.FP8, "f32": O.F32}[w["dtype"]]
    L, H, Hq, k, C = w["L"], w["Hkv"], w["Hq"], w["k"], w["C"]
    g = O.make_geom(n_req=n_req, group=w["group"], n_layers=L, kv_heads=H, q_heads=Hq, k=k, cap=C,
                    max_blocks=max_blocks, dtype=dt, host_blocks=host_blocks, seed=7,
                    value_std=0.5)
    q = np.random.default_rng(1).standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    cr = _CpuRun(g, host_bytes, host_scales, q)
    times, misses = [], []
    for t, (sel, resets) in enumerate(plan):  # step 0 is the cold fill, not timed
        t0 = time.perf_counter()
        rc = cr.step(sel, resets)
        dt_s = time.perf_counter() - t0
        if rc:
            raise RuntimeError(f"ora_cpu_step rc={rc}")
        if t:
            times.append(dt_s)
            misses.append(int(cr.cnt[1]))
    steps = len(plan) - 1
    t_step = float(np.mean(times))
    toks = float(np.mean([np.count_nonzero(sel.reshape(n_req, -1)[:, 0] != O.NONE)
                          for sel, _ in plan[1:]]))
    res = {"value": round(toks / t_step, 3), "unit": "tok/s", "cores": 1, "kind": "port",
           "sample": f"oracle C step (bookkeeping + memcpy gather + fp32 attention) on "
                     f"{n_req} of {w['B']} requests x {L} layers x {H} kv heads, {steps} {what} "
                     f"after one untimed one; {t_step * 1e3:.0f} ms/step",
           "miss_blocks_per_s": round(float(np.mean(misses)) / t_step, 1),
           "ms_per_step": round(t_step * 1e3, 1)}
    del cr
    res["all_cores"] = cpu_baseline_threads(g, host_bytes, host_scales, plan, q, toks, what)
    return res


def cpu_baseline_threads(g, host_bytes, host_scales, plan, q, toks, what):
    """The same oracle step on every host core the process may use (at most 16,
    the host share of one GPU): one independent replica of the sampled requests
    per thread, all stepping concurrently (the C calls release the GIL)."""
    import threading

    T = max(1, min(16, len(os.sched_getaffinity(0))))
    reps = [_CpuRun(g, host_bytes, host_scales, q) for _ in range(T)]
    start = threading.Barrier(T + 1)
    done = threading.Barrier(T + 1)

    def worker(r):
        r.step(*plan[0])  # cold fill, untimed
        start.wait()
        for sel, resets in plan[1:]:
            r.step(sel, resets)
        done.wait()

    th = [threading.Thread(target=worker, args=(r,)) for r in reps]
    for t in th:
        t.start()
    start.wait()
    t0 = time.perf_counter()
    done.wait()
    wall = time.perf_counter() - t0
    for t in th:
        t.join()
    if any(r.rc for r in reps):
        raise RuntimeError("ora_cpu_step failed in a worker thread")
    steps = len(plan) - 1
    return {"value": round(T * toks * steps / wall, 3), "unit": "tok/s", "cores": T,
            "host_cores": os.cpu_count(), "usable_cores": len(os.sched_getaffinity(0)),
            "why_not_all": "one GPU's share of the host is 16 cores; the other cores of a "
                           "multi-GPU host belong to the other GPUs' processes"
            if T < (os.cpu_count() or T) else None,
            "sample": f"{T} threads, each an independent replica of the same {g.n_req} requests, "
                      f"{steps} concurrent {what} after one untimed one; "
                      f"{wall / steps * 1e3:.0f} ms per concurrent step",
            "ms_per_step": round(wall / steps * 1e3, 1)}


def cpu_full_groups(w, max_blocks, host_bytes, host_scales, host_blocks, ctx, steps, reuse_r):
    """The oracle's C step over the whole batch of a prefix-group workload:
    every group of w["group"] requests in an executor of its own (a group's
    sets, LRU state, misses and bytes depend on its members' selections only,
    so the groups are independent), the groups spread over the usable host
    cores (at most 16), all stepping the same steps + 1 steps of the full
    batch's selections; step 0 (the cold fill) is untimed."""
    import threading
    from oracle import pyoracle as O

    dt = {"f16": O.F16, "bf16": O.BF16, "fp8": O.FP8, "f32": O.F32}[w["dtype"]]
    B, grp, L, H = w["B"], w["group"], w["L"], w["Hkv"]
    n_groups = B // grp
    sg = O.selgen(B, L, H, w["k"], ctx[:B], dist=1, zipf_s=w["zipf"], reuse=w["reuse"],
                  group=grp, prefix_blocks=w["prefix"], seed=3, reuse_r=reuse_r)
    sels = [O.selgen_step(sg, t).reshape(B, -1) for t in range(steps + 1)]
    g = O.make_geom(n_req=grp, group=grp, n_layers=L, kv_heads=H, q_heads=w["Hq"], k=w["k"],
                    cap=w["C"], max_blocks=max_blocks, dtype=dt, host_blocks=host_blocks, seed=7,
                    value_std=0.5)
    q = np.random.default_rng(1).standard_normal((grp, L, w["Hq"], 128)).astype(np.float32)
    runs = [_CpuRun(g, host_bytes, host_scales, q) for _ in range(n_groups)]
    plans = [[np.ascontiguousarray(sels[t][j * grp:(j + 1) * grp]).reshape(-1)
              for t in range(steps + 1)] for j in range(n_groups)]
    T = max(1, min(16, n_groups, len(os.sched_getaffinity(0))))
    mine = [list(range(i, n_groups, T)) for i in range(T)]
    start = threading.Barrier(T + 1)
    done = threading.Barrier(T + 1)

    def worker(js):
        for j in js:
            runs[j].step(plans[j][0])  # cold fill, untimed
        start.wait()
        for t in range(1, steps + 1):
            for j in js:
                runs[j].step(plans[j][t])
        done.wait()

    th = [threading.Thread(target=worker, args=(js,)) for js in mine]
    for t in th:
        t.start()
    start.wait()
    t0 = time.perf_counter()
    done.wait()
    wall = time.perf_counter() - t0
    for t in th:
        t.join()
    if any(r.rc for r in runs):
        raise RuntimeError("ora_cpu_step failed in a worker thread")
    return {"value": round(B * steps / wall, 3), "unit": "tok/s", "cores": T, "kind": "port",
            "sample": f"the whole batch: {B} requests ({n_groups} groups of {grp}) x {L} layers x "
                      f"{H} kv heads, {steps} steps after one untimed one, each group in an "
                      f"executor of its own, {T} threads; {wall / steps * 1e3:.0f} ms per step",
            "ms_per_step": round(wall / steps * 1e3, 1)}


PREROLL_WINDOW = 5      # steps per window of the settling test
PREROLL_MIN = 20        # at least this many untimed steps from the cold pool
PREROLL_MAX = 200       # and at most this many
PREROLL_TOL = 0.01      # settled: two consecutive windows' miss rates within 1%


def preroll(a, ex, sg, torch, dev, step_fn, gate, q, bufs):
    """Untimed steps from the cold pool until the per-step miss rate settles:
    the mean miss rate of the last window of PREROLL_WINDOW steps is within
    PREROLL_TOL (relative) of the window before it, after at least
    PREROLL_MIN steps.  Selections are drawn one step at a time.  With a gate
    (the oracle replaying the first owners) every step is checked against it.
    Returns the steps run and their miss rates."""
    rates = []
    W = PREROLL_WINDOW
    for t in range(PREROLL_MAX):
        sel = sg.step(t)
        dsel = torch.from_numpy(sel.view(np.int32)).to(dev)
        s0 = ex.stats()
        step_fn(dsel, q)
        torch.cuda.synchronize()
        s1 = ex.stats()
        if s1["device_error"]:
            raise RuntimeError(f"device error {s1['device_error']} in pre-roll step {t}")
        rates.append((s1["misses"] - s0["misses"]) / max(1, s1["selections"] - s0["selections"]))
        if gate is not None:
            gate.step(sel, bufs)
        n = len(rates)
        if n >= max(PREROLL_MIN, 2 * W):
            last, prev = np.mean(rates[-W:]), np.mean(rates[-2 * W:-W])
            if abs(last - prev) <= PREROLL_TOL * max(last, 1e-9):
                break
    return len(rates), rates


def distinct_per_set(sel, group):
    """Distinct selected blocks of every (owner, layer, kv head) set of one step
    (the blocks a group set's members select are read once by the group kernel)."""
    B, L, H, k = sel.shape
    n_own = -(-B // group)
    pad = np.full((n_own * group - B, L, H, k), 0xFFFFFFFF, np.uint32)
    s = np.concatenate([sel, pad]).reshape(n_own, group, L, H, k)
    s = np.sort(s.transpose(0, 2, 3, 1, 4).reshape(n_own * L * H, group * k), axis=1)
    new = np.ones(s.shape, bool)
    new[:, 1:] = s[:, 1:] != s[:, :-1]
    return (new & (s != 0xFFFFFFFF)).sum(axis=1)


def distinct_slots(slots, group, k):
    """The distinct pool slots of every group set of a slot table, set after set,
    padded to whole rows of k by repeating the last one (a cache hit)."""
    B, L, H = slots.shape[0], slots.shape[1], slots.shape[2]
    n_own = -(-B // group)
    out = []
    for o in range(n_own):
        rows = slots[o * group:(o + 1) * group]  # [members][L][H][k]
        for l in range(L):
            for h in range(H):
                u = np.unique(rows[:, l, h].reshape(-1))
                out.append(u[u != 0xFFFFFFFF])
    flat = np.concatenate(out).astype(np.uint32)
    pad = (-flat.size) % k
    return np.concatenate([flat, np.full(pad, flat[-1], np.uint32)])


_SIDE = []


def side_stream(torch):
    """The one side stream of the process (default priority), reused by every
    run: HIP maps a process's streams onto a few hardware queues round-robin,
    and a fresh stream per run can land on the main stream's queue, where the
    fetch and the attention it should overlap run one after the other (a
    config-3 row measured 41.2 ms per step that way against 37.4 ms)."""
    if not _SIDE:
        _SIDE.append(torch.cuda.Stream())
    return _SIDE[0]


def run(a, w, F, torch, steal=None, workers=None, zipf=None, assign=None, want_cpu=True,
        extras=True, steps=None, cpu_steps=None):
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    side = side_stream(torch)
    B, L, H, Hq, k, C = w["B"], w["L"], w["Hkv"], w["Hq"], w["k"], w["C"]
    dtype = {"f16": F.F16, "bf16": F.BF16, "fp8": F.FP8, "f32": F.F32}[w["dtype"]]
    steal = a.steal if steal is None else steal
    workers = a.workers if workers is None else workers
    zipf = w["zipf"] if zipf is None else zipf
    n_timed = a.steps if steps is None else steps
    ctx = contexts(F, w)
    sg = F.SelGen(B, L, H, k, ctx, dist=1, zipf_s=zipf, reuse=w["reuse"], group=w["group"],
                  prefix_blocks=w["prefix"], seed=3)
    reuse_r = None
    if w.get("lognormal"):
        reuse_r = lognormal_reuse(B, k)
        sg.set_reuse(reuse_r)
    qs = [torch.randn((B, L, Hq, 128), device=dev, dtype=torch.float32) for _ in range(2)]
    out = torch.empty_like(qs[0])
    if assign is None:
        assign = F.ASSIGN_AFFINITY if w.get("lognormal") else F.ASSIGN_SPREAD
    attn = {"auto": F.ATTN_AUTO, "valu": F.ATTN_VALU, "mfma": F.ATTN_MFMA,
            "group": F.ATTN_GROUP}[a.attn]
    ex = F.Executor(B, L, H, k, C, sg.max_blocks, q_heads=Hq, group=w["group"], dtype=dtype,
                    host_blocks=a.host_blocks, fetch_workers=workers, steal=steal, assign=assign,
                    attn=attn)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    torch.cuda.synchronize()

    def step_q(sel, q):
        if a.chunks != 1:
            ex.decode_step(sel, q, bufs, out, chunks=a.chunks, stream=stream, side_stream=side)
        else:
            ex.decode_step(sel, q, bufs, out, chunks=1, stream=stream)

    # untimed pre-roll to the steady state; the oracle (the cpu_baseline leg's
    # checker) replays the first owners of the same stream and gates the run
    gate = None
    if not a.no_cpu:
        from oracle.gate import OwnerReplay

        gate = OwnerReplay(n_req=B, group=w["group"], n_layers=L, kv_heads=H, q_heads=Hq, k=k,
                           slots_per_set=C, max_blocks=sg.max_blocks, dtype=dtype,
                           host_blocks=a.host_blocks)
    t0 = time.perf_counter()
    n_pre, pre_rates = preroll(a, ex, sg, torch, dev, step_q, gate, qs[0], bufs)
    gate_res = gate.final(ex, qs[0], out) if gate is not None else None
    pre_s = time.perf_counter() - t0
    n_steps = a.warmup + 2 * n_timed
    t0 = time.perf_counter()
    sels, distinct = [], []
    for t in range(n_steps):
        sel = sg.step(n_pre + t)
        if t >= a.warmup + n_timed:  # the steps whose kernels are timed one by one
            distinct.append(distinct_per_set(sel, w["group"]))
        sels.append(torch.from_numpy(sel.view(np.int32)).to(dev))
    gen_s = time.perf_counter() - t0
    torch.cuda.synchronize()

    def step(t):
        step_q(sels[t], qs[t & 1])

    for t in range(a.warmup):
        step(t)
    torch.cuda.synchronize()
    st0 = ex.stats()
    # timed region: K whole steps, synchronised on both sides; an event on the
    # main stream between steps (a step ends on it) gives each step's duration
    step_ev = [torch.cuda.Event(enable_timing=True) for _ in range(n_timed + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i, t in enumerate(range(a.warmup, a.warmup + n_timed)):
        step_ev[i].record(stream)
        step(t)
    step_ev[n_timed].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_ms = [step_ev[i].elapsed_time(step_ev[i + 1]) for i in range(n_timed)]
    st1 = ex.stats()
    if st1["device_error"]:
        raise RuntimeError(f"device error {st1['device_error']}")
    timed_misses = st1["misses"] - st0["misses"]
    timed_sel = st1["selections"] - st0["selections"]

    # per-kernel durations: K further steps, each kernel bracketed by HIP events
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_timed)]
    m0, s0 = ex.stats()["misses"], ex.stats()["steals"]
    for i in range(n_timed):
        t = a.warmup + n_timed + i
        e = evs[i]
        e[0].record(stream)
        ex.bookkeep_step(sels[t], bufs, flags=False)
        e[1].record(stream)
        ex.missq_drain()
        e[2].record(stream)
        ex.sparse_decode(qs[t & 1], bufs["slots"], out)
        e[3].record(stream)
    torch.cuda.synchronize()
    st2 = ex.stats()
    # attention alone, back to back over the last step's slot table
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record(stream)
    for i in range(n_timed):
        ex.sparse_decode(qs[i & 1], bufs["slots"], out)
    r1.record(stream)
    torch.cuda.synchronize()
    t_attn_rep = r0.elapsed_time(r1) / n_timed
    # top-k selection (Quest bound) over every request's whole context, the
    # step upstream of the miss queue: one launch reads the K summary of every
    # context block of every (request, layer, kv head)
    select = mass = handoff = None
    if extras and w["group"] == 1:
        # one summary record per (set, block): no two blocks share one, so no
        # summary read is served by another block's cache line
        hb = a.host_blocks
        ex.summaries_build(-(-ex.n_sets * sg.max_blocks // hb) * hb, stream)
        dctx = torch.from_numpy(np.ascontiguousarray(ctx, np.int32)).to(dev)
        tsel = torch.empty_like(sels[0])
        ex.select_topk(qs[0], dctx, tsel, stream=stream)
        es0, es1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        es0.record(stream)
        for i in range(n_timed):
            ex.select_topk(qs[i & 1], dctx, tsel, stream=stream)
        es1.record(stream)
        torch.cuda.synchronize()
        t_sel = es0.elapsed_time(es1) / n_timed
        rec = 2 * 128 * F.ESIZE[dtype] + (4 if dtype == F.FP8 else 0)
        sel_bytes = int(ctx.sum()) * L * H * rec + B * L * Hq * 128 * 4 + B * L * H * k * 4
        sel_gbs = sel_bytes / (t_sel * 1e-3) / 1e9
        # ceiling: the same summary records read in the kernel's lane pattern,
        # grid and LDS, no scores (every set's first max(ctx) blocks: the same
        # bytes where contexts are equal); a streaming read's rate on MI355X
        # depends on where the table sits in HBM, so it is measured here
        _, pms, pgbs = ex.bw_probe(F.PROBE_SUMS_READ, int(ctx.max()), iters=3, stream=stream)
        select = {"bound": "hbm", "kernel": f"k_select_topk<{w['dtype']},{Hq // H}>",
                  "ms": round(t_sel, 4), "context_blocks_per_launch": int(ctx.sum()) * L * H,
                  "achieved": round(sel_gbs, 1), "peak": HBM_PEAK_GBS,
                  "unit": "GB/s", "frac": round(sel_gbs / HBM_PEAK_GBS, 4),
                  "plain_read_gbs": round(pgbs, 1), "plain_read_ms": round(pms, 4),
                  "frac_of_plain_read": round(sel_gbs / pgbs, 4)}
        mass = run_mass(a, ex, F, torch, stream, dtype, w, ctx, dctx, qs, sels[0], sg.max_blocks,
                        n_timed)
    # ceilings: plain reads of the same bytes (attention slots; host-tier blocks)
    _, _, gather_gbs = ex.bw_probe(F.PROBE_HBM_GATHER, B * L * H, slots=bufs["slots"],
                                   iters=max(3, n_timed // 2), stream=stream)
    n_host = int(min(a.host_blocks, max(1, (st2["misses"] - m0) // n_timed)))
    _, _, hread_gbs = ex.bw_probe(F.PROBE_HOST_READ, n_host, iters=3, stream=stream)
    _, _, hdma_gbs = ex.bw_probe(F.PROBE_HOST_DMA, n_host, iters=3, stream=stream)
    if extras:
        handoff = run_handoff(a, ex, F, torch, stream, dtype, n_timed)
    ev_misses = st2["misses"] - m0
    t_book = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    t_fetch = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    t_attn = float(np.mean([e[2].elapsed_time(e[3]) for e in evs]))

    sel_per_step = B * L * H * k
    bb = ex.block_bytes
    scale_bytes = 8 if dtype == F.FP8 else 0
    attn_bytes = sel_per_step * (bb + scale_bytes) + 2 * B * L * Hq * 128 * 4 + sel_per_step * 4
    fetch_bytes = ev_misses / n_timed * (bb + scale_bytes)
    ms_step = elapsed / n_timed * 1e3
    attn_gbs = attn_bytes / (t_attn * 1e-3) / 1e9
    link_gbs = fetch_bytes / (t_fetch * 1e-3) / 1e9
    G = Hq // H
    kind, waves = ex.attn_kernel()
    attn_kernel = {F.ATTN_VALU: "k_attn", F.ATTN_MFMA: "k_attn_mfma",
                   F.ATTN_GROUP: "k_attn_group"}[kind] + f"<{w['dtype']},{G}>"
    grouped = None
    if kind == F.ATTN_GROUP:
        # algorithmic bytes of the group kernel: every distinct block of a group
        # set once per launch, plus q in, out and the slot table; the ceiling is
        # a plain gather of the same distinct blocks (last timed step's table)
        n_distinct = float(np.mean([d.sum() for d in distinct]))
        grp_bytes = (n_distinct * (bb + scale_bytes) + 2 * B * L * Hq * 128 * 4
                     + sel_per_step * 4)
        grp_gbs = grp_bytes / (t_attn * 1e-3) / 1e9
        flat = distinct_slots(bufs["slots"].cpu().numpy().view(np.uint32), w["group"], k)
        drows = torch.from_numpy(flat.view(np.int32)).to(dev)
        dbytes, _, dgather_gbs = ex.bw_probe(F.PROBE_HBM_GATHER, flat.size // k, slots=drows,
                                             iters=max(3, n_timed // 2), stream=stream)
        grouped = {"achieved": round(grp_gbs, 1), "frac": round(grp_gbs / HBM_PEAK_GBS, 4),
                   "waves": waves, "distinct_blocks_per_launch": round(n_distinct, 1),
                   "bytes_per_launch": int(grp_bytes),
                   "per_request_bytes_per_launch": int(attn_bytes),
                   "effective_gbs": round(attn_gbs, 1),
                   "plain_gather_distinct_gbs": round(dgather_gbs, 1),
                   "frac_of_plain_gather": round(grp_gbs / dgather_gbs, 4)}
    res = {
        "ms_per_step": round(ms_step, 3),
        "step_ms_p50": round(float(np.percentile(step_ms, 50)), 3),
        "step_ms_p99": round(float(np.percentile(step_ms, 99)), 3),
        "value": round(B / (ms_step * 1e-3), 2),
        "miss_rate": round(timed_misses / max(1, timed_sel), 4),
        "preroll": {"steps": n_pre, "seconds": round(pre_s, 1),
                    "miss_rate_first_window": round(float(np.mean(pre_rates[:PREROLL_WINDOW])), 4),
                    "miss_rate_last_window": round(float(np.mean(pre_rates[-PREROLL_WINDOW:])), 4),
                    "rule": f"untimed steps from the cold pool until two consecutive "
                            f"{PREROLL_WINDOW}-step windows' miss rates agree within "
                            f"{PREROLL_TOL:.0%} (at least {PREROLL_MIN}), then --warmup"},
        "miss_blocks_per_s": round(timed_misses / elapsed, 1),
        "miss_blocks_per_s_fetch_kernel": round(ev_misses / n_timed / (t_fetch * 1e-3), 1),
        "fetched_blocks_per_event_step": round(ev_misses / n_timed, 1),
        "attention_tok_per_s": round(B / (t_attn * 1e-3), 1),
        "kernel_ms": {"bookkeep": round(t_book, 4), "fetch": round(t_fetch, 4),
                      "attention": round(t_attn, 4), "attention_back_to_back": round(t_attn_rep, 4)},
        "roofline": ({"bound": "hbm", "kernel": attn_kernel,
                      "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                      "plain_gather_gbs": round(gather_gbs, 1),
                      "frac_of_plain_gather": round(attn_gbs / gather_gbs, 4)}
                     if grouped is None else
                     {"bound": "hbm", "kernel": attn_kernel, "peak": HBM_PEAK_GBS,
                      "unit": "GB/s", "traffic": None, **grouped}),
        "roofline_fetch": {"bound": "host-link", "kernel": f"k_fetch<{bb // 1024}>",
                           "achieved": round(link_gbs, 2), "peak": round(LINK_PEAK_GBS, 2),
                           "unit": "GB/s", "frac": round(link_gbs / LINK_PEAK_GBS, 4),
                           "plain_read_gbs": round(hread_gbs, 2), "dma_copy_gbs": round(hdma_gbs, 2),
                           "frac_of_plain_read": round(link_gbs / hread_gbs, 4)},
        "roofline_select": select,
        "roofline_select_mass": mass,
        "roofline_handoff": handoff,
        "steals_per_step": round((st2["steals"] - s0) / n_timed, 1),
        "gate": "pass" if gate_res is not None else "skipped (--no-cpu: no oracle leg)",
        "gate_detail": gate_res,
        "selection_gen_s": round(gen_s, 2),
        "config_extra": {"slots_per_set": C, "host_tier_blocks": a.host_blocks,
                         "fetch_workers": ex.cfg.fetch_workers, "steal": steal,
                         "assign": "affinity" if assign == F.ASSIGN_AFFINITY else "spread",
                         "chunks": a.chunks if a.chunks else
                         f"adaptive ({ex.decode_chunks(int(timed_misses / n_timed))})",
                         "zipf": zipf},
    }
    if want_cpu and not a.no_cpu:
        host, hsc = ex.hosttier_array()
        n_req = max(a.cpu_reqs, w["group"])  # a whole prefix group
        plan = cpu_plan(w, ctx, n_req, cpu_steps or a.cpu_steps, reuse_r)
        res["cpu_baseline"] = cpu_baseline(w, sg.max_blocks, host, hsc, a.host_blocks, n_req,
                                           plan, "steps")
        if w["group"] > 1:  # prefix groups: the whole batch, a group per thread
            res["cpu_baseline"]["in_full"] = cpu_full_groups(
                w, sg.max_blocks, host, hsc, a.host_blocks, ctx, cpu_steps or a.cpu_steps, reuse_r)
    ex.close()
    return res


def run_mass(a, ex, F, torch, stream, dtype, w, ctx, dctx, qs, sel0, max_blocks, n_timed):
    """The capture tool's mass selection over every request's whole context:
    one launch reads the K half of every context block of every (request,
    layer, kv head) from a dense K table in HBM.  The table gets one record per
    (set, block), so no two blocks share a record and no read is served by
    another block's cache line; when that table does not fit in free HBM the
    measurement is skipped and says why."""
    B, L, H, Hq, k = w["B"], w["L"], w["Hkv"], w["Hq"], w["k"]
    hb = a.host_blocks
    rec = 16 * 128 * F.ESIZE[dtype]
    n_rec = -(-ex.n_sets * max_blocks // hb) * hb
    free = torch.cuda.mem_get_info()[0]
    if n_rec * rec > 0.85 * free:
        return {"skipped": f"a K table with a record per (set, block) needs {n_rec * rec / 1e9:.0f} GB,"
                           f" {free / 1e9:.0f} GB of HBM free"}
    ex.ktiles_build(n_rec, stream)
    msel = torch.empty_like(sel0)
    ex.select_mass(qs[0], dctx, msel, stream=stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n_timed):
        ex.select_mass(qs[i & 1], dctx, msel, stream=stream)
    e1.record(stream)
    torch.cuda.synchronize()
    assert ex.stats()["device_error"] == 0
    t = e0.elapsed_time(e1) / n_timed
    nb = int(ctx.sum()) * L * H
    nbytes = nb * (rec + (4 if dtype == F.FP8 else 0)) + B * L * Hq * 128 * 4 + B * L * H * k * 4
    G = Hq // H
    kern = (f"k_select_mass<{w['dtype']},{G}>" if dtype == F.F32 else  # 16-bit and fp8 K: two launches
            f"k_mass_units<{w['dtype']},{G}> + k_mass_topk")
    gbs = nbytes / (t * 1e-3) / 1e9
    # ceiling: the same records read in the kernel's order and grid, no scores
    # (every set's first max(ctx) blocks: the same bytes where contexts are equal)
    pbytes, pms, pgbs = ex.bw_probe(F.PROBE_KTAB_READ, int(ctx.max()), iters=3, stream=stream)
    return {"bound": "hbm", "kernel": kern, "ms": round(t, 4),
            "context_blocks_per_launch": nb, "k_table_gb": round(n_rec * rec / 1e9, 1),
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "plain_read_gbs": round(pgbs, 1), "plain_read_ms": round(pms, 4),
            "frac_of_plain_read": round(gbs / pgbs, 4)}


def run_handoff(a, ex, F, torch, stream, dtype, n_timed):
    """Owner hand-off in steady state: export of owner 0's resident KV and LRU
    state into an image, and import of that image into owner 1 (the per-GPU
    halves of moving a request; the image crossing the link is not timed).
    Algorithmic bytes per launch pair: every resident block (and its fp8
    scales) read once and written once; the LRU metadata (about 40 bytes per
    block) is left out of the count."""
    img = ex.alloc_owner_image()
    ex.owner_export(0, img, stream)
    torch.cuda.synchronize()
    resident = int(img[24:32].cpu().numpy().view(np.uint64)[0])
    it = max(3, n_timed // 2)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record(stream)
    for _ in range(it):
        ex.owner_export(0, img, stream)
    ev[1].record(stream)
    for _ in range(it):
        ex.owner_import(1, img, stream)
    ev[2].record(stream)
    torch.cuda.synchronize()
    if ex.stats()["device_error"]:
        raise RuntimeError("owner import refused the exported image")
    t_exp = ev[0].elapsed_time(ev[1]) / it
    t_imp = ev[1].elapsed_time(ev[2]) / it
    per = ex.block_bytes + (8 if dtype == F.FP8 else 0)
    moved = 2 * resident * per
    # ceiling: a plain device-to-device copy of the same number of bytes
    src = img[: resident * per]
    dst = torch.empty_like(src)
    dst.copy_(src)
    ev[0].record(stream)
    for _ in range(it):
        dst.copy_(src)
    ev[1].record(stream)
    torch.cuda.synchronize()
    copy_gbs = moved / (ev[0].elapsed_time(ev[1]) / it * 1e-3) / 1e9
    del img, src, dst
    # and the streaming copy of as many pool blocks (non-temporal loads and stores)
    _, _, nt_copy_gbs = ex.bw_probe(F.PROBE_HBM_COPY, resident, iters=it, stream=stream)
    bb = ex.block_bytes // 1024
    return {"bound": "hbm", "kernel": f"k_owner_export_data<{bb}> + k_owner_import_data<{bb}>",
            "resident_blocks": resident, "image_gb": round(resident * per / 1e9, 3),
            "export_ms": round(t_exp, 4), "import_ms": round(t_imp, 4),
            "export_gbs": round(moved / (t_exp * 1e-3) / 1e9, 1),
            "import_gbs": round(moved / (t_imp * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac_export": round(moved / (t_exp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "frac_import": round(moved / (t_imp * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "plain_copy_gbs": round(copy_gbs, 1), "nt_copy_gbs": round(nt_copy_gbs, 1),
            "frac_of_nt_copy": [round(moved / (t_exp * 1e-3) / 1e9 / nt_copy_gbs, 4),
                                round(moved / (t_imp * 1e-3) / 1e9 / nt_copy_gbs, 4)]}


def arrival_plan(a, w, F, n_ticks, zipf, process, period_ticks, skew):
    """Virtual-clock schedule of an arrival run (one time unit = one tick).
    The first B requests are queued at t=0 with residual lengths so that the
    lanes start full; further requests arrive as a Poisson or Markov-modulated
    Poisson process at 0.9 of the lanes' service rate (the MMPP switches
    between rates 1x and 10x, with exponential sojourns of mean period_ticks).
    Returns per tick the selections, the lanes admitted (their sets are reset)
    and the resident count, plus the per-request arrival/admission ticks."""
    B, L, H, k = w["B"], w["L"], w["Hkv"], w["k"]
    if w["group"] != 1:
        raise SystemExit("arrivals need private sets (group 1): a prefix group's lanes share sets")
    lo_len, hi_len = map(int, a.len.split(","))
    gap = a.gap_ticks or (lo_len + hi_len) / 2.0 / B / 0.9  # mean gap over the run
    n_req = min(65535, B + int(n_ticks / gap * 2) + 16)
    kind = F.ARRIVAL_MMPP if process == "mmpp" else F.ARRIVAL_POISSON
    # the MMPP spends half its time at each rate (equal mean sojourns): its
    # slow-state gap is (1 + ratio) / 2 times the mean gap
    slow_gap = gap * (1 + MMPP_RATIO) / 2 if kind == F.ARRIVAL_MMPP else gap
    arrive = np.concatenate([np.zeros(B), F.arrivals(kind, n_req - B, slow_gap, period_ticks,
                                                     MMPP_RATIO, seed=5)])
    lens = F.ctx_uniform(6, n_req, lo_len, hi_len)
    lens[:B] = F.ctx_uniform(8, B, 1, hi_len)  # residual lengths of the initial batch
    lo, hi = w["ctx"]
    ctxs = F.ctx_uniform(7, n_req, lo, hi)
    sg = F.SelGen(B, L, H, k, np.full(B, hi, np.int32), dist=1, zipf_s=zipf, reuse=w["reuse"],
                  seed=3)
    reuse_req = lognormal_reuse(n_req, k) if skew else None
    lane_reuse = np.full(B, w["reuse"])
    for ln in range(B):
        sg.retire(ln)
    sched = F.Sched(B, arrive, lens)
    plan = []
    for t in range(n_ticks):
        r = sched.tick(float(t))
        for ln in r["retired"]:
            sg.retire(int(ln))
        for ln in r["admitted"]:
            rid = int(r["lane_req"][ln])
            sg.admit(int(ln), rid, int(ctxs[rid]), t)
            if reuse_req is not None:
                lane_reuse[ln] = reuse_req[rid]
        if reuse_req is not None and len(r["admitted"]):
            sg.set_reuse(lane_reuse)
        plan.append((sg.step(t), np.array(r["admitted"], np.int32), r["resident"]))
    admit, _ = sched.request_ticks()
    return plan, arrive, admit, sg.max_blocks, gap


def run_arrivals(a, w, F, torch, process, zipf=None, workers=None, steal=None, skew=False,
                 period_ticks=None, want_cpu=False, cpu_steps=3):
    """Arrival-driven run: warmup ticks (lanes turn over), then --steps timed
    ticks.  Each tick resets the sets of newly admitted lanes on the stream and
    runs one decode step over the resident lanes (idle lanes are empty rows).
    The warmup ticks are gated: the oracle replays the first two lanes (their
    resets included) and every tick their slots and miss lists must be
    bit-equal, then their LRU state, pool bytes and attention (oracle/gate.py).
    An event between timed ticks on the main stream gives each tick's time."""
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    side = side_stream(torch)
    B, L, H, Hq, k, C = w["B"], w["L"], w["Hkv"], w["Hq"], w["k"], w["C"]
    zipf = w["zipf"] if zipf is None else zipf
    period_ticks = a.mmpp_period if period_ticks is None else period_ticks
    lo_len, hi_len = map(int, a.len.split(","))
    warm = max(a.warmup, (lo_len + hi_len) // 2 + 8)
    n_ticks = warm + a.steps
    t0 = time.perf_counter()
    plan, arrive, admit, max_blocks, gap = arrival_plan(a, w, F, n_ticks, zipf, process,
                                                        period_ticks, skew)
    gen_s = time.perf_counter() - t0
    sels = [torch.from_numpy(p[0].view(np.int32)).to(dev) for p in plan]
    adm = [torch.from_numpy(p[1]).to(dev) if len(p[1]) else None for p in plan]
    dtype = {"f16": F.F16, "bf16": F.BF16, "fp8": F.FP8, "f32": F.F32}[w["dtype"]]
    ex = F.Executor(B, L, H, k, C, max_blocks, q_heads=Hq, dtype=dtype, host_blocks=a.host_blocks,
                    fetch_workers=a.workers if workers is None else workers,
                    steal=a.steal if steal is None else steal,
                    assign=F.ASSIGN_AFFINITY if skew else F.ASSIGN_SPREAD)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    qs = [torch.randn((B, L, Hq, 128), device=dev, dtype=torch.float32) for _ in range(2)]
    out = torch.empty_like(qs[0])
    torch.cuda.synchronize()
    gate = None
    if not a.no_cpu:
        from oracle.gate import OwnerReplay

        gate = OwnerReplay(n_req=B, group=1, n_layers=L, kv_heads=H, q_heads=Hq, k=k,
                           slots_per_set=C, max_blocks=max_blocks, dtype=dtype,
                           host_blocks=a.host_blocks)

    def tick(t):
        if adm[t] is not None:
            ex.reset_owners(adm[t], stream=stream)
        ex.decode_step(sels[t], qs[t & 1], bufs, out, chunks=a.chunks, stream=stream,
                       side_stream=side if a.chunks != 1 else None)

    for t in range(warm):
        tick(t)
        if gate is not None:
            torch.cuda.synchronize()
            gate.reset(plan[t][1])
            gate.step(plan[t][0], bufs)
    gate_res = gate.final(ex, qs[(warm - 1) & 1], out) if gate is not None else None
    torch.cuda.synchronize()
    st0 = ex.stats()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(a.steps + 1)]
    t0 = time.perf_counter()
    for i, t in enumerate(range(warm, n_ticks)):
        ev[i].record(stream)
        tick(t)
    ev[a.steps].record(stream)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tick_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(a.steps)]
    st1 = ex.stats()
    if st1["device_error"]:
        raise RuntimeError(f"device error {st1['device_error']}")
    cpu = None
    if want_cpu and not a.no_cpu:
        # the CPU path over the first two lanes of the same plan from its first
        # tick (their own resets included): a cold tick, then cpu_steps ticks
        host, hsc = ex.hosttier_array()
        nr = 2
        cplan = [(np.ascontiguousarray(p[0].reshape(B, -1)[:nr]).reshape(-1),
                  tuple(int(x) for x in p[1] if x < nr)) for p in plan[:cpu_steps + 1]]
        cpu = cpu_baseline(w, max_blocks, host, hsc, a.host_blocks, nr, cplan,
                           "ticks of the plan (ticks 0..%d, resident lanes counted)" % cpu_steps)
    ex.close()
    tokens = sum(p[2] for p in plan[warm:])
    ms_tick = elapsed / a.steps * 1e3
    waited = np.array([admit[r] - arrive[r] for r in range(len(arrive))
                       if warm <= admit[r] < n_ticks and arrive[r] > 0])
    misses = st1["misses"] - st0["misses"]
    sel = st1["selections"] - st0["selections"]
    res = {
        "ms_per_step": round(ms_tick, 3),
        "tick_ms_p50": round(float(np.percentile(tick_ms, 50)), 3),
        "tick_ms_p99": round(float(np.percentile(tick_ms, 99)), 3),
        "value": round(tokens / elapsed, 2),
        "unit": "tok/s",
        "miss_rate": round(misses / max(sel, 1), 4),
        "miss_blocks_per_s": round(misses / elapsed, 1),
        "steals_per_tick": round((st1["steals"] - st0["steals"]) / a.steps, 1),
        "arrivals": {"process": process, "mean_gap_ticks": round(gap, 4),
                     "mean_rate_req_per_s": round(1e3 / (gap * ms_tick), 2),
                     "mmpp_sojourn_ticks": round(period_ticks, 3) if process == "mmpp" else None,
                     "mmpp_sojourn_ms_at_measured_tick": round(period_ticks * ms_tick, 1)
                     if process == "mmpp" else None,
                     "decode_len_steps": [lo_len, hi_len], "warmup_ticks": warm,
                     "timed_ticks": a.steps,
                     "mean_resident_lanes": round(tokens / a.steps, 2), "lanes": B,
                     "admitted_in_timed_ticks": int(sum(len(p[1]) for p in plan[warm:])),
                     "queue_wait_ticks_mean": round(float(waited.mean()), 3) if waited.size else 0.0,
                     "queue_wait_ticks_p99": round(float(np.percentile(waited, 99)), 3)
                     if waited.size else 0.0},
        "gate": "pass (warmup ticks)" if gate_res is not None else "skipped (--no-cpu: no oracle leg)",
        "gate_detail": gate_res,
        "selection_gen_s": round(gen_s, 2),
    }
    if cpu is not None:
        res["cpu_baseline"] = cpu
    return res


def run_queue(F, iters=3):
    """bench_queue's throughput test (src/benches/bench_queue.cu:127-146): P
    producer and C consumer threads move n unique tasks through the ring (1 M
    cells) in one kernel, per-thread and wave-batched reservation, each run
    checked exactly-once.  Every pop takes one compare-and-swap ticket from the
    ring's head word, one compare-and-swap per wavefront for its lanes, so the
    ceiling is the ticket rate of one shared word taken that way by C threads
    (per-thread mode's pushes take one compare-and-swap per thread; fetch-add
    for reference).  Under a per-thread compare-and-swap each success costs
    about one attempt per contending thread, so the runs are sized to ~1-4 M
    tickets."""
    rows = []
    for P, Cn, n, reps in ((512, 512, 1 << 22, iters), (2048, 2048, 1 << 20, 1)):
        ceil = {}
        for kind, name in ((2, "wave_cas"), (1, "thread_cas"), (0, "fetch_add")):
            F.queue_ticket_probe(Cn, 16, kind)  # warm-up
            t, ms = F.queue_ticket_probe(Cn, (1 << 20) // Cn, kind)
            ceil[name] = round(t / (ms * 1e-3) / 1e6, 1)
        print(json.dumps({"threads": Cn, "ticket_ceiling_mops": ceil}), file=sys.stderr, flush=True)
        for mode, mname in ((0, "per-thread"), (1, "wave")):
            tot = 0.0
            for _ in range(reps):
                popped, dups, ms = F.queue_selftest(1 << 20, n, P, Cn, mode)
                assert popped == n and dups == 0
                tot += ms
            mops = n / (tot / reps * 1e-3) / 1e6
            # per-thread mode: pushes take per-thread tickets, pops per-wavefront ones
            bound = ceil["wave_cas"] if mode == 1 else min(ceil["wave_cas"], ceil["thread_cas"])
            rows.append({"producers": P, "consumers": Cn, "tasks": n, "mode": mname,
                         "ms": round(tot / reps, 3), "mops": round(mops, 2),
                         "ticket_ceiling_mops": ceil, "frac_of_ticket_ceiling": round(mops / bound, 4)})
            print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    return {"metric": "device MPMC ring push+pop Mops/s (exactly once)", "unit": "Mops/s",
            "capacity": 1 << 20, "higher_is_better": True, "rows": rows}


def skew_rows(a, F, torch, zipfs, steals, steps, cpu_zipf=None):
    """Config 3 steady: stealing on vs off over the Zipf sweep, 304 persistent
    fetch workgroups with request-affinity assignment, lognormal(2, 1.2)
    fresh blocks per request-step; each row pre-rolled and gated like the
    headline.  With cpu_zipf, the row of that skew also carries the CPU leg
    (the CPU path has no workgroups: one CPU figure serves both steal rows)."""
    w = WORKLOADS["skew"]
    rows, cpu = [], None
    for s in zipfs:
        for steal in steals:
            want = cpu_zipf is not None and s == cpu_zipf and cpu is None
            r = run(a, w, F, torch, steal=steal, workers=304, zipf=s, want_cpu=want,
                    extras=False, steps=steps)
            if want:
                cpu = r.get("cpu_baseline")
            rows.append({"zipf": s, "steal": steal, "ms_per_step": r["ms_per_step"],
                         "step_ms_p50": r["step_ms_p50"], "step_ms_p99": r["step_ms_p99"],
                         "value": r["value"], "unit": "tok/s",
                         "fetch_ms": r["kernel_ms"]["fetch"],
                         "attention_ms": r["kernel_ms"]["attention"],
                         "miss_rate": r["miss_rate"],
                         "link_gbs": r["roofline_fetch"]["achieved"],
                         "link_frac": r["roofline_fetch"]["frac"],
                         "steals_per_step": r["steals_per_step"],
                         "preroll_steps": r["preroll"]["steps"], "gate": r["gate"],
                         "gate_selections_compared": (r["gate_detail"] or {}).get(
                             "selections_compared")})
            print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    return rows, cpu


def run_config1(a, F, torch, ticks=1000, rate_per_s=200.0):
    """Config 1 as stated, in full on the GPU and on the CPU: 1 layer, 8 kv
    heads MHA, fp32 KV, 4 request lanes of 2048-token contexts (128 blocks),
    32 blocks per (request, head) uniform without replacement, 96 slots per
    set (the LRU's steady state misses 25% of selections), a host tier of
    all 4096 blocks, requests arriving by a Poisson process at 200/s on a
    virtual 1 ms tick for 1000 ticks, each decoding U[8, 24] steps.  Every
    tick resets newly admitted lanes and runs bookkeeping, fetch and
    attention for the resident lanes.  The GPU ticks are timed as a whole;
    the same ticks then run through the oracle's C step on one core.  The two
    must agree bit for bit in every tick's slot table and miss counts and in
    the final LRU state, and in the last tick's attention within 2e-3."""
    from oracle import pyoracle as O

    LANES, L, H, K, CTX, C, HB = 4, 1, 8, 32, 128, 96, 4096
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream()
    gap_ms = 1000.0 / rate_per_s
    arrive = F.arrivals(F.ARRIVAL_POISSON, int(ticks / gap_ms * 1.2), gap_ms, seed=11)
    arrive = arrive[arrive < ticks]
    lens = F.ctx_uniform(12, arrive.size, 8, 24)
    sched = F.Sched(LANES, arrive, lens)
    sg = F.SelGen(LANES, L, H, K, np.full(LANES, CTX, np.int32), dist=0, reuse=0.0, seed=13)
    for ln in range(LANES):
        sg.retire(ln)
    plan = []
    for t in range(ticks):
        r = sched.tick(float(t))
        for ln in r["retired"]:
            sg.retire(int(ln))
        for ln in r["admitted"]:
            sg.admit(int(ln), int(r["lane_req"][ln]), CTX, t)
        if r["resident"]:
            plan.append((sg.step(t), np.array(r["admitted"], np.int32), r["resident"]))
        elif len(r["admitted"]):
            raise RuntimeError("a lane was admitted on a tick with no resident request")
    n = len(plan)
    ex = F.Executor(LANES, L, H, K, C, sg.max_blocks, q_heads=H, dtype=F.F32, host_blocks=HB,
                    value_std=1.0)
    ex.hosttier_fill()
    sels = [torch.from_numpy(p[0].view(np.int32)).to(dev) for p in plan]
    adm = [torch.from_numpy(p[1]).to(dev) if len(p[1]) else None for p in plan]
    hist = torch.empty((n,) + tuple(ex.sel_shape), dtype=torch.int32, device=dev)
    hist_mc = torch.empty((n, ex.n_sets), dtype=torch.int32, device=dev)
    bufs = ex.alloc_step_buffers()
    qn = np.random.default_rng(1).standard_normal((LANES, L, H, 128)).astype(np.float32)
    q = torch.from_numpy(qn).to(dev)
    out = torch.empty_like(q)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n):
        ev[i].record(stream)
        if adm[i] is not None:
            ex.reset_owners(adm[i], stream=stream)
        b = dict(bufs, slots=hist[i], miss_count=hist_mc[i])
        ex.decode_step(sels[i], q, b, out, chunks=1, stream=stream)
    ev[n].record(stream)
    torch.cuda.synchronize()
    gpu_s = time.perf_counter() - t0
    st = ex.stats()
    if st["device_error"]:
        raise RuntimeError(f"device error {st['device_error']}")
    tick_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]
    # the CPU path over the same ticks, from the same pinned host tier
    host, _ = ex.hosttier_array()
    g = O.make_geom(n_req=LANES, n_layers=L, kv_heads=H, q_heads=H, k=K, cap=C,
                    max_blocks=sg.max_blocks, dtype=O.F32, host_blocks=HB, seed=7, value_std=1.0)
    cr = _CpuRun(g, host, None, qn)
    cpu_slots = np.empty((n, cr.slots.size), np.uint32)
    cpu_mc = np.empty((n, cr.mc.size), np.uint32)
    cpu_s = 0.0
    for i, (sel, lanes, _) in enumerate(plan):
        t1 = time.perf_counter()
        rc = cr.step(sel, lanes)
        cpu_s += time.perf_counter() - t1
        if rc:
            raise RuntimeError(f"ora_cpu_step rc={rc} at tick {i}")
        cpu_slots[i] = cr.slots
        cpu_mc[i] = cr.mc
    gs = hist.cpu().numpy().view(np.uint32).reshape(n, -1)
    gmc = hist_mc.cpu().numpy().view(np.uint32)
    bad = [i for i in range(n) if not (np.array_equal(gs[i], cpu_slots[i]) and
                                        np.array_equal(gmc[i], cpu_mc[i]))]
    fill, ord_, tag = ex.sets_state()
    ofill, oord, otag = cr.ex.state()
    live = np.arange(C)[None, :] < ofill[:, None]
    state_eq = (np.array_equal(fill, ofill) and np.array_equal(tag, otag)
                and np.array_equal(ord_[live], oord[live]))
    go = out.cpu().numpy().reshape(-1, 128).astype(np.float64)
    co = cr.out.reshape(-1, 128).astype(np.float64)
    den = np.abs(co).max(axis=1)
    rows = den > 0
    att = float((np.abs(go - co).max(axis=1)[rows] / den[rows]).max()) if rows.any() else 0.0
    if bad or not state_eq or not att < 2e-3:
        raise RuntimeError(f"config 1: GPU and CPU differ (ticks {bad[:5]}, state equal "
                           f"{state_eq}, attention {att:.3g})")
    ex.close()
    tokens = sum(p[2] for p in plan)
    sel_total = int(sum(np.count_nonzero(p[0] != O.NONE) for p in plan))
    return {"workload": "config 1: L=1, Hq=Hkv=8, D=128, fp32 KV, 16-token blocks, 4 lanes of "
                        "2048-token contexts, top-k 32 uniform without replacement, 96 slots/set, "
                        f"host tier {HB} blocks, Poisson arrivals {rate_per_s:.0f}/s on a 1 ms "
                        f"virtual tick, decode lengths U[8, 24]",
            "ticks": ticks, "decode_ticks": n, "requests": int(arrive.size),
            "miss_rate": round(int(st["misses"]) / max(1, sel_total), 4),
            "value": round(tokens / gpu_s, 1), "unit": "tok/s",
            "ms_per_tick": round(gpu_s / n * 1e3, 4),
            "tick_ms_p50": round(float(np.percentile(tick_ms, 50)), 4),
            "tick_ms_p99": round(float(np.percentile(tick_ms, 99)), 4),
            "bit_exact": {"ticks_compared": n, "slot_tables_equal": True,
                          "miss_counts_equal": True, "final_lru_state_equal": True,
                          "last_tick_attention_max_rel_diff": float(f"{att:.3g}")},
            "cpu_baseline": {"value": round(tokens / cpu_s, 1), "unit": "tok/s", "cores": 1,
                             "kind": "port", "ms_per_tick": round(cpu_s / n * 1e3, 4),
                             "sample": f"the same {n} decode ticks in full through the oracle's "
                                       f"C step (bookkeeping + memcpy gather + fp32 attention), "
                                       f"one thread: one stream of ticks, each depending on the "
                                       f"last"}}


def main():
    a = parse()
    if a.rocprof_summary:
        print(rocprof_summary(a.rocprof_summary, a.last))
        return
    if a.pmc_summary:
        print(pmc_summary(a.pmc_summary, a.last))
        return
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU (the executor has no multi-GPU path); "
              f"got --gpus {a.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    import ferry_amd as F

    torch.cuda.set_device(0)
    if a.pmc_copy:  # known-size copy: reads and writes exactly 1 GiB
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if a.queue:
        print(json.dumps(run_queue(F)), flush=True)
        return
    w = WORKLOADS[a.workload]
    if a.arrivals != "none":
        if a.workload == "skew":  # the stealing sweep of config 3 under MMPP arrivals
            rows = []
            for zs in map(float, a.zipf_list.split(",")):
                for steal in map(int, a.steal_list.split(",")):
                    r = run_arrivals(a, w, F, torch, a.arrivals, zipf=zs, workers=304,
                                     steal=steal, skew=True)
                    rows.append(dict({"zipf": zs, "steal": steal}, **r))
                    print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
            print(json.dumps({"workload": f"skew+{a.arrivals}", "rows": rows}), flush=True)
            return
        r = run_arrivals(a, w, F, torch, a.arrivals, want_cpu=True)
        print(json.dumps({"metric": "decode tok/s under request arrivals (lane turnover)",
                          "workload": f"{a.workload}+{a.arrivals}", "n_gpus": 1,
                          "steps": a.steps, "dtype": w["dtype"], "data": "synthetic",
                          "higher_is_better": True, **r}), flush=True)
        return
    if a.workload == "skew":
        rows, cpu = skew_rows(a, F, torch, list(map(float, a.zipf_list.split(","))),
                              list(map(int, a.steal_list.split(","))), a.steps)
        print(json.dumps({"workload": "skew", "rows": rows}), flush=True)
        return
    r = run(a, w, F, torch)
    # the other configurations, compact, in the same line
    others = {}
    if a.workload == "7b" and not a.no_configs:
        small = min(a.steps, 10)
        for name, extras, cpu_steps in (("gqa128k", True, None), ("prefix_fp8", False, 2)):
            torch.cuda.empty_cache()
            o = run(a, WORKLOADS[name], F, torch, want_cpu=True, extras=extras, steps=small,
                    cpu_steps=cpu_steps)
            others[name] = {k2: o[k2] for k2 in ("ms_per_step", "step_ms_p50", "step_ms_p99",
                                                  "value", "miss_rate", "miss_blocks_per_s",
                                                  "kernel_ms", "gate")}
            others[name]["unit"] = "tok/s"
            others[name]["steps"] = small
            others[name]["preroll_steps"] = o["preroll"]["steps"]
            others[name]["roofline"] = {k2: o["roofline"][k2] for k2 in
                                        ("kernel", "achieved", "peak", "unit", "frac",
                                         "plain_gather_gbs", "plain_gather_distinct_gbs",
                                         "frac_of_plain_gather", "distinct_blocks_per_launch",
                                         "bytes_per_launch", "effective_gbs")
                                        if k2 in o["roofline"]}
            others[name]["roofline_fetch"] = {k2: o["roofline_fetch"][k2] for k2 in
                                              ("kernel", "achieved", "peak", "unit", "frac",
                                               "plain_read_gbs", "frac_of_plain_read")}
            for k2 in ("roofline_select", "roofline_select_mass", "roofline_handoff",
                       "cpu_baseline"):
                if o.get(k2) is not None:
                    others[name][k2] = o[k2]
            print(json.dumps({name: others[name]}), file=sys.stderr, flush=True)
        # config 3: the stealing sweep, steady
        torch.cuda.empty_cache()
        rows, cpu = skew_rows(a, F, torch, [0.6, 1.0, 1.4], [0, 1], small, cpu_zipf=1.0)
        others["skew"] = {"workload": "config 3, steady: 7B shape, lognormal(2, 1.2) fresh "
                                      "blocks per request-step, 304 persistent fetch workgroups "
                                      "(request affinity), stealing off/on, Zipf swept",
                          "steps": small, "rows": rows}
        if cpu is not None:
            others["skew"]["cpu_baseline"] = dict(cpu, note="the Zipf 1.0 stream; the CPU path "
                                                  "has no fetch workgroups to steal between")
        # config 3 under its arrivals: Markov-modulated (1x / 10x) with mean
        # sojourns of 50 ms.  The tick loop's clock is virtual (a tick per
        # decode step), so the sojourn in ticks is 50 ms over the tick time: a
        # first pass with the steady step of the same row gives the tick time
        # under arrivals, and the reported pass uses that
        steady = {(row["zipf"], row["steal"]): row["ms_per_step"] for row in rows}
        mm = []
        for steal in (0, 1):
            first = run_arrivals(a, WORKLOADS["skew"], F, torch, "mmpp", zipf=1.4, workers=304,
                                 steal=steal, skew=True, period_ticks=50.0 / steady[(1.4, steal)])
            period = 50.0 / first["ms_per_step"]
            o = run_arrivals(a, WORKLOADS["skew"], F, torch, "mmpp", zipf=1.4, workers=304,
                             steal=steal, skew=True, period_ticks=period, want_cpu=steal == 0)
            o["arrivals"]["sojourn_calibration"] = (
                f"50 ms over the {first['ms_per_step']} ms tick of a first pass "
                f"(sojourn {50.0 / steady[(1.4, steal)]:.3f} ticks from the steady step)")
            mm.append(dict({"zipf": 1.4, "steal": steal}, **o))
            print(json.dumps(mm[-1]), file=sys.stderr, flush=True)
        others["skew_mmpp"] = {"workload": "config 3 with Markov-modulated arrivals (rates 1x "
                                           "and 10x, mean sojourn 50 ms of modelled time), Zipf "
                                           "1.4, stealing off/on", "rows": mm}
        if "cpu_baseline" in mm[0]:
            others["skew_mmpp"]["cpu_baseline"] = mm[0].pop("cpu_baseline")
        # config 2 under its Poisson arrivals (lane turnover)
        others["7b_poisson"] = run_arrivals(a, WORKLOADS["7b"], F, torch, "poisson",
                                            want_cpu=True)
        print(json.dumps({"7b_poisson": others["7b_poisson"]}), file=sys.stderr, flush=True)
        # config 1 in full, GPU and CPU
        others["config1"] = run_config1(a, F, torch)
        print(json.dumps({"config1": others["config1"]}), file=sys.stderr, flush=True)
    # HBM traffic per launch is not measured in this run: it comes from two
    # rocprofv3 counter runs of the same workload (FETCH_SIZE, WRITE_SIZE),
    # stored in profiles/traffic.json with the commit each entry was measured at
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    tj = json.load(open(tpath)) if os.path.exists(tpath) else {}
    src = tj.get("measured_at", {})

    def put(obj, key, fields):
        """obj["traffic"] = the stored entry's fields (one field: its value)."""
        if obj is None or obj.get("skipped"):
            return
        e = tj.get(key)
        bare = lambda s: re.sub(r"<[^>]*>", "", s)  # noqa: E731  kernel names without templates
        if e is None or bare(e.get("kernel", "")) != bare(obj.get("kernel", "")):
            obj["traffic"], obj["traffic_source"] = None, None  # no entry for this kernel
            return
        obj["traffic"] = e[fields[0]] if len(fields) == 1 else {f: e[f] for f in fields}
        obj["traffic_source"] = (f"stored counters: profiles/traffic.json[{key}], measured at "
                                 f"commit {e.get('commit', src.get('commit'))} "
                                 f"({src.get('source')})")

    put(r["roofline"], a.workload, ("bytes_per_launch",))
    put(r["roofline_fetch"], a.workload + "_fetch", ("read_bytes", "write_bytes"))
    put(r.get("roofline_select"), a.workload + "_select", ("bytes_per_launch",))
    put(r.get("roofline_select_mass"), a.workload + "_mass", ("bytes_per_launch",))
    put(r.get("roofline_handoff"), a.workload + "_handoff", ("export_bytes", "import_bytes"))
    for name, o in others.items():
        if "roofline" not in o:
            continue
        put(o["roofline"], name, ("bytes_per_launch",))
        put(o["roofline_fetch"], name + "_fetch", ("read_bytes", "write_bytes"))
        put(o.get("roofline_select"), name + "_select", ("bytes_per_launch",))
        put(o.get("roofline_select_mass"), name + "_mass", ("bytes_per_launch",))
        put(o.get("roofline_handoff"), name + "_handoff", ("export_bytes", "import_bytes"))
    lo, hi = w["ctx"]
    desc = (f"B={w['B']}, L={w['L']}, Hq={w['Hq']}, Hkv={w['Hkv']}, D=128, {w['dtype']} KV, "
            f"16-token blocks, ctx {'U[%d,%d]' % (lo * 16, hi * 16) if lo != hi else lo * 16} "
            f"tokens{' + %d shared prefix tokens in groups of %d' % (w['prefix'] * 16, w['group']) if w['group'] > 1 else ''}, "
            f"top-k {w['k']} (Zipf {w['zipf']}, reuse {w['reuse']}), {w['C']} slots/set")
    res = {
        "metric": METRIC,
        "value": r["value"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic",
        "config": dict({"workload": f"{a.workload}: {desc}", "batch": w["B"],
                        "layers": w["L"], "q_heads": w["Hq"], "kv_heads": w["Hkv"],
                        "top_k": w["k"]}, **r.pop("config_extra")),
    }
    for key in ("step_ms_p50", "step_ms_p99", "miss_rate", "preroll", "gate", "gate_detail",
                "miss_blocks_per_s",
                "miss_blocks_per_s_fetch_kernel", "fetched_blocks_per_event_step",
                "attention_tok_per_s", "kernel_ms", "roofline",
                "roofline_fetch", "roofline_select", "roofline_select_mass", "roofline_handoff",
                "steals_per_step", "selection_gen_s", "cpu_baseline"):
        if key in r:
            res[key] = r[key]
    if others:
        res["configs"] = others
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
