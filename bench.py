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

Prints ONE JSON line.  `value` is whole-step decode tokens/s (B / step time).
Kernel rates come from HIP events on the executor's stream:
  roofline        attention kernel vs 8 TB/s HBM (algorithmic bytes/launch)
  roofline_fetch  fetch kernel vs the PCIe Gen5 x16 host link (63.0 GB/s)
cpu_baseline times the oracle's C restatement of the same step (1 thread) on
2 of the 64 requests.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "miss-blocks/s + sparse-decode tok/s @7B shape; HBM & host-link GB/s vs peak"
HBM_PEAK_GBS = 8000.0
LINK_PEAK_GBS = 32e9 * 16 * 128 / 130 / 8 / 1e9  # PCIe Gen5 x16, one direction

WORKLOADS = {
    # name: (B, L, Hkv, Hq, k, ctx_lo_blocks, ctx_hi_blocks, slots_per_set, dtype, zipf, reuse)
    "7b": (64, 32, 32, 32, 64, 256, 2048, 320, "f16", 1.1, 0.66),
    "small": (8, 4, 8, 8, 64, 256, 2048, 320, "f16", 1.1, 0.66),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--workload", default="7b", choices=sorted(WORKLOADS))
    ap.add_argument("--host-blocks", type=int, default=1 << 20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the cpu_baseline leg")
    ap.add_argument("--cpu-reqs", type=int, default=2)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--steal", type=int, default=1)
    ap.add_argument("--workers", type=int, default=0)
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
    """Per-kernel dispatch statistics from a rocprofv3 database (markdown)."""
    import sqlite3

    if db_path.endswith(".csv"):  # rocprofv3 --output-format csv kernel_trace.csv
        import csv

        with open(db_path) as f:
            rows = sorted(((r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                           for r in csv.DictReader(f)), key=lambda x: x[1])
    else:
        cur = sqlite3.connect(db_path).cursor()
        rows = cur.execute("select name, start, end from kernels order by start").fetchall()
    per = {}
    for name, t0, t1 in rows:
        per.setdefault(name.split("(")[0].replace("void ", ""), []).append((t1 - t0) / 1e3)
    lines = ["| kernel | calls | avg us (all) | min us | max us |"
             + (f" avg us (last {last}) |" if last else ""),
             "|---|---|---|---|---|" + ("---|" if last else "")]
    for name, d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        row = f"| `{name}` | {len(d)} | {np.mean(d):.1f} | {min(d):.1f} | {max(d):.1f} |"
        if last:
            row += f" {np.mean(d[-last:]):.1f} |"
        lines.append(row)
    return "\n".join(lines)


def cpu_baseline(B, L, H, Hq, k, ctx, C, max_blocks, sg_seed, zipf, reuse, host_bytes,
                 host_blocks, n_req, steps):
    """Oracle C path (bookkeeping + memcpy gather + fp32 attention), 1 thread,
    on the first n_req requests of the same workload and the same host tier."""
    import ctypes as Cty
    from oracle import pyoracle as O

    g = O.make_geom(n_req=n_req, n_layers=L, kv_heads=H, q_heads=Hq, k=k, cap=C,
                    max_blocks=max_blocks, dtype=O.F16, host_blocks=host_blocks, seed=7,
                    value_std=0.5)
    ex = O.Executor(g)
    sg = O.selgen(n_req, L, H, k, ctx[:n_req], dist=1, zipf_s=zipf, reuse=reuse, seed=sg_seed)
    bb = O.lib.ora_block_bytes(Cty.byref(g))
    pool = np.zeros(ex.n_sets * C * bb, np.uint8)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((n_req, L, Hq, 128)).astype(np.float32)
    out = np.zeros(q.size, np.float32)
    slots = np.zeros(n_req * L * H * k, np.uint32)
    mc = np.zeros(ex.n_sets, np.uint32)
    ms = np.zeros(ex.n_sets * ex.max_sel, O.MISS_DTYPE)
    cnt = np.zeros(3, np.uint64)
    times, misses = [], []
    for t in range(steps + 1):  # step 0 is the cold fill, not timed
        sel = O.selgen_step(sg, t)
        t0 = time.perf_counter()
        rc = O.lib.ora_cpu_step(ex.ptr, sel, host_bytes.ctypes.data, None, pool.ctypes.data,
                                None, q.reshape(-1), out, slots, mc, ms, cnt)
        dt = time.perf_counter() - t0
        if rc:
            raise RuntimeError(f"ora_cpu_step rc={rc}")
        if t:
            times.append(dt)
            misses.append(int(cnt[1]))
    t_step = float(np.mean(times))
    return {"value": round(n_req / t_step, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"oracle C step (bookkeeping + memcpy gather + fp32 attention) on "
                      f"{n_req} of {B} requests x {L} layers x {H} heads, {steps} steps after "
                      f"one untimed cold step; {t_step * 1e3:.0f} ms/step",
            "miss_blocks_per_s": round(float(np.mean(misses)) / t_step, 1),
            "ms_per_step": round(t_step * 1e3, 1)}


def main():
    a = parse()
    if a.rocprof_summary:
        print(rocprof_summary(a.rocprof_summary, a.last))
        return
    if a.pmc_summary:
        print(pmc_summary(a.pmc_summary, a.last))
        return
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU (this build has no multi-GPU path); "
              f"got --gpus {a.gpus}", file=sys.stderr)
        sys.exit(2)
    import torch

    import ferry_amd as F

    B, L, H, Hq, k, clo, chi, C, dts, zipf, reuse = WORKLOADS[a.workload]
    dtype = {"f16": F.F16, "bf16": F.BF16, "fp8": F.FP8, "f32": F.F32}[dts]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream()
    if a.pmc_copy:  # known-size copy: reads and writes exactly 1 GiB
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    ctx = F.ctx_uniform(2, B, clo, chi)
    sg = F.SelGen(B, L, H, k, ctx, dist=1, zipf_s=zipf, reuse=reuse, seed=3)
    n_steps = a.warmup + a.steps
    t0 = time.perf_counter()
    sels = [torch.from_numpy(sg.step(t).view(np.int32)).to(dev) for t in range(n_steps)]
    gen_s = time.perf_counter() - t0
    qs = [torch.randn((B, L, Hq, 128), device=dev, dtype=torch.float32) for _ in range(2)]
    out = torch.empty_like(qs[0])

    ex = F.Executor(B, L, H, k, C, sg.max_blocks, q_heads=Hq, dtype=dtype,
                    host_blocks=a.host_blocks, fetch_workers=a.workers, steal=a.steal)
    ex.hosttier_fill()
    bufs = ex.alloc_step_buffers()
    torch.cuda.synchronize()

    def step(t, ev=None):
        if ev is not None:
            ev[0].record(stream)
        ex.bookkeep_step(sels[t], bufs, flags=False)
        if ev is not None:
            ev[1].record(stream)
        ex.missq_drain()
        if ev is not None:
            ev[2].record(stream)
        ex.sparse_decode(qs[t & 1], bufs["slots"], out)
        if ev is not None:
            ev[3].record(stream)

    for t in range(a.warmup):
        step(t)
    torch.cuda.synchronize()
    st0 = ex.stats()
    # timed region: K whole steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(a.warmup, n_steps):
        step(t)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    st1 = ex.stats()
    if st1["device_error"]:
        raise RuntimeError(f"device error {st1['device_error']}")
    timed_misses = st1["misses"] - st0["misses"]

    # per-kernel durations: the same steps again would change the LRU state, so
    # time K further steps with events between the launches
    extra = [torch.from_numpy(sg.step(n_steps + i).view(np.int32)).to(dev) for i in range(a.steps)]
    sels.extend(extra)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(a.steps)]
    miss_before = ex.stats()["misses"]
    for i in range(a.steps):
        step(n_steps + i, evs[i])
    torch.cuda.synchronize()
    ev_misses = ex.stats()["misses"] - miss_before
    t_book = np.mean([e[0].elapsed_time(e[1]) for e in evs])
    t_fetch = np.mean([e[1].elapsed_time(e[2]) for e in evs])
    t_attn = np.mean([e[2].elapsed_time(e[3]) for e in evs])

    sel_per_step = B * L * H * k
    bb = ex.block_bytes
    attn_bytes = sel_per_step * bb + 2 * B * L * Hq * 128 * 4 + sel_per_step * 4
    fetch_bytes = ev_misses / a.steps * bb
    ms_step = elapsed / a.steps * 1e3
    attn_gbs = attn_bytes / (t_attn * 1e-3) / 1e9
    link_gbs = fetch_bytes / (t_fetch * 1e-3) / 1e9

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("attention_bytes_per_launch")

    res = {
        "metric": METRIC,
        "value": round(B / (ms_step * 1e-3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dts,
        "data": "synthetic",
        "config": {
            "workload": f"7B-shape steady decode ({a.workload}): B={B}, L={L}, Hq={Hq}, Hkv={H}, "
                        f"D=128, {dts} KV, 16-token blocks, ctx U[{clo * 16},{chi * 16}] tokens, "
                        f"top-k {k} (Zipf {zipf}, reuse {reuse}), {C} slots/set",
            "batch": B, "layers": L, "q_heads": Hq, "kv_heads": H, "top_k": k,
            "slots_per_set": C, "host_tier_blocks": a.host_blocks,
            "fetch_workers": ex.cfg.fetch_workers, "steal": a.steal,
        },
        "miss_rate": round(timed_misses / (a.steps * sel_per_step), 4),
        "miss_blocks_per_s": round(timed_misses / elapsed, 1),
        "miss_blocks_per_s_fetch_kernel": round(ev_misses / a.steps / (t_fetch * 1e-3), 1),
        "attention_tok_per_s": round(B / (t_attn * 1e-3), 1),
        "kernel_ms": {"bookkeep": round(float(t_book), 4), "fetch": round(float(t_fetch), 4),
                      "attention": round(float(t_attn), 4)},
        "roofline": {"bound": "hbm", "kernel": "k_attn<f16,1>", "achieved": round(attn_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
        "roofline_fetch": {"bound": "host-link", "kernel": "k_fetch<8>",
                           "achieved": round(link_gbs, 2), "peak": round(LINK_PEAK_GBS, 2),
                           "unit": "GB/s", "frac": round(link_gbs / LINK_PEAK_GBS, 4)},
        "selection_gen_s": round(gen_s, 2),
    }
    if not a.no_cpu:
        host, _ = ex.hosttier_array()
        res["cpu_baseline"] = cpu_baseline(B, L, H, Hq, k, ctx, C, sg.max_blocks, 3, zipf, reuse,
                                           host, a.host_blocks, min(a.cpu_reqs, B), a.cpu_steps)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
