"""bench.py's host-side pieces on the CPU: the arrival plan of the tick loop,
the CPU leg (oracle C step, one thread and every core), and the distinct-block
accounting of the prefix-group roofline.  No device call."""
import os
import sys
import types

import numpy as np
import pytest

from oracle import pyoracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402
import ferry_amd as F  # noqa: E402  (host entry points only)

SMALL = dict(B=6, L=2, Hq=4, Hkv=2, k=8, ctx=(20, 40), C=24, dtype="f16", zipf=1.1,
             reuse=0.66, group=1, prefix=0)


def _args(**kw):
    a = dict(len="4,8", gap_ticks=0.0, mmpp_period=1.0, warmup=3, steps=4, chunks=0,
             host_blocks=257, workers=0, steal=1, no_cpu=False, cpu_reqs=2, cpu_steps=2)
    a.update(kw)
    return types.SimpleNamespace(**a)


def test_lognormal_reuse_range_and_mean():
    r = bench.lognormal_reuse(4096, 64)
    assert r.shape == (4096,) and np.all((r >= 0.0) & (r <= 1.0))
    fresh = (1.0 - r) * 64  # lognormal(2, 1.2) fresh blocks per step, capped at k
    assert abs(np.log(np.median(fresh)) - 2.0) < 0.1  # the median of lognormal(2, s) is e^2
    # the cap at k = 64 takes P(N(2, 1.2) > ln 64) = P(Z > 1.80) = 3.6 % of the requests
    assert fresh.max() <= 64.0 and 0.025 < np.mean(fresh >= 64.0 - 1e-9) < 0.05


def test_distinct_per_set_counts_each_block_once_per_group_set():
    none = 0xFFFFFFFF
    sel = np.array([[[[1, 2, 3]]], [[[3, 2, 9]]], [[[7, none, 7]]]], np.uint32)  # B=3, L=H=1, k=3
    assert list(bench.distinct_per_set(sel, 1)) == [3, 3, 1]
    assert list(bench.distinct_per_set(sel, 2)) == [4, 1]   # {1,2,3,9} and {7}
    assert list(bench.distinct_per_set(sel, 3)) == [5]      # {1,2,3,7,9}
    slots = sel.copy()
    flat = bench.distinct_slots(slots, 2, 3)
    assert flat.size % 3 == 0 and list(flat[:5]) == [1, 2, 3, 9, 7]


@pytest.mark.parametrize("process", ["poisson", "mmpp"])
def test_arrival_plan_is_a_valid_schedule(process):
    a = _args()
    plan, arrive, admit, max_blocks, gap = bench.arrival_plan(a, SMALL, F, 40, 1.1, process, 1.5,
                                                            skew=process == "mmpp")
    B, L, H, k = SMALL["B"], SMALL["L"], SMALL["Hkv"], SMALL["k"]
    assert len(plan) == 40 and gap > 0
    for sel, lanes, resident in plan:
        rows = sel.reshape(B, L * H * k)
        live = rows[:, 0] != O.NONE
        assert live.sum() == resident
        assert np.all((rows[live] < max_blocks) | (rows[live] == O.NONE))
        assert np.all(rows[~live] == O.NONE)  # idle lanes select nothing
        assert np.all((lanes >= 0) & (lanes < B))
    # every admitted request arrived before its admission tick
    got = [(r, admit[r]) for r in range(len(arrive)) if admit[r] >= 0]
    assert got and all(arrive[r] <= t for r, t in got)


def test_cpu_baseline_leg_on_a_small_workload():
    g = O.make_geom(n_req=1, n_layers=1, kv_heads=1, k=1, cap=1, max_blocks=1, dtype=O.F16,
                    host_blocks=257)
    host, _ = O.host_fill(g)
    ctx = O.ctx_uniform(2, SMALL["B"], *SMALL["ctx"])
    plan = bench.cpu_plan(SMALL, ctx, 2, 2, None)
    assert len(plan) == 3
    res = bench.cpu_baseline(SMALL, 64, host, None, 257, 2, plan, "steps")
    assert res["kind"] == "port" and res["cores"] == 1 and res["value"] > 0
    assert res["unit"] == "tok/s" and res["ms_per_step"] > 0
    ac = res["all_cores"]
    assert 1 <= ac["cores"] <= 16 and ac["value"] > 0 and ac["usable_cores"] >= ac["cores"]
    # a plan with a lane reset and an idle lane: resident lanes counted, no failure
    idle = plan[1][0].copy().reshape(2, -1)
    idle[1] = O.NONE
    res = bench.cpu_baseline(SMALL, 64, host, None, 257, 2,
                             [plan[0], (idle.reshape(-1), (0,)), plan[2]], "ticks")
    assert res["value"] > 0


def test_cpu_full_groups_runs_the_whole_batch():
    # a prefix-group workload of 3 groups: every group in an executor of its
    # own; its first group's selections are the sampled leg's (draws are keyed
    # per request), and the whole batch's tokens per step are all requests'
    w = dict(B=48, L=2, Hq=8, Hkv=2, k=8, ctx=(4, 32), C=256, dtype="fp8", zipf=1.1,
             reuse=0.66, group=16, prefix=16)
    ctx = O.ctx_uniform(2, w["B"], *w["ctx"]) + w["prefix"]
    sg = O.selgen(w["B"], w["L"], w["Hkv"], w["k"], ctx, dist=1, zipf_s=w["zipf"],
                  reuse=w["reuse"], group=w["group"], prefix_blocks=w["prefix"], seed=3)
    mb = O.selgen_max_blocks(sg)
    full0 = O.selgen_step(sg, 0).reshape(w["B"], -1)
    plan = bench.cpu_plan(w, ctx, w["group"], 2, None)
    assert np.array_equal(plan[0][0], full0[:w["group"]].reshape(-1))
    g = O.make_geom(n_req=1, n_layers=1, kv_heads=1, k=1, cap=1, max_blocks=1, dtype=O.FP8,
                    host_blocks=4099)
    host, hsc = O.host_fill(g)
    res = bench.cpu_full_groups(w, mb, host, hsc, 4099, ctx, 2, None)
    assert res["kind"] == "port" and res["unit"] == "tok/s" and res["value"] > 0
    assert 1 <= res["cores"] <= 3 and res["ms_per_step"] > 0
    assert "48 requests (3 groups of 16)" in res["sample"]
