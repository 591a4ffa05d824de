"""Correctness gate of a running GPU executor: the oracle replays its first
owners from the same cold start and every step is compared with the GPU's.

TEST INFRASTRUCTURE ONLY: used by tests/ and by the cpu_baseline leg of
bench.py, to check the GPU against.  The product never imports it.

Sets belong to one owner (a request, or a prefix group of `group` requests)
and selection draws are keyed per request, so owners [0, n) of a batch of B
requests evolve exactly as a batch of only their n*group requests would: the
oracle executor of that smaller batch has the same set ids, slot ids, block ids
and host-tier content.  Per step the gate requires bit-equal:
  * the pool slot of every selection of those requests;
  * every set's miss list (block, slot, evicted block, set) in miss order;
and at the end (`final`):
  * every set's LRU state (fill, order, tags);
  * the bytes (and fp8 scales) of the slots fetched in the last step, and of
    every resident slot of the first and last layer, against the host tier;
  * attention of those requests in three layers within the relative tolerance
    of the dtype (2e-3; fp8 1e-2) of the float64 oracle, row error =
    max|out - ref| / max|ref|.
These are the checks the reference's own drivers make on their structure
before reporting (src/benches/run_wla_multigpu.cu:607-623, 687-706), extended
to the block bytes and the attention this path adds.
"""
import numpy as np

from oracle import pyoracle as O


class GateError(AssertionError):
    pass


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


class OwnerReplay:
    def __init__(self, *, n_req, group, n_layers, kv_heads, q_heads, k, slots_per_set, max_blocks,
                 dtype, host_blocks, host_seed=7, value_std=0.5, n_owners=None):
        self.group = group
        self.n_owners = n_owners or max(1, 2 // group)
        self.nr = min(n_req, self.n_owners * group)
        self.L, self.H, self.Hq, self.k, self.C = n_layers, kv_heads, q_heads, k, slots_per_set
        self.dtype = dtype
        self.g = O.make_geom(n_req=self.nr, group=group, n_layers=n_layers, kv_heads=kv_heads,
                             q_heads=q_heads, k=k, cap=slots_per_set, max_blocks=max_blocks,
                             dtype=dtype, host_blocks=host_blocks, seed=host_seed,
                             value_std=value_std)
        self.ox = O.Executor(self.g)
        self.n_sets = self.ox.n_sets
        self.steps = 0
        self.selections = 0
        self.misses = 0
        self.last_sel = None
        self.last_misses = None

    def reset(self, owners):
        """Owners whose sets the executor reset before the next step (a new
        request took the lane): the replayed ones start empty too."""
        for o in owners:
            if int(o) < self.n_owners:
                self.ox.reset_owner(int(o))

    def step(self, sel, bufs):
        """sel: the step's [B, L, Hkv, k] block ids (numpy, uint32 view); bufs:
        the executor's step buffers after the step ran (synchronised)."""
        s = np.ascontiguousarray(sel.reshape(-1, self.L, self.H, self.k)[: self.nr])
        oslots, omc, oms, _ = self.ox.step(s)
        gslots = _u32(bufs["slots"][: self.nr]).reshape(-1)
        t = self.steps
        if not np.array_equal(gslots, oslots):
            bad = int(np.nonzero(gslots != oslots)[0][0])
            raise GateError(f"step {t}: slot of selection {bad} is {gslots[bad]}, oracle {oslots[bad]}")
        gmc = _u32(bufs["miss_count"][: self.n_sets])
        if not np.array_equal(gmc, omc):
            bad = int(np.nonzero(gmc != omc)[0][0])
            raise GateError(f"step {t}: set {bad} has {gmc[bad]} misses, oracle {omc[bad]}")
        gms = _u32(bufs["misses"][: self.n_sets]).reshape(self.n_sets, -1, 4)
        oms4 = oms.view(np.uint32).reshape(self.n_sets, -1, 4)
        live = np.arange(gms.shape[1])[None, :] < omc[:, None]
        if not np.array_equal(gms[live], oms4[live]):
            bad = np.nonzero(~np.all(gms == oms4, axis=2) & live)
            raise GateError(f"step {t}: miss list of set {int(bad[0][0])} differs at "
                            f"entry {int(bad[1][0])}")
        self.steps += 1
        self.selections += int(np.count_nonzero(s != O.NONE))
        self.misses += int(omc.sum())
        self.last_sel = s
        self.last_misses = (omc.copy(), oms4.copy())

    def final(self, ex, q, out, rng=None):
        """State, pool bytes and attention after the last replayed step; q and
        out are the q and attention output of that step (device tensors)."""
        fill, ord_, tag = ex.sets_state()
        ofill, oord, otag = self.ox.state()
        n = self.n_sets
        for name, a, b in (("fill", fill[:n], ofill), ("order", ord_[:n], oord), ("tags", tag[:n], otag)):
            if not np.array_equal(a, b):
                raise GateError(f"LRU {name} differs from the oracle after {self.steps} steps")
        # pool bytes: the blocks fetched in the last step, and every resident
        # slot of the first and last layer
        host, hsc = ex.hosttier_array()
        bb = ex.block_bytes
        hb = ex.cfg.host_blocks
        hostb = host.reshape(hb, bb)
        scales = None if hsc is None else hsc.reshape(hb, 2)
        omc, oms = self.last_misses
        fetched = np.concatenate([oms[s, : omc[s]] for s in range(n) if omc[s]] or
                                 [np.zeros((0, 4), np.uint32)])
        sets = np.arange(n)
        layer = (sets // self.H) % self.L
        edge = sets[(layer == 0) | (layer == self.L - 1)]
        res_set = np.repeat(edge, ofill[edge])
        res_loc = np.concatenate([np.arange(ofill[s]) for s in edge] or [np.zeros(0, np.int64)])
        pset = np.concatenate([fetched[:, 3].astype(np.int64), res_set.astype(np.int64)])
        ploc = np.concatenate([fetched[:, 1].astype(np.int64), res_loc.astype(np.int64)])
        blk = otag[pset, ploc].astype(np.int64)
        pslots = pset * self.C + ploc
        hidx = (pset * int(self.g.max_blocks) + blk) % hb
        got = ex.pool_slots_bytes(pslots)
        if not np.array_equal(got, hostb[hidx]):
            bad = int(np.nonzero(np.any(got != hostb[hidx], axis=1))[0][0])
            raise GateError(f"pool slot {int(pslots[bad])} (set {int(pset[bad])}, block "
                            f"{int(blk[bad])}) differs from the host tier")
        if scales is not None and not np.array_equal(ex.pool_slot_scales(pslots), scales[hidx]):
            raise GateError("fp8 scales of a pool slot differ from the host tier")
        # attention of the replayed requests in three layers (others EMPTY)
        keep = sorted({0, self.L // 2, self.L - 1})
        s = np.full_like(self.last_sel, O.NONE)
        s[:, keep] = self.last_sel[:, keep]
        qn = np.ascontiguousarray(q[: self.nr].cpu().numpy(), np.float32)
        ref = O.attention_f64(self.g, s, qn)[:, keep].reshape(-1, 128)
        got = out[: self.nr].cpu().numpy()[:, keep].reshape(-1, 128).astype(np.float64)
        den = np.abs(ref).max(axis=1)
        rows = den > 0
        err = float((np.abs(got - ref).max(axis=1)[rows] / den[rows]).max()) if rows.any() else 0.0
        tol = 1e-2 if self.dtype == O.FP8 else 2e-3
        if not err < tol:
            raise GateError(f"attention row error {err:.3g} >= {tol}")
        return {"owners": self.n_owners, "requests": self.nr, "steps": self.steps,
                "selections_compared": self.selections, "misses_compared": self.misses,
                "blocks_memcmp": int(pslots.size), "attention_rows": int(rows.sum()),
                "attention_max_rel_err": float(f"{err:.3g}"), "tolerance": tol}
