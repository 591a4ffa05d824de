// lru.hip -- miss bookkeeping of one decode step: dedup, LRU slot assignment
// and eviction, miss-ring push.  One wavefront owns one set (owner, layer, kv
// head) for the whole step, so no two waves ever touch the same set state.
//
// Rule (one "sub-step" = the whole step in FERRY_LRU_STEP, one selection in
// FERRY_LRU_SERIAL; with one selection it is exactly the reference's kv_touch,
// src/runtime/wla_multigpu.cuh:1937-1962 / missstream.cuh:137-161):
//   hit  = block resident when the sub-step starts;
//   miss = first occurrence, in canonical order (member request, then
//          selection index), of a non-resident block; later occurrences hit
//          the in-flight fetch (dedup, kv_exec.cuh:210-223 dedups per step);
//   the q-th miss takes free slot fill+q while free slots remain, else the
//          least recently used resident slot not touched in this sub-step;
//   new LRU order = untouched survivors in old order ++ touched slots ordered
//          by their last occurrence.
// A selection id of kNone (0xFFFFFFFF) is an empty position: it is neither a
// hit nor a miss, its slot is reported as kNone, and it touches no state.  A
// request that is not resident this step has a row of empty positions; a
// short context has a ragged row (fewer than k blocks to choose from).
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

struct SetView {
  int o, l, h, n;  // owner, layer, kv head, selections of the set this step
};

__device__ inline size_t sel_index(const Geo& g, const SetView& s, int p) {
  const int m = p / g.k, j = p - m * g.k;
  return ((size_t)((s.o * g.group + m) * g.L + s.l) * g.Hkv + s.h) * (size_t)g.k + j;
}

// Selection at position p of the set: from its LDS copy when the kernel staged
// one (ssel, wave-uniform), else from the step's selection table.  With the
// copy, ssel[max_sel + p] keeps the slot position p resolved to (pass 4b) for
// the passes after it.
__device__ inline uint32_t sel_at(const Geo& g, const SetView& s, const uint32_t* __restrict__ sel,
                                  const uint32_t* ssel, int p) {
  return ssel ? ssel[p] : sel[sel_index(g, s, p)];
}

// One batched sub-step over positions [p0, p0 + cnt).  Returns the number of
// misses appended at mo[0..), or a negative FERRY_E* code.  The passes that
// look positions up in the block->slot map load the entries of B rounds of 64
// positions before using any: a wavefront keeps B round trips in flight
// instead of one.  That is safe within each pass: classify only turns a
// non-resident entry into another non-resident one (the first occurrence's
// mark), which sends a position down the same path whichever it reads, and
// the later passes only read.
template <int B>
__device__ int substep(const Geo& g, const SetView& sv, uint32_t set, int p0, int cnt,
                       const uint32_t* __restrict__ sel, uint32_t* ssel,
                       uint32_t* __restrict__ slots_out,
                       uint8_t* __restrict__ miss_flag, uint32_t* __restrict__ map,
                       int* lastpos, uint32_t* sord, uint32_t* stag, uint32_t* smblk,
                       uint32_t* svict, uint32_t& fill, ferry_miss* __restrict__ mo,
                       const Ring& ring, uint32_t worker, uint32_t cap, uint32_t* sown) {
  const int lane = lane_id();
  const int C = g.C;
  const int pend = p0 + cnt;
  uint32_t xs[B], vs[B];
  // positions c0 + 64 u + lane of a batch; kNone past the sub-step
  auto gather = [&](int c0) {
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int p = c0 + u * kWave + lane;
      xs[u] = p < pend ? sel_at(g, sv, sel, ssel, p) : kNone;
    }
#pragma unroll
    for (int u = 0; u < B; ++u) vs[u] = xs[u] != kNone ? aload(map + xs[u]) : kNone;
  };
  // phase 1: classify (hits mark their slot; misses race for first occurrence)
  for (int c0 = p0; c0 < pend; c0 += B * kWave) {
    gather(c0);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int p = c0 + u * kWave + lane;
      if (xs[u] != kNone) {
        if (vs[u] < (uint32_t)C)
          atomicMax(lastpos + vs[u], p);
        else
          atomicMin(map + xs[u], kPend | (uint32_t)p);
      }
    }
  }
  wave_fence();
  // phase 2: rank misses by first occurrence
  int M = 0;
  for (int c0 = p0; c0 < pend; c0 += B * kWave) {
    gather(c0);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int p = c0 + u * kWave + lane;
      const bool is_miss = xs[u] != kNone && vs[u] == (kPend | (uint32_t)p);
      if (p < pend && miss_flag) miss_flag[sel_index(g, sv, p)] = is_miss ? 1 : 0;
      const uint64_t mask = ballot(is_miss);
      if (is_miss) smblk[M + lanes_below(mask)] = xs[u];
      M += __builtin_popcountll(mask);
    }
  }
  // phase 3: victims = least recent untouched residents, oldest first; the
  // set may use `cap` of its C slots (fewer under per-member capacity)
  const int freeslots = (int)cap > (int)fill ? (int)cap - (int)fill : 0;
  const int need = M > freeslots ? M - freeslots : 0;
  int nv = 0;
  for (int c = 0; c < (int)fill && nv < need; c += kWave) {
    const int i = c + lane;
    bool untouched = false;
    uint32_t o = 0;
    if (i < (int)fill) {
      o = sord[i];
      untouched = lastpos[o] < 0;
    }
    const uint64_t mask = ballot(untouched);
    const int r = nv + lanes_below(mask);
    if (untouched && r < need) svict[r] = o;
    nv += __builtin_popcountll(mask);
  }
  __builtin_amdgcn_wave_barrier();
  if (nv < need) {
    for (int q = lane; q < M; q += kWave) astore(map + smblk[q], kNone);
    wave_fence();
    return FERRY_ECAPACITY;
  }
  // reserve M entries at the tail of this set's worker deque
  ferry_miss* rdst = nullptr;
  if (M > 0) {
    uint64_t old = 0;
    if (lane == 0)
      old = atomicAdd((unsigned long long*)(ring.state + (size_t)worker * kStateStride),
                      (unsigned long long)M << 32);
    const uint32_t t0 = (uint32_t)(first_lane_u64(old) >> 32);
    if (t0 + (uint32_t)M > ring.cap[worker]) {
      for (int q = lane; q < M; q += kWave) astore(map + smblk[q], kNone);
      wave_fence();
      return FERRY_ESPIN;
    }
    rdst = ring.entries + ring.seg[worker] + t0;
  }
  // phase 4: assign slots, evict, publish block -> slot, write the ring
  for (int q = lane; q < M; q += kWave) {
    const uint32_t x = smblk[q];
    uint32_t v, ev = kNone;
    if (q < freeslots) {
      v = fill + (uint32_t)q;
    } else {
      v = svict[q - freeslots];
      ev = stag[v];
      if (ev < (uint32_t)g.max_blocks) astore(map + ev, kNone);
    }
    stag[v] = x;
    if (sown) sown[v] = 0u;  // a new block: the slot's old members are dropped
    astore(map + x, v);
    ferry_miss m;
    m.block = x;
    m.slot = v;
    m.evicted = ev;
    m.set = set;
    mo[q] = m;
    rdst[q] = m;
  }
  wave_fence();
  // phase 4b: slot of every position; last occurrence per touched slot
  for (int c0 = p0; c0 < pend; c0 += B * kWave) {
    gather(c0);
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int p = c0 + u * kWave + lane;
      if (p < pend) {
        const size_t gi = sel_index(g, sv, p);
        if (xs[u] == kNone) {
          slots_out[gi] = kNone;
        } else {
          const uint32_t v = vs[u];
          if (ssel) ssel[g.max_sel + p] = v;
          slots_out[gi] = set * (uint32_t)C + v;
          atomicMax(lastpos + v, p);
          if (sown) atomicOr(sown + v, 1u << (uint32_t)(p / g.k));  // member of position p
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  // phase 5: new LRU order
  int w = 0;
  for (int c = 0; c < (int)fill; c += kWave) {
    const int i = c + lane;
    bool keep = false;
    uint32_t o = 0;
    if (i < (int)fill) {
      o = sord[i];
      keep = lastpos[o] < 0;
    }
    const uint64_t mask = ballot(keep);
    __builtin_amdgcn_wave_barrier();
    if (keep && w + lanes_below(mask) < C) sord[w + lanes_below(mask)] = o;
    w += __builtin_popcountll(mask);
  }
  for (int c = p0; c < pend; c += kWave) {
    const int p = c + lane;
    bool emit = false;
    uint32_t v = 0;
    const uint32_t x = p < pend ? sel_at(g, sv, sel, ssel, p) : kNone;
    if (x != kNone) {
      v = ssel ? ssel[g.max_sel + p] : aload(map + x);
      emit = lastpos[v] == p;
    }
    const uint64_t mask = ballot(emit);
    if (emit && w + lanes_below(mask) < C) sord[w + lanes_below(mask)] = v;
    w += __builtin_popcountll(mask);
  }
  fill += (uint32_t)(M < freeslots ? M : freeslots);
  if (w != (int)fill) return FERRY_ESTATE;
  // phase 6: clear the marks of this sub-step
  for (int c = p0; c < pend; c += kWave) {
    const int p = c + lane;
    const uint32_t x = p < pend ? sel_at(g, sv, sel, ssel, p) : kNone;
    if (x != kNone) lastpos[ssel ? ssel[g.max_sel + p] : aload(map + x)] = -1;
  }
  __builtin_amdgcn_wave_barrier();
  return M;
}

}  // namespace

template <bool SERIAL>
__global__ __launch_bounds__(256) void k_lru_step(Geo g, const uint32_t* __restrict__ sel,
                                                  uint32_t* __restrict__ slots_out,
                                                  uint32_t* __restrict__ miss_count,
                                                  ferry_miss* __restrict__ misses,
                                                  uint8_t* __restrict__ miss_flag,
                                                  SetState st, Ring ring, int l0, int nl,
                                                  unsigned long long* __restrict__ sel_counts,
                                                  int* __restrict__ err) {
  extern __shared__ uint32_t lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wpb = blockDim.x >> 6;
  // this wave's set among those of layers [l0, l0 + nl)
  const int idx = blockIdx.x * wpb + wave;
  if (idx >= g.n_owners * nl * g.Hkv) return;  // no workgroup barriers follow
  const int set = ((idx / (nl * g.Hkv)) * g.L + l0 + (idx / g.Hkv) % nl) * g.Hkv + idx % g.Hkv;
  const int C = g.C;
  uint32_t* base = lds + (size_t)wave * lru_lds_wave_words(g);
  int* lastpos = (int*)base;
  uint32_t* sord = base + C;
  uint32_t* stag = base + 2 * C;
  uint32_t* smblk = base + 3 * C;
  uint32_t* svict = smblk + g.max_sel;
  uint32_t* sown = st.own ? svict + g.max_sel : nullptr;  // [C] member masks
  uint32_t* ssel = lru_stages_sel(g) ? base + lru_lds_words(g) : nullptr;  // [2 max_sel]

  SetView sv;
  sv.h = set % g.Hkv;
  sv.l = (set / g.Hkv) % g.L;
  sv.o = set / (g.Hkv * g.L);
  const int mem = min(g.group, g.n_req - sv.o * g.group);
  sv.n = mem * g.k;

  uint32_t* map = st.map + (size_t)set * (size_t)g.max_blocks;
  uint32_t* gord = st.ord + (size_t)set * C;
  uint32_t* gtag = st.tag + (size_t)set * C;
  uint32_t* gown = st.own ? st.own + (size_t)set * C : nullptr;
  uint32_t fill = st.fill[set];
  // the set's state into LDS, four rounds of loads in flight at a time
  for (int i0 = 0; i0 < C; i0 += 4 * kWave) {
    uint32_t o4[4], t4[4], w4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * kWave + lane;
      if (i < C) {
        o4[u] = gord[i];
        t4[u] = gtag[i];
        w4[u] = sown ? gown[i] : 0u;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * kWave + lane;
      if (i < C) {
        lastpos[i] = -1;
        sord[i] = o4[u];
        stag[i] = t4[u];
        if (sown) sown[i] = w4[u];
      }
    }
  }
  // range check of every selected id before touching the map
  bool bad = false;
  int nsel = 0;  // non-empty positions
  for (int p0 = 0; p0 < sv.n; p0 += 4 * kWave) {  // four rounds of loads in flight
    uint32_t x4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = p0 + u * kWave + lane;
      x4[u] = p < sv.n ? sel[sel_index(g, sv, p)] : kNone;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int p = p0 + u * kWave + lane;
      if (ssel && p < sv.n) ssel[p] = x4[u];
      bad |= x4[u] != kNone && x4[u] >= (uint32_t)g.max_blocks;
      nsel += __builtin_popcountll(ballot(x4[u] != kNone));
    }
  }
  if (ballot(bad)) {
    if (lane == 0) {
      set_error(err, FERRY_ERANGE);
      miss_count[set] = 0;
    }
    return;
  }
  __builtin_amdgcn_wave_barrier();

  ferry_miss* mo = misses + (size_t)set * g.max_sel;
  const uint32_t worker = ring.worker_of_set[set];
  const uint32_t cap = set_capacity(g, st.members[sv.o]);
  int total = 0, rc = 0;
  if (!SERIAL) {
    // eight or four rounds per map batch where a set has that many positions
    // (prefix groups: group * k), one otherwise
    if (g.max_sel >= 8 * kWave)
      rc = substep<8>(g, sv, (uint32_t)set, 0, sv.n, sel, ssel, slots_out, miss_flag, map, lastpos,
                      sord, stag, smblk, svict, fill, mo, ring, worker, cap, sown);
    else if (g.max_sel >= 4 * kWave)
      rc = substep<4>(g, sv, (uint32_t)set, 0, sv.n, sel, ssel, slots_out, miss_flag, map, lastpos,
                      sord, stag, smblk, svict, fill, mo, ring, worker, cap, sown);
    else
      rc = substep<1>(g, sv, (uint32_t)set, 0, sv.n, sel, ssel, slots_out, miss_flag, map, lastpos,
                      sord, stag, smblk, svict, fill, mo, ring, worker, cap, sown);
    if (rc >= 0) total = rc;
  } else {
    for (int p = 0; p < sv.n; ++p) {
      rc = substep<1>(g, sv, (uint32_t)set, p, 1, sel, ssel, slots_out, miss_flag, map, lastpos,
                      sord, stag, smblk, svict, fill, mo + total, ring, worker, cap, sown);
      if (rc < 0) break;
      total += rc;
    }
    if (rc >= 0) {
      // every selection's slot must still hold its block at the end of the step
      wave_fence();
      bool lost = false;
      for (int p = lane; p < sv.n; p += kWave) {
        const size_t gi = sel_index(g, sv, p);
        if (sel[gi] != kNone)
          lost |= stag[aload(slots_out + gi) - (uint32_t)set * (uint32_t)C] != sel[gi];
      }
      if (ballot(lost)) rc = FERRY_ECAPACITY;
    }
  }
  if (rc < 0) {
    if (lane == 0) {
      set_error(err, rc);
      miss_count[set] = 0;
    }
    return;
  }
  for (int i = lane; i < C; i += kWave) {
    gord[i] = i < (int)fill ? sord[i] : kNone;
    gtag[i] = stag[i];
    if (sown) gown[i] = sown[i];
  }
  if (lane == 0) {
    st.fill[set] = fill;
    miss_count[set] = (uint32_t)total;
    if (nsel)
      atomicAdd(sel_counts + (size_t)(set % kSelCounters) * kSelStride, (unsigned long long)nsel);
  }
}

template __global__ void k_lru_step<false>(Geo, const uint32_t*, uint32_t*, uint32_t*, ferry_miss*,
                                           uint8_t*, SetState, Ring, int, int,
                                           unsigned long long*, int*);
template __global__ void k_lru_step<true>(Geo, const uint32_t*, uint32_t*, uint32_t*, ferry_miss*,
                                          uint8_t*, SetState, Ring, int, int, unsigned long long*,
                                          int*);

// Reset the sets of the listed owners (a new request takes over a lane):
// one wavefront per set clears the map entries its tags point at, then the
// tags, the order and the fill.  Owner ids must be < n_owners (checked).
__global__ __launch_bounds__(256) void k_sets_reset_owners(Geo g, SetState st,
                                                           const uint32_t* __restrict__ owners,
                                                           uint32_t n, int* __restrict__ err) {
  const int wpb = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const size_t idx = (size_t)blockIdx.x * wpb + (threadIdx.x >> 6);
  const size_t per_owner = (size_t)g.L * g.Hkv;
  if (idx >= (size_t)n * per_owner) return;
  const uint32_t o = owners[idx / per_owner];
  if (o >= (uint32_t)g.n_owners) {
    if (lane == 0) set_error(err, FERRY_EINVAL);
    return;
  }
  const size_t set = (size_t)o * per_owner + idx % per_owner;
  uint32_t* map = st.map + set * (size_t)g.max_blocks;
  uint32_t* tag = st.tag + set * (size_t)g.C;
  uint32_t* ord = st.ord + set * (size_t)g.C;
  for (int i = lane; i < g.C; i += kWave) {
    const uint32_t b = tag[i];
    if (b < (uint32_t)g.max_blocks) map[b] = kNone;
    tag[i] = kNone;
    ord[i] = kNone;
    if (st.own) st.own[set * (size_t)g.C + i] = 0u;
  }
  if (lane == 0) st.fill[set] = 0;
}

// Resident members.  One thread per listed lane: leaving (delta -1) needs
// the lane resident and marks its owner for the trim of generation `gen`;
// joining (+1) needs it not resident.  A lane out of range or in the wrong
// state latches FERRY_EINVAL and changes nothing.
__global__ void k_members_update(Geo g, uint32_t* lane_live, uint32_t* members, uint32_t* trim_gen,
                                 const uint32_t* lanes, uint32_t n, int delta, uint32_t gen,
                                 int* err) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t lane = lanes[i];
  if (lane >= (uint32_t)g.n_req) {
    set_error(err, FERRY_EINVAL);
    return;
  }
  const uint32_t o = lane / (uint32_t)g.group;
  const uint32_t want = delta < 0 ? 1u : 0u;  // the state the lane must be in
  if (atomicCAS(lane_live + lane, want, 1u - want) != want) {
    set_error(err, FERRY_EINVAL);
    return;
  }
  if (delta < 0) {
    atomicSub(members + o, 1u);
    trim_gen[o] = gen;
  } else {
    atomicAdd(members + o, 1u);
  }
}

// Trim one set to its capacity (grp_trim, src/runtime/wla_multigpu.cuh:
// 1923-1936): the e = fill - cap least recently used blocks are evicted and the
// survivors keep their order.  Resident slots stay [0, fill): the survivors in
// slots >= cap ("movers", ascending) move into the evicted slots < cap
// ("holes", ascending), the i-th mover into the i-th hole, data and fp8
// scales included.  One wavefront per set; pos[C] (the LRU position of each
// slot) and the movers' list live in LDS.
template <int NV>
__global__ __launch_bounds__(64) void k_sets_trim(Geo g, SetState st, const uint32_t* lane_live,
                                                  const uint32_t* trim_gen, uint32_t gen,
                                                  uint8_t* __restrict__ pool,
                                                  float* __restrict__ pool_scales) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ uint32_t lds[];
  const int lane = threadIdx.x;
  const uint32_t set = blockIdx.x;
  const uint32_t o = set / (uint32_t)(g.L * g.Hkv);
  if (trim_gen[o] != gen) return;
  const uint32_t C = (uint32_t)g.C;
  const uint32_t fill = st.fill[set];
  uint32_t* own = st.own ? st.own + (size_t)set * C : nullptr;
  if (own) {  // own_release: members that left drop out of every mask
    uint32_t live = 0;
    for (int m = 0; m < g.group && (int)o * g.group + m < g.n_req; ++m)
      if (lane_live[o * g.group + m]) live |= 1u << m;
    for (uint32_t i = lane; i < fill; i += kWave) own[i] &= live;
    wave_fence();
  }
  const uint32_t cap = set_capacity(g, st.members[o]);
  if (fill <= cap) return;
  const uint32_t e = fill - cap;
  uint32_t* pos = lds;         // [C]
  uint32_t* movers = lds + C;  // [C - cap] at most
  uint32_t* ord = st.ord + (size_t)set * C;
  uint32_t* tag = st.tag + (size_t)set * C;
  uint32_t* map = st.map + (size_t)set * (size_t)g.max_blocks;
  for (uint32_t i = lane; i < fill; i += kWave) pos[ord[i]] = i;
  // the evicted blocks leave the map
  for (uint32_t i = lane; i < e; i += kWave) astore(map + tag[ord[i]], kNone);
  wave_fence();
  // movers: surviving slots >= cap, ascending
  uint32_t nm = 0;
  for (uint32_t c = cap; c < fill; c += kWave) {
    const uint32_t v = c + lane;
    const bool mv = v < fill && pos[v] >= e;
    const uint64_t mask = ballot(mv);
    if (mv) movers[nm + lanes_below(mask)] = v;
    nm += (uint32_t)__builtin_popcountll(mask);
  }
  __builtin_amdgcn_wave_barrier();
  // holes: evicted slots < cap, ascending; the r-th takes the r-th mover
  uint32_t nh = 0;
  for (uint32_t c = 0; c < cap && nh < nm; c += kWave) {
    const uint32_t v = c + lane;
    const bool hole = v < cap && pos[v] < e;
    uint64_t mask = ballot(hole);
    while (mask) {  // wavefront-uniform: one block at a time, all lanes copy
      const int b = __builtin_ctzll(mask);
      mask &= mask - 1;
      const uint32_t h = c + (uint32_t)b, m = movers[nh++];
      const u32x4* src = reinterpret_cast<const u32x4*>(pool + ((size_t)set * C + m) * g.bb);
      u32x4* dst = reinterpret_cast<u32x4*>(pool + ((size_t)set * C + h) * g.bb);
      u32x4 r[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) r[i] = __builtin_nontemporal_load(src + i * kWave + lane);
#pragma unroll
      for (int i = 0; i < NV; ++i) __builtin_nontemporal_store(r[i], dst + i * kWave + lane);
      if (pool_scales && lane < 2)
        pool_scales[((size_t)set * C + h) * 2 + lane] = pool_scales[((size_t)set * C + m) * 2 + lane];
      if (lane == 0) {
        const uint32_t blk = tag[m];
        tag[h] = blk;
        if (own) own[h] = own[m];
        astore(map + blk, h);
        ord[pos[m]] = h;
      }
    }
  }
  wave_fence();
  // new order: the survivors, shifted to the front; slots >= cap are free
  for (uint32_t c = 0; c < cap; c += kWave) {
    const uint32_t i = c + lane;
    const uint32_t v = i < cap ? ord[e + i] : 0u;
    __builtin_amdgcn_wave_barrier();
    if (i < cap) ord[i] = v;
    __builtin_amdgcn_wave_barrier();
  }
  for (uint32_t i = cap + lane; i < C; i += kWave) {
    ord[i] = kNone;
    tag[i] = kNone;
    if (own) own[i] = 0u;
  }
  if (lane == 0) st.fill[set] = cap;
}

template __global__ void k_sets_trim<4>(Geo, SetState, const uint32_t*, const uint32_t*, uint32_t,
                                        uint8_t*, float*);
template __global__ void k_sets_trim<8>(Geo, SetState, const uint32_t*, const uint32_t*, uint32_t,
                                        uint8_t*, float*);
template __global__ void k_sets_trim<16>(Geo, SetState, const uint32_t*, const uint32_t*, uint32_t,
                                         uint8_t*, float*);

// Reset all sets: empty order, no tags, map cleared.
__global__ void k_sets_reset(Geo g, SetState st) {
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t nslots = (size_t)g.n_sets * g.C;
  const size_t nmap = (size_t)g.n_sets * g.max_blocks;
  for (size_t i = tid; i < nslots; i += stride) {
    st.ord[i] = kNone;
    st.tag[i] = kNone;
    if (st.own) st.own[i] = 0u;
  }
  for (size_t i = tid; i < nmap; i += stride) st.map[i] = kNone;
  for (size_t i = tid; i < (size_t)g.n_sets; i += stride) st.fill[i] = 0;
}

}  // namespace ferry_amd
