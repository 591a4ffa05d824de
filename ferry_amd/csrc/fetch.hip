// fetch.hip -- drain of the device miss ring into the HBM slot pool.
//
// Persistent workgroups, one deque each.  Every wavefront pops one miss at a
// time from its own deque head; when that is empty it looks for a victim with
// more than its fair share ceil(remaining / deques) and steals
// min(steal_chunk, rem - fair, rem/2 + 1) entries from its tail (the
// reference's excess rule and take, src/runtime/wla_multigpu.cuh:882-884,
// 1147-1152, 1518-1526; src/runtime/multigpu.cuh:153-175).  Victims are
// searched 64 deques at a time (one per lane), starting at a window that
// differs per wavefront, and the fullest deque of the first window with an
// excess is robbed: thieves spread over the victims instead of all racing for
// the single fullest deque.  A thief whose CAS loses backs off briefly.  A
// wavefront stops when no deque holds twice its fair share (and two entries
// per wavefront of a workgroup more): a balanced drain's entries stay with
// their own deque's wavefronts (measured at the 7B shape: stealing on every
// excess made the step 4.5% slower than no stealing), while skewed deques are
// still robbed.  A miss is copied by one wavefront: 16-byte loads straight from
// the pinned host tier (one PCIe hop, no staging ring, unlike
// HostStagedChannel::submit, src/comm/host_staged_channel.cpp:43-74) into the
// slot.  The last workgroup to finish accounts the drain and rewinds every
// deque, so the ring is empty and reusable when the kernel ends.  Slot stores
// are non-temporal: a fetched block is next read by attention, whose
// non-temporal loads ran ~7% (7B MHA) to ~25% (GQA) slower on MI355X when the
// step's freshly stored lines were still held in cache.
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int NV>
__device__ inline void copy_block(const FetchArgs& a, const ferry_miss& m, int lane) {
  const uint64_t h = host_index(m.set, m.block, (uint64_t)a.g.max_blocks, a.g.host_blocks);
  const u32x4* src = reinterpret_cast<const u32x4*>(a.host + h * a.g.bb);
  u32x4* dst = reinterpret_cast<u32x4*>(a.pool + ((uint64_t)m.set * (uint64_t)a.g.C + m.slot) * a.g.bb);
  u32x4 r[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) r[i] = __builtin_nontemporal_load(src + i * kWave + lane);
#pragma unroll
  for (int i = 0; i < NV; ++i) __builtin_nontemporal_store(r[i], dst + i * kWave + lane);
  if (a.pool_scales && lane < 2)
    a.pool_scales[((uint64_t)m.set * (uint64_t)a.g.C + m.slot) * 2 + lane] = a.host_scales[h * 2 + lane];
}

__device__ inline ferry_miss load_entry(const ferry_miss* p) {
  ferry_miss m;
  m.block = p->block;
  m.slot = p->slot;
  m.evicted = p->evicted;
  m.set = p->set;
  return m;
}

// K consecutive ring entries copied by one wavefront with all K blocks in
// flight at once (a thief's stolen range; its own deque's entries come one at a
// time, shared with the other wavefronts of its workgroup).
template <int NV, int K>
__device__ inline void copy_blocks(const FetchArgs& a, const ferry_miss* e, int lane) {
  ferry_miss m[K];
#pragma unroll
  for (int b = 0; b < K; ++b) m[b] = load_entry(e + b);
  u32x4 r[K][NV];
  uint64_t h[K];
#pragma unroll
  for (int b = 0; b < K; ++b) {
    h[b] = host_index(m[b].set, m[b].block, (uint64_t)a.g.max_blocks, a.g.host_blocks);
    const u32x4* src = reinterpret_cast<const u32x4*>(a.host + h[b] * a.g.bb);
#pragma unroll
    for (int i = 0; i < NV; ++i) r[b][i] = __builtin_nontemporal_load(src + i * kWave + lane);
  }
#pragma unroll
  for (int b = 0; b < K; ++b) {
    const uint64_t slot = (uint64_t)m[b].set * (uint64_t)a.g.C + m[b].slot;
    u32x4* dst = reinterpret_cast<u32x4*>(a.pool + slot * a.g.bb);
#pragma unroll
    for (int i = 0; i < NV; ++i) __builtin_nontemporal_store(r[b][i], dst + i * kWave + lane);
    if (a.pool_scales && lane < 2) a.pool_scales[slot * 2 + lane] = a.host_scales[h[b] * 2 + lane];
  }
}

}  // namespace

template <int NV>
__global__ __launch_bounds__(256) void k_fetch(FetchArgs a) {
  // the fetch shares CUs with the attention it overlaps: its few wavefronts
  // issue first so the host link never waits on them
  if (a.prio) __builtin_amdgcn_s_setprio(3);
  const int lane = threadIdx.x & 63;
  const int W = gridDim.x;
  const int me = blockIdx.x;
  uint64_t* state = a.ring.state;
  uint64_t steals = 0, stolen = 0, copied = 0;
  uint32_t fair = 0;  // a thief's fair share from its last full pass (0: none yet)
  int backoff = 0;    // lost compare-and-swaps in a row
  // Every iteration either copies at least one miss or observes a CAS lost to
  // a peer that made progress; the guard only bounds a broken protocol.
  for (long guard = 0;; ++guard) {
    if (guard > (1L << 28)) {
      if (lane == 0) set_error(a.err, FERRY_ESPIN);
      break;
    }
    // own deque: pop one from the head
    int got = 0;
    uint32_t idx = 0;
    if (lane == 0) {
      const uint32_t capw = a.ring.cap[me];
      uint64_t st = aload64(state + (size_t)me * kStateStride);
      for (int tries = 0; tries < (1 << 20); ++tries) {
        const uint32_t h = (uint32_t)st;
        const uint32_t t = min((uint32_t)(st >> 32), capw);
        if (h >= t) break;
        const uint64_t prev = atomicCAS((unsigned long long*)(state + (size_t)me * kStateStride), st, st + 1);
        if (prev == st) {
          got = 1;
          idx = h;
          break;
        }
        st = prev;
      }
    }
    got = first_lane_i(got);
    if (got) {
      idx = first_lane_u(idx);
      copy_block<NV>(a, load_entry(a.ring.entries + a.ring.seg[me] + idx), lane);
      ++copied;
      continue;
    }
    // Thieves.  Only the first thief_waves wavefronts of a workgroup steal;
    // the others leave once their own deque is empty.  A thief keeps the
    // fair share ceil(remaining / deques) of its last full pass over the
    // deques and looks for a victim 64 deques at a time (one per lane), from a
    // window that differs per thief, taking the fullest deque of the
    // first window holding at least twice its share: thieves spread over the
    // victims instead of racing for one.  When no window has a victim it
    // makes a fresh pass and searches again, and leaves if there is still
    // none (a balanced drain's end: the rest stays with the deques' own
    // wavefronts).  A lost compare-and-swap backs off, longer each time in a
    // row.  Every deque state word is read coherently across the chip's
    // L2s, so each pass is fabric traffic shared with the overlapped
    // attention's loads: passes are made only when a search fails.
    if (!a.steal || (int)(threadIdx.x >> 6) >= a.thief_waves) break;
    const int nwin = (W + kWave - 1) / kWave;
    const int first_win = me * a.thief_waves + (int)(threadIdx.x >> 6);
    auto rem_of = [&](int w) -> uint32_t {
      if (w >= W) return 0u;
      const uint64_t st = aload64(state + (size_t)w * kStateStride);
      const uint32_t h = (uint32_t)st, t = min((uint32_t)(st >> 32), a.ring.cap[w]);
      return t > h ? t - h : 0u;
    };
    auto search = [&](uint32_t floor_rem, uint32_t& best, int& bw) {
      best = 0;
      bw = W;
      for (int i = 0; i < nwin && best == 0; ++i) {
        const int w = ((first_win + i) % nwin) * kWave + lane;
        const uint32_t rem = rem_of(w);
        best = rem > floor_rem ? rem : 0u;
        bw = best ? w : W;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          const uint32_t ob = __shfl_xor(best, off);
          const int ow = __shfl_xor(bw, off);
          if (ob > best || (ob == best && ow < bw)) {
            best = ob;
            bw = ow;
          }
        }
        best = first_lane_u(best);
        bw = first_lane_i(bw);
      }
    };
    // A victim must hold at least twice its share, and two entries per
    // wavefront of a workgroup above it.  The link, not the wavefronts, bounds
    // a drain: a deque a few entries or percent above the others finishes with
    // them, and robbing it only adds atomics and a late copy; a deque holding
    // several shares (skewed, request-affine misses) would end the drain late.
    auto floor_of = [&](uint32_t f) { return max(2u * f, f + 2u * (blockDim.x >> 6)); };
    uint32_t best = 0;
    int bw = W;
    if (fair) search(floor_of(fair), best, bw);
    if (best == 0) {  // fresh pass over every deque
      uint64_t total = 0;
      for (int i = 0; i < nwin; ++i) total += rem_of(i * kWave + lane);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
      total = first_lane_u64(total);
      if (total == 0) break;  // every deque is drained
      fair = (uint32_t)((total + (uint64_t)W - 1) / (uint64_t)W);
      search(floor_of(fair), best, bw);
      if (best == 0) break;  // no deque far enough above its fair share
    }
    const uint32_t floor_rem = floor_of(fair);
    int ok = 0;
    uint32_t s0 = 0, s1 = 0;
    if (lane == 0) {
      const uint64_t st = aload64(state + (size_t)bw * kStateStride);
      const uint32_t h = (uint32_t)st, t = min((uint32_t)(st >> 32), a.ring.cap[bw]);
      const uint32_t rem = t > h ? t - h : 0u;
      if (rem > floor_rem) {
        // the reference's take: min(k, cur - fair, cur/2 + 1)
        const uint32_t m = min(min(a.steal_chunk, rem - fair), rem / 2 + 1);
        const uint64_t nst = ((uint64_t)(t - m) << 32) | h;
        if (atomicCAS((unsigned long long*)(state + (size_t)bw * kStateStride), st, nst) == st) {
          ok = 1;
          s0 = t - m;
          s1 = t;
        }
      }
    }
    ok = first_lane_i(ok);
    if (!ok) {  // a peer took it first: back off before looking again
      backoff = min(backoff + 1, 6);
      for (int i = 0; i < (1 << backoff); ++i) __builtin_amdgcn_s_sleep(2);
      continue;
    }
    backoff = 0;
    s0 = first_lane_u(s0);
    s1 = first_lane_u(s1);
    const ferry_miss* seg = a.ring.entries + a.ring.seg[bw];
    uint32_t i = s0;
    if (a.steal_inflight >= 4 && NV <= 8)
      for (; i + 4 <= s1; i += 4) copy_blocks<NV, 4>(a, seg + i, lane);
    if (a.steal_inflight >= 2)
      for (; i + 2 <= s1; i += 2) copy_blocks<NV, 2>(a, seg + i, lane);
    for (; i < s1; ++i) copy_block<NV>(a, load_entry(seg + i), lane);
    ++steals;
    stolen += s1 - s0;
    copied += s1 - s0;
  }
  if (lane == 0) {
    if (copied) atomicAdd(a.stats + kStatDrain, (unsigned long long)copied);
    if (steals) {
      atomicAdd(a.stats + kStatSteals, (unsigned long long)steals);
      atomicAdd(a.stats + kStatStolen, (unsigned long long)stolen);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    const uint32_t prev = atomicAdd(a.done, 1u);
    if (prev == (uint32_t)W - 1) {
      __threadfence();
      for (int w = 0; w < W; ++w) astore64(state + (size_t)w * kStateStride, 0ull);
      const unsigned long long total = atomicExch(a.stats + kStatDrain, 0ull);
      atomicAdd(a.stats + kStatMisses, total);
      atomicAdd(a.stats + kStatBytes, total * a.g.bb);
      atomicExch(a.stats + kStatLast, total);
      atomicAdd(a.step_acc, total);
      astore(a.done, 0u);
      __threadfence();
    }
  }
}

template __global__ void k_fetch<4>(FetchArgs);
template __global__ void k_fetch<8>(FetchArgs);
template __global__ void k_fetch<16>(FetchArgs);

__global__ void k_step_close(unsigned long long* acc, unsigned long long* host) {
  // one lane moves the step's two counters into the mapped pinned words
  // (system-scope stores over the host link: no copy launch on the stream
  // ahead of the next step) and restarts them from zero.  host[2] is a
  // sequence word, odd while the counters change, so a host reader can tell
  // a torn pair (the host enqueues steps ahead and may read at any time)
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const unsigned long long seq = acc[2];
    const unsigned long long fetched = acc[0], attended = acc[1];
    __hip_atomic_store(host + 2, seq + 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __threadfence_system();
    __hip_atomic_store(host + 0, fetched, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(host + 1, attended, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(host + 2, seq + 2ull, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    acc[0] = 0ull;
    acc[1] = 0ull;
    acc[2] = seq + 2ull;
  }
}

// Queue externally built misses: each thread appends one entry to the tail of
// its set's worker deque.
__global__ void k_missq_push(Geo g, Ring ring, const ferry_miss* m, uint32_t n, int* err) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const ferry_miss e = m[i];
  if (e.set >= (uint32_t)g.n_sets || e.slot >= (uint32_t)g.C || e.block >= (uint32_t)g.max_blocks) {
    set_error(err, FERRY_EINVAL);
    return;
  }
  const uint32_t w = ring.worker_of_set[e.set];
  const uint64_t old = atomicAdd((unsigned long long*)(ring.state + (size_t)w * kStateStride), 1ull << 32);
  const uint32_t t = (uint32_t)(old >> 32);
  if (t >= ring.cap[w]) {
    set_error(err, FERRY_ESPIN);
    return;
  }
  ring.entries[ring.seg[w] + t] = e;
}

}  // namespace ferry_amd
