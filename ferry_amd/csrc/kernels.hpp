// kernels.hpp -- device data structures and kernel declarations.
#pragma once

#include "common.hpp"

namespace ferry_amd {

// Per-set LRU state in HBM (see lru.hip for the rule it implements).
struct SetState {
  uint32_t* fill;     // [n_sets] slots in use; free slots are [fill, C)
  uint32_t* ord;      // [n_sets][C] local slots, least recent first
  uint32_t* tag;      // [n_sets][C] block held by each slot (kNone if free)
  uint32_t* map;      // [n_sets][max_blocks] slot holding each block (kNone)
  uint32_t* members;  // [n_owners] resident member lanes of each owner
  uint32_t* own;      // [n_sets][C] members that touched each slot's block since it
                      // was loaded (bit m = member m); prefix groups only, else null
};

// LDS words of one bookkeeping wavefront: lastpos, order, tags, the step's
// misses and victims, and the member masks when the owner is a group.
__host__ __device__ inline size_t lru_lds_words(const Geo& g) {
  return (size_t)(3 + (g.group > 1 ? 1 : 0)) * g.C + 2 * (size_t)g.max_sel;
}
// The bookkeeping also stages a set's selections and, once assigned, their
// slots in LDS (one HBM read of each instead of one per pass) where they fit
// beside that state in 64 KiB.
__host__ __device__ inline bool lru_stages_sel(const Geo& g) {
  return (lru_lds_words(g) + 2 * (size_t)g.max_sel) * 4 <= 65536;
}
__host__ __device__ inline size_t lru_lds_wave_words(const Geo& g) {
  return lru_lds_words(g) + (lru_stages_sel(g) ? 2 * (size_t)g.max_sel : 0);
}

// Blocks an owner's sets may hold: C, or under FERRY_CAP_PER_MEMBER one
// member's share per resident member, at least one share (wla_group_cap,
// src/workloads/missstream.cuh:91-94).
__host__ __device__ inline uint32_t set_capacity(const Geo& g, uint32_t members) {
  if (g.cap_mode != FERRY_CAP_PER_MEMBER) return (uint32_t)g.C;
  const uint32_t m = members > 0 ? members : 1u;
  const uint64_t c = (uint64_t)g.member_slots * m;
  return c < (uint64_t)g.C ? (uint32_t)c : (uint32_t)g.C;
}

// Device miss ring: one deque per fetch worker, each a fixed segment of
// `entries`.  state[w] packs (tail << 32 | head) relative to the segment, so
// owner pops (head++) and thief steals (tail -= m) are single 64-bit CASes.
// Deque w's state word (head | tail << 32) is state[w * kStateStride]: one
// 128-byte line per deque, so owners' pops, pushes and thieves' scans of
// different deques do not contend for the same L2 lines.
constexpr int kStateStride = 16;

struct Ring {
  ferry_miss* entries;
  uint64_t* state;
  const uint32_t* seg;            // [W] segment start
  const uint32_t* cap;            // [W] segment capacity
  const uint32_t* worker_of_set;  // [n_sets]
};

// Device counters (unsigned long long).
enum StatSlot { kStatMisses = 0, kStatBytes, kStatSteals, kStatStolen, kStatLast, kStatDrain, kStatCount };

// Non-empty selections are counted by every set's wavefront; one counter
// would serialise tens of thousands of atomics, so set s adds into counter
// s % kSelCounters, each on its own 128-byte line (kSelStride u64 apart).
constexpr int kSelCounters = 256;
constexpr int kSelStride = 16;

struct FetchArgs {
  Geo g;
  Ring ring;
  const uint8_t* host;
  const float* host_scales;
  uint8_t* pool;
  float* pool_scales;
  int steal;
  uint32_t steal_chunk;
  int prio;              // raise the fetch wavefronts' issue priority
  int thief_waves;       // wavefronts per workgroup that steal once their deque is empty
  int steal_inflight;    // stolen blocks a thief keeps in flight (1, 2 or 4)
  unsigned long long* stats;
  unsigned long long* step_acc;  // blocks fetched since the last k_step_close
  uint32_t* done;
  int* err;
};

template <bool SERIAL>
__global__ void k_lru_step(Geo g, const uint32_t* sel, uint32_t* slots_out, uint32_t* miss_count,
                           ferry_miss* misses, uint8_t* miss_flag, SetState st, Ring ring, int l0,
                           int nl, unsigned long long* sel_counts, int* err);
__global__ void k_sets_reset(Geo g, SetState st);
__global__ void k_sets_reset_owners(Geo g, SetState st, const uint32_t* owners, uint32_t n, int* err);
// Resident members: lanes leave (delta -1) or join (+1); owners that lost a
// member are marked with trim generation `gen` for k_sets_trim.
__global__ void k_members_update(Geo g, uint32_t* lane_live, uint32_t* members, uint32_t* trim_gen,
                                 const uint32_t* lanes, uint32_t n, int delta, uint32_t gen, int* err);
// Trim the sets of owners marked with `gen` to their capacity (one wavefront
// per set, C words of LDS); NV 16-byte words per lane per block moved.
template <int NV>
__global__ void k_sets_trim(Geo g, SetState st, const uint32_t* lane_live, const uint32_t* trim_gen,
                            uint32_t gen, uint8_t* pool, float* pool_scales);

template <int NV>
__global__ void k_fetch(FetchArgs a);
__global__ void k_missq_push(Geo g, Ring ring, const ferry_miss* m, uint32_t n, int* err);
// End of a decode step: host[0..1] (mapped pinned memory) = the step's
// fetched and attended blocks (acc[0..1]), then acc[0..1] = 0.
__global__ void k_step_close(unsigned long long* acc, unsigned long long* host);

// Vector-ALU attention (attn.hip); W wavefronts per workgroup; NT selects
// non-temporal K/V loads.
template <int DT, int G, int W, bool NT>
__global__ void k_attn(Geo g, const float* q, const uint32_t* slots, const uint8_t* pool,
                       const float* pool_scales, float* out, float qscale, int l0, int nl, int* err);

// MFMA variant for GQA groups (G >= 2) of 16/8-bit KV (attn_mfma.hip); W
// wavefronts per workgroup; NT as for k_attn.
template <int DT, int G, int W, bool NT>
__global__ void k_attn_mfma(Geo g, const float* q, const uint32_t* slots, const uint8_t* pool,
                            const float* pool_scales, float* out, float qscale, int l0, int nl,
                            int* err);

// Prefix-group attention (attn_group.hip): one workgroup of W wavefronts per
// (group, layer, kv head) reads each distinct block of the group's set once
// and attends every member row; NTILE tiles of 16 query columns (group * G /
// 16 rounded up); dynamic LDS of attn_group_lds_bytes().  The LDS holds each
// wavefront's ring of blocks in flight: group_waves() = four wavefronts with
// three fp8 blocks (or two 16-bit blocks) each let two workgroups share a CU.
// Eight wavefronts with four fp8 blocks each (one workgroup per CU, 96 KiB in
// flight instead of 64) measured 5% slower for a whole launch and kept the
// overlapped fetch off the CUs: the shared-prefix step took 4.23 ms against
// 3.80.  A launch with no more group sets than CUs, which leaves CUs idle
// with four, runs kGroupWideWaves wavefronts per workgroup (the same rings):
// a workgroup that has its CU alone then keeps twice the blocks in flight and
// spreads its arithmetic over twice the wavefronts.
constexpr int kGroupMaxTiles = 4;         // query tiles every wavefront attends with (64 columns)
constexpr int kGroupMaxLds = 160 * 1024;  // LDS of one CU
constexpr int group_waves(int dtype) { return dtype == FERRY_F32 ? 0 : 4; }
constexpr int kGroupWideWaves = 8;
constexpr int group_ring_blocks(int dtype) { return dtype == FERRY_FP8_E4M3 ? 3 : 2; }
constexpr int group_ring_bytes(int dtype) {
  return group_ring_blocks(dtype) * 2 * 16 * 128 * (dtype == FERRY_FP8_E4M3 ? 1 : 2);
}
template <int DT, int G, int NTILE, int W>
__global__ void k_attn_group(Geo g, const float* q, const uint32_t* slots, const uint8_t* pool,
                             const float* pool_scales, float* out, float qscale, int l0, int nl,
                             int* err, unsigned long long* attn_blocks);
// LDS of one k_attn_group workgroup: the wavefronts' rings, the Q^T operands
// of every tile (fp16, or bf16 hi and lo parts: 4 KiB per part and tile), the
// distinct list (slot and member mask per entry, at most group * k entries),
// the merge's per-column max and sum of every wavefront, and the scan scratch.
inline size_t attn_group_lds_bytes(int dtype, int ntile, long group_k, int waves) {
  const size_t w = (size_t)waves, parts = dtype == FERRY_BF16 ? 2 : 1;
  return w * group_ring_bytes(dtype) + parts * ntile * 4096 + 8 * (size_t)group_k +
         8 * w * 16 * ntile + 4 * w;
}

// Bandwidth ceilings (probe.hip): the attention kernels' loads without their
// math, and device-direct host-tier reads without the fetch bookkeeping.
template <int NLD>
__global__ void k_probe_gather(const uint8_t* pool, uint64_t bb, const uint32_t* slots, int k,
                               uint64_t pool_slots, uint32_t* sink);
template <int NV>
__global__ void k_probe_copy(const uint8_t* src, uint8_t* dst, uint64_t bb, uint64_t n_blocks);
template <int NI, int W, int U, int UNITS>
__global__ void k_probe_ktab(Geo g, const uint8_t* kt, uint64_t kt_mod, int nb, uint32_t* sink);
template <int ES, int U>
__global__ void k_probe_sums(Geo g, const uint8_t* sums, uint64_t sum_mod, int nb, uint32_t* sink);
template <int NV>
__global__ void k_probe_host(const uint8_t* host, uint64_t bb, uint64_t n_blocks, uint32_t* sink);

__global__ void k_hosttier_fill(Geo g, uint8_t* host, float* scales, uint64_t seed, float mult,
                                float mult8, float scale_base);

// Byte offsets of an owner image (handoff.hip): header, fill[S], start[S],
// ord[S*C], tag[S*C], own[S*C], scales[S*C][2] (fp8 only), then the data from a
// 256-byte boundary, S = L * Hkv sets of C slots.
struct ImageLayout {
  uint64_t fill, start, ord, tag, own, scales, data, bytes;
};
__host__ __device__ inline ImageLayout make_image_layout(const Geo& g) {
  const uint64_t S = (uint64_t)g.L * (uint64_t)g.Hkv, N = S * (uint64_t)g.C;
  ImageLayout l;
  l.fill = 64;
  l.start = l.fill + 4 * S;
  l.ord = l.start + 4 * S;
  l.tag = l.ord + 4 * N;
  l.own = l.tag + 4 * N;
  l.scales = l.own + 4 * N;
  const uint64_t sc = g.dtype == FERRY_FP8_E4M3 ? 8 * N : 0;
  l.data = (l.scales + sc + 255) / 256 * 256;
  l.bytes = l.data + N * g.bb;
  return l;
}
// counts: the blocks each set exports (null: its fill); member_bit 0 for a
// whole-owner image, else the one member whose exclusive blocks it carries.
__global__ void k_owner_export_meta(Geo g, SetState st, uint32_t owner, uint8_t* image,
                                    const uint32_t* counts, uint32_t member_bit);
// Member carry: per set, the resident blocks only that member touched.
__global__ void k_member_export_count(Geo g, SetState st, uint32_t owner, uint32_t bit,
                                      uint8_t* image);
template <int NV>
__global__ void k_member_export_data(Geo g, SetState st, uint32_t owner, uint32_t bit,
                                     const uint8_t* pool, const float* pool_scales, uint8_t* image);
template <int NV>
__global__ void k_member_import(Geo g, SetState st, uint32_t owner, uint32_t bit, uint8_t* pool,
                                float* pool_scales, const uint8_t* image, int* err);
template <int NV>
__global__ void k_owner_export_data(Geo g, SetState st, uint32_t owner, const uint8_t* pool,
                                    const float* pool_scales, uint8_t* image);
__global__ void k_owner_import_meta(Geo g, SetState st, uint32_t owner, const uint8_t* image, int* err);
template <int NV>
__global__ void k_owner_import_data(Geo g, SetState st, uint32_t owner, uint8_t* pool, float* pool_scales,
                                    const uint8_t* image);

// Top-k block selection (select.hip): per-host-block K min/max summaries and
// the Quest-bound scoring + radix top-k kernel.
template <int DT>
__global__ void k_summaries_build(Geo g, const uint8_t* host, const float* host_scales, uint8_t* sums,
                                  float* sum_scales);
__global__ void k_summaries_tile(uint8_t* sums, float* scales, uint64_t host_blocks, uint64_t total,
                                 uint32_t rec);
template <int DT, int G, bool LAYER, int W>
__global__ void k_select_topk(Geo g, const float* q, const int32_t* ctx_blocks, const uint8_t* sums,
                              const float* sum_scales, uint64_t sum_mod, uint32_t* sel, int l0, int nl,
                              int max_n, int* err);

// Mass method of the top-k selection (select.hip): the dense K table, the
// softmax-mass scoring and the radix top-k of each (request, layer).
template <int NV>
__global__ void k_ktiles_build(Geo g, const uint8_t* host, const float* host_scales, uint8_t* kt,
                               float* kt_scales, int perm);
template <int DT, int G, int W>
__global__ void k_select_mass(Geo g, const float* q, const int32_t* ctx_blocks, const uint8_t* kt,
                              const float* kt_scales, uint64_t kt_mod, float* ws, uint32_t* sel, int l0,
                              int nl, int max_n, int* err);
// 16-bit and fp8 K: k_mass_units scores one (request, layer, kv head) unit
// per workgroup pass into mass[unit][block], then k_mass_topk sums each
// (request, layer) item's kv heads and takes its top k.
template <int DT, int G, int W, int U>
__global__ void k_mass_units(Geo g, const float* q, const int32_t* ctx_blocks, const uint8_t* kt,
                             const float* kt_scales, uint64_t kt_mod, float* ws, float* mass,
                             unsigned* counter, int l0, int nl, int max_n, int* err);
__global__ void k_mass_reset(unsigned* counter);
template <int W>
__global__ void k_mass_topk(Geo g, const int32_t* ctx_blocks, const float* mass, uint32_t* sel, int l0,
                            int nl, int max_n);
// persistent workgroups of k_select_mass (fp32 K); each holds max_blocks * G * 2
// floats of workspace
constexpr int kMassWgs = 2048;
// k_mass_units: wavefronts per workgroup, K records in flight per wavefront,
// and at most this many workgroups (the GPU's resident ones below that), each
// with a max_blocks * G * 2-float workspace slice.  At the long-context GQA
// shape (bf16, 138 VGPRs: one workgroup per CU) eight wavefronts with three
// records each measured 0.80-0.84 of HBM, four records 0.80-0.83, and four
// wavefronts (three workgroups per CU) 0.77-0.80 with four records, 0.82
// with six.
constexpr int kMassUnitWaves = 8;
constexpr int kMassUnitInflight = 3;
constexpr int kMassUnitWgs = 2048;
constexpr int kMassTopkWaves = 4;

// queue.hip: the ceiling of the ring's tickets (one shared 64-bit word)
__global__ void k_ticket_probe(unsigned long long* word, int iters, int kind, int* failed);

}  // namespace ferry_amd
