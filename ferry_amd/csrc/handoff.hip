// handoff.hip -- export and import of one owner's resident KV (the per-GPU
// halves of moving a request between executors).
//
// The reference migrates a request in "delta" mode (src/runtime/wla_multigpu.cuh:
// 1367-1428): the victim gathers the request's resident slots into a
// contiguous staging buffer (wla_slot_gather_kernel, :154-162), the buffer
// crosses the link, the consumer scatters it back to the same slot offsets
// (wla_slot_scatter_kernel, :163-171) and takes over the LRU state
// (kv_handoff, :1970-1994).  Here an owner's image holds, for each of its
// (layer, kv head) sets, the LRU fill, order and tags and the bytes of its
// resident slots, compacted in LRU order.  Resident slots are always
// [0, fill) (free slots are handed out in order and only reset returns them),
// so the importer keeps the exporter's slot ids and its state ends up equal
// bit for bit.
//
// Image layout (device memory, offsets in bytes from its start):
//   [0, 64)          header: magic, sets, slots_per_set, block_bytes, dtype,
//                    max_blocks, resident blocks (u64), member bit (0: the
//                    whole owner)
//   fill[sets], start[sets]                      u32 each
//   ord[sets * C], tag[sets * C], own[sets * C]  u32, per set from start[s]:
//                                                local slots in LRU order,
//                                                their blocks and member masks
//   scales[sets * C][2]                          fp32 (fp8 KV only)
//   data[sets * C][block_bytes]                  from a 256-byte boundary:
//                                                resident blocks, compacted
// Only data[0, resident) is filled; ferry_owner_image_bytes gives the
// capacity for a full owner.
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

constexpr uint32_t kImageMagic = 0x4E574F46u;  // "FOWN"

struct ImageHeader {
  uint32_t magic, sets, slots, bb, dtype, max_blocks;
  unsigned long long resident;
  uint32_t member_bit;  // 0: the whole owner; else the member whose exclusive blocks it holds
};

__device__ inline ImageLayout image_layout(const Geo& g) { return make_image_layout(g); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One block by one wavefront, NV 16-byte words per lane.  Both sides are
// streamed (non-temporal): each byte moves once, and the slots written here
// are next read by attention, whose own non-temporal loads run slower when
// the lines still sit in cache from ordinary stores.
template <int NV>
__device__ inline void copy_block(const uint8_t* src_b, uint8_t* dst_b, int lane) {
  const u32x4* src = reinterpret_cast<const u32x4*>(src_b);
  u32x4* dst = reinterpret_cast<u32x4*>(dst_b);
  u32x4 r[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) r[v] = __builtin_nontemporal_load(src + v * kWave + lane);
#pragma unroll
  for (int v = 0; v < NV; ++v) __builtin_nontemporal_store(r[v], dst + v * kWave + lane);
}

// Forget every block of one set (map entries of its tags, tags, order, fill).
// Every thread of the workgroup (NT threads) calls it; ends with a barrier.
// Thread t clears slots t, t + NT, ...: the map entry of its tag first, then
// the tag itself, so no thread needs another's writes in between.
template <int NT>
__device__ inline void clear_set(const Geo& g, SetState st, size_t set) {
  const uint32_t C = (uint32_t)g.C;
  uint32_t* map = st.map + set * (size_t)g.max_blocks;
  uint32_t* tag = st.tag + set * C;
  uint32_t* ord = st.ord + set * C;
  for (uint32_t i = threadIdx.x; i < C; i += NT) {
    const uint32_t b = aload(tag + i);  // other threads may have written it (L2 atomics)
    if (b < (uint32_t)g.max_blocks) map[b] = kNone;
    tag[i] = kNone;
    ord[i] = kNone;
    if (st.own) st.own[set * C + i] = 0u;
  }
  if (threadIdx.x == 0) st.fill[set] = 0;
  __syncthreads();
}

}  // namespace

// One workgroup of 256 threads: fill and start (exclusive prefix of the
// fills) of the owner's sets, and the header.  Thread t takes a run of
// consecutive sets; the runs' totals are scanned across the workgroup
// (wavefront shuffles, then the 4 wavefront totals through LDS).
__global__ __launch_bounds__(256) void k_owner_export_meta(Geo g, SetState st, uint32_t owner,
                                                           uint8_t* __restrict__ image,
                                                           const uint32_t* counts,
                                                           uint32_t member_bit) {
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv);
  uint32_t* fill = reinterpret_cast<uint32_t*>(image + lay.fill);
  uint32_t* start = reinterpret_cast<uint32_t*>(image + lay.start);
  __shared__ unsigned long long wsum[4];
  const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t per = (S + 255) / 256, s0 = min(S, t * per), s1 = min(S, s0 + per);
  unsigned long long run = 0;
  for (uint32_t s = s0; s < s1; ++s) {
    const uint32_t f = counts ? counts[s] : st.fill[(size_t)owner * S + s];
    fill[s] = f;
    run += f;
  }
  unsigned long long incl = run;
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned long long o = __shfl_up(incl, off);
    if ((int)lane >= off) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  unsigned long long acc = incl - run;
  for (uint32_t w = 0; w < wave; ++w) acc += wsum[w];
  for (uint32_t s = s0; s < s1; ++s) {
    start[s] = (uint32_t)acc;
    acc += fill[s];
  }
  if (t == 255) {
    ImageHeader* h = reinterpret_cast<ImageHeader*>(image);
    h->magic = kImageMagic;
    h->sets = S;
    h->slots = (uint32_t)g.C;
    h->bb = (uint32_t)g.bb;
    h->dtype = (uint32_t)g.dtype;
    h->max_blocks = (uint32_t)g.max_blocks;
    h->resident = acc;
    h->member_bit = member_bit;
  }
}

// One wavefront per (set, LRU position i): position i < fill copies its slot's
// block into the data area at start[set] + i (16-byte loads, NV per lane) and
// records slot, tag and fp8 scales.
template <int NV>
__global__ __launch_bounds__(256) void k_owner_export_data(Geo g, SetState st, uint32_t owner,
                                                           const uint8_t* __restrict__ pool,
                                                           const float* __restrict__ pool_scales,
                                                           uint8_t* __restrict__ image) {
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= (uint64_t)S * C) return;
  const uint32_t s = (uint32_t)(wave / C), i = (uint32_t)(wave % C);
  const uint32_t* fill = reinterpret_cast<const uint32_t*>(image + lay.fill);
  const uint32_t* start = reinterpret_cast<const uint32_t*>(image + lay.start);
  if (i >= fill[s]) return;
  const size_t set = (size_t)owner * S + s;
  const uint32_t slot = st.ord[set * C + i];
  const size_t pos = (size_t)start[s] + i;
  const size_t gslot = set * C + slot;
  if (lane == 0) {
    reinterpret_cast<uint32_t*>(image + lay.ord)[pos] = slot;
    reinterpret_cast<uint32_t*>(image + lay.tag)[pos] = st.tag[gslot];
    reinterpret_cast<uint32_t*>(image + lay.own)[pos] = st.own ? st.own[gslot] : 0u;
    if (pool_scales) {
      reinterpret_cast<float*>(image + lay.scales)[2 * pos] = pool_scales[2 * gslot];
      reinterpret_cast<float*>(image + lay.scales)[2 * pos + 1] = pool_scales[2 * gslot + 1];
    }
  }
  copy_block<NV>(pool + gslot * g.bb, image + lay.data + pos * g.bb, lane);
}

// One workgroup of 256 threads per set of the importing owner (one
// wavefront per set left each CU a single wavefront walking up to C entries):
// forget the set's blocks, check the image against this executor's geometry,
// then take the image's fill, order, tags and map entries.  A mismatching or
// malformed image latches FERRY_EINVAL and leaves the set empty (so the data
// kernel writes nothing).  Words other threads wrote are read with L1-bypassing
// atomics after a barrier.
__global__ __launch_bounds__(256) void k_owner_import_meta(Geo g, SetState st, uint32_t owner,
                                                           const uint8_t* __restrict__ image,
                                                           int* __restrict__ err) {
  constexpr int NT = 256;
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint32_t s = blockIdx.x;
  const uint32_t tid = threadIdx.x;
  if (s >= S) return;  // uniform
  const ImageHeader* h = reinterpret_cast<const ImageHeader*>(image);
  const uint32_t* fill = reinterpret_cast<const uint32_t*>(image + lay.fill);
  const uint32_t* start = reinterpret_cast<const uint32_t*>(image + lay.start);
  const uint32_t* iord = reinterpret_cast<const uint32_t*>(image + lay.ord);
  const uint32_t* itag = reinterpret_cast<const uint32_t*>(image + lay.tag);
  const size_t set = (size_t)owner * S + s;
  clear_set<NT>(g, st, set);
  const bool hdr_ok = h->magic == kImageMagic && h->sets == S && h->slots == C &&
                      h->bb == (uint32_t)g.bb && h->dtype == (uint32_t)g.dtype &&
                      h->max_blocks == (uint32_t)g.max_blocks && h->member_bit == 0u &&
                      h->resident <= (unsigned long long)S * C;
  const uint32_t f = hdr_ok ? fill[s] : 0, p0 = hdr_ok ? start[s] : 0;
  bool bad = !hdr_ok || f > C || (unsigned long long)p0 + f > h->resident;
  for (uint32_t i = tid; i < f && !bad; i += NT)
    bad |= iord[p0 + i] >= f || itag[p0 + i] >= (uint32_t)g.max_blocks;
  if (__syncthreads_or(bad)) {  // uniform
    if (tid == 0) set_error(err, FERRY_EINVAL);
    return;
  }
  uint32_t* map = st.map + set * (size_t)g.max_blocks;
  uint32_t* tag = st.tag + set * C;
  uint32_t* ord = st.ord + set * C;
  const uint32_t* iown = reinterpret_cast<const uint32_t*>(image + lay.own);
  for (uint32_t i = tid; i < f; i += NT) {
    const uint32_t slot = iord[p0 + i], b = itag[p0 + i];
    ord[i] = slot;
    astore(tag + slot, b);
    astore(map + b, slot);
    if (st.own) st.own[set * C + slot] = iown[p0 + i];
  }
  __syncthreads();
  // The order must be a permutation of [0, f) with distinct blocks: a repeated
  // slot leaves some slot below f untagged, and a slot or block repeated with
  // another partner fails to read back through tag or map.
  bool dup = false;
  for (uint32_t i = tid; i < f; i += NT) {
    const uint32_t slot = iord[p0 + i], b = itag[p0 + i];
    dup |= aload(tag + slot) != b || aload(map + b) != slot || aload(tag + i) == kNone;
  }
  if (__syncthreads_or(dup)) {  // uniform
    clear_set<NT>(g, st, set);
    if (tid == 0) set_error(err, FERRY_EINVAL);
    return;
  }
  if (tid == 0) st.fill[set] = f;
}

// One wavefront per (set, LRU position i < fill): the image block goes back to
// its slot (and its fp8 scales).  Runs after k_owner_import_meta validated the
// image; a set it refused has fill 0 in the importer and nothing is written.
template <int NV>
__global__ __launch_bounds__(256) void k_owner_import_data(Geo g, SetState st, uint32_t owner,
                                                           uint8_t* __restrict__ pool,
                                                           float* __restrict__ pool_scales,
                                                           const uint8_t* __restrict__ image) {
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wave >= (uint64_t)S * C) return;
  const uint32_t s = (uint32_t)(wave / C), i = (uint32_t)(wave % C);
  const size_t set = (size_t)owner * S + s;
  const uint32_t f = st.fill[set];  // 0 unless the meta kernel accepted the image
  if (i >= f) return;
  const size_t pos = (size_t)reinterpret_cast<const uint32_t*>(image + lay.start)[s] + i;
  const uint32_t slot = reinterpret_cast<const uint32_t*>(image + lay.ord)[pos];
  const size_t gslot = set * C + slot;
  if (lane == 0 && pool_scales) {
    pool_scales[2 * gslot] = reinterpret_cast<const float*>(image + lay.scales)[2 * pos];
    pool_scales[2 * gslot + 1] = reinterpret_cast<const float*>(image + lay.scales)[2 * pos + 1];
  }
  copy_block<NV>(image + lay.data + pos * g.bb, pool + gslot * g.bb, lane);
}

// ---- member carry (kv_handoff_owned, src/runtime/wla_multigpu.cuh:1901-1921) ----
// One wavefront per set of the owner: how many resident blocks only member
// `bit` touched (own == bit) -> the image's fill[set].
__global__ __launch_bounds__(256) void k_member_export_count(Geo g, SetState st, uint32_t owner,
                                                             uint32_t bit, uint8_t* __restrict__ image) {
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint32_t s = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (s >= S) return;
  const size_t set = (size_t)owner * S + s;
  const uint32_t f = st.fill[set];
  uint32_t n = 0;
  for (uint32_t c = 0; c < f; c += kWave) {
    const uint32_t i = c + lane;
    n += (uint32_t)__builtin_popcountll(ballot(i < f && st.own[set * C + st.ord[set * C + i]] == bit));
  }
  if (lane == 0) reinterpret_cast<uint32_t*>(image + lay.fill)[s] = n;
}

// One wavefront per set: the member's exclusive blocks in LRU order, each
// written at start[set] + its rank (slot, tag, mask, fp8 scales, data).
template <int NV>
__global__ __launch_bounds__(256) void k_member_export_data(Geo g, SetState st, uint32_t owner,
                                                            uint32_t bit,
                                                            const uint8_t* __restrict__ pool,
                                                            const float* __restrict__ pool_scales,
                                                            uint8_t* __restrict__ image) {
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint32_t s = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (s >= S) return;
  const size_t set = (size_t)owner * S + s;
  const uint32_t f = st.fill[set];
  size_t pos = reinterpret_cast<const uint32_t*>(image + lay.start)[s];
  for (uint32_t c = 0; c < f; c += kWave) {
    const uint32_t i = c + lane;
    const uint32_t slot = i < f ? st.ord[set * C + i] : 0u;
    uint64_t mask = ballot(i < f && st.own[set * C + slot] == bit);
    while (mask) {  // wavefront-uniform: one block at a time, all lanes copy
      const int b = __builtin_ctzll(mask);
      mask &= mask - 1;
      const uint32_t v = (uint32_t)__shfl((int)slot, b);
      const size_t gslot = set * C + v;
      if (lane == 0) {
        reinterpret_cast<uint32_t*>(image + lay.ord)[pos] = v;
        reinterpret_cast<uint32_t*>(image + lay.tag)[pos] = st.tag[gslot];
        reinterpret_cast<uint32_t*>(image + lay.own)[pos] = bit;
        if (pool_scales) {
          reinterpret_cast<float*>(image + lay.scales)[2 * pos] = pool_scales[2 * gslot];
          reinterpret_cast<float*>(image + lay.scales)[2 * pos + 1] = pool_scales[2 * gslot + 1];
        }
      }
      copy_block<NV>(pool + gslot * g.bb, image + lay.data + pos * g.bb, lane);
      ++pos;
    }
  }
}

// One wavefront per set of the importing owner merges the image's blocks in
// their order: a block already resident gains the member's bit and keeps its
// place; another becomes the most recent, taking the least recent block's
// slot when the set holds its capacity, else slot fill (resident slots stay
// [0, fill)).  The set's order is kept in LDS (2 C words: evictions advance
// its head).  A mismatching image, a count above C, a block id out of range or
// a set already above its capacity latch FERRY_EINVAL and stop that set.
template <int NV>
__global__ __launch_bounds__(64) void k_member_import(Geo g, SetState st, uint32_t owner, uint32_t bit,
                                                      uint8_t* __restrict__ pool,
                                                      float* __restrict__ pool_scales,
                                                      const uint8_t* __restrict__ image,
                                                      int* __restrict__ err) {
  extern __shared__ uint32_t lds[];  // [2 C]
  const ImageLayout lay = image_layout(g);
  const uint32_t S = (uint32_t)(g.L * g.Hkv), C = (uint32_t)g.C;
  const uint32_t s = blockIdx.x;
  const int lane = threadIdx.x;
  const ImageHeader* h = reinterpret_cast<const ImageHeader*>(image);
  const size_t set = (size_t)owner * S + s;
  const uint32_t cap = set_capacity(g, st.members[owner]);
  uint32_t fill = st.fill[set];
  const bool hdr_ok = h->magic == kImageMagic && h->sets == S && h->slots == C &&
                      h->bb == (uint32_t)g.bb && h->dtype == (uint32_t)g.dtype &&
                      h->max_blocks == (uint32_t)g.max_blocks && h->member_bit != 0u;
  const uint32_t n = hdr_ok ? reinterpret_cast<const uint32_t*>(image + lay.fill)[s] : 0u;
  const size_t p0 = hdr_ok ? reinterpret_cast<const uint32_t*>(image + lay.start)[s] : 0u;
  if (!hdr_ok || n > C || fill > cap || p0 + n > h->resident) {
    if (lane == 0) set_error(err, FERRY_EINVAL);
    return;
  }
  const uint32_t* itag = reinterpret_cast<const uint32_t*>(image + lay.tag);
  uint32_t* map = st.map + set * (size_t)g.max_blocks;
  uint32_t* tag = st.tag + set * C;
  uint32_t* ord = st.ord + set * C;
  uint32_t* own = st.own + set * C;
  for (uint32_t i = lane; i < fill; i += kWave) lds[i] = ord[i];
  __builtin_amdgcn_wave_barrier();
  uint32_t head = 0;
  for (uint32_t j = 0; j < n; ++j) {  // wavefront-uniform
    const uint32_t x = itag[p0 + j];
    if (x >= (uint32_t)g.max_blocks) {
      if (lane == 0) set_error(err, FERRY_EINVAL);
      break;
    }
    const uint32_t r = aload(map + x);
    if (r < C) {  // already resident: only the member's bit
      if (lane == 0) own[r] |= bit;
      continue;
    }
    uint32_t v = fill;
    if (fill >= cap) {  // the least recent block leaves; its slot takes the new one
      v = lds[head++];
      if (lane == 0) astore(map + tag[v], kNone);
      --fill;
    }
    if (lane == 0) {
      tag[v] = x;
      astore(map + x, v);
      own[v] = bit;
      lds[head + fill] = v;
      if (pool_scales) {
        pool_scales[2 * (set * C + v)] = reinterpret_cast<const float*>(image + lay.scales)[2 * (p0 + j)];
        pool_scales[2 * (set * C + v) + 1] =
            reinterpret_cast<const float*>(image + lay.scales)[2 * (p0 + j) + 1];
      }
    }
    ++fill;
    wave_fence();
    copy_block<NV>(image + lay.data + (p0 + j) * g.bb, pool + (set * C + v) * g.bb, lane);
  }
  __builtin_amdgcn_wave_barrier();
  for (uint32_t i = lane; i < C; i += kWave) ord[i] = i < fill ? lds[head + i] : kNone;
  if (lane == 0) st.fill[set] = fill;
}

#define FERRY_HANDOFF_INST(NV)                                                                    \
  template __global__ void k_owner_export_data<NV>(Geo, SetState, uint32_t, const uint8_t*,       \
                                                   const float*, uint8_t*);                        \
  template __global__ void k_owner_import_data<NV>(Geo, SetState, uint32_t, uint8_t*, float*,     \
                                                   const uint8_t*);
FERRY_HANDOFF_INST(4)
FERRY_HANDOFF_INST(8)
FERRY_HANDOFF_INST(16)

#define FERRY_MEMBER_INST(NV)                                                                      \
  template __global__ void k_member_export_data<NV>(Geo, SetState, uint32_t, uint32_t,             \
                                                    const uint8_t*, const float*, uint8_t*);        \
  template __global__ void k_member_import<NV>(Geo, SetState, uint32_t, uint32_t, uint8_t*, float*, \
                                               const uint8_t*, int*);
FERRY_MEMBER_INST(4)
FERRY_MEMBER_INST(8)
FERRY_MEMBER_INST(16)

}  // namespace ferry_amd
