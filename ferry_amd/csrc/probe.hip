// probe.hip -- bandwidth ceilings for the roofline.
//
// The executor's kernels are bound by HBM (attention) and by the host link
// (fetch).  These probes move the same bytes with no other work, so a kernel's
// achieved rate can be read against what plain reads reach on the same part:
//  * k_probe_gather: the attention kernels' loads (the k pool slots of every
//    (request, layer, kv head) row, ids staged in LDS, a two-block ring per
//    wavefront, non-temporal 16-byte loads) with the softmax and products
//    replaced by an XOR;
//  * k_probe_host: device-direct 16-byte reads of consecutive host-tier
//    blocks over the host link, as the fetch kernel issues them, without the
//    ring bookkeeping or the pool writes;
//  * k_probe_copy: a streaming device copy of consecutive pool blocks
//    (non-temporal 16-byte loads and stores), the ceiling of the owner
//    hand-off, which reads and writes every resident block once;
//  * k_probe_ktab: the mass selection's reads of the dense K table (every
//    record of the first n blocks of every set, kv head by kv head of each
//    (request, layer) item) with its grid, wavefronts and four records in
//    flight per wavefront, the scores replaced by an XOR.
// They play the role of the reference's host-staged bandwidth sweep
// (probe_host_staged_bandwidth, src/topo/topo.cpp:68-129), measured here for
// the one-hop device-direct path instead of the two-hop pinned ring.
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
}

template <int NLD>
__global__ __launch_bounds__(256) void k_probe_gather(const uint8_t* __restrict__ pool, uint64_t bb,
                                                      const uint32_t* __restrict__ slots, int k,
                                                      uint64_t pool_slots,
                                                      uint32_t* __restrict__ sink) {
  constexpr int W = 4, NPF = 2;
  __shared__ uint32_t ids[kMaxTopK];
  __shared__ uint32_t red[W];
  const int row = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t* sl = slots + (size_t)row * k;
  for (int j = threadIdx.x; j < k; j += W * 64) ids[j] = sl[j];
  __syncthreads();
  const int nb = k > wave ? (k - wave + W - 1) / W : 0;
  u32x4 buf[NPF][NLD];
  auto issue = [&](int j, int b) {
    uint64_t slot = (uint32_t)__builtin_amdgcn_readfirstlane((int)ids[wave + W * min(j, nb - 1)]);
    slot = slot < pool_slots ? slot : 0;
    const u32x4* p = reinterpret_cast<const u32x4*>(pool + slot * bb);
    const int live = j < nb ? 1 : 0;  // past the end: one line per instruction
#pragma unroll
    for (int ld = 0; ld < NLD; ++ld)
      buf[b][ld] = __builtin_nontemporal_load(p + (ld * 64 + lane) * live);
  };
  u32x4 acc = {0u, 0u, 0u, 0u};
  if (nb > 0) {
    issue(0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int i0 = 0; i0 < nb; i0 += NPF) {
#pragma unroll
    for (int b = 0; b < NPF; ++b) {
      const int i = i0 + b;
      if (i >= nb) break;
      issue(i + 1, (b + 1) % NPF);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ld = 0; ld < NLD; ++ld) acc ^= buf[b][ld];
    }
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  if (lane == 0) red[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[row] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

template <int NV>
__global__ __launch_bounds__(256) void k_probe_host(const uint8_t* __restrict__ host, uint64_t bb,
                                                    uint64_t n_blocks, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint64_t n_waves = (uint64_t)gridDim.x * (blockDim.x >> 6);
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (uint64_t b = wave; b < n_blocks; b += n_waves) {
    const u32x4* src = reinterpret_cast<const u32x4*>(host + b * bb);
    u32x4 r[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) r[i] = __builtin_nontemporal_load(src + i * kWave + lane);
#pragma unroll
    for (int i = 0; i < NV; ++i) acc ^= r[i];
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  if (lane == 0) sink[wave] = x;
}

template <int NV>
__global__ __launch_bounds__(256) void k_probe_copy(const uint8_t* __restrict__ src,
                                                    uint8_t* __restrict__ dst, uint64_t bb,
                                                    uint64_t n_blocks) {
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint64_t n_waves = (uint64_t)gridDim.x * (blockDim.x >> 6);
  for (uint64_t b = wave; b < n_blocks; b += n_waves) {
    const u32x4* s = reinterpret_cast<const u32x4*>(src + b * bb);
    u32x4* d = reinterpret_cast<u32x4*>(dst + b * bb);
    u32x4 r[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) r[i] = __builtin_nontemporal_load(s + i * kWave + lane);
#pragma unroll
    for (int i = 0; i < NV; ++i) __builtin_nontemporal_store(r[i], d + i * kWave + lane);
  }
}

// The mass selection's K-table reads without its scores: NI 1 KiB loads per
// record, U records in flight per wavefront, blocks [0, nb) of every set.
// UNITS = 1: one (request, layer, kv head) set per workgroup pass, as
// k_mass_units; UNITS = 0: a (request, layer) item's kv heads one after the
// other per workgroup, as k_select_mass.
template <int NI, int W, int U, int UNITS>
__global__ __launch_bounds__(W * 64) void k_probe_ktab(Geo g, const uint8_t* __restrict__ kt,
                                                      uint64_t kt_mod, int nb,
                                                      uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_work = UNITS ? g.n_req * g.L * g.Hkv : g.n_req * g.L;
  const int hs = UNITS ? 1 : g.Hkv;  // sets per work item
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int wi = blockIdx.x; wi < n_work; wi += gridDim.x) {
    for (int h = 0; h < hs; ++h) {
      const uint64_t set = (uint64_t)wi * hs + h;
      for (int b0 = wave; b0 < nb; b0 += W * U) {
        u32x4 w[U][NI];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = b0 + W * u;
          if (b < nb) {  // wavefront-uniform
            const uint64_t rec = host_index(set, (uint32_t)b, (uint64_t)g.max_blocks, kt_mod);
            const u32x4* base = reinterpret_cast<const u32x4*>(kt) + rec * (64 * NI) + lane;
#pragma unroll
            for (int i = 0; i < NI; ++i) w[u][i] = __builtin_nontemporal_load(base + 64 * i);
          } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) w[u][i] = u32x4{0u, 0u, 0u, 0u};
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int i = 0; i < NI; ++i) acc ^= w[u][i];
      }
    }
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  if (lane == 0) sink[(size_t)blockIdx.x * W + wave] = x;
}

// The Quest selection's summary reads without the scores: one workgroup of
// four wavefronts per (request, layer, kv head) set, blocks [0, nb) of it,
// sixteen lanes per record, each lane the same bytes of the record's min and
// max halves as k_select_topk's loads (16-bit: 16 B of each, fp8: 8 B, fp32:
// 32 B), U passes of four records per wavefront in flight.
template <int ES, int U>
__global__ __launch_bounds__(256) void k_probe_sums(Geo g, const uint8_t* __restrict__ sums,
                                                   uint64_t sum_mod, int nb,
                                                   uint32_t* __restrict__ sink) {
  constexpr int D = 128, W = 4, REC = 2 * D * ES, LB = 8 * ES;  // bytes per lane and half
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane >> 4, p = lane & 15;
  const uint64_t set = blockIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int b0 = 4 * wave; b0 < nb; b0 += 4 * W * U) {
    u32x4 lo[U][LB / 16 > 0 ? LB / 16 : 1], hi[U][LB / 16 > 0 ? LB / 16 : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int b = b0 + 4 * W * u + grp;
      const uint64_t rec = host_index(set, b < nb ? (uint32_t)b : 0u, (uint64_t)g.max_blocks, sum_mod);
      const uint8_t* r = sums + rec * REC;
      if constexpr (LB == 8) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 a = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(r + LB * p));
        const u32x2 c = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(r + D * ES + LB * p));
        lo[u][0] = u32x4{a[0], a[1], 0u, 0u};
        hi[u][0] = u32x4{c[0], c[1], 0u, 0u};
      } else {
#pragma unroll
        for (int i = 0; i < LB / 16; ++i) {
          lo[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r + LB * p) + i);
          hi[u][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(r + D * ES + LB * p) + i);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < (LB / 16 > 0 ? LB / 16 : 1); ++i) acc ^= lo[u][i] ^ hi[u][i];
  }
  uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x ^= __shfl_xor(x, off);
  if (lane == 0) sink[(size_t)blockIdx.x * W + wave] = x;
}

template __global__ void k_probe_sums<1, 2>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_sums<1, 4>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_sums<2, 2>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_sums<2, 4>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_sums<4, 2>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_sums<4, 4>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_ktab<2, kMassUnitWaves, kMassUnitInflight, 1>(Geo, const uint8_t*,
                                                                              uint64_t, int, uint32_t*);
template __global__ void k_probe_ktab<4, kMassUnitWaves, kMassUnitInflight, 1>(Geo, const uint8_t*,
                                                                              uint64_t, int, uint32_t*);
template __global__ void k_probe_ktab<8, 4, 4, 0>(Geo, const uint8_t*, uint64_t, int, uint32_t*);
template __global__ void k_probe_gather<4>(const uint8_t*, uint64_t, const uint32_t*, int, uint64_t,
                                           uint32_t*);
template __global__ void k_probe_gather<8>(const uint8_t*, uint64_t, const uint32_t*, int, uint64_t,
                                           uint32_t*);
template __global__ void k_probe_gather<16>(const uint8_t*, uint64_t, const uint32_t*, int,
                                            uint64_t, uint32_t*);
template __global__ void k_probe_host<4>(const uint8_t*, uint64_t, uint64_t, uint32_t*);
template __global__ void k_probe_host<8>(const uint8_t*, uint64_t, uint64_t, uint32_t*);
template __global__ void k_probe_host<16>(const uint8_t*, uint64_t, uint64_t, uint32_t*);
template __global__ void k_probe_copy<4>(const uint8_t*, uint8_t*, uint64_t, uint64_t);
template __global__ void k_probe_copy<8>(const uint8_t*, uint8_t*, uint64_t, uint64_t);
template __global__ void k_probe_copy<16>(const uint8_t*, uint8_t*, uint64_t, uint64_t);

}  // namespace ferry_amd
