// common.hpp -- shared definitions of the MI355X (gfx950) miss-stream executor.
//
// Host and device code both include this file: geometry, wave64 primitives,
// the counter-based hash, the KV element codecs and the host-tier content
// function (the content must be bit-identical wherever it is generated).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ferry_amd.h"

namespace ferry_amd {

constexpr uint32_t kNone = 0xFFFFFFFFu;
constexpr uint32_t kPend = 0x80000000u;  // map entry: pending miss, low bits = position
constexpr int kWave = 64;
// Largest top-k per (request, layer, kv head): the attention kernels stage a
// row's slot ids in LDS (4 KiB).
constexpr int kMaxTopK = 1024;

// Immutable executor geometry, passed to kernels by value.
struct Geo {
  int n_req, group, L, Hkv, Hq, D, T, k, C, max_blocks;
  int n_owners, n_sets, max_sel, dtype, esize, workers;
  int cap_mode;      // FERRY_CAP_GROUP or FERRY_CAP_PER_MEMBER
  int member_slots;  // C / group: one resident member's share under FERRY_CAP_PER_MEMBER
  uint64_t bb;           // K+V bytes of one block
  uint64_t host_blocks;  // host tier capacity (blocks)
  uint64_t pool_slots;   // n_sets * C
};

// ------------------------------------------------------------------ hashing
// splitmix64 finaliser over seed + idx * golden gamma (Vigna).
__host__ __device__ inline uint64_t mix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + idx * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Salts of the synthetic streams (one per independent draw family).
constexpr uint64_t kSaltCtx = 0x43545842ull;
constexpr uint64_t kSaltSel = 0x53454C31ull;
constexpr uint64_t kSaltPerm = 0x5045524Dull;
constexpr uint64_t kSaltHost = 0x484F5354ull;
constexpr uint64_t kSaltScale = 0x5343414Cull;
constexpr uint64_t kSaltKeep = 0x4B454550ull;

// ------------------------------------------------------------------ codecs
__host__ __device__ inline uint32_t f32_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
__host__ __device__ inline float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// binary32 -> binary16, round to nearest even.
__host__ __device__ inline uint16_t f32_to_f16(float x) {
  const uint32_t u = f32_bits(x);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t exp = (u >> 23) & 0xFFu;
  const uint32_t man = u & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (man ? 0x200u : 0u);
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t m = man | 0x800000u;
    const int shift = 14 - e;
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return sign | (uint16_t)q;
}

// binary32 -> bfloat16, round to nearest even.
__host__ __device__ inline uint16_t f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// binary32 -> OCP E4M3FN, round to nearest even, saturating at +-448.
__host__ __device__ inline uint8_t f32_to_e4m3(float x) {
  const uint32_t u = f32_bits(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;
  if (bits_f32(a) >= 464.0f) return sign | 0x7Eu;
  int e = (int)(a >> 23) - 127;
  if (e < -6) {
    const float n = __builtin_rintf(bits_f32(a) * 512.0f);
    return sign | (uint8_t)n;
  }
  const uint32_t man = a & 0x7FFFFFu;
  uint32_t q = man >> 20;
  const uint32_t rem = man & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
  if (q == 8u) {
    q = 0;
    e++;
  }
  return sign | (uint8_t)(((uint32_t)(e + 7) << 3) | q);
}

__host__ __device__ inline int32_t irwin_hall(uint64_t w) {
  return (int32_t)(w & 0xFFFFu) + (int32_t)((w >> 16) & 0xFFFFu) +
         (int32_t)((w >> 32) & 0xFFFFu) + (int32_t)(w >> 48) - 131070;
}

// Encoded element e of host block h.  Values are Irwin-Hall(4) sums of
// 16-bit uniforms, centred, times `mult` (= std / (65536/sqrt 3) as a float);
// fp8 stores codes of standard deviation 96 (mult8) and a per-block scale.
__host__ __device__ inline uint32_t host_elem(int dtype, uint64_t seed, uint64_t elems_per_block,
                                              uint64_t h, uint32_t e, float mult, float mult8) {
  const int32_t sv = irwin_hall(mix64(seed ^ kSaltHost, h * elems_per_block + e));
  if (dtype == FERRY_FP8_E4M3) return f32_to_e4m3((float)sv * mult8);
  const float x = (float)sv * mult;
  if (dtype == FERRY_F32) return f32_bits(x);
  if (dtype == FERRY_F16) return f32_to_f16(x);
  return f32_to_bf16(x);
}

__host__ __device__ inline float host_scale(int dtype, uint64_t seed, uint64_t h, int kv, float base) {
  if (dtype != FERRY_FP8_E4M3) return 1.0f;
  const uint64_t u = mix64(seed ^ kSaltScale, h * 2ull + (uint64_t)kv) >> 56;
  return base * (0.75f + (float)u / 512.0f);
}

// Host-tier index of (set, block): set*max_blocks + block, aliased modulo the
// tier capacity (the reference addresses its slab `block % cap`).
__host__ __device__ inline uint64_t host_index(uint64_t set, uint32_t block, uint64_t max_blocks,
                                               uint64_t host_blocks) {
  return (set * max_blocks + block) % host_blocks;
}

#if defined(__HIPCC__)
// ------------------------------------------------------------------ wave64 primitives
__device__ inline int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }
// Number of set bits of `mask` strictly below this lane.
__device__ inline int lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}
__device__ inline uint64_t ballot(bool p) { return __ballot(p); }
__device__ inline int first_lane_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ inline uint32_t first_lane_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ inline uint64_t first_lane_u64(uint64_t v) {
  const uint32_t lo = first_lane_u((uint32_t)v), hi = first_lane_u((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
// Ordering point for one wavefront's global + LDS traffic between phases.
// Every word that other lanes rewrite is read with an L1-bypassing relaxed
// atomic (aload) and written with atomics that complete in L2, so waiting for
// this wave's outstanding accesses (workgroup scope: s_waitcnt, no L2
// writeback or invalidate) is all the ordering one wavefront needs.
__device__ inline void wave_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}
// L1-bypassing relaxed accesses for words other lanes of the wave rewrite.
__device__ inline uint32_t aload(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void astore(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint64_t aload64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void astore64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Record the first error code (FERRY_E*) seen on the device.
__device__ inline void set_error(int* err, int code) { atomicCAS(err, 0, code); }
#endif

}  // namespace ferry_amd
