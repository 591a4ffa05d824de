// attn_common.hpp -- device helpers shared by the attention kernels and the
// matrix-core selection kernel.
#pragma once

#include "common.hpp"

namespace ferry_amd {

// A K/V load of the attention kernels.  NT = non-temporal: the line is
// streamed (inserted for early eviction) instead of kept, which lifts random
// 8 KiB block gathers on MI355X from ~6.2 to ~6.9 TB/s when nothing re-reads
// the block soon.  Blocks shared by the rows of one launch (prefix groups) are
// loaded temporally so the later rows hit in cache.
template <bool NT, typename T>
__device__ inline T load_kv(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

typedef uint32_t mx_u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 mx_f16x2 __attribute__((ext_vector_type(2)));

// 4 OCP E4M3 codes (one dword) -> 4 exact fp16 values (two dwords).
__device__ inline mx_u32x2 e4m3x4_to_f16(uint32_t w) {
  const mx_f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
  const mx_f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
  return mx_u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

// The two values of lane l's pair (l, l ^ 16) (X = 16) or (l, l ^ 32) (X = 32),
// the lower lane's first, on both lanes of the pair: with the same value in
// both operands, gfx950's v_permlane16_swap / v_permlane32_swap exchange
// those lanes on the VALU (lane layout checked on MI355X), where __shfl_xor
// takes an LDS permute and a wait.
template <int X>
__device__ inline mx_u32x2 pair_values(float x) {
  static_assert(X == 16 || X == 32, "lane distance 16 or 32");
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  if constexpr (X == 16) return __builtin_amdgcn_permlane16_swap(u, u, false, false);
  else return __builtin_amdgcn_permlane32_swap(u, u, false, false);
}

// Max / sum over lanes n, n + 16, n + 32, n + 48 (the four 16-lane groups),
// on every one of them.  The same bits as two __shfl_xor steps (16, then 32):
// max and a two-term sum do not depend on the operands' order.
__device__ inline float max_over_groups(float x) {
#pragma unroll
  for (int X = 16; X <= 32; X *= 2) {
    const mx_u32x2 p = X == 16 ? pair_values<16>(x) : pair_values<32>(x);
    x = fmaxf(__builtin_bit_cast(float, (uint32_t)p[0]), __builtin_bit_cast(float, (uint32_t)p[1]));
  }
  return x;
}
__device__ inline float sum_over_groups(float x) {
#pragma unroll
  for (int X = 16; X <= 32; X *= 2) {
    const mx_u32x2 p = X == 16 ? pair_values<16>(x) : pair_values<32>(x);
    x = __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
  }
  return x;
}

// A slot's two fp8 scales (K, V) by a vector load, counted on vmcnt in order
// with the block's own loads.  The address is wavefront-uniform, so the
// compiler would make it a scalar load, whose counter (lgkmcnt) it shares with
// the LDS reads and can only be waited for whole: the wait before the next
// LDS read or block would then include the scales just issued for a block
// further ahead.  An opaque zero in a VGPR keeps the address per lane.
__device__ inline float2 load_scales(const float* p) {
  int z;
  asm("v_mov_b32 %0, 0" : "=v"(z));
  return *reinterpret_cast<const float2*>(p + z);
}

// fp32 -> bf16 bits, round to nearest even (finite inputs)
__device__ inline uint16_t bf16_rne(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Stage the k slot ids of one (request, layer, kv head) row in LDS `ids`,
// dropping empty positions (kNone) and keeping the order of the others, and
// return how many were kept.  A row of a request that is not resident this
// step is all kNone (0 kept); a short context gives a ragged row.
// Every thread of the W-wavefront workgroup must call it: each thread holds
// up to kMaxTopK / (64 W) ids in registers and stores them in place, and each
// wavefront counts its 64-id chunks with a ballot.  After one barrier every
// thread sums the counts; when all k ids are kept (a full row, the common
// case) the in-place copy is the answer.  Otherwise (a workgroup-uniform
// branch) every kept id is rewritten at (ids kept in earlier chunks) + (kept
// lanes below it in its chunk), behind a second barrier.  `cnt` is LDS
// scratch of kMaxTopK / 64 ints.  Ends with a barrier.
template <int W>
__device__ inline int stage_row_ids(const uint32_t* __restrict__ sl, int k, uint32_t* ids,
                                    int* cnt) {
  constexpr int NT = W * 64;
  constexpr int PER = kMaxTopK / NT;
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = tid + i * NT;
    v[i] = j < k ? sl[j] : kNone;
    if (j < k) ids[j] = v[i];
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = tid + i * NT;  // chunk j / 64 is the same for the whole wavefront
    const uint64_t m = ballot(v[i] != kNone);
    if (lane == 0) cnt[j >> 6] = __builtin_popcountll(m);
  }
  __syncthreads();
  const int nchunks = (k + 63) >> 6;
  int total = 0;
  for (int c = 0; c < nchunks; ++c) total += cnt[c];
  if (total == k) return total;  // uniform: every thread read the same counts
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int j = tid + i * NT;
    const bool keep = v[i] != kNone;
    const uint64_t m = ballot(keep);
    if (j < k && keep) {
      int base = 0;
      for (int c = 0; c < (j >> 6); ++c) base += cnt[c];
      ids[base + lanes_below(m)] = v[i];
    }
  }
  __syncthreads();
  return total;
}

}  // namespace ferry_amd
