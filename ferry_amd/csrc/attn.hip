// attn.hip -- block-sparse decode attention over the selected pool slots.
//
// out[r,l,hq] = softmax(q K^T / sqrt(D)) V over every token of the k blocks
// selected for (r, l, kv head of hq).  The reference has no attention (an FMA
// proxy at src/workloads/kv_exec.cuh:30-37); this is textbook attention with
// the per-step top-k block selection of tools/capture_miss_trace.py:139-159.
//
// Work decomposition (HBM-bound, ~1-8 flop/byte): one workgroup per
// (request, layer, kv head); its W wavefronts take every W-th selected block.  A block is K[T][D] then V[T][D].  Each 16-byte load instruction of a
// wavefront covers one contiguous KiB of the tile, so lane l holds the
// EPV-element dim chunk (l % LPT) of token (l / LPT) + ld * TPL.  The q.K dot
// product is reduced over the LPT lanes of a row with DPP row ops (no LDS);
// every row of lanes then runs its own online softmax over the tokens it
// holds, and rows, then wavefronts, are merged at the end.  Q heads of one kv
// head (GQA group G) share every K/V load.
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ inline float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// Sum over groups of N consecutive lanes; every lane of the group gets the
// total.  Mirror/half-mirror pairings partition a row like xor 8 / xor 4 do.
template <int N>
__device__ inline float group_sum(float v) {
  if constexpr (N >= 32) v += __shfl_xor(v, 16);
  if constexpr (N >= 16) v += dpp<kRowMirror>(v);
  if constexpr (N >= 8) v += dpp<kRowHalfMirror>(v);
  if constexpr (N >= 4) v += dpp<kQuadXor2>(v);
  if constexpr (N >= 2) v += dpp<kQuadXor1>(v);
  return v;
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Decode the EPV elements of one 16-byte word to float.  fp8 E4M3 is widened
// through binary16 (same mantissa, exponent bias 15 instead of 7), which
// leaves a factor 2^-8 that the caller folds into the block scale.
template <int DT>
__device__ inline void decode(const u32x4& w, float* f) {
  if constexpr (DT == FERRY_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = w[i];  // bit_cast of a vector element would read element 0
      f[i] = __builtin_bit_cast(float, u);
    }
  } else if constexpr (DT == FERRY_F16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFFu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  } else if constexpr (DT == FERRY_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
      f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t v = (w[i] >> (8 * b)) & 0xFFu;
        const uint16_t h = (uint16_t)(((v & 0x80u) << 8) | ((v & 0x7Fu) << 7));
        f[4 * i + b] = (float)__builtin_bit_cast(_Float16, h);
      }
    }
  }
}

struct Softmax {
  float m, l;
};

}  // namespace

template <int DT, int G, int W, bool NT>
__global__ __launch_bounds__(W * 64) void k_attn(Geo g, const float* __restrict__ q,
                                              const uint32_t* __restrict__ slots,
                                              const uint8_t* __restrict__ pool,
                                              const float* __restrict__ pool_scales,
                                              float* __restrict__ out, float qscale, int l0,
                                              int nl, int* __restrict__ err) {
  constexpr int ES = DT == FERRY_F32 ? 4 : (DT == FERRY_FP8_E4M3 ? 1 : 2);
  constexpr int D = 128, T = 16;
  constexpr int EPV = 16 / ES;   // elements per 16-byte word
  constexpr int LPT = D / EPV;   // lanes per token row
  constexpr int TPL = 64 / LPT;  // tokens per load instruction
  constexpr int NLD = T / TPL;   // load instructions per K (or V) tile
  constexpr uint32_t TILE_WORDS = T * D * ES / 16;
  constexpr float kNeg = -1.0e30f;
  constexpr int NPF = G <= 2 ? 2 : 1;  // prefetch ring depth (wide groups keep occupancy)

  __shared__ float red[W][G][LPT][EPV + 2];
  __shared__ uint32_t ids[kMaxTopK];
  __shared__ int id_cnt[kMaxTopK / 64];

  // (request, layer in [l0, l0 + nl), kv head) of this workgroup
  const int h = blockIdx.x % g.Hkv;
  const int rl = (blockIdx.x / (nl * g.Hkv)) * g.L + l0 + (blockIdx.x / g.Hkv) % nl;
  const int row = rl * g.Hkv + h;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int dg = lane % LPT;

  float qv[G][EPV];
#pragma unroll
  for (int gq = 0; gq < G; ++gq) {
    const float* qp = q + ((size_t)rl * g.Hq + (size_t)h * G + gq) * D + dg * EPV;
#pragma unroll
    for (int e = 0; e < EPV; ++e) qv[gq][e] = qp[e] * qscale;
  }
  Softmax sm[G];
  float acc[G][EPV];
#pragma unroll
  for (int gq = 0; gq < G; ++gq) {
    sm[gq].m = kNeg;
    sm[gq].l = 0.0f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[gq][e] = 0.0f;
  }

  // The row's slot ids are staged in LDS: a slot lookup is then an LDS read
  // (lgkmcnt) that never waits on the block loads in flight (vmcnt).  Empty
  // positions are dropped, so k is the number of blocks this row attends to.
  const int k = stage_row_ids<W>(slots + (size_t)row * g.k, g.k, ids, id_cnt);
  // Ring of NPF block buffers (NPF = 1: load, then consume).  While block j
  // (= wave + W*j of the row) is consumed, blocks j+1 .. j+NPF-1 are in flight;
  // the loop is unrolled by NPF so every buffer index is static, and every
  // iteration issues its loads so the compiler's load counters stay exact.
  // Past the end of the row those loads are never consumed: every lane then
  // reads the same 16 bytes of the last block, one line per instruction
  // (non-temporal loads would not find a re-read whole block in cache).
  const int nb = k > wave ? (k - wave + W - 1) / W : 0;
  // A slot outside the pool is read as slot 0 and reported once at the end
  // (no branch in the block loop).
  bool bad_slot = false;
  auto slot_at = [&](int j) -> uint64_t {
    const uint64_t slot =
        (uint32_t)__builtin_amdgcn_readfirstlane((int)ids[wave + W * min(j, nb - 1)]);
    const bool bad = slot >= g.pool_slots;
    bad_slot |= bad;
    return bad ? 0 : slot;
  };
  u32x4 kb[NPF][NLD], vb[NPF][NLD];
  float ksb[NPF], vsb[NPF];
  auto issue = [&](int j, int b) {
    const uint64_t slot = slot_at(j);
    const u32x4* kp = reinterpret_cast<const u32x4*>(pool + slot * g.bb);
    const u32x4* vp = kp + TILE_WORDS;
    const int live = j < nb ? 1 : 0;  // wave-uniform
#pragma unroll
    for (int ld = 0; ld < NLD; ++ld) kb[b][ld] = load_kv<NT>(kp + (ld * 64 + lane) * live);
#pragma unroll
    for (int ld = 0; ld < NLD; ++ld) vb[b][ld] = load_kv<NT>(vp + (ld * 64 + lane) * live);
    if constexpr (DT == FERRY_FP8_E4M3) {
      ksb[b] = pool_scales[2 * slot] * 256.0f;
      vsb[b] = pool_scales[2 * slot + 1] * 256.0f;
    } else {
      ksb[b] = vsb[b] = 1.0f;
    }
  };
  if (nb > 0) {
#pragma unroll
    for (int b = 0; b < NPF - 1; ++b) issue(b, b);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int i0 = 0; i0 < nb; i0 += NPF) {
#pragma unroll
    for (int b = 0; b < NPF; ++b) {
      const int i = i0 + b;
      if (i >= nb) break;
      issue(i + NPF - 1, (b + NPF - 1) % NPF);
      // keep the prefetch here: the scheduler would sink it to its first use
      __builtin_amdgcn_sched_barrier(0);
      const u32x4* kr = kb[b];
      const u32x4* vr = vb[b];
      const float ks = ksb[b], vs = vsb[b];
      float kf[NLD][EPV];
#pragma unroll
      for (int ld = 0; ld < NLD; ++ld) decode<DT>(kr[ld], kf[ld]);
      float s[G][NLD];
#pragma unroll
      for (int gq = 0; gq < G; ++gq)
#pragma unroll
        for (int ld = 0; ld < NLD; ++ld) {
          float a = 0.0f;
#pragma unroll
          for (int e = 0; e < EPV; ++e) a = __builtin_fmaf(qv[gq][e], kf[ld][e], a);
          s[gq][ld] = group_sum<LPT>(a) * ks;
        }
      float vf[NLD][EPV];
#pragma unroll
      for (int ld = 0; ld < NLD; ++ld) decode<DT>(vr[ld], vf[ld]);
#pragma unroll
      for (int gq = 0; gq < G; ++gq) {
        float mb = s[gq][0];
#pragma unroll
        for (int ld = 1; ld < NLD; ++ld) mb = fmaxf(mb, s[gq][ld]);
        const float mn = fmaxf(sm[gq].m, mb);
        const float alpha = exp2_fast(sm[gq].m - mn);
        float p[NLD], psum = 0.0f;
#pragma unroll
        for (int ld = 0; ld < NLD; ++ld) {
          p[ld] = exp2_fast(s[gq][ld] - mn);
          psum += p[ld];
        }
        sm[gq].l = sm[gq].l * alpha + psum;
        sm[gq].m = mn;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          float a = acc[gq][e] * alpha;
#pragma unroll
          for (int ld = 0; ld < NLD; ++ld) a = __builtin_fmaf(p[ld] * vs, vf[ld][e], a);
          acc[gq][e] = a;
        }
      }
    }
  }

  if (bad_slot && lane == 0) set_error(err, FERRY_ERANGE);
  // merge the TPL rows of the wavefront (lanes with the same dim chunk)
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
#pragma unroll
    for (int gq = 0; gq < G; ++gq) {
      const float om = __shfl_xor(sm[gq].m, off);
      const float ol = __shfl_xor(sm[gq].l, off);
      const float mn = fmaxf(sm[gq].m, om);
      const float a1 = exp2_fast(sm[gq].m - mn), a2 = exp2_fast(om - mn);
      sm[gq].l = sm[gq].l * a1 + ol * a2;
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float oa = __shfl_xor(acc[gq][e], off);
        acc[gq][e] = acc[gq][e] * a1 + oa * a2;
      }
      sm[gq].m = mn;
    }
  }
  if (lane < LPT) {
#pragma unroll
    for (int gq = 0; gq < G; ++gq) {
      red[wave][gq][lane][0] = sm[gq].m;
      red[wave][gq][lane][1] = sm[gq].l;
#pragma unroll
      for (int e = 0; e < EPV; ++e) red[wave][gq][lane][2 + e] = acc[gq][e];
    }
  }
  __syncthreads();
  // merge the W wavefronts and write out
  for (int t = threadIdx.x; t < G * LPT; t += blockDim.x) {
    const int gq = t / LPT, c = t % LPT;
    float m = red[0][gq][c][0];
    for (int w = 1; w < W; ++w) m = fmaxf(m, red[w][gq][c][0]);
    float l = 0.0f, o[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) o[e] = 0.0f;
    for (int w = 0; w < W; ++w) {
      const float a = exp2_fast(red[w][gq][c][0] - m);
      l += red[w][gq][c][1] * a;
#pragma unroll
      for (int e = 0; e < EPV; ++e) o[e] += red[w][gq][c][2 + e] * a;
    }
    // a row with no selected block (request not resident) attends to nothing: 0
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* op = out + ((size_t)rl * g.Hq + (size_t)h * G + gq) * D + c * EPV;
#pragma unroll
    for (int e = 0; e < EPV; ++e) op[e] = o[e] * inv;
  }
}

#define FERRY_ATTN_INST(DT, G, W)                                                          \
  template __global__ void k_attn<DT, G, W, false>(Geo, const float*, const uint32_t*,        \
                                                   const uint8_t*, const float*, float*, float, \
                                                   int, int, int*);                            \
  template __global__ void k_attn<DT, G, W, true>(Geo, const float*, const uint32_t*,         \
                                                  const uint8_t*, const float*, float*, float,  \
                                                  int, int, int*);
#define FERRY_ATTN_INST_G(DT, W) \
  FERRY_ATTN_INST(DT, 1, W)      \
  FERRY_ATTN_INST(DT, 2, W)      \
  FERRY_ATTN_INST(DT, 4, W)      \
  FERRY_ATTN_INST(DT, 8, W)
#define FERRY_ATTN_INST_ALL(W)          \
  FERRY_ATTN_INST_G(FERRY_F32, W)       \
  FERRY_ATTN_INST_G(FERRY_F16, W)       \
  FERRY_ATTN_INST_G(FERRY_BF16, W)      \
  FERRY_ATTN_INST_G(FERRY_FP8_E4M3, W)
FERRY_ATTN_INST_ALL(4)
FERRY_ATTN_INST_ALL(8)

}  // namespace ferry_amd
