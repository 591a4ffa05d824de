// attn_mfma.hpp -- the matrix-core arithmetic of one 16-token block, shared by
// the per-row GQA attention kernel (attn_mfma.hip) and the prefix-group kernel
// (attn_group.hip), so both compute every score, weight and output the same way.
//
// One wavefront holds a 16-column query tile (columns = query heads, padded)
// and, per block:
//   S^T[16 tok][16 col] = K[16 tok][128] . Q^T[128][16 col]     (4x mfma 16x16x32)
//   O^T[128][16 col]   += V^T[128][16 tok] . P^T[16 tok][16 col] (8x mfma 16x16x16)
// Lane l: n = l % 16 is its column, grp = l / 16 its quarter of the K slice.
//  * K operand: lane l holds token n, the dims of its own 16-byte words (NKW
//    words per block, word w covering bytes 16*(4w + grp) of the row), and the
//    Q^T operand holds the same dims of column n.
//  * S^T leaves lane l with the scores of tokens 4*grp + i for column n: the
//    B operand P^T of the PV product, so the softmax runs in place.
//  * V^T operand: lane l holds V[4*grp + i][8n .. 8n + 7] (VW dwords per token);
//    output dims are permuted (MFMA nb, row m) -> dim 8*m + nb, so the O^T
//    accumulator of lane l holds dims 32*grp + 8*i + nb of column n.
// Precision: fp16 and fp8 K use one fp16 copy of q (scores within ~1e-4);
// bf16 K splits q into bf16 hi + lo parts (two MFMAs) and so does P for bf16
// V, keeping ~16 mantissa bits.  fp8 E4M3 is widened to fp16 exactly; the
// per-block K scale multiplies the scores.  The accumulator is kept in units
// of a reference V scale (the first nonzero one): each block's weights are
// multiplied by vs / vs_ref before the fp16 rounding of P, and a block whose
// ratio leaves [1/64, 16] moves the reference to its own scale first.
// Lazy rescaling: the running max m of a column is raised only when a block's
// max exceeds it by more than kRescale (log2 units); otherwise the weights
// 2^(s - m) may grow up to 2^kRescale, which fp16 holds exactly as well (its
// relative precision does not depend on the exponent).  The accumulator and
// the sum are rescaled only on such a raise, in a branch the whole wavefront
// takes together, instead of at every block.
#pragma once

#include "attn_common.hpp"
#include "common.hpp"

namespace ferry_amd {
namespace mx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSelLo = 0x05040100u;  // perm: low halves of (lo_src, hi_src)
constexpr uint32_t kSelHi = 0x07060302u;  // perm: high halves
constexpr float kNeg = -1.0e30f;
constexpr float kRescale = 8.0f;  // log2 of the largest weight between raises of the max
constexpr float kVsHi = 16.0f;        // largest V-scale ratio folded into the fp16 weights
constexpr float kVsLo = 1.0f / 64.0f;  // smallest

__device__ inline uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }


// Shapes of one block's operands for KV dtype DT.
template <int DT>
struct Shape {
  static constexpr bool F8 = DT == FERRY_FP8_E4M3, BF = DT == FERRY_BF16;
  static constexpr int D = 128, T = 16;
  static constexpr int ES = F8 ? 1 : 2;       // bytes per element
  static constexpr uint32_t ROW = D * ES;     // bytes of one token row
  static constexpr uint32_t KTILE = T * ROW;  // bytes of the K tile
  static constexpr int NKW = F8 ? 2 : 4;      // 16-byte K words per lane per block
  static constexpr int EPW = 16 / ES;         // elements per K word
  static constexpr int SUB = EPW / 8;         // 8-element MFMA k-slices per K word
  static constexpr int VW = F8 ? 2 : 4;       // dwords of V per token per lane
};

// The 32 fp32 query values of column n that this lane's group holds in the
// Q^T operand (k-slice kk: x[kk][0..7]); `qp` points at the column's 128
// values, nullptr for a padding column (zeros).
template <int DT>
__device__ inline void q_load(const float* __restrict__ qp, int grp, float (&x)[4][8]) {
  using S = Shape<DT>;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int d0 = S::EPW * (4 * (kk / S::SUB) + grp) + 8 * (kk % S::SUB);
    if (qp) {
      const float4* p = reinterpret_cast<const float4*>(qp + d0);
      const float4 a = p[0], b = p[1];
      x[kk][0] = a.x, x[kk][1] = a.y, x[kk][2] = a.z, x[kk][3] = a.w;
      x[kk][4] = b.x, x[kk][5] = b.y, x[kk][6] = b.z, x[kk][7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[kk][e] = 0.0f;
    }
  }
}

// Q^T operand of column n for this lane's group from the values q_load read,
// pre-scaled by qscale (log2(e) / sqrt(D)).
template <int DT>
__device__ inline void q_convert(const float (&x)[4][8], float qscale, uint32_t (&qhi)[4][4],
                                 uint32_t (&qlo)[4][4]) {
  using S = Shape<DT>;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float a = x[kk][e] * qscale, b = x[kk][e + 1] * qscale;
      if constexpr (S::BF) {
        const uint16_t ah = bf16_rne(a), bh = bf16_rne(b);
        const float ar = a - __builtin_bit_cast(float, (uint32_t)ah << 16);
        const float br = b - __builtin_bit_cast(float, (uint32_t)bh << 16);
        qhi[kk][e / 2] = (uint32_t)ah | ((uint32_t)bh << 16);
        qlo[kk][e / 2] = (uint32_t)bf16_rne(ar) | ((uint32_t)bf16_rne(br) << 16);
      } else {
        const f16x2 hv = {(_Float16)a, (_Float16)b};
        qhi[kk][e / 2] = __builtin_bit_cast(uint32_t, hv);
        qlo[kk][e / 2] = 0;
      }
    }
  }
}

// Q^T operand of column n for this lane's group: `qp` points at the column's
// 128 fp32 values (nullptr for a padding column: zeros), pre-scaled by qscale.
template <int DT>
__device__ inline void q_operand(const float* __restrict__ qp, int grp, float qscale,
                                 uint32_t (&qhi)[4][4], uint32_t (&qlo)[4][4]) {
  float x[4][8];
  q_load<DT>(qp, grp, x);
  q_convert<DT>(x, qscale, qhi, qlo);
}

// Running state of one wavefront's columns: online-softmax max and sum (lane
// partial over its 4 tokens of each block), the reference V scale the
// accumulator is kept in (0 until the first nonzero one), and O^T.  The column's
// output is o * vs_ref / (sum over the 4 lanes of lsum).
struct Acc {
  float m, lsum, vs_ref;
  f32x4 o[8];
  __device__ inline void init() {
    m = kNeg, lsum = 0.0f, vs_ref = 0.0f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
};

// The MFMA A operands of one block: K of the four 32-dim k-slices (16-bit
// elements) and V^T of the eight dim tiles (tokens 4*grp .. 4*grp+3).  Built
// once per block and shared by every query tile that attends to it.
struct Ops {
  u32x4 k[4];
  u32x2 v[8];
};

// K words kw and V dwords vw as loaded -> operands (fp8 widened to fp16
// exactly; V rows regrouped to dims 8n + nb).
template <int DT>
__device__ __forceinline__ void block_operands(const u32x4 (&kw)[Shape<DT>::NKW],
                                               const uint32_t (&vw)[4][Shape<DT>::VW],
                                               Ops& op) {
  using S = Shape<DT>;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int w = kk / S::SUB, sub = kk % S::SUB;
    if constexpr (S::F8) {
      const u32x2 lo = e4m3x4_to_f16(kw[w][2 * sub]);
      const u32x2 hi = e4m3x4_to_f16(kw[w][2 * sub + 1]);
      op.k[kk] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    } else {
      op.k[kk] = kw[w];
    }
  }
  uint32_t vh[4][4];  // per token: 8 halves of dims 8n..8n+7
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if constexpr (S::F8) {
      const u32x2 lo = e4m3x4_to_f16(vw[t][0]), hi = e4m3x4_to_f16(vw[t][1]);
      vh[t][0] = lo[0], vh[t][1] = lo[1], vh[t][2] = hi[0], vh[t][3] = hi[1];
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) vh[t][w] = vw[t][w];
    }
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    const int w = nb >> 1;
    const uint32_t sel = (nb & 1) ? kSelHi : kSelLo;
    op.v[nb] = u32x2{perm(vh[1][w], vh[0][w], sel), perm(vh[3][w], vh[2][w], sel)};
  }
}

// One query tile attends to one block: scores, online softmax, O^T += V^T P^T.
// ks / vs are the block scales (1 unless fp8).  MASK: `live` says whether this
// lane's column attends to the block; a dead column keeps its max, sum, V
// scale and accumulator exactly (its weights are 0).  `live` must be the same
// on the four lanes of a column.
template <int DT, bool MASK>
__device__ __forceinline__ void tile_block(const Ops& op, float ks, float vs,
                                           const uint32_t (&qhi)[4][4],
                                           const uint32_t (&qlo)[4][4], Acc& a, bool live) {
  using S = Shape<DT>;
  // ---- scores S^T = K . Q^T
  f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const u32x4 bh = {qhi[kk][0], qhi[kk][1], qhi[kk][2], qhi[kk][3]};
    if constexpr (S::BF) {
      const u32x4 bl = {qlo[kk][0], qlo[kk][1], qlo[kk][2], qlo[kk][3]};
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, op.k[kk]),
                                                  __builtin_bit_cast(bf16x8, bh), s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, op.k[kk]),
                                                  __builtin_bit_cast(bf16x8, bl), s, 0, 0, 0);
    } else {
      s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, op.k[kk]),
                                                 __builtin_bit_cast(f16x8, bh), s, 0, 0, 0);
    }
  }
  // ---- online softmax of column n over tokens 4*grp+i (max shared by the 4 groups)
  float sv[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) sv[t] = s[t] * ks;
  float bm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  bm = max_over_groups(bm);
  const bool raise = (!MASK || live) && bm > a.m + kRescale;
  if (__builtin_amdgcn_ballot_w64(raise)) {  // uniform: some column's max moved up
    const float alpha = raise ? exp2_fast(a.m - bm) : 1.0f;
    a.m = raise ? bm : a.m;
    a.lsum *= alpha;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) a.o[nb] *= alpha;
  }
  float p[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) p[t] = (!MASK || live) ? exp2_fast(sv[t] - a.m) : 0.0f;
  a.lsum += (p[0] + p[1]) + (p[2] + p[3]);
  if constexpr (S::F8) {  // weights in units of the reference V scale
    // r = vs / vs_ref is held in [kVsLo, kVsHi]: p * r <= 2^kRescale * kVsHi
    // stays far below fp16's 65504, and weights near the max stay normal.  A
    // block outside the band first moves the reference to its own scale (the
    // accumulator rescaled in fp32), in a branch the wavefront takes together:
    // vs and vs_ref are the same on every lane.  A zero V scale (an all-zero
    // block) adds nothing and sets no reference; while there is none, r is
    // inf and the first nonzero scale becomes the reference (o is still 0).
    float r = 0.0f;
    if (vs != 0.0f) {
      r = vs * __builtin_amdgcn_rcpf(a.vs_ref);
      const bool rebase = !(r >= kVsLo && r <= kVsHi);
      if (__builtin_amdgcn_ballot_w64(rebase)) {
        const float f = a.vs_ref * __builtin_amdgcn_rcpf(vs);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) a.o[nb] *= f;
        a.vs_ref = vs;
        r = 1.0f;
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] *= r;
  }
  // ---- P^T operand
  u32x2 ph, pl;
  if constexpr (S::BF) {
    uint32_t hb[4];
    float r[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      hb[t] = __builtin_bit_cast(uint32_t, p[t]) & 0xFFFF0000u;
      r[t] = p[t] - __builtin_bit_cast(float, hb[t]);
    }
    ph = u32x2{perm(hb[1], hb[0], kSelHi), perm(hb[3], hb[2], kSelHi)};
    const uint32_t r0 = __builtin_bit_cast(uint32_t, r[0]), r1 = __builtin_bit_cast(uint32_t, r[1]);
    const uint32_t r2 = __builtin_bit_cast(uint32_t, r[2]), r3 = __builtin_bit_cast(uint32_t, r[3]);
    pl = u32x2{perm(r1, r0, kSelHi), perm(r3, r2, kSelHi)};
  } else {
    const f16x4 pv = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
    ph = __builtin_bit_cast(u32x2, pv);
    pl = u32x2{0u, 0u};
  }
  // ---- O^T += V^T . P^T
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    if constexpr (S::BF) {
      a.o[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          __builtin_bit_cast(i16x4, op.v[nb]), __builtin_bit_cast(i16x4, ph), a.o[nb], 0, 0, 0);
      a.o[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
          __builtin_bit_cast(i16x4, op.v[nb]), __builtin_bit_cast(i16x4, pl), a.o[nb], 0, 0, 0);
    } else {
      a.o[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(
          __builtin_bit_cast(f16x4, op.v[nb]), __builtin_bit_cast(f16x4, ph), a.o[nb], 0, 0, 0);
    }
  }
}

// One block for one tile: block_operands then tile_block.
template <int DT, bool MASK>
__device__ __forceinline__ void consume_block(const u32x4 (&kw)[Shape<DT>::NKW],
                                              const uint32_t (&vw)[4][Shape<DT>::VW], float ks,
                                              float vs, const uint32_t (&qhi)[4][4],
                                              const uint32_t (&qlo)[4][4], Acc& a, bool live) {
  Ops op;
  block_operands<DT>(kw, vw, op);
  tile_block<DT, MASK>(op, ks, vs, qhi, qlo, a, live);
}

}  // namespace mx
}  // namespace ferry_amd
