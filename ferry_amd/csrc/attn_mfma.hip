// attn_mfma.hip -- block-sparse decode attention for GQA head groups on MFMA.
//
// Same contract as k_attn (attn.hip): out[r,l,hq] = softmax(q K^T / sqrt(D)) V
// over every token of the k blocks selected for (r, l, kv head of hq).  The
// reference has only an FMA proxy (src/workloads/kv_exec.cuh:30-37); the
// semantics are the textbook softmax attention of the top-k pages selected in
// tools/capture_miss_trace.py:139-159.
//
// When G = Hq/Hkv query heads share one kv head, QK^T and PV are real
// contractions over a [G x 128] query tile, so they run on the matrix cores:
//   S^T[16 tok][16 hd] = K[16 tok][128] . Q^T[128][16 hd]   (4x mfma 16x16x32)
//   O^T[128][16 hd]   += V^T[128][16 tok] . P^T[16 tok][16 hd] (8x mfma 16x16x16)
// with the G heads padded to the 16 columns of the tile.  One workgroup per
// (request, layer, kv head); its W wavefronts take every W-th block.
//
// Operand layouts (lane l, n = l % 16, grp = l / 16):
//  * A of 16x16xK: lane holds A[m = n][k in grp's K/4 slice]; B likewise with
//    n the column; C[m][n] sits at lane n + 16*(m/4), element m%4.
//  * The dot products are sums, so dims may be permuted freely as long as the
//    K operand and the Q operand agree: lane l takes token n of the K tile and
//    the dims of its own 16-byte words, each load instruction reading 64
//    contiguous bytes of every token row.
//  * S^T leaves lane l with scores of tokens 4*grp+i for head n: exactly the
//    B operand P^T of the PV product, so the softmax runs in place.
//  * V^T needs 4 tokens of one dim per lane; the output dims are permuted
//    (MFMA nb, row m) -> dim 8*m + nb, so lane l loads V[4*grp+i][8n..8n+7]
//    (four 16-byte words covering whole rows) and builds each A operand with
//    two byte permutes.  The O^T accumulator of lane l then holds dims
//    32*grp + 8*i + nb of head n.
// Precision: fp16 and fp8 K use one fp16 copy of q (scores within ~1e-4);
// bf16 K splits q into bf16 hi + lo parts (two MFMAs) and so does P for bf16
// V, keeping ~16 mantissa bits.  fp8 E4M3 is widened to fp16 exactly
// (v_cvt_scalef32_pk_f16_fp8 with scale 1); the per-block K scale multiplies
// the scores and the accumulator is kept in units of the current block's V
// scale (rescaled by vs_prev / vs at each block, times vs_last at the end).
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

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

__device__ inline uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace

template <int DT, int G, int W, bool NT>
__global__ __launch_bounds__(W * 64) void k_attn_mfma(Geo g, const float* __restrict__ q,
                                                   const uint32_t* __restrict__ slots,
                                                   const uint8_t* __restrict__ pool,
                                                   const float* __restrict__ pool_scales,
                                                   float* __restrict__ out, float qscale, int l0,
                                                   int nl, int* __restrict__ err) {
  static_assert(G >= 2 && G <= 16, "MFMA tile holds up to 16 query heads");
  static_assert(DT == FERRY_F16 || DT == FERRY_BF16 || DT == FERRY_FP8_E4M3, "16/8-bit KV");
  constexpr bool F8 = DT == FERRY_FP8_E4M3, BF = DT == FERRY_BF16;
  constexpr int D = 128, T = 16;
  constexpr int ES = F8 ? 1 : 2;
  constexpr uint32_t ROW = D * ES;     // bytes of one token row
  constexpr uint32_t KTILE = T * ROW;  // bytes of the K tile
  constexpr int NKW = F8 ? 2 : 4;      // 16-byte K words per lane per block
  constexpr int EPW = 16 / ES;         // elements per K word
  constexpr int SUB = EPW / 8;         // 8-element MFMA k-slices per K word
  constexpr float kNeg = -1.0e30f;
  constexpr int NPF = 3;  // prefetch ring depth

  __shared__ float red_o[W][G][D];
  __shared__ float red_ml[W][G][2];
  __shared__ uint32_t ids[kMaxTopK];
  __shared__ int id_cnt[kMaxTopK / 64];

  const int h = blockIdx.x % g.Hkv;
  const int rl = (blockIdx.x / (nl * g.Hkv)) * g.L + l0 + (blockIdx.x / g.Hkv) % nl;
  const int row = rl * g.Hkv + h;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, grp = lane >> 4;

  // ---- Q^T operand: dims of k-slice kk for this lane's group, head n (0 for pad heads)
  uint32_t qhi[4][4], qlo[4][4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int d0 = EPW * (4 * (kk / SUB) + grp) + 8 * (kk % SUB);
    float x[8];
    if (n < G) {
      const float4* qp =
          reinterpret_cast<const float4*>(q + ((size_t)rl * g.Hq + (size_t)h * G + n) * D + d0);
      const float4 a = qp[0], b = qp[1];
      x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z,
      x[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float a = x[e] * qscale, b = x[e + 1] * qscale;
      if constexpr (BF) {
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

  float m = kNeg, lsum = 0.0f, vs_cur = 1.0f;
  f32x4 acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) acc[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // The row's slot ids are staged in LDS: a slot lookup is then an LDS read
  // (lgkmcnt) that never waits on the block loads in flight (vmcnt).  Empty
  // positions are dropped, so k is the number of blocks this row attends to.
  const int k = stage_row_ids<W>(slots + (size_t)row * g.k, g.k, ids, id_cnt);
  const int nblk = k > wave ? (k - wave + W - 1) / W : 0;
  // A slot outside the pool is read as slot 0 and reported once at the end
  // (no branch in the block loop).
  bool bad_slot = false;
  auto slot_at = [&](int j) -> uint64_t {
    const uint64_t slot =
        (uint32_t)__builtin_amdgcn_readfirstlane((int)ids[wave + W * min(j, nblk - 1)]);
    const bool bad = slot >= g.pool_slots;
    bad_slot |= bad;
    return bad ? 0 : slot;
  };
  // K words: token n, byte offset 16*(4*w + grp) of its row.  V words: tokens
  // 4*grp+i, bytes [8n, 8n+8) elements of the row (16 B for 16-bit, 8 B fp8).
  constexpr int VW = F8 ? 2 : 4;  // dwords of V per token per lane
  // live = 0 (past the end of the row; the loads are never consumed): every
  // lane reads the block's first 16 bytes, one line per instruction.
  auto load_block = [&](uint64_t slot, int live, u32x4* kw, uint32_t (*vw)[VW]) {
    const uint8_t* base = pool + slot * g.bb;
#pragma unroll
    for (int w = 0; w < NKW; ++w)
      kw[w] = load_kv<NT>(
          reinterpret_cast<const u32x4*>(base + (n * ROW + 16 * (4 * w + grp)) * live));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* vp = base + (KTILE + (4 * grp + i) * ROW + 8 * ES * n) * live;
      if constexpr (F8) {
        const u32x2 v = load_kv<NT>(reinterpret_cast<const u32x2*>(vp));
        vw[i][0] = v[0], vw[i][1] = v[1];
      } else {
        const u32x4 v = load_kv<NT>(reinterpret_cast<const u32x4*>(vp));
        vw[i][0] = v[0], vw[i][1] = v[1], vw[i][2] = v[2], vw[i][3] = v[3];
      }
    }
  };

  // Ring of NPF block buffers: while block j (= wave + W*j of the row) is
  // consumed, blocks j+1 .. j+NPF-1 are in flight.  The loop is unrolled by NPF
  // so every buffer index is static, and every iteration issues its loads (past
  // the end, one line of the last block) so the compiler's load counters stay
  // exact.
  u32x4 kb[NPF][NKW];
  uint32_t vb[NPF][4][VW];
  float ksb[NPF], vsb[NPF];
  auto issue = [&](int j, int b) {
    const uint64_t slot = slot_at(j);
    load_block(slot, j < nblk ? 1 : 0, kb[b], vb[b]);
    if constexpr (F8) {
      ksb[b] = pool_scales[2 * slot];
      vsb[b] = pool_scales[2 * slot + 1];
    } else {
      ksb[b] = vsb[b] = 1.0f;
    }
  };
  if (nblk > 0) {
#pragma unroll
    for (int b = 0; b < NPF - 1; ++b) issue(b, b);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int i0 = 0; i0 < nblk; i0 += NPF) {
#pragma unroll
    for (int b = 0; b < NPF; ++b) {
      const int i = i0 + b;
      if (i < nblk) {
        issue(i + NPF - 1, (b + NPF - 1) % NPF);
      // keep the prefetch here: the scheduler would sink it to its first use
      __builtin_amdgcn_sched_barrier(0);
        const u32x4* kw = kb[b];
        const uint32_t(*vw)[VW] = vb[b];
        const float ks = ksb[b], vs = vsb[b];
        // ---- scores S^T = K . Q^T
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int w = kk / SUB, sub = kk % SUB;
          u32x4 a;
          if constexpr (F8) {
            const u32x2 lo = e4m3x4_to_f16(kw[w][2 * sub]);
            const u32x2 hi = e4m3x4_to_f16(kw[w][2 * sub + 1]);
            a = u32x4{lo[0], lo[1], hi[0], hi[1]};
          } else {
            a = kw[w];
          }
          const u32x4 bh = {qhi[kk][0], qhi[kk][1], qhi[kk][2], qhi[kk][3]};
          if constexpr (BF) {
            const u32x4 bl = {qlo[kk][0], qlo[kk][1], qlo[kk][2], qlo[kk][3]};
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                        __builtin_bit_cast(bf16x8, bh), s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                        __builtin_bit_cast(bf16x8, bl), s, 0, 0, 0);
          } else {
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                       __builtin_bit_cast(f16x8, bh), s, 0, 0, 0);
          }
        }
        // ---- online softmax of head n over tokens 4*grp+i (max shared by the 4 groups)
        float sv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) sv[t] = s[t] * ks;
        float bm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = fmaxf(m, bm);
        const float alpha = exp2_fast(m - mn);
        m = mn;
        float p[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) p[t] = exp2_fast(sv[t] - mn);
        lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        float fac = alpha;
        if constexpr (F8) {
          fac = alpha * (vs_cur * __builtin_amdgcn_rcpf(vs));
          vs_cur = vs;
        }
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[nb] *= fac;
        // ---- P^T operand
        u32x2 ph, pl;
        if constexpr (BF) {
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
        // ---- V^T operands (dim 8n + nb, tokens 4*grp + 0..3) and O^T += V^T . P^T
        uint32_t vh[4][4];  // per token: 8 halves of dims 8n..8n+7
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if constexpr (F8) {
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
          const u32x2 a = {perm(vh[1][w], vh[0][w], sel), perm(vh[3][w], vh[2][w], sel)};
          if constexpr (BF) {
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                __builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, ph), acc[nb], 0, 0, 0);
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
                __builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, pl), acc[nb], 0, 0, 0);
          } else {
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                __builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, ph), acc[nb], 0, 0, 0);
          }
        }
      }
    }
  }

  if (bad_slot && lane == 0) set_error(err, FERRY_ERANGE);
  // ---- per-wave totals: l over the 4 lane groups; O^T rows to LDS
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  if (n < G) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int t = 0; t < 4; ++t) red_o[wave][n][32 * grp + 8 * t + nb] = acc[nb][t] * vs_cur;
    if (grp == 0) {
      red_ml[wave][n][0] = m;
      red_ml[wave][n][1] = lsum;
    }
  }
  __syncthreads();
  // ---- merge the W wavefronts and write out
  for (int t = threadIdx.x; t < G * D; t += blockDim.x) {
    const int hq = t / D, d = t % D;
    float mx = red_ml[0][hq][0];
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, red_ml[w][hq][0]);
    float l = 0.0f, o = 0.0f;
    for (int w = 0; w < W; ++w) {
      const float a = exp2_fast(red_ml[w][hq][0] - mx);
      l += red_ml[w][hq][1] * a;
      o += red_o[w][hq][d] * a;
    }
    // a row with no selected block (request not resident) attends to nothing: 0
    out[((size_t)rl * g.Hq + (size_t)h * G + hq) * D + d] = l > 0.0f ? o / l : 0.0f;
  }
}

#define FERRY_ATTN_MFMA_INST(DT, G, W)                                                     \
  template __global__ void k_attn_mfma<DT, G, W, false>(Geo, const float*, const uint32_t*,   \
                                                        const uint8_t*, const float*, float*,  \
                                                        float, int, int, int*);                \
  template __global__ void k_attn_mfma<DT, G, W, true>(Geo, const float*, const uint32_t*,    \
                                                       const uint8_t*, const float*, float*,   \
                                                       float, int, int, int*);
#define FERRY_ATTN_MFMA_INST_G(DT, W) \
  FERRY_ATTN_MFMA_INST(DT, 2, W)      \
  FERRY_ATTN_MFMA_INST(DT, 4, W)      \
  FERRY_ATTN_MFMA_INST(DT, 8, W)
#define FERRY_ATTN_MFMA_INST_ALL(W)        \
  FERRY_ATTN_MFMA_INST_G(FERRY_F16, W)     \
  FERRY_ATTN_MFMA_INST_G(FERRY_BF16, W)    \
  FERRY_ATTN_MFMA_INST_G(FERRY_FP8_E4M3, W)
FERRY_ATTN_MFMA_INST_ALL(4)
FERRY_ATTN_MFMA_INST_ALL(8)

}  // namespace ferry_amd
