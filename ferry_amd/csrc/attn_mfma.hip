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
// Operand layouts, precision and the per-block arithmetic are in attn_mfma.hpp
// (shared with the prefix-group kernel of attn_group.hip).
#include "attn_mfma.hpp"
#include "kernels.hpp"

namespace ferry_amd {

using namespace mx;

template <int DT, int G, int W, bool NT>
__global__ __launch_bounds__(W * 64) void k_attn_mfma(Geo g, const float* __restrict__ q,
                                                   const uint32_t* __restrict__ slots,
                                                   const uint8_t* __restrict__ pool,
                                                   const float* __restrict__ pool_scales,
                                                   float* __restrict__ out, float qscale, int l0,
                                                   int nl, int* __restrict__ err) {
  static_assert(G >= 1 && G <= 16, "MFMA tile holds up to 16 query heads");
  static_assert(DT == FERRY_F16 || DT == FERRY_BF16 || DT == FERRY_FP8_E4M3, "16/8-bit KV");
  using S = Shape<DT>;
  constexpr bool F8 = S::F8;
  constexpr int D = S::D, ES = S::ES, NKW = S::NKW, VW = S::VW;
  constexpr uint32_t ROW = S::ROW, KTILE = S::KTILE;
  constexpr int NPF = 3;  // prefetch ring depth

  __shared__ float red_o[W][G][D + 4];  // +4: the 16 columns' rows start on different banks
  __shared__ float red_ml[W][G][2];
  __shared__ uint32_t ids[kMaxTopK];
  __shared__ int id_cnt[kMaxTopK / 64];

  const int h = blockIdx.x % g.Hkv;
  const int rl = (blockIdx.x / (nl * g.Hkv)) * g.L + l0 + (blockIdx.x / g.Hkv) % nl;
  const int row = rl * g.Hkv + h;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, grp = lane >> 4;

  // ---- Q^T operand of head n (0 for the padding columns n >= G)
  uint32_t qhi[4][4], qlo[4][4];
  q_operand<DT>(n < G ? q + ((size_t)rl * g.Hq + (size_t)h * G + n) * D : nullptr, grp, qscale,
                qhi, qlo);
  Acc acc;
  acc.init();

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
      const float2 sc = load_scales(pool_scales + 2 * slot);
      ksb[b] = sc.x;
      vsb[b] = sc.y;
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
        consume_block<DT, false>(kb[b], vb[b], ksb[b], vsb[b], qhi, qlo, acc, true);
      }
    }
  }

  if (bad_slot && lane == 0) set_error(err, FERRY_ERANGE);
  // ---- per-wave totals: l over the 4 lane groups; O^T rows to LDS
  float lsum = acc.lsum;
  lsum += __shfl_xor(lsum, 16);
  lsum += __shfl_xor(lsum, 32);
  const float vs_ref = F8 ? acc.vs_ref : 1.0f;
  if (n < G) {
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
#pragma unroll
      for (int t = 0; t < 4; ++t) red_o[wave][n][32 * grp + 8 * t + nb] = acc.o[nb][t] * vs_ref;
    if (grp == 0) {
      red_ml[wave][n][0] = acc.m;
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
// fp8 MHA (G = 1) too: widening fp8 and the dot products on the vector ALUs
// cost about twice as many instructions per byte as 16-bit KV, so one live
// column of the 16-column tile beats the VALU kernel there.
#define FERRY_ATTN_MFMA_INST_ALL(W)           \
  FERRY_ATTN_MFMA_INST_G(FERRY_F16, W)        \
  FERRY_ATTN_MFMA_INST_G(FERRY_BF16, W)       \
  FERRY_ATTN_MFMA_INST_G(FERRY_FP8_E4M3, W)   \
  FERRY_ATTN_MFMA_INST(FERRY_FP8_E4M3, 1, W)
FERRY_ATTN_MFMA_INST_ALL(4)
FERRY_ATTN_MFMA_INST_ALL(8)

}  // namespace ferry_amd
