// select.hip -- on-device top-k block selection (Quest bound) feeding the
// miss queue.
//
// The reference selects pages on the host side of a model hook
// (tools/capture_miss_trace.py:139-159): per page and KV head, the
// elementwise min and max of K over the page's tokens; per query head, the
// bound sum_d max(q_d * kmax_d, q_d * kmin_d) (an upper bound of q.k over the
// page); max over the query heads of a KV head; top-k pages, returned in
// ascending page order.  Its per-layer variant takes the max over every head
// of the layer and shares one selection (FERRY_TOPK_LAYER_MAX).  A page is
// one 16-token block here, and a context shorter than k selects all of its
// blocks (min(k, n_pages), :157-158), padding the row with FERRY_EMPTY.
//
// Block summaries live in HBM: record i holds the min and max of a K tile per
// dim, in the KV element type (fp8: E4M3 codes, the block's K scale kept
// beside them and applied to the bound).  Block (set, b) uses record
// (set * max_blocks + b) mod S.  S is a multiple of the host tier's size, so
// blocks that share a record share their host-tier content: S = host_blocks
// is the smallest table, S >= sets * max_blocks gives every block its own
// record, as a serving system that summarises each written page has.
//
// Since kmax >= kmin, max(q kmax, q kmin) = q * (q >= 0 ? kmax : kmin): which
// of the two a dim uses is fixed by the sign of q for the whole row, so the
// bound costs one select and one fused multiply-add per (head, dim).
// Every fp32 operation has a fixed order so the selection is bit-exact
// against the CPU oracle: lane p of a block's 16 lanes accumulates dims
// 8p..8p+7 left to right with fma (acc = fma(q_d, k_d, acc), acc = 0 first);
// the 16 partial sums are combined by an xor butterfly (8, 4, 2, 1); max is
// `a > b ? a : b`; keys are the order-preserving map of the float bits (so
// -0 < +0), and equal keys go to the lower block id.
#include "attn_common.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

namespace {

template <int DT>
__device__ inline uint32_t elem_bits(const uint8_t* p, int i) {
  if constexpr (DT == FERRY_F32) return reinterpret_cast<const uint32_t*>(p)[i];
  else if constexpr (DT == FERRY_FP8_E4M3) return p[i];
  else return reinterpret_cast<const uint16_t*>(p)[i];
}

// Exact decode of one stored element.
template <int DT>
__device__ inline float elem_f32(uint32_t v) {
  if constexpr (DT == FERRY_F32) {
    return bits_f32(v);
  } else if constexpr (DT == FERRY_F16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)v);
  } else if constexpr (DT == FERRY_BF16) {
    return bits_f32(v << 16);
  } else {  // OCP E4M3FN: (-1)^s 2^(e-7) (1 + m/8), subnormal m 2^-9
    const uint32_t s = (v & 0x80u) << 24, e = (v >> 3) & 0xFu, m = v & 7u;
    if (e == 0) return bits_f32(f32_bits((float)m * 0.001953125f) | s);
    return bits_f32(s | ((e + 120u) << 23) | (m << 20));
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The 8 elements [i0, i0 + 8) of a summary record, widened exactly to fp32,
// with one vector load (16 B for 16-bit elements, 8 B fp8, 2 x 16 B fp32).
// Every record is read once per launch, so the loads are non-temporal
// (streamed past the caches: ~87% of HBM peak for such reads on MI355X
// against ~79% for cached ones).
template <int DT>
__device__ inline void load8(const uint8_t* rec, int i0, float* f) {
  if constexpr (DT == FERRY_F32) {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rec + 4 * i0));
    const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rec + 4 * i0 + 16));
    const uint32_t w[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = bits_f32(w[e]);
  } else if constexpr (DT == FERRY_FP8_E4M3) {
    const u32x2 a = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(rec + i0));
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = elem_f32<DT>(((e < 4 ? a[0] : a[1]) >> (8 * (e & 3))) & 0xFFu);
  } else {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rec + 2 * i0));
    const uint32_t w[4] = {a[0], a[1], a[2], a[3]};
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = elem_f32<DT>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
  }
}

__device__ inline float fmax_det(float a, float b) { return a > b ? a : b; }

// order-preserving map of float bits to unsigned keys
__device__ inline uint32_t fkey(float x) {
  const uint32_t u = f32_bits(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// sum over the 16 lanes of a row: xor 8, 4, 2, 1 (ds_swizzle bitmask mode)
__device__ inline float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (8 << 10) | 0x1F));
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (4 << 10) | 0x1F));
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (2 << 10) | 0x1F));
  v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (1 << 10) | 0x1F));
  return v;
}

template <int X>
__device__ inline float swz_xor(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), (X << 10) | 0x1F));
}

// One transposition level of the G-head reduction over a 16-lane row: a lane
// holding N head partials keeps the lower half (bit X of its row position
// clear) or the upper half, and adds the partner's partials of the same heads,
// own value first, as the plain butterfly's step X does.
template <int X, int N>
__device__ inline void transpose_level(float* v, int p) {
  const bool hi = (p & X) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = hi ? v[i] : v[i + N / 2];
    const float keep = hi ? v[i + N / 2] : v[i];
    v[i] = keep + swz_xor<X>(send);
  }
}

// The Quest bound of every query head (acc[h]: this lane's 8-dim partial of
// head h) summed over the 16 lanes of the row, and their maximum taken in head
// order, valid in the row's lane 0.  With one head this is the xor 8, 4, 2, 1
// butterfly.  With G heads the first log2(G) levels are transposed, so each
// sum is formed in one lane group instead of all 16 lanes (G = 4: 5 swizzles
// and 5 adds instead of 16 and 16); every sum is the same additions in the
// same order as the butterfly's, and the maximum is the same chain, so the
// result is bit-identical.  Head h ends in lane h * 16 / G of the row.
template <int G>
__device__ inline float heads_bound_max(float (&acc)[G], int p) {
  if constexpr (G == 1) {
    return row16_sum(acc[0]);
  } else {
    transpose_level<8, G>(acc, p);
    if constexpr (G >= 4) transpose_level<4, G / 2>(acc, p);
    if constexpr (G >= 8) transpose_level<2, G / 4>(acc, p);
    float v = acc[0];
    if constexpr (G < 4) v += swz_xor<4>(v);
    if constexpr (G < 8) v += swz_xor<2>(v);
    v += swz_xor<1>(v);
    float sk = v;
#pragma unroll
    for (int h = 1; h < G; ++h) {
      float other;
      switch (h * 16 / G) {  // compile-time after unrolling
        case 2: other = swz_xor<2>(v); break;
        case 4: other = swz_xor<4>(v); break;
        case 6: other = swz_xor<6>(v); break;
        case 8: other = swz_xor<8>(v); break;
        case 10: other = swz_xor<10>(v); break;
        case 12: other = swz_xor<12>(v); break;
        default: other = swz_xor<14>(v); break;
      }
      sk = fmax_det(other, sk);
    }
    return sk;
  }
}

}  // namespace

// One wavefront per host-tier block: min and max over the 16 tokens of every
// K dim (lane l: dims 2l, 2l+1), stored as the element that attains them;
// the first of equal values (token order) is kept.
template <int DT>
__global__ __launch_bounds__(256) void k_summaries_build(Geo g, const uint8_t* __restrict__ host,
                                                         const float* __restrict__ host_scales,
                                                         uint8_t* __restrict__ sums,
                                                         float* __restrict__ sum_scales) {
  constexpr int ES = DT == FERRY_F32 ? 4 : (DT == FERRY_FP8_E4M3 ? 1 : 2);
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const uint64_t waves = (uint64_t)gridDim.x * (blockDim.x >> 6);
  for (uint64_t h = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); h < g.host_blocks;
       h += waves) {
    const uint8_t* kt = host + h * g.bb;
    uint8_t* out = sums + h * (uint64_t)(2 * D * ES);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int d = 2 * lane + c;
      uint32_t bmin = elem_bits<DT>(kt, d), bmax = bmin;
      float fmin = elem_f32<DT>(bmin), fmax = fmin;
      for (int t = 1; t < 16; ++t) {
        const uint32_t b = elem_bits<DT>(kt, t * D + d);
        const float f = elem_f32<DT>(b);
        if (f < fmin) {
          fmin = f;
          bmin = b;
        }
        if (f > fmax) {
          fmax = f;
          bmax = b;
        }
      }
      if constexpr (ES == 4) {
        reinterpret_cast<uint32_t*>(out)[d] = bmin;
        reinterpret_cast<uint32_t*>(out)[D + d] = bmax;
      } else if constexpr (ES == 2) {
        reinterpret_cast<uint16_t*>(out)[d] = (uint16_t)bmin;
        reinterpret_cast<uint16_t*>(out)[D + d] = (uint16_t)bmax;
      } else {
        out[d] = (uint8_t)bmin;
        out[D + d] = (uint8_t)bmax;
      }
    }
    if (DT == FERRY_FP8_E4M3 && lane == 0) sum_scales[h] = host_scales[2 * h];
  }
}

// Records [host_blocks, S) repeat records [0, host_blocks): record i is the
// summary of host block i mod host_blocks (16-byte copies, scales too).
__global__ __launch_bounds__(256) void k_summaries_tile(uint8_t* __restrict__ sums, float* __restrict__ scales,
                                                        uint64_t host_blocks, uint64_t total, uint32_t rec) {
  const uint64_t words = (uint64_t)rec / 16;
  const uint64_t n = (total - host_blocks) * words;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint4* dst = reinterpret_cast<uint4*>(sums + host_blocks * rec);
  const uint4* src = reinterpret_cast<const uint4*>(sums);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t r = i / words, w = i % words;
    dst[i] = src[((host_blocks + r) % host_blocks) * words + w];
  }
  if (scales)
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total - host_blocks; i += stride)
      scales[host_blocks + i] = scales[(host_blocks + i) % host_blocks];
}

// The kk largest of keys[0, n) (n > kk), ids written in ascending order to
// `nrows` output rows `row_stride` apart, ties to the lower ids.  Phase 1 finds
// the kk-th largest key by up to 4 radix passes of 8 bits over LDS histograms (a
// wavefront-wide suffix scan over the bins).  Scores of one row mostly share
// their top byte, so each 64-key step counts its first key's bin with one
// atomic for every lane in it (ballot) and only the other lanes add their own:
// the same counts without 64 lanes serialised on one LDS word.  Phase 2 gives
// each wavefront a contiguous range, counts the keys above the k-th and its
// ties by ballots, and writes the taken ids in order at ballot ranks; every
// LDS read is a contiguous 64-key row (one key per lane, no bank conflicts).
// (Per-thread chunks of n / 256 keys read 64 words one chunk apart per
// instruction, all in one bank; the Quest launch at 128K-token contexts is
// 2.51-2.55 ms with these two steps against 2.53-2.56 ms.)  With HIST1 the
// caller has counted the top bytes into hist while writing the keys.  A pass
// whose bin holds exactly the keys still needed ends the search: every key
// with that prefix is taken, so phase 2 compares the masked keys.  hist: 256
// LDS words, wtot: 2 W, sh: 3.  Every thread must call it.
template <int W, bool HIST1 = false>
__device__ void topk_ascending(const uint32_t* keys, int n, int kk, uint32_t* hist, uint32_t* wtot,
                               uint32_t* sh, uint32_t* out, int nrows, size_t row_stride) {
  constexpr int NT = W * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t prefix = 0, mask = 0, need = (uint32_t)kk;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (!HIST1 || shift != 24) {
      for (int i = tid; i < 256; i += NT) hist[i] = 0;
      __syncthreads();
    }
    for (int i0 = 64 * wave; (!HIST1 || shift != 24) && i0 < n; i0 += NT) {
      const int i = i0 + lane;
      const uint32_t key = i < n ? keys[i] : 0u;
      const bool valid = i < n && (key & mask) == prefix;
      const uint32_t bin = (key >> shift) & 0xFFu;
      const uint64_t vb = ballot(valid);
      if (vb) {
        const int first = __builtin_ctzll(vb);
        const uint32_t b0 = (uint32_t)__builtin_amdgcn_readlane((int)bin, first);
        const uint64_t same = ballot(valid && bin == b0);
        if (lane == first) atomicAdd(&hist[b0], (uint32_t)__builtin_popcountll(same));
        if (valid && bin != b0) atomicAdd(&hist[bin], 1u);
      }
    }
    __syncthreads();
    if (wave == 0) {
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c[e] = hist[255 - 4 * lane - e];
        sum += c[e];
      }
      uint32_t incl = sum;
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
      }
      const uint32_t excl = incl - sum;
      if (excl < need && incl >= need) {
        uint32_t acc = excl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (acc + c[e] >= need && acc < need) {
            sh[0] = prefix | ((uint32_t)(255 - 4 * lane - e) << shift);
            sh[1] = need - acc;
            sh[2] = acc + c[e] == need;
          }
          acc += c[e];
        }
      }
    }
    __syncthreads();
    prefix = sh[0];
    need = sh[1];
    mask |= 0xFFu << shift;
    if (sh[2]) break;
  }
  const uint32_t T = prefix;
  const int span = ((n + NT - 1) / NT) * 64;
  const int w0 = min(n, wave * span), w1 = min(n, w0 + span);
  uint32_t gt = 0, eq = 0;
  for (int i0 = w0; i0 < w1; i0 += 64) {
    const int i = i0 + lane;
    const uint32_t key = i < w1 ? keys[i] & mask : 0u;
    gt += (uint32_t)__builtin_popcountll(ballot(i < w1 && key > T));
    eq += (uint32_t)__builtin_popcountll(ballot(i < w1 && key == T));
  }
  if (lane == 0) {
    wtot[wave] = gt;
    wtot[W + wave] = eq;
  }
  __syncthreads();
  uint32_t gt_before = 0, ties = 0;
  for (int w = 0; w < wave; ++w) {
    gt_before += wtot[w];
    ties += wtot[W + w];
  }
  uint32_t pos = gt_before + min(ties, need);
  for (int i0 = w0; i0 < w1; i0 += 64) {
    const int i = i0 + lane;
    const uint32_t key = i < w1 ? keys[i] & mask : 0u;
    const bool is_eq = i < w1 && key == T;
    const uint64_t eqm = ballot(is_eq);
    const bool take = (i < w1 && key > T) || (is_eq && ties + (uint32_t)lanes_below(eqm) < need);
    const uint64_t tm = ballot(take);
    if (take) {
      const uint32_t at = pos + (uint32_t)lanes_below(tm);
      for (int r = 0; r < nrows; ++r) out[r * row_stride + at] = (uint32_t)i;
    }
    pos += (uint32_t)__builtin_popcountll(tm);
    ties += (uint32_t)__builtin_popcountll(eqm);
  }
}

// One workgroup (W wavefronts) per (request, layer, kv head) row, or per
// (request, layer) with LAYER.  Phase 1 scores every block of the request's
// context into LDS keys (16 lanes per block, 4 blocks per wavefront pass),
// counting their top bytes as the first radix pass; phase 2 finds the k-th
// largest key by at most 4 radix passes of 8 bits; phase 3 writes the
// selected block ids in ascending order (ties to lower ids).
// Dynamic LDS: q[Gq][128] floats, then keys[max_n].
template <int DT, int G, bool LAYER, int W>
__global__ __launch_bounds__(W * 64) void k_select_topk(Geo g, const float* __restrict__ q,
                                                        const int32_t* __restrict__ ctx_blocks,
                                                        const uint8_t* __restrict__ sums,
                                                        const float* __restrict__ sum_scales,
                                                        uint64_t sum_mod, uint32_t* __restrict__ sel,
                                                        int l0, int nl, int max_n,
                                                        int* __restrict__ err) {
  constexpr int ES = DT == FERRY_F32 ? 4 : (DT == FERRY_FP8_E4M3 ? 1 : 2);
  constexpr int D = 128, NT = W * 64;
  constexpr uint32_t REC = 2 * D * ES;  // summary bytes per block
  extern __shared__ uint32_t lds[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wtot[2 * W];
  __shared__ uint32_t sh[3];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nkv = LAYER ? g.Hkv : 1;  // kv heads scored per row
  const int Gq = G * nkv;             // query heads per row
  float* qs = reinterpret_cast<float*>(lds);
  uint32_t* keys = lds + Gq * D;

  const int hrow = LAYER ? 0 : blockIdx.x % g.Hkv;
  const int rl_idx = LAYER ? blockIdx.x : blockIdx.x / g.Hkv;  // (request, layer in range)
  const int r = rl_idx / nl, l = l0 + rl_idx % nl;
  const int rl = r * g.L + l;
  int n = ctx_blocks[r];
  if (n < 0) n = 0;
  if (n > max_n || n > g.max_blocks) {
    if (tid == 0) set_error(err, FERRY_ERANGE);
    n = 0;
  }
  const int k = g.k;
  const int kk = n < k ? n : k;
  auto out_row = [&](int hh) { return sel + ((size_t)rl * g.Hkv + hh) * (size_t)k; };

  if (n > k) {
    // ---- phase 1: scores, and the top-k's first radix pass (the keys' top
    // bytes counted as they are written, while the loads stream)
    const int grp = lane >> 4, p = lane & 15;
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    // the row's query dims of this lane (8 per head), and whether each uses kmax
    float qr[G][8];
    if (!LAYER) {
#pragma unroll
      for (int gq = 0; gq < G; ++gq)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          qr[gq][e] = q[((size_t)rl * g.Hq + (size_t)(hrow * G + gq)) * D + 8 * p + e];
      __syncthreads();
    } else {
      for (int i = tid; i < Gq * D; i += NT) qs[i] = q[(size_t)rl * g.Hq * D + i];
      __syncthreads();
    }
    // U passes of 4 blocks per wavefront are loaded before any is scored: the
    // keys take most of the LDS at long contexts, so few workgroups share a
    // CU and each wavefront must keep several records in flight
    constexpr int U = G >= 8 ? 2 : 4;
    for (int b0 = 4 * wave; b0 < n; b0 += 4 * W * U) {
      float score[U];
      for (int hh = 0; hh < nkv; ++hh) {
        const int hk = LAYER ? hh : hrow;
        const uint64_t set = (uint64_t)rl * g.Hkv + hk;
        float kmn[U][8], kmx[U][8];
        uint64_t hbs[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = b0 + 4 * W * u + grp;
          hbs[u] = host_index(set, b < n ? (uint32_t)b : 0u, (uint64_t)g.max_blocks, sum_mod);
          const uint8_t* rec = sums + hbs[u] * REC;
          load8<DT>(rec, 8 * p, kmn[u]);
          load8<DT>(rec, D + 8 * p, kmx[u]);
        }
        if (LAYER) {
#pragma unroll
          for (int gq = 0; gq < G; ++gq)
#pragma unroll
            for (int e = 0; e < 8; ++e) qr[gq][e] = qs[(hh * G + gq) * D + 8 * p + e];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float acc[G];
#pragma unroll
          for (int gq = 0; gq < G; ++gq) {
            acc[gq] = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
              acc[gq] = __fmaf_rn(qr[gq][e], qr[gq][e] >= 0.0f ? kmx[u][e] : kmn[u][e], acc[gq]);
          }
          float sk = heads_bound_max<G>(acc, p);
          if constexpr (DT == FERRY_FP8_E4M3) sk = __fmul_rn(sk, sum_scales[hbs[u]]);
          score[u] = hh == 0 ? sk : fmax_det(sk, score[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int b = b0 + 4 * W * u + grp;
        if (b < n && p == 0) {
          const uint32_t key = fkey(score[u]);
          keys[b] = key;
          atomicAdd(&hist[key >> 24], 1u);
        }
      }
    }
    __syncthreads();
    topk_ascending<W, true>(keys, n, kk, hist, wtot, sh, out_row(LAYER ? 0 : hrow),
                            LAYER ? g.Hkv : 1, (size_t)k);
  } else {
    // a context of at most k blocks: every block, in order
    for (int j = tid; j < kk; j += NT)
      for (int hh = 0; hh < (LAYER ? g.Hkv : 1); ++hh) out_row(LAYER ? hh : hrow)[j] = (uint32_t)j;
  }
  for (int j = kk + tid; j < k; j += NT)
    for (int hh = 0; hh < (LAYER ? g.Hkv : 1); ++hh) out_row(LAYER ? hh : hrow)[j] = kNone;
}

// ---------------------------------------------------------------- mass method
// The capture tool's second selection method (tools/capture_miss_trace.py:
// 147-155): a block's score is the softmax mass its tokens take, summed over
// every query head of the layer, and each layer gets one page list.  It needs
// every context token's key, so it reads a dense K table (the K half of each
// host-tier block, records addressed like the summaries) instead of the
// summaries.

// One wavefront per host-tier block: its K half (NV KiB) copied device-direct
// from the pinned tier into record h, and its K scale (fp8).  perm = 1 (16-bit
// and fp8 K) stores the record lane-transposed for the matrix-core kernel:
// 16-byte word c of token row t goes to word 64 (c / 4) + 16 (c % 4) + t, so
// each of that kernel's load instructions reads 1 KiB contiguous (lane l =
// 16 grp + n takes word 4 w + grp of row n).  perm = 0 keeps the row-major
// order (fp32 K, read by the vector-ALU kernel).
template <int NV>
__global__ __launch_bounds__(256) void k_ktiles_build(Geo g, const uint8_t* __restrict__ host,
                                                      const float* __restrict__ host_scales,
                                                      uint8_t* __restrict__ kt,
                                                      float* __restrict__ kt_scales, int perm) {
  const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const uint64_t nw = ((uint64_t)gridDim.x * blockDim.x) >> 6;
  const int lane = threadIdx.x & 63;
  constexpr int WPR = NV * 4;  // 16-byte words per token row (16 rows)
  for (uint64_t h = wave; h < (uint64_t)g.host_blocks; h += nw) {
    const u32x4* src = reinterpret_cast<const u32x4*>(host + h * g.bb);
    u32x4* dst = reinterpret_cast<u32x4*>(kt + h * (uint64_t)NV * 1024);
    u32x4 r[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) r[v] = __builtin_nontemporal_load(src + v * kWave + lane);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int c = (v * kWave + lane) % WPR, row = (v * kWave + lane) / WPR;
      dst[perm ? (c / 4) * 64 + (c % 4) * 16 + row : v * kWave + lane] = r[v];
    }
    if (kt_scales && lane == 0) kt_scales[h] = host_scales[2 * h];
  }
}

namespace {

// The 16/ES elements of one 16-byte word of a K row, decoded exactly.
template <int DT, int EPL>
__device__ inline void decode_word(const u32x4& w, float* f) {
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    if constexpr (DT == FERRY_F32) f[e] = bits_f32(w[e]);
    else if constexpr (DT == FERRY_FP8_E4M3) f[e] = elem_f32<DT>((w[e >> 2] >> (8 * (e & 3))) & 0xFFu);
    else f[e] = elem_f32<DT>((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
  }
}

// Sum of a lane's N partial dot products over the lanes of a token row (xor
// X, X/2, ..., 1): while a lane holds more than one partial the level is
// transposed (each lane keeps half and adds its partner's half of the same
// sums), after that it is the plain butterfly.  With N = V partials and
// X = LPT/2, lane p of the row ends with max(1, V/LPT) sums: sum k + NF p
// (V >= LPT) or sum p >> log2(LPT/V) (V < LPT).
template <int X, int N>
__device__ inline void reduce_rows(float* a, int p) {
  if constexpr (X >= 1) {
    if constexpr (N > 1) {
      transpose_level<X, N>(a, p);
      reduce_rows<X / 2, N / 2>(a, p);
    } else {
      a[0] += swz_xor<X>(a[0]);
      reduce_rows<X / 2, 1>(a, p);
    }
  }
}

__device__ inline float row16_max(float v) {
  v = fmaxf(v, swz_xor<8>(v));
  v = fmaxf(v, swz_xor<4>(v));
  v = fmaxf(v, swz_xor<2>(v));
  return fmaxf(v, swz_xor<1>(v));
}

constexpr int ilog2c(int x) { return x <= 1 ? 0 : 1 + ilog2c(x / 2); }

// (m, s) of a softmax in the exp2 domain merged with another
__device__ inline void lse_merge(float& m, float& s, float om, float os) {
  const float mn = fmaxf(m, om);
  s = mn == -INFINITY ? 0.0f : s * exp2f(m - mn) + os * exp2f(om - mn);
  m = mn;
}

}  // namespace

// Persistent workgroups of W wavefronts over the (request, layer) items, one
// pass over the K table per kv head:
//  * each wavefront takes U blocks at a time; lane (t, p) holds 16 bytes of
//    K rows t + TPI i (i < NI) and the matching query dims of the G query
//    heads, forms the V = NI G partial dot products and sums them over the
//    row's LPT lanes (transposed reduction);
//  * the logits go through a small LDS tile, one 16-lane row per (block,
//    query head), where a 16-lane butterfly gives the block's softmax maximum
//    m_b and sum s_b = sum_t exp2(x_t - m_b) (exp2 domain: q is pre-scaled by
//    log2(e) / sqrt(128)); (m_b, s_b) go to the workgroup's workspace slice
//    and are merged into the query head's running (M, S);
//  * once (M, S) is merged over the workgroup, block b's mass is
//    sum over query heads of exp2(m_b - M) s_b / S, added to its LDS score.
// The scores then go through the same radix top-k as the Quest method and the
// layer's list is written to every kv head's row.  Dynamic LDS: max_n floats;
// workspace: max_n * G * 2 floats per workgroup.
template <int DT, int G, int W>
__global__ __launch_bounds__(W * 64) void k_select_mass(Geo g, const float* __restrict__ q,
                                                        const int32_t* __restrict__ ctx_blocks,
                                                        const uint8_t* __restrict__ kt,
                                                        const float* __restrict__ kt_scales,
                                                        uint64_t kt_mod, float* __restrict__ ws_all,
                                                        uint32_t* __restrict__ sel, int l0, int nl,
                                                        int max_n, int* __restrict__ err) {
  constexpr int ES = DT == FERRY_F32 ? 4 : (DT == FERRY_FP8_E4M3 ? 1 : 2);
  constexpr int D = 128, T = 16, NT = W * 64;
  constexpr int EPL = 16 / ES, LPT = D / EPL, TPI = 64 / LPT, NI = T / TPI;
  constexpr int V = NI * G, NF = V >= LPT ? V / LPT : 1, SH = V >= LPT ? 0 : ilog2c(LPT / V);
  constexpr uint32_t KT = T * D * ES;
  constexpr int U = G >= 4 ? 2 : 4;             // blocks in flight per wavefront
  constexpr int XW = 16 * G * U;                // logits of one wavefront's U blocks
  constexpr int R = (XW + 63) / 64;             // LDS tile rows per lane
  constexpr int NE = W * 4 * R;                 // running (M, S) entries per workgroup
  extern __shared__ uint32_t lds[];
  float* score = reinterpret_cast<float*>(lds);
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wtot[2 * W];
  __shared__ uint32_t sh[3];
  __shared__ float xl[W][XW];
  __shared__ float red_m[NE], red_s[NE], lse_m[G], lse_zi[G];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int p = lane % LPT, t = lane / LPT;
  float* ws = ws_all + (size_t)blockIdx.x * max_n * G * 2;
  const int n_items = g.n_req * nl;
  const float qmul = 1.4426950408889634f / sqrtf((float)D);  // log2(e) / sqrt(D)

  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    __syncthreads();  // the previous item's top-k is done with the LDS
    const int r = item / nl, l = l0 + item % nl;
    const int rl = r * g.L + l;
    int n = ctx_blocks[r];
    if (n < 0) n = 0;
    if (n > max_n || n > g.max_blocks) {
      if (tid == 0) set_error(err, FERRY_ERANGE);
      n = 0;
    }
    const int k = g.k;
    const int kk = n < k ? n : k;
    uint32_t* out0 = sel + (size_t)rl * g.Hkv * (size_t)k;
    if (n <= k) {
      for (int j = tid; j < k; j += NT)
        for (int hh = 0; hh < g.Hkv; ++hh) out0[(size_t)hh * k + j] = j < kk ? (uint32_t)j : kNone;
      continue;
    }
    for (int h = 0; h < g.Hkv; ++h) {
      const uint64_t set = (uint64_t)rl * g.Hkv + h;
      float qr[G][EPL];
#pragma unroll
      for (int gq = 0; gq < G; ++gq)
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          qr[gq][e] = q[((size_t)rl * g.Hq + (size_t)(h * G + gq)) * D + p * EPL + e] * qmul;
      float run_m[R], run_s[R];
#pragma unroll
      for (int rr = 0; rr < R; ++rr) run_m[rr] = -INFINITY, run_s[rr] = 0.0f;
      for (int b0 = wave; b0 < n; b0 += W * U) {
        u32x4 w[U][NI];
        float ks[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int b = b0 + W * u;
          if (b < n) {  // wavefront-uniform
            const uint64_t rec = host_index(set, (uint32_t)b, (uint64_t)g.max_blocks, kt_mod);
            const u32x4* base = reinterpret_cast<const u32x4*>(kt + rec * KT);
#pragma unroll
            for (int i = 0; i < NI; ++i) w[u][i] = __builtin_nontemporal_load(base + i * 64 + lane);
            ks[u] = kt_scales ? kt_scales[rec] : 1.0f;
          } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) w[u][i] = u32x4{0u, 0u, 0u, 0u};
            ks[u] = 0.0f;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float a[V];
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            float kf[EPL];
            decode_word<DT, EPL>(w[u][i], kf);
#pragma unroll
            for (int gq = 0; gq < G; ++gq) {
              float acc = 0.0f;
#pragma unroll
              for (int e = 0; e < EPL; ++e) acc = __fmaf_rn(qr[gq][e], kf[e], acc);
              a[gq * NI + i] = acc;
            }
          }
          reduce_rows<LPT / 2, V>(a, p);
          if (V >= LPT || (p & ((LPT >> ilog2c(V)) - 1)) == 0) {
#pragma unroll
            for (int kq = 0; kq < NF; ++kq) {
              const int v = V >= LPT ? kq + NF * p : (p >> SH);
              const int gq = v / NI, i = v % NI;
              xl[wave][u * 16 * G + gq * 16 + t + TPI * i] = a[kq] * ks[u];
            }
          }
        }
        wave_fence();
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
          const int idx = lane + 64 * rr;
          if (XW % 64 == 0 || idx < XW) {
            const float x = xl[wave][idx];
            const float m = row16_max(x);
            const float sm = row16_sum(exp2f(x - m));
            const int b = b0 + W * (idx / (16 * G));
            if ((lane & 15) == 0 && b < n) {
              const int gq = (idx >> 4) % G;
              ws[((size_t)b * G + gq) * 2] = m;
              ws[((size_t)b * G + gq) * 2 + 1] = sm;
              lse_merge(run_m[rr], run_s[rr], m, sm);
            }
          }
        }
        wave_fence();
      }
      // the workgroup's (M, S) of every query head
      if ((lane & 15) == 0) {
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
          red_m[(wave * 4 + (lane >> 4)) * R + rr] = run_m[rr];
          red_s[(wave * 4 + (lane >> 4)) * R + rr] = run_s[rr];
        }
      }
      __syncthreads();
      if (tid < G) {
        float mm = -INFINITY, ss = 0.0f;
        for (int e = 0; e < NE; ++e) {
          const int c = e / R, rr = e % R;  // entry of lane 16 (c % 4) of wave c / 4, tile row rr
          const int idx = (c % 4) * 16 + 64 * rr;
          if (idx < XW && (idx >> 4) % G == tid) lse_merge(mm, ss, red_m[e], red_s[e]);
        }
        lse_m[tid] = mm;
        lse_zi[tid] = 1.0f / ss;
      }
      __syncthreads();
      for (int b = tid; b < n; b += NT) {
        float acc = 0.0f;
#pragma unroll
        for (int gq = 0; gq < G; ++gq)
          acc += exp2f(ws[((size_t)b * G + gq) * 2] - lse_m[gq]) * ws[((size_t)b * G + gq) * 2 + 1] *
                 lse_zi[gq];
        score[b] = h == 0 ? acc : score[b] + acc;
      }
      __syncthreads();
    }
    for (int b = tid; b < n; b += NT) lds[b] = fkey(score[b]);
    __syncthreads();
    topk_ascending<W>(lds, n, kk, hist, wtot, sh, out0, g.Hkv, (size_t)k);
    for (int j = kk + tid; j < k; j += NT)
      for (int hh = 0; hh < g.Hkv; ++hh) out0[(size_t)hh * k + j] = kNone;
  }
}

// Matrix-core mass selection for 16-bit and fp8 K, in two launches.
//
// k_mass_units: one (request, layer, kv head) unit per workgroup pass, each
// workgroup taking the next unit from a counter (k_mass_reset zeroes it before
// the launch), so a grid of the workgroups the GPU holds at once drains the
// units in order and evenly; the result does not depend on which workgroup
// scores a unit.  Per block the scores of the G query heads are
// one 16 x 16 tile on the matrix cores,
//   S^T[16 tok][16 hd] = K[16 tok][128] . Q^T[128][16 hd]   (4 k-steps of 32),
// with the heads padded to 16 columns, in the operand layout of k_attn_mfma:
// lane l (n = l % 16, grp = l / 16) holds the 16-byte words 4 w + grp of
// token n's K row (one contiguous 1 KiB load per w from the lane-transposed
// record), the matching query dims of head n, and receives the
// scores of tokens 4 grp + i (i < 4) of head n.  A block's (m_b, s_b) of head
// n is then a 4-element max/sum in the lane and two cross-lane steps (xor 16,
// 32); it goes into the wavefront's running (M, S) and is kept for the last
// pass: as l_b = m_b + log2(s_b) in LDS when max_n * G floats fit there
// (ws_all null), else as (m_b, s_b) in the workgroup's workspace slice in
// HBM.  Once (M, S) is merged over the workgroup (wavefront order), block b's
// mass for this kv head, sum over its query heads of exp2(l_b - M - log2 S)
// (or exp2(m_b - M) s_b / S), goes to mass[unit][b].  At the long-context GQA
// shape the round trip through HBM made the launch 0.80 or 0.84 of HBM by
// where the K table landed, and dropping it 0.85-0.86 wherever it did.  The query, pre-scaled by
// log2(e) / sqrt(128), is split into NQ operand-precision terms (fp16 hi + lo
// for fp16 and fp8 K, bf16 hi + mid + lo for bf16 K) so the fp32 accumulation
// sees ~22-24 bits of it; fp8 K is widened to fp16 exactly and its block scale
// multiplies the scores.
//
// One kv head per workgroup streams one contiguous run of the K table (32 MiB
// at 8192 blocks of 16-bit K): at the long-context GQA shape that measured
// 0.80-0.84 of HBM (by where the 137 GB table landed) against 0.79 for a
// whole (request, layer) item per workgroup, whose kv heads stream one after
// the other.
template <int DT, int G, int W, int U>
__global__ __launch_bounds__(W * 64) void k_mass_units(
    Geo g, const float* __restrict__ q, const int32_t* __restrict__ ctx_blocks,
    const uint8_t* __restrict__ kt, const float* __restrict__ kt_scales, uint64_t kt_mod,
    float* __restrict__ ws_all, float* __restrict__ mass, unsigned* __restrict__ counter, int l0,
    int nl, int max_n, int* __restrict__ err) {
  static_assert(G >= 1 && G <= 16, "the score tile holds up to 16 query heads");
  static_assert(DT == FERRY_F16 || DT == FERRY_BF16 || DT == FERRY_FP8_E4M3, "16/8-bit K");
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  constexpr bool F8 = DT == FERRY_FP8_E4M3, BF = DT == FERRY_BF16;
  constexpr int D = 128, T = 16, NT = W * 64;
  constexpr int ES = F8 ? 1 : 2;
  constexpr uint32_t ROW = D * ES, KT = T * ROW;
  constexpr int NKW = F8 ? 2 : 4;  // 16-byte K words per lane per block
  constexpr int EPW = 16 / ES, SUB = EPW / 8;
  constexpr int NQ = BF ? 3 : 2;   // query terms
  __shared__ float red_m[W][G], red_s[W][G], lse_m[G], lse_zi[G], lse_l[G];
  __shared__ unsigned next_unit;
  extern __shared__ float lws[];  // [max_n][G] block log-sums when ws_all is null
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, grp = lane >> 4;
  const bool head_lane = grp == 0 && n < G;
  const bool in_lds = ws_all == nullptr;  // workgroup-uniform
  float* ws = in_lds ? nullptr : ws_all + (size_t)blockIdx.x * max_n * G * 2;
  const unsigned n_units = (unsigned)(g.n_req * nl * g.Hkv);
  const float qmul = 1.4426950408889634f / sqrtf((float)D);  // log2(e) / sqrt(D)

  for (;;) {
    // the previous unit is done with the LDS and the workspace slice
    if (tid == 0) next_unit = atomicAdd(counter, 1u);
    __syncthreads();
    const unsigned un = next_unit;
    __syncthreads();  // every thread has read next_unit before it is rewritten
    if (un >= n_units) break;  // workgroup-uniform; every unit is taken once
    const int unit = (int)un;
    const int item = unit / g.Hkv, h = unit % g.Hkv;
    const int r = item / nl, l = l0 + item % nl;
    const int rl = r * g.L + l;
    int nb = ctx_blocks[r];
    if (nb < 0) nb = 0;
    if (nb > max_n || nb > g.max_blocks) {
      if (tid == 0 && h == 0) set_error(err, FERRY_ERANGE);
      nb = 0;
    }
    if (nb <= g.k) continue;  // workgroup-uniform: k_mass_topk lists every block
    const uint64_t set = (uint64_t)rl * g.Hkv + h;
    // ---- Q^T operand: k-step ks, this lane's 8 dims, head n (0 for pad heads)
    uint32_t qb[NQ][4][4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int d0 = EPW * (4 * (ks / SUB) + grp) + 8 * (ks % SUB);
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        x[e] = n < G ? q[((size_t)rl * g.Hq + (size_t)(h * G + n)) * D + d0 + e] * qmul : 0.0f;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float a = x[e], b = x[e + 1];
#pragma unroll
        for (int t = 0; t < NQ; ++t) {
          if constexpr (BF) {
            const uint16_t ah = bf16_rne(a), bh = bf16_rne(b);
            qb[t][ks][e / 2] = (uint32_t)ah | ((uint32_t)bh << 16);
            a -= __builtin_bit_cast(float, (uint32_t)ah << 16);
            b -= __builtin_bit_cast(float, (uint32_t)bh << 16);
          } else {
            const _Float16 ah = (_Float16)a, bh = (_Float16)b;
            qb[t][ks][e / 2] = (uint32_t)__builtin_bit_cast(uint16_t, ah) |
                               ((uint32_t)__builtin_bit_cast(uint16_t, bh) << 16);
            a -= (float)ah;
            b -= (float)bh;
          }
        }
      }
    }
    float run_m = -INFINITY, run_s = 0.0f;
    for (int b0 = wave; b0 < nb; b0 += W * U) {
      u32x4 kw[U][NKW];
      float ksc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int b = b0 + W * u;
        if (b < nb) {  // wavefront-uniform
          const uint64_t rec = host_index(set, (uint32_t)b, (uint64_t)g.max_blocks, kt_mod);
          // lane-transposed record: this lane's word w is word 64 w + lane
          const u32x4* base = reinterpret_cast<const u32x4*>(kt + rec * KT) + lane;
#pragma unroll
          for (int w = 0; w < NKW; ++w) kw[u][w] = __builtin_nontemporal_load(base + 64 * w);
          ksc[u] = F8 ? kt_scales[rec] : 1.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int b = b0 + W * u;
        if (b >= nb) break;  // wavefront-uniform
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int w = ks / SUB, sub = ks % SUB;
          u32x4 a;
          if constexpr (F8) {
            const mx_u32x2 lo = e4m3x4_to_f16(kw[u][w][2 * sub]);
            const mx_u32x2 hi = e4m3x4_to_f16(kw[u][w][2 * sub + 1]);
            a = u32x4{lo[0], lo[1], hi[0], hi[1]};
          } else {
            a = kw[u][w];
          }
#pragma unroll
          for (int t = 0; t < NQ; ++t) {
            const u32x4 bq = {qb[t][ks][0], qb[t][ks][1], qb[t][ks][2], qb[t][ks][3]};
            if constexpr (BF)
              s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                          __builtin_bit_cast(bf16x8, bq), s, 0, 0, 0);
            else
              s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                         __builtin_bit_cast(f16x8, bq), s, 0, 0, 0);
          }
        }
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = s[i] * ksc[u];
        float m = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
        m = max_over_groups(m);
        float e = (exp2f(x[0] - m) + exp2f(x[1] - m)) + (exp2f(x[2] - m) + exp2f(x[3] - m));
        e = sum_over_groups(e);
        if (head_lane) {
          if (in_lds) {
            lws[b * G + n] = m + log2f(e);  // the block's log2-sum-exp2
          } else {
            ws[((size_t)b * G + n) * 2] = m;
            ws[((size_t)b * G + n) * 2 + 1] = e;
          }
          lse_merge(run_m, run_s, m, e);
        }
      }
    }
    // the workgroup's (M, S) of every query head
    if (head_lane) {
      red_m[wave][n] = run_m;
      red_s[wave][n] = run_s;
    }
    __syncthreads();
    if (tid < G) {
      float mm = -INFINITY, ss = 0.0f;
      for (int w = 0; w < W; ++w) lse_merge(mm, ss, red_m[w][tid], red_s[w][tid]);
      lse_m[tid] = mm;
      lse_zi[tid] = 1.0f / ss;
      lse_l[tid] = mm + log2f(ss);  // the unit's log2-sum-exp2
    }
    __syncthreads();
    float* mrow = mass + (size_t)unit * max_n;
    for (int b = tid; b < nb; b += NT) {
      float acc = 0.0f;
      if (in_lds) {
#pragma unroll
        for (int gq = 0; gq < G; ++gq) acc += exp2f(lws[b * G + gq] - lse_l[gq]);
      } else {
#pragma unroll
        for (int gq = 0; gq < G; ++gq)
          acc += exp2f(ws[((size_t)b * G + gq) * 2] - lse_m[gq]) * ws[((size_t)b * G + gq) * 2 + 1] *
                 lse_zi[gq];
      }
      mrow[b] = acc;
    }
  }
}

__global__ void k_mass_reset(unsigned* counter) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *counter = 0u;
}

// k_mass_topk: one (request, layer) item per workgroup pass.  A block's score
// is its mass summed over the kv heads in head order (mass[unit][b] of the
// item's Hkv units, written by k_mass_units in the same stream); the scores go
// through the same radix top-k as the Quest method and the item's list is
// written to every kv head's row.  A context of at most k blocks lists every
// block in order.  Dynamic LDS: max_n keys.
template <int W>
__global__ __launch_bounds__(W * 64) void k_mass_topk(Geo g, const int32_t* __restrict__ ctx_blocks,
                                                      const float* __restrict__ mass,
                                                      uint32_t* __restrict__ sel, int l0, int nl,
                                                      int max_n) {
  constexpr int NT = W * 64;
  extern __shared__ uint32_t lds[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wtot[2 * W];
  __shared__ uint32_t sh[3];
  const int tid = threadIdx.x;
  const int n_items = g.n_req * nl;
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    __syncthreads();  // the previous item's top-k is done with the LDS
    const int r = item / nl, l = l0 + item % nl;
    const int rl = r * g.L + l;
    int nb = ctx_blocks[r];
    if (nb < 0 || nb > max_n || nb > g.max_blocks) nb = 0;  // k_mass_units latched the error
    const int k = g.k;
    const int kk = nb < k ? nb : k;
    uint32_t* out0 = sel + (size_t)rl * g.Hkv * (size_t)k;
    if (nb <= k) {
      for (int j = tid; j < k; j += NT)
        for (int hh = 0; hh < g.Hkv; ++hh) out0[(size_t)hh * k + j] = j < kk ? (uint32_t)j : kNone;
      continue;
    }
    const float* m0 = mass + (size_t)item * g.Hkv * max_n;
    for (int b = tid; b < nb; b += NT) {
      float s = m0[b];
      for (int hh = 1; hh < g.Hkv; ++hh) s += m0[(size_t)hh * max_n + b];
      lds[b] = fkey(s);
    }
    __syncthreads();
    topk_ascending<W>(lds, nb, kk, hist, wtot, sh, out0, g.Hkv, (size_t)k);
    for (int j = kk + tid; j < k; j += NT)
      for (int hh = 0; hh < g.Hkv; ++hh) out0[(size_t)hh * k + j] = kNone;
  }
}

#define FERRY_MASS_INST(DT, G)                                                                   \
  template __global__ void k_select_mass<DT, G, 4>(Geo, const float*, const int32_t*,              \
                                                   const uint8_t*, const float*, uint64_t, float*, \
                                                   uint32_t*, int, int, int, int*);
#define FERRY_MASS_UNITS_INST(DT, G)                                                          \
  template __global__ void k_mass_units<DT, G, kMassUnitWaves, kMassUnitInflight>(            \
      Geo, const float*, const int32_t*, const uint8_t*, const float*, uint64_t, float*, float*, \
      unsigned*, int, int, int, int*);
#define FERRY_MASS_UNITS_INST_G(DT) \
  FERRY_MASS_UNITS_INST(DT, 1)      \
  FERRY_MASS_UNITS_INST(DT, 2)      \
  FERRY_MASS_UNITS_INST(DT, 4)      \
  FERRY_MASS_UNITS_INST(DT, 8)
FERRY_MASS_INST(FERRY_F32, 1)
FERRY_MASS_INST(FERRY_F32, 2)
FERRY_MASS_INST(FERRY_F32, 4)
FERRY_MASS_INST(FERRY_F32, 8)
FERRY_MASS_UNITS_INST_G(FERRY_F16)
FERRY_MASS_UNITS_INST_G(FERRY_BF16)
FERRY_MASS_UNITS_INST_G(FERRY_FP8_E4M3)
template __global__ void k_mass_topk<kMassTopkWaves>(Geo, const int32_t*, const float*, uint32_t*, int,
                                                     int, int);
template __global__ void k_ktiles_build<2>(Geo, const uint8_t*, const float*, uint8_t*, float*, int);
template __global__ void k_ktiles_build<4>(Geo, const uint8_t*, const float*, uint8_t*, float*, int);
template __global__ void k_ktiles_build<8>(Geo, const uint8_t*, const float*, uint8_t*, float*, int);

#define FERRY_SUMS_INST(DT)                                                                 \
  template __global__ void k_summaries_build<DT>(Geo, const uint8_t*, const float*, uint8_t*, \
                                                 float*);
FERRY_SUMS_INST(FERRY_F32)
FERRY_SUMS_INST(FERRY_F16)
FERRY_SUMS_INST(FERRY_BF16)
FERRY_SUMS_INST(FERRY_FP8_E4M3)

#define FERRY_SEL_INST(DT, G, LAYER)                                                           \
  template __global__ void k_select_topk<DT, G, LAYER, 4>(Geo, const float*, const int32_t*,     \
                                                          const uint8_t*, const float*, uint64_t,  \
                                                          uint32_t*, int, int, int, int*);
#define FERRY_SEL_INST_G(DT, LAYER) \
  FERRY_SEL_INST(DT, 1, LAYER)      \
  FERRY_SEL_INST(DT, 2, LAYER)      \
  FERRY_SEL_INST(DT, 4, LAYER)      \
  FERRY_SEL_INST(DT, 8, LAYER)
#define FERRY_SEL_INST_ALL(LAYER)          \
  FERRY_SEL_INST_G(FERRY_F32, LAYER)       \
  FERRY_SEL_INST_G(FERRY_F16, LAYER)       \
  FERRY_SEL_INST_G(FERRY_BF16, LAYER)      \
  FERRY_SEL_INST_G(FERRY_FP8_E4M3, LAYER)
FERRY_SEL_INST_ALL(false)
FERRY_SEL_INST_ALL(true)

}  // namespace ferry_amd
