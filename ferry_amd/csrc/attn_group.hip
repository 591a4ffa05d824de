// attn_group.hip -- block-sparse decode attention of a whole prefix group per
// workgroup, reading every distinct selected block of the group's set once.
//
// Same result as k_attn_mfma (attn_mfma.hip) for every member row:
// out[r,l,hq] = softmax(q K^T / sqrt(D)) V over the tokens of the k blocks
// selected for (r, l, kv head of hq), a block selected twice in one row counted
// twice, a row with nothing selected giving 0.  The reference has only an FMA
// proxy (src/workloads/kv_exec.cuh:30-37); the semantics are the textbook
// softmax attention of the top-k pages selected in
// tools/capture_miss_trace.py:139-159.  Prefix groups share one LRU set per
// (group, layer, kv head) (src/runtime/wla_multigpu.cuh:323-349, wla_gslot_off),
// so the members' selections of the shared prefix land on the same slots.
//
// One workgroup of W = 4 wavefronts per (group, layer, kv head), two per CU
// (the LDS is mostly the wavefronts' block rings).  The group's
// query columns (member x query head, NTILE tiles of 16, attn_mfma.hpp) are
// held by every wavefront; the blocks are split between the wavefronts.
//  1. List: every member row's slots are OR-ed into a per-slot member mask in
//     LDS (one word per slot of the set).  A repeated selection in one row,
//     or a slot outside the row's set, becomes an entry of its own with that
//     member alone.  The masks are compacted in slot order, then the own
//     entries ordered by (member, slot), so the list and the summation order
//     do not depend on the order the atomics ran in.
//  2. Blocks: entry j of the list goes to wavefront j mod W, which streams its
//     entries through its own ring of R blocks in LDS (three fp8 or two 16-bit
//     blocks) with direct-to-LDS
//     16-byte loads (global_load_lds_dwordx4, non-temporal: each block is read
//     once), R blocks ahead: a slot takes the next block as soon as the
//     block it held is read into registers.  A wavefront waits only on its
//     own load counter: no workgroup barrier in the loop.  The block's rows and 16-byte chunks are
//     permuted (lds_row, lds_chunk) so that the K reads (one row per lane, one
//     chunk offset) and the V reads (four rows across the wavefront) hit
//     distinct banks whether the LDS serves 128 or 256 bytes per pass.
//  3. Attention: a block's K and V operands are built once (block_operands)
//     and every query tile with a member that selected the block attends to
//     it (tile_block); the columns of members that did not are masked, so
//     every member accumulates exactly its own blocks.  The tiles' Q^T
//     operands wait in LDS (one conflict-free 16-byte read per lane and
//     k-slice), so a wavefront's registers hold the accumulators of all its
//     columns but only one tile's queries at a time.
//  4. Merge: the W wavefronts' partial softmax states of each column are
//     combined through LDS (max, rescaled sums and outputs), as k_attn_mfma
//     merges its wavefronts.
// HBM bytes per launch: the distinct blocks of each group set once (plus q in,
// out and the slot table), against k blocks per member row for k_attn_mfma.
#include "attn_mfma.hpp"
#include "kernels.hpp"

namespace ferry_amd {

using namespace mx;

namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// Block layout in LDS.  Row t (0..15) of a K or V tile is stored as row
// lds_row(t), and its logical 16-byte chunk c at chunk c ^ lds_chunk(row).
// fp8 rows are 128 bytes, two to a 256-byte bank line: rows 4..7 and 12..15
// swap within their pairs, so the V rows 4g+i read together (g = 0..3) fall
// in different halves of a line, and the chunk key (p ^ p/8) mod 8 differs
// between the eight rows of one half and between rows 0..7 (and 8..15), so
// the K reads (rows 0..15, one chunk offset) are conflict-free.  16-bit rows
// are 256 bytes: the chunk key is the row number.
template <int ES>
__device__ inline int lds_row(int t) {
  return ES == 1 ? t ^ ((t >> 2) & 1) : t;  // an involution
}
template <int ES>
__device__ inline int lds_chunk(int p) {
  return ES == 1 ? (p ^ (p >> 3)) & 7 : p & 15;
}

// Wait until at most N vector-memory loads of this wavefront are outstanding.
// The "memory" clobber keeps the LDS reads of the landed block below it.
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until the oldest of this wavefront's outstanding block loads are done,
// leaving `later` (<= K) younger blocks of NI loads each in flight.
template <int NI, int K>
__device__ inline void wait_blocks(int later) {
  if constexpr (K == 0) {
    wait_vmcnt<0>();
  } else {
    if (later >= K) wait_vmcnt<K * NI>();
    else wait_blocks<NI, K - 1>(later);
  }
}

// Exclusive prefix sum of v over the workgroup's threads (thread order);
// *total = the sum over all.  `sh` is LDS scratch of W ints.  Barriers on
// entry and exit, so `sh` can be reused right after.
template <int W>
__device__ inline int block_exclusive_scan(int v, int* sh, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  __syncthreads();
  if (lane == 63) sh[wave] = x;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int c = sh[w];
    before += w < wave ? c : 0;
    tot += c;
  }
  *total = tot;
  __syncthreads();
  return before + x - v;
}

}  // namespace

template <int DT, int G, int NTILE, int W>
__global__ __launch_bounds__(W * 64) void k_attn_group(
    Geo g, const float* __restrict__ q, const uint32_t* __restrict__ slots,
    const uint8_t* __restrict__ pool, const float* __restrict__ pool_scales,
    float* __restrict__ out, float qscale, int l0, int nl, int* __restrict__ err,
    unsigned long long* __restrict__ attn_blocks) {
  static_assert(G == 2 || G == 4 || G == 8, "GQA group of 2, 4 or 8 query heads");
  static_assert(NTILE >= 1 && NTILE <= kGroupMaxTiles, "query tiles per workgroup");
  static_assert(DT == FERRY_F16 || DT == FERRY_BF16 || DT == FERRY_FP8_E4M3, "16/8-bit KV");
  using S = Shape<DT>;
  constexpr int D = S::D, T = S::T, NKW = S::NKW, VW = S::VW, ES = S::ES;
  constexpr int ROW = (int)S::ROW;     // bytes of one token row
  constexpr int RC = ROW / 16;         // 16-byte chunks of a row (8 or 16)
  constexpr int BB = 2 * T * ROW;      // bytes of one block, K tile then V tile
  constexpr int NI = BB / 1024;        // direct-to-LDS loads of one block per wavefront
  static_assert(W == group_waves(DT) || W == kGroupWideWaves, "wavefronts per workgroup");
  constexpr int NT = W * 64;           // threads
  constexpr int MPT = 16 / G;          // members per query tile
  constexpr int R = group_ring_blocks(DT);   // ring blocks per wavefront
  constexpr int RB = group_ring_bytes(DT);    // ring bytes per wavefront
  constexpr int NQ = S::BF ? 2 : 1;           // parts of the Q^T operands (bf16: hi, lo)
  constexpr int COLS = 16 * NTILE;            // query columns
  // tiles merged per round: W/2 wavefronts stage TT tiles of 8 KiB each in
  // the rings and the Q^T operands, free once the blocks are consumed
  constexpr int TT_FIT = (W * RB + NQ * NTILE * 4 * 64 * 16) / ((W / 2) * 8192);
  constexpr int TT = NTILE < TT_FIT ? NTILE : TT_FIT;
  static_assert(RB == R * BB && R >= 2 && (R - 1) * NI < 64, "ring depth and load counter");
  static_assert(TT >= 1, "a merge round fits the rings and the Q^T operands");
  static_assert(NTILE <= W, "each wavefront stages at most one query tile");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int GK = g.group * g.k;
  uint8_t* rings = smem;                                                  // [W][R][BB]
  u32x4* qops = reinterpret_cast<u32x4*>(smem + W * RB);                  // [NQ][NTILE][4][64]
  uint32_t* lslot = reinterpret_cast<uint32_t*>(qops + NQ * NTILE * 4 * 64);  // [GK] list
  uint32_t* lmask = lslot + GK;                                           // [GK] members
  float* red_ml = reinterpret_cast<float*>(lmask + GK);                   // [W][COLS][2]
  int* sh = reinterpret_cast<int*>(red_ml + W * COLS * 2);                // [W] scan
  uint32_t* msk = reinterpret_cast<uint32_t*>(rings);                     // [C] listing
  uint32_t* own = msk + g.C;                                              // [GK] listing
  uint32_t* mcnt = own + GK;                                              // [group] listing

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 15, grp = lane >> 4;
  const int h = blockIdx.x % g.Hkv;
  const int l = l0 + (blockIdx.x / g.Hkv) % nl;
  const int o = blockIdx.x / (nl * g.Hkv);
  const int mem = min(g.group, g.n_req - o * g.group);  // member rows of this owner
  const uint32_t base = (uint32_t)((o * g.L + l) * g.Hkv + h) * (uint32_t)g.C;

  // The global reads of the prologue go out together, so the workgroup pays
  // one round trip before its first block loads, not one per read: the query
  // values of the tile this wavefront stages, then this thread's first SB
  // selections (the other workgroups on the CU keep the memory busy meanwhile)
  float qx[4][8];
  if (wave < NTILE) {  // tile `wave`: column n is member wave*MPT + n/G
    const int mi = wave * MPT + n / G;
    const size_t qrow = (size_t)((o * g.group + mi) * g.L + l) * g.Hq + (size_t)h * G + n % G;
    q_load<DT>(mi < mem ? q + qrow * D : nullptr, grp, qx);
  }
  constexpr int SB = 4;  // selections in flight per thread
  auto load_sel = [&](int e0, uint32_t (&sv)[SB]) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int e = e0 + u * NT, mi = e / g.k;
      sv[u] = kNone;
      if (e < GK && mi < mem)
        sv[u] = slots[((size_t)((o * g.group + mi) * g.L + l) * g.Hkv + h) * g.k + (e - mi * g.k)];
    }
  };
  uint32_t sv[SB];
  load_sel(tid, sv);

  // ---- 1. the distinct list of the group's selections
  for (int i = tid; i < g.C; i += NT) msk[i] = 0u;
  for (int i = tid; i < g.group; i += NT) mcnt[i] = 0u;
  __syncthreads();
  bool bad = false;
  for (int e0 = tid; e0 < GK; e0 += NT * SB) {
    if (e0 != tid) load_sel(e0, sv);
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int e = e0 + u * NT, mi = e / g.k;
      if (e >= GK) break;
      uint32_t s = sv[u], mine = kNone;
      if (s != kNone) {
        if (s >= g.pool_slots) {  // read as slot 0 and reported, as k_attn_mfma does
          bad = true;
          s = 0;
        }
        const uint32_t loc = s - base;
        if (loc < (uint32_t)g.C) {
          const uint32_t bit = 1u << mi;
          if (atomicOr(&msk[loc], bit) & bit) mine = s;  // a repeat in this row
        } else {
          mine = s;  // outside the set
        }
      }
      own[e] = mine;
      if (mine != kNone) atomicAdd(&mcnt[mi], 1u);
    }
  }
  if (bad) set_error(err, FERRY_ERANGE);
  __syncthreads();
  // masks in slot order: each thread compacts a contiguous range of slots
  const int per = (g.C + NT - 1) / NT;
  const int c0 = min(g.C, tid * per), c1 = min(g.C, c0 + per);
  int cnt = 0;
  for (int i = c0; i < c1; ++i) cnt += msk[i] != 0u;
  int n_in = 0;
  int pos = block_exclusive_scan<W>(cnt, sh, &n_in);
  for (int i = c0; i < c1; ++i) {
    const uint32_t mm = msk[i];
    if (mm) {
      lslot[pos] = base + (uint32_t)i;
      lmask[pos] = mm;
      ++pos;
    }
  }
  // own entries after them, ordered by (member, slot); equal keys are the same
  // block for the same member, so their order among themselves does not matter.
  // An entry's rank: the own entries of earlier members (their counts) and
  // those of its own member's row before it, k positions instead of group * k
  int cown = 0;
  for (int e = tid; e < GK; e += NT) cown += own[e] != kNone;
  int n_own = 0;
  (void)block_exclusive_scan<W>(cown, sh, &n_own);
  if (n_own > 0) {  // uniform
    for (int e = tid; e < GK; e += NT) {
      const uint32_t s = own[e];
      if (s == kNone) continue;
      const int mi = e / g.k;
      int rank = 0;
      for (int m = 0; m < mi; ++m) rank += (int)mcnt[m];
      for (int e2 = mi * g.k; e2 < (mi + 1) * g.k; ++e2) {
        const uint32_t s2 = own[e2];
        rank += s2 != kNone && (s2 < s || (s2 == s && e2 < e));
      }
      lslot[n_in + rank] = s;
      lmask[n_in + rank] = 1u << mi;
    }
  }
  const int nlist = n_in + n_own;
  if (attn_blocks && tid == 0) atomicAdd(attn_blocks, (unsigned long long)nlist);
  __syncthreads();  // the rings may now overwrite msk / own

  // ---- Q^T operands of every tile, staged in LDS lane by lane (wavefront w
  // builds tile w from the values it read first): column n of tile t is
  // member t*MPT + n/G, query head h*G + n%G (zeros past the group's members)
  if (wave < NTILE) {
    const int t = wave;
    uint32_t qh[4][4], ql[4][4];
    q_convert<DT>(qx, qscale, qh, ql);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      qops[(t * 4 + kk) * 64 + lane] = u32x4{qh[kk][0], qh[kk][1], qh[kk][2], qh[kk][3]};
      if constexpr (NQ == 2)
        qops[((NTILE + t) * 4 + kk) * 64 + lane] = u32x4{ql[kk][0], ql[kk][1], ql[kk][2], ql[kk][3]};
    }
  }
  uint32_t tile_bits[NTILE], col_bit[NTILE];
  Acc acc[NTILE];
  const uint32_t mem_bits = (uint32_t)((1ull << mem) - 1ull);
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const int mi = t * MPT + n / G;
    tile_bits[t] = (((1u << MPT) - 1u) << (t * MPT)) & mem_bits;
    col_bit[t] = mi < mem ? 1u << mi : 0u;
    acc[t].init();
  }
  __syncthreads();  // Q^T operands staged

  // ---- 2./3. this wavefront's entries wave, wave + W, ... through its ring
  const int nb = nlist > wave ? (nlist - wave + W - 1) / W : 0;
  uint8_t* ring = rings + wave * RB;
  // block j of this wavefront into ring slot b: lane fills chunk p = i*64 +
  // lane of the block: LDS row pr of its tile holds token row lds_row(pr),
  // whose logical chunk (p mod RC) ^ lds_chunk(pr) sits there
  auto issue = [&](int j, int b) {
    const uint32_t slot = (uint32_t)__builtin_amdgcn_readfirstlane((int)lslot[wave + W * j]);
    const uint8_t* src = pool + (uint64_t)slot * BB;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int p = i * 64 + lane;
      const int tile = p / (T * RC), pr = (p / RC) % T;
      const int off = (tile * T + lds_row<ES>(pr)) * ROW + ((p % RC) ^ lds_chunk<ES>(pr)) * 16;
      __builtin_amdgcn_global_load_lds((glb_void*)(src + off),
                                       (lds_void*)(ring + b * BB + i * 1024), 16, 0, 2 /* nt */);
    }
  };
  // K word w of lane (n, grp): token n, logical chunk 4w + grp.  V of token i:
  // row 4*grp + i of the V tile, elements 8n..8n+7 (logical chunk n/2, half n%2
  // for fp8; chunk n for 16-bit).
  const int kr = lds_row<ES>(n);
  auto read_block = [&](const uint8_t* blk, u32x4 (&kw)[NKW], uint32_t (&vw)[4][VW]) {
#pragma unroll
    for (int w = 0; w < NKW; ++w)
      kw[w] = *reinterpret_cast<const u32x4*>(blk + kr * ROW +
                                              (((4 * w + grp) ^ lds_chunk<ES>(kr)) * 16));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int vr = lds_row<ES>(4 * grp + i);
      const uint8_t* vrow = blk + (T + vr) * ROW;
      if constexpr (S::F8) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(
            vrow + (((n >> 1) ^ lds_chunk<ES>(vr)) * 16) + (n & 1) * 8);
        vw[i][0] = v[0], vw[i][1] = v[1];
      } else {
        const u32x4 v = *reinterpret_cast<const u32x4*>(vrow + ((n ^ lds_chunk<ES>(vr)) * 16));
        vw[i][0] = v[0], vw[i][1] = v[1], vw[i][2] = v[2], vw[i][3] = v[3];
      }
    }
  };
#pragma unroll
  for (int b = 0; b < R; ++b)
    if (b < nb) issue(b, b);
  for (int j0 = 0; j0 < nb; j0 += R) {
#pragma unroll
    for (int b = 0; b < R; ++b) {
      const int j = j0 + b;
      if (j < nb) {  // uniform
        // block j landed once at most the later blocks issued are in flight
        wait_blocks<NI, R - 1>(min(R - 1, nb - 1 - j));
        const int li = wave + W * j;
        const uint32_t mm = (uint32_t)__builtin_amdgcn_readfirstlane((int)lmask[li]);
        float ks = 1.0f, vs = 1.0f;
        if constexpr (S::F8) {
          const uint32_t slot = (uint32_t)__builtin_amdgcn_readfirstlane((int)lslot[li]);
          ks = pool_scales[2 * (uint64_t)slot];
          vs = pool_scales[2 * (uint64_t)slot + 1];
        }
        u32x4 kw[NKW];
        uint32_t vw[4][VW];
        read_block(ring + b * BB, kw, vw);
        if (j + R < nb) {
          // the block's LDS reads have returned: its ring slot takes block
          // j + R, so R blocks stay in flight while this one is attended
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          issue(j + R, b);
        }
        Ops op;
        block_operands<DT>(kw, vw, op);
#pragma unroll
        for (int t = 0; t < NTILE; ++t) {
          if (mm & tile_bits[t]) {  // uniform: a member of tile t selected the block
            uint32_t qh[4][4], ql[4][4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
              const u32x4 a = qops[(t * 4 + kk) * 64 + lane];
              qh[kk][0] = a[0], qh[kk][1] = a[1], qh[kk][2] = a[2], qh[kk][3] = a[3];
              if constexpr (NQ == 2) {
                const u32x4 b = qops[((NTILE + t) * 4 + kk) * 64 + lane];
                ql[kk][0] = b[0], ql[kk][1] = b[1], ql[kk][2] = b[2], ql[kk][3] = b[3];
              } else {
                ql[kk][0] = ql[kk][1] = ql[kk][2] = ql[kk][3] = 0u;
              }
            }
            tile_block<DT, true>(op, ks, vs, qh, ql, acc[t], (mm & col_bit[t]) != 0u);
          }
        }
      }
    }
  }

  // ---- 4. merge the wavefronts' states.  (a) Every wavefront's per-column
  // max and sum go to LDS; (b) each wavefront scales its accumulators to the
  // column's final weights, o_w * vs_ref_w * 2^(m_w - M) / L with M the max
  // over the wavefronts and L = sum_w l_w 2^(m_w - M) (0 where the column
  // attended nothing); (c) the scaled accumulators are summed through LDS in
  // a tree (wavefronts [h, 2h) write, [0, h) add, h = W/2 .. 1), TT tiles at a
  // time, in a fixed order; (d) wavefront 0 writes the outputs.
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    float lsum = acc[t].lsum;
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (grp == 0) {
      red_ml[(wave * COLS + 16 * t + n) * 2] = acc[t].m;
      red_ml[(wave * COLS + 16 * t + n) * 2 + 1] = lsum;
    }
  }
  __syncthreads();  // red_ml complete; the rings and the Q^T operands are free
#pragma unroll
  for (int t = 0; t < NTILE; ++t) {
    const int col = 16 * t + n;
    float mx = kNeg;
#pragma unroll
    for (int w = 0; w < W; ++w) mx = fmaxf(mx, red_ml[(w * COLS + col) * 2]);
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w)
      lt += red_ml[(w * COLS + col) * 2 + 1] * exp2_fast(red_ml[(w * COLS + col) * 2] - mx);
    const float vref = S::F8 ? acc[t].vs_ref : 1.0f;
    const float f = lt > 0.0f ? exp2_fast(acc[t].m - mx) * vref / lt : 0.0f;
#pragma unroll
    for (int v = 0; v < 8; ++v) acc[t].o[v] *= f;
  }
  f32x4* stage = reinterpret_cast<f32x4*>(smem);  // [W/2][TT][8][64], lane-major
#pragma unroll
  for (int t0 = 0; t0 < NTILE; t0 += TT) {
    if (t0 > 0) __syncthreads();  // wavefront 0 has read the last round
#pragma unroll
    for (int hw = W / 2; hw >= 1; hw /= 2) {
      if (wave >= hw && wave < 2 * hw) {
#pragma unroll
        for (int t = t0; t < min(t0 + TT, NTILE); ++t)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            stage[(((wave - hw) * TT + (t - t0)) * 8 + v) * 64 + lane] = acc[t].o[v];
      }
      __syncthreads();
      if (wave < hw) {
#pragma unroll
        for (int t = t0; t < min(t0 + TT, NTILE); ++t)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            acc[t].o[v] += stage[((wave * TT + (t - t0)) * 8 + v) * 64 + lane];
      }
      if (hw > 1) __syncthreads();  // the adders have read before the next writers
    }
    if (wave == 0) {
      // lane (n, grp) holds dims 32 grp + 8 i + v of column n in o[v][i]
#pragma unroll
      for (int t = t0; t < min(t0 + TT, NTILE); ++t) {
        const int mi = t * MPT + n / G;
        if (mi >= mem) continue;
        const size_t qrow =
            (size_t)((o * g.group + mi) * g.L + l) * g.Hq + (size_t)h * G + n % G;
        float4* dst = reinterpret_cast<float4*>(out + qrow * D + 32 * grp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4* a = acc[t].o;
          dst[2 * i] = float4{a[0][i], a[1][i], a[2][i], a[3][i]};
          dst[2 * i + 1] = float4{a[4][i], a[5][i], a[6][i], a[7][i]};
        }
      }
    }
  }
}

#define FERRY_ATTN_GROUP_INST_W(DT, G, NTILE, W)                                          \
  template __global__ void k_attn_group<DT, G, NTILE, W>(Geo, const float*, const uint32_t*, \
                                                         const uint8_t*, const float*, float*, \
                                                         float, int, int, int*,              \
                                                         unsigned long long*);
#define FERRY_ATTN_GROUP_INST(DT, G, NTILE)                       \
  FERRY_ATTN_GROUP_INST_W(DT, G, NTILE, group_waves(DT))          \
  FERRY_ATTN_GROUP_INST_W(DT, G, NTILE, kGroupWideWaves)
#define FERRY_ATTN_GROUP_INST_DT(DT) \
  FERRY_ATTN_GROUP_INST(DT, 2, 1)    \
  FERRY_ATTN_GROUP_INST(DT, 2, 2)    \
  FERRY_ATTN_GROUP_INST(DT, 2, 3)    \
  FERRY_ATTN_GROUP_INST(DT, 2, 4)    \
  FERRY_ATTN_GROUP_INST(DT, 4, 1)    \
  FERRY_ATTN_GROUP_INST(DT, 4, 2)    \
  FERRY_ATTN_GROUP_INST(DT, 4, 3)    \
  FERRY_ATTN_GROUP_INST(DT, 4, 4)    \
  FERRY_ATTN_GROUP_INST(DT, 8, 1)    \
  FERRY_ATTN_GROUP_INST(DT, 8, 2)    \
  FERRY_ATTN_GROUP_INST(DT, 8, 3)    \
  FERRY_ATTN_GROUP_INST(DT, 8, 4)
FERRY_ATTN_GROUP_INST_DT(FERRY_F16)
FERRY_ATTN_GROUP_INST_DT(FERRY_BF16)
FERRY_ATTN_GROUP_INST_DT(FERRY_FP8_E4M3)

}  // namespace ferry_amd
