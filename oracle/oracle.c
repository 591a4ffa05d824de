/*
 * oracle.c -- CPU restatement of the per-GPU sparse KV miss-stream executor.
 *
 * TEST INFRASTRUCTURE ONLY (what the GPU is checked against).  Loaded by tests/, by
 * __graft_entry__.smoke() and by the cpu_baseline leg of bench.py; never by
 * the product.  See oracle.h for the map of functions to reference files.
 * Paths in citations are relative to the clearleo126/ferry source tree.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math, so the
 * float and double arithmetic below is plain IEEE and reproducible).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* primitives                                                          */
/* ------------------------------------------------------------------ */

/* splitmix64 finaliser (Vigna) applied to seed + idx * golden gamma: the
 * counter-based hash every synthetic draw in the executor derives from. */
uint64_t ora_mix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + idx * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to inf. */
uint16_t ora_f32_to_f16(float x) {
  uint32_t u = f32_bits(x);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t exp = (u >> 23) & 0xFFu;
  uint32_t man = u & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (man ? 0x200u : 0u);
  int e = (int)exp - 127 + 15;
  if (e >= 31) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    /* subnormal: shift the implicit-one mantissa right, RNE */
    uint32_t m = man | 0x800000u;
    int shift = 14 - e; /* 14..24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return sign | (uint16_t)q;
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* may carry into exp */
  return sign | (uint16_t)q;
}

float ora_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24 */
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7F800000u | (man << 13));
  return bits_f32(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

uint16_t ora_f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
    return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float ora_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* binary32 -> OCP FP8 E4M3 (E4M3FN: bias 7, no infinities, NaN = S.1111.111,
 * max finite 448), round to nearest even, saturating to +-448. */
uint8_t ora_f32_to_e4m3(float x) {
  uint32_t u = f32_bits(x);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;      /* NaN */
  if (bits_f32(a) >= 464.0f) return sign | 0x7Eu; /* saturate to 448 */
  int e = (int)(a >> 23) - 127;
  if (e < -6) {
    /* subnormal grid: multiples of 2^-9 (8 == smallest normal 0x08) */
    float n = rintf(bits_f32(a) * 512.0f);
    return sign | (uint8_t)n;
  }
  uint32_t man = a & 0x7FFFFFu;
  uint32_t q = man >> 20;
  uint32_t rem = man & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
  if (q == 8u) {
    q = 0;
    e++;
  }
  return sign | (uint8_t)(((uint32_t)(e + 7) << 3) | q);
}

float ora_e4m3_to_f32(uint8_t v) {
  int sign = v & 0x80;
  int exp = (v >> 3) & 0xF;
  int man = v & 0x7;
  float r;
  if (exp == 0xF && man == 0x7) return NAN;
  if (exp == 0)
    r = (float)man * (1.0f / 512.0f);
  else
    r = ldexpf(1.0f + (float)man / 8.0f, exp - 7);
  return sign ? -r : r;
}

double ora_decode(int dtype, uint32_t v) {
  switch (dtype) {
    case ORA_F32: return (double)bits_f32(v);
    case ORA_F16: return (double)ora_f16_to_f32((uint16_t)v);
    case ORA_BF16: return (double)ora_bf16_to_f32((uint16_t)v);
    default: return (double)ora_e4m3_to_f32((uint8_t)v);
  }
}

/* ------------------------------------------------------------------ */
/* mt19937_64 (Matsumoto-Nishimura 64-bit MT; C++ [rand.predef]).      */
/* replay_miss_stream seeds std::mt19937_64 (missstream.cuh:106).      */
/* ------------------------------------------------------------------ */
#define MT_N 312
#define MT_M 156
#define MT_UPPER 0xFFFFFFFF80000000ull
#define MT_LOWER 0x7FFFFFFFull

void ora_mt64_seed(ora_mt64* g, uint64_t seed) {
  g->mt[0] = seed;
  for (int i = 1; i < MT_N; ++i)
    g->mt[i] = 6364136223846793005ull * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) +
               (uint64_t)i;
  g->idx = MT_N;
}

uint64_t ora_mt64_next(ora_mt64* g) {
  static const uint64_t mag[2] = {0ull, 0xB5026F5AA96619E9ull};
  if (g->idx >= MT_N) {
    int i;
    uint64_t x;
    for (i = 0; i < MT_N - MT_M; ++i) {
      x = (g->mt[i] & MT_UPPER) | (g->mt[i + 1] & MT_LOWER);
      g->mt[i] = g->mt[i + MT_M] ^ (x >> 1) ^ mag[x & 1ull];
    }
    for (; i < MT_N - 1; ++i) {
      x = (g->mt[i] & MT_UPPER) | (g->mt[i + 1] & MT_LOWER);
      g->mt[i] = g->mt[i + (MT_M - MT_N)] ^ (x >> 1) ^ mag[x & 1ull];
    }
    x = (g->mt[MT_N - 1] & MT_UPPER) | (g->mt[0] & MT_LOWER);
    g->mt[MT_N - 1] = g->mt[MT_M - 1] ^ (x >> 1) ^ mag[x & 1ull];
    g->idx = 0;
  }
  uint64_t y = g->mt[g->idx++];
  y ^= (y >> 29) & 0x5555555555555555ull;
  y ^= (y << 17) & 0x71D67FFFEDA60000ull;
  y ^= (y << 37) & 0xFFF7EEE000000000ull;
  y ^= y >> 43;
  return y;
}

/* ------------------------------------------------------------------ */
/* reference replay: missstream.cuh:104-170                            */
/* ------------------------------------------------------------------ */
int ora_ref_replay(int R, int L, int S, int sel, int hot, uint64_t seed,
                   uint64_t* blocks, uint8_t* miss, uint64_t* counts) {
  if (R <= 0 || L <= 0 || S <= 0 || sel <= 0 || hot <= 0) return -1;
  ora_mt64 rng;
  ora_mt64_seed(&rng, seed);
  const size_t nrl = (size_t)R * L;
  /* per (r, l): deque of cached blocks (array, front = index 0), previous
   * step's selection */
  uint64_t* dq = (uint64_t*)malloc(nrl * (size_t)hot * sizeof(uint64_t));
  int* dq_n = (int*)calloc(nrl, sizeof(int));
  uint64_t* prev = (uint64_t*)malloc(nrl * (size_t)sel * sizeof(uint64_t));
  int* prev_n = (int*)calloc(nrl, sizeof(int));
  uint64_t* cur = (uint64_t*)malloc((size_t)sel * sizeof(uint64_t));
  if (!dq || !dq_n || !prev || !prev_n || !cur) return -2;
  uint64_t selects = 0, misses = 0;
  size_t ev = 0;
  for (int r = 0; r < R; ++r) {
    for (int s = 0; s < S; ++s) {
      const uint64_t hist_blocks = 64 + (uint64_t)s * 8; /* :118 */
      for (int l = 0; l < L; ++l) {
        const size_t rl = (size_t)r * L + l;
        uint64_t* d = dq + rl * (size_t)hot;
        uint64_t* pv = prev + rl * (size_t)sel;
        const int pn = prev_n[rl];
        for (int i = 0; i < sel; ++i) { /* :125-133 */
          uint64_t blk;
          if (pn > 0 && (double)(ora_mt64_next(&rng) % 1000) / 1000.0 < 0.66)
            blk = pv[ora_mt64_next(&rng) % (uint64_t)pn];
          else
            blk = ora_mt64_next(&rng) % hist_blocks;
          cur[i] = blk;
        }
        for (int i = 0; i < sel; ++i) { /* :137-161 */
          const uint64_t blk = cur[i];
          ++selects;
          int pos = -1;
          for (int j = 0; j < dq_n[rl]; ++j)
            if (d[j] == blk) {
              pos = j;
              break;
            }
          const int hit = pos >= 0;
          if (blocks) blocks[ev] = blk;
          if (miss) miss[ev] = (uint8_t)!hit;
          ++ev;
          if (hit) {
            memmove(d + pos, d + pos + 1,
                    (size_t)(dq_n[rl] - pos - 1) * sizeof(uint64_t));
            d[dq_n[rl] - 1] = blk;
          } else {
            ++misses;
            if (dq_n[rl] >= hot) {
              memmove(d, d + 1, (size_t)(dq_n[rl] - 1) * sizeof(uint64_t));
              dq_n[rl]--;
            }
            d[dq_n[rl]++] = blk;
          }
        }
        memcpy(pv, cur, (size_t)sel * sizeof(uint64_t)); /* :162 */
        prev_n[rl] = sel;
      }
    }
  }
  if (counts) {
    counts[0] = selects;
    counts[1] = misses;
  }
  free(dq);
  free(dq_n);
  free(prev);
  free(prev_n);
  free(cur);
  return 0;
}

/* ------------------------------------------------------------------ */
/* reference C-mode refill planner: kv_exec.cuh:188-292               */
/* ------------------------------------------------------------------ */
typedef struct {
  int layer;
  uint64_t block;
} ref_missref;

static int cmp_missref(const void* a, const void* b) {
  const ref_missref* x = (const ref_missref*)a;
  const ref_missref* y = (const ref_missref*)b;
  if (x->layer != y->layer) return x->layer < y->layer ? -1 : 1;
  if (x->block != y->block) return x->block < y->block ? -1 : 1;
  return 0;
}

/* AdaptiveBatchPolicy::choose_mb (adaptive_batch.cuh:31-36) */
static double choose_mb(double pending, double min_mb, double max_mb,
                        double target) {
  double g = pending / target;
  if (g < min_mb) g = min_mb;
  if (g > max_mb) g = max_mb;
  return g;
}

uint64_t ora_ref_cmode_runs(int R, int L, int S, int sel, int hot,
                            uint64_t c4, double min_mb, double max_mb,
                            double target_batches, const uint64_t* blocks,
                            const uint8_t* miss, uint64_t* refill_bytes) {
  const size_t per_step = (size_t)L * sel;
  ref_missref* ml = (ref_missref*)malloc(per_step * sizeof(ref_missref));
  uint64_t events = 0, bytes = 0;
  size_t ev_i = 0;
  for (int r = 0; r < R; ++r) {
    for (int s = 0; s < S; ++s) {
      size_t n = 0;
      for (int l = 0; l < L; ++l) /* :201-207 */
        for (int k = 0; k < sel; ++k) {
          const size_t e = ev_i + (size_t)l * sel + k;
          if (miss[e]) {
            ml[n].layer = l;
            ml[n].block = blocks[e];
            ++n;
          }
        }
      ev_i += per_step;
      qsort(ml, n, sizeof(ref_missref), cmp_missref); /* :211-217 */
      size_t u = 0;                                   /* :218-223 */
      for (size_t i = 0; i < n; ++i)
        if (u == 0 || ml[i].layer != ml[u - 1].layer ||
            ml[i].block != ml[u - 1].block)
          ml[u++] = ml[i];
      n = u;
      size_t i0 = 0;
      while (i0 < n) { /* :229-273 */
        const double pending_mb = (double)(n - i0) * (double)c4 / (1 << 20);
        const double gmb = choose_mb(pending_mb, min_mb, max_mb, target_batches);
        size_t take = (size_t)(gmb * (1 << 20) / (double)c4);
        if (take < 1) take = 1;
        if (take > n - i0) take = n - i0;
        size_t k = 0;
        while (k < take) {
          const ref_missref m0 = ml[i0 + k];
          size_t run = 1;
          while (k + run < take && ml[i0 + k + run].layer == m0.layer &&
                 ml[i0 + k + run].block == m0.block + run)
            ++run;
          bytes += run * c4; /* both branches move run*c4 bytes */
          (void)hot;
          ++events;
          k += run;
        }
        i0 += take;
      }
    }
  }
  free(ml);
  if (refill_bytes) *refill_bytes = bytes;
  return events;
}

/* ------------------------------------------------------------------ */
/* LRU set engine                                                      */
/* ------------------------------------------------------------------ */
#define PEND 0x80000000u

int ora_lru_init(ora_lru* s, int cap, int max_blocks) {
  s->cap = cap;
  s->lim = cap;
  s->max_blocks = max_blocks;
  s->ord = (uint32_t*)malloc((size_t)cap * 4);
  s->tag = (uint32_t*)malloc((size_t)cap * 4);
  s->map = (uint32_t*)malloc((size_t)max_blocks * 4);
  s->own = (uint32_t*)malloc((size_t)cap * 4);
  if (!s->ord || !s->tag || !s->map || !s->own) return -1;
  ora_lru_reset(s);
  return 0;
}

void ora_lru_free(ora_lru* s) {
  free(s->ord);
  free(s->tag);
  free(s->map);
  free(s->own);
  s->ord = s->tag = s->map = s->own = NULL;
}

void ora_lru_reset(ora_lru* s) {
  s->fill = 0;
  for (int i = 0; i < s->cap; ++i) {
    s->ord[i] = ORA_NONE;
    s->tag[i] = ORA_NONE;
    s->own[i] = 0;
  }
  for (int i = 0; i < s->max_blocks; ++i) s->map[i] = ORA_NONE;
}

/* One batched sub-step.  Semantics (the executor's bookkeeping rule):
 *  - hit  = block resident when the sub-step starts;
 *  - miss = first occurrence (canonical order) of a non-resident block; later
 *    occurrences of that block hit the in-flight fetch (dedup);
 *  - the q-th miss takes free slot fill+q while free slots remain, then the
 *    least recently used resident slot NOT touched in this sub-step;
 *  - afterwards the LRU order is: untouched survivors in their old order,
 *    then every touched slot ordered by its last occurrence.
 * With n == 1 this is exactly kv_touch / the replay LRU
 * (wla_multigpu.cuh:1937-1962, missstream.cuh:137-161): a hit moves to the
 * MRU end, a miss evicts the front when full and is appended. */
int ora_lru_substep(ora_lru* s, uint32_t set, const uint32_t* x, int n,
                    uint32_t* slot_out, ora_miss* miss_out, int* n_miss,
                    uint8_t* flag_out) {
  return ora_lru_substep_m(s, set, x, NULL, n, slot_out, miss_out, n_miss, flag_out);
}

int ora_lru_substep_m(ora_lru* s, uint32_t set, const uint32_t* x, const uint8_t* member, int n,
                      uint32_t* slot_out, ora_miss* miss_out, int* n_miss, uint8_t* flag_out) {
  const int cap = s->cap;
  for (int p = 0; p < n; ++p)
    if (x[p] != ORA_NONE && x[p] >= (uint32_t)s->max_blocks) return -1;
  int* lastpos = (int*)malloc((size_t)cap * sizeof(int));
  uint32_t* mblk = (uint32_t*)malloc((size_t)(n ? n : 1) * 4);
  uint32_t* victim = (uint32_t*)malloc((size_t)(n ? n : 1) * 4);
  uint32_t* nord = (uint32_t*)malloc((size_t)cap * 4);
  for (int i = 0; i < cap; ++i) lastpos[i] = -1;
  /* phase 1: classify */
  for (int p = 0; p < n; ++p) {
    if (x[p] == ORA_NONE) continue; /* empty position: touches nothing */
    const uint32_t v = s->map[x[p]];
    if (v == ORA_NONE)
      s->map[x[p]] = PEND | (uint32_t)p;
    else if (!(v & PEND))
      lastpos[v] = p;
  }
  /* phase 2: misses in order of first occurrence */
  int M = 0;
  for (int p = 0; p < n; ++p) {
    const int first = x[p] != ORA_NONE && s->map[x[p]] == (PEND | (uint32_t)p);
    if (flag_out) flag_out[p] = (uint8_t)first;
    if (first) mblk[M++] = x[p];
  }
  /* phase 3: victims; the set may use lim of its cap slots */
  const int freeslots = s->lim > (int)s->fill ? s->lim - (int)s->fill : 0;
  const int need = M > freeslots ? M - freeslots : 0;
  int nv = 0;
  for (uint32_t i = 0; i < s->fill && nv < need; ++i)
    if (lastpos[s->ord[i]] < 0) victim[nv++] = s->ord[i];
  if (nv < need) {
    for (int q = 0; q < M; ++q) s->map[mblk[q]] = ORA_NONE;
    free(lastpos);
    free(mblk);
    free(victim);
    free(nord);
    return -2;
  }
  /* phase 4: assign */
  for (int q = 0; q < M; ++q) {
    const uint32_t v = q < freeslots ? s->fill + (uint32_t)q : victim[q - freeslots];
    uint32_t ev = ORA_NONE;
    if (q >= freeslots) {
      ev = s->tag[v];
      s->map[ev] = ORA_NONE;
    }
    s->tag[v] = mblk[q];
    s->map[mblk[q]] = v;
    s->own[v] = 0; /* a new block: the slot's old members are dropped (own_drop) */
    miss_out[q].block = mblk[q];
    miss_out[q].slot = v;
    miss_out[q].evicted = ev;
    miss_out[q].set = set;
  }
  for (int p = 0; p < n; ++p) {
    if (x[p] == ORA_NONE) {
      slot_out[p] = ORA_NONE;
      continue;
    }
    const uint32_t v = s->map[x[p]];
    slot_out[p] = v;
    lastpos[v] = p;
    if (member) s->own[v] |= 1u << member[p]; /* own_mask |= own_bit(r) */
  }
  /* phase 5: new LRU order */
  uint32_t w = 0;
  for (uint32_t i = 0; i < s->fill; ++i)
    if (lastpos[s->ord[i]] < 0) nord[w++] = s->ord[i];
  for (int p = 0; p < n; ++p)
    if (slot_out[p] != ORA_NONE && lastpos[slot_out[p]] == p) nord[w++] = slot_out[p];
  s->fill += (uint32_t)(M < freeslots ? M : freeslots);
  memcpy(s->ord, nord, (size_t)w * 4);
  free(lastpos);
  free(mblk);
  free(victim);
  free(nord);
  *n_miss = M;
  return w == s->fill ? 0 : -4;
}

int ora_lru_trim(ora_lru* s, int lim, uint32_t* moves) {
  s->lim = lim;
  if ((int)s->fill <= lim) return 0;
  const uint32_t e = s->fill - (uint32_t)lim, f = s->fill;
  uint32_t* pos = (uint32_t*)malloc((size_t)s->cap * 4);
  for (uint32_t i = 0; i < f; ++i) pos[s->ord[i]] = i;
  for (uint32_t i = 0; i < e; ++i) s->map[s->tag[s->ord[i]]] = ORA_NONE;
  uint32_t hole = 0;  /* next candidate hole slot */
  int nm = 0;
  for (uint32_t m = (uint32_t)lim; m < f; ++m) {
    if (pos[m] < e) continue; /* evicted, not a mover */
    while (pos[hole] >= e) ++hole; /* next evicted slot below lim */
    const uint32_t blk = s->tag[m];
    s->tag[hole] = blk;
    s->own[hole] = s->own[m];
    s->map[blk] = hole;
    s->ord[pos[m]] = hole;
    if (moves) {
      moves[2 * nm] = m;
      moves[2 * nm + 1] = hole;
    }
    ++nm;
    ++hole;
  }
  memmove(s->ord, s->ord + e, (size_t)lim * 4);
  for (int i = lim; i < s->cap; ++i) {
    s->ord[i] = ORA_NONE;
    s->tag[i] = ORA_NONE;
    s->own[i] = 0;
  }
  s->fill = (uint32_t)lim;
  free(pos);
  return nm;
}

/* Deque LRU, restating the replay's per-touch loop (missstream.cuh:137-161)
 * over a single (request, layer) stream. */
int ora_deque_lru_run(int cap, const uint32_t* x, int n, uint8_t* miss_flag) {
  uint32_t* d = (uint32_t*)malloc((size_t)cap * 4);
  int dn = 0;
  for (int i = 0; i < n; ++i) {
    int pos = -1;
    for (int j = 0; j < dn; ++j)
      if (d[j] == x[i]) {
        pos = j;
        break;
      }
    miss_flag[i] = pos < 0;
    if (pos >= 0) {
      memmove(d + pos, d + pos + 1, (size_t)(dn - pos - 1) * 4);
      d[dn - 1] = x[i];
    } else {
      if (dn >= cap) {
        memmove(d, d + 1, (size_t)(dn - 1) * 4);
        dn--;
      }
      d[dn++] = x[i];
    }
  }
  free(d);
  return 0;
}

/* kv_touch with a capacity per touch and grp_trim at capacity drops
 * (wla_multigpu.cuh:1923-1962), as a plain deque. */
int ora_deque_lru_run_caps(const int* trim_at, const int* cap_at, const uint32_t* x, int n,
                           uint8_t* miss_flag, uint32_t* final_blocks) {
  int mx = 1;
  for (int i = 0; i < n; ++i)
    if (cap_at[i] > mx) mx = cap_at[i];
  uint32_t* d = (uint32_t*)malloc((size_t)(mx + 1) * 4);
  int dn = 0;
  for (int i = 0; i < n; ++i) {
    const int cap = cap_at[i];
    if (dn > trim_at[i]) { /* grp_trim: drop from the front down to the capacity */
      memmove(d, d + (dn - trim_at[i]), (size_t)trim_at[i] * 4);
      dn = trim_at[i];
    }
    int pos = -1;
    for (int j = 0; j < dn; ++j)
      if (d[j] == x[i]) {
        pos = j;
        break;
      }
    miss_flag[i] = pos < 0;
    if (pos >= 0) {
      memmove(d + pos, d + pos + 1, (size_t)(dn - pos - 1) * 4);
      d[dn - 1] = x[i];
    } else {
      while (dn >= cap) {
        memmove(d, d + 1, (size_t)(dn - 1) * 4);
        dn--;
      }
      d[dn++] = x[i];
    }
  }
  if (final_blocks) memcpy(final_blocks, d, (size_t)dn * 4);
  free(d);
  return dn;
}

/* Timestamp LRU with step-batched semantics, written independently of the
 * order-list engine above (linear scans; small sizes only). */
int ora_tslru_init(ora_tslru* s, int cap, int max_blocks) {
  s->cap = cap;
  s->max_blocks = max_blocks;
  s->tag = (uint32_t*)malloc((size_t)cap * 4);
  s->stamp = (uint64_t*)calloc((size_t)cap, 8);
  s->clock = 0;
  s->fill = 0;
  for (int i = 0; i < cap; ++i) s->tag[i] = ORA_NONE;
  return s->tag && s->stamp ? 0 : -1;
}

void ora_tslru_free(ora_tslru* s) {
  free(s->tag);
  free(s->stamp);
}

int ora_tslru_step(ora_tslru* s, const uint32_t* x, int n, uint32_t* slot_out,
                   uint32_t* miss_blocks, uint32_t* miss_slots, int* n_miss) {
  const int cap = s->cap;
  uint8_t* used = (uint8_t*)calloc((size_t)cap, 1);
  int M = 0;
  /* resident lookup at step start; collect first-occurrence misses */
  for (int p = 0; p < n; ++p) {
    int found = -1;
    for (uint32_t j = 0; j < s->fill; ++j)
      if (s->tag[j] == x[p]) found = (int)j;
    if (found >= 0) {
      used[found] = 1;
      slot_out[p] = (uint32_t)found;
      continue;
    }
    int dup = 0;
    for (int q = 0; q < M; ++q)
      if (miss_blocks[q] == x[p]) dup = 1;
    if (!dup) miss_blocks[M++] = x[p];
    slot_out[p] = ORA_NONE;
  }
  /* assign: free slots ascending, then least stamp among unused residents */
  for (int q = 0; q < M; ++q) {
    uint32_t v;
    if (s->fill < (uint32_t)cap) {
      v = s->fill++;
    } else {
      int best = -1;
      for (int j = 0; j < cap; ++j)
        if (!used[j] && (best < 0 || s->stamp[j] < s->stamp[best])) best = j;
      if (best < 0) {
        free(used);
        return -2;
      }
      v = (uint32_t)best;
    }
    used[v] = 1;
    s->tag[v] = miss_blocks[q];
    miss_slots[q] = v;
  }
  for (int p = 0; p < n; ++p) {
    if (slot_out[p] == ORA_NONE)
      for (int q = 0; q < M; ++q)
        if (miss_blocks[q] == x[p]) slot_out[p] = miss_slots[q];
    s->stamp[slot_out[p]] = s->clock + (uint64_t)p + 1;
  }
  s->clock += (uint64_t)n + 1;
  free(used);
  *n_miss = M;
  return 0;
}

/* ------------------------------------------------------------------ */
/* executor geometry and step                                          */
/* ------------------------------------------------------------------ */
int ora_n_owners(const ora_geom* g) { return (g->n_req + g->group - 1) / g->group; }
int ora_n_sets(const ora_geom* g) { return ora_n_owners(g) * g->n_layers * g->kv_heads; }
int ora_members(const ora_geom* g, int o) {
  const int m = g->n_req - o * g->group;
  return m < g->group ? m : g->group;
}
int ora_max_sel_per_set(const ora_geom* g) { return g->group * g->k; }

static int esize(int dtype) {
  return dtype == ORA_F32 ? 4 : (dtype == ORA_FP8 ? 1 : 2);
}

uint64_t ora_block_bytes(const ora_geom* g) {
  return 2ull * (uint64_t)g->block_tokens * (uint64_t)g->head_dim *
         (uint64_t)esize(g->dtype);
}

/* Host-tier block index of (set, block): the logical host tier holds every
 * (set, block) at set * max_blocks + block; the physical tier aliases it
 * modulo its capacity, as the reference's slab does (wla_multigpu.cuh:
 * 323-332, `block % cap`). */
uint64_t ora_host_index(const ora_geom* g, uint32_t set, uint32_t block) {
  return ((uint64_t)set * (uint64_t)g->max_blocks + block) % g->host_blocks;
}

struct ora_exec {
  ora_geom g;
  ora_lru* sets;
  uint32_t* x;
  uint32_t* slot;
  uint8_t* flag;
  uint32_t* members;  /* [n_owners] resident member lanes */
  uint8_t* live;      /* [n_req] lane resident */
  uint8_t* mem;       /* [max_sel] member index of each position of a set's step */
};

int ora_capacity(const ora_geom* g, int members) {
  if (g->cap_mode != 1) return g->cap;
  const int share = g->cap / g->group;
  const long c = (long)share * (members > 0 ? members : 1);
  return c < g->cap ? (int)c : g->cap;
}

ora_exec* ora_exec_create(const ora_geom* g) {
  ora_exec* e = (ora_exec*)calloc(1, sizeof(ora_exec));
  e->g = *g;
  const int ns = ora_n_sets(g);
  e->sets = (ora_lru*)calloc((size_t)ns, sizeof(ora_lru));
  for (int i = 0; i < ns; ++i)
    if (ora_lru_init(&e->sets[i], g->cap, g->max_blocks)) return NULL;
  e->x = (uint32_t*)malloc((size_t)ora_max_sel_per_set(g) * 4);
  e->slot = (uint32_t*)malloc((size_t)ora_max_sel_per_set(g) * 4);
  e->flag = (uint8_t*)malloc((size_t)ora_max_sel_per_set(g));
  e->members = (uint32_t*)malloc((size_t)ora_n_owners(g) * 4);
  e->live = (uint8_t*)malloc((size_t)g->n_req);
  e->mem = (uint8_t*)malloc((size_t)ora_max_sel_per_set(g));
  for (int p = 0; p < ora_max_sel_per_set(g); ++p) e->mem[p] = (uint8_t)(p / g->k);
  for (int o = 0; o < ora_n_owners(g); ++o) e->members[o] = (uint32_t)ora_members(g, o);
  memset(e->live, 1, (size_t)g->n_req);
  return e;
}

int ora_exec_members(ora_exec* e, const uint32_t* lanes, int n, int delta) {
  const ora_geom* g = &e->g;
  const int nown = ora_n_owners(g), per = g->n_layers * g->kv_heads;
  uint8_t* shrunk = (uint8_t*)calloc((size_t)nown, 1);
  int rc = 0;
  for (int i = 0; i < n; ++i) {
    const uint32_t ln = lanes[i];
    const uint8_t want = delta < 0 ? 1 : 0;
    if (ln >= (uint32_t)g->n_req || e->live[ln] != want) {
      rc = -1;
      continue;
    }
    e->live[ln] = (uint8_t)(1 - want);
    const uint32_t o = ln / (uint32_t)g->group;
    if (delta < 0) {
      e->members[o]--;
      shrunk[o] = 1;
    } else {
      e->members[o]++;
    }
  }
  for (int o = 0; o < nown; ++o) {
    if (!shrunk[o]) continue;
    /* own_release: the members that left drop out of every mask of the owner */
    uint32_t live = 0;
    for (int m = 0; m < g->group && o * g->group + m < g->n_req; ++m)
      if (e->live[o * g->group + m]) live |= 1u << m;
    for (int i = 0; i < per; ++i) {
      ora_lru* s = &e->sets[o * per + i];
      for (uint32_t v = 0; v < s->fill; ++v) s->own[v] &= live;
      if (g->cap_mode == 1) ora_lru_trim(s, ora_capacity(g, (int)e->members[o]), NULL);
    }
  }
  free(shrunk);
  return rc;
}

void ora_exec_own(const ora_exec* e, uint32_t* own) {
  const int ns = ora_n_sets(&e->g), cap = e->g.cap;
  for (int i = 0; i < ns; ++i) memcpy(own + (size_t)i * cap, e->sets[i].own, (size_t)cap * 4);
}

int ora_exec_export_member(const ora_exec* e, int lane, uint32_t* counts, uint32_t* blocks) {
  const ora_geom* g = &e->g;
  if (lane < 0 || lane >= g->n_req) return -1;
  const int o = lane / g->group, per = g->n_layers * g->kv_heads;
  const uint32_t bit = 1u << (uint32_t)(lane % g->group);
  for (int i = 0; i < per; ++i) {
    const ora_lru* s = &e->sets[o * per + i];
    uint32_t c = 0;
    for (uint32_t j = 0; j < s->fill; ++j) {
      const uint32_t v = s->ord[j];
      if (s->own[v] == bit) blocks[(size_t)i * g->cap + c++] = s->tag[v];
    }
    counts[i] = c;
  }
  return 0;
}

int ora_exec_import_member(ora_exec* e, int lane, const uint32_t* counts, const uint32_t* blocks) {
  const ora_geom* g = &e->g;
  if (lane < 0 || lane >= g->n_req) return -1;
  const int o = lane / g->group, per = g->n_layers * g->kv_heads;
  const uint32_t bit = 1u << (uint32_t)(lane % g->group);
  const uint32_t lim = (uint32_t)ora_capacity(g, (int)e->members[o]);
  for (int i = 0; i < per; ++i) {
    ora_lru* s = &e->sets[o * per + i];
    if (counts[i] > (uint32_t)g->cap || s->fill > lim) return -1;
    for (uint32_t j = 0; j < counts[i]; ++j) {
      const uint32_t x = blocks[(size_t)i * g->cap + j];
      if (x >= (uint32_t)g->max_blocks) return -1;
      if (s->map[x] != ORA_NONE) { /* already here: only the member bit */
        s->own[s->map[x]] |= bit;
        continue;
      }
      uint32_t v = s->fill;
      if (s->fill >= lim) { /* evict the least recent; the new block takes its slot */
        v = s->ord[0];
        s->map[s->tag[v]] = ORA_NONE;
        memmove(s->ord, s->ord + 1, (size_t)(s->fill - 1) * 4);
        s->fill--;
      }
      s->tag[v] = x;
      s->map[x] = v;
      s->own[v] = bit;
      s->ord[s->fill++] = v;
    }
  }
  return 0;
}

void ora_exec_members_get(const ora_exec* e, uint32_t* members) {
  memcpy(members, e->members, (size_t)ora_n_owners(&e->g) * 4);
}

const ora_geom* ora_exec_geom(const ora_exec* e) { return &e->g; }

void ora_exec_destroy(ora_exec* e) {
  if (!e) return;
  const int ns = ora_n_sets(&e->g);
  for (int i = 0; i < ns; ++i) ora_lru_free(&e->sets[i]);
  free(e->sets);
  free(e->x);
  free(e->slot);
  free(e->flag);
  free(e->members);
  free(e->live);
  free(e->mem);
  free(e);
}

int ora_exec_step(ora_exec* e, const uint32_t* sel, uint32_t* slots_out,
                  uint32_t* miss_count, ora_miss* misses, uint64_t* counts,
                  uint8_t* flags) {
  const ora_geom* g = &e->g;
  const int L = g->n_layers, H = g->kv_heads, k = g->k;
  const int nown = ora_n_owners(g), maxsel = ora_max_sel_per_set(g);
  uint64_t nsel = 0, nmiss = 0;
  for (int o = 0; o < nown; ++o)
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < H; ++h) {
        const uint32_t set = (uint32_t)((o * L + l) * H + h);
        const int mem = ora_members(g, o);
        const int n = mem * k;
        for (int m = 0; m < mem; ++m) {
          const int r = o * g->group + m;
          memcpy(e->x + (size_t)m * k, sel + ((size_t)(r * L + l) * H + h) * k,
                 (size_t)k * 4);
        }
        ora_miss* mo = misses + (size_t)set * maxsel;
        int M = 0;
        e->sets[set].lim = ora_capacity(g, (int)e->members[o]);
        const uint8_t* who = g->group > 1 ? e->mem : NULL; /* member masks for groups */
        if (g->granularity == 0) {
          const int rc = ora_lru_substep_m(&e->sets[set], set, e->x, who, n, e->slot, mo, &M, e->flag);
          if (rc) return rc;
        } else {
          for (int p = 0; p < n; ++p) {
            int m1 = 0;
            const int rc = ora_lru_substep_m(&e->sets[set], set, e->x + p, who ? who + p : NULL, 1,
                                             e->slot + p, mo + M, &m1, e->flag + p);
            if (rc) return rc;
            M += m1;
          }
          /* every selected block must still be resident at step end */
          for (int p = 0; p < n; ++p)
            if (e->x[p] != ORA_NONE && e->sets[set].tag[e->slot[p]] != e->x[p]) return -3;
        }
        miss_count[set] = (uint32_t)M;
        for (int p = 0; p < n; ++p) nsel += e->x[p] != ORA_NONE;
        nmiss += (uint64_t)M;
        for (int m = 0; m < mem; ++m) {
          const int r = o * g->group + m;
          uint32_t* so = slots_out + ((size_t)(r * L + l) * H + h) * k;
          for (int j = 0; j < k; ++j)
            so[j] = e->slot[m * k + j] == ORA_NONE ? ORA_NONE
                                                    : set * (uint32_t)g->cap + e->slot[m * k + j];
          if (flags)
            memcpy(flags + ((size_t)(r * L + l) * H + h) * k, e->flag + (size_t)m * k,
                   (size_t)k);
        }
      }
  if (counts) {
    counts[0] = nsel;
    counts[1] = nmiss;
    counts[2] = nsel - nmiss;
  }
  return 0;
}

int ora_exec_reset_owner(ora_exec* e, int owner) {
  const ora_geom* g = &e->g;
  if (owner < 0 || owner >= ora_n_owners(g)) return -1;
  const int per = g->n_layers * g->kv_heads;
  for (int i = 0; i < per; ++i) ora_lru_reset(&e->sets[owner * per + i]);
  return 0;
}

/* A request moved with its cache (kv_handoff with carry,
 * src/runtime/wla_multigpu.cuh:1970-1994): the sets of owner `dst_owner` of
 * `dst` become copies of the sets of `src_owner` of `src` (same geometry). */
int ora_exec_copy_owner(const ora_exec* src, int src_owner, ora_exec* dst, int dst_owner) {
  const ora_geom *a = &src->g, *b = &dst->g;
  if (a->cap != b->cap || a->max_blocks != b->max_blocks || a->n_layers != b->n_layers ||
      a->kv_heads != b->kv_heads || src_owner < 0 || src_owner >= ora_n_owners(a) ||
      dst_owner < 0 || dst_owner >= ora_n_owners(b))
    return -1;
  const int per = a->n_layers * a->kv_heads;
  for (int i = 0; i < per; ++i) {
    const ora_lru* s = &src->sets[src_owner * per + i];
    ora_lru* d = &dst->sets[dst_owner * per + i];
    d->fill = s->fill;
    memcpy(d->ord, s->ord, (size_t)s->cap * 4);
    memcpy(d->tag, s->tag, (size_t)s->cap * 4);
    memcpy(d->own, s->own, (size_t)s->cap * 4);
    memcpy(d->map, s->map, (size_t)s->max_blocks * 4);
  }
  return 0;
}

void ora_exec_state(const ora_exec* e, uint32_t* fill, uint32_t* ord,
                    uint32_t* tag) {
  const int ns = ora_n_sets(&e->g), cap = e->g.cap;
  for (int i = 0; i < ns; ++i) {
    fill[i] = e->sets[i].fill;
    memcpy(ord + (size_t)i * cap, e->sets[i].ord, (size_t)cap * 4);
    memcpy(tag + (size_t)i * cap, e->sets[i].tag, (size_t)cap * 4);
  }
}

/* ------------------------------------------------------------------ */
/* workload generators                                                 */
/* ------------------------------------------------------------------ */
#define SALT_CTX 0x43545842ull  /* context lengths */
#define SALT_SEL 0x53454C31ull  /* selection draws */
#define SALT_PERM 0x5045524Dull /* popularity permutation offsets */
#define SALT_HOST 0x484F5354ull /* host tier values */
#define SALT_SCALE 0x5343414Cull /* fp8 block scales */
#define SALT_KEEP 0x4B454550ull  /* inter-step reuse draws */
#define PERM_PRIME 1000003ull
#define DRAW_LIMIT 65536

void ora_ctx_uniform(uint64_t seed, int n_req, int lo, int hi, int* out) {
  const uint64_t span = (uint64_t)(hi - lo + 1);
  for (int r = 0; r < n_req; ++r)
    out[r] = lo + (int)(ora_mix64(seed ^ SALT_CTX, (uint64_t)r) % span);
}

/* permutation domain of an owner: its largest member context */
static int owner_nperm(const ora_selgen* s, int o) {
  int m = 0;
  for (int r = o * s->group; r < (o + 1) * s->group && r < s->n_req; ++r)
    if (s->ctx_blocks[r] > m) m = s->ctx_blocks[r];
  return m;
}

int ora_selgen_max_blocks(const ora_selgen* s) {
  const int nown = (s->n_req + s->group - 1) / s->group;
  const int ranges = s->private_ranges > s->group ? s->private_ranges : s->group;
  int mx = 0;
  for (int o = 0; o < nown; ++o) {
    const int np = s->nperm ? s->nperm[o] : owner_nperm(s, o);
    const int pre = s->prefix_blocks < np ? s->prefix_blocks : np;
    const int b = pre + ranges * (np - pre);
    if (b > mx) mx = b;
  }
  return mx;
}

static int cmp_u32(const void* a, const void* b) {
  const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? -1 : (x > y);
}

/* Selections of one step.  For every (request r, layer l, kv head h):
 *  - step 0 (or reuse == 0): nothing is carried over;
 *  - later steps: each block of r's previous selection is kept with
 *    probability `reuse` (inter-step reuse, the locality knob of the
 *    reference generator, missstream.cuh:127-128);
 *  - the selection is completed to k distinct blocks by drawing popularity
 *    ranks from Zipf(s) (or uniform) over the owner's permutation domain,
 *    mapping rank -> block through the owner's affine permutation
 *    (rank*P + off) mod n, and rejecting blocks outside r's context or
 *    already taken;
 *  - the k blocks are sorted ascending (top-k page indices are sorted,
 *    tools/capture_miss_trace.py:158-159); `state` keeps them (logical ids)
 *    for the next step, `out` names them in the set's id space (shared prefix
 *    ids first, then each member's private range). */
int ora_selgen_step(const ora_selgen* s, int step, uint32_t* state,
                    uint32_t* out) {
  const int L = s->n_layers, H = s->kv_heads, k = s->k;
  int nmax = 0; /* the largest permutation domain (Zipf weights and draw marks) */
  for (int r = 0; r < s->n_req; ++r)
    if (s->ctx_blocks[r] > nmax) nmax = s->ctx_blocks[r];
  if (s->nperm)
    for (int o = 0; o < (s->n_req + s->group - 1) / s->group; ++o)
      if (s->nperm[o] > nmax) nmax = s->nperm[o];
  double* cum = NULL;
  if (s->dist == 1) {
    cum = (double*)malloc((size_t)nmax * sizeof(double));
    double acc = 0.0;
    for (int i = 0; i < nmax; ++i) {
      acc += pow((double)(i + 1), -s->zipf_s);
      cum[i] = acc;
    }
  }
  uint8_t* taken = (uint8_t*)calloc((size_t)nmax, 1);
  for (int r = 0; r < s->n_req; ++r) {
    const size_t rows = (size_t)L * H * k;
    if (s->active && !s->active[r]) { /* idle lane: every position empty */
      for (size_t i = 0; i < rows; ++i) out[(size_t)r * rows + i] = ORA_NONE;
      continue;
    }
    const int o = r / s->group;
    const int m = s->prange ? s->prange[r] : r % s->group; /* private id range */
    const int nr = s->ctx_blocks[r];
    const int np = s->nperm ? s->nperm[o] : owner_nperm(s, o);
    const int pre = s->prefix_blocks < np ? s->prefix_blocks : np;
    const double reuse = s->reuse_r ? s->reuse_r[r] : s->reuse;
    const uint64_t keep_thr = (uint64_t)(reuse * 4294967296.0);
    /* the request in lane r: its id and the step it was admitted at */
    const uint64_t rid = s->rid ? (uint64_t)s->rid[r] : (uint64_t)r;
    const int start = s->start ? s->start[r] : 0;
    if (step < start || nr < 1) {
      free(cum);
      free(taken);
      return -1;
    }
    const uint64_t lstep = (uint64_t)(step - start);
    const int carry = lstep > 0;
    const int ke = k < nr ? k : nr; /* a short context selects all its blocks */
    const uint64_t pown = s->group == 1 ? rid : (uint64_t)o;
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < H; ++h) {
        const size_t row = ((size_t)(r * L + l) * H + h) * k;
        uint32_t* st = state + row;
        uint32_t* so = out + row;
        const uint64_t off =
            ora_mix64(s->seed ^ SALT_PERM, (pown * (uint64_t)L + (uint64_t)l) * (uint64_t)H +
                                               (uint64_t)h) %
            (uint64_t)np;
        const uint64_t base =
            ((((lstep << 16) | rid) * (uint64_t)L + (uint64_t)l) * (uint64_t)H + (uint64_t)h) *
            (uint64_t)DRAW_LIMIT;
        int got = 0;
        if (carry && reuse > 0.0)
          for (int j = 0; j < k; ++j) {
            if (st[j] == ORA_NONE) continue;
            const uint64_t u = ora_mix64(s->seed ^ SALT_KEEP, base + (uint64_t)j) >> 32;
            if (u < keep_thr) {
              so[got++] = st[j];
              taken[st[j]] = 1;
            }
          }
        for (int i = 0; i < DRAW_LIMIT && got < ke; ++i) {
          const uint64_t u = ora_mix64(s->seed ^ SALT_SEL, base + (uint64_t)i);
          uint64_t rank;
          if (s->dist == 1) {
            const double thr = (double)(u >> 11) * (1.0 / 9007199254740992.0) *
                               cum[np - 1];
            int lo = 0, hi = np - 1; /* first i with cum[i] > thr */
            while (lo < hi) {
              const int mid = (lo + hi) >> 1;
              if (cum[mid] > thr)
                hi = mid;
              else
                lo = mid + 1;
            }
            rank = (uint64_t)lo;
          } else {
            rank = ((u >> 32) * (uint64_t)np) >> 32;
          }
          const uint64_t b = (rank * PERM_PRIME + off) % (uint64_t)np;
          if (b >= (uint64_t)nr || taken[b]) continue;
          taken[b] = 1;
          so[got++] = (uint32_t)b;
        }
        for (int j = 0; j < got; ++j) taken[so[j]] = 0;
        if (got < ke) {
          free(cum);
          free(taken);
          return -2;
        }
        qsort(so, (size_t)ke, 4, cmp_u32);
        for (int j = ke; j < k; ++j) so[j] = ORA_NONE;
        memcpy(st, so, (size_t)k * 4);
        for (int j = 0; j < ke; ++j)
          if (so[j] >= (uint32_t)pre)
            so[j] = (uint32_t)pre + (uint32_t)m * (uint32_t)(np - pre) +
                    (so[j] - (uint32_t)pre);
      }
  }
  free(cum);
  free(taken);
  return 0;
}

/* ------------------------------------------------------------------ */
/* request arrivals                                                    */
/* ------------------------------------------------------------------ */
#define SALT_ARRIVE 0x41525256ull
#define SALT_SOJOURN 0x534F4A4Eull

static double unit_open0(uint64_t seed, uint64_t salt, uint64_t i) {
  /* 53 random bits + 1 over 2^53: uniform on (0, 1] */
  return (double)((ora_mix64(seed ^ salt, i) >> 11) + 1) / 9007199254740992.0;
}

/* Arrival times (ms).  Steady and bursty follow the reference's dispatcher
 * (src/runtime/wla_multigpu.cuh:497-501: t += gap, or t += 40 gap every 16th
 * request and 0.1 gap otherwise).  Poisson draws exponential gaps by
 * inversion.  The Markov-modulated process alternates a slow state (mean gap
 * `gap`) and a fast one (gap / ratio); state lifetimes are exponential of
 * mean `period`; a gap that would cross the state's end is dropped and
 * redrawn from the end at the new rate, which is exact by memorylessness. */
int ora_arrivals(int kind, uint32_t n, double gap, double period, double ratio,
                 uint64_t seed, double* out) {
  if (!(gap > 0.0)) return -1;
  double t = 0.0;
  if (kind == 0) {
    for (uint32_t r = 0; r < n; ++r) {
      t += gap;
      out[r] = t;
    }
  } else if (kind == 1) {
    for (uint32_t r = 0; r < n; ++r) {
      t += (r % 16 == 0) ? 40.0 * gap : 0.1 * gap;
      out[r] = t;
    }
  } else if (kind == 2) {
    for (uint32_t r = 0; r < n; ++r) {
      t += -gap * log(unit_open0(seed, SALT_ARRIVE, r));
      out[r] = t;
    }
  } else if (kind == 3) {
    if (!(period > 0.0) || !(ratio > 0.0)) return -1;
    uint64_t ia = 0, is = 0;
    int fast = 0;
    double state_end = -period * log(unit_open0(seed, SALT_SOJOURN, is++));
    for (uint32_t r = 0; r < n; ++r) {
      for (;;) {
        const double mean = fast ? gap / ratio : gap;
        const double d = -mean * log(unit_open0(seed, SALT_ARRIVE, ia++));
        if (t + d < state_end) {
          t += d;
          break;
        }
        t = state_end;
        fast = !fast;
        state_end = t - period * log(unit_open0(seed, SALT_SOJOURN, is++));
      }
      out[r] = t;
    }
  } else {
    return -1;
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* top-k block selection (Quest bound)                                 */
/* ------------------------------------------------------------------ */
/* K min/max of host block h per dim over its tokens (the page summary of
 * tools/capture_miss_trace.py:140-143), as decoded floats; of equal values
 * the first in token order is kept. */
void ora_summary(const ora_geom* g, uint64_t h, float* kmin, float* kmax) {
  const int D = g->head_dim, T = g->block_tokens;
  for (int d = 0; d < D; ++d) {
    float mn = (float)ora_decode(g->dtype, ora_host_elem(g, h, (uint32_t)d)), mx = mn;
    for (int t = 1; t < T; ++t) {
      const float f = (float)ora_decode(g->dtype, ora_host_elem(g, h, (uint32_t)(t * D + d)));
      if (f < mn) mn = f;
      if (f > mx) mx = f;
    }
    kmin[d] = mn;
    kmax[d] = mx;
  }
}

static float max_det(float a, float b) { return a > b ? a : b; }

/* The bound sum_d max(q_d kmax_d, q_d kmin_d) (capture_miss_trace.py:145),
 * written q_d * (q_d >= 0 ? kmax_d : kmin_d) since kmax >= kmin, in fp32 and in
 * one fixed order: 16 partial sums of 8 consecutive dims each, accumulated
 * left to right with correctly rounded fma from 0, then pairs (i, i^8),
 * (i, i^4), (i, i^2), (i, i^1). */
static float quest_bound(const float* q, const float* kmin, const float* kmax) {
  float s[16];
  for (int p = 0; p < 16; ++p) {
    float acc = 0.0f;
    for (int e = 0; e < 8; ++e) {
      const int d = 8 * p + e;
      acc = fmaf(q[d], q[d] >= 0.0f ? kmax[d] : kmin[d], acc);
    }
    s[p] = acc;
  }
  for (int w = 8; w >= 1; w >>= 1) {
    float t[16];
    for (int i = 0; i < 16; ++i) t[i] = s[i] + s[i ^ w];
    memcpy(s, t, sizeof s);
  }
  return s[0];
}

/* Score of block b for kv head h of (request r, layer l): the max of the
 * bound over the kv head's query heads (capture_miss_trace.py:146), times the
 * block's K scale for fp8. */
static float head_score(const ora_geom* g, const float* q, int r, int l, int h, uint32_t b,
                        float* kmin, float* kmax) {
  const int L = g->n_layers, Hk = g->kv_heads, Hq = g->q_heads, D = g->head_dim;
  const int G = Hq / Hk;
  const uint32_t set = (uint32_t)((r * L + l) * Hk + h);
  const uint64_t hb = ora_host_index(g, set, b);
  ora_summary(g, hb, kmin, kmax);
  float sc = 0.0f;
  for (int gq = 0; gq < G; ++gq) {
    const float* qv = q + ((size_t)(r * L + l) * Hq + (size_t)(h * G + gq)) * D;
    const float bd = quest_bound(qv, kmin, kmax);
    sc = gq == 0 ? bd : max_det(bd, sc);
  }
  if (g->dtype == ORA_FP8) sc = sc * ora_host_scale(g, hb, 0);
  return sc;
}

int ora_quest_scores(const ora_geom* g, const float* q, const int* ctx_blocks, int mode,
                     int stride, float* out) {
  const int L = g->n_layers, Hk = g->kv_heads, D = g->head_dim;
  float* kmin = (float*)malloc((size_t)D * sizeof(float));
  float* kmax = (float*)malloc((size_t)D * sizeof(float));
  size_t row = 0;
  for (int r = 0; r < g->n_req; ++r)
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < (mode ? 1 : Hk); ++h, ++row) {
        const int n = ctx_blocks[r] < stride ? ctx_blocks[r] : stride;
        for (int b = 0; b < n; ++b) {
          float sc;
          if (mode) { /* the layer's max over every head (capture_miss_trace.py:147) */
            sc = head_score(g, q, r, l, 0, (uint32_t)b, kmin, kmax);
            for (int hh = 1; hh < Hk; ++hh)
              sc = max_det(head_score(g, q, r, l, hh, (uint32_t)b, kmin, kmax), sc);
          } else {
            sc = head_score(g, q, r, l, h, (uint32_t)b, kmin, kmax);
          }
          out[row * (size_t)stride + b] = sc;
        }
      }
  free(kmin);
  free(kmax);
  return 0;
}

/* order-preserving key of a float's bits (-0 below +0) */
static uint32_t fkey(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

typedef struct {
  uint32_t key, id;
} keyed;

static int cmp_keyed(const void* a, const void* b) {
  const keyed *x = (const keyed*)a, *y = (const keyed*)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1; /* higher score first */
  return x->id < y->id ? -1 : (x->id > y->id); /* then the lower block id */
}

int ora_mass_scores(const ora_geom* g, const float* q, const int* ctx_blocks, int stride,
                    double* out) {
  const int L = g->n_layers, Hk = g->kv_heads, G = g->q_heads / g->kv_heads;
  const int D = g->head_dim, T = g->block_tokens;
  int nmax = 0;
  for (int r = 0; r < g->n_req; ++r) {
    if (ctx_blocks[r] > g->max_blocks) return -1;
    if (ctx_blocks[r] > nmax) nmax = ctx_blocks[r];
  }
  const double scaling = 1.0 / sqrt((double)D);
  double* logit = (double*)malloc((size_t)(nmax > 0 ? nmax : 1) * T * sizeof(double));
  for (int r = 0; r < g->n_req; ++r)
    for (int l = 0; l < L; ++l) {
      const int n = ctx_blocks[r] > 0 ? (ctx_blocks[r] < stride ? ctx_blocks[r] : stride) : 0;
      double* sc = out + (size_t)(r * L + l) * stride;
      for (int b = 0; b < n; ++b) sc[b] = 0.0;
      for (int h = 0; h < Hk; ++h) {
        const uint32_t set = (uint32_t)((r * L + l) * Hk + h);
        for (int gq = 0; gq < G; ++gq) {
          const float* qv = q + (((size_t)(r * L + l) * g->q_heads) + (size_t)(h * G + gq)) * D;
          double mx = -INFINITY;
          for (int b = 0; b < n; ++b) {
            const uint64_t hb = ora_host_index(g, set, (uint32_t)b);
            const double ks = (double)ora_host_scale(g, hb, 0);
            for (int t = 0; t < T; ++t) {
              double dot = 0.0;
              for (int d = 0; d < D; ++d)
                dot += (double)qv[d] * ora_decode(g->dtype, ora_host_elem(g, hb, (uint32_t)(t * D + d)));
              const double x = dot * ks * scaling;
              logit[(size_t)b * T + t] = x;
              if (x > mx) mx = x;
            }
          }
          double z = 0.0;
          for (size_t i = 0; i < (size_t)n * T; ++i) z += exp(logit[i] - mx);
          for (int b = 0; b < n; ++b) {
            double m = 0.0;
            for (int t = 0; t < T; ++t) m += exp(logit[(size_t)b * T + t] - mx);
            sc[b] += m / z;
          }
        }
      }
    }
  free(logit);
  return 0;
}

typedef struct {
  double score;
  uint32_t id;
} dkeyed;

static int cmp_dkeyed(const void* a, const void* b) {
  const dkeyed *x = (const dkeyed*)a, *y = (const dkeyed*)b;
  if (x->score != y->score) return x->score > y->score ? -1 : 1; /* more mass first */
  return x->id < y->id ? -1 : (x->id > y->id);                   /* then the lower id */
}

int ora_select_mass(const ora_geom* g, const float* q, const int* ctx_blocks, uint32_t* sel) {
  const int L = g->n_layers, Hk = g->kv_heads, k = g->k;
  int nmax = 1;
  for (int r = 0; r < g->n_req; ++r) {
    if (ctx_blocks[r] > g->max_blocks) return -1;
    if (ctx_blocks[r] > nmax) nmax = ctx_blocks[r];
  }
  double* sc = (double*)malloc((size_t)g->n_req * L * nmax * sizeof(double));
  dkeyed* kv = (dkeyed*)malloc((size_t)nmax * sizeof(dkeyed));
  uint32_t* pick = (uint32_t*)malloc((size_t)nmax * 4);
  ora_mass_scores(g, q, ctx_blocks, nmax, sc);
  for (int r = 0; r < g->n_req; ++r)
    for (int l = 0; l < L; ++l) {
      const int n = ctx_blocks[r] > 0 ? ctx_blocks[r] : 0;
      const int kk = n < k ? n : k;
      for (int b = 0; b < n; ++b) {
        kv[b].score = sc[(size_t)(r * L + l) * nmax + b];
        kv[b].id = (uint32_t)b;
      }
      qsort(kv, (size_t)n, sizeof(dkeyed), cmp_dkeyed);
      for (int j = 0; j < kk; ++j) pick[j] = kv[j].id;
      qsort(pick, (size_t)kk, 4, cmp_u32);
      for (int hh = 0; hh < Hk; ++hh) {
        uint32_t* o = sel + ((size_t)(r * L + l) * Hk + hh) * k;
        for (int j = 0; j < k; ++j) o[j] = j < kk ? pick[j] : ORA_NONE;
      }
    }
  free(sc);
  free(kv);
  free(pick);
  return 0;
}

/* Top-k blocks of every (request, layer, kv head) row: the min(k, n) highest
 * scores (capture_miss_trace.py:157-158: topk(score, min(sel, n_pages))),
 * written in ascending block order (:158 .sort()), padded with ORA_NONE.
 * mode 1 writes one selection per (request, layer) to every kv head's row. */
int ora_select_topk(const ora_geom* g, const float* q, const int* ctx_blocks, int mode,
                    uint32_t* sel) {
  const int L = g->n_layers, Hk = g->kv_heads, k = g->k;
  int nmax = 1;
  for (int r = 0; r < g->n_req; ++r) {
    if (ctx_blocks[r] > g->max_blocks) return -1;
    if (ctx_blocks[r] > nmax) nmax = ctx_blocks[r];
  }
  const size_t rows = (size_t)g->n_req * L * (mode ? 1 : Hk);
  float* sc = (float*)malloc(rows * (size_t)nmax * sizeof(float));
  keyed* kv = (keyed*)malloc((size_t)nmax * sizeof(keyed));
  uint32_t* pick = (uint32_t*)malloc((size_t)nmax * 4);
  ora_quest_scores(g, q, ctx_blocks, mode, nmax, sc);
  size_t row = 0;
  for (int r = 0; r < g->n_req; ++r)
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < (mode ? 1 : Hk); ++h, ++row) {
        const int n = ctx_blocks[r] > 0 ? ctx_blocks[r] : 0;
        const int kk = n < k ? n : k;
        for (int b = 0; b < n; ++b) {
          kv[b].key = fkey(sc[row * (size_t)nmax + b]);
          kv[b].id = (uint32_t)b;
        }
        qsort(kv, (size_t)n, sizeof(keyed), cmp_keyed);
        for (int j = 0; j < kk; ++j) pick[j] = kv[j].id;
        qsort(pick, (size_t)kk, 4, cmp_u32);
        for (int hh = 0; hh < Hk; ++hh) {
          if (!mode && hh != h) continue;
          uint32_t* o = sel + ((size_t)(r * L + l) * Hk + hh) * k;
          for (int j = 0; j < k; ++j) o[j] = j < kk ? pick[j] : ORA_NONE;
        }
      }
  free(sc);
  free(kv);
  free(pick);
  return 0;
}

/* ------------------------------------------------------------------ */
/* host tier content                                                   */
/* ------------------------------------------------------------------ */
/* Values are Irwin-Hall(4) sums of 16-bit uniforms from the hash, centred
 * and scaled by a float multiplier (std / (65536/sqrt(3))), i.e. zero mean and
 * the requested standard deviation; fp8 blocks store codes of std 96 and a
 * per-block float scale so that code*scale has the requested std. */
static float value_mult(float std) {
  return (float)((double)std / (65536.0 / sqrt(3.0)));
}

static int32_t irwin_hall(uint64_t w) {
  return (int32_t)(w & 0xFFFFu) + (int32_t)((w >> 16) & 0xFFFFu) +
         (int32_t)((w >> 32) & 0xFFFFu) + (int32_t)(w >> 48) - 131070;
}

uint32_t ora_host_elem(const ora_geom* g, uint64_t h, uint32_t e) {
  const uint64_t E = 2ull * (uint64_t)g->block_tokens * (uint64_t)g->head_dim;
  const int32_t sv = irwin_hall(ora_mix64(g->seed ^ SALT_HOST, h * E + e));
  if (g->dtype == ORA_FP8) {
    const float c = (float)sv * value_mult(96.0f);
    return ora_f32_to_e4m3(c);
  }
  const float x = (float)sv * value_mult(g->value_std);
  switch (g->dtype) {
    case ORA_F32: return f32_bits(x);
    case ORA_F16: return ora_f32_to_f16(x);
    default: return ora_f32_to_bf16(x);
  }
}

float ora_host_scale(const ora_geom* g, uint64_t h, int kv) {
  if (g->dtype != ORA_FP8) return 1.0f;
  const float base = (float)((double)g->value_std / 96.0);
  const uint64_t u = ora_mix64(g->seed ^ SALT_SCALE, h * 2ull + (uint64_t)kv) >> 56;
  return base * (0.75f + (float)u / 512.0f);
}

void ora_host_block(const ora_geom* g, uint64_t h, void* bytes, float* scales) {
  const uint32_t E = 2u * (uint32_t)g->block_tokens * (uint32_t)g->head_dim;
  const int es = esize(g->dtype);
  uint8_t* b = (uint8_t*)bytes;
  for (uint32_t e = 0; e < E; ++e) {
    const uint32_t v = ora_host_elem(g, h, e);
    memcpy(b + (size_t)e * es, &v, (size_t)es); /* little endian */
  }
  if (scales) {
    scales[0] = ora_host_scale(g, h, 0);
    scales[1] = ora_host_scale(g, h, 1);
  }
}

void ora_host_fill(const ora_geom* g, uint8_t* host, float* host_scales) {
  const uint64_t bb = ora_block_bytes(g);
  for (uint64_t h = 0; h < g->host_blocks; ++h)
    ora_host_block(g, h, host + h * bb, host_scales ? host_scales + 2 * h : NULL);
}

/* ------------------------------------------------------------------ */
/* attention                                                           */
/* ------------------------------------------------------------------ */
/* Textbook decode attention over the selected blocks: s_t = q.K_t/sqrt(D),
 * p = softmax(s) over every token of every selected block, out = sum p_t V_t
 * (the semantics the reference's FMA proxy stands in for,
 * src/workloads/kv_exec.cuh:30-37; selection as in
 * tools/capture_miss_trace.py:146-159).  Rows name their blocks by host-tier
 * index: hidx [B][L][Hkv][k], ORA_NONE64 for an empty position (skipped); a
 * block named twice in a row is attended twice. */
static float load_elem_f32(int dtype, const uint8_t* p, size_t i);

/* Element e of host block hi, decoded: from the caller's tier image `host`
 * when given, else from the generator (the two agree where the image is
 * ora_host_fill's). */
static double tier_elem(const ora_geom* g, const uint8_t* host, uint64_t hi, uint32_t e) {
  if (!host) return ora_decode(g->dtype, ora_host_elem(g, hi, e));
  return (double)load_elem_f32(g->dtype, host + hi * ora_block_bytes(g), e);
}

static double tier_scale(const ora_geom* g, const float* host_scales, uint64_t hi, int kv) {
  if (g->dtype != ORA_FP8) return 1.0;
  return host_scales ? (double)host_scales[2 * hi + (uint64_t)kv] : (double)ora_host_scale(g, hi, kv);
}

static int attention_rows_f64(const ora_geom* g, const uint64_t* hidx, const uint8_t* host,
                              const float* host_scales, const float* q, double* out) {
  const int L = g->n_layers, Hq = g->q_heads, Hk = g->kv_heads, D = g->head_dim;
  const int T = g->block_tokens, k = g->k, grp = Hq / Hk;
  const int ntok_max = k * T;
  double* s = (double*)malloc((size_t)ntok_max * sizeof(double));
  double* V = (double*)malloc((size_t)ntok_max * D * sizeof(double));
  double* K = (double*)malloc((size_t)ntok_max * D * sizeof(double));
  if (!s || !V || !K) {
    free(s);
    free(V);
    free(K);
    return -1;
  }
  const double isd = 1.0 / sqrt((double)D);
  for (int r = 0; r < g->n_req; ++r) {
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < Hk; ++h) {
        const uint64_t* bl = hidx + ((size_t)(r * L + l) * Hk + h) * k;
        int nv = 0; /* selected blocks of the row, empty positions skipped */
        for (int jj = 0; jj < k; ++jj) {
          if (bl[jj] == ORA_NONE64) continue;
          const int j = nv++;
          const uint64_t hi = bl[jj];
          const double sk = tier_scale(g, host_scales, hi, 0);
          const double sv = tier_scale(g, host_scales, hi, 1);
          for (int t = 0; t < T; ++t)
            for (int d = 0; d < D; ++d) {
              const size_t row = (size_t)(j * T + t) * D + d;
              K[row] = tier_elem(g, host, hi, (uint32_t)(t * D + d)) * sk;
              V[row] = tier_elem(g, host, hi, (uint32_t)((T + t) * D + d)) * sv;
            }
        }
        const int ntok = nv * T;
        for (int gq = 0; gq < grp; ++gq) {
          const int hq = h * grp + gq;
          const float* qv = q + ((size_t)(r * L + l) * Hq + hq) * D;
          double* ov = out + ((size_t)(r * L + l) * Hq + hq) * D;
          if (ntok == 0) { /* nothing selected (request not resident): 0 */
            for (int d = 0; d < D; ++d) ov[d] = 0.0;
            continue;
          }
          double mx = -INFINITY;
          for (int t = 0; t < ntok; ++t) {
            double acc = 0.0;
            for (int d = 0; d < D; ++d) acc += (double)qv[d] * K[(size_t)t * D + d];
            s[t] = acc * isd;
            if (s[t] > mx) mx = s[t];
          }
          double den = 0.0;
          for (int t = 0; t < ntok; ++t) {
            s[t] = exp(s[t] - mx);
            den += s[t];
          }
          for (int d = 0; d < D; ++d) {
            double acc = 0.0;
            for (int t = 0; t < ntok; ++t) acc += s[t] * V[(size_t)t * D + d];
            ov[d] = acc / den;
          }
        }
      }
  }
  free(s);
  free(V);
  free(K);
  return 0;
}

int ora_attention_hidx_f64(const ora_geom* g, const uint64_t* hidx, const float* q,
                           double* out) {
  return attention_rows_f64(g, hidx, NULL, NULL, q, out);
}

/* The same over a caller's host tier image (bytes [host_blocks][bb], fp8
 * scales [host_blocks][2]) instead of the generated content: the reference
 * for a tier registered with ferry_hosttier_register. */
int ora_attention_tier_f64(const ora_geom* g, const uint64_t* hidx, const uint8_t* host,
                           const float* host_scales, const float* q, double* out) {
  if (!host || (g->dtype == ORA_FP8 && !host_scales)) return -1;
  return attention_rows_f64(g, hidx, host, host_scales, q, out);
}

/* The same over block ids: row (r, l, h) selects blocks of its owner's set
 * (r / group, l, h), host index ora_host_index(set, block). */
int ora_attention_f64(const ora_geom* g, const uint32_t* sel, const float* q,
                      double* out) {
  const int L = g->n_layers, Hk = g->kv_heads, k = g->k;
  const size_t n = (size_t)g->n_req * L * Hk * k;
  uint64_t* hidx = (uint64_t*)malloc(n * sizeof(uint64_t));
  if (!hidx) return -1;
  for (int r = 0; r < g->n_req; ++r) {
    const int o = r / g->group;
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < Hk; ++h) {
        const uint32_t set = (uint32_t)((o * L + l) * Hk + h);
        const size_t row = ((size_t)(r * L + l) * Hk + h) * k;
        for (int jj = 0; jj < k; ++jj)
          hidx[row + jj] =
              sel[row + jj] == ORA_NONE ? ORA_NONE64 : ora_host_index(g, set, sel[row + jj]);
      }
  }
  const int rc = ora_attention_hidx_f64(g, hidx, q, out);
  free(hidx);
  return rc;
}

static float load_elem_f32(int dtype, const uint8_t* p, size_t i) {
  switch (dtype) {
    case ORA_F32: {
      float v;
      memcpy(&v, p + i * 4, 4);
      return v;
    }
    case ORA_F16: {
      uint16_t v;
      memcpy(&v, p + i * 2, 2);
      return ora_f16_to_f32(v);
    }
    case ORA_BF16: {
      uint16_t v;
      memcpy(&v, p + i * 2, 2);
      return ora_bf16_to_f32(v);
    }
    default: return ora_e4m3_to_f32(p[i]);
  }
}

