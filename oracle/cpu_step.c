/*
 * cpu_step.c -- the CPU path of one executor step, timed beside the GPU by
 * bench.py's cpu_baseline leg: the oracle's LRU bookkeeping (ora_exec_step),
 * a memcpy gather of every missing block from the host tier image into a
 * host pool image, and block-sparse decode attention with fp32 accumulation.
 *
 * TEST INFRASTRUCTURE ONLY, like the rest of oracle/: the product never
 * links, loads or calls it.
 *
 * The step follows the reference's C engine for one request-step
 * (src/workloads/kv_exec.cuh:188-292: gather the misses, fetch them, run the
 * attention of every layer); the reference's attention is an FMA proxy
 * (src/workloads/kv_exec.cuh:30-37), so the attention is the textbook softmax
 * attention over the selected blocks that the float64 oracle restates.
 * Built at -O3 (without contraction): each block is decoded once per kv head
 * and shared by the head's query heads, dot products keep eight partial sums.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float e4m3_tab[256];
static float f16_tab[65536];

__attribute__((constructor)) static void cpu_step_tables(void) {
  for (int i = 0; i < 256; ++i) e4m3_tab[i] = ora_e4m3_to_f32((uint8_t)i);
  for (int i = 0; i < 65536; ++i) f16_tab[i] = ora_f16_to_f32((uint16_t)i);
}

/* n elements of a block's bytes -> floats, exactly (scales not applied). */
static void decode(int dtype, const uint8_t* p, int n, float* dst) {
  switch (dtype) {
    case ORA_F32: memcpy(dst, p, (size_t)n * 4); break;
    case ORA_F16:
      for (int i = 0; i < n; ++i) {
        uint16_t v;
        memcpy(&v, p + 2 * (size_t)i, 2);
        dst[i] = f16_tab[v];
      }
      break;
    case ORA_BF16:
      for (int i = 0; i < n; ++i) {
        uint16_t v;
        memcpy(&v, p + 2 * (size_t)i, 2);
        const uint32_t u = (uint32_t)v << 16;
        memcpy(dst + i, &u, 4);
      }
      break;
    default:
      for (int i = 0; i < n; ++i) dst[i] = e4m3_tab[p[i]];
  }
}

static float dot(const float* a, const float* b, int D) {
  float s[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  int d = 0;
  for (; d + 8 <= D; d += 8)
    for (int i = 0; i < 8; ++i) s[i] += a[d + i] * b[d + i];
  float t = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  for (; d < D; ++d) t += a[d] * b[d];
  return t;
}

int ora_attention_pool_f32(const ora_geom* g, const uint32_t* slots,
                           const uint8_t* pool, const float* pool_scales,
                           const float* q, float* out) {
  const int L = g->n_layers, Hq = g->q_heads, Hk = g->kv_heads, D = g->head_dim;
  const int T = g->block_tokens, k = g->k, grp = Hq / Hk;
  const uint64_t bb = ora_block_bytes(g);
  const float isd = 1.0f / sqrtf((float)D);
  float* kv = (float*)malloc((size_t)2 * T * D * sizeof(float));  /* K tile, V tile */
  float* acc = (float*)malloc((size_t)grp * D * sizeof(float));
  float* st = (float*)malloc((size_t)grp * 2 * sizeof(float));   /* max, sum per head */
  float* sc = (float*)malloc((size_t)T * sizeof(float));
  if (!kv || !acc || !st || !sc) {
    free(kv);
    free(acc);
    free(st);
    free(sc);
    return -1;
  }
  for (int r = 0; r < g->n_req; ++r)
    for (int l = 0; l < L; ++l)
      for (int h = 0; h < Hk; ++h) {
        const uint32_t* sl = slots + ((size_t)(r * L + l) * Hk + h) * k;
        const float* qh = q + ((size_t)(r * L + l) * Hq + (size_t)h * grp) * D;
        for (int gq = 0; gq < grp; ++gq) {
          st[2 * gq] = -INFINITY;
          st[2 * gq + 1] = 0.0f;
        }
        memset(acc, 0, (size_t)grp * D * sizeof(float));
        for (int j = 0; j < k; ++j) {
          if (sl[j] == ORA_NONE) continue; /* empty position */
          decode(g->dtype, pool + (size_t)sl[j] * bb, 2 * T * D, kv);
          const float sk = pool_scales ? pool_scales[2 * (size_t)sl[j]] : 1.0f;
          const float sv = pool_scales ? pool_scales[2 * (size_t)sl[j] + 1] : 1.0f;
          const float* V = kv + (size_t)T * D;
          for (int gq = 0; gq < grp; ++gq) {
            const float* qv = qh + (size_t)gq * D;
            float* a = acc + (size_t)gq * D;
            float bm = -INFINITY;
            for (int t = 0; t < T; ++t) {
              sc[t] = dot(qv, kv + (size_t)t * D, D) * sk * isd;
              if (sc[t] > bm) bm = sc[t];
            }
            const float m = st[2 * gq];
            const float mn = bm > m ? bm : m;
            if (mn > m) {
              const float alpha = expf(m - mn);
              st[2 * gq + 1] *= alpha;
              for (int d = 0; d < D; ++d) a[d] *= alpha;
            }
            float den = st[2 * gq + 1];
            for (int t = 0; t < T; ++t) {
              const float p = expf(sc[t] - mn);
              den += p;
              const float pv = p * sv;
              const float* vt = V + (size_t)t * D;
              for (int d = 0; d < D; ++d) a[d] += pv * vt[d];
            }
            st[2 * gq] = mn;
            st[2 * gq + 1] = den;
          }
        }
        for (int gq = 0; gq < grp; ++gq) {
          float* ov = out + ((size_t)(r * L + l) * Hq + (size_t)h * grp + gq) * D;
          const float den = st[2 * gq + 1];
          for (int d = 0; d < D; ++d) ov[d] = den > 0.0f ? acc[(size_t)gq * D + d] / den : 0.0f;
        }
      }
  free(kv);
  free(acc);
  free(st);
  free(sc);
  return 0;
}

int ora_cpu_step(ora_exec* e, const uint32_t* sel, const uint8_t* host,
                 const float* host_scales, uint8_t* pool, float* pool_scales,
                 const float* q, float* out, uint32_t* slots_scratch,
                 uint32_t* miss_count, ora_miss* misses, uint64_t* counts) {
  const ora_geom* g = ora_exec_geom(e);
  int rc = ora_exec_step(e, sel, slots_scratch, miss_count, misses, counts, NULL);
  if (rc) return rc;
  const uint64_t bb = ora_block_bytes(g);
  const int ns = ora_n_sets(g), maxsel = ora_max_sel_per_set(g);
  for (int s = 0; s < ns; ++s)
    for (uint32_t i = 0; i < miss_count[s]; ++i) {
      const ora_miss* m = misses + (size_t)s * maxsel + i;
      const uint64_t hi = ora_host_index(g, m->set, m->block);
      const uint64_t dst = (uint64_t)m->set * (uint64_t)g->cap + m->slot;
      memcpy(pool + dst * bb, host + hi * bb, bb);
      if (pool_scales && host_scales) {
        pool_scales[2 * dst] = host_scales[2 * hi];
        pool_scales[2 * dst + 1] = host_scales[2 * hi + 1];
      }
    }
  return ora_attention_pool_f32(g, slots_scratch, pool, pool_scales, q, out);
}
