/*
 * oracle.h -- CPU restatement of the per-GPU sparse KV miss-stream executor.
 *
 * TEST INFRASTRUCTURE ONLY.  The GPU is checked against this library: only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py may load it.
 * The product (ferry_amd/) never links, loads or calls it.
 *
 * Contents (each function cites the reference file:line it restates; paths
 * are relative to the clearleo126/ferry source tree):
 *   - std::mt19937_64 (the generator replay_miss_stream seeds)
 *   - ora_ref_replay: src/workloads/missstream.cuh:104-170
 *   - ora_ref_cmode_runs: src/workloads/kv_exec.cuh:188-292 and
 *     src/runtime/wla_multigpu.cuh:2527-2604 (dedup + adaptive batches +
 *     run coalescing), with AdaptiveBatchPolicy::choose_mb
 *     (src/runtime/adaptive_batch.cuh:31-36)
 *   - the executor's LRU set engine (generalises kv_touch,
 *     src/runtime/wla_multigpu.cuh:1937-1962, to (owner, layer, kv head)
 *     sets with explicit slot ids), plus two independent restatements used
 *     only to cross-check it (a deque LRU and a timestamp LRU)
 *   - synthetic selection generators for the five workloads
 *   - host-tier addressing and content (the reference aliases its host slab
 *     modulo capacity: src/runtime/wla_multigpu.cuh:323-332)
 *   - fp64 block-sparse decode attention (textbook softmax attention; the
 *     reference only has an FMA proxy at src/workloads/kv_exec.cuh:30-37 and
 *     the selection semantics of tools/capture_miss_trace.py:139-159), over the
 *     generated host tier or over a caller's tier image
 *   - a timed fp32 CPU executor step (cpu_baseline of bench.py; cpu_step.c)
 *   - lane turnover: owner reset, empty selection positions and request
 *     arrivals (steady and bursty: src/runtime/wla_multigpu.cuh:497-501;
 *     Poisson and Markov-modulated), the owner copy of a hand-off
 *     (kv_handoff with carry, src/runtime/wla_multigpu.cuh:1970-1994)
 *   - top-k block selection by the Quest bound: per-block K min/max
 *     summaries, scores and ascending top-k
 *     (tools/capture_miss_trace.py:139-159)
 *
 * Parity pins (tests/test_oracle.py, test_arrivals.py, test_select.py,
 * test_trace.py): golden counts held in the reference's logs, the C++
 * standard's mt19937_64 known answer, a build of the reference's own header
 * under oracle/_ref, and brute-force, closed-form or independent numpy
 * restatements for everything the reference does not hold.  Every function
 * here has such a check.
 */
#ifndef FERRY_ORACLE_H
#define FERRY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORA_NONE 0xFFFFFFFFu
#define ORA_NONE64 0xFFFFFFFFFFFFFFFFull

/* dtype codes shared with include/ferry_amd.h */
enum { ORA_F32 = 0, ORA_F16 = 1, ORA_BF16 = 2, ORA_FP8 = 3 };

/* ---------------- primitives ---------------- */
uint64_t ora_mix64(uint64_t seed, uint64_t idx);
uint16_t ora_f32_to_f16(float x);
float ora_f16_to_f32(uint16_t h);
uint16_t ora_f32_to_bf16(float x);
float ora_bf16_to_f32(uint16_t h);
uint8_t ora_f32_to_e4m3(float x);
float ora_e4m3_to_f32(uint8_t v);

/* ---------------- mt19937_64 ---------------- */
typedef struct {
  uint64_t mt[312];
  int idx;
} ora_mt64;
void ora_mt64_seed(ora_mt64* g, uint64_t seed);
uint64_t ora_mt64_next(ora_mt64* g);

/* ---------------- reference replay ---------------- */
/* Restates replay_miss_stream (missstream.cuh:104-170).  Event order is
 * (r, s, l, k) exactly as the reference pushes MissEvent.  blocks/miss may be
 * NULL.  counts[0] = total_selects, counts[1] = total_misses. */
int ora_ref_replay(int R, int L, int S, int sel, int hot, uint64_t seed,
                   uint64_t* blocks, uint8_t* miss, uint64_t* counts);

/* Restates the C-mode refill planner of run_miss_workload
 * (kv_exec.cuh:188-292): per (r, s) gather all-layer misses, sort by
 * (layer, block), unique, cut adaptive batches, coalesce consecutive blocks of
 * one layer inside a batch unless the direct-mapped slot range wraps.
 * Returns refill_events (submits); *refill_bytes receives the bytes. */
uint64_t ora_ref_cmode_runs(int R, int L, int S, int sel, int hot,
                            uint64_t c4_bytes, double min_mb, double max_mb,
                            double target_batches, const uint64_t* blocks,
                            const uint8_t* miss, uint64_t* refill_bytes);

/* ---------------- LRU set engine ---------------- */
typedef struct {
  uint32_t block;   /* block id fetched into the slot */
  uint32_t slot;    /* local slot index in [0, cap) */
  uint32_t evicted; /* block id evicted from the slot, or ORA_NONE */
  uint32_t set;     /* set id */
} ora_miss;

typedef struct {
  int cap;         /* slots per set */
  int lim;         /* slots the set may use now (<= cap; fewer under per-member capacity) */
  int max_blocks;  /* block ids are < max_blocks */
  uint32_t fill;   /* slots in use; free slots are [fill, cap) */
  uint32_t* ord;   /* [cap] local slots, LRU first; first `fill` valid */
  uint32_t* tag;   /* [cap] block id per slot (ORA_NONE when free) */
  uint32_t* map;   /* [max_blocks] local slot per block (ORA_NONE) */
  uint32_t* own;   /* [cap] members that touched each slot's block since it was loaded
                      (bit m = member m of the owner); own_mask, wla_multigpu.cuh:1871-1921 */
} ora_lru;

int ora_lru_init(ora_lru* s, int cap, int max_blocks);
void ora_lru_free(ora_lru* s);
void ora_lru_reset(ora_lru* s);
/* One batched sub-step over x[0..n) in canonical order.  slot_out[p] gets
 * the local slot holding x[p] after the sub-step; misses (first occurrences of
 * non-resident blocks, in order) are appended to miss_out with set id `set`.
 * Returns 0, -1 (block id out of range) or -2 (more distinct blocks than the
 * slots that may be reused in this sub-step). */
int ora_lru_substep(ora_lru* s, uint32_t set, const uint32_t* x, int n,
                    uint32_t* slot_out, ora_miss* miss_out, int* n_miss,
                    uint8_t* flag_out);
/* The same, with member[p] the member (bit index) of position p: every
 * selected slot's mask gains its members' bits, and a newly loaded slot's
 * mask starts empty (NULL: masks untouched). */
int ora_lru_substep_m(ora_lru* s, uint32_t set, const uint32_t* x, const uint8_t* member, int n,
                      uint32_t* slot_out, ora_miss* miss_out, int* n_miss, uint8_t* flag_out);

/* Trim a set to `lim` blocks (grp_trim, wla_multigpu.cuh:1923-1936): the
 * fill - lim least recently used blocks are evicted, the survivors keep their
 * order and are compacted into slots [0, lim): the i-th surviving slot >= lim
 * (ascending) moves into the i-th evicted slot < lim (ascending).  Sets
 * s->lim = lim.  moves (may be NULL) gets (from, to) pairs; returns their
 * number. */
int ora_lru_trim(ora_lru* s, int lim, uint32_t* moves);

/* Independent restatements (cross-checks only). */
/* Deque LRU with per-touch semantics (missstream.cuh:137-161). */
int ora_deque_lru_run(int cap, const uint32_t* x, int n, uint8_t* miss_flag);
/* The same with a capacity per touch, as kv_touch under per-member capacity
 * (wla_multigpu.cuh:1923-1962): before touch i the deque is trimmed from the
 * front to trim_at[i] (grp_trim: the smallest capacity members leaving left
 * since the previous touch), and a miss pops the front while the deque holds
 * cap_at[i] or more.  final_blocks (may be NULL) gets the deque at the end,
 * least recent first; returns its length. */
int ora_deque_lru_run_caps(const int* trim_at, const int* cap_at, const uint32_t* x, int n,
                           uint8_t* miss_flag, uint32_t* final_blocks);
/* Timestamp LRU with step-batched semantics (victim = least recent stamp
 * among slots not selected in the step). */
typedef struct {
  int cap, max_blocks;
  uint32_t* tag;
  uint64_t* stamp;
  uint64_t clock;
  uint32_t fill;
} ora_tslru;
int ora_tslru_init(ora_tslru* s, int cap, int max_blocks);
void ora_tslru_free(ora_tslru* s);
int ora_tslru_step(ora_tslru* s, const uint32_t* x, int n, uint32_t* slot_out,
                   uint32_t* miss_blocks, uint32_t* miss_slots, int* n_miss);

/* ---------------- executor geometry ---------------- */
typedef struct {
  int n_req;       /* B requests */
  int group;       /* requests per owner (1 = private sets) */
  int n_layers;    /* L */
  int kv_heads;    /* Hkv */
  int q_heads;     /* Hq */
  int head_dim;    /* D */
  int block_tokens;/* T */
  int k;           /* selected blocks per (request, layer, kv head) */
  int cap;         /* slots per set */
  int max_blocks;  /* set block ids < max_blocks */
  int dtype;       /* ORA_F32 / ORA_F16 / ORA_BF16 / ORA_FP8 */
  int granularity; /* 0 = step-batched, 1 = serial (per selection) */
  uint64_t host_blocks; /* host tier capacity in blocks */
  uint64_t seed;   /* host tier content seed */
  float value_std; /* std of K/V values */
  int cap_mode;    /* 0: every set holds cap blocks; 1: (cap / group) per resident member */
} ora_geom;

int ora_n_owners(const ora_geom* g);
int ora_n_sets(const ora_geom* g);
int ora_members(const ora_geom* g, int owner);
int ora_max_sel_per_set(const ora_geom* g);
uint64_t ora_block_bytes(const ora_geom* g); /* K+V bytes, scales excluded */
uint64_t ora_host_index(const ora_geom* g, uint32_t set, uint32_t block);

/* Executor state = one ora_lru per set. */
typedef struct ora_exec ora_exec;
ora_exec* ora_exec_create(const ora_geom* g);
void ora_exec_destroy(ora_exec* e);
const ora_geom* ora_exec_geom(const ora_exec* e);
/* One decode step of bookkeeping.  sel: [B][L][Hkv][k] set block ids.
 * slots_out: [B][L][Hkv][k] global slot ids (set * cap + local).
 * miss_count: [n_sets]; misses: [n_sets][max_sel_per_set].  counts[0..2] =
 * selections, misses, hits.  Returns 0 or a negative error. */
int ora_exec_step(ora_exec* e, const uint32_t* sel, uint32_t* slots_out,
                  uint32_t* miss_count, ora_miss* misses, uint64_t* counts,
                  uint8_t* flags);
/* Empty the sets of one owner (a new request takes over its lane). */
int ora_exec_reset_owner(ora_exec* e, int owner);
/* Per-slot member masks of every set: own[n_sets][cap]. */
void ora_exec_own(const ora_exec* e, uint32_t* own);
/* Per-request carry of a member (kv_handoff_owned, wla_multigpu.cuh:1901-1921):
 * ora_exec_export_member lists, per set of lane's owner, the resident blocks
 * only lane's member touched (own == its bit), least recently used first:
 * counts[L*Hkv] and blocks[L*Hkv][cap].  ora_exec_import_member merges such a
 * list into `lane`'s owner of `dst`: a block already resident gains the lane's
 * member bit and keeps its place; another is appended as most recent after
 * evicting the least recent block while the set holds its capacity or more,
 * the new block taking the evicted slot (else slot fill).  Returns 0 or -1. */
int ora_exec_export_member(const ora_exec* e, int lane, uint32_t* counts, uint32_t* blocks);
int ora_exec_import_member(ora_exec* e, int lane, const uint32_t* counts, const uint32_t* blocks);
/* Resident members (every lane starts resident): the requests of lanes[0..n)
 * leave (delta -1) or join (+1) their owners; a leaving member's bit is
 * cleared from every slot of its owner (own_release, wla_multigpu.cuh:
 * 1896-1909) and the owner is trimmed to its new capacity under cap_mode 1
 * (ora_lru_trim).  A lane out of range,
 * leaving while not resident or joining while resident is skipped and makes
 * the call return -1.  ora_exec_members_get copies the per-owner counts. */
int ora_exec_members(ora_exec* e, const uint32_t* lanes, int n, int delta);
void ora_exec_members_get(const ora_exec* e, uint32_t* members);
/* Blocks the sets of an owner with `members` resident members may hold. */
int ora_capacity(const ora_geom* g, int members);
/* Copy owner src_owner's sets of src onto owner dst_owner of dst. */
int ora_exec_copy_owner(const ora_exec* src, int src_owner, ora_exec* dst, int dst_owner);
/* Per-set state export for parity: fill[n_sets], ord[n_sets][cap],
 * tag[n_sets][cap]. */
void ora_exec_state(const ora_exec* e, uint32_t* fill, uint32_t* ord,
                    uint32_t* tag);

/* ---------------- workload generators ---------------- */
typedef struct {
  int n_req, group, n_layers, kv_heads, k;
  int dist;          /* 0 = uniform, 1 = zipf */
  double zipf_s;
  double reuse;      /* probability a selected block is kept next step */
  int prefix_blocks; /* shared prefix blocks per group (0 = none) */
  uint64_t seed;
  const int* ctx_blocks; /* [n_req] logical context length in blocks */
  const double* reuse_r; /* [n_req] per-request reuse, or NULL (use reuse) */
  /* Lane turnover (NULL = lane r holds request r from step 0, all active):
   * the request id in each lane, the step it was admitted at, and whether
   * the lane holds a request at all (idle lanes give empty rows). */
  const int* rid;
  const int* start;
  const uint8_t* active;
  /* Prefix-group turnover (NULL / 0 = none): the private id range of the
   * request in each lane (default: its member index r % group), the number
   * of such ranges per owner (0 = group), and each owner's permutation
   * domain fixed at creation (NULL = the largest current member context). */
  const int* prange;
  int private_ranges;
  const int* nperm;
} ora_selgen;

/* Per-request context lengths: uniform integer in [lo, hi]. */
void ora_ctx_uniform(uint64_t seed, int n_req, int lo, int hi, int* out);
/* Set block-id bound for a generator (max over owners). */
int ora_selgen_max_blocks(const ora_selgen* s);
/* Selections of one step: out [B][L][Hkv][k] set block ids; state [same]
 * carries each request's logical selection from step to step.  A row of a
 * context shorter than k holds all its blocks, then ORA_NONE. */
int ora_selgen_step(const ora_selgen* s, int step, uint32_t* state,
                    uint32_t* out);

/* ---------------- request arrivals ---------------- */
/* kind 0 steady, 1 bursty, 2 Poisson, 3 Markov-modulated Poisson; out[n] ms. */
int ora_arrivals(int kind, uint32_t n, double gap, double period, double ratio,
                 uint64_t seed, double* out);

/* ---------------- host tier ---------------- */
/* Element e of host block h (K then V, [T][D] each) as the stored encoding
 * widened to uint32 (f32 bits, f16/bf16 bits, or an e4m3 byte). */
uint32_t ora_host_elem(const ora_geom* g, uint64_t h, uint32_t e);
/* Per-block dequant scales (fp8 only; 1.0 otherwise): kv = 0 K, 1 V. */
float ora_host_scale(const ora_geom* g, uint64_t h, int kv);
/* Fill one host block's bytes (bb bytes) and its two scales. */
void ora_host_block(const ora_geom* g, uint64_t h, void* bytes, float* scales);
double ora_decode(int dtype, uint32_t v);

/* ---------------- top-k block selection ---------------- */
/* K min/max of host block h per dim (decoded floats). */
void ora_summary(const ora_geom* g, uint64_t h, float* kmin, float* kmax);
/* Quest scores of blocks [0, min(ctx, stride)) of every row (mode 0: rows are
 * (request, layer, kv head); mode 1: (request, layer), max over all heads);
 * out[row][stride]. */
int ora_quest_scores(const ora_geom* g, const float* q, const int* ctx_blocks, int mode,
                     int stride, float* out);
/* Top-k selection into sel [B][L][Hkv][k] (ascending ids, ORA_NONE padding). */
int ora_select_topk(const ora_geom* g, const float* q, const int* ctx_blocks, int mode,
                    uint32_t* sel);

/* Exact softmax mass per block, the capture tool's "mass" method
 * (tools/capture_miss_trace.py:147-155), in double: for (request r, layer l),
 * each kv head h (set (r*L + l)*Hkv + h; block b's K = the K half of host
 * block ora_host_index(set, b), fp8 K times its scale) and each of its G query
 * heads, p_t = softmax over the context's n*T tokens of q . k_t / sqrt(D), and
 * score[b] = sum over h, its query heads and b's T tokens of p_t.
 * out[(r*L + l) * stride + b] for b < min(ctx, stride). */
int ora_mass_scores(const ora_geom* g, const float* q, const int* ctx_blocks, int stride,
                    double* out);
/* The min(k, n) blocks of highest mass of every (request, layer), ties to the
 * lower ids, in ascending order, written to every kv head's row of sel
 * [B][L][Hkv][k] (ORA_NONE padding): the tool keeps one page list per layer. */
int ora_select_mass(const ora_geom* g, const float* q, const int* ctx_blocks, uint32_t* sel);

/* ---------------- attention ---------------- */
/* fp64 block-sparse decode attention with keys read from the host tier by
 * (set, block).  q, out: [B][L][Hq][D] (q fp32, out fp64). */
int ora_attention_f64(const ora_geom* g, const uint32_t* sel, const float* q,
                      double* out);
/* The same with every row's blocks named by host-tier index: hidx
 * [B][L][Hkv][k], ORA_NONE64 for an empty position; a block named twice in
 * one row is attended twice. */
int ora_attention_hidx_f64(const ora_geom* g, const uint64_t* hidx, const float* q,
                           double* out);
/* The same over a caller's host tier image instead of the generated content:
 * host [host_blocks][bb] bytes, host_scales [host_blocks][2] (fp8 only; K
 * scale, V scale).  -1 if an image the dtype needs is missing. */
int ora_attention_tier_f64(const ora_geom* g, const uint64_t* hidx, const uint8_t* host,
                           const float* host_scales, const float* q, double* out);
/* Same attention, but K/V read from a host pool image laid out like the HBM
 * pool (slot-major, bb bytes per slot, scales[slot][2]) through the slot
 * table; fp32 accumulation.  The CPU path timed beside the GPU (cpu_step.c). */
int ora_attention_pool_f32(const ora_geom* g, const uint32_t* slots,
                           const uint8_t* pool, const float* pool_scales,
                           const float* q, float* out);

/* ---------------- CPU executor step (cpu_baseline) ---------------- */
/* Bookkeeping + memcpy gather from the host tier image into the pool image +
 * fp32 attention.  host: [host_blocks][bb] bytes, host_scales [host_blocks][2].
 * pool: [n_sets*cap][bb], pool_scales [n_sets*cap][2]. */
int ora_cpu_step(ora_exec* e, const uint32_t* sel, const uint8_t* host,
                 const float* host_scales, uint8_t* pool, float* pool_scales,
                 const float* q, float* out, uint32_t* slots_scratch,
                 uint32_t* miss_count, ora_miss* misses, uint64_t* counts);
/* Materialise the host tier image (used by the CPU baseline). */
void ora_host_fill(const ora_geom* g, uint8_t* host, float* host_scales);

#ifdef __cplusplus
}
#endif
#endif
