/*
 * ferry_amd.h -- C-ABI of the MI355X-native sparse KV miss-stream executor.
 *
 * One GPU, one process.  Every entry point takes plain pointers and sizes;
 * device buffers are caller-owned unless stated; every call that launches
 * work takes an explicit hipStream_t (passed as void*, 0 = null stream).
 * Every function returns an int status (FERRY_OK == 0, negative on error) and
 * never exits the process; the reference aborted instead
 * (src/common/cuda_check.cuh:9-28, src/workloads/miss_trace.cuh:64-71).
 * Buffers a kernel reads or writes must be device, managed or pinned host
 * memory: a null pointer or one into pageable host memory returns
 * FERRY_EINVAL before anything is launched.  Their sizes follow from the
 * context's geometry and are the caller's to get right.
 *
 * The reference exposes this path as header-only C++ (namespace ferry) with
 * no FFI; each entry point below names the reference interface it replaces.
 * Reference paths are relative to the clearleo126/ferry source tree.
 */
#ifndef FERRY_AMD_H
#define FERRY_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define FERRY_OK 0
#define FERRY_EINVAL (-1)    /* invalid argument or configuration */
#define FERRY_EHIP (-2)      /* HIP runtime error (see ferry_last_error) */
#define FERRY_ERANGE (-3)    /* a selected block id >= max_blocks */
#define FERRY_ECAPACITY (-4) /* a step selects more distinct blocks than a set can hold */
#define FERRY_ENOMEM (-5)    /* device or pinned host allocation failed */
#define FERRY_ESPIN (-6)     /* a bounded device wait ran out (queue protocol) */
#define FERRY_ESTATE (-7)    /* inconsistent set state detected on device */

/* ---- KV element types ---- */
#define FERRY_F32 0
#define FERRY_F16 1
#define FERRY_BF16 2
#define FERRY_FP8_E4M3 3 /* OCP E4M3FN + one fp32 scale per block for K and V */

/* ---- LRU granularity ---- */
#define FERRY_LRU_STEP 0   /* one batched update per decode step (executor rule) */
#define FERRY_LRU_SERIAL 1 /* one update per selection: replay_miss_stream/kv_touch */

/* ---- miss -> fetch-worker assignment ---- */
#define FERRY_ASSIGN_SPREAD 0   /* hash of the set id modulo workers */
#define FERRY_ASSIGN_AFFINITY 1 /* request (owner) modulo workers */

/* ---- attention kernel selection ---- */
#define FERRY_ATTN_AUTO 0 /* MFMA for GQA groups (q_heads/kv_heads >= 2) of 16/8-bit KV and for
                            fp8 MHA, else VALU; prefix groups (group > 1) that fit
                            FERRY_ATTN_GROUP use it */
#define FERRY_ATTN_VALU 1 /* vector-ALU kernel for every shape */
#define FERRY_ATTN_MFMA 2 /* MFMA kernel per (request, layer, kv head) row; needs 16/8-bit KV
                            and q_heads/kv_heads >= 2, or fp8 KV */
#define FERRY_ATTN_GROUP 3 /* MFMA kernel per (prefix group, layer, kv head): every distinct
                             block of the group's set is read from HBM once for all members.
                             Needs group > 1, q_heads/kv_heads >= 2, 16/8-bit KV,
                             group * q_heads/kv_heads <= 64, group * k <= 2048 and
                             slots_per_set + group * k <= 12288 */

/* Geometry and policy of one executor.  Sets are (owner, layer, kv head)
 * with owner = request / group; each set owns slots_per_set slots of the HBM
 * pool.  Replaces MissSpec (src/workloads/missstream.cuh:23-76) widened from
 * (request, layer, 4-token all-head block) to (request, layer, head,
 * block_tokens block). */
typedef struct ferry_config {
  int32_t n_req;         /* decode batch B */
  int32_t group;         /* requests per owner (prefix group); 1 = private sets */
  int32_t n_layers;      /* L */
  int32_t kv_heads;      /* Hkv */
  int32_t q_heads;       /* Hq (multiple of Hkv) */
  int32_t head_dim;      /* D (128) */
  int32_t block_tokens;  /* tokens per block (16) */
  int32_t k;             /* selected blocks per (request, layer, kv head) */
  int32_t slots_per_set; /* HBM slots per set */
  int32_t max_blocks;    /* block ids of a set are < max_blocks */
  int32_t dtype;         /* FERRY_F32 .. FERRY_FP8_E4M3 */
  int32_t lru_mode;      /* FERRY_LRU_STEP or FERRY_LRU_SERIAL */
  uint64_t host_blocks;  /* host-tier capacity in blocks (aliased modulo) */
  uint64_t host_seed;    /* host-tier content seed */
  float value_std;       /* standard deviation of K/V values */
  int32_t fetch_workers; /* persistent fetch workgroups; 0 = 1 per 4 CUs */
  int32_t steal;         /* 1 = fetch workers steal from each other */
  int32_t assign;        /* FERRY_ASSIGN_SPREAD or FERRY_ASSIGN_AFFINITY */
  int32_t attn;          /* FERRY_ATTN_AUTO, FERRY_ATTN_VALU or FERRY_ATTN_MFMA */
  int32_t cap_mode;      /* FERRY_CAP_GROUP or FERRY_CAP_PER_MEMBER */
} ferry_config;

/* ---- capacity of an owner's sets (MissSpec::cap_mode, wla_group_cap,
 * src/workloads/missstream.cuh:40-47, 91-94) ---- */
#define FERRY_CAP_GROUP 0      /* every set holds slots_per_set blocks */
#define FERRY_CAP_PER_MEMBER 1 /* (slots_per_set / group) x resident members, at least one share */

/* One fetched block: written per set in miss order. */
typedef struct ferry_miss {
  uint32_t block;   /* block id fetched */
  uint32_t slot;    /* local slot in the set, [0, slots_per_set) */
  uint32_t evicted; /* block id evicted from that slot, 0xFFFFFFFF if none */
  uint32_t set;     /* set id = (owner * n_layers + layer) * kv_heads + head */
} ferry_miss;

/* Counters; replaces WlAStats / WlaMultiStats (src/workloads/kv_exec.cuh:39-45,
 * src/runtime/wla_multigpu.cuh:177-233). */
typedef struct ferry_stats {
  uint64_t steps;          /* fetch steps run */
  uint64_t selections;     /* non-empty selections processed */
  uint64_t misses;         /* unique blocks fetched (refill events of 1 block) */
  uint64_t fetched_bytes;  /* host-tier bytes moved into the pool */
  uint64_t steals;         /* successful steals between fetch workers */
  uint64_t stolen;         /* misses moved by steals */
  uint64_t last_misses;    /* misses of the most recent step */
  int32_t device_error;    /* first device-side error (FERRY_E*), 0 if none */
  int32_t pad;
} ferry_stats;

typedef struct ferry_ctx ferry_ctx;

/* Text of the last error on this thread (never NULL). */
const char* ferry_last_error(void);
/* Library version string. */
const char* ferry_version(void);

/* Create an executor on `device`: allocates the HBM slot pool, the per-set
 * LRU state, the miss ring and the pinned host tier.  Replaces the
 * allocations inside run_miss_workload (src/workloads/kv_exec.cuh:78-99) and
 * WlaMultiGpuCtx (src/runtime/wla_multigpu.cuh:435-623). */
int ferry_ctx_create(const ferry_config* cfg, int device, ferry_ctx** out);
int ferry_ctx_destroy(ferry_ctx* ctx);
int ferry_ctx_config(const ferry_ctx* ctx, ferry_config* out);
/* Sizes: n_sets, max selections per set, block bytes (K+V, no scales),
 * pool slots. */
int ferry_ctx_sizes(const ferry_ctx* ctx, uint32_t* n_sets, uint32_t* max_sel,
                    uint64_t* block_bytes, uint64_t* pool_slots);

/* Fill the pinned host tier with its deterministic content (K then V,
 * [block_tokens][head_dim] each; fp8 adds two fp32 scales per block).  The
 * reference fills its slab with uniform halves (src/workloads/kv_exec.cuh:78-86)
 * or a tile (src/runtime/wla_multigpu.cuh:532-544). */
int ferry_hosttier_fill(ferry_ctx* ctx, void* stream);
/* Use the caller's pinned host memory as the tier instead of the context's
 * own: `host` holds host_blocks * block_bytes bytes in the same layout (block
 * i at i * block_bytes), `scales` host_blocks * 2 fp32 for fp8 KV (NULL
 * otherwise).  Both must be pinned and mapped into the device's address space
 * (hipHostMalloc; registering pageable memory is not supported), stay valid
 * until the context is destroyed and are not freed by it.  Waits for the
 * device, then frees the context's own tier.  Replaces the host slab that
 * run_miss_workload allocated for itself (src/workloads/kv_exec.cuh:78-92) with
 * the caller-owned slab the reference's ownership model describes. */
int ferry_hosttier_register(ferry_ctx* ctx, void* host, uint64_t host_bytes, float* scales,
                            uint64_t scale_bytes);
/* Host pointers of the pinned tier (bytes: host_blocks*block_bytes; scales:
 * host_blocks*2 floats, NULL unless fp8). */
int ferry_hosttier_view(ferry_ctx* ctx, void** bytes, float** scales);
/* Device pointers of the HBM pool (slot-major, block_bytes per slot) and its
 * scales (2 floats per slot, NULL unless fp8). */
int ferry_pool_view(ferry_ctx* ctx, void** pool, float** scales);

/* Forget every resident block (all sets empty).  Replaces
 * GPUBoundedQueue::reset + cache re-init (src/queue/gpu_bounded_queue.cuh:176-181). */
int ferry_sets_reset(ferry_ctx* ctx, void* stream);
/* Forget the resident blocks of the listed owners only: owners is a device
 * array of n owner ids (request / group), n <= number of owners.  Used when a
 * new request takes over a lane of the batch; other owners' sets are
 * untouched.  An owner id out of range is latched as FERRY_EINVAL in the
 * device error word.  The reference gives every request id its own hot
 * cache segment for the whole run (src/runtime/wla_multigpu.cuh:468, 517)
 * and trims a group's LRU when a member leaves (grp_trim, :1923-1936); here
 * a batch lane is reused by successive requests, so it starts cold. */
int ferry_sets_reset_owners(ferry_ctx* ctx, const uint32_t* owners, uint32_t n, void* stream);
/* Copy per-set LRU state to host arrays: fill[n_sets], ord[n_sets][slots]
 * (local slots, LRU first), tag[n_sets][slots] (block per slot). */
int ferry_sets_state(ferry_ctx* ctx, uint32_t* fill, uint32_t* ord, uint32_t* tag);
/* Per-slot member masks of prefix groups (group > 1): own[n_sets][slots],
 * bit m set when member m (lane % group) of the set's owner touched the
 * slot's block since it became resident and is still resident itself
 * (cleared when the member leaves; 0 for a free slot).  Replaces the
 * reference's own_mask table (src/runtime/wla_multigpu.cuh:1871-1912);
 * synchronises. */
int ferry_sets_own(ferry_ctx* ctx, uint32_t* own);

/* Resident members of prefix groups.  Every batch lane (request row) is a
 * member of its owner (lane / group) and starts resident.  ferry_members_leave
 * takes the requests of the listed lanes (device array of n lane ids) out:
 * each owner loses one resident member per lane, and under
 * FERRY_CAP_PER_MEMBER its sets are trimmed to the new capacity, least
 * recently used blocks first; the surviving blocks keep their LRU order and
 * are compacted into slots [0, capacity) (blocks in higher slots move into
 * the freed lower ones, data and fp8 scales included), so a set's resident
 * slots stay [0, fill).  ferry_members_join makes the listed lanes resident
 * again (a new request of the group takes the lane): its owner gains a
 * member, and with it capacity; nothing is evicted or reset.  Lanes must
 * alternate leave / join: leaving a lane that is not resident, or joining one
 * that is, latches FERRY_EINVAL in the device error word.  Replaces
 * grp_member_add at dispatch and tick_end plus grp_trim
 * (src/runtime/wla_multigpu.cuh:801, 846-862, 1923-1936).  ferry_members_get
 * copies the resident members of every owner to members[n_owners]
 * (synchronises). */
int ferry_members_leave(ferry_ctx* ctx, const uint32_t* lanes, uint32_t n, void* stream);
int ferry_members_join(ferry_ctx* ctx, const uint32_t* lanes, uint32_t n, void* stream);
int ferry_members_get(ferry_ctx* ctx, uint32_t* members);

/* Empty positions.  A selection id of FERRY_EMPTY (0xFFFFFFFF) selects
 * nothing: it is neither hit nor miss, its slot comes back as FERRY_EMPTY,
 * and attention skips it.  A request that is not resident this step passes a
 * row of FERRY_EMPTY (its attention output is 0); a context shorter than k
 * blocks passes a ragged row (the reference's trace format allows fewer
 * selected pages at a short tail, tools/capture_miss_trace.py:36-37). */
#define FERRY_EMPTY 0xFFFFFFFFu

/* One decode step of bookkeeping + miss fetch:
 *   sel        [B][L][Hkv][k] set block ids (device, u32; FERRY_EMPTY allowed)
 *   slots      [B][L][Hkv][k] out: pool slot of each selection (device, u32)
 *   miss_count [n_sets] out: misses per set (device, u32)
 *   misses     [n_sets][max_sel] out: fetched blocks per set in miss order
 *   miss_flag  [B][L][Hkv][k] out, optional (NULL): 1 where the selection
 *              missed (first toucher), else 0
 * dedups, assigns and evicts slots by LRU, pushes the misses onto the device
 * miss ring and drains it with persistent fetch workgroups that read the host
 * tier directly (16-byte loads over the host link) into the HBM pool.
 * Replaces run_miss_workload mode C (src/workloads/kv_exec.cuh:188-292) and
 * the exec_step C engine + kv_touch (src/runtime/wla_multigpu.cuh:2527-2604,
 * 1937-1962). */
int ferry_fetch_step(ferry_ctx* ctx, const uint32_t* sel, uint32_t* slots,
                     uint32_t* miss_count, ferry_miss* misses,
                     uint8_t* miss_flag, void* stream);

/* The two halves of ferry_fetch_step, for callers that place them on
 * different streams or interpose work.  ferry_bookkeep_step leaves the
 * misses queued on the device miss ring; ferry_missq_drain fetches them. */
int ferry_bookkeep_step(ferry_ctx* ctx, const uint32_t* sel, uint32_t* slots,
                        uint32_t* miss_count, ferry_miss* misses,
                        uint8_t* miss_flag, void* stream);
/* Bookkeeping of layers [l0, l0 + nl) only (same buffers and semantics as
 * ferry_bookkeep_step, which is l0 = 0, nl = n_layers). */
int ferry_bookkeep_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const uint32_t* sel,
                          uint32_t* slots, uint32_t* miss_count, ferry_miss* misses,
                          uint8_t* miss_flag, void* stream);
/* Queue n externally built misses (device array) onto the ring.  Replaces
 * dq_push producers of GPUBoundedQueue (src/queue/gpu_bounded_queue.cuh:70-126). */
int ferry_missq_push(ferry_ctx* ctx, const ferry_miss* misses, uint32_t n,
                     void* stream);
/* Drain the ring: persistent workgroups pop their own deque and steal from
 * the tail of a peer holding at least twice its fair share.  Replaces
 * HostStagedChannel::submit/sync (src/comm/host_staged_channel.cpp:43-87) and
 * the cross-GPU steal rules (src/runtime/wla_multigpu.cuh:882-884, 1147-1152,
 * 1518-1526). */
int ferry_missq_drain(ferry_ctx* ctx, void* stream);

/* Block-sparse decode attention over the selected blocks:
 *   q     [B][L][Hq][D] fp32 (device)
 *   slots [B][L][Hkv][k] pool slots from ferry_fetch_step (device)
 *   out   [B][L][Hq][D] fp32 (device)
 * softmax(q K^T / sqrt(D)) V over every token of the k blocks, fp32
 * accumulation, online softmax.  A slot selected twice in one row counts
 * twice; a row with no slot (all FERRY_EMPTY) gives 0; a slot outside the pool
 * is read as slot 0 and reported as FERRY_ERANGE.  With the prefix-group
 * kernel (FERRY_ATTN_GROUP) a member row's slots are expected in its group's
 * set (as ferry_fetch_step assigns them); other in-pool slots are attended
 * correctly on a slower path.  Replaces the FMA proxy attn_kernel /
 * wla_attn_kernel (src/workloads/kv_exec.cuh:30-37,
 * src/runtime/wla_multigpu.cuh:96-103). */
int ferry_sparse_decode(ferry_ctx* ctx, const float* q, const uint32_t* slots,
                        float* out, void* stream);

/* Which attention kernel ferry_sparse_decode runs for this context:
 * *kind = FERRY_ATTN_VALU, FERRY_ATTN_MFMA (one workgroup per request row) or
 * FERRY_ATTN_GROUP (one per prefix-group set), *waves = wavefronts per
 * workgroup of ferry_sparse_decode's launch over all L layers.  The
 * prefix-group kernel runs eight on a launch of no more group sets than the
 * GPU has CUs where its LDS allows, else four, so the smaller launches of
 * ferry_sparse_decode_layers and of ferry_decode_step's layer ranges may run
 * eight where four is reported.  No reference counterpart (the reference has
 * one proxy kernel); for callers that report rooflines per kernel. */
int ferry_attn_kernel(const ferry_ctx* ctx, int32_t* kind, int32_t* waves);

/* Attention of layers [l0, l0 + nl) only. */
int ferry_sparse_decode_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                               const uint32_t* slots, float* out, void* stream);

/* One whole decode step with the fetch overlapped with attention: layers are
 * cut into `chunks` ranges; the fetch of each range runs on side_stream, and
 * attention of a range starts on `stream` as soon as its fetch is done, while
 * the next range is fetched.  Bookkeeping runs on `stream`, two ranges ahead
 * (range c + 2 is booked, into the miss ring the fetch of range c has just
 * drained, before range c is attended), so the fetch of a range waits for
 * neither its bookkeeping nor any attention.  The overlap needs the two streams on
 * different hardware queues: HIP shares a few queues (4 by default) among a
 * process's streams round-robin as they are created, and two streams on one
 * queue run in turn, so a caller creates its side stream once and keeps it (a
 * fresh stream per step can land on the main stream's queue).  The context
 * creates no stream of its own.  side_stream NULL (or
 * equal to stream) runs the same sequence on one stream.  When this returns,
 * work queued on `stream` after it observes the whole step.  Replaces the refill /
 * compute overlap of run_miss_workload mode C: batches submitted to the
 * channel, compute waiting on the last arrival (src/workloads/kv_exec.cuh:
 * 228-286, src/comm/host_staged_channel.cuh:55-63). */
int ferry_decode_step(ferry_ctx* ctx, const uint32_t* sel, const float* q, uint32_t* slots,
                      float* out, uint32_t* miss_count, ferry_miss* misses, int32_t chunks,
                      void* stream, void* side_stream);
/* chunks == 0 chooses the chunk count with the reference's adaptive batch
 * rule (AdaptiveBatchPolicy::choose_mb, src/runtime/adaptive_batch.cuh:31-36;
 * take rule kv_exec.cuh:230-235): the bytes the last finished step fetched
 * are `pending`, a chunk moves g = clamp(pending / target_batches, min_mb,
 * max_mb) MB, and the step runs ceil(pending / g) chunks (1 .. n_layers; 1
 * before any step has finished).  A chunk costs three launches and a drain,
 * so the GPU policy works in larger units than the reference's channel
 * submits: defaults min 32 MB, max 512 MB, target 8 batches.  The count is
 * read from pinned memory that each step's end copies into, so the host never
 * waits for the device.  ferry_decode_chunks gives the count for a pending
 * number of blocks.  The adaptive step also shortens the last range (down to
 * one layer) when attention is cheap next to the fetch, since its attention
 * is the part the fetch cannot hide; an explicit count gives even ranges. */
int ferry_set_batch_policy(ferry_ctx* ctx, double min_mb, double max_mb, double target_batches);
int ferry_decode_chunks(const ferry_ctx* ctx, uint64_t pending_blocks, int32_t* chunks);

/* ---- top-k block selection (Quest bound) ----
 * The step upstream of the miss queue: choose each request's k blocks from
 * the query, as tools/capture_miss_trace.py:139-159 does with its "quest"
 * method.  Per block (= page of 16 tokens) and kv head, the elementwise min
 * and max of K over the block's tokens bound the attention score of any of
 * its tokens: bound = sum_d max(q_d kmax_d, q_d kmin_d).  The score of a
 * block is the max of the bound over the query heads of the kv head
 * (FERRY_TOPK_PER_HEAD: one selection per (request, layer, kv head)), or
 * over every head of the layer (FERRY_TOPK_LAYER_MAX: one selection per
 * (request, layer), written to every kv head's row, as the capture tool
 * does).  The k highest scores win, ties to the lower block id; the row is
 * written in ascending block order.  A context of n < k blocks selects all n
 * and pads the row with FERRY_EMPTY; n = 0 gives an empty row (a request that
 * is not resident).  fp32 scores are computed in a fixed order, so the
 * selection is reproducible bit for bit.
 *
 * ferry_summaries_build computes the K min/max of every host-tier block
 * (reading the pinned tier once; call it again after writing the tier) into
 * n_records records [n_records][2][head_dim] in the KV element type (fp8:
 * E4M3 codes; the block's K scale is kept beside them and multiplies the
 * bound).  Block (set, b) reads record (set*max_blocks + b) mod n_records.
 * n_records must be a multiple of host_blocks (0 means host_blocks, the
 * smallest table); n_records >= sets*max_blocks gives every block a record
 * of its own, as a server that summarises each page it writes has, and is
 * what the selection's memory traffic should be measured with.
 * ferry_summaries_view returns their device pointers and record count.
 * ferry_select_topk: q [B][L][Hq][D] fp32 (device), ctx_blocks [B] int32
 * (device, context length of each request in blocks, <= max_blocks), sel
 * [B][L][Hkv][k] u32 out (device) -- the input of ferry_fetch_step.  Needs
 * group == 1 and (query heads per row * D + max_blocks) * 4 <= 64 KiB. */
#define FERRY_TOPK_PER_HEAD 0
#define FERRY_TOPK_LAYER_MAX 1
int ferry_summaries_build(ferry_ctx* ctx, uint64_t n_records, void* stream);
int ferry_summaries_view(ferry_ctx* ctx, void** sums, float** scales, uint64_t* n_records);
int ferry_select_topk(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks, int mode,
                      uint32_t* sel, void* stream);
/* Selection of layers [l0, l0 + nl) only. */
int ferry_select_topk_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                             const int32_t* ctx_blocks, int mode, uint32_t* sel, void* stream);

/* The capture tool's "mass" method (tools/capture_miss_trace.py:147-155): a
 * block's score is the softmax probability its tokens take, softmax over the
 * whole context of q . k / sqrt(head_dim), summed over every query head of the
 * layer; each (request, layer) gets the min(k, ctx) blocks of highest score in
 * ascending order (ties to the lower ids), written to every kv head's row of
 * sel, EMPTY-padded.  It reads every context token's key from a dense K table
 * in HBM: ferry_ktiles_build copies the K half of each host-tier block into
 * n_records records (a multiple of host_blocks; 0 = one per host block; block
 * (set, b) reads record (set * max_blocks + b) mod n_records, as the
 * summaries), device-direct from the pinned tier, fp8 K scales included.
 * fp32 records keep the block's row-major order; 16-bit and fp8 records are
 * lane-transposed for the matrix-core kernel (16-byte word c of token row t
 * at word 64 (c / 4) + 16 (c % 4) + t), as ferry_ktiles_view shows them.
 * q [B][L][Hq][128] fp32 and ctx_blocks [B] int32 on the device; group 1
 * only; max_blocks <= 15360 (one score per block in LDS).  A context longer
 * than max_blocks latches FERRY_ERANGE and leaves that row EMPTY.
 * The table is a snapshot of the host tier: rebuild it after the tier's
 * content changes.  The selection keeps each block's mass per kv head (16-bit
 * and fp8 K, about n_req * L * kv_heads * max_blocks * 4 bytes) and, for fp32
 * and fp8 K or where max_blocks * q_heads / kv_heads floats exceed 144 KiB of
 * LDS, each block's softmax max and sum in a workspace of the context
 * allocated by ferry_ktiles_build, so two ferry_select_mass calls on one
 * context must not run concurrently. */
int ferry_ktiles_build(ferry_ctx* ctx, uint64_t n_records, void* stream);
int ferry_ktiles_view(ferry_ctx* ctx, void** ktiles, float** scales, uint64_t* n_records);
int ferry_select_mass(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks, uint32_t* sel,
                      void* stream);
int ferry_select_mass_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                             const int32_t* ctx_blocks, uint32_t* sel, void* stream);
/* ferry_select_mass over every layer, allocating nothing: the per-workgroup
 * softmax (max, sum) workspace lives in a static 64 MiB array of the library
 * (one per GPU, held until the process ends) instead of the context's.  No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  It calls no hipMalloc/hipFree.  Needs the K table
 * (ferry_ktiles_build, which the caller runs beforehand) and, within the
 * 64 MiB, one workgroup's workspace slice where the softmax max and sum stay
 * in HBM (see ferry_select_mass), max_blocks * (q_heads / kv_heads) * 8
 * bytes, plus for 16-bit and fp8 K the masses of one layer,
 * n_req * kv_heads * max_blocks * 4 bytes, and 512 bytes (FERRY_EINVAL
 * otherwise).  The layers run in ranges one after the other when the masses
 * of all of them do not fit, and fewer workgroups share the work when the
 * array holds fewer slices than ferry_select_mass would launch.  Output equals
 * ferry_select_mass's bit for bit.  Every call on one GPU uses the same array:
 * calls that overlap on one GPU (other streams, other contexts, other host
 * threads) race and must be serialised by the caller. */
int ferry_select_mass_noalloc(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks,
                              uint32_t* sel, void* stream);

/* ---- owner hand-off (the per-GPU halves of moving a request) ----
 * ferry_owner_export writes an image of one owner's sets: per (layer, kv
 * head) set its LRU fill, order and tags, fp8 scales, and the bytes of its
 * resident slots compacted in LRU order.  ferry_owner_import makes `owner`'s
 * sets of this (or another) executor of the same geometry equal to the image:
 * same fill, order, tags and slot ids, same pool bytes; the owner's previous
 * blocks are forgotten.  `image` is device memory of at least
 * ferry_owner_image_bytes (256-byte aligned).  Only the first part of the
 * data area is used: the blocks resident in the owner, which is what crosses
 * a link when the request moves.  An image that does not match this
 * executor (geometry, dtype, slots, max_blocks) or is malformed latches
 * FERRY_EINVAL and leaves the affected sets empty.  Replaces the delta
 * migration of steal_from -- slot gather, transfer, slot scatter and
 * kv_handoff(carry) (src/runtime/wla_multigpu.cuh:154-171, 1367-1428,
 * 1970-1994); dropping a request's cache instead (kv_handoff without carry)
 * is ferry_sets_reset_owners. */
int ferry_owner_image_bytes(const ferry_ctx* ctx, uint64_t* bytes);
int ferry_owner_export(ferry_ctx* ctx, uint32_t owner, void* image, uint64_t image_bytes, void* stream);
int ferry_owner_import(ferry_ctx* ctx, uint32_t owner, const void* image, uint64_t image_bytes,
                       void* stream);
/* Member carry for prefix groups (group > 1): moving one request of a group
 * carries only the blocks that request alone touched.  ferry_owner_export_member
 * writes an image (same layout and size as above) of the blocks of `lane`'s
 * owner whose member mask is exactly lane's bit, per set in LRU order, with
 * their bytes and fp8 scales; blocks other members touched stay where they
 * are.  ferry_owner_import_member merges such an image into `lane`'s owner of
 * this (or another) executor: a block already resident gains lane's bit and
 * keeps its place; another becomes the most recent, taking the least recent
 * block's slot (which is evicted) when the set holds its capacity, else slot
 * fill.  Call ferry_members_join for the lane first, so that the capacity
 * counts it.  A whole-owner image, a geometry mismatch, a malformed image or
 * a set above its capacity latches FERRY_EINVAL; sets before the failure keep
 * their merged blocks.  Replaces kv_handoff(carry) with own_carry,
 * kv_handoff_owned and kv_live_owned (src/runtime/wla_multigpu.cuh:
 * 1901-1911, 1970-2016). */
int ferry_owner_export_member(ferry_ctx* ctx, uint32_t lane, void* image, uint64_t image_bytes,
                              void* stream);
int ferry_owner_import_member(ferry_ctx* ctx, uint32_t lane, const void* image, uint64_t image_bytes,
                              void* stream);

/* ---- bandwidth ceilings ----
 * Plain reads of the bytes the executor's kernels move, timed with HIP events
 * on `stream` over `iters` launches after one warm-up (synchronises):
 *   FERRY_PROBE_HBM_GATHER  the attention loads without the math: the k pool
 *                           slots of each of the n rows of `slots` ([n][k],
 *                           device); bytes = n*k*block_bytes
 *   FERRY_PROBE_HOST_READ   device-direct 16-byte reads of host-tier blocks
 *                           [0, n) by the fetch workgroups, no pool writes
 *   FERRY_PROBE_HOST_DMA    hipMemcpyAsync of host-tier blocks [0, n) into
 *                           device memory (the copy engines)
 *   FERRY_PROBE_HBM_COPY    a streaming copy of pool slots [0, n) into device
 *                           memory (non-temporal loads and stores, the owner
 *                           hand-off's ceiling); bytes = 2*n*block_bytes
 *   FERRY_PROBE_KTAB_READ   the mass selection's reads of the K table built by
 *                           ferry_ktiles_build: the records of blocks [0, n)
 *                           of every set, in its order and grid, no scores;
 *                           bytes = n_req*L*Hkv*n*(block_bytes/2)
 *   FERRY_PROBE_SUMS_READ   the Quest selection's reads of the summary table
 *                           built by ferry_summaries_build: the records of
 *                           blocks [0, n) of every set, in its lane pattern,
 *                           grid and LDS, no scores; bytes =
 *                           n_req*L*Hkv*n*2*128*element_size
 * `bytes` gets the bytes moved per launch, `ms` the mean launch time.  The
 * reference sweeps its host-staged channel the same way
 * (probe_host_staged_bandwidth, src/topo/topo.cpp:68-129). */
#define FERRY_PROBE_HBM_GATHER 0
#define FERRY_PROBE_HOST_READ 1
#define FERRY_PROBE_HOST_DMA 2
#define FERRY_PROBE_HBM_COPY 3
#define FERRY_PROBE_KTAB_READ 4
#define FERRY_PROBE_SUMS_READ 5
int ferry_bw_probe(ferry_ctx* ctx, int kind, const uint32_t* slots, uint64_t n, int iters,
                   uint64_t* bytes, float* ms, void* stream);

/* Counters (synchronises the device). */
int ferry_stats_get(ferry_ctx* ctx, ferry_stats* out);
int ferry_stats_reset(ferry_ctx* ctx);

/* ---- device queue self-test (bench_queue equivalent) ----
 * Producers push n_tasks unique ids through the MPMC ring (dq_push), consumers
 * pop them (dq_pop) and mark a seen[] map; returns popped count and duplicate
 * flag.  mode: 0 per-thread reservation, 1 wave-batched (64-slot) reservation.
 * Replaces pc_kernel/run_once (src/benches/bench_queue.cu:26-123). */
int ferry_queue_selftest(int device, uint64_t capacity, uint64_t n_tasks,
                         int producers, int consumers, int mode,
                         uint64_t* popped, uint64_t* duplicates, float* ms);

/* The ceiling of the ring's throughput: `threads` threads take `iters` tickets
 * each from one shared 64-bit word, by fetch-add per thread (kind 0), by the
 * relaxed load + compare-and-swap retry per thread that kPerThread's push
 * reservation uses (kind 1), or by that retry once per wavefront for its 64
 * lanes (kind 2), as the wave-batched push and every pop reserve.  Every pop
 * takes its ticket from the head word that way, so tickets/s of kind 2 bound
 * the pops/s of ferry_queue_selftest.  Returns the tickets taken
 * (threads * iters) and the kernel time.  No counterpart in the
 * reference: it is the ceiling bench_queue's Mops/s
 * (src/benches/bench_queue.cu:127-146) is compared against. */
int ferry_queue_ticket_probe(int device, int threads, int iters, int kind, uint64_t* tickets,
                             float* ms);

/* ---- synthetic workload generator (host) ----
 * Stateful per-(request, layer, kv head) top-k selection: keep each previous
 * block with probability `reuse`, complete to k distinct blocks by Zipf(s)
 * (or uniform) popularity draws over an owner-shared permutation.  The
 * reference's generator is replay_miss_stream (src/workloads/missstream.cuh:
 * 104-170); ferry_refgen_* below reproduces that one exactly. */
typedef struct ferry_selgen_config {
  int32_t n_req, group, n_layers, kv_heads, k;
  int32_t dist;          /* 0 uniform, 1 Zipf */
  double zipf_s;
  double reuse;
  int32_t prefix_blocks; /* blocks shared by a group (ids [0, prefix)) */
  int32_t pad;
  uint64_t seed;
} ferry_selgen_config;
typedef struct ferry_selgen ferry_selgen;
/* ctx_blocks: per-request context length in blocks (copied). */
int ferry_selgen_create(const ferry_selgen_config* cfg, const int32_t* ctx_blocks,
                        ferry_selgen** out);
int ferry_selgen_destroy(ferry_selgen* g);
/* Per-request reuse probabilities (array of n_req in [0, 1]; NULL restores
 * the configured reuse for every request). */
int ferry_selgen_set_reuse(ferry_selgen* g, const double* reuse);
/* Set block-id bound (use as ferry_config.max_blocks). */
int ferry_selgen_max_blocks(const ferry_selgen* g, int32_t* out);
/* Generate step `step` (steps must be generated in order) into host array
 * out [B][L][Hkv][k]. */
int ferry_selgen_step(ferry_selgen* g, int32_t step, uint32_t* out);
/* Per-request context lengths uniform in [lo, hi] blocks. */
int ferry_ctx_uniform(uint64_t seed, int32_t n_req, int32_t lo, int32_t hi,
                      int32_t* out);
/* Lane turnover (group 1 only).  ferry_selgen_admit puts request
 * `request_id` (< 65536) with a context of ctx_blocks (1 .. the largest
 * context given at creation) into `lane` from step `step` on: its draws are
 * keyed by (request id, steps since admission), it starts with no carried
 * selection, and a context shorter than k selects all its blocks and pads
 * the row with FERRY_EMPTY.  ferry_selgen_retire makes a lane produce rows of
 * FERRY_EMPTY until its next admission.  Replaces the request lifetime of
 * the reference's per-GPU executor: a request is resident from its arrival
 * until it has run len[r] steps (src/runtime/wla_multigpu.cuh:829-864,
 * src/workloads/missstream.cuh:68-81). */
int ferry_selgen_admit(ferry_selgen* g, int32_t lane, int32_t request_id, int32_t ctx_blocks,
                       int32_t step);
int ferry_selgen_retire(ferry_selgen* g, int32_t lane);
/* Prefix-group turnover.  A group's members share its prefix ids [0, prefix)
 * and each has a private range of (np - prefix) ids after them, np = the
 * owner's largest member context at creation.  ferry_selgen_set_private_ranges
 * makes `ranges` (>= group) such ranges per owner (read max_blocks after it);
 * ferry_selgen_admit_member puts request `request_id` (context <= np) into a
 * lane of the group from step `step` on, its private blocks in range
 * `private_range` (< ranges), so that successive requests of one lane select
 * different private ids.  For group 1 it is ferry_selgen_admit (range 0).
 * Replaces the group membership of the reference's C2 prefix affinity
 * (src/workloads/missstream.cuh:33-38, src/runtime/wla_multigpu.cuh:355-369). */
int ferry_selgen_set_private_ranges(ferry_selgen* g, int32_t ranges);
int ferry_selgen_admit_member(ferry_selgen* g, int32_t lane, int32_t request_id, int32_t ctx_blocks,
                              int32_t step, int32_t private_range);

/* ---- request arrivals and the per-GPU tick scheduler ----
 * Arrival times in ms of n requests (out_ms[n], non-decreasing, first
 * arrival after one gap):
 *   FERRY_ARRIVAL_STEADY   every gap_ms
 *   FERRY_ARRIVAL_BURSTY   request r after 40*gap_ms when r % 16 == 0, else
 *                          after 0.1*gap_ms (the reference's bursty rule,
 *                          src/runtime/wla_multigpu.cuh:497-501)
 *   FERRY_ARRIVAL_POISSON  exponential gaps of mean gap_ms
 *   FERRY_ARRIVAL_MMPP     Markov-modulated Poisson: two states of rate
 *                          1/gap_ms and ratio/gap_ms, exponential sojourns
 *                          of mean period_ms, starting in the slow state
 * Draws are counter-based hashes of (seed, index). */
#define FERRY_ARRIVAL_STEADY 0
#define FERRY_ARRIVAL_BURSTY 1
#define FERRY_ARRIVAL_POISSON 2
#define FERRY_ARRIVAL_MMPP 3
int ferry_arrivals(int kind, uint32_t n, double gap_ms, double period_ms, double ratio,
                   uint64_t seed, double* out_ms);

/* Tick scheduler of one GPU's executor: `lanes` batch lanes, n requests
 * with arrival times arrive_ms[n] and decode lengths len_steps[n] (>= 1).
 * Each ferry_sched_tick(now_ms) is one executor tick:
 *   1. every request resident in the previous tick has run one more step;
 *      those that reached len_steps leave their lanes (tick_end,
 *      src/runtime/wla_multigpu.cuh:834-864);
 *   2. requests with arrive_ms <= now_ms join a FIFO in arrival order (ties
 *      by id) and take free lanes, lowest lane first.  With policy
 *      FERRY_SCHED_PINNED request r only ever runs in lane r % lanes (one
 *      FIFO per lane): lanes >= n gives every request its own lane, as the
 *      reference's per-request hot caches do, and a request stays in its
 *      prefix group's lanes;
 *   3. out: lane_req[lanes] = request in each lane (-1 idle),
 *      lane_step[lanes] = that request's step index in this tick,
 *      admitted[0..*n_admitted) = lanes that received a new request,
 *      retired[0..*n_retired) = lanes whose request left in step 1 (and
 *      were not refilled), *n_resident, *done = 1 once every request has
 *      finished (then nothing is resident).
 * The reference's exec loop runs every resident request once per tick
 * (src/runtime/wla_multigpu.cuh:2610-2665); its residency is unbounded, which
 * is lanes >= n here. */
#define FERRY_SCHED_FIFO 0
#define FERRY_SCHED_PINNED 1
typedef struct ferry_sched ferry_sched;
int ferry_sched_create(int32_t lanes, int32_t policy, uint32_t n, const double* arrive_ms,
                       const int32_t* len_steps, ferry_sched** out);
int ferry_sched_destroy(ferry_sched* s);
int ferry_sched_tick(ferry_sched* s, double now_ms, int32_t* lane_req, int32_t* lane_step,
                     int32_t* admitted, int32_t* n_admitted, int32_t* retired,
                     int32_t* n_retired, int32_t* n_resident, int32_t* done);
/* Arrival time of the next request not yet admitted (+inf if none), and the
 * per-request admission tick and completion tick (-1 until known). */
int ferry_sched_next_arrival(const ferry_sched* s, double* ms);
int ferry_sched_request_ticks(const ferry_sched* s, int32_t* admit_tick, int32_t* done_tick);

/* ---- FMT1 selection traces ----
 * tools/capture_miss_trace.py records real top-k selections as FMT1 (header
 * :27-38: "FMT1", version 1, R, steps, layers, page_tokens, block_tokens,
 * kv_heads, head_dim, sel_pages as u32; then per (request, step, layer) a u16
 * count and count u32 chained-hash block ids).  ferry_trace_load reads one:
 * raw ids are renamed to dense ids in order of first appearance over the
 * whole trace, as load_miss_trace does (src/workloads/miss_trace.cuh:75-185).
 * out_ids (NULL: header and counts only) gets R*steps*layers*sel_blocks ids
 * in (r, s, l, k) order, sel_blocks = sel_pages*page_tokens/block_tokens.  A
 * record with fewer ids is FERRY_EINVAL when `strict` (the reference refuses
 * it, :123-129) and is padded with FERRY_EMPTY otherwise.  Bad files return
 * FERRY_EINVAL with the reason in ferry_last_error(); nothing exits. */
typedef struct ferry_trace_info {
  uint32_t requests, steps, layers, page_tokens, block_tokens, kv_heads, head_dim, sel_pages;
  uint32_t sel_blocks;         /* ids per (request, step, layer) record */
  uint32_t short_records;      /* records padded with FERRY_EMPTY */
  uint64_t unique_blocks;      /* distinct raw ids; dense ids are [0, unique_blocks) */
  uint64_t max_blocks_per_req; /* most distinct ids one request selects */
} ferry_trace_info;
int ferry_trace_load(const char* path, int strict, ferry_trace_info* info, uint32_t* out_ids,
                     uint64_t capacity);

/* Reference generator: the selections replay_miss_stream draws
 * (src/workloads/missstream.cuh:104-133, std::mt19937_64(seed)) for
 * R requests x S steps x L layers x sel, in the reference's (r, s, l, k)
 * event order, as u32 block ids in out[R*S*L*sel].  The hit/miss flags are
 * not produced here: run them through ferry_fetch_step with
 * FERRY_LRU_SERIAL, group 1, kv_heads 1, k = sel, slots_per_set = hot. */
int ferry_refgen_selections(int32_t R, int32_t L, int32_t S, int32_t sel,
                            uint64_t seed, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
