// runtime.hip -- executor context and the C-ABI (include/ferry_amd.h).
//
// The context owns every buffer of the path: the HBM slot pool, per-set LRU
// state, the device miss ring and the pinned host tier.  Entry points launch
// on the caller's stream and never synchronise, except the explicitly
// synchronous ones (stats, state copies, the queue self-test).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <initializer_list>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "common.hpp"
#include "errors.hpp"
#include "kernels.hpp"
#include "../../include/ferry/gpu_bounded_queue.hpp"

using namespace ferry_amd;

namespace ferry_amd {
__global__ void k_queue_pc(ferry::DeviceQueue* q, uint64_t per_thread, uint32_t n_prod_blocks,
                           uint32_t* seen, unsigned long long* popped, unsigned long long* dups,
                           int* done, int* prod_blocks_done, ferry::ReservationMode mode);
}

namespace {

thread_local std::string g_err = "";

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

}  // namespace

int ferry_amd::report(int code, const std::string& msg) { return fail(code, msg); }

namespace {

#define HIPC(expr)                                                                         \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return fail(e_ == hipErrorOutOfMemory ? FERRY_ENOMEM : FERRY_EHIP,                   \
                  std::string(#expr) + ": " + hipGetErrorString(e_) + " (" __FILE__ ":" + \
                      std::to_string(__LINE__) + ")");                                     \
  } while (0)

int esize_of(int dtype) { return dtype == FERRY_F32 ? 4 : (dtype == FERRY_FP8_E4M3 ? 1 : 2); }

float value_mult(double std_) { return (float)(std_ / (65536.0 / std::sqrt(3.0))); }

}  // namespace

// Workspace of ferry_select_mass_noalloc: one array per GPU, part of the
// library's code object, so that entry point allocates nothing.  Each GPU the
// library runs on holds it until the process ends.  Host code never passes
// the array's name to a kernel (on the host it is a stand-in, not a device
// address): ferry_ctx_create resolves each device's own address once, with
// that device current, and the entry point uses that address.
static constexpr size_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
std::mutex g_scratch_mu;
std::map<int, float*> g_scratch_ptr;  // device -> address of its `scratch`

// The calling thread's current device must be `device`.
int resolve_scratch(int device, float** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(device);
  if (it == g_scratch_ptr.end()) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(FERRY_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    it = g_scratch_ptr.emplace(device, static_cast<float*>(p)).first;
  }
  *out = it->second;
  return FERRY_OK;
}
}  // namespace

struct ferry_ctx {
  ferry_config cfg{};
  int device = 0;
  Geo g{};
  uint8_t* pool = nullptr;
  float* pool_scales = nullptr;
  SetState st{};
  ferry_miss* ring_entries = nullptr;
  uint64_t* ring_state = nullptr;
  ferry_miss* ring_entries2 = nullptr;  // second ring: decode_step alternates layer ranges
  uint64_t* ring_state2 = nullptr;
  uint32_t* ring_seg = nullptr;
  uint32_t* ring_cap = nullptr;
  uint32_t* worker_of_set = nullptr;
  unsigned long long* stats = nullptr;
  unsigned long long* sel_counts = nullptr;  // [kSelCounters * kSelStride]
  // [3]: blocks fetched and blocks the prefix-group attention read in this
  // step (moved to pend_host and cleared by k_step_close), and the count of
  // closed steps
  unsigned long long* step_acc = nullptr;
  // mapped pinned [3]: the last closed step's two counts and a sequence word
  // (odd while k_step_close rewrites them)
  unsigned long long* pend_host = nullptr;
  unsigned long long* pend_dev = nullptr;    // ... its device address
  double pol_min_mb = 32.0, pol_max_mb = 512.0, pol_target = 8.0;  // adaptive layer chunking
  uint32_t* done = nullptr;
  int* err = nullptr;
  uint8_t* host = nullptr;      // host pointer of the pinned tier
  bool host_owned = true;       // false once the caller registered its own tier
  uint8_t* host_dev = nullptr;  // its device-visible address
  float* host_scales = nullptr;
  float* host_scales_dev = nullptr;
  int lru_wpb = 1;
  size_t lru_lds = 0;
  uint64_t steps = 0;
  std::vector<hipEvent_t> events;   // layer-chunk pipeline of ferry_decode_step: fetch done
  std::vector<hipEvent_t> booked;   // ... and bookkeeping done
  int attn_waves = 0;              // wavefronts per attention workgroup (FERRY_ATTN_WAVES), 0 = default
  int cus = 256;                   // compute units of the device
  int mass_resident = 0;           // k_mass_units workgroups resident at once (0: not yet asked)
  int mass_lds = -1;               // k_mass_units keeps block log-sums in LDS (-1: not yet decided)
  int group_waves_env = 0;         // prefix-group kernel wavefronts (FERRY_GROUP_WAVES=4|8), 0 = by launch
  int fetch_waves = 0;             // wavefronts per fetch workgroup (FERRY_FETCH_WAVES: 1, 2, 4; 0 = by rule)
  int fetch_prio = 1;              // fetch wavefronts issue first (FERRY_FETCH_PRIO=0: not)
  uint32_t steal_chunk = 8;        // most entries one steal takes (FERRY_STEAL_CHUNK)
  int thief_waves = 1;             // wavefronts per fetch workgroup that steal (FERRY_THIEF_WAVES)
  int steal_inflight = 2;          // stolen blocks in flight per thief (FERRY_STEAL_INFLIGHT)
  int attn_loads = 0;              // K/V loads (FERRY_ATTN_LOADS): 0 = by plan, 1 = nt, 2 = temporal
  bool attn_grouped = true;        // FERRY_ATTN_AUTO may pick the prefix-group kernel (FERRY_ATTN_GROUPED)
  uint32_t* probe_sink = nullptr;  // bandwidth probes: one word per row / wavefront
  size_t probe_sink_words = 0;
  uint8_t* probe_dst = nullptr;    // bandwidth probes: DMA destination
  size_t probe_dst_bytes = 0;
  uint8_t* sums = nullptr;         // top-k selection: K min/max records [sum_blocks][2][D]
  float* sum_scales = nullptr;     // ... and their K scales (fp8)
  uint64_t sum_blocks = 0;         // records; block (set, b) uses (set*max_blocks + b) mod this
  uint8_t* ktab = nullptr;         // mass selection: K halves of host blocks [kt_records][T][D]
  float* ktab_scales = nullptr;    // ... and their K scales (fp8)
  uint64_t kt_records = 0;         // records, addressed like the summaries
  float* mass_ws = nullptr;        // per-workgroup (max, sum) of every block and query head
  int kt_perm = 0;                 // K table words lane-transposed for the matrix-core loads
  float* scratch_dev = nullptr;    // this device's address of the static `scratch` array
  uint32_t* lane_live = nullptr;   // [n_req] 1 while the lane's request is a resident member
  uint32_t* trim_gen = nullptr;    // [n_owners] last ferry_members_leave that shrank the owner
  uint32_t member_calls = 0;       // ferry_members_leave calls so far (trim generations)

  Ring ring(int which = 0) const {
    Ring r;
    r.entries = which ? ring_entries2 : ring_entries;
    r.state = which ? ring_state2 : ring_state;
    r.seg = ring_seg;
    r.cap = ring_cap;
    r.worker_of_set = worker_of_set;
    return r;
  }
};

namespace {

// Whether the prefix-group attention kernel (k_attn_group) can run this
// geometry: every wavefront holds all group * G query columns (at most
// kGroupMaxTiles tiles of 16), the workgroup's LDS fits one CU, and the
// per-slot member masks plus the list's scratch (a slot per selection and a
// count per member) fit the block rings while the list is built.
bool group_attn_fits(const ferry_config* c) {
  const int G = c->q_heads / c->kv_heads;
  if (c->group < 2 || G < 2 || c->dtype == FERRY_F32 || c->group * G > 16 * kGroupMaxTiles)
    return false;
  const long gk = (long)c->group * c->k;
  const int ntile = (c->group * G + 15) / 16;
  return attn_group_lds_bytes(c->dtype, ntile, gk, group_waves(c->dtype)) <= (size_t)kGroupMaxLds &&
         4 * ((long)c->slots_per_set + gk + c->group) <=
             (long)group_waves(c->dtype) * group_ring_bytes(c->dtype);
}

int validate(const ferry_config* c) {
  if (!c) return fail(FERRY_EINVAL, "null config");
  if (c->n_req < 1 || c->group < 1 || c->n_layers < 1 || c->kv_heads < 1 || c->q_heads < 1 ||
      c->k < 1 || c->slots_per_set < 1 || c->max_blocks < 1 || c->host_blocks < 1)
    return fail(FERRY_EINVAL, "sizes must be positive");
  if (c->k > kMaxTopK) return fail(FERRY_EINVAL, "k must be <= 1024");
  if (c->q_heads % c->kv_heads) return fail(FERRY_EINVAL, "q_heads must be a multiple of kv_heads");
  const int grp = c->q_heads / c->kv_heads;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8)
    return fail(FERRY_EINVAL, "q_heads/kv_heads must be 1, 2, 4 or 8");
  if (c->head_dim != 128) return fail(FERRY_EINVAL, "head_dim must be 128");
  if (c->block_tokens != 16) return fail(FERRY_EINVAL, "block_tokens must be 16");
  if (c->dtype < FERRY_F32 || c->dtype > FERRY_FP8_E4M3) return fail(FERRY_EINVAL, "bad dtype");
  if (c->lru_mode != FERRY_LRU_STEP && c->lru_mode != FERRY_LRU_SERIAL)
    return fail(FERRY_EINVAL, "bad lru_mode");
  if (c->assign != FERRY_ASSIGN_SPREAD && c->assign != FERRY_ASSIGN_AFFINITY)
    return fail(FERRY_EINVAL, "bad assign");
  if (c->attn != FERRY_ATTN_AUTO && c->attn != FERRY_ATTN_VALU && c->attn != FERRY_ATTN_MFMA &&
      c->attn != FERRY_ATTN_GROUP)
    return fail(FERRY_EINVAL, "bad attn");
  if (c->attn == FERRY_ATTN_MFMA &&
      (c->dtype == FERRY_F32 || (grp < 2 && c->dtype != FERRY_FP8_E4M3)))
    return fail(FERRY_EINVAL,
                "the MFMA attention kernel needs 16/8-bit KV and q_heads/kv_heads >= 2 (any for fp8)");
  if (c->attn == FERRY_ATTN_GROUP && (grp < 2 || c->dtype == FERRY_F32))
    return fail(FERRY_EINVAL, "the prefix-group attention kernel needs q_heads/kv_heads >= 2 and 16/8-bit KV");
  if (c->attn == FERRY_ATTN_GROUP && !group_attn_fits(c))
    return fail(FERRY_EINVAL,
                "the prefix-group attention kernel needs group > 1, group * q_heads/kv_heads <= 64, "
                "its LDS (rings, queries, group * k list entries) within 160 KiB and "
                "slots_per_set + group * k within its rings");
  if (c->fetch_workers < 0) return fail(FERRY_EINVAL, "fetch_workers < 0");
  if (c->cap_mode != FERRY_CAP_GROUP && c->cap_mode != FERRY_CAP_PER_MEMBER)
    return fail(FERRY_EINVAL, "bad cap_mode");
  if (c->cap_mode == FERRY_CAP_PER_MEMBER && c->slots_per_set % c->group)
    return fail(FERRY_EINVAL, "per-member capacity needs slots_per_set to be a multiple of group");
  if (c->group > 32) return fail(FERRY_EINVAL, "group must be <= 32 (one mask bit per member)");
  if ((uint64_t)c->max_blocks >= (uint64_t)kPend) return fail(FERRY_EINVAL, "max_blocks too large");
  return FERRY_OK;
}

template <typename T>
int dalloc(T** p, size_t n) {
  HIPC(hipMalloc((void**)p, std::max<size_t>(n, 1) * sizeof(T)));
  return FERRY_OK;
}

void release(ferry_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  void* dev[] = {c->pool, c->pool_scales, c->st.fill, c->st.ord, c->st.tag, c->st.map,
                 c->st.members, c->st.own, c->lane_live, c->trim_gen,
                 c->ring_entries, c->ring_state, c->ring_entries2, c->ring_state2,
                 c->ring_seg, c->ring_cap, c->worker_of_set,
                 c->stats, c->sel_counts, c->step_acc, c->done, c->err, c->probe_sink,
                 c->probe_dst, c->sums, c->sum_scales, c->ktab, c->ktab_scales, c->mass_ws};
  for (void* p : dev)
    if (p) (void)hipFree(p);
  if (c->pend_host) (void)hipHostFree(c->pend_host);
  if (c->host_owned) {
    if (c->host) (void)hipHostFree(c->host);
    if (c->host_scales) (void)hipHostFree(c->host_scales);
  }
  for (hipEvent_t e : c->events) (void)hipEventDestroy(e);
  for (hipEvent_t e : c->booked) (void)hipEventDestroy(e);
  delete c;
}

// Spread assignment hashes the set id (lowbias32, C. Wellons' published
// 32-bit integer hash).  Set id modulo the worker count put every owner's
// sets of one layer range on the same few workers whenever L * Hkv is a
// multiple of it, so a layer chunk's misses filled a quarter of the deques.
uint32_t spread_hash(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

int check_ctx(const ferry_ctx* c) { return c ? FERRY_OK : fail(FERRY_EINVAL, "null context"); }

}  // namespace

namespace {

struct AttnArgs {
  Geo g;
  const float* q;
  const uint32_t* slots;
  const uint8_t* pool;
  const float* pool_scales;
  float* out;
  float qscale;
  int l0, nl;
  int* err;
  unsigned long long* attn_blocks;  // the group kernel adds the blocks it read (or null)
};

// Which attention kernel runs and how many wavefronts share one (request,
// layer, kv head) row.  MFMA for GQA groups of 16/8-bit KV unless the config
// asks for the VALU kernel.  Four wavefronts per row; eight (FERRY_ATTN_WAVES=8)
// measured the same on MI355X.  K/V loads are non-temporal unless requests
// share prefix-group sets (group > 1), whose blocks the member rows of one
// launch re-read from cache; FERRY_ATTN_LOADS=nt|temporal overrides.
// Prefix groups that fit it run the group kernel instead (one workgroup per
// group set, each distinct block read once), unless the config asks for the
// per-row MFMA kernel or FERRY_ATTN_GROUPED=0 is set.
struct AttnPlan {
  bool mfma, nt, grouped;
  int dtype, G, waves, tiles, cus;
  int group_w;  // FERRY_GROUP_WAVES: 4 or 8 forced, else by launch size
};

AttnPlan attn_plan(const ferry_ctx* ctx) {
  const Geo& g = ctx->g;
  AttnPlan p;
  p.dtype = g.dtype;
  p.G = g.Hq / g.Hkv;
  p.mfma = g.dtype != FERRY_F32 && (p.G >= 2 || g.dtype == FERRY_FP8_E4M3) &&
           ctx->cfg.attn != FERRY_ATTN_VALU;
  p.grouped = ctx->cfg.attn == FERRY_ATTN_GROUP ||
              (ctx->cfg.attn == FERRY_ATTN_AUTO && ctx->attn_grouped && group_attn_fits(&ctx->cfg));
  p.waves = 4;
  if (ctx->attn_waves == 8) p.waves = 8;
  p.tiles = 0;
  if (p.grouped) {  // tiles of 16 query columns held by every wavefront
    p.waves = group_waves(g.dtype);
    p.tiles = (g.group * p.G + 15) / 16;
  }
  p.nt = ctx->attn_loads ? ctx->attn_loads == 1 : g.group == 1;
  p.cus = ctx->cus;
  p.group_w = ctx->group_waves_env;
  return p;
}

template <int DT, int G, int W>
void launch_valu(const AttnPlan& p, const dim3& grid, hipStream_t s, const AttnArgs& a) {
  if (p.nt)
    hipLaunchKernelGGL((k_attn<DT, G, W, true>), grid, dim3(W * 64), 0, s, a.g, a.q, a.slots,
                       a.pool, a.pool_scales, a.out, a.qscale, a.l0, a.nl, a.err);
  else
    hipLaunchKernelGGL((k_attn<DT, G, W, false>), grid, dim3(W * 64), 0, s, a.g, a.q, a.slots,
                       a.pool, a.pool_scales, a.out, a.qscale, a.l0, a.nl, a.err);
}
template <int DT, int G, int W>
void launch_mfma(const AttnPlan& p, const dim3& grid, hipStream_t s, const AttnArgs& a) {
  if (p.nt)
    hipLaunchKernelGGL((k_attn_mfma<DT, G, W, true>), grid, dim3(W * 64), 0, s, a.g, a.q,
                       a.slots, a.pool, a.pool_scales, a.out, a.qscale, a.l0, a.nl, a.err);
  else
    hipLaunchKernelGGL((k_attn_mfma<DT, G, W, false>), grid, dim3(W * 64), 0, s, a.g, a.q,
                       a.slots, a.pool, a.pool_scales, a.out, a.qscale, a.l0, a.nl, a.err);
}
template <int DT, int G, int NT, int W>
void launch_group_w(const dim3& grid, size_t lds, hipStream_t s, const AttnArgs& a) {
  // more than the default 64 KiB of dynamic LDS: allowed once per instance and
  // device (the caller has made the context's device current)
  static std::atomic<uint64_t> allowed{0};
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && !((allowed.load() >> dev) & 1u) &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_group<DT, G, NT, W>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kGroupMaxLds) == hipSuccess)
    allowed.fetch_or(1ull << dev);
  hipLaunchKernelGGL((k_attn_group<DT, G, NT, W>), grid, dim3(W * 64), lds, s, a.g, a.q, a.slots,
                     a.pool, a.pool_scales, a.out, a.qscale, a.l0, a.nl, a.err, a.attn_blocks);
}
// Wavefronts per workgroup of a prefix-group launch over `sets` group sets:
// eight where the launch has no more sets than the GPU has CUs and the wider
// LDS fits one CU, four otherwise; `force` (4 or 8) overrides the launch rule.
int group_launch_waves(int dtype, int ntile, long gk, long sets, int cus, int force) {
  const bool want = force ? force == kGroupWideWaves : sets <= (long)cus;
  return want && attn_group_lds_bytes(dtype, ntile, gk, kGroupWideWaves) <= (size_t)kGroupMaxLds
             ? kGroupWideWaves
             : group_waves(dtype);
}
template <int DT, int G, int NT>
void launch_group(const dim3& grid, int cus, int force, hipStream_t s, const AttnArgs& a) {
  const long gk = (long)a.g.group * a.g.k;
  if (group_launch_waves(DT, NT, gk, grid.x, cus, force) == kGroupWideWaves)
    launch_group_w<DT, G, NT, kGroupWideWaves>(
        grid, attn_group_lds_bytes(DT, NT, gk, kGroupWideWaves), s, a);
  else
    launch_group_w<DT, G, NT, group_waves(DT)>(
        grid, attn_group_lds_bytes(DT, NT, gk, group_waves(DT)), s, a);
}
template <int DT, int G>
void launch_g(const AttnPlan& p, const dim3& grid, hipStream_t s, const AttnArgs& a) {
  if constexpr (DT != FERRY_F32 && G >= 2) {
    if (p.grouped) {
      const dim3 ggrid((unsigned)(a.g.n_owners * a.nl * a.g.Hkv));
      switch (p.tiles) {
        case 1: launch_group<DT, G, 1>(ggrid, p.cus, p.group_w, s, a); return;
        case 2: launch_group<DT, G, 2>(ggrid, p.cus, p.group_w, s, a); return;
        case 3: launch_group<DT, G, 3>(ggrid, p.cus, p.group_w, s, a); return;
        default: launch_group<DT, G, 4>(ggrid, p.cus, p.group_w, s, a); return;
      }
    }
  }
  if constexpr (DT != FERRY_F32 && (G >= 2 || DT == FERRY_FP8_E4M3)) {
    if (p.mfma) {
      switch (p.waves) {
        case 8: launch_mfma<DT, G, 8>(p, grid, s, a); return;
        default: launch_mfma<DT, G, 4>(p, grid, s, a); return;
      }
    }
  }
  switch (p.waves) {
    case 8: launch_valu<DT, G, 8>(p, grid, s, a); return;
    default: launch_valu<DT, G, 4>(p, grid, s, a); return;
  }
}
template <int DT>
void launch_dt(const AttnPlan& p, const dim3& grid, hipStream_t s, const AttnArgs& a) {
  switch (p.G) {
    case 1: launch_g<DT, 1>(p, grid, s, a); return;
    case 2: launch_g<DT, 2>(p, grid, s, a); return;
    case 4: launch_g<DT, 4>(p, grid, s, a); return;
    default: launch_g<DT, 8>(p, grid, s, a); return;
  }
}
void launch_attn(const AttnPlan& p, const dim3& grid, hipStream_t s, const AttnArgs& a) {
  switch (p.dtype) {
    case FERRY_F32: launch_dt<FERRY_F32>(p, grid, s, a); return;
    case FERRY_F16: launch_dt<FERRY_F16>(p, grid, s, a); return;
    case FERRY_BF16: launch_dt<FERRY_BF16>(p, grid, s, a); return;
    default: launch_dt<FERRY_FP8_E4M3>(p, grid, s, a); return;
  }
}

}  // namespace

namespace {

int bookkeep_ring(ferry_ctx* ctx, int32_t l0, int32_t nl, const uint32_t* sel, uint32_t* slots,
                  uint32_t* miss_count, ferry_miss* misses, uint8_t* miss_flag, void* stream,
                  int which);
int drain_ring(ferry_ctx* ctx, void* stream, int which);

}  // namespace

namespace {
// A buffer a kernel reads or writes must be memory HIP knows: device, managed
// or pinned host memory.  Pageable host memory would fault the kernel, so it
// is refused here.  Sizes cannot be checked (the entry points take bare
// pointers); the Python mirror checks them.
int check_buf(const void* p, const char* name) {
  if (!p) return fail(FERRY_EINVAL, std::string("null ") + name);
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess || a.type == hipMemoryTypeUnregistered) {
    (void)hipGetLastError();
    return fail(FERRY_EINVAL, std::string(name) +
                                  " is not device-accessible memory (device, managed or pinned host)");
  }
  return FERRY_OK;
}

// check_buf over several buffers, in order
int check_bufs(std::initializer_list<std::pair<const void*, const char*>> bufs) {
  for (const auto& b : bufs)
    if (int rc = check_buf(b.first, b.second)) return rc;
  return FERRY_OK;
}

// Attention of layers [l0, l0 + nl).  attn_blocks (decode steps only): the
// prefix-group kernel adds the distinct blocks it reads there, which the next
// step's layer chunking takes as the attention's bytes.
int decode_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q, const uint32_t* slots,
                  float* out, void* stream, unsigned long long* attn_blocks) {
  if (int rc = check_bufs({{q, "q"}, {slots, "slots"}, {out, "out"}})) return rc;
  const Geo& g = ctx->g;
  if (l0 < 0 || nl < 1 || l0 + nl > g.L) return fail(FERRY_EINVAL, "bad layer range");
  HIPC(hipSetDevice(ctx->device));
  const dim3 grid((unsigned)(g.n_req * nl * g.Hkv));
  const float qscale = (float)(1.4426950408889634 / std::sqrt((double)g.D));
  const AttnArgs a{g, q, slots, ctx->pool, ctx->pool_scales, out, qscale, l0, nl, ctx->err,
                   attn_blocks};
  const AttnPlan p = attn_plan(ctx);
  launch_attn(p, grid, (hipStream_t)stream, a);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

// A record table and its fp8 scales, allocated together or not at all: on a
// failure nothing stays allocated and the caller keeps no table (a table whose
// record count is 0 would send the selection's record index through mod 0).
int alloc_table(uint64_t bytes, uint64_t scale_count, uint8_t** table, float** scales) {
  *table = nullptr;
  *scales = nullptr;
  if (hipMalloc(table, bytes) != hipSuccess) {
    (void)hipGetLastError();
    *table = nullptr;
    return fail(FERRY_ENOMEM, "record table allocation failed (" + std::to_string(bytes) + " B)");
  }
  if (scale_count && hipMalloc(scales, scale_count * 4) != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(*table);
    *table = nullptr;
    *scales = nullptr;
    return fail(FERRY_ENOMEM, "record scale allocation failed");
  }
  return FERRY_OK;
}

// Device buffers and events of a one-off measurement, released on every
// return path (hipFree waits for the device first).
struct Scratch {
  std::vector<void*> bufs;
  std::vector<hipEvent_t> events;
  Scratch() = default;
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  ~Scratch() {
    for (void* p : bufs) (void)hipFree(p);
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
  }
};
}  // namespace

extern "C" {

const char* ferry_last_error(void) { return g_err.c_str(); }
const char* ferry_version(void) { return "ferry_amd 0.1 (gfx950)"; }

int ferry_ctx_create(const ferry_config* cfg, int device, ferry_ctx** out) {
  if (!out) return fail(FERRY_EINVAL, "null out");
  *out = nullptr;
  int rc = validate(cfg);
  if (rc) return rc;
  HIPC(hipSetDevice(device));
  ferry_ctx* c = new ferry_ctx();
  c->cfg = *cfg;
  if (const char* e = std::getenv("FERRY_ATTN_WAVES")) c->attn_waves = std::atoi(e);
  if (const char* e = std::getenv("FERRY_GROUP_WAVES")) c->group_waves_env = std::atoi(e);
  if (const char* e = std::getenv("FERRY_FETCH_WAVES")) {
    const int v = std::atoi(e);
    c->fetch_waves = v == 1 || v == 2 ? v : 4;
  }
  if (const char* e = std::getenv("FERRY_FETCH_PRIO")) c->fetch_prio = std::atoi(e) != 0;
  if (const char* e = std::getenv("FERRY_STEAL_CHUNK")) c->steal_chunk = (uint32_t)std::max(1, std::atoi(e));
  if (const char* e = std::getenv("FERRY_THIEF_WAVES")) c->thief_waves = std::max(1, std::atoi(e));
  if (const char* e = std::getenv("FERRY_STEAL_INFLIGHT")) c->steal_inflight = std::max(1, std::atoi(e));
  if (const char* e = std::getenv("FERRY_ATTN_GROUPED")) c->attn_grouped = std::atoi(e) != 0;
  if (const char* e = std::getenv("FERRY_ATTN_LOADS"))
    c->attn_loads = std::string(e) == "nt" ? 1 : (std::string(e) == "temporal" ? 2 : 0);
  c->device = device;
  if ((rc = resolve_scratch(device, &c->scratch_dev))) {
    delete c;
    return rc;
  }
  Geo& g = c->g;
  g.n_req = cfg->n_req;
  g.group = cfg->group;
  g.L = cfg->n_layers;
  g.Hkv = cfg->kv_heads;
  g.Hq = cfg->q_heads;
  g.D = cfg->head_dim;
  g.T = cfg->block_tokens;
  g.k = cfg->k;
  g.C = cfg->slots_per_set;
  g.max_blocks = cfg->max_blocks;
  g.n_owners = (cfg->n_req + cfg->group - 1) / cfg->group;
  g.n_sets = g.n_owners * g.L * g.Hkv;
  g.pool_slots = 0;
  g.max_sel = cfg->group * cfg->k;
  g.dtype = cfg->dtype;
  g.esize = esize_of(cfg->dtype);
  g.bb = 2ull * g.T * g.D * g.esize;
  g.host_blocks = cfg->host_blocks;
  g.pool_slots = (uint64_t)g.n_sets * (uint64_t)g.C;
  g.cap_mode = cfg->cap_mode;
  g.member_slots = g.C / g.group;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus < 1)
    cus = 256;
  c->cus = cus;
  // One fetch workgroup per 4 CUs by default: 256 wavefronts with a block each
  // in flight fill the host link (57.5 GB/s at the 7B shape, against 55 GB/s
  // with 2 per CU), and the CUs they leave idle run the attention that
  // overlaps the fetch (the 7B step: 64.2 ms, against 67-68 ms).
  g.workers = cfg->fetch_workers > 0 ? cfg->fetch_workers : std::max(1, cus / 4);
  // Wavefronts per fetch workgroup.  About 256 copying wavefronts with one
  // block in flight each fill the link; more only hold host reads in the
  // memory system's queues, ahead of the loads of the kernels the fetch
  // overlaps (measured with 304 workgroups of 4: the attention and the
  // bookkeeping running beside a stealing drain took 4-8 times their time
  // alone).  With stealing every wavefront can reach any deque, so the count
  // follows the link: 256 / workgroups, 1 to 4.  Without stealing a deque's
  // own wavefronts are all that copy it: 4.
  if (c->fetch_waves == 0) {
    c->fetch_waves = 4;
    if (cfg->steal)
      while (c->fetch_waves > 1 && g.workers * c->fetch_waves > 256) c->fetch_waves >>= 1;
  }
  if ((uint64_t)g.n_sets * (uint64_t)g.C >= 0xFFFFFFFFull ||
      (uint64_t)g.n_sets * (uint64_t)g.max_sel >= 0xFFFFFFFFull) {
    delete c;
    return fail(FERRY_EINVAL, "too many slots or selections for 32-bit ids");
  }
  // bookkeeping launch shape: waves per workgroup bounded by 64 KiB of LDS
  const size_t per_wave = lru_lds_words(g) * 4;
  if (per_wave > 65536) {
    delete c;
    return fail(FERRY_EINVAL, "slots_per_set/group*k too large for the bookkeeping LDS budget");
  }
  const size_t wave_lds = lru_lds_wave_words(g) * 4;  // with the staged selections
  c->lru_wpb = 4;
  while (c->lru_wpb > 1 && wave_lds * c->lru_wpb > 65536) c->lru_wpb >>= 1;
  c->lru_lds = wave_lds * c->lru_wpb;

  const size_t nslots = (size_t)g.n_sets * g.C;
#define TRY(x)        \
  do {                \
    rc = (x);         \
    if (rc) {         \
      release(c);     \
      return rc;      \
    }                 \
  } while (0)
  TRY(dalloc(&c->pool, nslots * g.bb));
  if (g.dtype == FERRY_FP8_E4M3) TRY(dalloc(&c->pool_scales, nslots * 2));
  TRY(dalloc(&c->st.fill, g.n_sets));
  TRY(dalloc(&c->st.ord, nslots));
  TRY(dalloc(&c->st.tag, nslots));
  TRY(dalloc(&c->st.map, (size_t)g.n_sets * g.max_blocks));
  TRY(dalloc(&c->st.members, g.n_owners));
  if (g.group > 1) TRY(dalloc(&c->st.own, nslots));
  TRY(dalloc(&c->lane_live, g.n_req));
  TRY(dalloc(&c->trim_gen, g.n_owners));
  // ring: worker segments sized for every miss their sets can produce
  const int W = g.workers;
  std::vector<uint32_t> wos(g.n_sets), cnt(W, 0), seg(W, 0), cap(W, 0);
  for (int s = 0; s < g.n_sets; ++s) {
    const int owner = s / (g.L * g.Hkv);
    wos[s] = cfg->assign == FERRY_ASSIGN_AFFINITY ? (uint32_t)(owner % W)
                                                  : spread_hash((uint32_t)s) % (uint32_t)W;
    cnt[wos[s]]++;
  }
  uint64_t total = 0;
  for (int w = 0; w < W; ++w) {
    seg[w] = (uint32_t)total;
    cap[w] = cnt[w] * (uint32_t)g.max_sel;
    total += cap[w];
  }
  TRY(dalloc(&c->ring_entries, total));
  TRY(dalloc(&c->ring_state, (size_t)W * kStateStride));
  TRY(dalloc(&c->ring_entries2, total));
  TRY(dalloc(&c->ring_state2, (size_t)W * kStateStride));
  TRY(dalloc(&c->ring_seg, W));
  TRY(dalloc(&c->ring_cap, W));
  TRY(dalloc(&c->worker_of_set, g.n_sets));
  TRY(dalloc(&c->stats, kStatCount));
  TRY(dalloc(&c->sel_counts, (size_t)kSelCounters * kSelStride));
  TRY(dalloc(&c->step_acc, 3));
  TRY(dalloc(&c->done, 1));
  TRY(dalloc(&c->err, 1));
#define HIPT(x)                                                                        \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      release(c);                                                                      \
      return fail(FERRY_EHIP, std::string(#x) + ": " + hipGetErrorString(e_));         \
    }                                                                                  \
  } while (0)
  HIPT(hipMemcpy(c->ring_seg, seg.data(), W * 4, hipMemcpyHostToDevice));
  HIPT(hipMemcpy(c->ring_cap, cap.data(), W * 4, hipMemcpyHostToDevice));
  HIPT(hipMemcpy(c->worker_of_set, wos.data(), (size_t)g.n_sets * 4, hipMemcpyHostToDevice));
  HIPT(hipMemset(c->ring_state, 0, (size_t)W * kStateStride * 8));
  HIPT(hipMemset(c->ring_state2, 0, (size_t)W * kStateStride * 8));
  HIPT(hipMemset(c->stats, 0, kStatCount * 8));
  HIPT(hipMemset(c->sel_counts, 0, (size_t)kSelCounters * kSelStride * 8));
  HIPT(hipMemset(c->step_acc, 0, 24));
  if (hipHostMalloc((void**)&c->pend_host, 24, hipHostMallocMapped) != hipSuccess) {
    c->pend_host = nullptr;
    release(c);
    return fail(FERRY_ENOMEM, "hipHostMalloc of the step counter failed");
  }
  c->pend_host[0] = c->pend_host[1] = c->pend_host[2] = 0;
  HIPT(hipHostGetDevicePointer((void**)&c->pend_dev, c->pend_host, 0));
  HIPT(hipMemset(c->done, 0, 4));
  HIPT(hipMemset(c->err, 0, 4));
  HIPT(hipMemset(c->pool, 0, nslots * g.bb));
  // pinned host tier, mapped into the device address space
  const size_t hbytes = (size_t)g.host_blocks * g.bb;
  if (hipHostMalloc((void**)&c->host, hbytes, hipHostMallocMapped) != hipSuccess) {
    c->host = nullptr;
    release(c);
    return fail(FERRY_ENOMEM, "hipHostMalloc of the host tier failed");
  }
  HIPT(hipHostGetDevicePointer((void**)&c->host_dev, c->host, 0));
  if (g.dtype == FERRY_FP8_E4M3) {
    if (hipHostMalloc((void**)&c->host_scales, (size_t)g.host_blocks * 8, hipHostMallocMapped) != hipSuccess) {
      c->host_scales = nullptr;
      release(c);
      return fail(FERRY_ENOMEM, "hipHostMalloc of the host scales failed");
    }
    HIPT(hipHostGetDevicePointer((void**)&c->host_scales_dev, c->host_scales, 0));
  }
  hipLaunchKernelGGL(k_sets_reset, dim3(1024), dim3(256), 0, 0, g, c->st);
  HIPT(hipGetLastError());
  {  // every lane starts as a resident member of its owner
    std::vector<uint32_t> mem(g.n_owners), live(g.n_req, 1u);
    for (int o = 0; o < g.n_owners; ++o) mem[o] = (uint32_t)std::min(g.group, g.n_req - o * g.group);
    HIPT(hipMemcpy(c->st.members, mem.data(), (size_t)g.n_owners * 4, hipMemcpyHostToDevice));
    HIPT(hipMemcpy(c->lane_live, live.data(), (size_t)g.n_req * 4, hipMemcpyHostToDevice));
    HIPT(hipMemset(c->trim_gen, 0, (size_t)g.n_owners * 4));
  }
  c->events.resize((size_t)g.L, nullptr);
  for (auto& e : c->events) HIPT(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  c->booked.resize((size_t)g.L, nullptr);
  for (auto& e : c->booked) HIPT(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  HIPT(hipDeviceSynchronize());
#undef TRY
#undef HIPT
  *out = c;
  return FERRY_OK;
}

int ferry_ctx_destroy(ferry_ctx* ctx) {
  if (!ctx) return FERRY_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipDeviceSynchronize();
  release(ctx);
  return FERRY_OK;
}

int ferry_ctx_config(const ferry_ctx* ctx, ferry_config* out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!out) return fail(FERRY_EINVAL, "null out");
  *out = ctx->cfg;
  out->fetch_workers = ctx->g.workers;
  return FERRY_OK;
}

int ferry_ctx_sizes(const ferry_ctx* ctx, uint32_t* n_sets, uint32_t* max_sel,
                    uint64_t* block_bytes, uint64_t* pool_slots) {
  if (int rc = check_ctx(ctx)) return rc;
  if (n_sets) *n_sets = (uint32_t)ctx->g.n_sets;
  if (max_sel) *max_sel = (uint32_t)ctx->g.max_sel;
  if (block_bytes) *block_bytes = ctx->g.bb;
  if (pool_slots) *pool_slots = (uint64_t)ctx->g.n_sets * ctx->g.C;
  return FERRY_OK;
}

int ferry_hosttier_fill(ferry_ctx* ctx, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  HIPC(hipSetDevice(ctx->device));
  const Geo& g = ctx->g;
  const float mult = value_mult(ctx->cfg.value_std);
  const float mult8 = value_mult(96.0);
  const float base = (float)((double)ctx->cfg.value_std / 96.0);
  hipLaunchKernelGGL(k_hosttier_fill, dim3(4096), dim3(256), 0, (hipStream_t)stream, g,
                     ctx->host_dev, ctx->host_scales_dev, ctx->cfg.host_seed, mult, mult8, base);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_hosttier_register(ferry_ctx* ctx, void* host, uint64_t host_bytes, float* scales,
                            uint64_t scale_bytes) {
  if (int rc = check_ctx(ctx)) return rc;
  const Geo& g = ctx->g;
  const bool f8 = g.dtype == FERRY_FP8_E4M3;
  if (!host) return fail(FERRY_EINVAL, "null host tier");
  if (host_bytes < (uint64_t)g.host_blocks * g.bb)
    return fail(FERRY_EINVAL, "host tier smaller than host_blocks * block_bytes");
  if (f8 && (!scales || scale_bytes < (uint64_t)g.host_blocks * 8))
    return fail(FERRY_EINVAL, "fp8 needs host_blocks * 2 fp32 scales");
  if (!f8 && scales) return fail(FERRY_EINVAL, "scales are for fp8 KV only");
  HIPC(hipSetDevice(ctx->device));
  void* dev = nullptr;
  void* sdev = nullptr;
  if (hipHostGetDevicePointer(&dev, host, 0) != hipSuccess || !dev) {
    (void)hipGetLastError();
    return fail(FERRY_EINVAL, "host tier must be pinned, device-mapped memory (hipHostMalloc)");
  }
  if (scales && (hipHostGetDevicePointer(&sdev, scales, 0) != hipSuccess || !sdev)) {
    (void)hipGetLastError();
    return fail(FERRY_EINVAL, "host scales must be pinned, device-mapped memory (hipHostMalloc)");
  }
  HIPC(hipDeviceSynchronize());  // nothing may still read the tier being replaced
  if (ctx->host_owned) {
    if (ctx->host) HIPC(hipHostFree(ctx->host));
    if (ctx->host_scales) HIPC(hipHostFree(ctx->host_scales));
  }
  ctx->host = (uint8_t*)host;
  ctx->host_dev = (uint8_t*)dev;
  ctx->host_scales = scales;
  ctx->host_scales_dev = (float*)sdev;
  ctx->host_owned = false;
  return FERRY_OK;
}

int ferry_hosttier_view(ferry_ctx* ctx, void** bytes, float** scales) {
  if (int rc = check_ctx(ctx)) return rc;
  if (bytes) *bytes = ctx->host;
  if (scales) *scales = ctx->host_scales;
  return FERRY_OK;
}

int ferry_pool_view(ferry_ctx* ctx, void** pool, float** scales) {
  if (int rc = check_ctx(ctx)) return rc;
  if (pool) *pool = ctx->pool;
  if (scales) *scales = ctx->pool_scales;
  return FERRY_OK;
}

int ferry_sets_reset(ferry_ctx* ctx, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  HIPC(hipSetDevice(ctx->device));
  hipLaunchKernelGGL(k_sets_reset, dim3(1024), dim3(256), 0, (hipStream_t)stream, ctx->g, ctx->st);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_sets_reset_owners(ferry_ctx* ctx, const uint32_t* owners, uint32_t n, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (n == 0) return FERRY_OK;
  if (int rc = check_buf(owners, "owners")) return rc;
  if (n > (uint32_t)ctx->g.n_owners) return fail(FERRY_EINVAL, "more owners than the executor has");
  HIPC(hipSetDevice(ctx->device));
  const uint64_t waves = (uint64_t)n * ctx->g.L * ctx->g.Hkv;
  hipLaunchKernelGGL(k_sets_reset_owners, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, ctx->g, ctx->st, owners, n, ctx->err);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_sets_state(ferry_ctx* ctx, uint32_t* fill, uint32_t* ord, uint32_t* tag) {
  if (int rc = check_ctx(ctx)) return rc;
  HIPC(hipSetDevice(ctx->device));
  HIPC(hipDeviceSynchronize());
  const size_t ns = (size_t)ctx->g.n_sets, nsl = ns * ctx->g.C;
  if (fill) HIPC(hipMemcpy(fill, ctx->st.fill, ns * 4, hipMemcpyDeviceToHost));
  if (ord) HIPC(hipMemcpy(ord, ctx->st.ord, nsl * 4, hipMemcpyDeviceToHost));
  if (tag) HIPC(hipMemcpy(tag, ctx->st.tag, nsl * 4, hipMemcpyDeviceToHost));
  return FERRY_OK;
}

int ferry_sets_own(ferry_ctx* ctx, uint32_t* own) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!own) return fail(FERRY_EINVAL, "null out");
  if (!ctx->st.own) return fail(FERRY_EINVAL, "member masks exist only for prefix groups (group > 1)");
  HIPC(hipSetDevice(ctx->device));
  HIPC(hipDeviceSynchronize());
  HIPC(hipMemcpy(own, ctx->st.own, (size_t)ctx->g.n_sets * ctx->g.C * 4, hipMemcpyDeviceToHost));
  return FERRY_OK;
}

}  // extern "C"

namespace {
int members_update(ferry_ctx* ctx, const uint32_t* lanes, uint32_t n, int delta, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (n == 0) return FERRY_OK;
  if (int rc = check_buf(lanes, "lanes")) return rc;
  const Geo& g = ctx->g;
  if (n > (uint32_t)g.n_req) return fail(FERRY_EINVAL, "more lanes than the executor has");
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  const uint32_t gen = delta < 0 ? ++ctx->member_calls : 0u;
  hipLaunchKernelGGL(k_members_update, dim3((n + 255) / 256), dim3(256), 0, s, g, ctx->lane_live,
                     ctx->st.members, ctx->trim_gen, lanes, n, delta, gen, ctx->err);
  HIPC(hipGetLastError());
  if (delta < 0 && (g.cap_mode == FERRY_CAP_PER_MEMBER || g.group > 1)) {
    const size_t lds = (size_t)2 * g.C * 4;
    const dim3 grid((unsigned)g.n_sets), block(64);
    switch (g.bb / 1024) {
      case 4: hipLaunchKernelGGL(k_sets_trim<4>, grid, block, lds, s, g, ctx->st, ctx->lane_live, ctx->trim_gen, gen, ctx->pool, ctx->pool_scales); break;
      case 8: hipLaunchKernelGGL(k_sets_trim<8>, grid, block, lds, s, g, ctx->st, ctx->lane_live, ctx->trim_gen, gen, ctx->pool, ctx->pool_scales); break;
      case 16: hipLaunchKernelGGL(k_sets_trim<16>, grid, block, lds, s, g, ctx->st, ctx->lane_live, ctx->trim_gen, gen, ctx->pool, ctx->pool_scales); break;
      default: return fail(FERRY_EINVAL, "unsupported block size");
    }
    HIPC(hipGetLastError());
  }
  return FERRY_OK;
}
}  // namespace

extern "C" {

int ferry_members_leave(ferry_ctx* ctx, const uint32_t* lanes, uint32_t n, void* stream) {
  return members_update(ctx, lanes, n, -1, stream);
}

int ferry_members_join(ferry_ctx* ctx, const uint32_t* lanes, uint32_t n, void* stream) {
  return members_update(ctx, lanes, n, +1, stream);
}

int ferry_members_get(ferry_ctx* ctx, uint32_t* members) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!members) return fail(FERRY_EINVAL, "null out");
  HIPC(hipSetDevice(ctx->device));
  HIPC(hipDeviceSynchronize());
  HIPC(hipMemcpy(members, ctx->st.members, (size_t)ctx->g.n_owners * 4, hipMemcpyDeviceToHost));
  return FERRY_OK;
}

int ferry_bookkeep_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const uint32_t* sel,
                          uint32_t* slots, uint32_t* miss_count, ferry_miss* misses,
                          uint8_t* miss_flag, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_bufs({{sel, "sel"}, {slots, "slots"}, {miss_count, "miss_count"}, {misses, "misses"}}))
    return rc;
  if (miss_flag)
    if (int rc = check_buf(miss_flag, "miss_flag")) return rc;
  return bookkeep_ring(ctx, l0, nl, sel, slots, miss_count, misses, miss_flag, stream, 0);
}

int ferry_missq_drain(ferry_ctx* ctx, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return drain_ring(ctx, stream, 0);
}

}  // extern "C"

namespace {

int bookkeep_ring(ferry_ctx* ctx, int32_t l0, int32_t nl, const uint32_t* sel, uint32_t* slots,
                  uint32_t* miss_count, ferry_miss* misses, uint8_t* miss_flag, void* stream,
                  int which) {
  if (!sel || !slots || !miss_count || !misses) return fail(FERRY_EINVAL, "null buffer");
  const Geo& g = ctx->g;
  if (l0 < 0 || nl < 1 || l0 + nl > g.L) return fail(FERRY_EINVAL, "bad layer range");
  HIPC(hipSetDevice(ctx->device));
  const int wpb = ctx->lru_wpb;
  const int nsets = g.n_owners * nl * g.Hkv;
  const dim3 grid((nsets + wpb - 1) / wpb), block(64 * wpb);
  if (ctx->cfg.lru_mode == FERRY_LRU_SERIAL)
    hipLaunchKernelGGL(k_lru_step<true>, grid, block, ctx->lru_lds, (hipStream_t)stream, g, sel, slots,
                       miss_count, misses, miss_flag, ctx->st, ctx->ring(which), l0, nl,
                       ctx->sel_counts, ctx->err);
  else
    hipLaunchKernelGGL(k_lru_step<false>, grid, block, ctx->lru_lds, (hipStream_t)stream, g, sel, slots,
                       miss_count, misses, miss_flag, ctx->st, ctx->ring(which), l0, nl,
                       ctx->sel_counts, ctx->err);
  HIPC(hipGetLastError());
  if (l0 + nl == g.L) ctx->steps++;
  return FERRY_OK;
}

int drain_ring(ferry_ctx* ctx, void* stream, int which) {
  HIPC(hipSetDevice(ctx->device));
  FetchArgs a;
  a.g = ctx->g;
  a.ring = ctx->ring(which);
  a.host = ctx->host_dev;
  a.host_scales = ctx->host_scales_dev;
  a.pool = ctx->pool;
  a.pool_scales = ctx->pool_scales;
  a.steal = ctx->cfg.steal;
  a.steal_chunk = ctx->steal_chunk;
  a.prio = ctx->fetch_prio;
  a.thief_waves = ctx->thief_waves;
  a.steal_inflight = ctx->steal_inflight;
  a.stats = ctx->stats;
  a.step_acc = ctx->step_acc;
  a.done = ctx->done;
  a.err = ctx->err;
  const dim3 grid(ctx->g.workers), block(64 * ctx->fetch_waves);
  switch (ctx->g.bb / 1024) {
    case 4: hipLaunchKernelGGL(k_fetch<4>, grid, block, 0, (hipStream_t)stream, a); break;
    case 8: hipLaunchKernelGGL(k_fetch<8>, grid, block, 0, (hipStream_t)stream, a); break;
    case 16: hipLaunchKernelGGL(k_fetch<16>, grid, block, 0, (hipStream_t)stream, a); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  return FERRY_OK;
}

}  // namespace

extern "C" {

int ferry_bookkeep_step(ferry_ctx* ctx, const uint32_t* sel, uint32_t* slots,
                        uint32_t* miss_count, ferry_miss* misses, uint8_t* miss_flag,
                        void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return ferry_bookkeep_layers(ctx, 0, ctx->g.L, sel, slots, miss_count, misses, miss_flag, stream);
}

int ferry_missq_push(ferry_ctx* ctx, const ferry_miss* misses, uint32_t n, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (n == 0) return FERRY_OK;
  if (int rc = check_buf(misses, "misses")) return rc;
  HIPC(hipSetDevice(ctx->device));
  hipLaunchKernelGGL(k_missq_push, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, ctx->g,
                     ctx->ring(), misses, n, ctx->err);
  HIPC(hipGetLastError());
  return FERRY_OK;
}


int ferry_fetch_step(ferry_ctx* ctx, const uint32_t* sel, uint32_t* slots, uint32_t* miss_count,
                     ferry_miss* misses, uint8_t* miss_flag, void* stream) {
  int rc = ferry_bookkeep_step(ctx, sel, slots, miss_count, misses, miss_flag, stream);
  if (rc) return rc;
  return ferry_missq_drain(ctx, stream);
}

int ferry_sparse_decode_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                               const uint32_t* slots, float* out, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return decode_layers(ctx, l0, nl, q, slots, out, stream, nullptr);
}

int ferry_attn_kernel(const ferry_ctx* ctx, int32_t* kind, int32_t* waves) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!kind || !waves) return fail(FERRY_EINVAL, "null output");
  const AttnPlan p = attn_plan(ctx);
  *kind = p.grouped ? FERRY_ATTN_GROUP : p.mfma ? FERRY_ATTN_MFMA : FERRY_ATTN_VALU;
  *waves = p.waves;
  if (p.grouped)  // ferry_sparse_decode's launch: every layer's group sets
    *waves = group_launch_waves(p.dtype, p.tiles, (long)ctx->g.group * ctx->g.k,
                                (long)ctx->g.n_owners * ctx->g.L * ctx->g.Hkv, p.cus, p.group_w);
  return FERRY_OK;
}

int ferry_sparse_decode(ferry_ctx* ctx, const float* q, const uint32_t* slots, float* out,
                        void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return ferry_sparse_decode_layers(ctx, 0, ctx->g.L, q, slots, out, stream);
}

int ferry_set_batch_policy(ferry_ctx* ctx, double min_mb, double max_mb, double target_batches) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!(min_mb > 0.0) || !(max_mb >= min_mb) || !(target_batches > 0.0))
    return fail(FERRY_EINVAL, "need 0 < min_mb <= max_mb and target_batches > 0");
  ctx->pol_min_mb = min_mb;
  ctx->pol_max_mb = max_mb;
  ctx->pol_target = target_batches;
  return FERRY_OK;
}

int ferry_decode_chunks(const ferry_ctx* ctx, uint64_t pending_blocks, int32_t* chunks) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!chunks) return fail(FERRY_EINVAL, "null out");
  const double mb = (double)pending_blocks * (double)ctx->g.bb / 1048576.0;
  // AdaptiveBatchPolicy::choose_mb: clamp(pending / target, min, max) MB per batch
  const double g = std::min(std::max(mb / ctx->pol_target, ctx->pol_min_mb), ctx->pol_max_mb);
  const double n = std::ceil(mb / g);
  *chunks = (int32_t)std::min<double>(std::max(n, 1.0), (double)ctx->g.L);
  return FERRY_OK;
}

int ferry_decode_step(ferry_ctx* ctx, const uint32_t* sel, const float* q, uint32_t* slots,
                      float* out, uint32_t* miss_count, ferry_miss* misses, int32_t chunks,
                      void* stream, void* side_stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_bufs({{sel, "sel"}, {q, "q"}, {slots, "slots"}, {out, "out"},
                           {miss_count, "miss_count"}, {misses, "misses"}}))
    return rc;
  const int L = ctx->g.L;
  if (chunks < 0) return fail(FERRY_EINVAL, "chunks < 0");
  const bool adaptive = chunks == 0;
  uint64_t last = 0, last_attn = 0;
  if (adaptive) {
    // from the blocks the last closed step fetched (and attended): the host
    // enqueues ahead of the GPU, so that step may be one or more steps back;
    // the sequence word makes the two counts come from the same step
    const volatile unsigned long long* pend = ctx->pend_host;
    for (int tries = 0; tries < 1000; ++tries) {
      const unsigned long long s0 = pend[2];
      std::atomic_thread_fence(std::memory_order_acquire);
      last = pend[0];
      last_attn = pend[1];
      std::atomic_thread_fence(std::memory_order_acquire);
      if (!(s0 & 1ull) && pend[2] == s0) break;
    }
    if (int rc = ferry_decode_chunks(ctx, last, &chunks)) return rc;
  }
  chunks = std::min(chunks, L);
  // Layer ranges: `chunks` even ranges, except that the adaptive count also
  // shortens the last one.  Its attention is the one the fetch cannot hide;
  // the range before it attends while the last range is fetched, which takes
  // longer as long as the last range has at least 2 r times its layers, r =
  // (attention time) / (fetch time) of a layer at typical MI355X rates
  // (6.5 TB/s HBM reads, 55 GB/s host link; 2 for the slowdown of sharing the
  // GPU with the fetch).  At the 7B shape r = 0.08: the last range is one layer.
  std::vector<int> first(chunks + 1, L);
  {
    int tail = (L + chunks - 1) / chunks;
    if (adaptive && chunks >= 2 && last > 0) {
      const Geo& g = ctx->g;
      const double kv = (double)g.bb + (g.dtype == FERRY_FP8_E4M3 ? 8.0 : 0.0);
      // the blocks attention reads: k per row, or the distinct blocks the
      // prefix-group kernel counted in the last step
      const double blocks = last_attn ? (double)last_attn : (double)g.n_req * g.L * g.Hkv * g.k;
      const double attn_s = blocks * kv / 6.5e12;
      const double fetch_s = (double)last * (double)g.bb / 55e9;
      const int rest = (L - 1 + chunks - 2) / (chunks - 1);  // layers of the other ranges
      const double want = std::ceil(2.0 * attn_s / fetch_s * rest);
      if (want < (double)tail) tail = std::max(1, (int)want);
    }
    // the other chunks - 1 ranges split L - tail layers as evenly as possible
    const int head = L - tail, nh = chunks - 1;
    for (int c = 0; c < nh; ++c) first[c] = c * head / nh;
    first[nh] = head;
    first[chunks] = L;
  }
  hipStream_t ms = (hipStream_t)stream, ss = (hipStream_t)side_stream;
  const bool overlap = ss != nullptr && ss != ms;
  HIPC(hipSetDevice(ctx->device));
  if (!sel || !slots || !miss_count || !misses) return fail(FERRY_EINVAL, "null buffer");
  if (!overlap) {  // one stream: bookkeeping, fetch and attention range by range
    for (int c = 0; c < chunks; ++c) {
      const int l0 = first[c], nl = first[c + 1] - first[c];
      if (nl <= 0) continue;
      int rc = bookkeep_ring(ctx, l0, nl, sel, slots, miss_count, misses, nullptr, ms, 0);
      if (!rc) rc = drain_ring(ctx, ms, 0);
      if (!rc) rc = decode_layers(ctx, l0, nl, q, slots, out, ms, ctx->step_acc + 1);
      if (rc) return rc;
    }
  } else {
    // Two streams, the caller's.  Ranges 0 and 1 are booked up front (rings 0
    // and 1); then for each range c the main stream waits for its fetch, books
    // range c + 2 into the ring that fetch has just drained (c mod 2), and
    // attends c, while the side stream fetches each range once it is booked.
    // Booking c + 2 runs beside the fetch of c + 1 and never waits for an
    // attention, which beside a fetch can run several times slower than alone
    // (the fetch's wavefronts share the CUs).  Ranges touch disjoint sets,
    // slots and outputs.  No stream of the context's own: a third stream can
    // share a hardware queue with the side stream (HIP hands a process a few
    // queues, shared among its streams) and then serialise with the fetch.
    std::vector<int> live;  // ranges with layers
    for (int c = 0; c < chunks; ++c)
      if (first[c + 1] > first[c]) live.push_back(c);
    auto book_fetch = [&](int i) -> int {
      const int c = live[(size_t)i], l0 = first[c], nl = first[c + 1] - first[c];
      int rc = bookkeep_ring(ctx, l0, nl, sel, slots, miss_count, misses, nullptr, ms, i & 1);
      if (rc) return rc;
      HIPC(hipEventRecord(ctx->booked[i], ms));
      HIPC(hipStreamWaitEvent(ss, ctx->booked[i], 0));
      if ((rc = drain_ring(ctx, ss, i & 1))) return rc;
      HIPC(hipEventRecord(ctx->events[i], ss));
      return FERRY_OK;
    };
    const int n = (int)live.size();
    for (int i = 0; i < std::min(n, 2); ++i)
      if (int rc = book_fetch(i)) return rc;
    for (int i = 0; i < n; ++i) {
      const int c = live[(size_t)i];
      HIPC(hipStreamWaitEvent(ms, ctx->events[i], 0));
      if (i + 2 < n)  // ring i mod 2 is drained
        if (int rc = book_fetch(i + 2)) return rc;
      if (int rc = decode_layers(ctx, first[c], first[c + 1] - first[c], q, slots, out, ms,
                                 ctx->step_acc + 1))
        return rc;
    }
  }
  // the step's fetched blocks, for the next step's adaptive chunking
  hipLaunchKernelGGL(k_step_close, dim3(1), dim3(64), 0, ms, ctx->step_acc, ctx->pend_dev);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_summaries_build(ferry_ctx* ctx, uint64_t n_records, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  const Geo& g = ctx->g;
  const uint64_t S = n_records ? n_records : g.host_blocks;
  if (S % g.host_blocks)
    return fail(FERRY_EINVAL, "summary records must be a multiple of the host tier's blocks");
  const uint64_t rec = 2ull * g.D * g.esize;
  HIPC(hipSetDevice(ctx->device));
  if (ctx->sums && ctx->sum_blocks != S) {
    HIPC(hipDeviceSynchronize());
    HIPC(hipFree(ctx->sums));
    if (ctx->sum_scales) HIPC(hipFree(ctx->sum_scales));
    ctx->sums = nullptr;
    ctx->sum_scales = nullptr;
    ctx->sum_blocks = 0;
  }
  if (!ctx->sums) {
    if (int rc = alloc_table(S * rec, g.dtype == FERRY_FP8_E4M3 ? S : 0, &ctx->sums, &ctx->sum_scales))
      return rc;
    ctx->sum_blocks = S;
  }
  const unsigned blocks = (unsigned)std::min<uint64_t>((g.host_blocks + 3) / 4, 16384);
  hipStream_t s = (hipStream_t)stream;
  switch (g.dtype) {
    case FERRY_F32:
      hipLaunchKernelGGL(k_summaries_build<FERRY_F32>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev,
                         ctx->host_scales_dev, ctx->sums, ctx->sum_scales);
      break;
    case FERRY_F16:
      hipLaunchKernelGGL(k_summaries_build<FERRY_F16>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev,
                         ctx->host_scales_dev, ctx->sums, ctx->sum_scales);
      break;
    case FERRY_BF16:
      hipLaunchKernelGGL(k_summaries_build<FERRY_BF16>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev,
                         ctx->host_scales_dev, ctx->sums, ctx->sum_scales);
      break;
    default:
      hipLaunchKernelGGL(k_summaries_build<FERRY_FP8_E4M3>, dim3(blocks), dim3(256), 0, s, g,
                         ctx->host_dev, ctx->host_scales_dev, ctx->sums, ctx->sum_scales);
  }
  HIPC(hipGetLastError());
  if (S > g.host_blocks) {
    hipLaunchKernelGGL(k_summaries_tile, dim3(8192), dim3(256), 0, s, ctx->sums, ctx->sum_scales,
                       g.host_blocks, S, (uint32_t)rec);
    HIPC(hipGetLastError());
  }
  return FERRY_OK;
}

int ferry_summaries_view(ferry_ctx* ctx, void** sums, float** scales, uint64_t* n_records) {
  if (int rc = check_ctx(ctx)) return rc;
  if (sums) *sums = ctx->sums;
  if (scales) *scales = ctx->sum_scales;
  if (n_records) *n_records = ctx->sum_blocks;
  return FERRY_OK;
}

}  // extern "C"

namespace {

struct SelArgs {
  Geo g;
  const float* q;
  const int32_t* ctx_blocks;
  const uint8_t* sums;
  const float* sum_scales;
  uint64_t sum_mod;
  uint32_t* sel;
  int l0, nl, max_n;
  int* err;
};

template <int DT, int G, bool LAYER>
void launch_sel(const dim3& grid, size_t lds, hipStream_t s, const SelArgs& a) {
  hipLaunchKernelGGL((k_select_topk<DT, G, LAYER, 4>), grid, dim3(256), lds, s, a.g, a.q, a.ctx_blocks,
                     a.sums, a.sum_scales, a.sum_mod, a.sel, a.l0, a.nl, a.max_n, a.err);
}
template <int DT, bool LAYER>
void launch_sel_g(int G, const dim3& grid, size_t lds, hipStream_t s, const SelArgs& a) {
  switch (G) {
    case 1: launch_sel<DT, 1, LAYER>(grid, lds, s, a); return;
    case 2: launch_sel<DT, 2, LAYER>(grid, lds, s, a); return;
    case 4: launch_sel<DT, 4, LAYER>(grid, lds, s, a); return;
    default: launch_sel<DT, 8, LAYER>(grid, lds, s, a); return;
  }
}
template <bool LAYER>
void launch_sel_dt(int dtype, int G, const dim3& grid, size_t lds, hipStream_t s, const SelArgs& a) {
  switch (dtype) {
    case FERRY_F32: launch_sel_g<FERRY_F32, LAYER>(G, grid, lds, s, a); return;
    case FERRY_F16: launch_sel_g<FERRY_F16, LAYER>(G, grid, lds, s, a); return;
    case FERRY_BF16: launch_sel_g<FERRY_BF16, LAYER>(G, grid, lds, s, a); return;
    default: launch_sel_g<FERRY_FP8_E4M3, LAYER>(G, grid, lds, s, a); return;
  }
}

}  // namespace

extern "C" {

int ferry_select_topk_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                             const int32_t* ctx_blocks, int mode, uint32_t* sel, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_bufs({{q, "q"}, {ctx_blocks, "ctx_blocks"}, {sel, "sel"}})) return rc;
  const Geo& g = ctx->g;
  if (l0 < 0 || nl < 1 || l0 + nl > g.L) return fail(FERRY_EINVAL, "bad layer range");
  if (mode != FERRY_TOPK_PER_HEAD && mode != FERRY_TOPK_LAYER_MAX) return fail(FERRY_EINVAL, "bad mode");
  if (g.group != 1)
    return fail(FERRY_EINVAL, "top-k selection needs private sets (group 1): a group's members select "
                              "from their own contexts");
  if (!ctx->sums || !ctx->sum_blocks)
    return fail(FERRY_EINVAL, "block summaries not built (ferry_summaries_build)");
  const bool layer = mode == FERRY_TOPK_LAYER_MAX;
  const int G = g.Hq / g.Hkv;
  const int Gq = layer ? g.Hq : G;
  const size_t lds = ((size_t)Gq * g.D + (size_t)g.max_blocks) * 4;
  if (lds > 65536)
    return fail(FERRY_EINVAL, "max_blocks (plus the query heads of a row) exceed the selection's 64 KiB "
                              "of LDS");
  HIPC(hipSetDevice(ctx->device));
  const dim3 grid((unsigned)((size_t)g.n_req * nl * (layer ? 1 : g.Hkv)));
  const SelArgs a{g,   q,   ctx_blocks,    ctx->sums, ctx->sum_scales, ctx->sum_blocks,
                  sel, l0,  nl,            g.max_blocks, ctx->err};
  if (layer)
    launch_sel_dt<true>(g.dtype, G, grid, lds, (hipStream_t)stream, a);
  else
    launch_sel_dt<false>(g.dtype, G, grid, lds, (hipStream_t)stream, a);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_select_topk(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks, int mode, uint32_t* sel,
                      void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return ferry_select_topk_layers(ctx, 0, ctx->g.L, q, ctx_blocks, mode, sel, stream);
}

// one float score per context block in LDS
constexpr uint64_t kMassLds = 60 * 1024;

}  // extern "C"

namespace {

// Whether k_mass_units keeps its per-block log-sums in LDS: 16-bit K whose
// max_blocks * G floats fit kMassLdsWs (FERRY_MASS_WS=hbm keeps the HBM
// workspace).  At the long-context GQA shape the LDS copy measured 0.86-0.88
// of HBM against 0.80-0.84 for bf16 and 0.86 against 0.80 for fp16; fp8 K
// (2 KiB records, twice the arithmetic per byte) measured 0.69 against 0.77,
// the LDS leaving one workgroup per CU instead of two, so it keeps HBM.
constexpr uint64_t kMassLdsWs = 144 * 1024;
bool mass_in_lds(ferry_ctx* ctx) {
  if (ctx->mass_lds < 0) {
    const Geo& g = ctx->g;
    const char* e = std::getenv("FERRY_MASS_WS");
    ctx->mass_lds = (g.dtype == FERRY_F16 || g.dtype == FERRY_BF16) && !(e && std::string(e) == "hbm") &&
                    (uint64_t)g.max_blocks * (uint64_t)(g.Hq / g.Hkv) * 4 <= kMassLdsWs;
  }
  return ctx->mass_lds != 0;
}
size_t mass_lds_bytes(ferry_ctx* ctx) {
  return mass_in_lds(ctx) ? (size_t)ctx->g.max_blocks * (size_t)(ctx->g.Hq / ctx->g.Hkv) * 4 : 0;
}

// One workgroup's workspace slice of the mass selection in HBM: a (max, sum)
// pair per context block and query head (none when the log-sums stay in LDS).
uint64_t mass_slice_bytes(ferry_ctx* ctx) {
  const Geo& g = ctx->g;
  if (g.dtype != FERRY_F32 && mass_in_lds(ctx)) return 0;
  return (uint64_t)g.max_blocks * (uint64_t)(g.Hq / g.Hkv) * 2 * sizeof(float);
}

// Workgroups of k_mass_units the device holds at once (occupancy x CUs),
// computed once per context.
int mass_units_resident(ferry_ctx* ctx) {
  if (ctx->mass_resident > 0) return ctx->mass_resident;
  const Geo& g = ctx->g;
  const int G = g.Hq / g.Hkv;
  const void* fn = nullptr;
#define FERRY_MASS_FN(DT)                                                                           \
  fn = G == 1   ? reinterpret_cast<const void*>(&k_mass_units<DT, 1, kMassUnitWaves, kMassUnitInflight>) \
       : G == 2 ? reinterpret_cast<const void*>(&k_mass_units<DT, 2, kMassUnitWaves, kMassUnitInflight>) \
       : G == 4 ? reinterpret_cast<const void*>(&k_mass_units<DT, 4, kMassUnitWaves, kMassUnitInflight>) \
                : reinterpret_cast<const void*>(&k_mass_units<DT, 8, kMassUnitWaves, kMassUnitInflight>)
  if (g.dtype == FERRY_F16) FERRY_MASS_FN(FERRY_F16);
  else if (g.dtype == FERRY_BF16) FERRY_MASS_FN(FERRY_BF16);
  else FERRY_MASS_FN(FERRY_FP8_E4M3);
#undef FERRY_MASS_FN
  int per_cu = 0;
  const size_t lds = mass_lds_bytes(ctx);
  const bool on_dev = hipSetDevice(ctx->device) == hipSuccess;
  if (on_dev && lds > 65536)
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMassLdsWs);
  if (!on_dev || hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 64 * kMassUnitWaves, lds) != hipSuccess ||
      per_cu < 1) {
    (void)hipGetLastError();
    per_cu = 1;  // still correct: the workgroups take the units from the counter
  }
  ctx->mass_resident = per_cu * ctx->cus;
  return ctx->mass_resident;
}

// Workgroups of a mass selection over nl layers, at most cap: (request,
// layer) items for fp32 K (k_select_mass, at most kMassWgs); for 16-bit and
// fp8 K (k_mass_units) at most the (request, layer, kv head) units, the
// resident workgroups and kMassUnitWgs.
uint64_t mass_wgs(ferry_ctx* ctx, int nl, uint64_t cap) {
  const Geo& g = ctx->g;
  if (g.dtype == FERRY_F32)
    return std::min<uint64_t>(std::min<uint64_t>((uint64_t)g.n_req * nl, kMassWgs), cap);
  const uint64_t units = (uint64_t)g.n_req * nl * g.Hkv;
  const uint64_t res = std::min<uint64_t>((uint64_t)mass_units_resident(ctx), kMassUnitWgs);
  return std::min<uint64_t>(std::min<uint64_t>(units, res), cap);
}

// Workspace of a mass selection over nl layers with wgs workgroups: their
// slices; for 16-bit and fp8 K first a 256-byte unit counter, and after the
// slices a float mass per context block of every (request, layer, kv head)
// unit, 256-byte aligned.
constexpr uint64_t kMassCounterBytes = 256;
uint64_t mass_mass_offset(ferry_ctx* ctx, uint64_t wgs) {
  return kMassCounterBytes + (wgs * mass_slice_bytes(ctx) + 255) / 256 * 256;
}
uint64_t mass_ws_bytes(ferry_ctx* ctx, int nl, uint64_t wgs) {
  const Geo& g = ctx->g;
  if (g.dtype == FERRY_F32) return wgs * mass_slice_bytes(ctx);
  return mass_mass_offset(ctx, wgs) + (uint64_t)g.n_req * nl * g.Hkv * g.max_blocks * sizeof(float);
}

}  // namespace

extern "C" {

int ferry_ktiles_build(ferry_ctx* ctx, uint64_t n_records, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  const Geo& g = ctx->g;
  const uint64_t S = n_records ? n_records : g.host_blocks;
  if (S % g.host_blocks) return fail(FERRY_EINVAL, "K records must be a multiple of the host tier's blocks");
  const uint64_t KT = g.bb / 2;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  if (ctx->ktab && ctx->kt_records != S) {
    HIPC(hipDeviceSynchronize());
    HIPC(hipFree(ctx->ktab));
    if (ctx->ktab_scales) HIPC(hipFree(ctx->ktab_scales));
    ctx->ktab = nullptr;
    ctx->ktab_scales = nullptr;
    ctx->kt_records = 0;
  }
  if (!ctx->ktab) {
    if (int rc = alloc_table(S * KT, g.dtype == FERRY_FP8_E4M3 ? S : 0, &ctx->ktab, &ctx->ktab_scales))
      return rc;
    ctx->kt_records = S;
  }
  if (!ctx->mass_ws && (uint64_t)g.max_blocks * 4 <= kMassLds)
    HIPC(hipMalloc(&ctx->mass_ws, mass_ws_bytes(ctx, g.L, mass_wgs(ctx, g.L, ~0ull))));
  ctx->kt_perm = g.dtype != FERRY_F32;
  const unsigned blocks = (unsigned)std::min<uint64_t>((g.host_blocks + 3) / 4, 16384);
  switch (KT / 1024) {
    case 2: hipLaunchKernelGGL(k_ktiles_build<2>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev, ctx->host_scales_dev, ctx->ktab, ctx->ktab_scales, ctx->kt_perm); break;
    case 4: hipLaunchKernelGGL(k_ktiles_build<4>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev, ctx->host_scales_dev, ctx->ktab, ctx->ktab_scales, ctx->kt_perm); break;
    case 8: hipLaunchKernelGGL(k_ktiles_build<8>, dim3(blocks), dim3(256), 0, s, g, ctx->host_dev, ctx->host_scales_dev, ctx->ktab, ctx->ktab_scales, ctx->kt_perm); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  // records past the host tier's repeat it: block (set, b) reads record
  // (set * max_blocks + b) mod S, whose content is host block (... ) mod host_blocks
  const uint64_t hb = g.host_blocks;
  for (uint64_t c = 1; c < S / hb; ++c) {
    HIPC(hipMemcpyAsync(ctx->ktab + c * hb * KT, ctx->ktab, hb * KT, hipMemcpyDeviceToDevice, s));
    if (ctx->ktab_scales)
      HIPC(hipMemcpyAsync(ctx->ktab_scales + c * hb, ctx->ktab_scales, hb * 4, hipMemcpyDeviceToDevice, s));
  }
  return FERRY_OK;
}

int ferry_ktiles_view(ferry_ctx* ctx, void** ktiles, float** scales, uint64_t* n_records) {
  if (int rc = check_ctx(ctx)) return rc;
  if (ktiles) *ktiles = ctx->ktab;
  if (scales) *scales = ctx->ktab_scales;
  if (n_records) *n_records = ctx->kt_records;
  return FERRY_OK;
}

}  // extern "C"

namespace {

// The mass selection of layers [l0, l0 + nl) with `wgs` workgroups
// (mass_wgs) and workspace `ws` of mass_ws_bytes(ctx, nl, wgs).
int launch_select_mass(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                       const int32_t* ctx_blocks, uint32_t* sel, void* stream, float* ws,
                       uint64_t wgs) {
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  const int G = g.Hq / g.Hkv;
  const size_t lds = (size_t)g.max_blocks * 4;
  if (g.dtype == FERRY_F32) {  // vector ALUs, one (request, layer) item per workgroup pass
#define FERRY_MASS_LAUNCH(GG)                                                                  \
  hipLaunchKernelGGL((k_select_mass<FERRY_F32, GG, 4>), dim3((unsigned)wgs), dim3(256), lds, s, g, \
                     q, ctx_blocks, ctx->ktab, ctx->ktab_scales, ctx->kt_records, ws, sel, l0, nl, \
                     g.max_blocks, ctx->err)
    switch (G) {
      case 1: FERRY_MASS_LAUNCH(1); break;
      case 2: FERRY_MASS_LAUNCH(2); break;
      case 4: FERRY_MASS_LAUNCH(4); break;
      default: FERRY_MASS_LAUNCH(8); break;
    }
#undef FERRY_MASS_LAUNCH
    HIPC(hipGetLastError());
    return FERRY_OK;
  }
  // matrix cores: the units' masses, then each item's sum over kv heads and top k
  unsigned* counter = reinterpret_cast<unsigned*>(ws);
  const size_t ulds = mass_lds_bytes(ctx);  // block log-sums in LDS, else HBM slices
  float* slices = ulds ? nullptr : reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + kMassCounterBytes);
  float* mass = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + mass_mass_offset(ctx, wgs));
  hipLaunchKernelGGL(k_mass_reset, dim3(1), dim3(64), 0, s, counter);
  HIPC(hipGetLastError());
#define FERRY_MASS_UNITS(DT, GG)                                                                 \
  hipLaunchKernelGGL((k_mass_units<DT, GG, kMassUnitWaves, kMassUnitInflight>), dim3((unsigned)wgs), \
                     dim3(64 * kMassUnitWaves), ulds, s, g, q, ctx_blocks, ctx->ktab, ctx->ktab_scales, \
                     ctx->kt_records, slices, mass, counter, l0, nl, g.max_blocks, ctx->err)
#define FERRY_MASS_UNITS_G(DT)                \
  switch (G) {                                \
    case 1: FERRY_MASS_UNITS(DT, 1); break;   \
    case 2: FERRY_MASS_UNITS(DT, 2); break;   \
    case 4: FERRY_MASS_UNITS(DT, 4); break;   \
    default: FERRY_MASS_UNITS(DT, 8); break;  \
  }
  switch (g.dtype) {
    case FERRY_F16: FERRY_MASS_UNITS_G(FERRY_F16); break;
    case FERRY_BF16: FERRY_MASS_UNITS_G(FERRY_BF16); break;
    default: FERRY_MASS_UNITS_G(FERRY_FP8_E4M3); break;
  }
#undef FERRY_MASS_UNITS_G
#undef FERRY_MASS_UNITS
  HIPC(hipGetLastError());
  const unsigned items = (unsigned)std::min<uint64_t>((uint64_t)g.n_req * nl, kMassWgs);
  hipLaunchKernelGGL((k_mass_topk<kMassTopkWaves>), dim3(items), dim3(64 * kMassTopkWaves), lds, s, g,
                     ctx_blocks, mass, sel, l0, nl, g.max_blocks);
  HIPC(hipGetLastError());
  return FERRY_OK;
}

// Arguments every mass selection needs, checked before anything launches.
int check_select_mass(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                      const int32_t* ctx_blocks, uint32_t* sel) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_bufs({{q, "q"}, {ctx_blocks, "ctx_blocks"}, {sel, "sel"}})) return rc;
  const Geo& g = ctx->g;
  if (l0 < 0 || nl < 1 || l0 + nl > g.L) return fail(FERRY_EINVAL, "bad layer range");
  if (g.group != 1)
    return fail(FERRY_EINVAL, "top-k selection needs private sets (group 1): a group's members select "
                              "from their own contexts");
  if (!ctx->ktab || !ctx->kt_records) return fail(FERRY_EINVAL, "K table not built (ferry_ktiles_build)");
  if ((size_t)g.max_blocks * 4 > kMassLds)
    return fail(FERRY_EINVAL, "max_blocks exceed the mass selection's 60 KiB of LDS");
  return FERRY_OK;
}

}  // namespace

extern "C" {

int ferry_select_mass_layers(ferry_ctx* ctx, int32_t l0, int32_t nl, const float* q,
                             const int32_t* ctx_blocks, uint32_t* sel, void* stream) {
  if (int rc = check_select_mass(ctx, l0, nl, q, ctx_blocks, sel)) return rc;
  if (!ctx->mass_ws) return fail(FERRY_EINVAL, "no mass-selection workspace (ferry_ktiles_build failed)");
  return launch_select_mass(ctx, l0, nl, q, ctx_blocks, sel, stream, ctx->mass_ws,
                            mass_wgs(ctx, nl, ~0ull));
}

int ferry_select_mass(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks, uint32_t* sel,
                      void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  return ferry_select_mass_layers(ctx, 0, ctx->g.L, q, ctx_blocks, sel, stream);
}

int ferry_select_mass_noalloc(ferry_ctx* ctx, const float* q, const int32_t* ctx_blocks,
                              uint32_t* sel, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = check_select_mass(ctx, 0, ctx->g.L, q, ctx_blocks, sel)) return rc;
  const Geo& g = ctx->g;
  if (!ctx->scratch_dev) return fail(FERRY_EHIP, "static scratch not resolved for this device");
  // the largest layer range whose workspace (the masses of its units, 16-bit
  // and fp8 K) leaves room in the static array for at least one workgroup
  // slice; ranges run one after the other on the stream
  const uint64_t slice = mass_slice_bytes(ctx);
  auto wgs_cap = [&](int n) -> uint64_t {
    const uint64_t fixed = mass_ws_bytes(ctx, n, 0) + 256;
    if (fixed + slice > kNoAllocScratchBytes) return 0;
    return slice ? (kNoAllocScratchBytes - fixed) / slice : ~0ull;
  };
  int nl = g.L;
  while (nl > 0 && wgs_cap(nl) == 0) --nl;
  if (nl == 0)
    return fail(FERRY_EINVAL, "ferry_select_mass_noalloc: the workspace of one layer (" +
                                  std::to_string(mass_ws_bytes(ctx, 1, 1)) +
                                  " B) exceeds the static scratch of " +
                                  std::to_string(kNoAllocScratchBytes) + " B");
  for (int l0 = 0; l0 < g.L; l0 += nl) {
    const int n = std::min(nl, g.L - l0);
    if (int rc = launch_select_mass(ctx, l0, n, q, ctx_blocks, sel, stream, ctx->scratch_dev,
                                    mass_wgs(ctx, n, wgs_cap(n))))
      return rc;
  }
  return FERRY_OK;
}

int ferry_owner_image_bytes(const ferry_ctx* ctx, uint64_t* bytes) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!bytes) return fail(FERRY_EINVAL, "null out");
  *bytes = make_image_layout(ctx->g).bytes;
  return FERRY_OK;
}

}  // extern "C"

namespace {

int owner_check(ferry_ctx* ctx, uint32_t owner, const void* image, uint64_t image_bytes) {
  if (int rc = check_buf(image, "image")) return rc;
  if (owner >= (uint32_t)ctx->g.n_owners) return fail(FERRY_EINVAL, "owner out of range");
  if (image_bytes < make_image_layout(ctx->g).bytes)
    return fail(FERRY_EINVAL, "image buffer smaller than ferry_owner_image_bytes");
  if ((uintptr_t)image % 256) return fail(FERRY_EINVAL, "image must be 256-byte aligned");
  return FERRY_OK;
}

}  // namespace

extern "C" {

int ferry_owner_export(ferry_ctx* ctx, uint32_t owner, void* image, uint64_t image_bytes, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = owner_check(ctx, owner, image, image_bytes)) return rc;
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* im = (uint8_t*)image;
  hipLaunchKernelGGL(k_owner_export_meta, dim3(1), dim3(256), 0, s, g, ctx->st, owner, im,
                     (const uint32_t*)nullptr, 0u);
  HIPC(hipGetLastError());
  const uint64_t waves = (uint64_t)g.L * g.Hkv * g.C;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  switch (g.bb / 1024) {
    case 4: hipLaunchKernelGGL(k_owner_export_data<4>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    case 8: hipLaunchKernelGGL(k_owner_export_data<8>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    case 16: hipLaunchKernelGGL(k_owner_export_data<16>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_owner_import(ferry_ctx* ctx, uint32_t owner, const void* image, uint64_t image_bytes,
                       void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (int rc = owner_check(ctx, owner, image, image_bytes)) return rc;
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* im = (const uint8_t*)image;
  const unsigned sets = (unsigned)(g.L * g.Hkv);
  hipLaunchKernelGGL(k_owner_import_meta, dim3(sets), dim3(256), 0, s, g, ctx->st, owner, im,
                     ctx->err);
  HIPC(hipGetLastError());
  const uint64_t waves = (uint64_t)sets * g.C;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  switch (g.bb / 1024) {
    case 4: hipLaunchKernelGGL(k_owner_import_data<4>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    case 8: hipLaunchKernelGGL(k_owner_import_data<8>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    case 16: hipLaunchKernelGGL(k_owner_import_data<16>, grid, block, 0, s, g, ctx->st, owner, ctx->pool, ctx->pool_scales, im); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  return FERRY_OK;
}

}  // extern "C"

namespace {

int member_check(ferry_ctx* ctx, uint32_t lane, const void* image, uint64_t image_bytes) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!ctx->st.own) return fail(FERRY_EINVAL, "member carry needs prefix groups (group > 1)");
  if (lane >= (uint32_t)ctx->g.n_req) return fail(FERRY_EINVAL, "lane out of range");
  return owner_check(ctx, lane / (uint32_t)ctx->g.group, image, image_bytes);
}

}  // namespace

extern "C" {

int ferry_owner_export_member(ferry_ctx* ctx, uint32_t lane, void* image, uint64_t image_bytes,
                              void* stream) {
  if (int rc = member_check(ctx, lane, image, image_bytes)) return rc;
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  uint8_t* im = (uint8_t*)image;
  const uint32_t owner = lane / (uint32_t)g.group, bit = 1u << (lane % (uint32_t)g.group);
  const unsigned sets = (unsigned)(g.L * g.Hkv);
  const dim3 grid((sets + 3) / 4), block(256);
  hipLaunchKernelGGL(k_member_export_count, grid, block, 0, s, g, ctx->st, owner, bit, im);
  HIPC(hipGetLastError());
  const uint32_t* counts = (const uint32_t*)(im + make_image_layout(g).fill);
  hipLaunchKernelGGL(k_owner_export_meta, dim3(1), dim3(256), 0, s, g, ctx->st, owner, im, counts, bit);
  HIPC(hipGetLastError());
  switch (g.bb / 1024) {
    case 4: hipLaunchKernelGGL(k_member_export_data<4>, grid, block, 0, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im); break;
    case 8: hipLaunchKernelGGL(k_member_export_data<8>, grid, block, 0, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im); break;
    case 16: hipLaunchKernelGGL(k_member_export_data<16>, grid, block, 0, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_owner_import_member(ferry_ctx* ctx, uint32_t lane, const void* image, uint64_t image_bytes,
                              void* stream) {
  if (int rc = member_check(ctx, lane, image, image_bytes)) return rc;
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* im = (const uint8_t*)image;
  const uint32_t owner = lane / (uint32_t)g.group, bit = 1u << (lane % (uint32_t)g.group);
  const dim3 grid((unsigned)(g.L * g.Hkv)), block(64);
  const size_t lds = 2 * (size_t)g.C * 4;
  switch (g.bb / 1024) {
    case 4: hipLaunchKernelGGL(k_member_import<4>, grid, block, lds, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im, ctx->err); break;
    case 8: hipLaunchKernelGGL(k_member_import<8>, grid, block, lds, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im, ctx->err); break;
    case 16: hipLaunchKernelGGL(k_member_import<16>, grid, block, lds, s, g, ctx->st, owner, bit, ctx->pool, ctx->pool_scales, im, ctx->err); break;
    default: return fail(FERRY_EINVAL, "unsupported block size");
  }
  HIPC(hipGetLastError());
  return FERRY_OK;
}

int ferry_bw_probe(ferry_ctx* ctx, int kind, const uint32_t* slots, uint64_t n, int iters,
                   uint64_t* bytes, float* ms, void* stream) {
  if (int rc = check_ctx(ctx)) return rc;
  if (kind < FERRY_PROBE_HBM_GATHER || kind > FERRY_PROBE_SUMS_READ) return fail(FERRY_EINVAL, "bad kind");
  if (n < 1 || iters < 1) return fail(FERRY_EINVAL, "n and iters must be positive");
  if (kind == FERRY_PROBE_HBM_GATHER && (check_buf(slots, "slots") || n > 0x7FFFFFFFull))
    return fail(FERRY_EINVAL, "gather needs a device slot table of at most 2^31 rows");
  if ((kind == FERRY_PROBE_HOST_READ || kind == FERRY_PROBE_HOST_DMA) && n > ctx->g.host_blocks)
    return fail(FERRY_EINVAL, "more blocks than the host tier holds");
  if (kind == FERRY_PROBE_HBM_COPY && n > ctx->g.pool_slots)
    return fail(FERRY_EINVAL, "more blocks than the pool holds");
  if (kind == FERRY_PROBE_KTAB_READ && (!ctx->ktab || n > (uint64_t)ctx->g.max_blocks))
    return fail(FERRY_EINVAL, "the K-table probe needs ferry_ktiles_build and n <= max_blocks");
  if (kind == FERRY_PROBE_SUMS_READ && (!ctx->sums || !ctx->sum_blocks || n > (uint64_t)ctx->g.max_blocks))
    return fail(FERRY_EINVAL, "the summary probe needs ferry_summaries_build and n <= max_blocks");
  const Geo& g = ctx->g;
  HIPC(hipSetDevice(ctx->device));
  hipStream_t s = (hipStream_t)stream;
  const int host_waves = g.workers * 4;
  // the K-table probe: the mass selection's order and wavefronts; for 16-bit
  // and fp8 records one workgroup per (request, layer, kv head) unit, which
  // the GPU dispatches in unit order as k_mass_units takes them
  const int kt_w = g.dtype == FERRY_F32 ? 4 : kMassUnitWaves;
  const uint64_t kt_grid = g.dtype == FERRY_F32 ? mass_wgs(ctx, g.L, ~0ull)
                                                : (uint64_t)g.n_req * g.L * g.Hkv;
  // and as many of its workgroups per CU as of k_mass_units (unused LDS
  // reserved for the purpose: the probe needs fewer registers)
  size_t kt_lds = 0;
  if (kind == FERRY_PROBE_KTAB_READ && g.dtype != FERRY_F32) {
    const int per_cu = std::max(1, mass_units_resident(ctx) / std::max(1, ctx->cus));
    kt_lds = (size_t)kGroupMaxLds / (size_t)per_cu / 256 * 256;
  }
  // the summary probe: k_select_topk's grid (one workgroup per set) with its
  // LDS, so as many of its workgroups share a CU
  const uint64_t sum_grid = (uint64_t)g.n_req * g.L * g.Hkv;
  const size_t sum_lds = ((size_t)(g.Hq / g.Hkv) * g.D + (size_t)g.max_blocks) * 4;
  if (kind == FERRY_PROBE_SUMS_READ && sum_lds > 65536)
    return fail(FERRY_EINVAL, "max_blocks exceeds the selection's 64 KiB of LDS");
  const size_t words = kind == FERRY_PROBE_HBM_GATHER ? (size_t)n
                       : kind == FERRY_PROBE_KTAB_READ ? (size_t)(kt_grid * kt_w)
                       : kind == FERRY_PROBE_SUMS_READ ? (size_t)(sum_grid * 4)
                                                       : (size_t)host_waves;
  if (ctx->probe_sink_words < words) {
    if (ctx->probe_sink) HIPC(hipFree(ctx->probe_sink));
    ctx->probe_sink = nullptr;
    ctx->probe_sink_words = 0;
    HIPC(hipMalloc(&ctx->probe_sink, words * 4));
    ctx->probe_sink_words = words;
  }
  // bytes per launch: read, plus written for the device copy
  const uint64_t moved = kind == FERRY_PROBE_HBM_GATHER ? n * (uint64_t)g.k * g.bb
                         : kind == FERRY_PROBE_HBM_COPY ? 2 * n * g.bb
                         : kind == FERRY_PROBE_KTAB_READ
                             ? (uint64_t)g.n_req * g.L * g.Hkv * n * (g.bb / 2)
                         : kind == FERRY_PROBE_SUMS_READ
                             ? sum_grid * n * (uint64_t)(2 * g.D * g.esize)
                             : n * g.bb;
  const uint64_t dst_bytes = n * g.bb;
  if ((kind == FERRY_PROBE_HOST_DMA || kind == FERRY_PROBE_HBM_COPY) && ctx->probe_dst_bytes < dst_bytes) {
    if (ctx->probe_dst) HIPC(hipFree(ctx->probe_dst));
    ctx->probe_dst = nullptr;
    ctx->probe_dst_bytes = 0;
    HIPC(hipMalloc(&ctx->probe_dst, dst_bytes));
    ctx->probe_dst_bytes = dst_bytes;
  }
  const int nld = (int)(g.bb / 1024);
  if (nld != 4 && nld != 8 && nld != 16) return fail(FERRY_EINVAL, "unsupported block size");
  auto launch = [&]() -> hipError_t {
    if (kind == FERRY_PROBE_HBM_GATHER) {
      const dim3 grid((unsigned)n), block(256);
      if (nld == 4)
        hipLaunchKernelGGL(k_probe_gather<4>, grid, block, 0, s, ctx->pool, g.bb, slots, g.k, g.pool_slots, ctx->probe_sink);
      else if (nld == 8)
        hipLaunchKernelGGL(k_probe_gather<8>, grid, block, 0, s, ctx->pool, g.bb, slots, g.k, g.pool_slots, ctx->probe_sink);
      else
        hipLaunchKernelGGL(k_probe_gather<16>, grid, block, 0, s, ctx->pool, g.bb, slots, g.k, g.pool_slots, ctx->probe_sink);
      return hipGetLastError();
    }
    if (kind == FERRY_PROBE_HOST_READ) {
      const dim3 grid((unsigned)g.workers), block(256);
      if (nld == 4)
        hipLaunchKernelGGL(k_probe_host<4>, grid, block, 0, s, ctx->host_dev, g.bb, n, ctx->probe_sink);
      else if (nld == 8)
        hipLaunchKernelGGL(k_probe_host<8>, grid, block, 0, s, ctx->host_dev, g.bb, n, ctx->probe_sink);
      else
        hipLaunchKernelGGL(k_probe_host<16>, grid, block, 0, s, ctx->host_dev, g.bb, n, ctx->probe_sink);
      return hipGetLastError();
    }
    if (kind == FERRY_PROBE_KTAB_READ) {
      const dim3 grid((unsigned)kt_grid);
      const int nb = (int)n;
      if (g.dtype == FERRY_F32)
        hipLaunchKernelGGL((k_probe_ktab<8, 4, 4, 0>), grid, dim3(256), 0, s, g, ctx->ktab,
                           ctx->kt_records, nb, ctx->probe_sink);
      else if (g.dtype == FERRY_FP8_E4M3)
        hipLaunchKernelGGL((k_probe_ktab<2, kMassUnitWaves, kMassUnitInflight, 1>), grid,
                           dim3(64 * kMassUnitWaves), kt_lds, s, g, ctx->ktab, ctx->kt_records, nb,
                           ctx->probe_sink);
      else
        hipLaunchKernelGGL((k_probe_ktab<4, kMassUnitWaves, kMassUnitInflight, 1>), grid,
                           dim3(64 * kMassUnitWaves), kt_lds, s, g, ctx->ktab, ctx->kt_records, nb,
                           ctx->probe_sink);
      return hipGetLastError();
    }
    if (kind == FERRY_PROBE_SUMS_READ) {
      const dim3 grid((unsigned)sum_grid), block(256);
      const int nb = (int)n, es = g.esize;
      const bool u2 = g.Hq / g.Hkv >= 8;  // k_select_topk's passes in flight
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, sum_lds, s, g, ctx->sums, ctx->sum_blocks, nb,
                           ctx->probe_sink);
      };
      if (es == 1) u2 ? go(k_probe_sums<1, 2>) : go(k_probe_sums<1, 4>);
      else if (es == 2) u2 ? go(k_probe_sums<2, 2>) : go(k_probe_sums<2, 4>);
      else u2 ? go(k_probe_sums<4, 2>) : go(k_probe_sums<4, 4>);
      return hipGetLastError();
    }
    if (kind == FERRY_PROBE_HBM_COPY) {
      const dim3 grid((unsigned)std::min<uint64_t>((n + 3) / 4, 8192)), block(256);
      if (nld == 4)
        hipLaunchKernelGGL(k_probe_copy<4>, grid, block, 0, s, ctx->pool, ctx->probe_dst, g.bb, n);
      else if (nld == 8)
        hipLaunchKernelGGL(k_probe_copy<8>, grid, block, 0, s, ctx->pool, ctx->probe_dst, g.bb, n);
      else
        hipLaunchKernelGGL(k_probe_copy<16>, grid, block, 0, s, ctx->pool, ctx->probe_dst, g.bb, n);
      return hipGetLastError();
    }
    return hipMemcpyAsync(ctx->probe_dst, ctx->host, dst_bytes, hipMemcpyHostToDevice, s);
  };
  HIPC(launch());  // warm-up
  Scratch sc;
  hipEvent_t e0, e1;
  HIPC(hipEventCreate(&e0));
  sc.events.push_back(e0);
  HIPC(hipEventCreate(&e1));
  sc.events.push_back(e1);
  HIPC(hipEventRecord(e0, s));
  for (int i = 0; i < iters; ++i) HIPC(launch());
  HIPC(hipEventRecord(e1, s));
  HIPC(hipEventSynchronize(e1));
  float t = 0.0f;
  HIPC(hipEventElapsedTime(&t, e0, e1));
  if (bytes) *bytes = moved;
  if (ms) *ms = t / (float)iters;
  return FERRY_OK;
}

int ferry_stats_get(ferry_ctx* ctx, ferry_stats* out) {
  if (int rc = check_ctx(ctx)) return rc;
  if (!out) return fail(FERRY_EINVAL, "null out");
  HIPC(hipSetDevice(ctx->device));
  HIPC(hipDeviceSynchronize());
  unsigned long long s[kStatCount];
  std::vector<unsigned long long> sc((size_t)kSelCounters * kSelStride);
  int err = 0;
  HIPC(hipMemcpy(s, ctx->stats, sizeof(s), hipMemcpyDeviceToHost));
  HIPC(hipMemcpy(sc.data(), ctx->sel_counts, sc.size() * 8, hipMemcpyDeviceToHost));
  unsigned long long nsel = 0;
  for (int i = 0; i < kSelCounters; ++i) nsel += sc[(size_t)i * kSelStride];
  HIPC(hipMemcpy(&err, ctx->err, 4, hipMemcpyDeviceToHost));
  std::memset(out, 0, sizeof(*out));
  out->steps = ctx->steps;
  out->selections = nsel;
  out->misses = s[kStatMisses];
  out->fetched_bytes = s[kStatBytes];
  out->steals = s[kStatSteals];
  out->stolen = s[kStatStolen];
  out->last_misses = s[kStatLast];
  out->device_error = err;
  return FERRY_OK;
}

int ferry_stats_reset(ferry_ctx* ctx) {
  if (int rc = check_ctx(ctx)) return rc;
  HIPC(hipSetDevice(ctx->device));
  HIPC(hipDeviceSynchronize());
  HIPC(hipMemset(ctx->stats, 0, kStatCount * 8));
  HIPC(hipMemset(ctx->sel_counts, 0, (size_t)kSelCounters * kSelStride * 8));
  HIPC(hipMemset(ctx->err, 0, 4));
  ctx->steps = 0;
  return FERRY_OK;
}

int ferry_queue_selftest(int device, uint64_t capacity, uint64_t n_tasks, int producers,
                         int consumers, int mode, uint64_t* popped, uint64_t* duplicates,
                         float* ms) {
  if (producers < 256 || consumers < 256 || producers % 256 || consumers % 256)
    return fail(FERRY_EINVAL, "producers/consumers must be positive multiples of 256");
  if (producers + consumers > 8192) return fail(FERRY_EINVAL, "at most 8192 threads (co-residency)");
  if (n_tasks == 0 || n_tasks % (uint64_t)producers) return fail(FERRY_EINVAL, "n_tasks must be a multiple of producers");
  if (n_tasks > (1ull << 28)) return fail(FERRY_EINVAL, "n_tasks too large");
  if (mode != 0 && mode != 1) return fail(FERRY_EINVAL, "bad mode");
  HIPC(hipSetDevice(device));
  ferry::GPUBoundedQueue q(capacity, mode ? ferry::ReservationMode::kWaveBatched
                                          : ferry::ReservationMode::kPerThread);
  if (!q.ok()) return fail(FERRY_ENOMEM, "queue allocation failed");
  Scratch sc;
  uint32_t* seen = nullptr;
  unsigned long long* counters = nullptr;
  int* flags = nullptr;
  HIPC(hipMalloc(&seen, n_tasks * 4));
  sc.bufs.push_back(seen);
  HIPC(hipMalloc(&counters, 16));
  sc.bufs.push_back(counters);
  HIPC(hipMalloc(&flags, 8));
  sc.bufs.push_back(flags);
  HIPC(hipMemset(seen, 0, n_tasks * 4));
  HIPC(hipMemset(counters, 0, 16));
  HIPC(hipMemset(flags, 0, 8));
  hipEvent_t e0, e1;
  HIPC(hipEventCreate(&e0));
  sc.events.push_back(e0);
  HIPC(hipEventCreate(&e1));
  sc.events.push_back(e1);
  const uint32_t pb = producers / 256, cb = consumers / 256;
  HIPC(hipEventRecord(e0, 0));
  hipLaunchKernelGGL(k_queue_pc, dim3(pb + cb), dim3(256), 0, 0, q.device_ptr(),
                     n_tasks / (uint64_t)producers, pb, seen, counters, counters + 1, flags, flags + 1,
                     q.mode());
  HIPC(hipGetLastError());
  HIPC(hipEventRecord(e1, 0));
  HIPC(hipEventSynchronize(e1));
  float t = 0.0f;
  HIPC(hipEventElapsedTime(&t, e0, e1));
  unsigned long long c[2];
  HIPC(hipMemcpy(c, counters, 16, hipMemcpyDeviceToHost));
  // every id must have arrived exactly once
  std::vector<uint32_t> h(n_tasks);
  HIPC(hipMemcpy(h.data(), seen, n_tasks * 4, hipMemcpyDeviceToHost));
  uint64_t missing = 0, twice = 0;
  for (uint32_t v : h) {
    missing += v == 0;
    twice += v > 1;
  }
  c[1] += twice;
  const auto snap = q.snapshot();
  if (popped) *popped = c[0];
  if (duplicates) *duplicates = c[1];
  if (ms) *ms = t;
  if (snap.status) return fail(FERRY_ESPIN, "queue wait bound exceeded (status " + std::to_string(snap.status) + ")");
  if (missing) return fail(FERRY_ESTATE, std::to_string(missing) + " task ids never popped");
  return FERRY_OK;
}

int ferry_queue_ticket_probe(int device, int threads, int iters, int kind, uint64_t* tickets,
                             float* ms) {
  if (threads < 256 || threads % 256 || threads > 8192)
    return fail(FERRY_EINVAL, "threads must be a multiple of 256, at most 8192");
  if (iters < 1 || iters > (1 << 20)) return fail(FERRY_EINVAL, "iters must be in [1, 2^20]");
  if (kind < 0 || kind > 2) return fail(FERRY_EINVAL, "bad kind");
  HIPC(hipSetDevice(device));
  Scratch sc;
  unsigned long long* word = nullptr;
  HIPC(hipMalloc(&word, 16));
  sc.bufs.push_back(word);
  HIPC(hipMemset(word, 0, 16));
  int* failed = reinterpret_cast<int*>(word + 1);
  hipEvent_t e0, e1;
  HIPC(hipEventCreate(&e0));
  sc.events.push_back(e0);
  HIPC(hipEventCreate(&e1));
  sc.events.push_back(e1);
  HIPC(hipEventRecord(e0, 0));
  hipLaunchKernelGGL(k_ticket_probe, dim3(threads / 256), dim3(256), 0, 0, word, iters, kind, failed);
  HIPC(hipGetLastError());
  HIPC(hipEventRecord(e1, 0));
  HIPC(hipEventSynchronize(e1));
  float t = 0.0f;
  HIPC(hipEventElapsedTime(&t, e0, e1));
  unsigned long long h[2];
  HIPC(hipMemcpy(h, word, 16, hipMemcpyDeviceToHost));
  if (tickets) *tickets = h[0];
  if (ms) *ms = t;
  if ((int)h[1] == 1) return fail(FERRY_ESPIN, "ticket retries exceeded the spin bound");
  if (h[0] != (uint64_t)threads * iters) return fail(FERRY_ESTATE, "ticket count mismatch");
  return FERRY_OK;
}

}  // extern "C"
