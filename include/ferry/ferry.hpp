// ferry.hpp -- the reference's workload/executor C++ names over the C-ABI.
//
// Header-only C++17 (compile with hipcc, link libferry_amd.so).  Keeps the
// names, fields and argument meanings of the reference's
// src/workloads/missstream.cuh (MissSpec, MissEvent, MissTrace,
// replay_miss_stream, wla_group_cap), src/workloads/miss_trace.cuh
// (MissTraceInfo, load_miss_trace, fnv1a64_file, ferry_miss_trace_path),
// src/runtime/adaptive_batch.cuh (AdaptiveBatchPolicy, MoveStrategy),
// src/workloads/kv_exec.cuh (WlAStats, slab_offset, run_miss_workload) and
// the one-GPU slice of src/runtime/wla_multigpu.cuh (WlaKvMode,
// WlaStealPolicy, WlaMultiStats, run_wla_multigpu) so that code written
// against them builds unchanged; the work runs on the gfx950 path.
// cache_slot_off has no counterpart: pool slots are assigned by LRU, not
// direct-mapped.
//
// Differences a caller can observe:
//  * replay_miss_stream computes is_miss with the GPU bookkeeping kernel in
//    per-selection (serial) LRU mode; the stream is identical to the
//    reference's (tests/test_driver.py checks 589,824 / 79,550).
//  * run_miss_workload moves each (request, layer, block) miss as one block of
//    the HBM pool (fp32 blocks of 16 tokens x 128 dims = 16 KiB, the
//    reference's c4 at its defaults) and runs real attention over the
//    selected blocks instead of the FMA proxy (attn_iters, the proxy's FMA
//    count, has nothing to set).  refill_events / refill_bytes keep the
//    reference's meaning per mode -- A: one per selected block, hits
//    included; B: one per miss; C: one per submit of the coalesced,
//    policy-batched step misses -- although the GPU moves every missing
//    block with device-direct reads and has no submits; the blocks it
//    actually moved are WlAStats::fetched_blocks / WlaMultiStats::
//    fetched_blocks.
//  * errors are reported through WlAStats::status / MissTrace::status /
//    WlaMultiStats::status (a FERRY_E* code) instead of exiting the process.
//  * run_wla_multigpu accepts exactly one device: it is the per-GPU executor
//    (tick loop over resident requests) without the cross-GPU control plane.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <thread>
#include <vector>

#include "../ferry_amd.h"
#include "common.hpp"

namespace ferry {

struct MissSpec {
  int num_requests = 4;
  int num_layers = 12;
  int steps = 64;
  int sel_blocks = 128;
  int hot_blocks = 512;
  int kv_heads = 8;
  int head_dim = 128;
  std::string arrival = "steady";
  uint64_t seed = 42;
  int prefix_group = 1;
  int prefix_steps = 8;
  int cap_mode = 0;
  int own_carry = 0;
  int slab_blocks = 0;
  size_t c4_bytes() const { return (size_t)4 * 2 * kv_heads * head_dim * 2; }
  std::vector<int> len;
};

inline int wla_len_of(const MissSpec& sp, int r) { return sp.len.empty() ? sp.steps : sp.len[(size_t)r]; }

struct MissEvent {
  int req, layer, step;
  uint64_t block_id;
  bool is_miss;
};

inline int wla_group_cap(const MissSpec& sp, int members) {
  if (sp.cap_mode != 1) return sp.hot_blocks;
  return sp.hot_blocks * (members > 0 ? members : 1);
}

struct MissTrace {
  std::vector<MissEvent> events;
  uint64_t total_selects = 0;
  uint64_t total_misses = 0;
  uint64_t miss_bytes = 0;
  double hit_rate = 0.0;
  int status = FERRY_OK;
};

enum class MoveStrategy { kNonBatched = 0, kFixed = 1, kAdaptive = 2 };

struct AdaptiveBatchPolicy {
  double min_mb = 1.0;
  double max_mb = 4.0;
  double target_batches = 4.0;
  double saturation_mb = 1.0;
  double choose_mb(double pending_mb) const {
    return std::min(std::max(pending_mb / target_batches, min_mb), max_mb);
  }
};

struct WlAStats {
  double makespan_ms = 0.0;
  double p50_step_ms = 0.0, p99_step_ms = 0.0;
  uint64_t refill_events = 0;  // the reference's transfer count of the mode
  uint64_t refill_bytes = 0;   // ... and its bytes
  double throughput_steps = 0.0;
  uint64_t fetched_blocks = 0;  // blocks the GPU fetch moved into the pool
  int status = FERRY_OK;
};

// Host-tier and pool offsets of (request, layer, block) in this library's
// layout (one set per (request, layer), one pool slot per block).
inline size_t slab_offset(const MissSpec& sp, int req, int layer, uint64_t block) {
  const uint64_t max_blocks = 64 + (uint64_t)sp.steps * 8;
  return ((size_t)(req * sp.num_layers + layer) * max_blocks + block) * sp.c4_bytes();
}

namespace detail {

// One executor of the reference geometry: sets = (request or prefix group,
// layer), one kv head, k = sel_blocks selections per step, C = hot slots,
// fp32 16-token blocks (16 KiB, the reference's c4 at its defaults).
struct Exec {
  ferry_ctx* ctx = nullptr;
  uint32_t *sel = nullptr, *slots = nullptr, *mc = nullptr;
  ferry_miss* misses = nullptr;
  uint8_t* flags = nullptr;
  float *q = nullptr, *out = nullptr;
  int status = FERRY_OK;
  uint32_t n_sets = 0, max_sel = 0;

  Exec(const MissSpec& sp, int device, int lru_mode, int hot, int max_blocks = 0, int group = 1,
       int cap_mode = FERRY_CAP_GROUP) {
    ferry_config c{};
    c.n_req = sp.num_requests;
    c.group = group;
    c.cap_mode = cap_mode;
    c.n_layers = sp.num_layers;
    c.kv_heads = 1;
    c.q_heads = 1;
    c.head_dim = 128;
    c.block_tokens = 16;
    c.k = sp.sel_blocks;
    c.slots_per_set = hot;
    c.max_blocks = max_blocks > 0 ? max_blocks : (int)(64 + (uint64_t)sp.steps * 8);
    c.dtype = FERRY_F32;
    c.lru_mode = lru_mode;
    c.host_blocks = 1 << 14;
    c.host_seed = 11;
    c.value_std = 1.0f;
    c.steal = 1;
    c.assign = FERRY_ASSIGN_SPREAD;
    if ((status = ferry_ctx_create(&c, device, &ctx))) return;
    uint64_t bb, ps;
    ferry_ctx_sizes(ctx, &n_sets, &max_sel, &bb, &ps);
    const size_t nsel = (size_t)sp.num_requests * sp.num_layers * sp.sel_blocks;
    const size_t nq = (size_t)sp.num_requests * sp.num_layers * 128;
    if (hipMalloc(&sel, nsel * 4) || hipMalloc(&slots, nsel * 4) || hipMalloc(&mc, n_sets * 4) ||
        hipMalloc(&misses, (size_t)n_sets * max_sel * sizeof(ferry_miss)) ||
        hipMalloc(&flags, nsel) || hipMalloc(&q, nq * 4) || hipMalloc(&out, nq * 4)) {
      status = FERRY_ENOMEM;
      return;
    }
    std::vector<float> hq(nq);
    for (size_t i = 0; i < nq; ++i) hq[i] = (float)((i * 2654435761u) % 1000) / 500.0f - 1.0f;
    if (hipMemcpy(q, hq.data(), nq * 4, hipMemcpyHostToDevice)) status = FERRY_EHIP;
    if (!status) status = ferry_hosttier_fill(ctx, nullptr);
  }
  ~Exec() {
    for (void* p : {(void*)sel, (void*)slots, (void*)mc, (void*)misses, (void*)flags, (void*)q, (void*)out})
      if (p) (void)hipFree(p);
    if (ctx) ferry_ctx_destroy(ctx);
  }
};

// Submits of one request-step under the reference's C engine
// (src/workloads/kv_exec.cuh:200-268, src/runtime/wla_multigpu.cuh:2529-2601):
// the step's misses over every layer, sorted by (layer, block) and
// deduplicated, are cut into batches of pol.choose_mb(pending) MB; inside a
// batch each run of consecutive blocks of one layer counts as one refill
// event (a run that would wrap the reference's direct-mapped slot range is
// sent block by block there, but is still counted once, kv_exec.cuh:250-266).
// `ml` holds (layer, block) and is reordered.  Returns the events and adds
// their bytes to *bytes.
inline uint64_t cmode_submits(std::vector<std::pair<int, uint64_t>>& ml, size_t c4,
                              const AdaptiveBatchPolicy& pol, uint64_t* bytes) {
  std::sort(ml.begin(), ml.end());
  ml.erase(std::unique(ml.begin(), ml.end()), ml.end());
  uint64_t submits = 0;
  const size_t n = ml.size();
  for (size_t i0 = 0; i0 < n;) {
    const double gmb = pol.choose_mb((double)(n - i0) * (double)c4 / 1048576.0);
    const size_t take = std::min(std::max<size_t>((size_t)(gmb * 1048576.0 / (double)c4), 1), n - i0);
    for (size_t k = 0; k < take;) {
      size_t run = 1;
      while (k + run < take && ml[i0 + k + run].first == ml[i0 + k].first &&
             ml[i0 + k + run].second == ml[i0 + k].second + run)
        ++run;
      ++submits;
      *bytes += run * c4;
      k += run;
    }
    i0 += take;
  }
  return submits;
}

// The (layer, block) misses of one owner in the last bookkeeping step, read
// back from the executor's per-set miss lists (kv_heads 1: set = owner * L +
// layer).
inline int owner_misses(const Exec& ex, int owner, int L, std::vector<uint32_t>& mc,
                        std::vector<ferry_miss>& ms, bool download,
                        std::vector<std::pair<int, uint64_t>>* out) {
  if (download) {
    if (hipMemcpy(mc.data(), ex.mc, mc.size() * 4, hipMemcpyDeviceToHost) ||
        hipMemcpy(ms.data(), ex.misses, ms.size() * sizeof(ferry_miss), hipMemcpyDeviceToHost))
      return FERRY_EHIP;
  }
  out->clear();
  for (int l = 0; l < L; ++l) {
    const size_t set = (size_t)owner * L + l;
    for (uint32_t i = 0; i < mc[set]; ++i) out->push_back({l, (uint64_t)ms[set * ex.max_sel + i].block});
  }
  return FERRY_OK;
}

}  // namespace detail

// Selections of the reference generator (missstream.cuh:104-133), hit/miss
// from the GPU's per-selection LRU of hot_blocks slots per (request, layer).
inline MissTrace replay_miss_stream(const MissSpec& spec, int device = 0) {
  MissTrace tr;
  const int R = spec.num_requests, L = spec.num_layers, S = spec.steps, G = spec.sel_blocks;
  std::vector<uint32_t> all((size_t)R * S * L * G);
  if ((tr.status = ferry_refgen_selections(R, L, S, G, spec.seed, all.data()))) return tr;
  detail::Exec ex(spec, device, FERRY_LRU_SERIAL, spec.hot_blocks);
  if ((tr.status = ex.status)) return tr;
  std::vector<uint32_t> step((size_t)R * L * G);
  std::vector<uint8_t> flags(step.size());
  std::vector<uint8_t> miss(all.size());
  for (int s = 0; s < S; ++s) {
    for (int r = 0; r < R; ++r)
      std::copy_n(all.data() + ((size_t)r * S + s) * L * G, (size_t)L * G, step.data() + (size_t)r * L * G);
    if (hipMemcpy(ex.sel, step.data(), step.size() * 4, hipMemcpyHostToDevice)) {
      tr.status = FERRY_EHIP;
      return tr;
    }
    if ((tr.status = ferry_fetch_step(ex.ctx, ex.sel, ex.slots, ex.mc, ex.misses, ex.flags, nullptr))) return tr;
    if (hipMemcpy(flags.data(), ex.flags, flags.size(), hipMemcpyDeviceToHost)) {
      tr.status = FERRY_EHIP;
      return tr;
    }
    for (int r = 0; r < R; ++r)
      std::copy_n(flags.data() + (size_t)r * L * G, (size_t)L * G, miss.data() + ((size_t)r * S + s) * L * G);
  }
  ferry_stats st{};
  ferry_stats_get(ex.ctx, &st);
  if (st.device_error) {
    tr.status = st.device_error;
    return tr;
  }
  tr.events.reserve(all.size());
  size_t i = 0;
  for (int r = 0; r < R; ++r)
    for (int s = 0; s < S; ++s)
      for (int l = 0; l < L; ++l)
        for (int k = 0; k < G; ++k, ++i) {
          tr.events.push_back({r, l, s, (uint64_t)all[i], miss[i] != 0});
          ++tr.total_selects;
          if (miss[i]) {
            ++tr.total_misses;
            tr.miss_bytes += spec.c4_bytes();
          }
        }
  tr.hit_rate = tr.total_selects ? 1.0 - (double)tr.total_misses / (double)tr.total_selects : 0.0;
  return tr;
}

// Executes a trace on `dst_dev` (src_dev is unused: the host tier is pinned
// memory visible to the device).  mode 0 (A): no reuse, every distinct
// selection of a step is fetched; modes 1 (B) and 2 (C): per-selection LRU of
// hot_blocks slots, one fetch launch per step (B's per-miss submits modelled
// the host-staged channel, which this library does not have).  Each step then
// runs sparse attention over the selected blocks.  The refill counters are
// the reference's (src/workloads/kv_exec.cuh:108-145, 148-185, 188-292): A
// counts every selected block, B every miss, C the submits of each
// request-step's coalesced misses under `pol` (cmode_submits, computed from
// the executor's own miss lists after each step, outside its timing).
inline WlAStats run_miss_workload(int src_dev, int dst_dev, const MissSpec& sp, const MissTrace& tr,
                                  int mode, const AdaptiveBatchPolicy& pol, int attn_iters = 8) {
  (void)src_dev;
  (void)attn_iters;
  WlAStats st;
  const int R = sp.num_requests, L = sp.num_layers, S = sp.steps, G = sp.sel_blocks;
  if (tr.events.size() != (size_t)R * S * L * G || mode < 0 || mode > 2) {
    st.status = FERRY_EINVAL;
    return st;
  }
  const int hot = mode == 0 ? std::max(G, 1) : sp.hot_blocks;
  detail::Exec ex(sp, dst_dev, FERRY_LRU_SERIAL, hot);
  if ((st.status = ex.status)) return st;
  std::vector<uint32_t> step((size_t)R * L * G);
  std::vector<uint32_t> mc(ex.n_sets);
  std::vector<ferry_miss> ms((size_t)ex.n_sets * ex.max_sel);
  std::vector<std::pair<int, uint64_t>> ml;
  std::vector<double> step_ms;
  uint64_t c_events = 0, c_bytes = 0;
  HostTimer ht;  // the makespan and each step's interval, as the reference times them
  for (int s = 0; s < S; ++s) {
    const double ts = ht.toc_ms();
    for (int r = 0; r < R; ++r)
      for (int l = 0; l < L; ++l)
        for (int k = 0; k < G; ++k)
          step[((size_t)r * L + l) * G + k] = (uint32_t)tr.events[(((size_t)r * S + s) * L + l) * G + k].block_id;
    if (hipMemcpy(ex.sel, step.data(), step.size() * 4, hipMemcpyHostToDevice)) {
      st.status = FERRY_EHIP;
      return st;
    }
    if (mode == 0 && (st.status = ferry_sets_reset(ex.ctx, nullptr))) return st;
    if ((st.status = ferry_bookkeep_step(ex.ctx, ex.sel, ex.slots, ex.mc, ex.misses, nullptr, nullptr))) return st;
    if ((st.status = ferry_missq_drain(ex.ctx, nullptr))) return st;
    if ((st.status = ferry_sparse_decode(ex.ctx, ex.q, ex.slots, ex.out, nullptr))) return st;
    if (hipDeviceSynchronize()) {
      st.status = FERRY_EHIP;
      return st;
    }
    step_ms.push_back(ht.toc_ms() - ts);
    if (mode == 2)
      for (int r = 0; r < R; ++r) {
        if ((st.status = detail::owner_misses(ex, r, L, mc, ms, r == 0, &ml))) return st;
        c_events += detail::cmode_submits(ml, sp.c4_bytes(), pol, &c_bytes);
      }
  }
  st.makespan_ms = ht.toc_ms();
  ferry_stats fs{};
  ferry_stats_get(ex.ctx, &fs);
  if (fs.device_error) st.status = fs.device_error;
  st.fetched_blocks = fs.misses;
  if (mode == 0) {  // one synchronous copy per selected block, hits included
    st.refill_events = (uint64_t)tr.events.size();
    st.refill_bytes = st.refill_events * sp.c4_bytes();
  } else if (mode == 1) {  // one channel submit per miss
    st.refill_events = fs.misses;
    st.refill_bytes = fs.misses * sp.c4_bytes();
  } else {
    st.refill_events = c_events;
    st.refill_bytes = c_bytes;
  }
  st.throughput_steps = st.makespan_ms > 0 ? (double)(R * S) / (st.makespan_ms / 1000.0) : 0.0;
  std::sort(step_ms.begin(), step_ms.end());
  if (!step_ms.empty()) {
    st.p50_step_ms = step_ms[step_ms.size() / 2];
    st.p99_step_ms = step_ms[(size_t)(0.99 * (step_ms.size() - 1))];
  }
  return st;
}

// ---------------------------------------------------------------- real traces
// src/workloads/miss_trace.cuh:28-35
struct MissTraceInfo {
  std::string path;
  int requests = 0, steps = 0, layers = 0;
  int page_tokens = 0, block_tokens = 0, sel_pages = 0;
  int kv_heads = 0, head_dim = 0;
  uint64_t unique_blocks = 0;
  uint64_t max_blocks_per_req = 0;
};

// FERRY_MISS_TRACE=<path.bin> selects a real trace (miss_trace.cuh:37-43).
inline bool ferry_miss_trace_path(std::string* out) {
  const char* p = std::getenv("FERRY_MISS_TRACE");
  if (!p || !*p) return false;
  *out = p;
  return true;
}

// FNV-1a 64 of a file's bytes (0 if it cannot be opened), as the reference
// fingerprints traces (miss_trace.cuh:45-62).
inline uint64_t fnv1a64_file(const std::string& path, uint64_t* size_out = nullptr) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return 0;
  uint64_t h = 0xcbf29ce484222325ull, n = 0;
  std::vector<unsigned char> buf(1 << 20);
  size_t got;
  while ((got = std::fread(buf.data(), 1, buf.size(), f)) > 0) {
    for (size_t i = 0; i < got; ++i) {
      h ^= buf[i];
      h *= 0x100000001b3ull;
    }
    n += got;
  }
  std::fclose(f);
  if (size_out) *size_out = n;
  return h;
}

namespace detail {

// Read a trace and check it against the spec as load_miss_trace does
// (miss_trace.cuh:94-103); ids are dense, (r, s, l, k) order.
inline int read_trace(const std::string& path, const MissSpec& spec, ferry_trace_info* ti,
                      std::vector<uint32_t>* ids) {
  int rc = ferry_trace_load(path.c_str(), 1, ti, nullptr, 0);
  if (rc) return rc;
  const bool ok = (int)ti->requests == spec.num_requests && (int)ti->steps == spec.steps &&
                  (int)ti->layers == spec.num_layers && (int)ti->kv_heads == spec.kv_heads &&
                  (int)ti->head_dim == spec.head_dim && ti->block_tokens == 4 &&
                  (int)ti->sel_blocks == spec.sel_blocks;
  if (!ok) return FERRY_EINVAL;  // the reference aborts: trace and spec disagree
  ids->resize((size_t)ti->requests * ti->steps * ti->layers * ti->sel_blocks);
  return ferry_trace_load(path.c_str(), 1, ti, ids->data(), ids->size());
}

// Per-(request, layer) LRU flags of an (r, s, l, k) id stream, computed on
// the GPU with per-selection (serial) bookkeeping.
inline int stream_flags(const MissSpec& spec, const std::vector<uint32_t>& all, int max_blocks,
                        int device, std::vector<uint8_t>* miss) {
  const int R = spec.num_requests, L = spec.num_layers, S = spec.steps, G = spec.sel_blocks;
  Exec ex(spec, device, FERRY_LRU_SERIAL, spec.hot_blocks, max_blocks);
  if (ex.status) return ex.status;
  std::vector<uint32_t> step((size_t)R * L * G);
  std::vector<uint8_t> flags(step.size());
  miss->assign(all.size(), 0);
  for (int s = 0; s < S; ++s) {
    for (int r = 0; r < R; ++r)
      std::copy_n(all.data() + ((size_t)r * S + s) * L * G, (size_t)L * G, step.data() + (size_t)r * L * G);
    if (hipMemcpy(ex.sel, step.data(), step.size() * 4, hipMemcpyHostToDevice)) return FERRY_EHIP;
    if (int rc = ferry_fetch_step(ex.ctx, ex.sel, ex.slots, ex.mc, ex.misses, ex.flags, nullptr)) return rc;
    if (hipMemcpy(flags.data(), ex.flags, flags.size(), hipMemcpyDeviceToHost)) return FERRY_EHIP;
    for (int r = 0; r < R; ++r)
      std::copy_n(flags.data() + (size_t)r * L * G, (size_t)L * G, miss->data() + ((size_t)r * S + s) * L * G);
  }
  ferry_stats st{};
  ferry_stats_get(ex.ctx, &st);
  return st.device_error;
}

}  // namespace detail

// Reads an FMT1 trace into (r, s, l, k) events with dense block ids and the
// per-(request, layer) LRU hit/miss of each (miss_trace.cuh:75-185), the
// flags computed by the GPU bookkeeping kernel in per-selection mode.  Sets
// spec.slab_blocks.  A trace that disagrees with the spec or is malformed
// returns status FERRY_EINVAL (ferry_last_error() says why) instead of
// exiting.
inline MissTrace load_miss_trace(const std::string& path, MissSpec& spec, MissTraceInfo* info = nullptr,
                                 int device = 0) {
  MissTrace tr;
  ferry_trace_info ti{};
  std::vector<uint32_t> ids;
  if ((tr.status = detail::read_trace(path, spec, &ti, &ids))) return tr;
  std::vector<uint8_t> miss;
  if ((tr.status = detail::stream_flags(spec, ids, (int)std::max<uint64_t>(ti.unique_blocks, 1), device, &miss)))
    return tr;
  const int R = spec.num_requests, L = spec.num_layers, S = spec.steps, G = spec.sel_blocks;
  tr.events.reserve(ids.size());
  size_t i = 0;
  for (int r = 0; r < R; ++r)
    for (int s = 0; s < S; ++s)
      for (int l = 0; l < L; ++l)
        for (int k = 0; k < G; ++k, ++i) {
          tr.events.push_back({r, l, s, (uint64_t)ids[i], miss[i] != 0});
          ++tr.total_selects;
          if (miss[i]) {
            ++tr.total_misses;
            tr.miss_bytes += spec.c4_bytes();
          }
        }
  tr.hit_rate = tr.total_selects ? 1.0 - (double)tr.total_misses / (double)tr.total_selects : 0.0;
  spec.slab_blocks = (int)ti.max_blocks_per_req;
  if (info) {
    info->path = path;
    info->requests = (int)ti.requests;
    info->steps = (int)ti.steps;
    info->layers = (int)ti.layers;
    info->page_tokens = (int)ti.page_tokens;
    info->block_tokens = (int)ti.block_tokens;
    info->sel_pages = (int)ti.sel_pages;
    info->kv_heads = (int)ti.kv_heads;
    info->head_dim = (int)ti.head_dim;
    info->unique_blocks = ti.unique_blocks;
    info->max_blocks_per_req = ti.max_blocks_per_req;
  }
  return tr;
}

// ---------------------------------------------------------------- per-GPU closed loop
// Names of src/runtime/wla_multigpu.cuh:129, 177-233, 244-318.  On one GPU
// there is nothing to steal from or migrate to, so the policy and kv mode are
// accepted and have no effect, and the migration counters stay 0.
enum class WlaKvMode { Full = 0, Delta = 1, Drop = 2, DeltaNaive = 3 };

struct WlaStealPolicy {
  bool cost_filter = false;
  double b_ref_gbs = 16.6;
  double cost_scale = 3.0;
  double margin = 2.0;
  double steal_delay_ms = 0.0;
  bool steal_thread = false;
  bool speed_aware = false;
};

struct WlaMultiStats {
  double makespan_ms = 0.0;
  double p50_step_ms = 0.0, p99_step_ms = 0.0;  // tick durations
  double throughput_steps = 0.0;                // completed requests / s
  size_t migrated_bytes = 0;
  uint64_t steals = 0;
  uint64_t migrated_reqs = 0;
  uint64_t refill_events = 0;  // the reference's transfer count of the mode
  size_t refill_bytes = 0;     // ... and its bytes
  double imbalance = 0.0;
  double hit_rate = 0.0;
  int n_gpus = 0;
  uint64_t ticks = 0;
  uint64_t fetched_blocks = 0;  // blocks the GPU fetch moved into the pool
  int status = FERRY_OK;
};

// Applies the C2 prefix transform (wla_multigpu.cuh:355-369): members of a
// prefix group repeat their group head's selections for the first
// prefix_steps steps.  ids are (r, s, l, k).
inline void wla_apply_prefix_sharing(std::vector<uint32_t>& ids, const MissSpec& sp) {
  if (sp.prefix_group <= 1 || sp.prefix_steps <= 0) return;
  const size_t per_rs = (size_t)sp.num_layers * sp.sel_blocks;
  for (int r = 0; r < sp.num_requests; ++r) {
    const int head = (r / sp.prefix_group) * sp.prefix_group;
    if (r == head) continue;
    for (int s = 0; s < std::min(sp.prefix_steps, sp.steps); ++s)
      std::copy_n(ids.data() + ((size_t)head * sp.steps + s) * per_rs, per_rs,
                  ids.data() + ((size_t)r * sp.steps + s) * per_rs);
  }
}

// The per-GPU executor of run_wla_multigpu (wla_multigpu.cuh:2291-2705) on
// one device: requests arrive (`arrival` "bursty" or steady, every gap_ms,
// :497-501), are resident in their own lane until they have run
// wla_len_of(sp, r) steps (tick_end, :834-864), and every tick runs one step
// of every resident request as ONE batched decode step (for prefix groups,
// one per member index, so the group's LRU is touched in request order as by
// kv_touch, :1937-1962): bookkeeping, the miss fetch and attention.  Modes: 0 (A) keeps nothing between ticks (every selected block
// is fetched); 1 (B), 2 (C) and the steal/dispatch variants 3-7 use the LRU
// (with one GPU they differ only in cross-GPU policy).  The selections are
// replay_miss_stream's (+ the prefix transform), or the trace named by
// FERRY_MISS_TRACE.  The clock is the wall clock from the start, as in the
// reference; FERRY_VIRTUAL_TICK_MS=x makes tick t start at t*x ms, which
// fixes the tick composition (tests).  Requests join their prefix group when
// admitted and leave it when finished (ferry_members_join / _leave); with
// cap_mode 1 the group's capacity is hot_blocks per resident member and a
// leave trims it (wla_group_cap, grp_trim, wla_multigpu.cuh:1923-1936).
inline WlaMultiStats run_wla_multigpu(const std::vector<int>& devices, MissSpec sp, int mode,
                                      const AdaptiveBatchPolicy& pol, const WlaStealPolicy& spol,
                                      const std::string& skew, const std::string& arrival, double gap_ms,
                                      int steal_batch, int attn_iters, WlaKvMode kvmode = WlaKvMode::Full,
                                      double rebal_interval_ms = 50.0, double rebal_thr = 0.25) {
  (void)spol, (void)skew, (void)steal_batch, (void)attn_iters, (void)kvmode;
  (void)rebal_interval_ms, (void)rebal_thr;
  WlaMultiStats st;
  st.n_gpus = (int)devices.size();
  if (devices.size() != 1 || mode < 0 || mode > 7 || sp.cap_mode < 0 || sp.cap_mode > 1 ||
      !(gap_ms > 0.0)) {
    st.status = FERRY_EINVAL;
    return st;
  }
  const int dev = devices[0];
  const int R = sp.num_requests, L = sp.num_layers, S = sp.steps, G = sp.sel_blocks;
  const int group = std::max(sp.prefix_group, 1);
  std::vector<uint32_t> ids;
  int max_blocks = 64 + 8 * S;  // replay_miss_stream draws ids below 64 + 8 s
  std::string path;
  if (ferry_miss_trace_path(&path)) {
    ferry_trace_info ti{};
    if ((st.status = detail::read_trace(path, sp, &ti, &ids))) return st;
    max_blocks = (int)std::max<uint64_t>(ti.unique_blocks, 1);
  } else {
    ids.resize((size_t)R * S * L * G);
    if ((st.status = ferry_refgen_selections(R, L, S, G, sp.seed, ids.data()))) return st;
    wla_apply_prefix_sharing(ids, sp);
  }
  std::vector<double> arrive(R);
  if ((st.status = ferry_arrivals(arrival == "bursty" ? FERRY_ARRIVAL_BURSTY : FERRY_ARRIVAL_STEADY,
                                  (uint32_t)R, gap_ms, 0.0, 0.0, 0, arrive.data())))
    return st;
  std::vector<int32_t> len(R);
  for (int r = 0; r < R; ++r) len[r] = std::min(std::max(wla_len_of(sp, r), 1), S);
  ferry_sched* sched = nullptr;
  if ((st.status = ferry_sched_create(R, FERRY_SCHED_PINNED, (uint32_t)R, arrive.data(), len.data(), &sched)))
    return st;
  // per-request capacity (cap_mode 1, wla_group_cap): the group's sets have a
  // share of hot_blocks per member, and members arrive and leave
  const bool per_member = sp.cap_mode == 1 && mode != 0;
  const int hot = mode == 0 ? G * group : sp.hot_blocks * (per_member ? group : 1);
  detail::Exec ex(sp, dev, FERRY_LRU_SERIAL, hot, max_blocks, group,
                  per_member ? FERRY_CAP_PER_MEMBER : FERRY_CAP_GROUP);
  if ((st.status = ex.status)) {
    ferry_sched_destroy(sched);
    return st;
  }
  uint32_t *owners = nullptr, *lanes = nullptr;
  if (hipMalloc(&owners, (size_t)R * 4) || hipMalloc(&lanes, (size_t)R * 4)) {
    ferry_sched_destroy(sched);
    (void)hipFree(owners);
    st.status = FERRY_ENOMEM;
    return st;
  }
  // Members join at dispatch and leave at tick_end (grp_member_add,
  // wla_multigpu.cuh:801, 846-862): every lane starts out of its group.
  auto members = [&](const int32_t* ids, int n, bool join) -> int {
    if (n == 0) return FERRY_OK;
    if (hipMemcpy(lanes, ids, (size_t)n * 4, hipMemcpyHostToDevice)) return FERRY_EHIP;
    return join ? ferry_members_join(ex.ctx, lanes, (uint32_t)n, nullptr)
                : ferry_members_leave(ex.ctx, lanes, (uint32_t)n, nullptr);
  };
  {
    std::vector<int32_t> all(R);
    for (int r = 0; r < R; ++r) all[r] = r;
    if ((st.status = members(all.data(), R, false))) {
      ferry_sched_destroy(sched);
      (void)hipFree(owners);
      (void)hipFree(lanes);
      return st;
    }
  }
  double vtick = 0.0;
  if (const char* e = std::getenv("FERRY_VIRTUAL_TICK_MS")) vtick = std::atof(e);
  std::vector<int32_t> lane_req(R), lane_step(R), admitted(R), retired(R);
  std::vector<uint32_t> step_ids((size_t)R * L * G);
  std::vector<uint32_t> own;
  std::vector<double> tick_ms;
  std::vector<uint32_t> mc(ex.n_sets);
  std::vector<ferry_miss> ms((size_t)ex.n_sets * ex.max_sel);
  std::vector<std::pair<int, uint64_t>> ml;
  uint64_t a_events = 0, c_events = 0, c_bytes = 0;
  const HostTimer ht;
  auto elapsed = [&]() { return ht.toc_ms(); };
  for (uint64_t t = 0;; ++t) {
    const double now = vtick > 0.0 ? (double)t * vtick : elapsed();
    int32_t na = 0, nr = 0, nres = 0, done = 0;
    if ((st.status = ferry_sched_tick(sched, now, lane_req.data(), lane_step.data(), admitted.data(), &na,
                                      retired.data(), &nr, &nres, &done)))
      break;
    // finished requests leave their groups (trimmed under cap_mode 1), then
    // the arrived ones join
    if ((st.status = members(retired.data(), nr, false))) break;
    if ((st.status = members(admitted.data(), na, true))) break;
    if (done) break;
    if (nres == 0) {  // nothing resident: wait for the next arrival (wait_arrival, :1535-1540)
      if (vtick <= 0.0) {
        double next = 0.0;
        ferry_sched_next_arrival(sched, &next);
        const double wait = std::min(std::max(next - elapsed(), 0.0), 0.5);
        std::this_thread::sleep_for(std::chrono::duration<double, std::milli>(wait));
      }
      continue;
    }
    const double ts = elapsed();
    // mode A: nothing is kept from the previous tick
    own.clear();
    for (int r = 0; r < R; ++r)
      if (mode == 0 && lane_req[r] >= 0 && (own.empty() || own.back() != (uint32_t)(r / group)))
        own.push_back((uint32_t)(r / group));
    if (!own.empty()) {
      if (hipMemcpy(owners, own.data(), own.size() * 4, hipMemcpyHostToDevice)) {
        st.status = FERRY_EHIP;
        break;
      }
      if ((st.status = ferry_sets_reset_owners(ex.ctx, owners, (uint32_t)own.size(), nullptr))) break;
    }
    // The reference refills and attends one resident request after the other
    // (:2643-2648), so members of a prefix group touch the group's LRU in
    // request order and may evict what an earlier member already used.  Sub-
    // tick j runs member j of every group: bookkeeping, fetch and attention.
    for (int j = 0; j < group && !st.status; ++j) {
      bool any = false;
      for (int r = 0; r < R; ++r) {
        uint32_t* row = step_ids.data() + (size_t)r * L * G;
        const int q = lane_req[r];
        if (q < 0 || r % group != j) {
          std::fill(row, row + (size_t)L * G, FERRY_EMPTY);
          continue;
        }
        std::copy_n(ids.data() + ((size_t)q * S + lane_step[r]) * L * G, (size_t)L * G, row);
        any = true;
      }
      if (!any) continue;
      if (hipMemcpy(ex.sel, step_ids.data(), step_ids.size() * 4, hipMemcpyHostToDevice)) {
        st.status = FERRY_EHIP;
        break;
      }
      if ((st.status = ferry_fetch_step(ex.ctx, ex.sel, ex.slots, ex.mc, ex.misses, nullptr, nullptr))) break;
      if ((st.status = ferry_sparse_decode(ex.ctx, ex.q, ex.slots, ex.out, nullptr))) break;
      // the reference's refill count of this sub-tick's requests
      bool first = true;
      for (int r = 0; r < R && !st.status; ++r) {
        if (lane_req[r] < 0 || r % group != j) continue;
        if (mode == 0) {
          a_events += (uint64_t)L * G;
        } else if (mode >= 2) {
          st.status = detail::owner_misses(ex, r / group, L, mc, ms, first, &ml);
          first = false;
          c_events += detail::cmode_submits(ml, sp.c4_bytes(), pol, &c_bytes);
        }
      }
    }
    if (st.status) break;
    if (hipDeviceSynchronize()) {
      st.status = FERRY_EHIP;
      break;
    }
    tick_ms.push_back(elapsed() - ts);
    ++st.ticks;
  }
  st.makespan_ms = elapsed();
  (void)hipFree(owners);
  (void)hipFree(lanes);
  ferry_sched_destroy(sched);
  ferry_stats fs{};
  ferry_stats_get(ex.ctx, &fs);
  if (!st.status && fs.device_error) st.status = fs.device_error;
  st.fetched_blocks = fs.misses;
  if (mode == 0) {  // every selected block of every resident request, hits included (:2489-2504)
    st.refill_events = a_events;
    st.refill_bytes = (size_t)a_events * sp.c4_bytes();
  } else if (mode == 1) {  // one submit per miss (:2505-2526)
    st.refill_events = fs.misses;
    st.refill_bytes = (size_t)fs.misses * sp.c4_bytes();
  } else {  // coalesced, policy-batched submits per request-step (:2527-2604)
    st.refill_events = c_events;
    st.refill_bytes = (size_t)c_bytes;
  }
  st.hit_rate = fs.selections ? 1.0 - (double)fs.misses / (double)fs.selections : 0.0;
  st.throughput_steps = st.makespan_ms > 0 ? (double)R / (st.makespan_ms / 1000.0) : 0.0;
  std::sort(tick_ms.begin(), tick_ms.end());
  if (!tick_ms.empty()) {
    st.p50_step_ms = tick_ms[tick_ms.size() / 2];
    st.p99_step_ms = tick_ms[(size_t)(0.99 * (tick_ms.size() - 1))];
  }
  return st;
}

}  // namespace ferry
