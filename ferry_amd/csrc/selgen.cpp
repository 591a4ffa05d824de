// selgen.cpp -- synthetic selection streams (host side of the workload).
//
// ferry_selgen_*: the executor's workloads.  For every (request r, layer l,
// kv head h) a step keeps each block of r's previous selection with
// probability `reuse` (inter-step locality, the knob of the reference's
// generator, src/workloads/missstream.cuh:127-128), then completes the
// selection to k distinct blocks with popularity-rank draws (Zipf(s) or
// uniform) mapped through an owner-shared affine permutation and rejected when
// outside r's context or already taken.  The k blocks are sorted (top-k page
// indices are sorted, tools/capture_miss_trace.py:158-159) and group members'
// private blocks are renamed into the set's id space after the shared prefix.
// Every draw is a counter-based hash of (seed, step, r, l, h, draw index), so
// requests are generated independently in parallel.
//
// Lanes and requests: row r of a step is batch lane r.  By default lane r
// holds request r from step 0.  ferry_selgen_admit puts a new request (id,
// context) into a lane from a given step on; its draws are then keyed by
// (request id, steps since admission) and it starts without carry-over, as a
// fresh decode does.  A retired lane produces rows of FERRY_EMPTY.  A context
// shorter than k blocks selects all of them and pads the row with FERRY_EMPTY.
// In a prefix group a new member keeps the owner's permutation and shared
// prefix ids, and ferry_selgen_admit_member gives its private blocks their
// own id range, so a lane's successive requests never share private ids.
//
// ferry_refgen_selections: the selection half of replay_miss_stream
// (src/workloads/missstream.cuh:104-133) with std::mt19937_64.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/ferry_amd.h"

namespace {

uint64_t mix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + idx * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr uint64_t kSaltCtx = 0x43545842ull;
constexpr uint64_t kSaltSel = 0x53454C31ull;
constexpr uint64_t kSaltPerm = 0x5045524Dull;
constexpr uint64_t kSaltKeep = 0x4B454550ull;
constexpr uint64_t kPermPrime = 1000003ull;
constexpr int kDrawLimit = 65536;

}  // namespace

struct ferry_selgen {
  ferry_selgen_config cfg;
  std::vector<int32_t> ctx;
  std::vector<int32_t> nperm;  // per owner: largest member context
  std::vector<double> cum;     // Zipf cumulative weights of ranks 0..nmax-1
  std::vector<uint32_t> state; // previous logical selection per (r, l, h)
  std::vector<double> reuse;   // per-request reuse (empty = cfg.reuse for all)
  std::vector<int32_t> rid;    // request id held by each lane
  std::vector<int32_t> start;  // step at which that request was admitted
  std::vector<uint8_t> active; // lane holds a request
  std::vector<int32_t> prange; // private id range of the lane's request (prefix groups)
  int ranges = 0;              // private id ranges per owner (>= group)
  int nmax = 0;
  int max_blocks = 0;
};

namespace {
// Largest block id + 1 over owners: shared prefix, then `ranges` private
// ranges of (np - prefix) ids each.
int selgen_max_blocks(const ferry_selgen* g) {
  int mx = 0;
  for (size_t o = 0; o < g->nperm.size(); ++o) {
    const int np = g->nperm[o];
    const int pre = std::min(g->cfg.prefix_blocks, np);
    mx = std::max(mx, pre + g->ranges * (np - pre));
  }
  return mx;
}
}  // namespace

extern "C" {

int ferry_ctx_uniform(uint64_t seed, int32_t n_req, int32_t lo, int32_t hi, int32_t* out) {
  if (n_req < 0 || hi < lo || !out) return FERRY_EINVAL;
  const uint64_t span = (uint64_t)(hi - lo + 1);
  for (int r = 0; r < n_req; ++r) out[r] = lo + (int32_t)(mix64(seed ^ kSaltCtx, (uint64_t)r) % span);
  return FERRY_OK;
}

int ferry_selgen_create(const ferry_selgen_config* cfg, const int32_t* ctx_blocks, ferry_selgen** out) {
  if (!cfg || !ctx_blocks || !out) return FERRY_EINVAL;
  if (cfg->n_req < 1 || cfg->n_req > 65536 || cfg->group < 1 || cfg->n_layers < 1 || cfg->kv_heads < 1 || cfg->k < 1 ||
      cfg->reuse < 0.0 || cfg->reuse > 1.0 || cfg->prefix_blocks < 0)
    return FERRY_EINVAL;
  ferry_selgen* g = new ferry_selgen();
  g->cfg = *cfg;
  g->ctx.assign(ctx_blocks, ctx_blocks + cfg->n_req);
  for (int r = 0; r < cfg->n_req; ++r) {
    if (g->ctx[r] < 1 || g->ctx[r] >= (int)kPermPrime) {
      delete g;
      return FERRY_EINVAL;
    }
    g->nmax = std::max(g->nmax, g->ctx[r]);
  }
  const int nown = (cfg->n_req + cfg->group - 1) / cfg->group;
  g->nperm.assign(nown, 0);
  for (int r = 0; r < cfg->n_req; ++r) g->nperm[r / cfg->group] = std::max(g->nperm[r / cfg->group], g->ctx[r]);
  (void)nown;
  g->ranges = cfg->group;
  g->max_blocks = selgen_max_blocks(g);
  if (cfg->dist == 1) {
    g->cum.resize(g->nmax);
    double acc = 0.0;
    for (int i = 0; i < g->nmax; ++i) {
      acc += std::pow((double)(i + 1), -cfg->zipf_s);
      g->cum[i] = acc;
    }
  }
  g->state.assign((size_t)cfg->n_req * cfg->n_layers * cfg->kv_heads * cfg->k, 0u);
  g->rid.resize(cfg->n_req);
  for (int r = 0; r < cfg->n_req; ++r) g->rid[r] = r;
  g->start.assign(cfg->n_req, 0);
  g->active.assign(cfg->n_req, 1);
  g->prange.resize(cfg->n_req);
  for (int r = 0; r < cfg->n_req; ++r) g->prange[r] = r % cfg->group;
  *out = g;
  return FERRY_OK;
}

int ferry_selgen_admit(ferry_selgen* g, int32_t lane, int32_t request_id, int32_t ctx_blocks,
                       int32_t step) {
  if (!g || lane < 0 || lane >= g->cfg.n_req) return FERRY_EINVAL;
  if (g->cfg.group != 1) return FERRY_EINVAL;  // a group's lanes share one permutation
  if (request_id < 0 || request_id >= 65536 || step < 0) return FERRY_EINVAL;
  if (ctx_blocks < 1 || ctx_blocks > g->nmax) return FERRY_EINVAL;
  g->rid[lane] = request_id;
  g->ctx[lane] = ctx_blocks;
  g->nperm[lane] = ctx_blocks;
  g->start[lane] = step;
  g->active[lane] = 1;
  return FERRY_OK;
}

int ferry_selgen_set_private_ranges(ferry_selgen* g, int32_t ranges) {
  if (!g || ranges < g->cfg.group || ranges > 65536) return FERRY_EINVAL;
  g->ranges = ranges;
  g->max_blocks = selgen_max_blocks(g);
  return FERRY_OK;
}

int ferry_selgen_admit_member(ferry_selgen* g, int32_t lane, int32_t request_id, int32_t ctx_blocks,
                              int32_t step, int32_t private_range) {
  if (!g || lane < 0 || lane >= g->cfg.n_req) return FERRY_EINVAL;
  if (g->cfg.group == 1)
    return private_range == 0 ? ferry_selgen_admit(g, lane, request_id, ctx_blocks, step) : FERRY_EINVAL;
  const int o = lane / g->cfg.group;
  if (request_id < 0 || request_id >= 65536 || step < 0) return FERRY_EINVAL;
  if (ctx_blocks < 1 || ctx_blocks > g->nperm[o]) return FERRY_EINVAL;
  if (private_range < 0 || private_range >= g->ranges) return FERRY_EINVAL;
  g->rid[lane] = request_id;
  g->ctx[lane] = ctx_blocks;
  g->start[lane] = step;
  g->active[lane] = 1;
  g->prange[lane] = private_range;
  return FERRY_OK;
}

int ferry_selgen_retire(ferry_selgen* g, int32_t lane) {
  if (!g || lane < 0 || lane >= g->cfg.n_req) return FERRY_EINVAL;
  g->active[lane] = 0;
  return FERRY_OK;
}

int ferry_selgen_set_reuse(ferry_selgen* g, const double* reuse) {
  if (!g) return FERRY_EINVAL;
  if (!reuse) {
    g->reuse.clear();
    return FERRY_OK;
  }
  for (int r = 0; r < g->cfg.n_req; ++r)
    if (!(reuse[r] >= 0.0 && reuse[r] <= 1.0)) return FERRY_EINVAL;
  g->reuse.assign(reuse, reuse + g->cfg.n_req);
  return FERRY_OK;
}

int ferry_selgen_destroy(ferry_selgen* g) {
  delete g;
  return FERRY_OK;
}

int ferry_selgen_max_blocks(const ferry_selgen* g, int32_t* out) {
  if (!g || !out) return FERRY_EINVAL;
  *out = g->max_blocks;
  return FERRY_OK;
}

int ferry_selgen_step(ferry_selgen* g, int32_t step, uint32_t* out) {
  if (!g || !out || step < 0) return FERRY_EINVAL;
  const ferry_selgen_config& c = g->cfg;
  const int L = c.n_layers, H = c.kv_heads, k = c.k;
  for (int r = 0; r < c.n_req; ++r)
    if (g->active[r] && step < g->start[r]) return FERRY_EINVAL;
  int nthreads = (int)std::min<unsigned>(16u, std::max(1u, std::thread::hardware_concurrency()));
  nthreads = std::min(nthreads, c.n_req);
  std::vector<int> rc(nthreads, 0);
  auto work = [&](int tid) {
    std::vector<uint8_t> taken(g->nmax, 0);
    for (int r = tid; r < c.n_req; r += nthreads) {
      if (!g->active[r]) {
        std::fill(out + (size_t)r * L * H * k, out + (size_t)(r + 1) * L * H * k, FERRY_EMPTY);
        continue;
      }
      const int o = r / c.group, m = g->prange[r];  // m: the lane's private id range
      const int nr = g->ctx[r];
      const int np = g->nperm[o];
      const int pre = std::min(c.prefix_blocks, np);
      const double reuse = g->reuse.empty() ? c.reuse : g->reuse[r];
      const uint64_t keep_thr = (uint64_t)(reuse * 4294967296.0);
      const uint64_t rid = (uint64_t)g->rid[r];
      const uint64_t lstep = (uint64_t)(step - g->start[r]);  // steps since admission
      const bool carry = lstep > 0;
      const int ke = std::min(k, nr);  // a short context selects all its blocks
      // permutation of the owner; a lane taken over by request `rid` gets rid's
      const uint64_t pown = c.group == 1 ? rid : (uint64_t)o;
      for (int l = 0; l < L; ++l)
        for (int h = 0; h < H; ++h) {
          const size_t row = ((size_t)(r * L + l) * H + h) * k;
          uint32_t* st = g->state.data() + row;
          uint32_t* so = out + row;
          const uint64_t off = mix64(c.seed ^ kSaltPerm, (pown * L + l) * H + h) % (uint64_t)np;
          // draw index of (steps since admission, request, l, h): independent
          // of the batch size and of the lane
          const uint64_t base =
              ((((lstep << 16) | rid) * (uint64_t)L + (uint64_t)l) * (uint64_t)H + (uint64_t)h) *
              (uint64_t)kDrawLimit;
          int got = 0;
          if (carry && reuse > 0.0)
            for (int j = 0; j < k; ++j)
              if (st[j] != FERRY_EMPTY &&
                  (mix64(c.seed ^ kSaltKeep, base + (uint64_t)j) >> 32) < keep_thr) {
                so[got++] = st[j];
                taken[st[j]] = 1;
              }
          for (int i = 0; i < kDrawLimit && got < ke; ++i) {
            const uint64_t u = mix64(c.seed ^ kSaltSel, base + (uint64_t)i);
            uint64_t rank;
            if (c.dist == 1) {
              const double thr = (double)(u >> 11) * (1.0 / 9007199254740992.0) * g->cum[np - 1];
              rank = (uint64_t)(std::upper_bound(g->cum.begin(), g->cum.begin() + np, thr) - g->cum.begin());
            } else {
              rank = ((u >> 32) * (uint64_t)np) >> 32;
            }
            const uint64_t b = (rank * kPermPrime + off) % (uint64_t)np;
            if (b >= (uint64_t)nr || taken[b]) continue;
            taken[b] = 1;
            so[got++] = (uint32_t)b;
          }
          for (int j = 0; j < got; ++j) taken[so[j]] = 0;
          if (got < ke) {
            rc[tid] = FERRY_ESTATE;
            return;
          }
          std::sort(so, so + ke);
          std::fill(so + ke, so + k, FERRY_EMPTY);
          std::memcpy(st, so, (size_t)k * 4);
          for (int j = 0; j < ke; ++j)
            if (so[j] >= (uint32_t)pre)
              so[j] = (uint32_t)pre + (uint32_t)m * (uint32_t)(np - pre) + (so[j] - (uint32_t)pre);
        }
    }
  };
  std::vector<std::thread> th;
  for (int t = 1; t < nthreads; ++t) th.emplace_back(work, t);
  work(0);
  for (auto& t : th) t.join();
  for (int v : rc)
    if (v) return v;
  return FERRY_OK;
}

int ferry_refgen_selections(int32_t R, int32_t L, int32_t S, int32_t sel, uint64_t seed, uint32_t* out) {
  if (R < 1 || L < 1 || S < 1 || sel < 1 || !out) return FERRY_EINVAL;
  std::mt19937_64 rng(seed);
  std::vector<std::vector<uint32_t>> prev((size_t)R * L);
  size_t ev = 0;
  for (int r = 0; r < R; ++r)
    for (int s = 0; s < S; ++s) {
      const uint64_t hist = 64 + (uint64_t)s * 8;
      for (int l = 0; l < L; ++l) {
        auto& pv = prev[(size_t)r * L + l];
        std::vector<uint32_t> cur(sel);
        for (int i = 0; i < sel; ++i) {
          uint64_t blk;
          if (!pv.empty() && (double)(rng() % 1000) / 1000.0 < 0.66)
            blk = pv[rng() % pv.size()];
          else
            blk = rng() % hist;
          cur[i] = (uint32_t)blk;
          out[ev++] = (uint32_t)blk;
        }
        pv.swap(cur);
      }
    }
  return FERRY_OK;
}

}  // extern "C"
