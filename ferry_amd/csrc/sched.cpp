// sched.cpp -- request arrivals and the tick scheduler of one GPU's executor.
//
// The reference's per-GPU exec thread loops over ticks: tick_begin takes the
// resident requests, exec_step runs one decode step of each, tick_end
// advances their step counters and retires those that reached their length
// (src/runtime/wla_multigpu.cuh:829-864, 2610-2665).  Requests become resident
// at their arrival time, which is steady or bursty in the reference
// (:497-501).  Here residency is bounded by the executor's batch lanes: an
// arrived request waits in a FIFO until a lane is free (any lane, or with
// FERRY_SCHED_PINNED only lane r mod lanes, which keeps a request's lane --
// and so its prefix group's sets -- fixed), and one executor decode step runs
// every resident lane at once.  The scheduler is pure host
// logic; the caller supplies the clock (wall or virtual) and applies the
// admissions (lane reset, generator admission) before launching the step.
#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <vector>

#include "../../include/ferry_amd.h"

namespace {

uint64_t mix64(uint64_t seed, uint64_t idx) {
  uint64_t z = seed + idx * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

constexpr uint64_t kSaltArrive = 0x41525256ull;
constexpr uint64_t kSaltSojourn = 0x534F4A4Eull;

// Uniform in (0, 1]: 53 random bits, never 0 (so log() is finite).
double u01(uint64_t seed, uint64_t salt, uint64_t i) {
  return (double)((mix64(seed ^ salt, i) >> 11) + 1) * (1.0 / 9007199254740992.0);
}

// Exponential of mean `mean` by inversion.
double expo(double mean, uint64_t seed, uint64_t salt, uint64_t i) {
  return -mean * std::log(u01(seed, salt, i));
}

}  // namespace

struct ferry_sched {
  int32_t lanes = 0;
  int32_t policy = FERRY_SCHED_FIFO;
  uint32_t n = 0;
  std::vector<double> arrive;
  std::vector<int32_t> len;
  std::vector<uint32_t> order;  // requests by (arrival, id)
  uint32_t head = 0;            // order[head, next) are waiting
  uint32_t next = 0;            // order[next, n) have not arrived
  std::vector<std::vector<uint32_t>> lane_q;  // FERRY_SCHED_PINNED: waiting per lane
  std::vector<size_t> lane_qh;                 // ... and the head of each
  std::vector<int32_t> lane_req, lane_step;
  std::vector<int32_t> steps_done, admit_tick, done_tick;
  uint32_t completed = 0;
  int32_t tick = 0;
};

extern "C" {

int ferry_arrivals(int kind, uint32_t n, double gap_ms, double period_ms, double ratio,
                   uint64_t seed, double* out_ms) {
  if (!out_ms && n) return FERRY_EINVAL;
  if (!(gap_ms > 0.0) || !std::isfinite(gap_ms)) return FERRY_EINVAL;
  double t = 0.0;
  switch (kind) {
    case FERRY_ARRIVAL_STEADY:
      for (uint32_t r = 0; r < n; ++r) out_ms[r] = t += gap_ms;
      return FERRY_OK;
    case FERRY_ARRIVAL_BURSTY:
      for (uint32_t r = 0; r < n; ++r) out_ms[r] = t += (r % 16 == 0) ? 40.0 * gap_ms : 0.1 * gap_ms;
      return FERRY_OK;
    case FERRY_ARRIVAL_POISSON:
      for (uint32_t r = 0; r < n; ++r) out_ms[r] = t += expo(gap_ms, seed, kSaltArrive, r);
      return FERRY_OK;
    case FERRY_ARRIVAL_MMPP: {
      if (!(period_ms > 0.0) || !(ratio > 0.0)) return FERRY_EINVAL;
      // exact simulation: an exponential gap that crosses the end of the
      // current state is discarded (memoryless) and redrawn at the new rate
      const double mean[2] = {gap_ms, gap_ms / ratio};
      int state = 0;
      uint64_t a = 0, b = 0;
      double end = expo(period_ms, seed, kSaltSojourn, b++);
      for (uint32_t r = 0; r < n; ++r) {
        for (;;) {
          const double gap = expo(mean[state], seed, kSaltArrive, a++);
          if (t + gap < end) {
            t += gap;
            break;
          }
          t = end;
          state ^= 1;
          end = t + expo(period_ms, seed, kSaltSojourn, b++);
        }
        out_ms[r] = t;
      }
      return FERRY_OK;
    }
    default:
      return FERRY_EINVAL;
  }
}

int ferry_sched_create(int32_t lanes, int32_t policy, uint32_t n, const double* arrive_ms,
                       const int32_t* len_steps, ferry_sched** out) {
  if (!out || lanes < 1 || (n && (!arrive_ms || !len_steps))) return FERRY_EINVAL;
  if (policy != FERRY_SCHED_FIFO && policy != FERRY_SCHED_PINNED) return FERRY_EINVAL;
  for (uint32_t r = 0; r < n; ++r)
    if (len_steps[r] < 1 || !std::isfinite(arrive_ms[r])) return FERRY_EINVAL;
  ferry_sched* s = new ferry_sched();
  s->lanes = lanes;
  s->policy = policy;
  s->n = n;
  s->lane_q.assign(lanes, {});
  s->lane_qh.assign(lanes, 0);
  s->arrive.assign(arrive_ms, arrive_ms + n);
  s->len.assign(len_steps, len_steps + n);
  s->order.resize(n);
  std::iota(s->order.begin(), s->order.end(), 0u);
  std::stable_sort(s->order.begin(), s->order.end(),
                   [&](uint32_t a, uint32_t b) { return s->arrive[a] < s->arrive[b]; });
  s->lane_req.assign(lanes, -1);
  s->lane_step.assign(lanes, 0);
  s->steps_done.assign(n, 0);
  s->admit_tick.assign(n, -1);
  s->done_tick.assign(n, -1);
  *out = s;
  return FERRY_OK;
}

int ferry_sched_destroy(ferry_sched* s) {
  delete s;
  return FERRY_OK;
}

int ferry_sched_tick(ferry_sched* s, double now_ms, int32_t* lane_req, int32_t* lane_step,
                     int32_t* admitted, int32_t* n_admitted, int32_t* retired,
                     int32_t* n_retired, int32_t* n_resident, int32_t* done) {
  if (!s || !(now_ms == now_ms)) return FERRY_EINVAL;
  std::vector<int32_t> left;
  // 1. the previous tick ran one step of every resident request
  if (s->tick > 0)
    for (int32_t ln = 0; ln < s->lanes; ++ln) {
      const int32_t r = s->lane_req[ln];
      if (r < 0) continue;
      if (++s->steps_done[r] >= s->len[r]) {
        s->done_tick[r] = s->tick - 1;
        s->lane_req[ln] = -1;
        ++s->completed;
        left.push_back(ln);
      }
    }
  // 2. arrivals join the FIFO (FERRY_SCHED_PINNED: their lane's FIFO); free
  //    lanes take the head, lowest lane first
  while (s->next < s->n && s->arrive[s->order[s->next]] <= now_ms) {
    const uint32_t r = s->order[s->next++];
    if (s->policy == FERRY_SCHED_PINNED) s->lane_q[r % (uint32_t)s->lanes].push_back(r);
  }
  int32_t na = 0;
  for (int32_t ln = 0; ln < s->lanes; ++ln) {
    if (s->lane_req[ln] >= 0) continue;
    uint32_t r;
    if (s->policy == FERRY_SCHED_PINNED) {
      if (s->lane_qh[ln] == s->lane_q[ln].size()) continue;
      r = s->lane_q[ln][s->lane_qh[ln]++];
    } else {
      if (s->head == s->next) break;
      r = s->order[s->head++];
    }
    s->lane_req[ln] = (int32_t)r;
    s->admit_tick[r] = s->tick;
    if (admitted) admitted[na] = ln;
    ++na;
  }
  // a lane that lost its request and got a new one in the same tick is an
  // admission, not a retirement
  int32_t nr = 0;
  for (int32_t ln : left)
    if (s->lane_req[ln] < 0) {
      if (retired) retired[nr] = ln;
      ++nr;
    }
  int32_t res = 0;
  for (int32_t ln = 0; ln < s->lanes; ++ln) {
    const int32_t r = s->lane_req[ln];
    s->lane_step[ln] = r >= 0 ? s->steps_done[r] : 0;
    res += r >= 0;
  }
  if (lane_req) std::copy(s->lane_req.begin(), s->lane_req.end(), lane_req);
  if (lane_step) std::copy(s->lane_step.begin(), s->lane_step.end(), lane_step);
  if (n_admitted) *n_admitted = na;
  if (n_retired) *n_retired = nr;
  if (n_resident) *n_resident = res;
  if (done) *done = s->completed == s->n ? 1 : 0;
  ++s->tick;
  return FERRY_OK;
}

int ferry_sched_next_arrival(const ferry_sched* s, double* ms) {
  if (!s || !ms) return FERRY_EINVAL;
  *ms = s->next < s->n ? s->arrive[s->order[s->next]] : std::numeric_limits<double>::infinity();
  return FERRY_OK;
}

int ferry_sched_request_ticks(const ferry_sched* s, int32_t* admit_tick, int32_t* done_tick) {
  if (!s) return FERRY_EINVAL;
  if (admit_tick) std::copy(s->admit_tick.begin(), s->admit_tick.end(), admit_tick);
  if (done_tick) std::copy(s->done_tick.begin(), s->done_tick.end(), done_tick);
  return FERRY_OK;
}

}  // extern "C"
