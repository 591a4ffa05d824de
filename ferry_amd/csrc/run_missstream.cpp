// run_missstream -- the reference's single-GPU Workload-A driver
// (src/benches/run_missstream.cu:33-112) over include/ferry/ferry.hpp.
// Same flags (--hot 1|2|4, --steps, --requests, --layers, --sel, --arrival,
// --all; --attn is accepted and ignored) and the same output rows, each with
// a status field and the blocks the GPU fetched appended.  Unknown flags are
// an error (exit 2) instead of being ignored.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/ferry/ferry.hpp"

namespace {

void print_wla(const char* name, const ferry::WlAStats& st, float gpu_ms) {
  std::printf("  %-10s makespan=%9.2fms steps/s=%8.1f p50=%7.3f p99=%8.3f refill=%8llu bytes=%9.2fMB status=%d "
              "fetched=%llu gpu=%.2fms\n",
              name, st.makespan_ms, st.throughput_steps, st.p50_step_ms, st.p99_step_ms,
              (unsigned long long)st.refill_events, st.refill_bytes / 1048576.0, st.status,
              (unsigned long long)st.fetched_blocks, gpu_ms);
  std::fflush(stdout);
}

// One mode's run, its interval also taken on the GPU's clock (events on the
// default stream around it).
ferry::WlAStats run_mode(const char* name, const ferry::MissSpec& sp, const ferry::MissTrace& tr, int mode,
                         const ferry::AdaptiveBatchPolicy& pol) {
  ferry::HipTimer gt;
  gt.tick();
  const ferry::WlAStats st = ferry::run_miss_workload(0, 0, sp, tr, mode, pol);
  gt.toc();
  FERRY_HIP_CHECK(hipEventSynchronize(gt.end));
  print_wla(name, st, gt.elapsed_ms());
  return st;
}

int run_scenario(const ferry::MissSpec& sp, const ferry::AdaptiveBatchPolicy& pol) {
  std::printf("[wlA] reqs=%d layers=%d steps=%d sel=%d hot=%d c4=%zuB arrival=%s\n", sp.num_requests,
              sp.num_layers, sp.steps, sp.sel_blocks, sp.hot_blocks, sp.c4_bytes(), sp.arrival.c_str());
  ferry::MissTrace tr = ferry::replay_miss_stream(sp);
  if (tr.status) {
    std::printf("  trace failed: %d %s\n", tr.status, ferry_last_error());
    return 1;
  }
  // miss bytes per selected token: a selection is one 4-token c4 block
  const double b_per_token =
      tr.total_selects ? (double)tr.miss_bytes / ((double)tr.total_selects * 4.0) : 0.0;
  std::printf("  trace: selects=%llu miss=%llu hit_rate=%.3f miss_bytes=%.2fMB miss_B/token=%.1f\n",
              (unsigned long long)tr.total_selects, (unsigned long long)tr.total_misses, tr.hit_rate,
              tr.miss_bytes / 1048576.0, b_per_token);
  std::fflush(stdout);
  const ferry::WlAStats a = run_mode("baseline-A", sp, tr, 0, pol);
  const ferry::WlAStats b = run_mode("baseline-B", sp, tr, 1, pol);
  const ferry::WlAStats c = run_mode("ferry-C", sp, tr, 2, pol);
  if (a.status || b.status || c.status) return 1;
  const double refill_ratio = b.refill_events ? (double)c.refill_events / (double)b.refill_events : 1.0;
  std::printf("  => C/A %.2fx  C/B %.2fx  refill C/B %.3f\n\n", a.makespan_ms / c.makespan_ms,
              b.makespan_ms / c.makespan_ms, refill_ratio);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  ferry::MissSpec sp;
  int hot_mult = 4, steps = 48;
  bool run_all = false;
  for (int i = 1; i < argc; ++i) {
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "missing value for %s\n", argv[i]);
        std::exit(2);
      }
      return argv[++i];
    };
    if (!std::strcmp(argv[i], "--hot")) hot_mult = std::atoi(next());
    else if (!std::strcmp(argv[i], "--steps")) steps = std::atoi(next());
    else if (!std::strcmp(argv[i], "--requests")) sp.num_requests = std::atoi(next());
    else if (!std::strcmp(argv[i], "--layers")) sp.num_layers = std::atoi(next());
    else if (!std::strcmp(argv[i], "--sel")) sp.sel_blocks = std::atoi(next());
    else if (!std::strcmp(argv[i], "--attn")) (void)next();
    else if (!std::strcmp(argv[i], "--arrival")) sp.arrival = next();
    else if (!std::strcmp(argv[i], "--all")) run_all = true;
    else {
      std::fprintf(stderr, "unknown flag %s\n", argv[i]);
      return 2;
    }
  }
  sp.steps = steps;
  sp.hot_blocks = sp.sel_blocks * (hot_mult == 1 ? 2 : (hot_mult == 2 ? 4 : 8));
  ferry::AdaptiveBatchPolicy pol;
  pol.target_batches = 8.0;
  int rc = 0;
  if (run_all) {
    for (const char* arr : {"steady", "bursty", "mixed"}) {
      ferry::MissSpec s = sp;
      s.arrival = arr;
      rc |= run_scenario(s, pol);
    }
  } else {
    rc = run_scenario(sp, pol);
  }
  return rc;
}
