// run_wla -- the per-GPU slice of the reference's closed-loop Workload-A
// driver (src/benches/run_wla_multigpu.cu:78-734) over include/ferry/ferry.hpp.
// The reference driver needs two or more GPUs (:280-283) and compares
// cross-GPU policies; on one GPU those collapse onto the C engine, so this
// driver runs modes A, B and C of the same tick loop and prints one row each.
// Flags keep the reference's names: --gpus (one id), --requests, --steps,
// --layers, --sel, --hot, --arrival steady|bursty, --gap, --prefix-group,
// --prefix-steps, --cap-mode group|perreq, --miss-trace (sets
// FERRY_MISS_TRACE), --kv-heads, --head-dim.  Unknown flags are an error
// (exit 2).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/ferry/ferry.hpp"

namespace {

void print_row(const char* name, const ferry::WlaMultiStats& st) {
  std::printf("  %-9s makespan=%9.2fms steps/s=%7.1f p50=%7.3f p99=%8.3f refill=%8llu seg %9.2fMB "
              "hit=%.3f ticks=%llu status=%d fetched=%llu\n",
              name, st.makespan_ms, st.throughput_steps, st.p50_step_ms, st.p99_step_ms,
              (unsigned long long)st.refill_events, st.refill_bytes / 1048576.0, st.hit_rate,
              (unsigned long long)st.ticks, st.status, (unsigned long long)st.fetched_blocks);
  std::fflush(stdout);
}

}  // namespace

int main(int argc, char** argv) {
  ferry::MissSpec sp;
  sp.num_requests = 48;
  sp.steps = 16;
  sp.num_layers = 12;
  sp.sel_blocks = 64;
  sp.hot_blocks = 128;
  std::string arrival = "steady", trace;
  double gap_ms = 1.0;
  int device = 0;
  for (int i = 1; i < argc; ++i) {
    auto next = [&]() -> const char* {
      if (i + 1 >= argc) {
        std::fprintf(stderr, "missing value for %s\n", argv[i]);
        std::exit(2);
      }
      return argv[++i];
    };
    if (!std::strcmp(argv[i], "--gpus")) {
      const char* v = next();
      if (std::strchr(v, ',')) {
        std::fprintf(stderr, "run_wla drives one GPU; got --gpus %s\n", v);
        return 2;
      }
      device = std::atoi(v);
    } else if (!std::strcmp(argv[i], "--requests")) sp.num_requests = std::atoi(next());
    else if (!std::strcmp(argv[i], "--steps")) sp.steps = std::atoi(next());
    else if (!std::strcmp(argv[i], "--layers")) sp.num_layers = std::atoi(next());
    else if (!std::strcmp(argv[i], "--sel")) sp.sel_blocks = std::atoi(next());
    else if (!std::strcmp(argv[i], "--hot")) sp.hot_blocks = std::atoi(next());
    else if (!std::strcmp(argv[i], "--arrival")) arrival = next();
    else if (!std::strcmp(argv[i], "--gap")) gap_ms = std::atof(next());
    else if (!std::strcmp(argv[i], "--prefix-group")) sp.prefix_group = std::atoi(next());
    else if (!std::strcmp(argv[i], "--prefix-steps")) sp.prefix_steps = std::atoi(next());
    else if (!std::strcmp(argv[i], "--cap-mode")) {
      const char* v = next();
      if (!std::strcmp(v, "group")) sp.cap_mode = 0;
      else if (!std::strcmp(v, "perreq")) sp.cap_mode = 1;
      else {
        std::fprintf(stderr, "--cap-mode group|perreq, got %s\n", v);
        return 2;
      }
    }
    else if (!std::strcmp(argv[i], "--miss-trace")) trace = next();
    else if (!std::strcmp(argv[i], "--kv-heads")) sp.kv_heads = std::atoi(next());
    else if (!std::strcmp(argv[i], "--head-dim")) sp.head_dim = std::atoi(next());
    else {
      std::fprintf(stderr, "unknown flag %s\n", argv[i]);
      return 2;
    }
  }
  if (!trace.empty()) {
    setenv("FERRY_MISS_TRACE", trace.c_str(), 1);
    uint64_t bytes = 0;
    const uint64_t h = ferry::fnv1a64_file(trace, &bytes);
    std::printf("[trace] %s fnv1a64=%016llx bytes=%llu\n", trace.c_str(), (unsigned long long)h,
                (unsigned long long)bytes);
  }
  std::printf("[wla] gpu=%d reqs=%d layers=%d steps=%d sel=%d hot=%d arrival=%s gap=%.3fms prefix_group=%d "
              "cap_mode=%s%s%s\n",
              device, sp.num_requests, sp.num_layers, sp.steps, sp.sel_blocks, sp.hot_blocks, arrival.c_str(),
              gap_ms, sp.prefix_group, sp.cap_mode ? "perreq" : "group", trace.empty() ? "" : " trace=",
              trace.c_str());
  ferry::AdaptiveBatchPolicy pol;
  ferry::WlaStealPolicy spol;
  int rc = 0;
  const char* names[] = {"A", "B", "C"};
  for (int mode = 0; mode < 3; ++mode) {
    const ferry::WlaMultiStats st =
        ferry::run_wla_multigpu({device}, sp, mode, pol, spol, "balanced", arrival, gap_ms, 4, 8);
    print_row(names[mode], st);
    if (st.status) {
      std::printf("  error: %s\n", ferry_last_error());
      rc = 1;
    }
  }
  return rc;
}
