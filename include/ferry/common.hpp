// common.hpp -- the reference's support layer for code written against it
// (src/common/cuda_check.cuh:9-28, src/common/timer.cuh:11-46): checks that
// print the failing call's site and end the process, and a host and a GPU
// timer with the reference's calls.
//
// The executor never exits: every entry point of include/ferry_amd.h returns
// a status.  FERRY_CHECK gives a driver the reference's behaviour for those
// statuses; FERRY_HIP_CHECK does the same for the caller's own HIP calls.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>

#include "../ferry_amd.h"

// A HIP call that does not return hipSuccess: file:line, the call and HIP's
// message on stderr, then exit(EXIT_FAILURE) (the reference's CUDA_CHECK).
#define FERRY_HIP_CHECK(call)                                                                \
  do {                                                                                       \
    const hipError_t ferry_e_ = (call);                                                      \
    if (ferry_e_ != hipSuccess) {                                                            \
      std::fprintf(stderr, "%s:%d: %s failed: %s\n", __FILE__, __LINE__, #call,              \
                   hipGetErrorString(ferry_e_));                                             \
      std::exit(EXIT_FAILURE);                                                               \
    }                                                                                        \
  } while (0)

// The last launch's error, checked the same way (the reference's CUDA_CHECK_LAST).
#define FERRY_HIP_CHECK_LAST() FERRY_HIP_CHECK(hipGetLastError())

// An executor entry point whose status is not FERRY_OK: file:line, the call,
// the status and ferry_last_error() on stderr, then exit(EXIT_FAILURE).
#define FERRY_CHECK(call)                                                                    \
  do {                                                                                       \
    const int ferry_s_ = (call);                                                             \
    if (ferry_s_ != FERRY_OK) {                                                              \
      std::fprintf(stderr, "%s:%d: %s failed: status %d: %s\n", __FILE__, __LINE__, #call,   \
                   ferry_s_, ferry_last_error());                                            \
      std::exit(EXIT_FAILURE);                                                               \
    }                                                                                        \
  } while (0)

namespace ferry {

// Wall-clock interval on the host's monotonic clock, in milliseconds.
struct HostTimer {
  std::chrono::steady_clock::time_point start = std::chrono::steady_clock::now();

  void tick() { start = std::chrono::steady_clock::now(); }
  double toc_ms() const {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
  }
};

// GPU interval between two events recorded on a stream (or two streams, for
// work that spans them), in milliseconds: the reference's CudaTimer on HIP.
// elapsed_ms() needs the end event complete (hipEventSynchronize(end) or a
// synchronisation of its stream).
struct HipTimer {
  hipEvent_t begin = nullptr, end = nullptr;

  HipTimer() {
    FERRY_HIP_CHECK(hipEventCreate(&begin));
    FERRY_HIP_CHECK(hipEventCreate(&end));
  }
  ~HipTimer() {
    if (begin) (void)hipEventDestroy(begin);
    if (end) (void)hipEventDestroy(end);
  }
  HipTimer(const HipTimer&) = delete;
  HipTimer& operator=(const HipTimer&) = delete;

  void tick(hipStream_t stream = nullptr) { FERRY_HIP_CHECK(hipEventRecord(begin, stream)); }
  void toc(hipStream_t stream = nullptr) { FERRY_HIP_CHECK(hipEventRecord(end, stream)); }
  float elapsed_ms() const {
    float ms = 0.0f;
    FERRY_HIP_CHECK(hipEventElapsedTime(&ms, begin, end));
    return ms;
  }
};

}  // namespace ferry
