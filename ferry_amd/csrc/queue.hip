// queue.hip -- exactly-once acceptance of the device MPMC ring.
//
// One kernel, roles split by block index as in the reference's pc_kernel
// (src/benches/bench_queue.cu:26-59): producer blocks push unique task ids,
// consumer blocks pop them and count arrivals per id in seen[].  The grid is
// small enough to be co-resident, and every wait in the queue is bounded.
// Consumers count each id's arrivals in seen[]; the host then finds ids that
// arrived twice or never.
#include "common.hpp"
#include "../../include/ferry/gpu_bounded_queue.hpp"

namespace ferry_amd {

__global__ __launch_bounds__(256) void k_queue_pc(ferry::DeviceQueue* q, uint64_t per_thread,
                                                  uint32_t n_prod_blocks, uint32_t* seen,
                                                  unsigned long long* popped,
                                                  unsigned long long* dups, int* done,
                                                  int* prod_blocks_done, ferry::ReservationMode mode) {
  if (blockIdx.x < n_prod_blocks) {
    const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (uint64_t i = 0; i < per_thread; ++i) {
      const uint64_t task = tid * per_thread + i;
      long tries = 0;
      while (!ferry::dq_push(q, task, mode)) {
        if (__hip_atomic_load(&q->status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ||
            ++tries > ferry::kQueueSpinLimit) {
          atomicExch(&q->status, 2);
          break;
        }
        __builtin_amdgcn_s_sleep(4);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      __threadfence();
      if (atomicAdd(prod_blocks_done, 1) + 1 == (int)n_prod_blocks) atomicExch(done, 1);
    }
  } else {
    const uint64_t n_tasks = per_thread * n_prod_blocks * (uint64_t)blockDim.x;
    long idle = 0;
    unsigned long long mine = 0;
    while (true) {
      uint64_t task;
      if (ferry::dq_pop(q, &task)) {
        // the count's old value is not read back (a non-returning atomic, no
        // round trip per pop); the host finds ids seen twice or never
        if (task < n_tasks) atomicAdd(seen + task, 1u);
        else atomicAdd(dups, 1ull);  // an id no producer pushed
        ++mine;
        idle = 0;
      } else {
        const int d = __hip_atomic_load(done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
        if ((d && ferry::dq_size(q) == 0) ||
            __hip_atomic_load(&q->status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          break;
        if (++idle > ferry::kQueueSpinLimit) {
          atomicExch(&q->status, 3);
          break;
        }
        __builtin_amdgcn_s_sleep(4);
      }
    }
    atomicAdd(popped, mine);
  }
}

// The ceiling of the ring's tickets: every thread takes `iters` tickets from
// one shared 64-bit word, by
//  * kind 0: fetch-add per thread (the rate one address accepts returning
//    atomics);
//  * kind 1: a relaxed load + compare-and-swap retry per thread, as
//    kPerThread's push reservation does;
//  * kind 2: the same retry by the first lane of each wavefront for all 64
//    lanes, as the wave-batched push and every pop do.
// A thread whose retries on one ticket pass the queue's spin bound stops and
// latches `failed`, so every wavefront ends.
__global__ __launch_bounds__(256) void k_ticket_probe(unsigned long long* word, int iters, int kind,
                                                      int* failed) {
  unsigned long long acc = 0;
  const int lane = threadIdx.x & 63;
  for (int i = 0; i < iters; ++i) {
    if (kind == 0) {
      acc += atomicAdd(word, 1ull);
      continue;
    }
    if (kind == 2 && lane != 0) continue;
    const unsigned long long n = kind == 2 ? 64 : 1;
    for (long spin = 0;; ++spin) {
      const unsigned long long v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (atomicCAS(word, v, v + n) == v) {
        acc += v;
        break;
      }
      if (spin > ferry::kQueueSpinLimit) {
        atomicExch(failed, 1);
        return;
      }
    }
  }
  if (acc == ~0ull) atomicExch(failed, 2);  // keeps the returned tickets live
}

}  // namespace ferry_amd
