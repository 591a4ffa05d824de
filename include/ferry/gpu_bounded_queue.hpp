// gpu_bounded_queue.hpp -- device-resident bounded MPMC ring for HIP (gfx950).
//
// Keeps the reference's interface (src/queue/gpu_bounded_queue.cuh:50-198):
// ReservationMode, DeviceQueue, dq_size, dq_push, dq_pop and the host wrapper
// GPUBoundedQueue with device_ptr/mode/capacity/reset/snapshot.  Differences,
// all deliberate:
//  * slots carry a sequence word instead of a 0/1 ready flag: the producer of
//    ticket i waits for seq == i and publishes seq = i + 1, the consumer of
//    ticket i requires seq == i + 1 and releases seq = i + capacity.  A 0/1
//    flag cannot tell a not-yet-released cell of lap i - capacity from a
//    published cell of lap i, so a consumer could read the older task;
//  * kWaveBatched reserves one ticket per active lane of the 64-wide
//    wavefront with a single CAS by the first active lane (the reference
//    reserves a fixed 32 per warp) and broadcasts with readfirstlane; a ring
//    with fewer cells than active lanes takes them one per lane;
//  * a lane publishes (and a consumer takes its task) as soon as its own cell
//    is ready, inside the wait: lanes of one wavefront may hold tickets a lap
//    apart, and a lane that waited for its siblings could stall them all;
//  * dq_pop reserves for the wavefront in the same way, in both modes: the
//    first active lane takes up to one ticket per active lane (fewer when
//    fewer are queued) with one CAS on head.  A per-lane CAS loop, as in the
//    reference, makes the 64 lanes of a wavefront race each other for the
//    same word, one winner per round; on MI355X that holds a ring to ~0.1 M
//    pops/s under 512 consumers;
//  * every wait is bounded; a wait that runs out sets `status` and the call
//    returns false, so a broken protocol ends the kernel instead of hanging.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ferry {

enum class ReservationMode { kPerThread = 0, kWaveBatched = 1 };

// head and tail each own a 128-byte line: producers' CAS on tail and
// consumers' CAS on head then never contend for one L2 line, nor with the
// read-mostly fields.
struct DeviceQueue {
  uint64_t* slots = nullptr;  // [capacity] payloads
  uint64_t* seq = nullptr;    // [capacity] cell sequence words
  uint64_t capacity = 0;
  int status = 0;             // nonzero once a bounded wait ran out
  alignas(128) uint64_t head = 0;  // next ticket to pop
  alignas(128) uint64_t tail = 0;  // next ticket to push
};

constexpr long kQueueSpinLimit = 1L << 22;

#if defined(__HIPCC__)
__device__ inline uint64_t q_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void q_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void q_fail(DeviceQueue* q) { atomicExch(&q->status, 1); }

__device__ inline uint64_t dq_size(DeviceQueue* q) {
  const uint64_t t = q_load(&q->tail);
  const uint64_t h = q_load(&q->head);
  return t > h ? t - h : 0;
}

// Reserve `n` consecutive tickets if the ring has room; false when full.
__device__ inline bool q_reserve(DeviceQueue* q, uint64_t n, uint64_t* base) {
  for (long spin = 0; spin < kQueueSpinLimit; ++spin) {
    const uint64_t t = q_load(&q->tail);
    const uint64_t h = q_load(&q->head);
    if (t - h + n > q->capacity) return false;
    if (atomicCAS((unsigned long long*)&q->tail, t, t + n) == t) {
      *base = t;
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  q_fail(q);
  return false;
}

// Publish every active lane's task once its cell has been released for its
// ticket.  A lane publishes inside the wait, as soon as its own cell is ready:
// lanes of one wavefront can hold tickets a lap apart (per-thread reservation
// under more producers than cells), and the later one's cell is released only
// after the earlier one's task is consumed, so a lane that waited for its
// siblings before publishing would stall the wavefront for good.
__device__ inline bool q_publish(DeviceQueue* q, uint64_t ticket, uint64_t task) {
  const uint64_t cell = ticket % q->capacity;
  bool done = false;
  for (long spin = 0;; ++spin) {
    if (!done && q_load(q->seq + cell) == ticket) {
      q->slots[cell] = task;
      q_store(q->seq + cell, ticket + 1);
      done = true;
    }
    if (!__ballot(!done)) return true;
    if (spin >= kQueueSpinLimit) {
      if (!done) q_fail(q);
      return done;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Push one task.  true on success, false when the ring is full (backpressure
// is the caller's decision) or a bounded wait ran out (status set).
__device__ inline bool dq_push(DeviceQueue* q, uint64_t task, ReservationMode mode) {
  const uint64_t active = __ballot(true);
  const int n = __builtin_popcountll(active);
  // a ring with fewer cells than the wavefront's active lanes could never
  // hold the batch: its lanes reserve one ticket each instead
  if (mode == ReservationMode::kPerThread || (uint64_t)n > q->capacity) {
    uint64_t t;
    if (!q_reserve(q, 1, &t)) return false;
    return q_publish(q, t, task);
  }
  const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(active >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)active, 0));
  uint64_t base = 0;
  int ok = 0;
  if (below == 0) ok = q_reserve(q, (uint64_t)n, &base) ? 1 : 0;
  ok = __builtin_amdgcn_readfirstlane(ok);
  if (!ok) return false;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
  base = ((uint64_t)hi << 32) | lo;
  return q_publish(q, base + (uint64_t)below, task);
}

// Take up to `n` consecutive tickets of pushed tasks; returns how many (0
// when the ring is empty).  Tickets past the tail are never taken; a taken
// ticket's task may still be in the producer's hands (reserved, not yet
// published), and its consumer waits for it.
__device__ inline uint64_t q_take(DeviceQueue* q, uint64_t n, uint64_t* base) {
  for (long spin = 0; spin < kQueueSpinLimit; ++spin) {
    const uint64_t h = q_load(&q->head);
    const uint64_t t = q_load(&q->tail);
    if (h >= t) return 0;
    const uint64_t m = t - h < n ? t - h : n;
    if (atomicCAS((unsigned long long*)&q->head, h, h + m) == h) {
      *base = h;
      return m;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  q_fail(q);
  return 0;
}

// Pop one task into *out.  false when empty (or a bounded wait ran out).
// Call it from whole or partial wavefronts alike: the active lanes share one
// reservation, and a lane left without a ticket sees an empty ring.
__device__ inline bool dq_pop(DeviceQueue* q, uint64_t* out) {
  const uint64_t active = __ballot(true);
  const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(active >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)active, 0));
  uint64_t base = 0;
  int got = 0;
  if (below == 0) got = (int)q_take(q, (uint64_t)__builtin_popcountll(active), &base);
  got = __builtin_amdgcn_readfirstlane(got);
  if (below >= got) return false;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(base >> 32));
  const uint64_t h = (((uint64_t)hi << 32) | lo) + (uint64_t)below;
  const uint64_t cell = h % q->capacity;
  // a taken ticket may be reserved and not yet published: each lane consumes
  // (and releases its cell) as soon as its own task is there, as q_publish does
  bool done = false;
  for (long spin = 0;; ++spin) {
    if (!done && q_load(q->seq + cell) == h + 1) {
      *out = q->slots[cell];
      q_store(q->seq + cell, h + q->capacity);
      done = true;
    }
    if (!__ballot(!done)) return true;
    if (spin >= kQueueSpinLimit) {
      if (!done) q_fail(q);
      return done;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}
#endif

// Host wrapper (owns the device ring).  Errors are reported through ok().
class GPUBoundedQueue {
 public:
  GPUBoundedQueue(uint64_t capacity, ReservationMode mode) : mode_(mode), capacity_(capacity) {
    ok_ = capacity > 0 &&
          hipMalloc(&state_.slots, capacity * sizeof(uint64_t)) == hipSuccess &&
          hipMalloc(&state_.seq, capacity * sizeof(uint64_t)) == hipSuccess &&
          hipMalloc(&dev_, sizeof(DeviceQueue)) == hipSuccess;
    state_.capacity = capacity;
    if (ok_) ok_ = reset();
  }
  ~GPUBoundedQueue() {
    if (state_.slots) (void)hipFree(state_.slots);
    if (state_.seq) (void)hipFree(state_.seq);
    if (dev_) (void)hipFree(dev_);
  }
  GPUBoundedQueue(const GPUBoundedQueue&) = delete;
  GPUBoundedQueue& operator=(const GPUBoundedQueue&) = delete;

  bool ok() const { return ok_; }
  DeviceQueue* device_ptr() { return dev_; }
  ReservationMode mode() const { return mode_; }
  uint64_t capacity() const { return capacity_; }

  // Empty the ring: cursors to zero, every cell's sequence to its index.
  bool reset() {
    state_.head = state_.tail = 0;
    state_.status = 0;
    uint64_t* init = new uint64_t[capacity_];
    for (uint64_t i = 0; i < capacity_; ++i) init[i] = i;
    const bool a = hipMemcpy(state_.seq, init, capacity_ * sizeof(uint64_t), hipMemcpyHostToDevice) == hipSuccess;
    delete[] init;
    return a && hipMemcpy(dev_, &state_, sizeof(DeviceQueue), hipMemcpyHostToDevice) == hipSuccess;
  }

  struct Snapshot {
    uint64_t head, tail, capacity;
    int status;
  };
  Snapshot snapshot() const {
    DeviceQueue q;
    if (hipMemcpy(&q, dev_, sizeof(DeviceQueue), hipMemcpyDeviceToHost) != hipSuccess) q.status = -1;
    return {q.head, q.tail, q.capacity, q.status};
  }

 private:
  ReservationMode mode_;
  uint64_t capacity_;
  DeviceQueue state_{};
  DeviceQueue* dev_ = nullptr;
  bool ok_ = false;
};

}  // namespace ferry
