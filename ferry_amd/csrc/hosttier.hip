// hosttier.hip -- fill of the pinned host tier with its deterministic content.
//
// The host tier is pinned host memory mapped into the GPU address space; this
// kernel writes it directly over the host link, 16 bytes per thread.  Content
// is a pure function of (seed, host block, element) so that any reader can
// regenerate it.  The reference fills its slab on the CPU with uniform halves
// (src/workloads/kv_exec.cuh:78-86).
#include "common.hpp"
#include "kernels.hpp"

namespace ferry_amd {

__global__ void k_hosttier_fill(Geo g, uint8_t* host, float* scales, uint64_t seed, float mult,
                                float mult8, float scale_base) {
  const uint64_t words_per_block = g.bb / 16;
  const uint64_t total = g.host_blocks * words_per_block;
  const uint64_t elems_per_block = 2ull * (uint64_t)g.T * (uint64_t)g.D;
  const int epw = 16 / g.esize;  // elements per 16-byte word
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint64_t h = i / words_per_block;
    const uint32_t e0 = (uint32_t)((i % words_per_block) * (uint64_t)epw);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    for (int j = 0; j < epw; ++j) {
      const uint32_t v = host_elem(g.dtype, seed, elems_per_block, h, e0 + j, mult, mult8);
      const int bit = j * g.esize * 8;
      w[bit >> 5] |= v << (bit & 31);
    }
    uint4 o;
    o.x = w[0];
    o.y = w[1];
    o.z = w[2];
    o.w = w[3];
    reinterpret_cast<uint4*>(host)[i] = o;
  }
  if (scales) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < g.host_blocks * 2; i += stride)
      scales[i] = host_scale(g.dtype, seed, i >> 1, (int)(i & 1), scale_base);
  }
}

}  // namespace ferry_amd
