// trace.cpp -- reader of FMT1 selection traces.
//
// FMT1 is the reference's on-disk record of real top-k selections
// (tools/capture_miss_trace.py:27-38 for the header, :316-317 and :366-370
// for the records): little-endian "FMT1", version 1, R, steps, layers,
// page_tokens, block_tokens, kv_heads, head_dim, sel_pages (u32 each), then
// for every (request, step, layer) a u16 count and count u32 block ids.  The
// ids are chained content hashes, so blocks of a shared prefix have the same
// id in every request of a group.  As the reference's loader does
// (src/workloads/miss_trace.cuh:75-185), ids are renamed to dense ids in
// order of first appearance over the whole trace, and the largest number of
// distinct ids one request touches is reported (the reference sizes its host
// slab with it).  Unlike the reference, errors are returned (FERRY_EINVAL with
// the reason in ferry_last_error) instead of exiting, and a short record may
// be accepted (strict == 0) and padded with FERRY_EMPTY.
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/ferry_amd.h"
#include "errors.hpp"

using ferry_amd::report;

namespace {

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

bool read_u32(FILE* f, uint32_t* v) {
  unsigned char b[4];
  if (std::fread(b, 1, 4, f) != 4) return false;
  *v = (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24;
  return true;
}

bool read_u16(FILE* f, uint32_t* v) {
  unsigned char b[2];
  if (std::fread(b, 1, 2, f) != 2) return false;
  *v = (uint32_t)b[0] | (uint32_t)b[1] << 8;
  return true;
}

}  // namespace

extern "C" {

int ferry_trace_load(const char* path, int strict, ferry_trace_info* info, uint32_t* out_ids,
                     uint64_t capacity) {
  if (!path || !info) return report(FERRY_EINVAL, "null path or info");
  const std::string where = std::string(path) + ": ";
  File fh;
  fh.f = std::fopen(path, "rb");
  if (!fh.f) return report(FERRY_EINVAL, where + "cannot open");
  FILE* f = fh.f;
  char magic[4];
  if (std::fread(magic, 1, 4, f) != 4 || std::memcmp(magic, "FMT1", 4) != 0)
    return report(FERRY_EINVAL, where + "magic is not FMT1");
  uint32_t h[9];
  for (uint32_t& v : h)
    if (!read_u32(f, &v)) return report(FERRY_EINVAL, where + "truncated header");
  if (h[0] != 1) return report(FERRY_EINVAL, where + "version is not 1");
  ferry_trace_info in{};
  in.requests = h[1];
  in.steps = h[2];
  in.layers = h[3];
  in.page_tokens = h[4];
  in.block_tokens = h[5];
  in.kv_heads = h[6];
  in.head_dim = h[7];
  in.sel_pages = h[8];
  if (in.block_tokens == 0 || in.page_tokens == 0 || in.page_tokens % in.block_tokens)
    return report(FERRY_EINVAL, where + "page_tokens is not a positive multiple of block_tokens");
  const uint64_t sel64 = (uint64_t)in.sel_pages * (in.page_tokens / in.block_tokens);
  if (sel64 == 0 || sel64 > 65535) return report(FERRY_EINVAL, where + "selected blocks per record out of range");
  in.sel_blocks = (uint32_t)sel64;
  const uint64_t total = (uint64_t)in.requests * in.steps * in.layers * in.sel_blocks;
  if (out_ids && capacity < total)
    return report(FERRY_EINVAL, where + "output holds " + std::to_string(capacity) + " ids, the trace has " +
                                    std::to_string(total));
  std::unordered_map<uint32_t, uint32_t> dense;
  std::vector<uint32_t> ids(in.sel_blocks);
  uint64_t pos = 0;
  for (uint32_t r = 0; r < in.requests; ++r) {
    std::unordered_set<uint32_t> mine;
    for (uint32_t s = 0; s < in.steps; ++s)
      for (uint32_t l = 0; l < in.layers; ++l, pos += in.sel_blocks) {
        uint32_t cnt = 0;
        if (!read_u16(f, &cnt)) return report(FERRY_EINVAL, where + "truncated payload (record count)");
        const std::string rec =
            " at (r=" + std::to_string(r) + ", s=" + std::to_string(s) + ", l=" + std::to_string(l) + ")";
        if (cnt > in.sel_blocks)
          return report(FERRY_EINVAL, where + std::to_string(cnt) + " ids" + rec + ", more than " +
                                          std::to_string(in.sel_blocks));
        if (cnt < in.sel_blocks) {
          if (strict)
            return report(FERRY_EINVAL, where + std::to_string(cnt) + " ids" + rec + ", expected " +
                                            std::to_string(in.sel_blocks));
          ++in.short_records;
        }
        for (uint32_t k = 0; k < cnt; ++k)
          if (!read_u32(f, &ids[k])) return report(FERRY_EINVAL, where + "truncated payload (block ids)");
        for (uint32_t k = 0; k < in.sel_blocks; ++k) {
          uint32_t d = FERRY_EMPTY;
          if (k < cnt) {
            const uint32_t raw = ids[k];
            mine.insert(raw);
            auto it = dense.find(raw);
            if (it == dense.end()) it = dense.emplace(raw, (uint32_t)dense.size()).first;
            d = it->second;
          }
          if (out_ids) out_ids[pos + k] = d;
        }
      }
    if (mine.size() > in.max_blocks_per_req) in.max_blocks_per_req = mine.size();
  }
  in.unique_blocks = dense.size();
  *info = in;
  return FERRY_OK;
}

}  // extern "C"
