// ref_replay_main.cpp -- driver that links the reference's own generator.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile from this file plus the
// reference header src/workloads/missstream.cuh (host-only C++, no CUDA
// includes) taken where it lies in the reference tree; output goes to
// oracle/_ref/ only.  It runs ferry::replay_miss_stream (missstream.cuh:104)
// and writes, for every MissEvent in order, the block id (u64) and the miss
// flag (u8), so tests can compare the oracle's restatement event by event.
//
// usage: ref_replay R L S sel hot seed out.bin   (prints "selects misses")
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "workloads/missstream.cuh"

int main(int argc, char** argv) {
  if (argc != 8) {
    std::fprintf(stderr, "usage: %s R L S sel hot seed out.bin\n", argv[0]);
    return 2;
  }
  ferry::MissSpec sp;
  sp.num_requests = std::atoi(argv[1]);
  sp.num_layers = std::atoi(argv[2]);
  sp.steps = std::atoi(argv[3]);
  sp.sel_blocks = std::atoi(argv[4]);
  sp.hot_blocks = std::atoi(argv[5]);
  sp.seed = std::strtoull(argv[6], nullptr, 10);
  ferry::MissTrace tr = ferry::replay_miss_stream(sp);
  std::FILE* f = std::fopen(argv[7], "wb");
  if (!f) return 1;
  std::vector<unsigned long long> blk(tr.events.size());
  std::vector<unsigned char> mis(tr.events.size());
  for (size_t i = 0; i < tr.events.size(); ++i) {
    blk[i] = tr.events[i].block_id;
    mis[i] = tr.events[i].is_miss ? 1 : 0;
  }
  std::fwrite(blk.data(), 8, blk.size(), f);
  std::fwrite(mis.data(), 1, mis.size(), f);
  std::fclose(f);
  std::printf("%llu %llu\n", (unsigned long long)tr.total_selects,
              (unsigned long long)tr.total_misses);
  return 0;
}
