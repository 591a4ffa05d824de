"""The reference-API shim's C-engine refill count (include/ferry/ferry.hpp,
ferry::detail::cmode_submits) on the CPU: compiled into a small host program
and fed the restated replay_miss_stream of the reference's golden commands.
It must give the reference's golden submit counts -- 59,863 for the default
stream under the default policy (target 4 batches, results/wla_7rep_20260930/
*.log), 1,227 for the 4-request single-GPU run under run_missstream's policy
(target 8, 实验设计.txt:495) -- and agree with the oracle's restated planner
(ora_ref_cmode_runs, kv_exec.cuh:188-292) on random streams and policies."""
import os
import subprocess

import numpy as np
import pytest

from oracle import pyoracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROG = r'''
#include <cstdio>
#include <vector>
#include "ferry/ferry.hpp"
int main(int argc, char** argv) {
  FILE* f = std::fopen(argv[1], "rb");
  int hdr[4];
  double pol3[3];
  unsigned long long c4;
  if (std::fread(hdr, 4, 4, f) != 4 || std::fread(&c4, 8, 1, f) != 1 || std::fread(pol3, 8, 3, f) != 3) return 2;
  const int R = hdr[0], L = hdr[1], S = hdr[2], G = hdr[3];
  const size_t n = (size_t)R * S * L * G;
  std::vector<unsigned long long> blk(n);
  std::vector<unsigned char> miss(n);
  if (std::fread(blk.data(), 8, n, f) != n || std::fread(miss.data(), 1, n, f) != n) return 2;
  ferry::AdaptiveBatchPolicy pol;
  pol.min_mb = pol3[0];
  pol.max_mb = pol3[1];
  pol.target_batches = pol3[2];
  unsigned long long events = 0, bytes = 0;
  std::vector<std::pair<int, uint64_t>> ml;
  for (int r = 0; r < R; ++r)
    for (int s = 0; s < S; ++s) {
      ml.clear();
      for (int l = 0; l < L; ++l)
        for (int k = 0; k < G; ++k) {
          const size_t e = (((size_t)r * S + s) * L + l) * G + k;
          if (miss[e]) ml.push_back({l, blk[e]});
        }
      uint64_t b = 0;
      events += ferry::detail::cmode_submits(ml, (size_t)c4, pol, &b);
      bytes += b;
    }
  std::printf("%llu %llu\n", events, bytes);
  return 0;
}
'''


@pytest.fixture(scope="module")
def prog(tmp_path_factory):
    d = tmp_path_factory.mktemp("shim")
    src, exe = d / "count.cpp", d / "count"
    src.write_text(PROG)
    res = subprocess.run(["/opt/rocm/bin/hipcc", "-O1", "-std=c++17", "-I", os.path.join(ROOT, "include"),
                          str(src), "-o", str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return exe, d


def _count(prog, R, L, S, G, blocks, miss, c4, min_mb=1.0, max_mb=4.0, target=4.0):
    exe, d = prog
    path = d / "stream.bin"
    with open(path, "wb") as f:
        f.write(np.array([R, L, S, G], np.int32).tobytes())
        f.write(np.array([c4], np.uint64).tobytes())
        f.write(np.array([min_mb, max_mb, target], np.float64).tobytes())
        f.write(np.ascontiguousarray(blocks, np.uint64).tobytes())
        f.write(np.ascontiguousarray(miss, np.uint8).tobytes())
    out = subprocess.run([str(exe), str(path)], capture_output=True, text=True, check=True).stdout
    ev, by = map(int, out.split())
    return ev, by


def test_shim_golden_submit_counts(prog):
    blocks, miss, _, nm = O.ref_replay(48, 12, 16, 64, 128)
    assert nm == 79550
    assert _count(prog, 48, 12, 16, 64, blocks, miss, 16384) == (59863, 79550 * 16384)
    ev8 = _count(prog, 48, 12, 16, 64, blocks, miss, 16384, target=8.0)
    assert ev8 == O.ref_cmode_runs(48, 12, 16, 64, 128, 16384, blocks, miss, target=8.0)
    blocks, miss, _, nm = O.ref_replay(4, 12, 4, 128, 1024)
    assert nm == 3690
    assert _count(prog, 4, 12, 4, 128, blocks, miss, 16384, target=8.0) == (1227, 3690 * 16384)


@pytest.mark.parametrize("seed", range(4))
def test_shim_matches_oracle_planner(prog, seed):
    rng = np.random.default_rng(seed)
    R, L, S, G = int(rng.integers(1, 6)), int(rng.integers(1, 9)), int(rng.integers(1, 6)), \
        int(rng.integers(8, 200))
    hot = int(rng.integers(G, 4 * G + 1))
    blocks, miss, _, _ = O.ref_replay(R, L, S, G, hot, seed=int(rng.integers(1 << 30)))
    c4 = int(rng.choice([4096, 16384, 65536]))
    mn = float(rng.choice([0.0625, 0.25, 1.0]))
    mx = mn * float(rng.choice([1, 2, 8]))
    tg = float(rng.choice([1.0, 2.0, 4.0, 8.0]))
    got = _count(prog, R, L, S, G, blocks, miss, c4, mn, mx, tg)
    assert got == O.ref_cmode_runs(R, L, S, G, hot, c4, blocks, miss, min_mb=mn, max_mb=mx, target=tg)
