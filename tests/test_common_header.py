"""include/ferry/common.hpp on the CPU: the reference's support layer
(src/common/cuda_check.cuh:9-28, timer.cuh:11-46) for code written against
it.  A host program built with hipcc times an interval with HostTimer, and a
failing executor status (FERRY_CHECK) or HIP call (FERRY_HIP_CHECK) prints
its call site and ends the process with EXIT_FAILURE, as the reference's
checks do.  No device call succeeds or is needed."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROG = r'''
#include <chrono>
#include <cstdio>
#include <cstring>
#include <thread>
#include "ferry/common.hpp"
int main(int argc, char** argv) {
  if (argc > 1 && !std::strcmp(argv[1], "timer")) {
    ferry::HostTimer t;
    t.tick();
    std::this_thread::sleep_for(std::chrono::milliseconds(30));
    std::printf("%.3f\n", t.toc_ms());
    return 0;
  }
  if (argc > 1 && !std::strcmp(argv[1], "status")) {
    ferry_ctx* ctx = nullptr;
    FERRY_CHECK(ferry_ctx_create(nullptr, 0, &ctx));  // no config: FERRY_EINVAL
    return 0;
  }
  if (argc > 1 && !std::strcmp(argv[1], "hip")) {
    FERRY_HIP_CHECK(hipSetDevice(99999));  // no such device anywhere
    return 0;
  }
  FERRY_CHECK(FERRY_OK);
  FERRY_HIP_CHECK(hipSuccess);
  std::puts("ok");
  return 0;
}
'''


@pytest.fixture(scope="module")
def prog(tmp_path_factory):
    lib = os.path.join(ROOT, "ferry_amd")
    if not os.path.exists(os.path.join(lib, "libferry_amd.so")):
        pytest.skip("libferry_amd.so not built")
    d = tmp_path_factory.mktemp("common")
    src, exe = d / "common.cpp", d / "common"
    src.write_text(PROG)
    res = subprocess.run(["/opt/rocm/bin/hipcc", "-O1", "-std=c++17", "-I", os.path.join(ROOT, "include"),
                          str(src), "-o", str(exe), "-L", lib, "-lferry_amd", "-Wl,-rpath," + lib],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return exe


def test_host_timer_measures_an_interval(prog):
    out = subprocess.run([str(prog), "timer"], capture_output=True, text=True, check=True).stdout
    assert 29.0 <= float(out) < 1000.0


def test_passing_checks_do_nothing(prog):
    assert subprocess.run([str(prog)], capture_output=True, text=True, check=True).stdout == "ok\n"


def test_failed_status_exits_with_its_site_and_reason(prog):
    res = subprocess.run([str(prog), "status"], capture_output=True, text=True)
    assert res.returncode == 1  # EXIT_FAILURE
    # the call site, the call, the status (FERRY_EINVAL) and ferry_last_error()
    assert "common.cpp:" in res.stderr
    assert "ferry_ctx_create(nullptr, 0, &ctx) failed: status -1: null config" in res.stderr


def test_failed_hip_call_exits_with_its_site(prog):
    res = subprocess.run([str(prog), "hip"], capture_output=True, text=True)
    assert res.returncode == 1
    assert "common.cpp:" in res.stderr and "hipSetDevice(99999) failed" in res.stderr
