// Host-side driver for the C ABI of libtjhip (include/tensorjit_hip.h), built together with
// csrc/runtime.cpp under AddressSanitizer + UndefinedBehaviorSanitizer (host code only) by
// tests/test_abi_sanitized.py.  It exercises every path that needs no GPU: versions, hipRTC
// compile errors and success, and every argument-validation failure of program creation and
// the run entry points; each must return nonzero with the expected message.
#include "../../include/tensorjit_hip.h"

#include <cstdio>
#include <cstring>
#include <vector>

static int failures = 0;

static void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL: %s (last error: %s)\n", what, tj_hip_last_error());
    ++failures;
  }
}

static bool error_has(const char* needle) { return std::strstr(tj_hip_last_error(), needle) != nullptr; }

static int create_one(const std::vector<tj_argref>& refs, size_t arena, int n_in, int n_out) {
  const char* names[1] = {"k"};
  tj_launch launch{};
  launch.grid[0] = launch.grid[1] = launch.grid[2] = 1;
  launch.block[0] = 64;
  launch.block[1] = launch.block[2] = 1;
  launch.nargs = static_cast<uint32_t>(refs.size());
  void* handle = reinterpret_cast<void*>(0x1);
  const char code[] = "not a code object";
  int rc = tj_hip_program_create(0, code, sizeof(code), 1, names, &launch, refs.data(), arena, n_in, n_out, &handle);
  expect(handle == nullptr, "failed create leaves the handle null");
  return rc;
}

int main() {
  expect(tj_hip_abi_version() == TJ_HIP_ABI_VERSION, "abi version");
  int major = 0, minor = 0, runtime = 0;
  expect(tj_hip_toolchain_version(&major, &minor, &runtime) == 0 && major > 0 && runtime > 0, "toolchain version");
  expect(tj_hip_toolchain_version(nullptr, &minor, &runtime) != 0, "toolchain version rejects null");

  // hipRTC: an error carries the compiler log; a good source gives a code object
  void* code = nullptr;
  size_t size = 0;
  const char* opts[] = {"--offload-arch=gfx950", "-O3"};
  expect(tj_hip_compile("extern \"C\" __global__ void k() { not hip; }", "bad.hip", opts, 2, &code, &size) != 0 &&
             error_has("hipRTC compile failed") && code == nullptr,
         "compile error");
  expect(tj_hip_compile("extern \"C\" __global__ void k(float* p) { p[threadIdx.x] = 1.0f; }", "ok.hip", opts, 2,
                        &code, &size) == 0 && code != nullptr && size > 0,
         "compile");
  tj_hip_free(code);
  expect(tj_hip_compile(nullptr, "x", opts, 2, &code, &size) != 0, "compile rejects a null source");

  // program creation: every reference is validated before any device work
  void* h = nullptr;
  expect(tj_hip_program_create(0, nullptr, 0, 0, nullptr, nullptr, nullptr, 0, 0, 0, &h) != 0 &&
             error_has("empty code object"),
         "empty code object");
  expect(tj_hip_program_create(0, "x", 1, 0, nullptr, nullptr, nullptr, 0, 0, 0, nullptr) != 0, "null handle");
  expect(tj_hip_program_create(0, "x", 1, 1, nullptr, nullptr, nullptr, 0, 0, 0, &h) != 0, "null kernel table");
  expect(tj_hip_program_create(0, "x", 1, 0, nullptr, nullptr, nullptr, 0, -1, 0, &h) != 0, "negative input count");
  expect(create_one({{TJ_ARG_INPUT, 0, 1, 0}}, 0, 1, 0) != 0 && error_has("input index out of range"), "input index");
  expect(create_one({{TJ_ARG_OUTPUT, 0, 2, 0}}, 0, 0, 2) != 0 && error_has("output index out of range"), "output index");
  expect(create_one({{TJ_ARG_ARENA, 0, 0, 4097}}, 4096, 0, 0) != 0 && error_has("outside the 4096-byte arena"),
         "arena overrun");
  expect(create_one({{TJ_ARG_ARENA, 0, 4096, 1}}, 4096, 0, 0) != 0 && error_has("outside"), "arena offset at end");
  expect(create_one({{TJ_ARG_ARENA, 0, -64, 64}}, 4096, 0, 0) != 0 && error_has("outside"), "negative arena offset");
  expect(create_one({{TJ_ARG_ARENA, 0, 0, 0}}, 4096, 0, 0) != 0 && error_has("outside"), "unsized arena reference");
  expect(create_one({{TJ_ARG_ARENA, 0, 64, INT64_MAX}}, 4096, 0, 0) != 0 && error_has("outside"), "huge arena size");
  expect(create_one({{7, 0, 0, 0}}, 0, 0, 0) != 0 && error_has("bad argument kind"), "argument kind");
  std::vector<tj_argref> many(65, tj_argref{TJ_ARG_INPUT, 0, 0, 0});
  expect(create_one(many, 0, 1, 0) != 0 && error_has("too many kernel arguments"), "argument count");
  // valid references get as far as the (bogus) code object
  expect(create_one({{TJ_ARG_INPUT, 0, 0, 0}, {TJ_ARG_ARENA, 0, 64, 4032}, {TJ_ARG_OUTPUT, 0, 0, 0}}, 4096, 1, 1) != 0 &&
             error_has("hipModuleLoadData"),
         "valid references reach the loader");

  // run entry points on a null program
  expect(tj_hip_program_run(nullptr, nullptr, nullptr, nullptr) != 0 && error_has("null program"), "run null");
  expect(tj_hip_program_run_static(nullptr, nullptr, nullptr, nullptr) != 0 && error_has("null program"),
         "run_static null");
  expect(tj_hip_program_replay(nullptr, nullptr, nullptr, nullptr) != 0, "replay null");
  expect(tj_hip_program_capture(nullptr, nullptr, nullptr) != 0, "capture null");
  tj_stats st;
  expect(tj_hip_program_stats(nullptr, &st) != 0, "stats null");
  float ms = 0.f;
  expect(tj_hip_kernel_time(nullptr, 0, nullptr, nullptr, nullptr, 1, 1, &ms) != 0, "kernel_time null");
  expect(tj_hip_program_time_kernels(nullptr, nullptr, nullptr, nullptr, &ms) != 0 && error_has("null argument"),
         "time_kernels null");
  expect(tj_hip_program_destroy(nullptr) == 0, "destroy null");
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
