/* tensorjit HIP executor: C ABI.
 *
 * The `hip` backend generates shape-specialised HIP C++ for a fused kernel
 * program, compiles it with hipRTC and runs it through these entry points.
 * Plain C types only (pointers, sizes, handles); the caller owns input and
 * output device buffers, the program owns its code object, its arena (one
 * hipMalloc) and its graph executables.
 *
 * Every function returns 0 on success and a nonzero status on failure; the
 * message (hipRTC log included) is then available from tj_hip_last_error()
 * on the calling thread.
 *
 * What each entry point replaces in the reference (sanjaybharvad007/mlir-gpu-kernel-compiler):
 *   tj_hip_compile          NVRTC compile_to_ptx          tensorjit/backends/cuda_driver.py:79-96
 *   tj_hip_program_create   _runtime.Program(...) ctor    csrc/runtime.cpp:46-78 (arg-ref validation
 *                           + arena) and Module(ptx)      tensorjit/backends/cuda_driver.py:99-113
 *   tj_hip_program_run      _runtime.Program.run          csrc/runtime.cpp:88-110, and the per-kernel
 *                           Module.launch loop            tensorjit/backends/cuda_backend.py:511-514,
 *                                                         tensorjit/backends/cuda_driver.py:115-124
 *   tj_hip_program_capture  Graph.capture                 tensorjit/backends/cuda_driver.py:144-154
 *   tj_hip_program_replay   Graph.launch                  tensorjit/backends/cuda_driver.py:156-159
 *   tj_hip_program_stats    Program.calls / mean_us and   csrc/runtime.cpp:112-120,
 *                           CudaProgram.stats             tensorjit/backends/cuda_backend.py:491
 *   tj_hip_program_destroy  ~Program / Module.__del__ /   csrc/runtime.cpp:80-83,
 *                           Graph.__del__                 tensorjit/backends/cuda_driver.py:126-131,161-168
 *   tj_hip_last_error       CudaError message             tensorjit/backends/cuda_driver.py:22-23,54-72
 *   tj_hip_device_info      compute_capability()          tensorjit/backends/cuda_driver.py:75-76
 *   tj_hip_toolchain_version  the toolchain part of the   tensorjit/runtime/native.py:38-41,
 *                           reference's build-cache keys  tensorjit/backends/cuda_backend.py:474
 *   tj_hip_kernel_time      (no counterpart: hipEvent timing of one kernel of a program, used
 *                           by the autotuner and the benchmark)
 *   tj_hip_program_time_kernels  (no counterpart: one call of a program with a hipEvent between
 *                           its kernels, for per-kernel times in the program's own context)
 */
#ifndef TENSORJIT_HIP_H_
#define TENSORJIT_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TJ_HIP_ABI_VERSION 3

/* Where a kernel argument points: caller input i, arena + offset, caller output j. */
enum { TJ_ARG_INPUT = 0, TJ_ARG_ARENA = 1, TJ_ARG_OUTPUT = 2 };

typedef struct tj_argref {
  int32_t kind;   /* TJ_ARG_* */
  int32_t pad_;
  int64_t value;  /* input index, arena byte offset, or output index */
  int64_t bytes;  /* ARENA: size of the buffer at that offset (offset + bytes <= arena_bytes);
                     ignored for INPUT / OUTPUT */
} tj_argref;

typedef struct tj_launch {
  uint32_t grid[3];
  uint32_t block[3];
  uint32_t lds_bytes;  /* dynamic LDS */
  uint32_t nargs;      /* number of pointer arguments of this kernel */
} tj_launch;

typedef struct tj_stats {
  uint64_t calls;            /* run + replay calls */
  uint64_t graph_replays;
  uint64_t graph_captures;
  uint64_t host_ns;          /* host time spent inside run/replay (launch overhead) */
  uint64_t direct_fallbacks; /* replay calls that launched directly (pointer sets not recurring) */
} tj_stats;

typedef struct tj_device_info {
  int32_t cu_count;
  int32_t lds_per_block;
  int32_t warp_size;
  int32_t max_threads_per_block;
  int32_t clock_khz;
  int32_t mem_clock_khz;
  int32_t mem_bus_width;
  int32_t l2_bytes;
  int64_t total_mem;
  char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} tj_device_info;

int tj_hip_abi_version(void);
const char* tj_hip_last_error(void);
int tj_hip_device_info(int device, tj_device_info* out);

/* hipRTC version (hiprtcVersion) and HIP runtime version (hipRuntimeGetVersion), for
 * keying cached code objects by toolchain.  Needs no device. */
int tj_hip_toolchain_version(int* hiprtc_major, int* hiprtc_minor, int* hip_runtime);

/* hipRTC: source -> code object (malloc'ed; release with tj_hip_free). */
int tj_hip_compile(const char* source, const char* name, const char* const* opts, int nopts,
                   void** code, size_t* code_size);
void tj_hip_free(void* p);

/* Load the code object on `device`, resolve `nkernels` kernels, validate argument
 * references (args holds sum(launches[k].nargs) entries, kernel by kernel; every
 * ARENA reference must lie inside the arena: 0 < bytes and offset + bytes <=
 * arena_bytes) and allocate the arena with one hipMalloc. */
int tj_hip_program_create(int device, const void* code, size_t code_size, int nkernels,
                          const char* const* names, const tj_launch* launches, const tj_argref* args,
                          size_t arena_bytes, int n_inputs, int n_outputs, void** handle);

/* Launch every kernel in order on `stream` (a hipStream_t; NULL = default stream).
 * Asynchronous: never synchronises. */
int tj_hip_program_run(void* handle, const void* const* inputs, void* const* outputs, void* stream);

/* Allocation-free variant of tj_hip_program_run.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under stream capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The program's intermediates and
 * split-K partials go to a static device array of TJ_HIP_STATIC_ARENA_BYTES per GPU
 * instead of the program's own arena; a program whose arena is larger is rejected
 * with an error.  The call allocates nothing: tj_hip_program_create looks the
 * array's address up (once per device), so even a program's first call may be
 * issued under stream capture.  Every call on one GPU shares that array, which keeps
 * the last call's contents: calls that overlap on one GPU (two streams, two threads)
 * race.
 * Nothing in it needs clearing -- every call writes each intermediate before reading it. */
#define TJ_HIP_STATIC_ARENA_BYTES ((size_t)64 << 20)
int tj_hip_program_run_static(void* handle, const void* const* inputs, void* const* outputs, void* stream);

/* Capture the launch sequence for this input/output pointer set into a hipGraph exec
 * (kept in a small per-program cache keyed by the pointer set). */
int tj_hip_program_capture(void* handle, const void* const* inputs, void* const* outputs);

/* Replay the graph captured for this pointer set on `stream`, capturing it first if
 * this pointer set has not been seen.  After 4 captures in a row with no replay of a
 * cached exec (the caller keeps its outputs or passes fresh inputs), a pointer set is
 * captured on its second sighting only; calls in between launch the kernels directly
 * (counted in direct_fallbacks), so captures stay bounded. */
int tj_hip_program_replay(void* handle, const void* const* inputs, void* const* outputs, void* stream);

int tj_hip_program_stats(void* handle, tj_stats* out);
int tj_hip_program_arena(void* handle, void** ptr, size_t* bytes);

/* Average device time (ms) of kernel `k` launched `iters` times back to back on
 * `stream`, measured with hipEvents recorded on that stream (synchronises). */
int tj_hip_kernel_time(void* handle, int k, const void* const* inputs, void* const* outputs, void* stream,
                       int warmup, int iters, float* avg_ms);

/* One call of the program, launched exactly as tj_hip_program_run (own arena, same
 * order, `stream`), with a hipEvent recorded before the first kernel and after each
 * one; synchronises and writes each kernel's elapsed time (ms) to ms_per_kernel[k]
 * (one float per launch).  The kernels see the caches and clocks of the program's
 * own sequence, unlike repeated launches of one kernel. */
int tj_hip_program_time_kernels(void* handle, const void* const* inputs, void* const* outputs, void* stream,
                                float* ms_per_kernel);

int tj_hip_program_destroy(void* handle);

#ifdef __cplusplus
}
#endif

#endif /* TENSORJIT_HIP_H_ */
