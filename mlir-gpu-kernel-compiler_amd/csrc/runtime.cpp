// tensorjit HIP executor (C ABI, declared in include/tensorjit_hip.h).
//
// A program is one hipRTC-built code object holding every kernel of a fused
// kernel program.  At creation each kernel argument is resolved to
//   INPUT  i   -> i-th caller input pointer
//   ARENA  off -> arena base + off   (intermediate placed by the memory planner)
//   OUTPUT j   -> j-th caller output pointer
// and validated, so a call only fills small pointer tables and issues one
// hipModuleLaunchKernel per kernel on the caller's stream.  The arena is a
// single hipMalloc owned by the program and reused by every call.  A call
// can instead replay a hipGraph exec captured for its exact pointer set;
// execs are cached per pointer set, so alternating output buffers (the
// caller's pool) replay without re-capture.  A caller whose pointer sets do
// not recur (it keeps every output, or passes fresh inputs) would pay a
// capture and an instantiation per call: after kMissLimit captures in a row
// with no replay of a cached exec, a pointer set is captured only on its
// second sighting, and calls in between launch directly.
//
// Design follows the reference's pybind11 executor (csrc/runtime.cpp:31-129:
// pre-resolved INPUT/ARENA/OUTPUT references, one call per program, bounds
// validation) moved onto the GPU, plus the module/launch/graph duties of its
// ctypes CUDA driver (tensorjit/backends/cuda_driver.py:79-168).
#include "../../include/tensorjit_hip.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <list>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

// Arena of tj_hip_program_run_static: file-scope device memory, so that entry point
// never allocates.  Every GPU the library runs on holds its own copy until the
// process ends.  Host code never uses this name as an address: the device address
// comes from hipGetSymbolAddress, once per device (static_arena below).
static __device__ __align__(256) char scratch[TJ_HIP_STATIC_ARENA_BYTES];

namespace {

thread_local std::string g_error;

int fail(const std::string& msg) {
  g_error = msg;
  return 1;
}

int hip_fail(hipError_t e, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return static_cast<int>(e) == 0 ? 1 : static_cast<int>(e);
}

#define TJ_HIP(call)                                 \
  do {                                               \
    hipError_t e_ = (call);                          \
    if (e_ != hipSuccess) return hip_fail(e_, #call); \
  } while (0)

constexpr int kMaxArgs = 64;
constexpr size_t kMaxGraphs = 8;
constexpr int kMissLimit = 4;        // captures in a row before pointer sets must recur
constexpr size_t kMaxSightings = 8;  // pointer sets seen once since then, most recent first

struct KernelRec {
  hipFunction_t fn = nullptr;
  std::string name;
  tj_launch launch{};
  std::vector<tj_argref> refs;
  // per-launch argument storage: values[i] holds the pointer, params[i] points at values[i]
  std::vector<void*> values;
  std::vector<void*> params;
};

struct GraphRec {
  std::vector<const void*> key;  // inputs then outputs
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

// Restores the calling thread's current device on scope exit.
class DeviceScope {
 public:
  explicit DeviceScope(int dev) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != dev) (void)hipSetDevice(dev);
  }
  ~DeviceScope() {
    int cur = -1;
    if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1;
};

struct Program {
  int device = 0;
  hipModule_t module = nullptr;
  std::vector<KernelRec> kernels;
  char* arena = nullptr;
  size_t arena_bytes = 0;
  int n_in = 0, n_out = 0;
  hipStream_t capture_stream = nullptr;
  std::list<GraphRec> graphs;  // most recently used first
  int miss_streak = 0;         // captures since the last replay of a cached exec
  std::list<std::vector<const void*>> sightings;
  // device address of the static arena for tj_hip_program_run_static, looked up at
  // creation (null when the arena does not fit it or the lookup failed: static_error)
  char* static_base = nullptr;
  std::string static_error;
  tj_stats stats{};

  ~Program() {
    DeviceScope scope(device);
    for (GraphRec& g : graphs) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      if (g.graph) (void)hipGraphDestroy(g.graph);
    }
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
    if (arena) (void)hipFree(arena);
    if (module) (void)hipModuleUnload(module);
  }

  // Fill every kernel's pointer table; `base` is the arena the ARENA offsets refer to
  // (the program's own, or the static one of tj_hip_program_run_static).
  void bind(const void* const* in, void* const* out, char* base) {
    for (KernelRec& k : kernels) {
      for (size_t i = 0; i < k.refs.size(); ++i) {
        const tj_argref& r = k.refs[i];
        switch (r.kind) {
          case TJ_ARG_INPUT: k.values[i] = const_cast<void*>(in[r.value]); break;
          case TJ_ARG_ARENA: k.values[i] = base + r.value; break;
          default: k.values[i] = out[r.value]; break;
        }
      }
    }
  }

  int launch_one(KernelRec& k, hipStream_t stream) {
    const tj_launch& l = k.launch;
    if (k.values.empty()) {
      TJ_HIP(hipModuleLaunchKernel(k.fn, l.grid[0], l.grid[1], l.grid[2], l.block[0], l.block[1], l.block[2],
                                   l.lds_bytes, stream, k.params.data(), nullptr));
      return 0;
    }
    // every kernel argument is a pointer, so values[] already is the packed argument
    // buffer: handed over whole, HIP copies it instead of walking the kernel's argument
    // list per parameter
    size_t bytes = k.values.size() * sizeof(void*);
    void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, k.values.data(), HIP_LAUNCH_PARAM_BUFFER_SIZE, &bytes,
                     HIP_LAUNCH_PARAM_END};
    TJ_HIP(hipModuleLaunchKernel(k.fn, l.grid[0], l.grid[1], l.grid[2], l.block[0], l.block[1], l.block[2],
                                 l.lds_bytes, stream, nullptr, extra));
    return 0;
  }

  int launch_all(hipStream_t stream) {
    for (KernelRec& k : kernels) {
      int rc = launch_one(k, stream);
      if (rc) return fail(g_error + " [kernel " + k.name + "]");
    }
    return 0;
  }

  std::vector<const void*> key_of(const void* const* in, void* const* out) const {
    std::vector<const void*> key;
    key.reserve(n_in + n_out);
    for (int i = 0; i < n_in; ++i) key.push_back(in[i]);
    for (int j = 0; j < n_out; ++j) key.push_back(out[j]);
    return key;
  }

  GraphRec* find(const std::vector<const void*>& key) {
    for (auto it = graphs.begin(); it != graphs.end(); ++it) {
      if (it->key == key) {
        graphs.splice(graphs.begin(), graphs, it);
        return &graphs.front();
      }
    }
    return nullptr;
  }

  // True when `key` was seen once before (and forgets it); otherwise remembers it.
  bool seen_before(const std::vector<const void*>& key) {
    for (auto it = sightings.begin(); it != sightings.end(); ++it) {
      if (*it == key) {
        sightings.erase(it);
        return true;
      }
    }
    sightings.push_front(key);
    if (sightings.size() > kMaxSightings) sightings.pop_back();
    return false;
  }

  // The exec for this pointer set, captured now if needed; *rec_out stays null when the
  // miss policy says to launch directly instead (only when `may_skip`).
  int capture(const void* const* in, void* const* out, GraphRec** rec_out, bool may_skip = false) {
    *rec_out = nullptr;
    std::vector<const void*> key = key_of(in, out);
    if (GraphRec* hit = find(key)) {
      miss_streak = 0;
      *rec_out = hit;
      return 0;
    }
    if (may_skip) {
      if (miss_streak >= kMissLimit && !seen_before(key)) return 0;
      miss_streak++;
    }
    if (!capture_stream) TJ_HIP(hipStreamCreateWithFlags(&capture_stream, hipStreamNonBlocking));
    bind(in, out, arena);
    GraphRec rec;
    rec.key = std::move(key);
    TJ_HIP(hipStreamBeginCapture(capture_stream, hipStreamCaptureModeThreadLocal));
    int rc = launch_all(capture_stream);
    hipError_t end = hipStreamEndCapture(capture_stream, &rec.graph);
    if (rc) {
      if (rec.graph) (void)hipGraphDestroy(rec.graph);
      return rc;
    }
    if (end != hipSuccess) return hip_fail(end, "hipStreamEndCapture");
    hipError_t inst = hipGraphInstantiate(&rec.exec, rec.graph, nullptr, nullptr, 0);
    if (inst != hipSuccess) {
      (void)hipGraphDestroy(rec.graph);
      return hip_fail(inst, "hipGraphInstantiate");
    }
    graphs.push_front(std::move(rec));
    while (graphs.size() > kMaxGraphs) {
      GraphRec& old = graphs.back();
      (void)hipGraphExecDestroy(old.exec);
      (void)hipGraphDestroy(old.graph);
      graphs.pop_back();
    }
    stats.graph_captures++;
    *rec_out = &graphs.front();
    return 0;
  }
};

Program* as_program(void* h) { return static_cast<Program*>(h); }

constexpr int kMaxDevices = 64;
std::mutex g_static_mu;
std::atomic<char*> g_static_arena[kMaxDevices];

// Device address of `scratch` on `device`, which must be the current device; looked up
// with hipGetSymbolAddress the first time a program is created on that device, and kept.
int static_arena(int device, char** out) {
  if (device < 0 || device >= kMaxDevices) return fail("static arena: device index out of range");
  char* ptr = g_static_arena[device].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_static_mu);
    ptr = g_static_arena[device].load(std::memory_order_relaxed);
    if (!ptr) {
      void* addr = nullptr;
      hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      if (!addr) return fail("hipGetSymbolAddress(scratch) returned a null address");
      ptr = static_cast<char*>(addr);
      g_static_arena[device].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return 0;
}

uint64_t now_ns() {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace

extern "C" {

int tj_hip_abi_version(void) { return TJ_HIP_ABI_VERSION; }

const char* tj_hip_last_error(void) { return g_error.c_str(); }

int tj_hip_device_info(int device, tj_device_info* out) {
  if (!out) return fail("tj_hip_device_info: null output");
  hipDeviceProp_t p;
  TJ_HIP(hipGetDeviceProperties(&p, device));
  std::memset(out, 0, sizeof(*out));
  out->cu_count = p.multiProcessorCount;
  out->lds_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
  out->warp_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->clock_khz = p.clockRate;
  out->mem_clock_khz = p.memoryClockRate;
  out->mem_bus_width = p.memoryBusWidth;
  out->l2_bytes = p.l2CacheSize;
  out->total_mem = static_cast<int64_t>(p.totalGlobalMem);
  std::snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
  return 0;
}

int tj_hip_toolchain_version(int* hiprtc_major, int* hiprtc_minor, int* hip_runtime) {
  if (!hiprtc_major || !hiprtc_minor || !hip_runtime) return fail("tj_hip_toolchain_version: null argument");
  hiprtcResult r = hiprtcVersion(hiprtc_major, hiprtc_minor);
  if (r != HIPRTC_SUCCESS) return fail(std::string("hiprtcVersion: ") + hiprtcGetErrorString(r));
  TJ_HIP(hipRuntimeGetVersion(hip_runtime));
  return 0;
}

int tj_hip_compile(const char* source, const char* name, const char* const* opts, int nopts, void** code,
                   size_t* code_size) {
  if (!source || !code || !code_size) return fail("tj_hip_compile: null argument");
  *code = nullptr;
  *code_size = 0;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "tensorjit.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, nopts, const_cast<const char**>(opts));
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return fail(std::string("hipRTC compile failed (") + hiprtcGetErrorString(r) + "):\n" + log);
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  if (r != HIPRTC_SUCCESS || n == 0) {
    hiprtcDestroyProgram(&prog);
    return fail("hiprtcGetCodeSize failed");
  }
  void* buf = std::malloc(n);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return fail("out of host memory for code object");
  }
  r = hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    std::free(buf);
    return fail(std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
  }
  *code = buf;
  *code_size = n;
  return 0;
}

void tj_hip_free(void* p) { std::free(p); }

int tj_hip_program_create(int device, const void* code, size_t code_size, int nkernels, const char* const* names,
                          const tj_launch* launches, const tj_argref* args, size_t arena_bytes, int n_inputs,
                          int n_outputs, void** handle) {
  if (!handle) return fail("tj_hip_program_create: null handle");
  *handle = nullptr;
  if (!code || code_size == 0) return fail("tj_hip_program_create: empty code object");
  if (nkernels < 0 || (nkernels > 0 && (!names || !launches))) return fail("tj_hip_program_create: bad kernel table");
  if (n_inputs < 0 || n_outputs < 0) return fail("tj_hip_program_create: negative input/output count");
  std::unique_ptr<Program> p(new Program());
  p->device = device;
  p->n_in = n_inputs;
  p->n_out = n_outputs;
  p->arena_bytes = arena_bytes;
  // 1. validate the whole launch and argument table (no device work yet)
  size_t pos = 0;
  for (int k = 0; k < nkernels; ++k) {
    KernelRec rec;
    if (!names[k]) return fail("tj_hip_program_create: null kernel name");
    rec.name = names[k];
    rec.launch = launches[k];
    const tj_launch& l = rec.launch;
    if (l.nargs > static_cast<uint32_t>(kMaxArgs)) return fail("too many kernel arguments in " + rec.name);
    if (!l.grid[0] || !l.grid[1] || !l.grid[2] || !l.block[0] || !l.block[1] || !l.block[2])
      return fail("zero-sized launch for " + rec.name);
    if (static_cast<uint64_t>(l.block[0]) * l.block[1] * l.block[2] > 1024) return fail("block too large for " + rec.name);
    if (l.lds_bytes > 160u * 1024u) return fail("dynamic LDS over 160 KiB for " + rec.name);
    if (l.nargs && !args) return fail("tj_hip_program_create: null argument table");
    for (uint32_t i = 0; i < l.nargs; ++i) {
      const tj_argref& a = args[pos++];
      if (a.kind == TJ_ARG_INPUT) {
        if (a.value < 0 || a.value >= n_inputs) return fail("input index out of range in " + rec.name);
      } else if (a.kind == TJ_ARG_OUTPUT) {
        if (a.value < 0 || a.value >= n_outputs) return fail("output index out of range in " + rec.name);
      } else if (a.kind == TJ_ARG_ARENA) {
        // the whole buffer, not just its first byte, must lie inside the arena
        if (a.value < 0 || a.bytes <= 0 || static_cast<uint64_t>(a.value) > arena_bytes ||
            static_cast<uint64_t>(a.bytes) > arena_bytes - static_cast<uint64_t>(a.value))
          return fail("arena buffer [" + std::to_string(a.value) + ", +" + std::to_string(a.bytes) +
                      ") outside the " + std::to_string(arena_bytes) + "-byte arena in " + rec.name);
      } else {
        return fail("bad argument kind in " + rec.name);
      }
      rec.refs.push_back(a);
    }
    rec.values.assign(rec.refs.size(), nullptr);
    rec.params.resize(rec.refs.size());
    p->kernels.push_back(std::move(rec));
  }
  for (KernelRec& k : p->kernels)
    for (size_t i = 0; i < k.values.size(); ++i) k.params[i] = &k.values[i];
  // 2. load the code object, resolve the kernels, allocate the arena
  DeviceScope scope(device);
  TJ_HIP(hipModuleLoadData(&p->module, code));
  for (KernelRec& k : p->kernels) {
    hipError_t e = hipModuleGetFunction(&k.fn, p->module, k.name.c_str());
    if (e != hipSuccess) return hip_fail(e, ("hipModuleGetFunction " + k.name).c_str());
  }
  if (arena_bytes) {
    void* a = nullptr;
    TJ_HIP(hipMalloc(&a, arena_bytes));
    p->arena = static_cast<char*>(a);
  }
  // tj_hip_program_run_static's arena: looked up here, where loading and allocating are
  // expected, so that entry point never makes the runtime load or place anything.  A
  // failed lookup leaves the program usable through the other entry points.
  if (arena_bytes && arena_bytes <= TJ_HIP_STATIC_ARENA_BYTES) {
    const std::string saved = g_error;
    if (static_arena(device, &p->static_base) != 0) {
      p->static_error = g_error;
      p->static_base = nullptr;
      g_error = saved;
    }
  }
  *handle = p.release();
  return 0;
}

int tj_hip_program_run(void* handle, const void* const* inputs, void* const* outputs, void* stream) {
  Program* p = as_program(handle);
  if (!p) return fail("tj_hip_program_run: null program");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_program_run: null pointer table");
  const uint64_t t0 = now_ns();
  DeviceScope scope(p->device);
  p->bind(inputs, outputs, p->arena);
  int rc = p->launch_all(static_cast<hipStream_t>(stream));
  if (rc) return rc;
  p->stats.calls++;
  p->stats.host_ns += now_ns() - t0;
  return 0;
}

int tj_hip_program_run_static(void* handle, const void* const* inputs, void* const* outputs, void* stream) {
  Program* p = as_program(handle);
  if (!p) return fail("tj_hip_program_run_static: null program");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_program_run_static: null pointer table");
  if (p->arena_bytes > TJ_HIP_STATIC_ARENA_BYTES)
    return fail("tj_hip_program_run_static: the program's intermediates need " + std::to_string(p->arena_bytes) +
                " bytes, more than the " + std::to_string(static_cast<size_t>(TJ_HIP_STATIC_ARENA_BYTES)) +
                "-byte static arena (use tj_hip_program_run)");
  if (p->arena_bytes && !p->static_base)
    return fail("tj_hip_program_run_static: no static arena on device " + std::to_string(p->device) + ": " +
                p->static_error);
  const uint64_t t0 = now_ns();
  DeviceScope scope(p->device);
  p->bind(inputs, outputs, p->static_base);
  int rc = p->launch_all(static_cast<hipStream_t>(stream));
  if (rc) return rc;
  p->stats.calls++;
  p->stats.host_ns += now_ns() - t0;
  return 0;
}

int tj_hip_program_capture(void* handle, const void* const* inputs, void* const* outputs) {
  Program* p = as_program(handle);
  if (!p) return fail("tj_hip_program_capture: null program");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_program_capture: null pointer table");
  DeviceScope scope(p->device);
  GraphRec* rec = nullptr;
  return p->capture(inputs, outputs, &rec);
}

int tj_hip_program_replay(void* handle, const void* const* inputs, void* const* outputs, void* stream) {
  Program* p = as_program(handle);
  if (!p) return fail("tj_hip_program_replay: null program");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_program_replay: null pointer table");
  const uint64_t t0 = now_ns();
  DeviceScope scope(p->device);
  GraphRec* rec = nullptr;
  int rc = p->capture(inputs, outputs, &rec, /*may_skip=*/true);
  if (rc) return rc;
  if (rec) {
    TJ_HIP(hipGraphLaunch(rec->exec, static_cast<hipStream_t>(stream)));
    p->stats.graph_replays++;
  } else {
    p->bind(inputs, outputs, p->arena);
    rc = p->launch_all(static_cast<hipStream_t>(stream));
    if (rc) return rc;
    p->stats.direct_fallbacks++;
  }
  p->stats.calls++;
  p->stats.host_ns += now_ns() - t0;
  return 0;
}

int tj_hip_program_stats(void* handle, tj_stats* out) {
  Program* p = as_program(handle);
  if (!p || !out) return fail("tj_hip_program_stats: null argument");
  *out = p->stats;
  return 0;
}

int tj_hip_program_arena(void* handle, void** ptr, size_t* bytes) {
  Program* p = as_program(handle);
  if (!p || !ptr || !bytes) return fail("tj_hip_program_arena: null argument");
  *ptr = p->arena;
  *bytes = p->arena_bytes;
  return 0;
}

int tj_hip_kernel_time(void* handle, int k, const void* const* inputs, void* const* outputs, void* stream,
                       int warmup, int iters, float* avg_ms) {
  Program* p = as_program(handle);
  if (!p || !avg_ms) return fail("tj_hip_kernel_time: null argument");
  if (k < 0 || k >= static_cast<int>(p->kernels.size())) return fail("tj_hip_kernel_time: kernel index out of range");
  if (iters <= 0 || warmup < 0) return fail("tj_hip_kernel_time: iters must be positive");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_kernel_time: null pointer table");
  DeviceScope scope(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  p->bind(inputs, outputs, p->arena);
  KernelRec& kr = p->kernels[k];
  for (int i = 0; i < warmup; ++i)
    if (int rc = p->launch_one(kr, s)) return rc;
  hipEvent_t start, stop;
  TJ_HIP(hipEventCreate(&start));
  hipError_t e = hipEventCreate(&stop);
  if (e != hipSuccess) {
    (void)hipEventDestroy(start);
    return hip_fail(e, "hipEventCreate");
  }
  int rc = 0;
  e = hipEventRecord(start, s);
  for (int i = 0; e == hipSuccess && rc == 0 && i < iters; ++i) rc = p->launch_one(kr, s);
  if (e == hipSuccess && rc == 0) e = hipEventRecord(stop, s);
  if (e == hipSuccess && rc == 0) e = hipEventSynchronize(stop);
  float ms = 0.f;
  if (e == hipSuccess && rc == 0) e = hipEventElapsedTime(&ms, start, stop);
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "tj_hip_kernel_time events");
  *avg_ms = ms / iters;
  return 0;
}

int tj_hip_program_time_kernels(void* handle, const void* const* inputs, void* const* outputs, void* stream,
                                float* ms_per_kernel) {
  Program* p = as_program(handle);
  if (!p || !ms_per_kernel) return fail("tj_hip_program_time_kernels: null argument");
  if ((p->n_in && !inputs) || (p->n_out && !outputs)) return fail("tj_hip_program_time_kernels: null pointer table");
  const size_t n = p->kernels.size();
  if (n == 0) return 0;
  DeviceScope scope(p->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::vector<hipEvent_t> ev(n + 1, nullptr);
  hipError_t e = hipSuccess;
  for (size_t i = 0; i <= n && e == hipSuccess; ++i) e = hipEventCreate(&ev[i]);
  int rc = 0;
  if (e == hipSuccess) {
    p->bind(inputs, outputs, p->arena);
    e = hipEventRecord(ev[0], s);
    for (size_t k = 0; k < n && e == hipSuccess && rc == 0; ++k) {
      rc = p->launch_one(p->kernels[k], s);
      if (rc == 0) e = hipEventRecord(ev[k + 1], s);
    }
    if (e == hipSuccess && rc == 0) e = hipEventSynchronize(ev[n]);
    for (size_t k = 0; k < n && e == hipSuccess && rc == 0; ++k) e = hipEventElapsedTime(&ms_per_kernel[k], ev[k], ev[k + 1]);
  }
  for (hipEvent_t x : ev)
    if (x) (void)hipEventDestroy(x);
  if (rc) return rc;
  if (e != hipSuccess) return hip_fail(e, "tj_hip_program_time_kernels events");
  p->stats.calls++;
  return 0;
}

int tj_hip_program_destroy(void* handle) {
  delete as_program(handle);
  return 0;
}

}  // extern "C"
