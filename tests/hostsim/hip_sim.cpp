// A host-memory simulation of the HIP runtime calls that libjmodels_attn's host runtime
// (models_amd/csrc/jma_runtime.cpp) and the Python tools (models_amd/hip_runtime.py) make. Built
// as libamdhip64.so.7 with AddressSanitizer by tests/test_hostsim_cpu.py, so the library built
// against it (with tests/hostsim/launch_stubs.cpp in place of the kernels) and the Python drivers
// that load it run on a machine without a GPU.
//
// "Device" allocations are host heap blocks, tracked while live. Kernels never run: each launch
// stub names the device ranges its kernel would read or write, and the simulation checks every
// range against the live allocations when the launch executes, which for a launch recorded
// during stream capture is every replay of the graph. A range outside any live allocation (a
// buffer freed while a graph still names it, a buffer smaller than the launch assumes) is an
// error, counted and printed. Copies run as host memcpy (AddressSanitizer checks the host side);
// a memset recorded into a graph is an error too (the library never records one).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace {

std::mutex g_mu;
std::map<uintptr_t, size_t> g_live;  // base -> bytes
long g_errors = 0, g_launches = 0;

void error(const char* fmt, const char* a, const char* b = "") {
  ++g_errors;
  fprintf(stderr, "hipsim ERROR: ");
  fprintf(stderr, fmt, a, b);
  fprintf(stderr, "\n");
}

bool in_live(const void* p, size_t bytes) {
  const uintptr_t x = (uintptr_t)p;
  auto it = g_live.upper_bound(x);
  if (it == g_live.begin()) return false;
  --it;
  return x >= it->first && x + bytes <= it->first + it->second;
}

struct Op {
  enum Kind { kKernel, kCopy, kSet } kind;
  const char* name = "";
  void (*check)(void*) = nullptr;
  std::shared_ptr<void> arg;
  void* dst = nullptr;
  const void* src = nullptr;
  size_t bytes = 0;
  int value = 0;
  hipMemcpyKind copy_kind = hipMemcpyDefault;
};

void run_copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  if (bytes == 0) return;
  const bool d_dst = kind == hipMemcpyHostToDevice || kind == hipMemcpyDeviceToDevice;
  const bool d_src = kind == hipMemcpyDeviceToHost || kind == hipMemcpyDeviceToDevice;
  bool ok = true;
  {
    std::lock_guard<std::mutex> l(g_mu);
    if (d_dst && !in_live(dst, bytes)) {
      error("copy destination %s outside live device memory%s", "", "");
      ok = false;
    }
    if (d_src && !in_live(src, bytes)) {
      error("copy source %s outside live device memory%s", "", "");
      ok = false;
    }
  }
  if (ok) memcpy(dst, src, bytes);
}

void run_op(const Op& op) {
  switch (op.kind) {
    case Op::kKernel: {
      {
        std::lock_guard<std::mutex> l(g_mu);
        ++g_launches;
      }
      op.check(op.arg.get());
      break;
    }
    case Op::kCopy: run_copy(op.dst, op.src, op.bytes, op.copy_kind); break;
    case Op::kSet: {
      bool ok;
      {
        std::lock_guard<std::mutex> l(g_mu);
        ok = in_live(op.dst, op.bytes);
        if (!ok) error("memset %s outside live device memory%s", "", "");
      }
      if (ok) memset(op.dst, op.value, op.bytes);
      break;
    }
  }
}

// At exit: a summary line, and exit status 86 when any check failed.
struct Summary {
  Summary() {
    atexit([] {
      fprintf(stderr, "hipsim: %ld launches checked, %ld errors\n", g_launches, g_errors);
      fflush(stderr);
      if (g_errors > 0) _exit(86);
    });
  }
} g_summary;

}  // namespace

struct ihipStream_t {
  bool capturing = false;
  std::vector<Op> ops;
};
struct SimGraph {
  std::vector<Op> ops;
};
struct SimEvent {
  int recorded = 0;
};

extern "C" {

hipError_t hipMalloc(void** ptr, size_t size) {
  if (!ptr) return hipErrorInvalidValue;
  void* p = nullptr;
  if (posix_memalign(&p, 256, size ? size : 1) != 0) return hipErrorOutOfMemory;
  memset(p, 0x5A, size);  // device memory starts undefined; never zero by accident
  std::lock_guard<std::mutex> l(g_mu);
  g_live[(uintptr_t)p] = size ? size : 1;
  *ptr = p;
  return hipSuccess;
}

hipError_t hipFree(void* ptr) {
  if (!ptr) return hipSuccess;
  {
    std::lock_guard<std::mutex> l(g_mu);
    auto it = g_live.find((uintptr_t)ptr);
    if (it == g_live.end()) {
      error("hipFree of %s a pointer that is not a live allocation%s", "", "");
      return hipErrorInvalidValue;
    }
    g_live.erase(it);
  }
  free(ptr);
  return hipSuccess;
}

hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
  run_copy(dst, src, bytes, kind);
  return hipSuccess;
}

hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t s) {
  if (s && s->capturing) {
    Op op{Op::kCopy};
    op.dst = dst;
    op.src = src;
    op.bytes = bytes;
    op.copy_kind = kind;
    s->ops.push_back(op);
    return hipSuccess;
  }
  run_copy(dst, src, bytes, kind);
  return hipSuccess;
}

hipError_t hipMemset(void* dst, int value, size_t bytes) {
  Op op{Op::kSet};
  op.dst = dst;
  op.value = value;
  op.bytes = bytes;
  run_op(op);
  return hipSuccess;
}

hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t s) {
  if (s && s->capturing) {
    std::lock_guard<std::mutex> l(g_mu);
    error("hipMemsetAsync %s recorded into a graph%s", "", "");
    return hipErrorStreamCaptureUnsupported;
  }
  return hipMemset(dst, value, bytes);
}

hipError_t hipSetDevice(int device) { return device == 0 ? hipSuccess : hipErrorInvalidDevice; }

hipError_t hipGetDeviceCount(int* count) {
  *count = 1;
  return hipSuccess;
}

hipError_t hipGetDeviceProperties(hipDeviceProp_t* prop, int device) {
  if (device != 0) return hipErrorInvalidDevice;
  memset(prop, 0, sizeof(*prop));
  strcpy(prop->name, "host simulation");
  strcpy(prop->gcnArchName, "gfx950:sramecc+:xnack-");
  prop->totalGlobalMem = size_t(288) << 30;
  prop->multiProcessorCount = 256;
  return hipSuccess;
}

hipError_t hipStreamCreate(hipStream_t* stream) {
  *stream = new ihipStream_t();
  return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int) { return hipStreamCreate(stream); }

hipError_t hipStreamDestroy(hipStream_t stream) {
  delete stream;
  return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }

hipError_t hipStreamIsCapturing(hipStream_t s, hipStreamCaptureStatus* status) {
  *status = s && s->capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}

hipError_t hipStreamBeginCapture(hipStream_t s, int) {
  if (!s || s->capturing) return hipErrorInvalidValue;
  s->capturing = true;
  s->ops.clear();
  return hipSuccess;
}

hipError_t hipStreamEndCapture(hipStream_t s, void** graph) {
  if (!s || !s->capturing) return hipErrorInvalidValue;
  SimGraph* g = new SimGraph();
  g->ops.swap(s->ops);
  s->capturing = false;
  *graph = g;
  return hipSuccess;
}

hipError_t hipGraphInstantiate(void** exec, void* graph, void*, void*, size_t) {
  *exec = new SimGraph(*(SimGraph*)graph);
  return hipSuccess;
}

hipError_t hipGraphLaunch(void* exec, hipStream_t s) {
  if (s && s->capturing) return hipErrorStreamCaptureUnsupported;
  for (const Op& op : ((SimGraph*)exec)->ops) run_op(op);
  return hipSuccess;
}

hipError_t hipGraphExecDestroy(void* exec) {
  delete (SimGraph*)exec;
  return hipSuccess;
}

hipError_t hipGraphDestroy(void* graph) {
  delete (SimGraph*)graph;
  return hipSuccess;
}

hipError_t hipEventCreate(void** event) {
  *event = new SimEvent();
  return hipSuccess;
}
hipError_t hipEventDestroy(void* event) {
  delete (SimEvent*)event;
  return hipSuccess;
}
hipError_t hipEventRecord(void* event, hipStream_t) {
  ((SimEvent*)event)->recorded++;
  return hipSuccess;
}
hipError_t hipEventSynchronize(void*) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, void*, void*) {
  *ms = 0.001f;
  return hipSuccess;
}

const char* hipGetErrorString(hipError_t error) {
  switch (error) {
    case hipSuccess: return "hipSuccess";
    case hipErrorInvalidValue: return "hipErrorInvalidValue";
    case hipErrorOutOfMemory: return "hipErrorOutOfMemory";
    case hipErrorInvalidDevice: return "hipErrorInvalidDevice";
    case hipErrorStreamCaptureUnsupported: return "hipErrorStreamCaptureUnsupported";
    default: return "hipErrorUnknown";
  }
}

void hipsim_check_range(const void* p, size_t bytes, const char* what) {
  std::lock_guard<std::mutex> l(g_mu);
  if (bytes == 0) return;
  if (!p || !in_live(p, bytes)) {
    char size[64];
    snprintf(size, sizeof(size), " (%zu bytes)", bytes);
    error("launch range %s outside live device memory%s", what, size);
  }
}

void hipsim_fail(const char* what) {
  std::lock_guard<std::mutex> l(g_mu);
  error("launch stub check failed: %s", what);
}

hipError_t hipsim_launch(hipStream_t s, const char* kernel, void (*check)(void*), void* arg,
                         void (*drop)(void*)) {
  Op op{Op::kKernel};
  op.name = kernel;
  op.check = check;
  op.arg = std::shared_ptr<void>(arg, drop);
  if (s && s->capturing) {
    s->ops.push_back(op);
    return hipSuccess;
  }
  run_op(op);
  return hipSuccess;
}

long hipsim_errors(void) {
  std::lock_guard<std::mutex> l(g_mu);
  return g_errors;
}

long hipsim_launches(void) {
  std::lock_guard<std::mutex> l(g_mu);
  return g_launches;
}

}  // extern "C"
