// Host-only stand-in for <hip/hip_runtime.h>, used to build the library's host runtime
// (models_amd/csrc/jma_runtime.cpp) with g++ and AddressSanitizer for tests/test_hostsim_cpu.py.
// It declares the part of the HIP runtime API the runtime and tests/hostsim/hip_sim.cpp use;
// hip_sim.cpp implements it on host memory. Not a HIP implementation: kernels never run.
#pragma once

#include <stddef.h>
#include <stdint.h>

#define __host__
#define __device__

typedef enum hipError_t {
  hipSuccess = 0,
  hipErrorInvalidValue = 1,
  hipErrorOutOfMemory = 2,
  hipErrorInvalidDevice = 101,
  hipErrorInvalidResourceHandle = 400,
  hipErrorStreamCaptureUnsupported = 900,
  hipErrorUnknown = 999,
} hipError_t;

typedef enum hipMemcpyKind {
  hipMemcpyHostToHost = 0,
  hipMemcpyHostToDevice = 1,
  hipMemcpyDeviceToHost = 2,
  hipMemcpyDeviceToDevice = 3,
  hipMemcpyDefault = 4,
} hipMemcpyKind;

typedef enum hipStreamCaptureStatus {
  hipStreamCaptureStatusNone = 0,
  hipStreamCaptureStatusActive = 1,
  hipStreamCaptureStatusInvalidated = 2,
} hipStreamCaptureStatus;

#define hipStreamNonBlocking 0x01

typedef struct ihipStream_t* hipStream_t;

typedef struct hipDeviceProp_t {
  char name[256];
  char gcnArchName[256];
  size_t totalGlobalMem;
  int multiProcessorCount;
} hipDeviceProp_t;

extern "C" {
hipError_t hipMalloc(void** ptr, size_t size);
hipError_t hipFree(void* ptr);
hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t stream);
hipError_t hipMemset(void* dst, int value, size_t bytes);
hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t stream);
hipError_t hipSetDevice(int device);
hipError_t hipGetDeviceCount(int* count);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* prop, int device);
hipError_t hipStreamCreate(hipStream_t* stream);
hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int flags);
hipError_t hipStreamDestroy(hipStream_t stream);
hipError_t hipStreamSynchronize(hipStream_t stream);
hipError_t hipStreamIsCapturing(hipStream_t stream, hipStreamCaptureStatus* status);
hipError_t hipDeviceSynchronize(void);
const char* hipGetErrorString(hipError_t error);

// Not HIP: the simulation's own entry points for the kernel-launch stubs.
// hipsim_check_range: [p, p + bytes) must lie inside one live allocation (an error is recorded and
// printed otherwise). hipsim_launch: runs `check(arg)` now, or records it into the stream's capture
// so that every replay of the graph runs it; `drop(arg)` frees arg with the last graph using it.
void hipsim_check_range(const void* p, size_t bytes, const char* what);
// hipsim_fail: records (and prints) an error found by a launch stub's own check.
void hipsim_fail(const char* what);
hipError_t hipsim_launch(hipStream_t stream, const char* kernel, void (*check)(void*), void* arg,
                         void (*drop)(void*));
long hipsim_errors(void);
long hipsim_launches(void);
}

// HIP's typed overload (hip_runtime_api.h offers the same for C++ callers).
template <class T>
inline hipError_t hipMalloc(T** ptr, size_t size) {
  return hipMalloc((void**)ptr, size);
}
