// Host-only stand-in for the few HIP runtime pieces libmxq's host C++
// (mxq_api.cpp, mxq_safetensors.cpp) uses, so that code builds with g++ under
// AddressSanitizer / UndefinedBehaviorSanitizer on a machine without a GPU.
// "Device" memory is ordinary host memory in this build: copies are memcpy,
// pinned buffers are malloc, streams and events complete immediately. Test
// infrastructure only (tests/test_sanitize.py); never part of libmxq.
#pragma once

#include <cstddef>
#include <cstdlib>
#include <cstring>

#define __host__
#define __device__
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))

typedef int hipError_t;
enum : int { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2,
             hipErrorNotSupported = 801 };
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice = 1,
                     hipMemcpyDeviceToHost = 2 };
#define hipHostMallocDefault 0u
#define hipEventDisableTiming 2u

inline const char* hipGetErrorString(hipError_t) { return "host-only build"; }
inline hipError_t hipHostMalloc(void** p, size_t n, unsigned) {
  *p = std::malloc(n);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipHostFree(void* p) {
  std::free(p);
  return hipSuccess;
}
inline hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind,
                                 hipStream_t) {
  std::memcpy(dst, src, n);
  return hipSuccess;
}
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamCreate(hipStream_t* s) {
  *s = reinterpret_cast<hipStream_t>(std::malloc(1));
  return *s ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipStreamDestroy(hipStream_t s) {
  std::free(s);
  return hipSuccess;
}
inline hipError_t hipMalloc(void** p, size_t n) {
  *p = std::malloc(n);
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipFree(void* p) {
  std::free(p);
  return hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) {
  *e = reinterpret_cast<hipEvent_t>(std::malloc(1));
  return *e ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipEventDestroy(hipEvent_t e) {
  std::free(e);
  return hipSuccess;
}
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipGetDevice(int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipStreamGetDevice(hipStream_t, int* d) {
  *d = 0;
  return hipSuccess;
}
inline hipError_t hipGetLastError() { return hipSuccess; }
// stream-ordered allocation from a pool: host memory here, refused above 64 MiB so the
// fallback to the in-place kernel is exercised too
typedef struct ihipMemPool_t* hipMemPool_t;
enum hipMemAllocationType { hipMemAllocationTypeInvalid = 0, hipMemAllocationTypePinned = 1 };
enum hipMemAllocationHandleType { hipMemHandleTypeNone = 0 };
enum hipMemLocationType { hipMemLocationTypeInvalid = 0, hipMemLocationTypeDevice = 1 };
struct hipMemLocation { hipMemLocationType type; int id; };
struct hipMemPoolProps {
  hipMemAllocationType allocType;
  hipMemAllocationHandleType handleTypes;
  hipMemLocation location;
  void* win32SecurityAttributes;
  size_t maxSize;
  unsigned char reserved[56];
};
enum hipMemPoolAttr { hipMemPoolAttrReleaseThreshold = 4 };
enum hipDeviceAttribute_t { hipDeviceAttributeMemoryPoolsSupported = 1 };
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  *v = 1;
  return hipSuccess;
}
inline hipError_t hipMemPoolCreate(hipMemPool_t* p, const hipMemPoolProps*) {
  *p = reinterpret_cast<hipMemPool_t>(std::malloc(1));
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipMemPoolSetAttribute(hipMemPool_t, hipMemPoolAttr, void*) {
  return hipSuccess;
}
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* c) {
  *c = hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipMallocFromPoolAsync(void** p, size_t n, hipMemPool_t, hipStream_t) {
  *p = n <= (size_t(64) << 20) ? std::malloc(n) : nullptr;
  return *p ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipFreeAsync(void* p, hipStream_t) {
  std::free(p);
  return hipSuccess;
}
template <typename T>
inline hipError_t hipGetSymbolAddress(void** p, const T* symbol) {
  *p = const_cast<void*>(static_cast<const void*>(symbol));
  return hipSuccess;
}
