// Device, stream, event, pinned-memory and copy entry points over the HIP
// runtime: the MI355X rewrite of the CUDA runtime FFI in
// turbo_src/cuda_ffi.rs:26-69 (there declared by hand and linked against
// libcudart; here taken from <hip/hip_runtime.h>).
//
// Streams are created non-blocking at the default priority. The reference
// asks for a high-priority copy stream (src/stagehand/config.py:28,
// src/stagehand/transfer.py:95-98); streams of different priorities have hung
// on this platform, so every stream this library creates uses the default.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "sh_internal.h"
#include "stagehand_native.h"

namespace {
thread_local char g_last_error[1024] = {0};
}

namespace sh {

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace sh

extern "C" const char* sh_last_error(void) { return g_last_error; }

extern "C" int sh_abi_version(void) { return SH_ABI_VERSION; }

extern "C" int sh_device_count(int* count) {
  sh::clear_error();
  if (count == nullptr) return sh::fail(SH_ERR_INVALID, "sh_device_count: count is NULL");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return SH_OK;
  }
  SH_HIP(e);
  return SH_OK;
}

extern "C" int sh_set_device(int device) {
  sh::clear_error();
  SH_HIP(hipSetDevice(device));
  return SH_OK;
}

extern "C" int sh_get_device(int* device) {
  sh::clear_error();
  if (device == nullptr) return sh::fail(SH_ERR_INVALID, "sh_get_device: device is NULL");
  SH_HIP(hipGetDevice(device));
  return SH_OK;
}

extern "C" int sh_host_alloc(size_t bytes, void** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_host_alloc: out is NULL");
  *out = nullptr;
  if (bytes == 0) return sh::fail(SH_ERR_INVALID, "sh_host_alloc: zero-byte request");
  hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return sh::fail(SH_ERR_OOM, "sh_host_alloc: could not pin %zu bytes (HIP error %d)", bytes, (int)e);
  SH_HIP(e);
  return SH_OK;
}

extern "C" int sh_host_free(void* ptr) {
  sh::clear_error();
  if (ptr == nullptr) return SH_OK;
  SH_HIP(hipHostFree(ptr));
  return SH_OK;
}

extern "C" int sh_stream_create(void** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_stream_create: out is NULL");
  hipStream_t s = nullptr;
  SH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = (void*)s;
  return SH_OK;
}

extern "C" int sh_stream_destroy(void* stream) {
  sh::clear_error();
  if (stream == nullptr) return SH_OK;
  SH_HIP(hipStreamDestroy((hipStream_t)stream));
  return SH_OK;
}

extern "C" int sh_stream_sync(void* stream) {
  sh::clear_error();
  SH_HIP(hipStreamSynchronize((hipStream_t)stream));
  return SH_OK;
}

extern "C" int sh_stream_wait_event(void* stream, void* event) {
  sh::clear_error();
  if (event == nullptr) return sh::fail(SH_ERR_INVALID, "sh_stream_wait_event: event is NULL");
  SH_HIP(hipStreamWaitEvent((hipStream_t)stream, (hipEvent_t)event, 0));
  return SH_OK;
}

extern "C" int sh_event_create(int timing, void** out) {
  sh::clear_error();
  if (out == nullptr) return sh::fail(SH_ERR_INVALID, "sh_event_create: out is NULL");
  hipEvent_t ev = nullptr;
  SH_HIP(hipEventCreateWithFlags(&ev, timing ? hipEventDefault : hipEventDisableTiming));
  *out = (void*)ev;
  return SH_OK;
}

extern "C" int sh_event_destroy(void* event) {
  sh::clear_error();
  if (event == nullptr) return SH_OK;
  SH_HIP(hipEventDestroy((hipEvent_t)event));
  return SH_OK;
}

extern "C" int sh_event_record(void* event, void* stream) {
  sh::clear_error();
  if (event == nullptr) return sh::fail(SH_ERR_INVALID, "sh_event_record: event is NULL");
  SH_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
  return SH_OK;
}

extern "C" int sh_event_query(void* event) {
  sh::clear_error();
  if (event == nullptr) return sh::fail(SH_ERR_INVALID, "sh_event_query: event is NULL");
  hipError_t e = hipEventQuery((hipEvent_t)event);
  if (e == hipErrorNotReady) return SH_ERR_NOT_READY;
  SH_HIP(e);
  return SH_OK;
}

extern "C" int sh_event_sync(void* event) {
  sh::clear_error();
  if (event == nullptr) return sh::fail(SH_ERR_INVALID, "sh_event_sync: event is NULL");
  SH_HIP(hipEventSynchronize((hipEvent_t)event));
  return SH_OK;
}

extern "C" int sh_event_elapsed_ms(void* start, void* end, float* ms) {
  sh::clear_error();
  if (start == nullptr || end == nullptr || ms == nullptr)
    return sh::fail(SH_ERR_INVALID, "sh_event_elapsed_ms: NULL argument");
  SH_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
  return SH_OK;
}

namespace {
int copy_async(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, void* stream, const char* who) {
  sh::clear_error();
  if (bytes == 0) return SH_OK;
  if (dst == nullptr || src == nullptr) return sh::fail(SH_ERR_INVALID, "%s: NULL pointer", who);
  SH_HIP(hipMemcpyAsync(dst, src, bytes, kind, (hipStream_t)stream));
  return SH_OK;
}
}  // namespace

extern "C" int sh_memcpy_h2d_async(void* dst_dev, const void* src_host, size_t bytes, void* stream) {
  return copy_async(dst_dev, src_host, bytes, hipMemcpyHostToDevice, stream, "sh_memcpy_h2d_async");
}

extern "C" int sh_memcpy_d2h_async(void* dst_host, const void* src_dev, size_t bytes, void* stream) {
  return copy_async(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, stream, "sh_memcpy_d2h_async");
}

extern "C" int sh_memcpy_d2d_async(void* dst_dev, const void* src_dev, size_t bytes, void* stream) {
  return copy_async(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, stream, "sh_memcpy_d2d_async");
}
