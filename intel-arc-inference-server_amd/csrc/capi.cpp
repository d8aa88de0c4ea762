// capi.cpp - the host side of the C ABI that is not a kernel launch: error reporting,
// device memory and streams for callers that do not bring their own runtime, and
// event timing on a caller's stream.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "mi_capi_internal.h"

namespace {
thread_local std::string g_last;
}

int mi_fail(int code, const char* msg) {
  g_last = msg ? msg : "";
  return code;
}
int mi_hip(int e, const char* where) {
  if (e != 0) {
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s: %s (%d)", where, hipGetErrorString(static_cast<hipError_t>(e)), e);
    g_last = buf;
  }
  return e;
}

extern "C" {

const char* mi_last_error(void) { return g_last.c_str(); }

int mi_malloc(void** p, size_t bytes) {
  if (!p) return mi_fail(MI_ERR_ARG, "mi_malloc: null out pointer");
  return mi_hip(static_cast<int>(hipMalloc(p, bytes ? bytes : 1)), "hipMalloc");
}
int mi_free(void* p) { return mi_hip(static_cast<int>(hipFree(p)), "hipFree"); }
int mi_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  return mi_hip(static_cast<int>(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                                                static_cast<hipStream_t>(stream))),
                "hipMemcpyAsync h2d");
}
int mi_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  int e = static_cast<int>(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                                          static_cast<hipStream_t>(stream)));
  if (e == 0) e = static_cast<int>(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return mi_hip(e, "hipMemcpyAsync d2h");
}
int mi_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  return mi_hip(static_cast<int>(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                                static_cast<hipStream_t>(stream))),
                "hipMemcpyAsync d2d");
}
int mi_stream_sync(void* stream) {
  return mi_hip(static_cast<int>(hipStreamSynchronize(static_cast<hipStream_t>(stream))),
                "hipStreamSynchronize");
}
int mi_device_sync(void) { return mi_hip(static_cast<int>(hipDeviceSynchronize()), "hipDeviceSynchronize"); }

// Times `reps` replays of nothing but the caller's own enqueued work: record a start
// event, let the caller enqueue, then read the elapsed milliseconds.
int mi_event_create(void** ev) {
  hipEvent_t e;
  int r = static_cast<int>(hipEventCreate(&e));
  if (r == 0) *ev = e;
  return mi_hip(r, "hipEventCreate");
}
int mi_event_record(void* ev, void* stream) {
  return mi_hip(static_cast<int>(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream))),
                "hipEventRecord");
}
int mi_event_elapsed_ms(void* start, void* stop, float* ms) {
  int r = static_cast<int>(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  if (r == 0) r = static_cast<int>(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return mi_hip(r, "hipEventElapsedTime");
}
int mi_event_destroy(void* ev) { return mi_hip(static_cast<int>(hipEventDestroy(static_cast<hipEvent_t>(ev))), "hipEventDestroy"); }

}  // extern "C"

// server::accept_greedy (src/server/spec_accept.cc:81-85): accept d_i while it equals the
// verify argmax of the row before it; the next token is the argmax at the first mismatch.
extern "C" uint32_t mi_accept_greedy(const uint32_t* verify_argmax, const uint32_t* drafts, uint32_t k,
                                     uint32_t* next) {
  uint32_t j = 0;
  while (j < k && drafts[j] == verify_argmax[j]) ++j;
  if (next) *next = verify_argmax[j];
  return j;
}
