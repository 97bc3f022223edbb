// Core of the libaneforge_hip C ABI: error reporting, device facts, stream/graph helpers.
//
// Error convention (replaces the reference's int rc / NULL-handle + stderr convention,
// aneforge/_lib/ane_e5rt_dispatch.mm:528-713): every entry point returns 0 on success and
// a negative code on failure; afx_last_error() returns the calling thread's message.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include "afx_common.h"

namespace {
thread_local char g_err[1024] = "";
}

namespace afx {
int set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return -1;
}
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}
}  // namespace afx

extern "C" {

const char* afx_last_error(void) { return g_err; }

int afx_abi_version(void) { return 2; }

// Device facts the host planner uses (CU count for grid sizing, LDS and L2 sizes).
int afx_device_info(int device, int* cu_count, int* lds_bytes, int* l2_bytes, int* gcn_arch) {
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, device);
  if (e != hipSuccess) return afx::set_error("hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (lds_bytes) *lds_bytes = (int)p.sharedMemPerBlock;
  if (l2_bytes) *l2_bytes = p.l2CacheSize;
  if (gcn_arch) {
    int v = 0;
    if (sscanf(p.gcnArchName, "gfx%x", &v) != 1) v = 0;
    *gcn_arch = v;
  }
  return 0;
}

int afx_stream_sync(void* stream) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return afx::set_error("hipStreamSynchronize: %s", hipGetErrorString(e));
  return 0;
}

// ---- HIP graph capture of a kernel sequence (the decode step is replayed as one graph) ----
int afx_graph_begin(void* stream) {
  hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return afx::set_error("hipStreamBeginCapture: %s", hipGetErrorString(e));
  return 0;
}

int afx_graph_end(void* stream, void** exec_out) {
  AFX_REQUIRE(exec_out, "afx_graph_end: null exec_out");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
  if (e != hipSuccess) return afx::set_error("hipStreamEndCapture: %s", hipGetErrorString(e));
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  const hipError_t d = hipGraphDestroy(g);       // the executable graph keeps what it needs
  if (e != hipSuccess) return afx::set_error("hipGraphInstantiate: %s", hipGetErrorString(e));
  if (d != hipSuccess) {
    (void)hipGraphExecDestroy(ex);
    return afx::set_error("hipGraphDestroy: %s", hipGetErrorString(d));
  }
  *exec_out = (void*)ex;
  return 0;
}

int afx_graph_launch(void* exec, void* stream) {
  hipError_t e = hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream);
  if (e != hipSuccess) return afx::set_error("hipGraphLaunch: %s", hipGetErrorString(e));
  return 0;
}

int afx_graph_destroy(void* exec) {
  if (!exec) return 0;
  hipError_t e = hipGraphExecDestroy((hipGraphExec_t)exec);
  if (e != hipSuccess) return afx::set_error("hipGraphExecDestroy: %s", hipGetErrorString(e));
  return 0;
}

// ---- events on the caller's stream (timing the stream the kernels actually run on) ----
int afx_event_create(void** ev) {
  AFX_REQUIRE(ev, "afx_event_create: null output pointer");
  hipEvent_t e;
  hipError_t r = hipEventCreate(&e);
  if (r != hipSuccess) return afx::set_error("hipEventCreate: %s", hipGetErrorString(r));
  *ev = (void*)e;
  return 0;
}
int afx_event_record(void* ev, void* stream) {
  hipError_t r = hipEventRecord((hipEvent_t)ev, (hipStream_t)stream);
  if (r != hipSuccess) return afx::set_error("hipEventRecord: %s", hipGetErrorString(r));
  return 0;
}
int afx_event_elapsed_ms(void* start, void* stop, float* ms) {
  AFX_REQUIRE(start && stop && ms, "afx_event_elapsed_ms: null argument");
  hipError_t r = hipEventSynchronize((hipEvent_t)stop);
  if (r != hipSuccess) return afx::set_error("hipEventSynchronize: %s", hipGetErrorString(r));
  r = hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
  if (r != hipSuccess) return afx::set_error("hipEventElapsedTime: %s", hipGetErrorString(r));
  return 0;
}
int afx_event_destroy(void* ev) {
  if (!ev) return 0;
  const hipError_t r = hipEventDestroy((hipEvent_t)ev);
  if (r != hipSuccess) return afx::set_error("hipEventDestroy: %s", hipGetErrorString(r));
  return 0;
}

}  // extern "C"
