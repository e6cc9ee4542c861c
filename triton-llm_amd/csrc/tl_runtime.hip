// Runtime half of the C ABI: device selection, the library stream, the
// allocator and copies.  The Python allocator (triton_llm/gpu.py) binds these
// instead of binding libamdhip64 symbols directly, so every copy and every
// kernel launch shares one in-order HIP stream.
#include "tl_common.h"

#include <stdlib.h>

namespace {
hipStream_t g_stream = nullptr;
int g_device = -1;

// Byte fill: 16-byte stores over the aligned middle, single bytes for the
// unaligned head and tail (at most 15 each, taken by the first threads).
__global__ __launch_bounds__(256) void fill_bytes_kernel(unsigned char* dst, unsigned char v, size_t n) {
  const size_t head = min(n, (size_t)((16 - ((uintptr_t)dst & 15)) & 15));
  const size_t words = (n - head) / 16;
  const size_t tail = head + words * 16;
  const uint32_t w = 0x01010101u * v;
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  u32x4* body = (u32x4*)(dst + head);
  for (size_t i = tid; i < words; i += stride) body[i] = u32x4{w, w, w, w};
  if (tid < head) dst[tid] = v;
  if (tid < n - tail) dst[tail + tid] = v;
}
}  // namespace

// A kernel, not hipMemsetAsync, so that a fill issued while a caller records
// a HIP graph becomes a kernel node (memset nodes have replayed wrongly).
int tl_fill_bytes(void* dst, unsigned char value, size_t nbytes, hipStream_t st) {
  if (nbytes == 0) return 0;
  const size_t words = nbytes / 16 + 1;
  size_t blocks = (words + 255) / 256;
  blocks = blocks < 4096 ? blocks : 4096;
  hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (unsigned char*)dst, value,
                     nbytes);
  return tl_launch_status();
}

hipStream_t tl_resolve_stream(void* stream) {
  return stream ? (hipStream_t)stream : g_stream;
}

int tl_device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  int n = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (cus[dev] == 0) {
      int c = 0;
      if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
      cus[dev] = c;
    }
    n = cus[dev];
  }
  const int c = tl_overrides.max_cus;
  if (c > 0 && c < n) n = c;
  return n;
}

TlOverrides tl_overrides = {0, 0, 0, 0, 0};

namespace {
int env_int(const char* name) {
  const char* v = getenv(name);
  return v ? atoi(v) : 0;
}
}  // namespace

extern "C" {

int tl_device_count(int* count) {
  if (!count) return TL_ERR_INVALID;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  *count = (e == hipSuccess) ? n : 0;
  return (int)e;
}

int tl_init(int device) {
  tl_overrides.max_cus = env_int("TRITON_LLM_HIP_MAX_CUS");
  tl_overrides.decode_shares = env_int("TRITON_LLM_HIP_DECODE_SHARES") != 0;
  tl_overrides.prefill_w64 = env_int("TRITON_LLM_HIP_PREFILL_W64") != 0;
  tl_overrides.prefill_one_list = env_int("TRITON_LLM_HIP_PREFILL_ONE_LIST") != 0;
  tl_overrides.prefill_no_split = env_int("TRITON_LLM_HIP_PREFILL_NO_SPLIT") != 0;
  if (g_stream && g_device == device) return 0;
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return (int)e;
  if (g_stream) {
    // Re-initialising on another device: drop the old stream first.
    (void)hipStreamDestroy(g_stream);
    g_stream = nullptr;
  }
  // Default priority, non-blocking with respect to the legacy null stream.
  e = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
  if (e != hipSuccess) return (int)e;
  g_device = device;
  return 0;
}

void* tl_default_stream(void) { return (void*)g_stream; }

int tl_malloc(void** ptr, size_t nbytes) {
  if (!ptr) return TL_ERR_INVALID;
  *ptr = nullptr;
  if (nbytes == 0) return 0;  // zero-byte tensors carry a NULL pointer
  return (int)hipMalloc(ptr, nbytes);
}

int tl_free(void* ptr) {
  if (!ptr) return 0;
  return (int)hipFree(ptr);
}

int tl_memcpy_htod(void* dst, const void* host_src, size_t nbytes) {
  if (nbytes == 0) return 0;
  if (!dst || !host_src) return TL_ERR_INVALID;
  hipError_t e = hipMemcpyAsync(dst, host_src, nbytes, hipMemcpyHostToDevice, g_stream);
  if (e != hipSuccess) return (int)e;
  // The host buffer may be released by the caller right after return.
  return (int)hipStreamSynchronize(g_stream);
}

int tl_memcpy_dtoh(void* host_dst, const void* src, size_t nbytes) {
  if (nbytes == 0) return 0;
  if (!host_dst || !src) return TL_ERR_INVALID;
  hipError_t e = hipMemcpyAsync(host_dst, src, nbytes, hipMemcpyDeviceToHost, g_stream);
  if (e != hipSuccess) return (int)e;
  return (int)hipStreamSynchronize(g_stream);
}

int tl_memcpy_dtod(void* dst, const void* src, size_t nbytes) {
  if (nbytes == 0) return 0;
  if (!dst || !src) return TL_ERR_INVALID;
  return (int)hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, g_stream);
}

int tl_memset(void* dst, int value, size_t nbytes) {
  if (nbytes == 0) return 0;
  if (!dst) return TL_ERR_INVALID;
  return tl_fill_bytes(dst, (unsigned char)value, nbytes, g_stream);
}

int tl_synchronize(void) {
  hipError_t e = g_stream ? hipStreamSynchronize(g_stream) : hipSuccess;
  if (e != hipSuccess) return (int)e;
  return (int)hipDeviceSynchronize();
}

int tl_graph_capture_begin(void* stream) {
  // Relaxed mode: calls on other threads (and cached-block allocations on
  // this one) stay legal while the stream records.
  return (int)hipStreamBeginCapture(tl_resolve_stream(stream), hipStreamCaptureModeRelaxed);
}

int tl_graph_capture_end(void* stream, void** exec) {
  if (!exec) return TL_ERR_INVALID;
  *exec = nullptr;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(tl_resolve_stream(stream), &graph);
  if (e != hipSuccess) return (int)e;
  hipGraphExec_t ge = nullptr;
  e = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return (int)e;
  *exec = (void*)ge;
  return 0;
}

int tl_graph_launch(void* exec, void* stream) {
  if (!exec) return TL_ERR_INVALID;
  return (int)hipGraphLaunch((hipGraphExec_t)exec, tl_resolve_stream(stream));
}

int tl_graph_destroy(void* exec) {
  if (!exec) return 0;
  return (int)hipGraphExecDestroy((hipGraphExec_t)exec);
}

const char* tl_error_string(int status) {
  if (status == 0) return "success";
  return hipGetErrorString((hipError_t)status);
}

int tl_event_create(void** event) {
  if (!event) return TL_ERR_INVALID;
  return (int)hipEventCreate((hipEvent_t*)event);
}

int tl_event_destroy(void* event) { return (int)hipEventDestroy((hipEvent_t)event); }

int tl_event_record(void* event, void* stream) {
  return (int)hipEventRecord((hipEvent_t)event, tl_resolve_stream(stream));
}

int tl_event_synchronize(void* event) { return (int)hipEventSynchronize((hipEvent_t)event); }

int tl_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms) return TL_ERR_INVALID;
  return (int)hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop);
}

}  // extern "C"
