// The model step's elementwise and row-reduction layers around the
// projections: RMSNorm, residual add + RMSNorm fused, SwiGLU, add.
//
// Reference behaviour being replaced:
//   * rms_norm (triton_llm/kernels/rms_norm.py:21-116): one program per row,
//     rms = sqrt(sum(x^2) / N + eps), y = (x / rms) * w (:47-56);
//   * swiglu (swiglu.py:21-125): silu(x) * y with the single-exp stable
//     sigmoid, exp(-|x|) (:46-54);
//   * add (add.py:14-104): z = x + y.
// In the model every RMSNorm after the first of a layer reads the sum the
// residual add just wrote (smollm2_triton/model.py:352-357 and the next
// layer's :279-280); tl_add_rms_norm does both in one pass over the row,
// writing the sum (the next residual) and the normalised row.
//
// All are HBM-bound (or launch-bound at decode sizes): lane-contiguous
// loads, fp32 arithmetic whatever the storage type.
#include "tl_common.h"

#include <math.h>

namespace {

constexpr int kRowThreads = 256;
constexpr int kEltThreads = 256;

template <typename T>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  return to_f32<T>(((const typename T::bits*)p)[i]);
}
template <typename T>
__device__ __forceinline__ void st(void* p, int64_t i, float x) {
  ((typename T::bits*)p)[i] = from_f32<T>(x);
}

__device__ __forceinline__ float block_sum(float v, float* s_red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) t += s_red[w];
  return t;
}

// One workgroup per row, the row held in registers (VPT elements per
// thread, element tid + 256 j), so it is read from memory once.  With
// b != nullptr the row is a + b, written to h (the residual for the next add)
// and normalised as stored, i.e. after rounding to T, as a separate add then
// RMSNorm would.  Rows longer than 256 * 32 take rms_norm_kernel below.
template <typename T, int VPT>
__global__ __launch_bounds__(kRowThreads) void rms_norm_row_kernel(const void* a, const void* b, void* h, const void* w,
                                                                   void* y, int n, float eps) {
  __shared__ float s_red[kRowThreads / 64];
  const int64_t row = (int64_t)blockIdx.x * n;
  float x[VPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int i = threadIdx.x + kRowThreads * j;
    float v = 0.f;
    if (i < n) {
      v = ld<T>(a, row + i);
      if (b) {
        const typename T::bits r = from_f32<T>(v + ld<T>(b, row + i));
        ((typename T::bits*)h)[row + i] = r;
        v = to_f32<T>(r);
      }
    }
    x[j] = v;
    ss += v * v;
  }
  const float rms = sqrtf(block_sum(ss, s_red) / (float)n + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int i = threadIdx.x + kRowThreads * j;
    if (i < n) st<T>(y, row + i, (x[j] / rms) * ld<T>(w, i));
  }
}

// Any row length: two passes over the row (the second mostly from L2).
template <typename T>
// No __restrict__: callers may update the residual in place (h == a) or
// normalise in place (y == x); every element is read before it is written by
// the same thread.
__global__ __launch_bounds__(kRowThreads) void rms_norm_kernel(const void* a, const void* b, void* h, const void* w,
                                                               void* y, int n, float eps) {
  __shared__ float s_red[kRowThreads / 64];
  const int64_t row = (int64_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x; i < n; i += kRowThreads) {
    float x = ld<T>(a, row + i);
    if (b) {
      x += ld<T>(b, row + i);
      st<T>(h, row + i, x);
      x = ld<T>(h, row + i);  // normalise the stored (rounded) sum, as a separate add then RMSNorm would
    }
    ss += x * x;
  }
  const float rms = sqrtf(block_sum(ss, s_red) / (float)n + eps);
  const void* src = b ? (const void*)h : a;
  for (int i = threadIdx.x; i < n; i += kRowThreads) st<T>(y, row + i, (ld<T>(src, row + i) / rms) * ld<T>(w, i));
}

template <typename T>
__global__ __launch_bounds__(kEltThreads) void swiglu_kernel(const void* __restrict__ g, const void* __restrict__ u,
                                                             void* __restrict__ o, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; i < count; i += (int64_t)gridDim.x * kEltThreads) {
    const float x = ld<T>(g, i);
    const float e = expf(-fabsf(x));  // <= 1, never overflows
    const float sig = x >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
    st<T>(o, i, x * sig * ld<T>(u, i));
  }
}

template <typename T>
__global__ __launch_bounds__(kEltThreads) void add_kernel(const void* __restrict__ x, const void* __restrict__ y,
                                                          void* __restrict__ z, int64_t count) {
  for (int64_t i = (int64_t)blockIdx.x * kEltThreads + threadIdx.x; i < count; i += (int64_t)gridDim.x * kEltThreads)
    st<T>(z, i, ld<T>(x, i) + ld<T>(y, i));
}

unsigned elt_blocks(int64_t count) {
  const int64_t b = (count + kEltThreads - 1) / kEltThreads;
  return (unsigned)(b < 65536 ? b : 65536);
}

bool dtype_ok(int dtype) { return dtype == TL_DTYPE_F32 || dtype == TL_DTYPE_F16 || dtype == TL_DTYPE_BF16; }

template <template <typename> class Launch, typename... Args>
int by_dtype(int dtype, Args... args) {
  switch (dtype) {
    case TL_DTYPE_F32: return Launch<F32>::run(args...);
    case TL_DTYPE_F16: return Launch<F16>::run(args...);
    default: return Launch<BF16>::run(args...);
  }
}

template <typename T>
struct RmsLaunch {
  static int run(const void* a, const void* b, void* h, const void* w, void* y, int m, int n, float eps, hipStream_t st) {
    const dim3 grid((unsigned)m), block(kRowThreads);
    if (n <= kRowThreads * 4)
      hipLaunchKernelGGL((rms_norm_row_kernel<T, 4>), grid, block, 0, st, a, b, h, w, y, n, eps);
    else if (n <= kRowThreads * 8)
      hipLaunchKernelGGL((rms_norm_row_kernel<T, 8>), grid, block, 0, st, a, b, h, w, y, n, eps);
    else if (n <= kRowThreads * 16)
      hipLaunchKernelGGL((rms_norm_row_kernel<T, 16>), grid, block, 0, st, a, b, h, w, y, n, eps);
    else if (n <= kRowThreads * 32)
      hipLaunchKernelGGL((rms_norm_row_kernel<T, 32>), grid, block, 0, st, a, b, h, w, y, n, eps);
    else
      hipLaunchKernelGGL((rms_norm_kernel<T>), grid, block, 0, st, a, b, h, w, y, n, eps);
    return tl_launch_status();
  }
};
template <typename T>
struct SwigluLaunch {
  static int run(const void* g, const void* u, void* o, int64_t count, hipStream_t st) {
    hipLaunchKernelGGL((swiglu_kernel<T>), dim3(elt_blocks(count)), dim3(kEltThreads), 0, st, g, u, o, count);
    return tl_launch_status();
  }
};
template <typename T>
struct AddLaunch {
  static int run(const void* x, const void* y, void* z, int64_t count, hipStream_t st) {
    hipLaunchKernelGGL((add_kernel<T>), dim3(elt_blocks(count)), dim3(kEltThreads), 0, st, x, y, z, count);
    return tl_launch_status();
  }
};

}  // namespace

extern "C" {

int tl_rms_norm(const void* x, const void* w, void* y, int m, int n, float eps, int dtype, void* stream) {
  if (m < 0 || n < 0 || !dtype_ok(dtype)) return TL_ERR_INVALID;
  if (m == 0) return 0;
  if (n == 0 || !x || !w || !y) return TL_ERR_INVALID;
  return by_dtype<RmsLaunch>(dtype, x, (const void*)nullptr, (void*)nullptr, w, y, m, n, eps, tl_resolve_stream(stream));
}

int tl_add_rms_norm(const void* a, const void* b, void* h, const void* w, void* y, int m, int n, float eps, int dtype,
                    void* stream) {
  if (m < 0 || n < 0 || !dtype_ok(dtype)) return TL_ERR_INVALID;
  if (m == 0) return 0;
  if (n == 0 || !a || !b || !h || !w || !y) return TL_ERR_INVALID;
  return by_dtype<RmsLaunch>(dtype, a, b, h, w, y, m, n, eps, tl_resolve_stream(stream));
}

int tl_swiglu(const void* gate, const void* up, void* out, int64_t count, int dtype, void* stream) {
  if (count < 0 || !dtype_ok(dtype)) return TL_ERR_INVALID;
  if (count == 0) return 0;
  if (!gate || !up || !out) return TL_ERR_INVALID;
  return by_dtype<SwigluLaunch>(dtype, gate, up, out, count, tl_resolve_stream(stream));
}

int tl_add(const void* x, const void* y, void* z, int64_t count, int dtype, void* stream) {
  if (count < 0 || !dtype_ok(dtype)) return TL_ERR_INVALID;
  if (count == 0) return 0;
  if (!x || !y || !z) return TL_ERR_INVALID;
  return by_dtype<AddLaunch>(dtype, x, y, z, count, tl_resolve_stream(stream));
}

}  // extern "C"
