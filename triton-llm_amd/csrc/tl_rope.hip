// RoPE (half-split pairing) in place, and RoPE fused with the KV-cache append.
//
// Pairing and position rule follow the reference kernel
// (triton_llm/kernels/rope.py:49-66): element i pairs with i + d_k/2,
//   out[i]        = x[i] * cos[pos, i] - x[i + h] * sin[pos, i]
//   out[i + h]    = x[i] * sin[pos, i] + x[i + h] * cos[pos, i]
// Each product and the sum/difference are rounded separately in fp32, which
// is exactly how NumPy evaluates the same expression, so the fp32 result is
// bit-identical to the host restatement; 16-bit outputs are then rounded once
// (RNE) to the storage type.  hipcc contracts a*b - c*d into an FMA by default
// (even when written with __fmul_rn / __fsub_rn), so the rotation helper
// switches contraction off for its own expressions.
#include "tl_common.h"

namespace {

__device__ __forceinline__ void rotate_pair(float xe, float xo, float c, float s,
                                            float& oe, float& oo) {
#pragma clang fp contract(off)
  const float a = xe * c, b = xo * s, d = xe * s, e = xo * c;
  oe = a - b;
  oo = d + e;
}

// One thread per (row, pair index).  Rows are flattened (..., seq) so the
// position is row % seq_len + offset, as in rope.py:49.
template <typename T>
__global__ void rope_inplace_kernel(typename T::bits* __restrict__ x,
                                    const float* __restrict__ cos_t,
                                    const float* __restrict__ sin_t,
                                    int64_t n_rows, int64_t row_stride, int half,
                                    int seq_len, int offset) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = n_rows * half;
  if (tid >= total) return;
  const int64_t row = tid / half;
  const int i = (int)(tid - row * half);
  const int pos = (int)(row % seq_len) + offset;
  typename T::bits* xr = x + row * row_stride;
  const float xe = to_f32<T>(xr[i]);
  const float xo = to_f32<T>(xr[i + half]);
  const float c = cos_t[(int64_t)pos * half + i];
  const float s = sin_t[(int64_t)pos * half + i];
  float oe, oo;
  rotate_pair(xe, xo, c, s, oe, oo);
  xr[i] = from_f32<T>(oe);
  xr[i + half] = from_f32<T>(oo);
}

struct AppendParams {
  void* q;
  const void* k_new;
  const void* v_new;
  void* k_cache;
  void* v_cache;
  const int32_t* lens;
  const float* cos_t;
  const float* sin_t;
  int rope_rows;
  int batch, n_new, n_head, n_kv, max_ctx, half;
  int64_t q_sb, q_ss, q_sh;
  int64_t kn_sb, kn_ss, kn_sh;
  int64_t vn_sb, vn_ss, vn_sh;
  int64_t kc_sb, kc_sh, kc_ss;
  int64_t vc_sb, vc_sh, vc_ss;
};

// grid.x = batch * n_new tokens, grid.y = n_head + 2*n_kv row kinds (q heads,
// k heads, v heads); the threads of a block stride over the pair index i.
template <typename T>
__global__ void rope_kv_append_kernel(AppendParams p) {
  using B = typename T::bits;
  const int kind = blockIdx.y;
  const int b = blockIdx.x / p.n_new;
  const int s = blockIdx.x - b * p.n_new;
  const int pos = p.lens[b] + s;
  const bool rope = p.cos_t != nullptr;
  const bool pos_ok = pos >= 0 && pos < p.max_ctx && (!rope || pos < p.rope_rows);
  for (int i = threadIdx.x; i < p.half; i += blockDim.x) {
  float c = 1.f, sn = 0.f;
  if (rope && pos_ok) {
    c = p.cos_t[(int64_t)pos * p.half + i];
    sn = p.sin_t[(int64_t)pos * p.half + i];
  }
  if (kind < p.n_head) {
    if (!p.q || !rope || !pos_ok) continue;
    B* qr = (B*)p.q + b * p.q_sb + s * p.q_ss + kind * p.q_sh;
    float oe, oo;
    rotate_pair(to_f32<T>(qr[i]), to_f32<T>(qr[i + p.half]), c, sn, oe, oo);
    qr[i] = from_f32<T>(oe);
    qr[i + p.half] = from_f32<T>(oo);
  } else if (kind < p.n_head + p.n_kv) {
    if (!pos_ok) continue;
    const int h = kind - p.n_head;
    const B* kr = (const B*)p.k_new + b * p.kn_sb + s * p.kn_ss + h * p.kn_sh;
    B* dst = (B*)p.k_cache + b * p.kc_sb + h * p.kc_sh + (int64_t)pos * p.kc_ss;
    if (rope) {
      float oe, oo;
      rotate_pair(to_f32<T>(kr[i]), to_f32<T>(kr[i + p.half]), c, sn, oe, oo);
      dst[i] = from_f32<T>(oe);
      dst[i + p.half] = from_f32<T>(oo);
    } else {
      dst[i] = kr[i];
      dst[i + p.half] = kr[i + p.half];
    }
  } else {
    if (!pos_ok) continue;
    const int h = kind - p.n_head - p.n_kv;
    const B* vr = (const B*)p.v_new + b * p.vn_sb + s * p.vn_ss + h * p.vn_sh;
    B* dst = (B*)p.v_cache + b * p.vc_sb + h * p.vc_sh + (int64_t)pos * p.vc_ss;
    dst[i] = vr[i];
    dst[i + p.half] = vr[i + p.half];
  }
  }
}

template <typename T>
int launch_rope_inplace(void* x, const float* c, const float* s, int64_t n_rows,
                        int64_t row_stride, int d_k, int seq_len, int offset,
                        hipStream_t st) {
  const int half = d_k / 2;
  const int64_t total = n_rows * half;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(rope_inplace_kernel<T>, dim3((unsigned)blocks), dim3(threads), 0, st,
                     (typename T::bits*)x, c, s, n_rows, row_stride, half, seq_len, offset);
  return tl_launch_status();
}

template <typename T>
int launch_append(const AppendParams& p, hipStream_t st) {
  const int threads = p.half <= 64 ? 64 : (p.half <= 128 ? 128 : 256);
  dim3 grid((unsigned)p.batch * (unsigned)p.n_new, p.n_head + 2 * p.n_kv, 1);
  hipLaunchKernelGGL(rope_kv_append_kernel<T>, grid, dim3(threads), 0, st, p);
  return tl_launch_status();
}

}  // namespace

extern "C" {

int tl_rope_inplace(void* x, const float* cos_table, const float* sin_table,
                    int64_t n_rows, int64_t row_stride, int d_k, int seq_len,
                    int position_offset, int dtype, void* stream) {
  if (n_rows == 0) return 0;
  if (!x || !cos_table || !sin_table || d_k < 2 || (d_k & 1) || seq_len < 1 ||
      position_offset < 0 || n_rows < 0 || row_stride < d_k)
    return TL_ERR_INVALID;
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: return launch_rope_inplace<F32>(x, cos_table, sin_table, n_rows, row_stride, d_k, seq_len, position_offset, st);
    case TL_DTYPE_F16: return launch_rope_inplace<F16>(x, cos_table, sin_table, n_rows, row_stride, d_k, seq_len, position_offset, st);
    case TL_DTYPE_BF16: return launch_rope_inplace<BF16>(x, cos_table, sin_table, n_rows, row_stride, d_k, seq_len, position_offset, st);
    default: return TL_ERR_INVALID;
  }
}

int tl_rope_kv_append(void* q, const void* k_new, const void* v_new,
                      void* k_cache, void* v_cache, const int32_t* cache_lens,
                      const float* cos_table, const float* sin_table,
                      int rope_rows, int batch, int n_new, int n_head,
                      int n_kv_head, int max_ctx, int d_k,
                      const int64_t* q_strides, const int64_t* k_new_strides,
                      const int64_t* v_new_strides,
                      const int64_t* k_cache_strides,
                      const int64_t* v_cache_strides, int dtype, void* stream) {
  if (batch == 0 || n_new == 0) return 0;
  if (!k_new || !v_new || !k_cache || !v_cache || !cache_lens || batch < 0 ||
      n_new < 0 || n_head < 0 || n_kv_head < 1 || d_k < 2 || (d_k & 1) ||
      max_ctx < 1 || !k_new_strides || !v_new_strides || !k_cache_strides ||
      !v_cache_strides)
    return TL_ERR_INVALID;
  if ((cos_table == nullptr) != (sin_table == nullptr)) return TL_ERR_INVALID;
  if (q && !q_strides) return TL_ERR_INVALID;
  AppendParams p{};
  p.q = q;
  p.k_new = k_new;
  p.v_new = v_new;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.lens = cache_lens;
  p.cos_t = cos_table;
  p.sin_t = sin_table;
  p.rope_rows = rope_rows;
  p.batch = batch;
  p.n_new = n_new;
  p.n_head = q ? n_head : 0;
  p.n_kv = n_kv_head;
  p.max_ctx = max_ctx;
  p.half = d_k / 2;
  if (q) {
    p.q_sb = q_strides[0];
    p.q_ss = q_strides[1];
    p.q_sh = q_strides[2];
  }
  p.kn_sb = k_new_strides[0];
  p.kn_ss = k_new_strides[1];
  p.kn_sh = k_new_strides[2];
  p.vn_sb = v_new_strides[0];
  p.vn_ss = v_new_strides[1];
  p.vn_sh = v_new_strides[2];
  p.kc_sb = k_cache_strides[0];
  p.kc_sh = k_cache_strides[1];
  p.kc_ss = k_cache_strides[2];
  p.vc_sb = v_cache_strides[0];
  p.vc_sh = v_cache_strides[1];
  p.vc_ss = v_cache_strides[2];
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: return launch_append<F32>(p, st);
    case TL_DTYPE_F16: return launch_append<F16>(p, st);
    case TL_DTYPE_BF16: return launch_append<BF16>(p, st);
    default: return TL_ERR_INVALID;
  }
}

}  // extern "C"
