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
  rope_rotate_pair(xe, xo, c, s, oe, oo);
}

// VEC consecutive table entries (fp32) from row offset `at`: 16-byte loads.
template <int VEC>
__device__ __forceinline__ void load_table(const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                           int64_t at, float (&c)[VEC], float (&sn)[VEC]) {
#pragma unroll
  for (int v = 0; v < VEC; v += 4) {
    const f32x4 cv = *(const f32x4*)(cos_t + at + v);
    const f32x4 sv = *(const f32x4*)(sin_t + at + v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      c[v + e] = cv[e];
      sn[v + e] = sv[e];
    }
  }
}

// Rotate the 16-byte chunks lo (elements i..) and hi (elements i + half..)
// of one row, element by element, rounding each result once to T.
template <typename T, int VEC = 16 / T::size>
__device__ __forceinline__ void rotate_chunk(const u32x4& wl, const u32x4& wh, const float (&c)[VEC],
                                             const float (&sn)[VEC], u32x4& ol, u32x4& oh) {
  using B = typename T::bits;
  B xl[VEC], xh[VEC], yl[VEC], yh[VEC];
  __builtin_memcpy(xl, &wl, 16);
  __builtin_memcpy(xh, &wh, 16);
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    float oe, oo;
    rotate_pair(to_f32<T>(xl[e]), to_f32<T>(xh[e]), c[e], sn[e], oe, oo);
    yl[e] = from_f32<T>(oe);
    yh[e] = from_f32<T>(oo);
  }
  __builtin_memcpy(&ol, yl, 16);
  __builtin_memcpy(&oh, yh, 16);
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

// 16-byte form of rope_inplace_kernel: thread (row, j) rotates the VEC
// pairs (i, i + half) for i in [VEC j, VEC j + VEC) with one 16-byte load
// and store per half row and VEC cos / sin values per table.  Same
// arithmetic per element, so the same bits.
template <typename T>
__global__ __launch_bounds__(256) void rope_inplace_vec_kernel(typename T::bits* __restrict__ x,
                                                               const float* __restrict__ cos_t,
                                                               const float* __restrict__ sin_t,
                                                               int64_t n_rows, int64_t row_stride, int half,
                                                               int seq_len, int offset) {
  constexpr int VEC = 16 / T::size;
  const int cph = half / VEC;  // 16-byte chunks per half row
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= n_rows * cph) return;
  const int64_t row = tid / cph;
  const int j = (int)(tid - row * cph);
  const int pos = (int)(row % seq_len) + offset;
  typename T::bits* lo = x + row * row_stride + j * VEC;
  typename T::bits* hi = lo + half;
  const u32x4 wl = *(const u32x4*)lo, wh = *(const u32x4*)hi;
  float c[VEC], sn[VEC];
  load_table<VEC>(cos_t, sin_t, (int64_t)pos * half + j * VEC, c, sn);
  u32x4 ol, oh;
  rotate_chunk<T>(wl, wh, c, sn, ol, oh);
  *(u32x4*)lo = ol;
  *(u32x4*)hi = oh;
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

// 16-byte form of rope_kv_append_kernel.  A token's rows are its n_head q
// rows, then n_kv k rows, then n_kv v rows.  Thread t takes chunk j = t % cph
// of a half row (elements [VEC j, VEC j + VEC) and the same + half), row
// group g = (t / cph) % R and token t / (cph R), and walks rows g, g + R,
// ... of that token, UNROLL rows' loads in flight at a time.  Its cos / sin
// values are loaded once for all of them.  Adjacent lanes take adjacent
// chunks and then adjacent rows, so one instruction covers contiguous
// memory (a token's q heads, say).
// Global-memory (address space 1) view of a pointer, so loads and stores are
// global_* instructions rather than flat ones (which also count in lgkmcnt).
template <typename X>
__device__ __forceinline__ __attribute__((address_space(1))) X* gmem(X* p) {
  return (__attribute__((address_space(1))) X*)p;
}

// Rows r in [lo, hi) with r = g (mod R) of one row kind, UNROLL rows' loads
// in flight at a time: src row r at src + (r - lo) * src_step, written to dst
// + (r - lo) * dst_step, rotated or copied.
template <typename T, int UNROLL, bool ROT>
__device__ __forceinline__ void append_rows(const typename T::bits* src, int64_t src_step,
                                            typename T::bits* dst, int64_t dst_step, int lo, int hi, int g,
                                            int R, int half, const float (&c)[16 / T::size],
                                            const float (&sn)[16 / T::size]) {
  int r = lo + ((g - lo) % R + R) % R;  // first row of this group in [lo, hi)
  for (; r < hi; r += UNROLL * R) {
    u32x4 wl[UNROLL], wh[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (r + u * R < hi) {
        const auto* sp = gmem(src + (int64_t)(r + u * R - lo) * src_step);
        wl[u] = *(const __attribute__((address_space(1))) u32x4*)sp;
        wh[u] = *(const __attribute__((address_space(1))) u32x4*)(sp + half);
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      if (r + u * R < hi) {
        u32x4 ol = wl[u], oh = wh[u];
        if constexpr (ROT) rotate_chunk<T>(wl[u], wh[u], c, sn, ol, oh);
        auto* dp = gmem(dst + (int64_t)(r + u * R - lo) * dst_step);
        *(__attribute__((address_space(1))) u32x4*)dp = ol;
        *(__attribute__((address_space(1))) u32x4*)(dp + half) = oh;
      }
    }
  }
}

// 16-byte form of rope_kv_append_kernel.  A token's rows are its n_head q
// rows, then n_kv k rows, then n_kv v rows.  Thread t takes chunk j = t % cph
// of a half row (elements [VEC j, VEC j + VEC) and the same + half), row
// group g = (t / cph) % R and token t / (cph R), and handles that token's
// rows g, g + R, ... (q rotated in place, k rotated into the cache, v copied
// into it), four rows' loads in flight at a time, with its cos / sin values
// loaded once for all of them.  Adjacent lanes take adjacent chunks and
// then adjacent rows, so one instruction covers contiguous memory (a
// token's q heads, say).
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_append_vec_kernel(AppendParams p, int R) {
  using B = typename T::bits;
  constexpr int VEC = 16 / T::size;
  constexpr int UNROLL = 4;
  const int cph = p.half / VEC;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tok = (int64_t)cph * R;
  if (tid >= (int64_t)p.batch * p.n_new * per_tok) return;
  const int tok = (int)(tid / per_tok);
  const int rest = (int)(tid - (int64_t)tok * per_tok);
  const int j = rest % cph;
  const int g = rest / cph;
  const int b = tok / p.n_new;
  const int s = tok - b * p.n_new;
  const int pos = p.lens[b] + s;
  const bool rope = p.cos_t != nullptr;
  if (pos < 0 || pos >= p.max_ctx || (rope && pos >= p.rope_rows)) return;  // nothing is written
  float c[VEC], sn[VEC];
  const int col = j * VEC;
  const int hq = p.n_head, hk = p.n_head + p.n_kv, hv = p.n_head + 2 * p.n_kv;
  if (rope) {
    load_table<VEC>(p.cos_t, p.sin_t, (int64_t)pos * p.half + col, c, sn);
    if (hq > 0) {
      B* q = (B*)p.q + b * p.q_sb + s * p.q_ss + col;
      append_rows<T, UNROLL, true>(q, p.q_sh, q, p.q_sh, 0, hq, g, R, p.half, c, sn);
    }
    append_rows<T, UNROLL, true>((const B*)p.k_new + b * p.kn_sb + s * p.kn_ss + col, p.kn_sh,
                                 (B*)p.k_cache + b * p.kc_sb + (int64_t)pos * p.kc_ss + col, p.kc_sh, hq, hk, g, R,
                                 p.half, c, sn);
  } else {
    append_rows<T, UNROLL, false>((const B*)p.k_new + b * p.kn_sb + s * p.kn_ss + col, p.kn_sh,
                                  (B*)p.k_cache + b * p.kc_sb + (int64_t)pos * p.kc_ss + col, p.kc_sh, hq, hk, g, R,
                                  p.half, c, sn);
  }
  append_rows<T, UNROLL, false>((const B*)p.v_new + b * p.vn_sb + s * p.vn_ss + col, p.vn_sh,
                                (B*)p.v_cache + b * p.vc_sb + (int64_t)pos * p.vc_ss + col, p.vc_sh, hk, hv, g, R,
                                p.half, c, sn);
}

inline bool al16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

template <typename T>
int launch_rope_inplace(void* x, const float* c, const float* s, int64_t n_rows,
                        int64_t row_stride, int d_k, int seq_len, int offset,
                        hipStream_t st) {
  const int half = d_k / 2;
  constexpr int VEC = 16 / T::size;
  const int threads = 256;
  if (half % VEC == 0 && row_stride % VEC == 0 && al16(x) && al16(c) && al16(s)) {
    const int64_t total = n_rows * (half / VEC);
    hipLaunchKernelGGL(rope_inplace_vec_kernel<T>, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads),
                       0, st, (typename T::bits*)x, c, s, n_rows, row_stride, half, seq_len, offset);
    return tl_launch_status();
  }
  const int64_t total = n_rows * half;
  const int64_t blocks = (total + threads - 1) / threads;
  hipLaunchKernelGGL(rope_inplace_kernel<T>, dim3((unsigned)blocks), dim3(threads), 0, st,
                     (typename T::bits*)x, c, s, n_rows, row_stride, half, seq_len, offset);
  return tl_launch_status();
}

template <typename T>
bool append_vec_ok(const AppendParams& p) {
  constexpr int VEC = 16 / T::size;
  if (p.half % VEC) return false;
  const int64_t st[] = {p.kn_sb, p.kn_ss, p.kn_sh, p.vn_sb, p.vn_ss, p.vn_sh,
                        p.kc_sb, p.kc_sh, p.kc_ss, p.vc_sb, p.vc_sh, p.vc_ss};
  for (int64_t x : st)
    if (x % VEC) return false;
  if (p.q && (p.q_sb % VEC || p.q_ss % VEC || p.q_sh % VEC || !al16(p.q))) return false;
  if (p.cos_t && (!al16(p.cos_t) || !al16(p.sin_t))) return false;
  return al16(p.k_new) && al16(p.v_new) && al16(p.k_cache) && al16(p.v_cache);
}

template <typename T>
int launch_append(const AppendParams& p, hipStream_t st) {
  if (append_vec_ok<T>(p)) {
    // Row groups per token: all rows at once for small steps (a decoded
    // token: one row per thread), about 2^18 threads for prompts (each
    // thread then walks several rows with its table values loaded once).
    constexpr int VEC = 16 / T::size;
    const int n_rows = p.n_head + 2 * p.n_kv;
    const int64_t lanes_per_row = (int64_t)p.batch * p.n_new * (p.half / VEC);
    int64_t groups = ((int64_t)1 << 18) / lanes_per_row;
    groups = groups < 1 ? 1 : (groups > n_rows ? n_rows : groups);
    const int64_t total = lanes_per_row * groups;
    hipLaunchKernelGGL(rope_kv_append_vec_kernel<T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, p,
                       (int)groups);
    return tl_launch_status();
  }
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
