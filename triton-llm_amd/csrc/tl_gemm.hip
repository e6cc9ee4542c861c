// Dense projections of the model step: C = A . B on the library stream.
//
// Reference behaviour being replaced: triton_llm/kernels/gemm.py:14-108, a
// Triton fp32 tile GEMM (64 x 64 x 32 blocks, tl.dot) used for every
// projection of the model (q/k/v/o, gate/up/down, lm_head).
//
// Two regimes:
//   * a prompt (m > kSkinnyMaxM rows) is a plain compute-bound GEMM: it goes
//     to rocBLAS (Tensile's gfx950 MFMA kernels), fp32 accumulation.
//     Row-major operands map onto column-major rocBLAS as C^T = B^T . A^T
//     with no copies.  rocBLAS keeps one handle per device (created on first
//     use), which owns rocBLAS's own small device workspace.
//   * a decoded token (m <= kSkinnyMaxM rows) reads every weight once for a
//     handful of multiply-adds per element: an HBM-bound skinny product,
//     where rocBLAS measured 0.4-0.7 TB/s.  skinny_partial_kernel cuts B
//     into (64-column x TK-row) tiles, about a thousand of them, so enough
//     weight bytes are in flight to stream at HBM speed; each tile's
//     partial sums go to the workspace and skinny_reduce_kernel adds the
//     K-slices and rounds to the output type.
#include "tl_common.h"

#include <rocblas/rocblas.h>

#include <mutex>

namespace {

constexpr int kSkinnyMaxM = 8;     // rows of A handled by the skinny path
constexpr int kSkThreads = 256;    // 4 waves
constexpr int kSkUnroll = 16;      // row loads in flight per lane
constexpr int kSkMaxTk = 1024;     // rows per K-slice at most (A's slice is staged in LDS)
constexpr int kSkRowsPerStep = 16; // rows one workgroup load instruction round covers
constexpr int kSkTargetTiles = 1024;
constexpr int kAuxNt = 2;          // buffer-load cache policy: nontemporal (weights are read once)

constexpr int kMaxDevices = 64;
rocblas_handle g_handles[kMaxDevices] = {};
std::mutex g_handle_mu;

rocblas_handle device_handle() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_handle_mu);
  if (!g_handles[dev] && rocblas_create_handle(&g_handles[dev]) != rocblas_status_success) g_handles[dev] = nullptr;
  return g_handles[dev];
}

bool fits_int(int64_t x) { return x >= 0 && x <= INT32_MAX; }

// Skinny tiling: 64 fp32 (or 128 16-bit) columns per tile -- 16 lanes x 16
// bytes per row -- and TK rows, TK a multiple of the 16 rows one workgroup
// load round covers, chosen for about kSkTargetTiles tiles.  (A slice that
// ends inside an unrolled step loads zeros past its end, with no memory
// access.)
struct SkinnyPlan {
  int cols;     // columns per tile
  int n_tiles;  // column tiles
  int tk;       // rows per K-slice
  int ks;       // K-slices
};

SkinnyPlan skinny_plan(int n, int k, int esize) {
  SkinnyPlan s;
  s.cols = 256 / esize;
  s.n_tiles = (n + s.cols - 1) / s.cols;
  const int step = kSkRowsPerStep;
  const int ks_target = kSkTargetTiles / s.n_tiles > 1 ? kSkTargetTiles / s.n_tiles : 1;
  int tk = (k + ks_target - 1) / ks_target;
  tk = (tk + step - 1) / step * step;
  tk = tk < kSkMaxTk ? tk : kSkMaxTk;
  s.tk = tk;
  s.ks = (k + tk - 1) / tk;
  return s;
}

size_t skinny_workspace_bytes(int m, int n, int k, int esize) {
  const SkinnyPlan s = skinny_plan(n, k, esize);
  return (size_t)s.ks * m * n * sizeof(float);
}

template <typename T>
__device__ __forceinline__ void unpack_words(const u32x4& w, float (&f)[16 / T::size]) {
  if constexpr (T::size == 4) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y); f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  } else {
    unpack2<T>(w.x, f[0], f[1]); unpack2<T>(w.y, f[2], f[3]); unpack2<T>(w.z, f[4], f[5]); unpack2<T>(w.w, f[6], f[7]);
  }
}

// One workgroup: K-slice blockIdx.y (rows [k0, k0 + tk)) x column tile
// blockIdx.x.  Lane (wave w, row group r = lane / 16, chunk c = lane % 16)
// reads 16 bytes of row k0 + 16 i + 4 w + r, columns chunk c; its MT x CPC
// sums cover the rows it read.  The four row groups of a wave, then the four
// waves, are added up and the slice's partial product is stored.
// With a single K-slice (gridDim.y == 1) the sums are the result: they are
// rounded and stored to C directly, and no reduce pass follows.
template <typename T, int MT>
__global__ __launch_bounds__(kSkThreads) void skinny_partial_kernel(const void* __restrict__ a, const void* __restrict__ b,
                                                                     float* __restrict__ ws, void* __restrict__ out,
                                                                     int m, int n, int k, int64_t lda, int64_t ldb,
                                                                     int64_t ldc, int tk) {
  constexpr int CPC = 16 / T::size;  // columns per 16-byte chunk
  constexpr int COLS = 16 * CPC;     // columns per tile
  using Bits = typename T::bits;
  __shared__ float s_a[MT][kSkMaxTk];
  __shared__ float s_sum[4][MT][COLS];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r = lane >> 4, c = lane & 15;
  const int k0 = blockIdx.y * tk;
  const int k1 = min(k, k0 + tk);
  // The tile's rows of B as one buffer that ends at the last row's last
  // column inside the matrix: loads of rows past the slice read zeros with no
  // memory access.  (Chunks past column n of earlier rows read the next
  // row's data; those columns are never stored.)
  const int tile_col0 = blockIdx.x * COLS;
  const Bits* bbase = (const Bits*)b + (int64_t)k0 * ldb + tile_col0;
  const int rows = k1 - k0;
  const int last_cols = min(COLS, n - tile_col0);
  const uint32_t nbytes = (uint32_t)((int64_t)(rows - 1) * ldb * T::size + (int64_t)last_cols * T::size);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)bbase, (short)0, (int)nbytes, kBufRsrcWord3);
  const uint32_t row_bytes = (uint32_t)(ldb * T::size);
  float acc[MT][CPC];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < CPC; ++j) acc[i][j] = 0.f;
  u32x4 w[kSkUnroll];
  auto load_round = [&](int kb) {
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      const int row = kb + kSkRowsPerStep * u + 4 * wave + r;  // row within the slice
      w[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)row * row_bytes + (uint32_t)(c * 16), 0, kAuxNt));
    }
  };
  // The first round's weight loads go out before A's slice is staged, so
  // the two latencies overlap.
  load_round(0);
  for (int idx = tid; idx < MT * rows; idx += kSkThreads) {
    const int mi = idx / rows, kk = idx - mi * rows;
    s_a[mi][kk] = mi < m ? to_f32<T>(((const Bits*)a)[(int64_t)mi * lda + k0 + kk]) : 0.f;
  }
  __syncthreads();
  for (int kb = 0; kb < rows; kb += kSkRowsPerStep * kSkUnroll) {
    if (kb > 0) load_round(kb);
#pragma unroll
    for (int u = 0; u < kSkUnroll; ++u) {
      float f[CPC];
      unpack_words<T>(w[u], f);
      const int kk = kb + kSkRowsPerStep * u + 4 * wave + r;
      if (kk < rows) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const float x = s_a[i][kk];
#pragma unroll
          for (int j = 0; j < CPC; ++j) acc[i][j] = fmaf(x, f[j], acc[i][j]);
        }
      }
    }
  }
  // Row groups of the wave (lanes 16 apart), then the waves through LDS.
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < CPC; ++j) {
      float v = acc[i][j];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[i][j] = v;
    }
  __syncthreads();
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < CPC; ++j) s_sum[wave][i][c * CPC + j] = acc[i][j];
  }
  __syncthreads();
  for (int idx = tid; idx < MT * COLS; idx += kSkThreads) {
    const int mi = idx / COLS, cc = idx % COLS;
    const int col = blockIdx.x * COLS + cc;
    if (mi < m && col < n) {
      const float v = s_sum[0][mi][cc] + s_sum[1][mi][cc] + s_sum[2][mi][cc] + s_sum[3][mi][cc];
      if (gridDim.y == 1)
        ((Bits*)out)[(int64_t)mi * ldc + col] = from_f32<T>(v);
      else
        ws[((int64_t)blockIdx.y * m + mi) * n + col] = v;
    }
  }
}

// C[mi][col] = sum over K-slices of the partials, rounded to T.  Eight
// slices' loads are in flight at a time (the sum is latency-bound).
template <typename T>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ ws, void* __restrict__ c, int m,
                                                            int n, int64_t ldc, int ks) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)m * n) return;
  const int mi = (int)(idx / n), col = (int)(idx % n);
  const int64_t stride = (int64_t)m * n;
  float s = 0.f;
  for (int q0 = 0; q0 < ks; q0 += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = q0 + j < ks ? ws[(int64_t)(q0 + j) * stride + idx] : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[j];
  }
  ((typename T::bits*)c)[(int64_t)mi * ldc + col] = from_f32<T>(s);
}

template <typename T>
int launch_skinny(const void* a, const void* b, void* c, int m, int n, int k, int64_t lda, int64_t ldb, int64_t ldc,
                  void* ws, hipStream_t st) {
  const SkinnyPlan s = skinny_plan(n, k, T::size);
  dim3 grid((unsigned)s.n_tiles, (unsigned)s.ks);
  if (m <= 1)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 1>), grid, dim3(kSkThreads), 0, st, a, b, (float*)ws, c, m, n, k, lda, ldb,
                       ldc, s.tk);
  else if (m <= 2)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 2>), grid, dim3(kSkThreads), 0, st, a, b, (float*)ws, c, m, n, k, lda, ldb,
                       ldc, s.tk);
  else if (m <= 4)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 4>), grid, dim3(kSkThreads), 0, st, a, b, (float*)ws, c, m, n, k, lda, ldb,
                       ldc, s.tk);
  else
    hipLaunchKernelGGL((skinny_partial_kernel<T, 8>), grid, dim3(kSkThreads), 0, st, a, b, (float*)ws, c, m, n, k, lda, ldb,
                       ldc, s.tk);
  int e = tl_launch_status();
  if (e || s.ks == 1) return e;
  const int64_t outs = (int64_t)m * n;
  hipLaunchKernelGGL((skinny_reduce_kernel<T>), dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st,
                     (const float*)ws, c, m, n, ldc, s.ks);
  return tl_launch_status();
}

}  // namespace

extern "C" {

size_t tl_gemm_workspace_bytes(int m, int n, int k, int dtype) {
  if (m <= 0 || n <= 0 || k <= 0 || m > kSkinnyMaxM) return 0;
  return skinny_workspace_bytes(m, n, k, dtype == TL_DTYPE_F32 ? 4 : 2);
}

int tl_gemm(const void* a, const void* b, void* c, int m, int n, int k, int64_t lda, int64_t ldb, int64_t ldc,
            void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  if (m < 0 || n < 0 || k < 0) return TL_ERR_INVALID;
  if (dtype != TL_DTYPE_F32 && dtype != TL_DTYPE_F16 && dtype != TL_DTYPE_BF16) return TL_ERR_INVALID;
  if (m == 0 || n == 0) return 0;
  if (!c || ldc < n || (k > 0 && (!a || !b || lda < k || ldb < n))) return TL_ERR_INVALID;
  if (!fits_int(lda) || !fits_int(ldb) || !fits_int(ldc)) return TL_ERR_UNSUPPORTED;
  const size_t esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  hipStream_t st = tl_resolve_stream(stream);
  if (k == 0) {  // empty sum: zeros, row by row when C is a strided view
    return (int)hipMemset2DAsync(c, (size_t)ldc * esize, 0, (size_t)n * esize, (size_t)m, st);
  }
  if (m <= kSkinnyMaxM) {
    if (!workspace || workspace_bytes < tl_gemm_workspace_bytes(m, n, k, dtype)) return TL_ERR_INVALID;
    // 16-byte row chunks: the row stride and the row length must keep chunks aligned.
    const int cpc = 16 / (int)esize;
    if (n % cpc == 0 && ldb % cpc == 0 && ((uintptr_t)b % 16) == 0 && (int64_t)(k - 1) * ldb * esize < INT32_MAX) {
      switch (dtype) {
        case TL_DTYPE_F32: return launch_skinny<F32>(a, b, c, m, n, k, lda, ldb, ldc, workspace, st);
        case TL_DTYPE_F16: return launch_skinny<F16>(a, b, c, m, n, k, lda, ldb, ldc, workspace, st);
        default: return launch_skinny<BF16>(a, b, c, m, n, k, lda, ldb, ldc, workspace, st);
      }
    }
  }
  rocblas_handle h = device_handle();
  if (!h) return TL_ERR_INVALID;
  if (rocblas_set_stream(h, st) != rocblas_status_success) return TL_ERR_INVALID;
  const float alpha = 1.f, beta = 0.f;
  const rocblas_datatype t = dtype == TL_DTYPE_F32   ? rocblas_datatype_f32_r
                             : dtype == TL_DTYPE_F16 ? rocblas_datatype_f16_r
                                                     : rocblas_datatype_bf16_r;
  // Column-major view: C^T (n x m, ld ldc) = B^T (n x k, ld ldb) . A^T (k x m, ld lda).
  const rocblas_status s = rocblas_gemm_ex(h, rocblas_operation_none, rocblas_operation_none, n, m, k, &alpha, b, t,
                                           (rocblas_int)ldb, a, t, (rocblas_int)lda, &beta, c, t, (rocblas_int)ldc, c,
                                           t, (rocblas_int)ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  if (s != rocblas_status_success) return s == rocblas_status_invalid_size ? TL_ERR_UNSUPPORTED : TL_ERR_INVALID;
  return tl_launch_status();
}

}  // extern "C"
