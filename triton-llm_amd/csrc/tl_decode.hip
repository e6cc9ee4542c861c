// Single-token decode attention over a resident KV cache: split-K pass plus a
// log-sum-exp combine.
//
// Reference behaviour being replaced: per decode step the reference runs
// attention_gqa(q, K[:L], V[:L], causal=False) (smollm2_triton/model.py:310-314)
// whose kernel (attention_gqa.py:21-146) launches one program per query head,
// re-reading each KV head once per query head of its group.  Here one
// workgroup owns (sequence b, KV head, split of the positions) and serves all
// G query heads of that KV head from a single pass over K/V.
//
// Work layout inside a workgroup (256 threads = 4 waves):
//   * a key row (d_k elements) is read by 16 consecutive lanes, EPL = d_k/16
//     elements each, so one wave load instruction covers 4 consecutive rows
//     (1 KiB contiguous for d_k = 128 bf16);
//   * the 16 lane-groups of the workgroup are 16 independent key streams
//     (stream s takes keys start + s, start + s + 16, ...), each keeping its
//     own online-softmax state (max m, sum l, accumulator) in the log2 domain;
//   * U keys per stream are loaded before any is consumed so each lane keeps
//     2*U row slices in flight;
//   * at the end the 16 streams are merged (lane shuffles, then LDS) and the
//     split's (m, l, acc[d_k]) is written to the workspace.
// The combine kernel merges the splits of each (b, query head) and
// normalises, as the reference's final acc / row_sum (attention_gqa.py:143).
#include "tl_common.h"

#include <math.h>

namespace {

constexpr int kThreads = 256;
constexpr int kStreams = 16;  // lane-groups per workgroup
constexpr int kUnroll = 4;    // keys in flight per stream

template <typename T, int EPL>
struct RowSlice {
  static constexpr int kBytes = EPL * T::size;
  static constexpr int kWords = kBytes / 4;
  static_assert(kBytes % 4 == 0, "row slice must be whole 32-bit words");
  uint32_t w[kWords];

  __device__ __forceinline__ void load(const void* ptr) {
    if constexpr (kWords % 4 == 0) {
#pragma unroll
      for (int i = 0; i < kWords / 4; ++i) {
        u32x4 v = ((const u32x4*)ptr)[i];
        w[4 * i + 0] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
      }
    } else if constexpr (kWords == 2) {
      u32x2 v = *(const u32x2*)ptr;
      w[0] = v.x; w[1] = v.y;
    } else {
      w[0] = *(const uint32_t*)ptr;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int i = 0; i < kWords; ++i) w[i] = 0u;
  }
  __device__ __forceinline__ void to_float(float (&f)[EPL]) const {
    if constexpr (T::size == 4) {
#pragma unroll
      for (int i = 0; i < EPL; ++i) f[i] = __uint_as_float(w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kWords; ++i) unpack2<T>(w[i], f[2 * i], f[2 * i + 1]);
    }
  }
};

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* lens;
  float* ws_ml;   // [B][Hq][max_splits][2]  (m in log2 domain, l)
  float* ws_acc;  // [B][Hq][max_splits][D]  unnormalised
  void* o;
  int len_add;
  int batch, n_head, n_kv, group, max_ctx, split, max_splits;
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh;
  float scale_log2;  // sm_scale * log2(e)
};

__device__ __forceinline__ int ctx_len(const DecodeParams& p, int b) {
  int c = p.lens[b] + p.len_add;
  c = c < 0 ? 0 : c;
  return c > p.max_ctx ? p.max_ctx : c;
}

// Merge (m2, l2, a2) into (m, l, a); m values are log2-domain maxima.
__device__ __forceinline__ void merge_weights(float m, float m2, float& w1, float& w2, float& mn) {
  mn = fmaxf(m, m2);
  const float base = (mn == -INFINITY) ? 0.f : mn;
  w1 = fast_exp2(m - base);
  w2 = fast_exp2(m2 - base);
}

// G: query heads handled by this workgroup (<= group); blockIdx.y encodes
// (kv head, head chunk).
template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams p) {
  constexpr int EPL = D / 16;
  using Slice = RowSlice<T, EPL>;
  using Bits = typename T::bits;

  const int split = blockIdx.x;
  const int b = blockIdx.z;
  const int n_chunks = (p.group + G - 1) / G;
  const int hkv = blockIdx.y / n_chunks;
  const int hq0 = hkv * p.group + (blockIdx.y - hkv * n_chunks) * G;
  const int n_g = min(G, hkv * p.group + p.group - hq0);  // heads valid in this chunk

  const int ctx = ctx_len(p, b);
  const int start = split * p.split;
  if (start >= ctx) return;  // this split is past the sequence end
  const int end = min(ctx, start + p.split);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane & 15;
  const int stream = wave * 4 + (lane >> 4);

  // Query slices for the G heads (fp32).
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Slice s;
    if (g < n_g) {
      s.load((const Bits*)p.q + b * p.q_sb + (int64_t)(hq0 + g) * p.q_sh + sub * EPL);
    } else {
      s.zero();
    }
    s.to_float(qf[g]);
  }

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  const Bits* kbase = (const Bits*)p.k + b * p.k_sb + hkv * p.k_sh + sub * EPL;
  const Bits* vbase = (const Bits*)p.v + b * p.v_sb + hkv * p.v_sh + sub * EPL;
  const float c = p.scale_log2;
  const int n_iter = (end - start + kStreams * kUnroll - 1) / (kStreams * kUnroll);

  for (int it = 0; it < n_iter; ++it) {
    const int key0 = start + it * (kStreams * kUnroll) + stream;
    Slice kr[kUnroll], vr[kUnroll];
    bool valid[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int key = key0 + u * kStreams;
      valid[u] = key < end;
      if (valid[u]) {
        kr[u].load(kbase + (int64_t)key * p.k_ss);
        vr[u].load(vbase + (int64_t)key * p.v_ss);
      } else {
        kr[u].zero();
        vr[u].zero();
      }
    }
    float s[G][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float kf[EPL];
      kr[u].to_float(kf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) d = fmaf(qf[g][e], kf[e], d);
        d = row16_sum(d);
        s[g][u] = valid[u] ? d * c : -INFINITY;
      }
    }
    float vf[kUnroll][EPL];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) vr[u].to_float(vf[u]);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mb = s[g][0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mb = fmaxf(mb, s[g][u]);
      const float mn = fmaxf(m[g], mb);
      const float base = (mn == -INFINITY) ? 0.f : mn;
      const float alpha = fast_exp2(m[g] - base);
      m[g] = mn;
      l[g] *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float pu = fast_exp2(s[g][u] - base);
        l[g] += pu;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pu, vf[u][e], acc[g][e]);
      }
    }
  }

  // Merge the 4 streams of this wave (lane groups 16 apart).
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m2 = __shfl_xor(m[g], off);
      const float l2 = __shfl_xor(l[g], off);
      float w1, w2, mn;
      merge_weights(m[g], m2, w1, w2, mn);
      m[g] = mn;
      l[g] = l[g] * w1 + l2 * w2;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float a2 = __shfl_xor(acc[g][e], off);
        acc[g][e] = acc[g][e] * w1 + a2 * w2;
      }
    }
  }

  // Merge the 4 waves through LDS.
  __shared__ float s_m[4][G], s_l[4][G];
  __shared__ float s_acc[4][G][D];
  if (lane < 16) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (lane == 0) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[wave][g][sub * EPL + e] = acc[g][e];
    }
  }
  __syncthreads();
  const int64_t row_base = ((int64_t)b * p.n_head + hq0) * p.max_splits + split;
  for (int idx = tid; idx < n_g * D; idx += kThreads) {
    const int g = idx / D;
    const int d = idx - g * D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_m[w][g]);
    const float base = (mx == -INFINITY) ? 0.f : mx;
    float a = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wt = fast_exp2(s_m[w][g] - base);
      a += s_acc[w][g][d] * wt;
      lsum += s_l[w][g] * wt;
    }
    const int64_t row = row_base + (int64_t)g * p.max_splits;
    p.ws_acc[row * D + d] = a;
    if (d == 0) {
      p.ws_ml[row * 2 + 0] = mx;
      p.ws_ml[row * 2 + 1] = lsum;
    }
  }
}

// One workgroup per (b, query head): merge the splits and normalise.
template <typename T, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
  using Bits = typename T::bits;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int ctx = ctx_len(p, b);
  Bits* out = (Bits*)p.o + b * p.o_sb + (int64_t)hq * p.o_sh;
  if (ctx == 0) {
    // Nothing to attend to: zeros, the reference's empty-KV result
    // (tests/test_attention_gqa.py:297).
    for (int d = threadIdx.x; d < D; d += 64) out[d] = from_f32<T>(0.f);
    return;
  }
  const int n_split = (ctx + p.split - 1) / p.split;
  const int64_t row0 = ((int64_t)b * p.n_head + hq) * p.max_splits;
  float mx = -INFINITY;
  for (int s = 0; s < n_split; ++s) mx = fmaxf(mx, p.ws_ml[(row0 + s) * 2]);
  const float base = (mx == -INFINITY) ? 0.f : mx;
  float lsum = 0.f;
  float a[(D + 63) / 64];
#pragma unroll
  for (int j = 0; j < (D + 63) / 64; ++j) a[j] = 0.f;
  for (int s = 0; s < n_split; ++s) {
    const float wt = fast_exp2(p.ws_ml[(row0 + s) * 2] - base);
    lsum += p.ws_ml[(row0 + s) * 2 + 1] * wt;
#pragma unroll
    for (int j = 0; j < (D + 63) / 64; ++j) {
      const int d = threadIdx.x + 64 * j;
      if (d < D) a[j] += p.ws_acc[(row0 + s) * D + d] * wt;
    }
  }
  const float inv = 1.f / lsum;
#pragma unroll
  for (int j = 0; j < (D + 63) / 64; ++j) {
    const int d = threadIdx.x + 64 * j;
    if (d < D) out[d] = from_f32<T>(a[j] * inv);
  }
}

template <typename T, int D, int G>
int launch_decode_g(const DecodeParams& p, hipStream_t st) {
  const int n_chunks = (p.group + G - 1) / G;
  dim3 grid(p.max_splits, p.n_kv * n_chunks, p.batch);
  hipLaunchKernelGGL((decode_split_kernel<T, D, G>), grid, dim3(kThreads), 0, st, p);
  int e = tl_launch_status();
  if (e) return e;
  hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3(p.n_head, p.batch), dim3(64), 0, st, p);
  return tl_launch_status();
}

template <typename T, int D>
int launch_decode_d(const DecodeParams& p, hipStream_t st) {
  switch (p.group) {
    case 1: return launch_decode_g<T, D, 1>(p, st);
    case 2: return launch_decode_g<T, D, 2>(p, st);
    case 3: return launch_decode_g<T, D, 3>(p, st);
    case 4: return launch_decode_g<T, D, 4>(p, st);
    case 5: return launch_decode_g<T, D, 5>(p, st);
    case 6: return launch_decode_g<T, D, 6>(p, st);
    case 7: return launch_decode_g<T, D, 7>(p, st);
    default: return launch_decode_g<T, D, 8>(p, st);  // groups > 8 run in chunks of 8
  }
}

template <typename T>
int launch_decode_t(const DecodeParams& p, int d_k, hipStream_t st) {
  switch (d_k) {
    case 64: return launch_decode_d<T, 64>(p, st);
    case 128: return launch_decode_d<T, 128>(p, st);
    default: return TL_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" {

int tl_decode_split_size(int batch, int n_kv_head, int max_ctx) {
  // Aim for a few thousand workgroups: enough to fill 256 CUs several times
  // over while keeping each split long enough to amortise its partial write.
  const int64_t heads = (int64_t)batch * (n_kv_head > 0 ? n_kv_head : 1);
  int split = 64;
  while (split < 2048 && heads * ((max_ctx + 2 * split - 1) / (2 * split)) >= 4096) split *= 2;
  return split;
}

size_t tl_attention_decode_workspace_bytes(int batch, int n_head, int max_ctx,
                                           int d_k, int split_size) {
  if (batch <= 0 || n_head <= 0 || max_ctx <= 0 || d_k <= 0 || split_size <= 0) return 0;
  const size_t splits = (size_t)((max_ctx + split_size - 1) / split_size);
  const size_t rows = (size_t)batch * n_head * splits;
  // ml block first, then acc; both 256-byte aligned.
  const size_t ml = (rows * 2 * sizeof(float) + 255) & ~(size_t)255;
  return ml + rows * (size_t)d_k * sizeof(float);
}

int tl_attention_decode(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* cache_lens, int len_add, void* o,
                        void* workspace, size_t workspace_bytes, int batch,
                        int n_head, int n_kv_head, int max_ctx, int d_k,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        float sm_scale, int split_size, int dtype,
                        void* stream) {
  if (batch == 0 || n_head == 0) return 0;
  if (!q || !k_cache || !v_cache || !cache_lens || !o || !workspace || batch < 0 ||
      n_head < 0 || n_kv_head < 1 || n_head % n_kv_head != 0 || max_ctx < 1 ||
      !q_strides || !k_strides || !v_strides || !o_strides)
    return TL_ERR_INVALID;
  if (split_size == 0) split_size = tl_decode_split_size(batch, n_kv_head, max_ctx);
  if (split_size < 16 || split_size % 16 != 0) return TL_ERR_INVALID;
  if (workspace_bytes < tl_attention_decode_workspace_bytes(batch, n_head, max_ctx, d_k, split_size))
    return TL_ERR_INVALID;
  DecodeParams p{};
  p.q = q;
  p.k = k_cache;
  p.v = v_cache;
  p.lens = cache_lens;
  p.o = o;
  p.len_add = len_add;
  p.batch = batch;
  p.n_head = n_head;
  p.n_kv = n_kv_head;
  p.group = n_head / n_kv_head;
  p.max_ctx = max_ctx;
  p.split = split_size;
  p.max_splits = (max_ctx + split_size - 1) / split_size;
  const size_t rows = (size_t)batch * n_head * p.max_splits;
  p.ws_ml = (float*)workspace;
  p.ws_acc = (float*)((char*)workspace + ((rows * 2 * sizeof(float) + 255) & ~(size_t)255));
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.k_ss = k_strides[2];
  p.v_sb = v_strides[0];
  p.v_sh = v_strides[1];
  p.v_ss = v_strides[2];
  p.o_sb = o_strides[0];
  p.o_sh = o_strides[1];
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  // Each lane loads d_k/16 contiguous elements with one vector load, so
  // every row start must be aligned to that slice.
  const int esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  const int64_t slice = d_k / 16;
  const uintptr_t align = (uintptr_t)(slice * esize);
  const int64_t st_all[] = {p.q_sb, p.q_sh, p.k_sb, p.k_sh, p.k_ss, p.v_sb, p.v_sh, p.v_ss};
  for (int64_t s : st_all)
    if (slice == 0 || s % slice) return TL_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % align) return TL_ERR_UNSUPPORTED;
  if (((uintptr_t)workspace) % 16) return TL_ERR_INVALID;
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: return launch_decode_t<F32>(p, d_k, st);
    case TL_DTYPE_F16: return launch_decode_t<F16>(p, d_k, st);
    case TL_DTYPE_BF16: return launch_decode_t<BF16>(p, d_k, st);
    default: return TL_ERR_INVALID;
  }
}

}  // extern "C"
