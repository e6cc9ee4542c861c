// Single-token decode attention over a resident KV cache: a split-K pass and
// a log-sum-exp combine of the splits.
//
// Reference behaviour being replaced: per decode step the reference runs
// attention_gqa(q, K[:L], V[:L], causal=False) (smollm2_triton/model.py:310-314)
// whose kernel (attention_gqa.py:21-146) launches one program per query head,
// re-reading each KV head once per query head of its group.  Here one
// workgroup owns (sequence b, KV head, split of the positions) and serves all
// G query heads of that KV head from a single pass over K/V.
//
// The pass is HBM-bound (every K/V byte is read exactly once), so the design
// goal is to keep the VALU work per byte well under the issue budget:
//   * a key row (d_k elements) is read by 16 consecutive lanes with one
//     16-byte (or 8/32-byte) nontemporal buffer load each, so one wave load
//     covers 4 consecutive rows; the row offset lives in one 32-bit VGPR and
//     the per-unroll step in an SGPR (no 64-bit address math per load);
//   * q.k of 16-bit types uses packed dot2 (v_dot2c_f32_bf16 / _f16) straight
//     on the stored words; the 16-lane row sum is 4 DPP-fused adds;
//   * the 16 lane-groups of the workgroup are 16 independent key streams
//     (stream s takes keys start + s, start + s + 16, ...), each keeping its
//     own online-softmax state (max m, sum l, accumulator) in the log2 domain,
//     rescaled lazily: only when a new score exceeds the running max by
//     2^kRescaleLog2 (exact either way -- the max only bounds exponent range);
//   * full 64-key iterations run without masks; one masked iteration takes
//     the remainder.
// At the end the 16 streams are merged (lane shuffles, then LDS).  A sequence
// that fits one split writes its normalised output directly; otherwise each
// split stores (m, l, acc[d_k]) to the workspace and a second, small kernel
// merges the splits and normalises (attention_gqa.py:143 acc / row_sum).
// The merge is a separate launch on purpose: on MI355X each XCD has its own
// L2, so a device-scope fence inside the split kernel (to let the last
// workgroup combine) writes back and invalidates the whole L2 per workgroup,
// which costs far more than one extra launch.
#include "tl_common.h"

#include <math.h>

#include <type_traits>

namespace {

constexpr int kThreads = 256;
constexpr int kStreams = 16;  // lane-groups per workgroup
constexpr int kUnroll = 4;    // keys in flight per stream
constexpr int kKeysPerIter = kStreams * kUnroll;
constexpr float kRescaleLog2 = 8.f;
constexpr int kAuxNontemporal = 2;  // buffer-load cache policy: nt

template <int W>
struct Slice {
  uint32_t w[W];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufRsrcWord3);
}

// Nontemporal load of one W-word row slice at byte offset voff + soff.
template <int W>
__device__ __forceinline__ void load_slice(Slice<W>& s, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff) {
  if constexpr (W == 2) {
    u32x2 a = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kAuxNontemporal));
    s.w[0] = a.x; s.w[1] = a.y;
  } else {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      u32x4 a = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16 * i, soff, kAuxNontemporal));
      s.w[4 * i + 0] = a.x; s.w[4 * i + 1] = a.y; s.w[4 * i + 2] = a.z; s.w[4 * i + 3] = a.w;
    }
  }
}

// Partial dot product of a query slice and a key slice (same storage type).
template <typename T, int W>
__device__ __forceinline__ float dot_slice(const Slice<W>& q, const Slice<W>& k) {
  float d = 0.f;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    if constexpr (T::code == TL_DTYPE_BF16) {
      d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q.w[i]),
                                          __builtin_bit_cast(bf16x2, k.w[i]), d, false);
    } else if constexpr (T::code == TL_DTYPE_F16) {
      d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, q.w[i]), __builtin_bit_cast(f16x2, k.w[i]), d,
                                 false);
    } else {
      d = fmaf(__uint_as_float(q.w[i]), __uint_as_float(k.w[i]), d);
    }
  }
  return d;
}

template <typename T, int W, int EPL>
__device__ __forceinline__ void slice_to_float(const Slice<W>& s, float (&f)[EPL]) {
  if constexpr (T::size == 4) {
#pragma unroll
    for (int i = 0; i < EPL; ++i) f[i] = __uint_as_float(s.w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) unpack2<T>(s.w[i], f[2 * i], f[2 * i + 1]);
  }
}

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
  int64_t k_sb, k_sh;
  int64_t v_sb, v_sh;
  uint32_t k_row_bytes, v_row_bytes;        // seq strides in bytes
  uint32_t k_region_bytes, v_region_bytes;  // bytes addressable from one (b, head) base
  int64_t o_sb, o_sh;
  float scale_log2;  // sm_scale * log2(e)
};

__device__ __forceinline__ int ctx_len(const DecodeParams& p, int b) {
  int c = p.lens[b] + p.len_add;
  c = c < 0 ? 0 : c;
  return c > p.max_ctx ? p.max_ctx : c;
}

// Weights that merge two log2-domain (max, sum) states into max mn.
__device__ __forceinline__ void merge_weights(float m, float m2, float& w1, float& w2, float& mn) {
  mn = fmaxf(m, m2);
  const float base = (mn == -INFINITY) ? 0.f : mn;
  w1 = fast_exp2(m - base);
  w2 = fast_exp2(m2 - base);
}

template <typename T>
__device__ __forceinline__ void store_out(void* base, int64_t idx, float x) {
  ((typename T::bits*)base)[idx] = from_f32<T>(x);
}

// G: query heads handled by this workgroup (<= group); blockIdx.y encodes
// (kv head, head chunk).
template <typename T, int D, int G>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams p) {
  constexpr int EPL = D / 16;           // elements per lane per row
  constexpr int W = EPL * T::size / 4;  // 32-bit words per lane per row
  using Bits = typename T::bits;

  const int split = blockIdx.x;
  const int b = blockIdx.z;
  const int n_chunks = (p.group + G - 1) / G;
  const int hkv = blockIdx.y / n_chunks;
  const int hq0 = hkv * p.group + (blockIdx.y - hkv * n_chunks) * G;
  const int n_g = min(G, hkv * p.group + p.group - hq0);  // heads valid in this chunk

  const int tid = threadIdx.x;
  const int ctx = ctx_len(p, b);
  if (ctx == 0) {
    // Nothing to attend to: zeros, the reference's empty-KV result
    // (tests/test_attention_gqa.py:297).
    if (split == 0)
      for (int idx = tid; idx < n_g * D; idx += kThreads)
        store_out<T>(p.o, b * p.o_sb + (int64_t)(hq0 + idx / D) * p.o_sh + idx % D, 0.f);
    return;
  }
  const int start = split * p.split;
  if (start >= ctx) return;  // this split is past the sequence end
  const int end = min(ctx, start + p.split);
  const int n_split = (ctx + p.split - 1) / p.split;

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane & 15;
  const int stream = wave * 4 + (lane >> 4);

  // Query slices of the G heads, kept in storage format.
  Slice<W> qs[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint32_t* src = (const uint32_t*)((const Bits*)p.q + b * p.q_sb +
                                            (int64_t)min(hq0 + g, hq0 + n_g - 1) * p.q_sh + sub * EPL);
#pragma unroll
    for (int i = 0; i < W; ++i) qs[g].w[i] = (g < n_g) ? src[i] : 0u;
  }

  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[g][e] = 0.f;
  }

  const __amdgpu_buffer_rsrc_t krs = make_rsrc((const Bits*)p.k + b * p.k_sb + hkv * p.k_sh, p.k_region_bytes);
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc((const Bits*)p.v + b * p.v_sb + hkv * p.v_sh, p.v_region_bytes);
  const uint32_t lane_bytes = sub * (EPL * T::size);
  const float c = p.scale_log2;

  // One iteration: kUnroll keys per stream, 64 per workgroup.
  auto iteration = [&](int key0, auto masked) {
    constexpr bool kMasked = decltype(masked)::value;
    Slice<W> kr[kUnroll], vr[kUnroll];
    bool valid[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int key = key0 + u * kStreams;
      if constexpr (kMasked) {
        // Out-of-range keys re-read this split's first row (always inside
        // the sequence) and are masked out of the softmax below.
        valid[u] = key < end;
        const uint32_t row = valid[u] ? key : start;
        load_slice(kr[u], krs, row * p.k_row_bytes + lane_bytes, 0);
        load_slice(vr[u], vrs, row * p.v_row_bytes + lane_bytes, 0);
      } else {
        valid[u] = true;
        load_slice(kr[u], krs, (uint32_t)key0 * p.k_row_bytes + lane_bytes, u * kStreams * p.k_row_bytes);
        load_slice(vr[u], vrs, (uint32_t)key0 * p.v_row_bytes + lane_bytes, u * kStreams * p.v_row_bytes);
      }
    }
    float s[G][kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = row16_sum(dot_slice<T>(qs[g], kr[u])) * c;
        s[g][u] = (!kMasked || valid[u]) ? d : -INFINITY;
      }
    }
    // Lazy rescale: move the running max only when a score would exceed it
    // by more than 2^kRescaleLog2.
    bool grow = false;
    float mb[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mb[g] = s[g][0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mb[g] = fmaxf(mb[g], s[g][u]);
      grow |= mb[g] > m[g] + kRescaleLog2;
    }
    if (__any(grow)) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float mn = fmaxf(m[g], mb[g]);
        const float alpha = fast_exp2(m[g] - ((mn == -INFINITY) ? 0.f : mn));
        m[g] = mn;
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
      }
    }
    float pu[G][kUnroll];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float base = (m[g] == -INFINITY) ? 0.f : m[g];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        pu[g][u] = fast_exp2(s[g][u] - base);
        l[g] += pu[g][u];
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      float vf[EPL];
      slice_to_float<T>(vr[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pu[g][u], vf[e], acc[g][e]);
    }
  };

  const int n_full = (end - start) / kKeysPerIter;
  int key0 = start + stream;
  for (int it = 0; it < n_full; ++it, key0 += kKeysPerIter) iteration(key0, std::false_type{});
  if (start + n_full * kKeysPerIter < end) iteration(key0, std::true_type{});

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
  const int64_t row_base = ((int64_t)b * p.n_head + hq0) * p.max_splits;
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
    if (n_split == 1) {
      store_out<T>(p.o, b * p.o_sb + (int64_t)(hq0 + g) * p.o_sh + d, a / lsum);
    } else {
      const int64_t row = row_base + (int64_t)g * p.max_splits + split;
      p.ws_acc[row * D + d] = a;
      if (d == 0) {
        p.ws_ml[row * 2 + 0] = mx;
        p.ws_ml[row * 2 + 1] = lsum;
      }
    }
  }
}

// One workgroup per (b, query head): merge the splits and normalise.
// Sequences that fit one split (or are empty) were finished by the split
// kernel.
template <typename T, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int ctx = ctx_len(p, b);
  const int n_split = (ctx + p.split - 1) / p.split;
  if (n_split <= 1) return;
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
    if (d < D) store_out<T>(p.o, b * p.o_sb + (int64_t)hq * p.o_sh + d, a[j] * inv);
  }
}

template <typename T, int D, int G>
int launch_decode_g(const DecodeParams& p, hipStream_t st) {
  const int n_chunks = (p.group + G - 1) / G;
  dim3 grid(p.max_splits, p.n_kv * n_chunks, p.batch);
  hipLaunchKernelGGL((decode_split_kernel<T, D, G>), grid, dim3(kThreads), 0, st, p);
  int e = tl_launch_status();
  if (e || p.max_splits == 1) return e;
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

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

int tl_decode_split_size(int batch, int n_kv_head, int max_ctx) {
  // Aim for several thousand workgroups over the longest sequence: enough to
  // fill 256 CUs several times over, while keeping each split at up to 1024
  // positions (512 KiB of K+V at d_k 128 bf16) so its partial write stays
  // negligible.
  const int64_t heads = (int64_t)batch * (n_kv_head > 0 ? n_kv_head : 1);
  int split = 64;
  while (split < 1024 && heads * ((max_ctx + 2 * split - 1) / (2 * split)) >= 8192) split *= 2;
  return split;
}

size_t tl_attention_decode_workspace_bytes(int batch, int n_head, int max_ctx,
                                           int d_k, int split_size) {
  if (batch <= 0 || n_head <= 0 || max_ctx <= 0 || d_k <= 0 || split_size <= 0) return 0;
  const size_t splits = (size_t)((max_ctx + split_size - 1) / split_size);
  const size_t rows = (size_t)batch * n_head * splits;
  // (m, l) pairs, then accumulators (256-byte aligned).
  return round256(rows * 2 * sizeof(float)) + rows * (size_t)d_k * sizeof(float);
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
  if (dtype != TL_DTYPE_F32 && dtype != TL_DTYPE_F16 && dtype != TL_DTYPE_BF16) return TL_ERR_INVALID;
  if (split_size == 0) split_size = tl_decode_split_size(batch, n_kv_head, max_ctx);
  if (split_size < 16 || split_size % 16 != 0) return TL_ERR_INVALID;
  if (workspace_bytes < tl_attention_decode_workspace_bytes(batch, n_head, max_ctx, d_k, split_size))
    return TL_ERR_INVALID;
  if (d_k != 64 && d_k != 128) return TL_ERR_UNSUPPORTED;
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
  char* ws = (char*)workspace;
  p.ws_ml = (float*)ws;
  ws += round256(rows * 2 * sizeof(float));
  p.ws_acc = (float*)ws;
  p.q_sb = q_strides[0];
  p.q_sh = q_strides[1];
  p.k_sb = k_strides[0];
  p.k_sh = k_strides[1];
  p.v_sb = v_strides[0];
  p.v_sh = v_strides[1];
  p.o_sb = o_strides[0];
  p.o_sh = o_strides[1];
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  // Each lane loads d_k/16 contiguous elements with one vector load, so
  // every row start must be aligned to that slice; positions are addressed
  // with 32-bit byte offsets from the (b, head) base.
  const int esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  const int64_t slice = d_k / 16;
  const uintptr_t align = (uintptr_t)(slice * esize);
  const int64_t st_all[] = {p.q_sb, p.q_sh, p.k_sb, p.k_sh, k_strides[2], p.v_sb, p.v_sh, v_strides[2]};
  for (int64_t s : st_all)
    if (s < 0 || s % slice) return TL_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) % align) return TL_ERR_UNSUPPORTED;
  if (((uintptr_t)workspace) % 16) return TL_ERR_INVALID;
  const int64_t k_region = ((int64_t)(max_ctx - 1) * k_strides[2] + d_k) * esize;
  const int64_t v_region = ((int64_t)(max_ctx - 1) * v_strides[2] + d_k) * esize;
  if (k_region > INT32_MAX || v_region > INT32_MAX) return TL_ERR_UNSUPPORTED;
  p.k_row_bytes = (uint32_t)(k_strides[2] * esize);
  p.v_row_bytes = (uint32_t)(v_strides[2] * esize);
  p.k_region_bytes = (uint32_t)k_region;
  p.v_region_bytes = (uint32_t)v_region;
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: return launch_decode_t<F32>(p, d_k, st);
    case TL_DTYPE_F16: return launch_decode_t<F16>(p, d_k, st);
    default: return launch_decode_t<BF16>(p, d_k, st);
  }
}

}  // extern "C"
