// Single-token decode attention over a resident KV cache: a split-K pass and
// a log-sum-exp combine of the splits.
//
// Reference behaviour being replaced: per decode step the reference runs
// attention_gqa(q, K[:L], V[:L], causal=False) (smollm2_triton/model.py:310-314)
// whose kernel (attention_gqa.py:21-146) launches one program per query head,
// re-reading each KV head once per query head of its group.  Here a
// workgroup streams K/V rows of one KV head and serves all G query heads of
// it (up to 8; larger groups run as several pairs of the same KV head), so
// each K/V byte is read once.
//
// Work partition.  The cached positions of every (sequence, pair) stream are
// laid end to end and cut into equal shares, one per workgroup, with exactly
// as many workgroups as the device holds at once.  Every workgroup therefore
// streams the same number of bytes whatever the sequence lengths are, and no
// second round of workgroups is left to straggle.  (A grid of one workgroup
// per (sequence, head, fixed-size split) leaves the late splits of long
// sequences running alone, and measured 6.1 TB/s where the equal shares
// reach 6.5 TB/s.)  A share may end inside one pair and continue into the
// next; each piece is a segment with its own softmax state.
//
// Small caches (max_ctx <= 2048, at most 384 KiB of K/V per (sequence, KV
// head) and 64 MiB in all, e.g. GPT-2's
// 1024-position cache) are latency-bound instead: a few MB spread over a
// thousand shares cost a combine launch and dependent loads for little
// streaming.  There one 16-wave workgroup (64 key streams -- 128 for
// 128-byte rows -- 8 keys each per iteration) takes a whole (sequence,
// pair), finishes it and writes its output (zeros for an empty sequence),
// and no combine runs (GPT-2 decode 14.5 -> 9.7 us).
//
// The pass is HBM-bound (every K/V byte is read exactly once), so the design
// goal is to keep the VALU work per byte well under the issue budget:
//   * a key row (d_k elements) is read by 16 consecutive lanes with one
//     16-byte (or 8/32-byte) nontemporal buffer load each, so one wave load
//     covers 4 consecutive rows (pair mode, 128-byte rows: 8 lanes with
//     16-byte loads, 8 rows); the row offset lives in one 32-bit VGPR and
//     the per-unroll step in an SGPR (no 64-bit address math per load);
//   * q.k of 16-bit types uses packed dot2 (v_dot2c_f32_bf16 / _f16) straight
//     on the stored words; the 16-lane row sum is 4 DPP-fused adds (8-lane:
//     3);
//   * the lane groups of the workgroup are independent key streams (stream
//     s takes keys start + s, start + s + n_streams, ...), each keeping its
//     own online-softmax state (max m, sum l, accumulator) in the log2 domain,
//     rescaled lazily: only when a new score exceeds the running max by
//     2^kRescaleLog2 (exact either way -- the max only bounds exponent range);
//   * full 64-key iterations run without masks; one masked iteration takes
//     the remainder.
// At the end of a segment the streams are merged (lane shuffles, then
// LDS).  A pair inside one share is normalised and written directly;
// otherwise each share's segment stores (m, l, acc[d_k]) to the workspace and
// a second, small kernel merges them and normalises (attention_gqa.py:143
// acc / row_sum).  The merge is a separate launch on purpose: on MI355X each
// XCD has its own L2, so a device-scope fence inside the split kernel (to let
// the last workgroup combine) writes back and invalidates the whole L2 per
// workgroup, which costs far more than one extra launch.
#include "tl_common.h"

#include <math.h>
#include <stdlib.h>

#include <mutex>

#include <type_traits>

namespace {

constexpr int kThreads = 256;  // equal-share workgroups: 4 waves
constexpr int kPairUnroll = 8;  // pair mode, small lane state: keys in flight per stream (4 and 16 measured slower)
// pair-mode workgroups: 16 waves while a lane's state (G heads x D / 16
// elements) fits the 128 VGPRs of a 1024-thread workgroup, else 8
template <typename T, int D, int G>
constexpr int pair_waves() { return D * G * T::size <= 512 ? 16 : 8; }
// Lanes that read one key row.  In pair mode rows of 128 bytes (16-bit d_k
// 64) are read by 8 lanes with 16-byte loads (8 keys per wave load), which
// halves the lane-sum steps and loads per key (GPT-2 decode 12.5 -> 11.8
// us); the equal shares measured the same either way (SmolLM2-360M 41.7
// against 42.1 us) and keep 16 lanes, as do larger rows.
template <typename T, int D, int G, bool PAIR>
constexpr int lanes_per_row() { return PAIR && D * T::size == 128 && G <= 4 ? 8 : 16; }
constexpr int kPairMaxCtx = 2048;                  // pair mode: max_ctx at most
constexpr int64_t kPairMaxBytes = 64ll << 20;      // pair mode: K/V cache bytes at most
// pair mode: K/V bytes of one (sequence, KV head) at max_ctx at most.  One
// workgroup streams a whole pair at about one CU's load rate (60 GB/s), so a
// long pair outlasts the shares' extra combine launch: at batch 1, 256 KiB
// per pair took 6.7 us in pair mode against 8.6 with shares, 512 KiB 16.3
// against 10.6, 1 MiB 23.4 against 12.4.
constexpr int64_t kPairMaxPairBytes = 384ll << 10;
constexpr int kUnroll = 4;    // keys in flight per stream
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
  float* ws_ml;   // [B][Hq][max_slots][2]  (m in log2 domain, l) of partial shares
  float* ws_acc;  // [B][Hq][max_slots][D]  unnormalised
  void* o;
  int len_add;
  int batch, n_head, n_kv, group, max_ctx;
  int min_share;  // fewest positions in a workgroup share (the split_size argument)
  int max_slots;  // partial slots per (b, query head): ceil(max_ctx / min_share) + 1
  int heads_per_pair;  // query heads of one (kv head, chunk) pair: min(group, 8)
  int n_pairs;         // (kv head, chunk) pairs per sequence
  int n_blocks;        // workgroups launched by the split kernel
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh;
  int64_t v_sb, v_sh;
  uint32_t k_row_bytes, v_row_bytes;        // seq strides in bytes
  uint32_t k_region_bytes, v_region_bytes;  // bytes addressable from one (b, head) base
  int64_t o_sb, o_sh;
  float scale_log2;  // sm_scale * log2(e)
  // Fused RoPE + KV append (tl_attention_decode_append, small-cache mode
  // only): before streaming, the workgroup of each (sequence, pair) rotates
  // its query heads in place and writes the new token's rotated k and its v
  // to cache row lens[b] (every chunk of a KV head writes the same bytes).
  int append;
  const void* kn;
  const void* vn;
  const float* cos_t;  // NULL: no rotation
  const float* sin_t;
  int rope_rows;
  int64_t kn_sb, kn_sh, vn_sb, vn_sh;
  int64_t k_ss, v_ss;  // cache seq strides in elements
};

__device__ __forceinline__ int ctx_len(const DecodeParams& p, int b) {
  int c = (p.lens ? p.lens[b] : 0) + p.len_add;
  c = c < 0 ? 0 : c;
  return c > p.max_ctx ? p.max_ctx : c;
}

// ---- Equal-work partition ------------------------------------------------
// The cached positions of all (sequence, pair) streams are laid end to end in
// the order (b, pair, position): pair q of sequence b occupies rows
// [S_b + q*ctx_b, S_b + (q+1)*ctx_b), S_b = n_pairs * sum_{b' < b} ctx_b'.
// Workgroup i takes rows [i*rpb, (i+1)*rpb), so every workgroup streams the
// same number of K/V bytes whatever the sequence lengths, and a workgroup
// may cover the end of one pair and the start of the next.
template <typename I>
__device__ __forceinline__ I wave_incl_scan(I x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const I y = __shfl_up(x, d);
    if (lane >= d) x += y;
  }
  return x;
}

__device__ __forceinline__ int64_t wave_sum64(int64_t x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Values equal on every lane, moved to scalar registers (the compiler cannot
// see through the lane shuffles that produced them).
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uniform(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)x >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Rows in the flattened order (uniform across the wave).
__device__ __forceinline__ int64_t total_rows(const DecodeParams& p, int lane) {
  int64_t t = 0;
  for (int b0 = 0; b0 < p.batch; b0 += 64)
    t += wave_sum64(b0 + lane < p.batch ? (int64_t)ctx_len(p, b0 + lane) : 0);
  return uniform(t) * p.n_pairs;
}

// Rows per workgroup: an even share of the rows, at least min_share, rounded up
// to whole 64-position iterations.
__device__ __forceinline__ int64_t rows_per_block(const DecodeParams& p, int64_t rows) {
  int64_t r = (rows + p.n_blocks - 1) / p.n_blocks;
  r = r < p.min_share ? p.min_share : r;
  return (r + 63) & ~(int64_t)63;
}

// The sequence owning flattened row r (r < total rows): b, S_b and ctx_b.
struct SeqPos {
  int b;
  int ctx;
  int64_t start;
};

// Lane b's view of sequences 0..63: ctx_b and the flattened rows of
// sequences 0..b.  With batch <= 64 one load of the lengths serves the whole
// workgroup life (every dependent load costs microseconds under full HBM
// load).
struct SeqScan {
  int c;
  int64_t incl;
};
__device__ __forceinline__ SeqScan scan_first64(const DecodeParams& p, int lane) {
  SeqScan s;
  s.c = lane < p.batch ? ctx_len(p, lane) : 0;
  s.incl = wave_incl_scan((int64_t)s.c * p.n_pairs, lane);
  return s;
}
__device__ __forceinline__ SeqPos locate_in(const SeqScan& s, int64_t r, int n_pairs) {
  const uint64_t hit = __ballot(s.incl > r);
  const int l = __ffsll((unsigned long long)hit) - 1;
  SeqPos q;
  q.b = uniform(l);
  q.ctx = uniform(__shfl(s.c, l));
  q.start = uniform(__shfl(s.incl - (int64_t)s.c * n_pairs, l));
  return q;
}
__device__ __forceinline__ SeqPos locate_row(const DecodeParams& p, int64_t r, int lane) {
  int64_t base = 0;
  for (int b0 = 0; b0 < p.batch; b0 += 64) {
    const int c = b0 + lane < p.batch ? ctx_len(p, b0 + lane) : 0;
    const int64_t rows = (int64_t)c * p.n_pairs;
    const int64_t incl = base + wave_incl_scan(rows, lane);
    const uint64_t hit = __ballot(incl > r);
    if (hit) {
      const int l = __ffsll((unsigned long long)hit) - 1;
      SeqPos s;
      s.b = uniform(b0 + l);
      s.ctx = uniform(__shfl(c, l));
      s.start = uniform(__shfl(incl - rows, l));
      return s;
    }
    base = uniform(__shfl(incl, 63));
  }
  return SeqPos{p.batch, 0, base};  // not reached for r < total rows
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

// Wave priority from the share's progress: a wave with less of its share
// done wins instruction issue (and so memory issue) over waves that are
// further along.  Without it the hardware's age order lets the oldest
// workgroup of a CU run ahead while the youngest starves, so the equal
// shares finish up to 140 us apart; with it, within 50 us.
__device__ __forceinline__ void set_progress_priority(int64_t done, int64_t share) {
  const int64_t q = done * 4 / share;
  if (q <= 0) __builtin_amdgcn_s_setprio(3);
  else if (q == 1) __builtin_amdgcn_s_setprio(2);
  else if (q == 2) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// The fused append of tl_attention_decode_append for the pair of one
// workgroup: the same arithmetic and rounding as rope_kv_append_kernel
// (tl_rope.hip), so the cache bytes and rotated q are identical to a
// tl_rope_kv_append call followed by tl_attention_decode.
template <typename T, int D>
__device__ void append_token(const DecodeParams& p, int b, int pair) {
  using B = typename T::bits;
  constexpr int H = D / 2;
  const int n_chunks = p.n_pairs / p.n_kv;
  const int hkv = pair / n_chunks;
  const int hq0 = hkv * p.group + (pair - hkv * n_chunks) * p.heads_per_pair;
  const int n_g = min(p.heads_per_pair, hkv * p.group + p.group - hq0);
  const int pos = p.lens[b];
  const bool rope = p.cos_t != nullptr;
  if (pos < 0 || pos >= p.max_ctx || (rope && pos >= p.rope_rows)) return;
  // jobs: n_g query rows (RoPE only), then the k row, then the v row; job j
  // is element pair (i, i + D/2) of row j / H
  for (int j = threadIdx.x; j < (n_g + 2) * H; j += blockDim.x) {
    const int r = j / H, i = j - r * H;
    float c = 1.f, sn = 0.f;
    if (rope) {
      c = p.cos_t[(int64_t)pos * H + i];
      sn = p.sin_t[(int64_t)pos * H + i];
    }
    if (r < n_g) {
      if (!rope) continue;
      B* qr = (B*)p.q + b * p.q_sb + (int64_t)(hq0 + r) * p.q_sh;
      float oe, oo;
      rope_rotate_pair(to_f32<T>(qr[i]), to_f32<T>(qr[i + H]), c, sn, oe, oo);
      qr[i] = from_f32<T>(oe);
      qr[i + H] = from_f32<T>(oo);
    } else if (r == n_g) {
      const B* kr = (const B*)p.kn + b * p.kn_sb + hkv * p.kn_sh;
      B* dst = (B*)p.k + b * p.k_sb + hkv * p.k_sh + (int64_t)pos * p.k_ss;
      if (rope) {
        float oe, oo;
        rope_rotate_pair(to_f32<T>(kr[i]), to_f32<T>(kr[i + H]), c, sn, oe, oo);
        dst[i] = from_f32<T>(oe);
        dst[i + H] = from_f32<T>(oo);
      } else {
        dst[i] = kr[i];
        dst[i + H] = kr[i + H];
      }
    } else {
      const B* vr = (const B*)p.vn + b * p.vn_sb + hkv * p.vn_sh;
      B* dst = (B*)p.v + b * p.v_sb + hkv * p.v_sh + (int64_t)pos * p.v_ss;
      dst[i] = vr[i];
      dst[i + H] = vr[i + H];
    }
  }
}

// G: query heads of one (kv head, chunk) pair (<= group).  NW: waves per
// workgroup (4 streams each).  PAIR: the pair-aligned mode for small caches
// -- workgroup i streams all of pair i % n_pairs of sequence i / n_pairs and
// finishes it (no partials, no combine launch); otherwise equal shares.
template <typename T, int D, int G, int NW, bool PAIR>
__global__ __launch_bounds__(64 * NW) void decode_split_kernel(DecodeParams p) {
  constexpr int LPR = lanes_per_row<T, D, G, PAIR>();
  constexpr int EPL = D / LPR;          // elements per lane per row
  constexpr int W = EPL * T::size / 4;  // 32-bit words per lane per row
  constexpr int kThr = 64 * NW;
  constexpr int kStr = (64 / LPR) * NW;  // key streams (LPR-lane groups)
  // keys in flight per stream: a pair workgroup streams its whole pair, so
  // it takes more per iteration where a lane's state is small
  constexpr int kU = PAIR && D * G * T::size <= 256 ? kPairUnroll : kUnroll;
  constexpr int kKPI = kStr * kU;       // keys per iteration
  using Bits = typename T::bits;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int sub = lane & (LPR - 1);
  const int stream = wave * (64 / LPR) + lane / LPR;
  const int n_chunks = p.n_pairs / p.n_kv;

  __shared__ float s_m[NW][G], s_l[NW][G];
  __shared__ float s_acc[NW][G][D];
  const uint32_t lane_bytes = sub * (EPL * T::size);
  const float c = p.scale_log2;

  // One segment: positions [start, end) of pair `pair` of sequence b (ctx
  // positions).  whole: the pair lies in this workgroup alone, so its output
  // is finished here; otherwise the partial goes to slot `slot`.
  auto segment = [&](const int b, const int ctx, const int pair, const int start, const int end,
                     const bool whole, const int slot, const int64_t seg_done0, const int64_t share) {
    const int hkv = pair / n_chunks;
    const int hq0 = hkv * p.group + (pair - hkv * n_chunks) * G;
    const int n_g = min(G, hkv * p.group + p.group - hq0);  // heads valid in this pair

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

    // One iteration: kU keys per stream, kKPI per workgroup.
    auto iteration = [&](int key0, auto masked) {
      constexpr bool kMasked = decltype(masked)::value;
      Slice<W> kr[kU], vr[kU];
      bool valid[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int key = key0 + u * kStr;
        if constexpr (kMasked) {
          // Out-of-range keys re-read this segment's first row (always
          // inside the sequence) and are masked out of the softmax below.
          valid[u] = key < end;
          const uint32_t row = valid[u] ? key : start;
          load_slice(kr[u], krs, row * p.k_row_bytes + lane_bytes, 0);
          load_slice(vr[u], vrs, row * p.v_row_bytes + lane_bytes, 0);
        } else {
          valid[u] = true;
          load_slice(kr[u], krs, (uint32_t)key0 * p.k_row_bytes + lane_bytes, u * kStr * p.k_row_bytes);
          load_slice(vr[u], vrs, (uint32_t)key0 * p.v_row_bytes + lane_bytes, u * kStr * p.v_row_bytes);
        }
      }
      float s[G][kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float dp = dot_slice<T>(qs[g], kr[u]);
          const float d = (LPR == 8 ? row8_sum(dp) : row16_sum(dp)) * c;
          s[g][u] = (!kMasked || valid[u]) ? d : -INFINITY;
        }
      }
      // Lazy rescale: move the running max only when a score would exceed
      // it by more than 2^kRescaleLog2.
      bool grow = false;
      float mb[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        mb[g] = s[g][0];
#pragma unroll
        for (int u = 1; u < kU; ++u) mb[g] = fmaxf(mb[g], s[g][u]);
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
      float pu[G][kU];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float base = (m[g] == -INFINITY) ? 0.f : m[g];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          pu[g][u] = fast_exp2(s[g][u] - base);
          l[g] += pu[g][u];
        }
      }
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        float vf[EPL];
        slice_to_float<T>(vr[u], vf);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[g][e] = fmaf(pu[g][u], vf[e], acc[g][e]);
      }
    };

    const int n_full = (end - start) / kKPI;
    int key0 = start + stream;
    for (int it = 0; it < n_full; ++it, key0 += kKPI) {
      if constexpr (!PAIR) {
        if ((it & 3) == 0) set_progress_priority(seg_done0 + (int64_t)it * kKPI, share);
      }
      iteration(key0, std::false_type{});
    }
    if (start + n_full * kKPI < end) iteration(key0, std::true_type{});

    // Merge the streams of this wave (lane groups LPR apart).
#pragma unroll
    for (int off = LPR; off <= 32; off <<= 1) {
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

    // Merge the NW waves through LDS (the barrier in front protects the
    // previous segment's reads of the same arrays).
    __syncthreads();
    if (lane < LPR) {
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
    const int64_t row_base = ((int64_t)b * p.n_head + hq0) * p.max_slots;
    for (int idx = tid; idx < n_g * D; idx += kThr) {
      const int g = idx / D;
      const int d = idx - g * D;
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_m[w][g]);
      const float base = (mx == -INFINITY) ? 0.f : mx;
      float a = 0.f, lsum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float wt = fast_exp2(s_m[w][g] - base);
        a += s_acc[w][g][d] * wt;
        lsum += s_l[w][g] * wt;
      }
      if (whole) {
        // (an empty sequence reads as zeros, the reference's empty-KV result)
        store_out<T>(p.o, b * p.o_sb + (int64_t)(hq0 + g) * p.o_sh + d, ctx == 0 ? 0.f : a / lsum);
      } else {
        const int64_t row = row_base + (int64_t)g * p.max_slots + slot;
        p.ws_acc[row * D + d] = a;
        if (d == 0) {
          p.ws_ml[row * 2 + 0] = mx;
          p.ws_ml[row * 2 + 1] = lsum;
        }
      }
    }
  };

  if constexpr (PAIR) {
    const int b = (int)blockIdx.x / p.n_pairs;
    const int pair = (int)blockIdx.x - b * p.n_pairs;
    if (p.append) {
      // the new token first: rotated q rows and cache row lens[b], visible
      // to every thread of the workgroup before any of them reads them
      append_token<T, D>(p, b, pair);
      __threadfence_block();
      __syncthreads();
    }
    const int ctx = uniform(ctx_len(p, b));
    segment(b, ctx, pair, 0, ctx, true, 0, 0, 0);
  } else {
    const SeqScan scan = scan_first64(p, lane);
    const bool in_regs = p.batch <= 64;
    const int64_t total = in_regs ? uniform(__shfl(scan.incl, 63)) : total_rows(p, lane);
    const int64_t rpb = uniform(rows_per_block(p, total));
    const int64_t r0 = (int64_t)blockIdx.x * rpb;
    if (r0 >= total) return;
    const int64_t r1 = r0 + rpb < total ? r0 + rpb : total;
    for (int64_t r = r0; r < r1;) {
      // The segment [r, seg_end) of this workgroup's rows lies in one pair.
      const SeqPos sp = in_regs ? locate_in(scan, r, p.n_pairs) : locate_row(p, r, lane);
      const int pair = uniform((int)((r - sp.start) / sp.ctx));
      const int64_t pair_row0 = sp.start + (int64_t)pair * sp.ctx;
      const int start = (int)(r - pair_row0);
      const int end = (int)((r1 - pair_row0) < sp.ctx ? (r1 - pair_row0) : sp.ctx);
      r = pair_row0 + end;
      // Workgroups covering this pair: the partial of this one goes to slot
      // blockIdx.x - first; a pair inside one workgroup is finished here.
      const int64_t first = uniform((int64_t)(pair_row0 / rpb));
      const bool whole = uniform((int)((pair_row0 + sp.ctx - 1) / rpb - first)) == 0;
      const int slot = (int)(blockIdx.x - first);
      segment(sp.b, sp.ctx, pair, start, end, whole, slot, pair_row0 + start - r0, r1 - r0);
    }
  }
}

// One wave per (b, query head): merge the partials of the workgroups that
// covered this head's pair and normalise.  A pair inside one workgroup was
// finished by the split kernel; an empty sequence gets zeros here (the
// reference's empty-KV result, tests/test_attention_gqa.py:297).
// The kernel is latency-bound (a few KiB per head), so every load it can
// issue early is issued early: lane s holds partial s's (m, l) pair, the
// accumulator rows are read eight partials at a time, the next eight in
// flight while the current ones are summed, and a partial's weight reaches
// the other lanes with v_readlane.
template <typename T, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeParams p) {
  constexpr int NJ = (D + 63) / 64;
  constexpr int R = 8;
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int ctx = ctx_len(p, b);
  if (ctx == 0) {
    for (int d = lane; d < D; d += 64) store_out<T>(p.o, b * p.o_sb + (int64_t)hq * p.o_sh + d, 0.f);
    return;
  }
  int64_t total = 0, before = 0;
  for (int b0 = 0; b0 < p.batch; b0 += 64) {
    const int bb = b0 + lane;
    const int64_t cb = bb < p.batch ? ctx_len(p, bb) : 0;
    total += wave_sum64(cb);
    before += wave_sum64(bb < b ? cb : 0);
  }
  total = uniform(total);
  before = uniform(before);
  const int64_t rpb = rows_per_block(p, total * p.n_pairs);
  const int hkv = hq / p.group;
  const int pair = hkv * (p.n_pairs / p.n_kv) + (hq - hkv * p.group) / p.heads_per_pair;
  const int64_t pair_row0 = before * p.n_pairs + (int64_t)pair * ctx;
  const int64_t first = pair_row0 / rpb;
  const int n_parts = (int)((pair_row0 + ctx - 1) / rpb - first) + 1;
  if (n_parts <= 1) return;
  const int64_t row0 = ((int64_t)b * p.n_head + hq) * p.max_slots;
  const float2* ml = (const float2*)p.ws_ml + row0;
  const float* acc = p.ws_acc + row0 * D;
  auto load_rows = [&](int s0, float (&r)[R][NJ]) {
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = lane + 64 * j;
        r[k][j] = (s0 + k < n_parts && d < D) ? acc[(int64_t)(s0 + k) * D + d] : 0.f;
      }
  };
  float r[R][NJ];
  load_rows(0, r);
  const float2 e0 = lane < n_parts ? ml[lane] : make_float2(-INFINITY, 0.f);
  float mx = e0.x;
  for (int s = lane + 64; s < n_parts; s += 64) mx = fmaxf(mx, ml[s].x);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
  const float base = (mx == -INFINITY) ? 0.f : mx;
  float lsum = 0.f, a[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) a[j] = 0.f;
  float wl = 0.f;  // weight of partial (s0 & ~63) + lane
  for (int s0 = 0; s0 < n_parts; s0 += R) {
    if ((s0 & 63) == 0) {
      const int s = s0 + lane;
      const float2 e = s0 == 0 ? e0 : (s < n_parts ? ml[s] : make_float2(-INFINITY, 0.f));
      wl = s < n_parts ? fast_exp2(e.x - base) : 0.f;
      lsum += e.y * wl;
    }
    float rn[R][NJ];
    if (s0 + R < n_parts) load_rows(s0 + R, rn);
#pragma unroll
    for (int k = 0; k < R; ++k) {
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), (s0 + k) & 63));
#pragma unroll
      for (int j = 0; j < NJ; ++j) a[j] = fmaf(r[k][j], w, a[j]);
    }
#pragma unroll
    for (int k = 0; k < R; ++k)
#pragma unroll
      for (int j = 0; j < NJ; ++j) r[k][j] = rn[k][j];
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
  const float inv = 1.f / lsum;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int d = lane + 64 * j;
    if (d < D) store_out<T>(p.o, b * p.o_sb + (int64_t)hq * p.o_sh + d, a[j] * inv);
  }
}

// Whether a call runs in pair mode (small caches; see launch_decode_g).
// (tl_overrides.decode_shares forces the shares, so tests can run both
// paths on the same small inputs.)
bool pair_mode(const DecodeParams& p, int d_k, int esize) {
  const int64_t cache_bytes = (int64_t)p.batch * p.n_pairs * p.max_ctx * 2 * d_k * esize;
  const int64_t pair_bytes = (int64_t)p.max_ctx * 2 * d_k * esize;
  return !tl_overrides.decode_shares && p.max_ctx <= kPairMaxCtx && cache_bytes <= kPairMaxBytes &&
         pair_bytes <= kPairMaxPairBytes;
}

template <typename T, int D, int G>
int launch_decode_g(DecodeParams& p, hipStream_t st) {
  // Small caches: one 16-wave workgroup per (sequence, pair), which finishes
  // the pair itself -- no partials and no combine launch.  The cache bound
  // is known on the host (max_ctx), the lengths are not: pair mode needs a
  // short max_ctx (a workgroup streams its pair in a few iterations of 256
  // keys) and a small whole cache (no equal-share spreading needed).
  if (pair_mode(p, D, T::size)) {
    p.n_blocks = p.batch * p.n_pairs;
    constexpr int NW = pair_waves<T, D, G>();
    hipLaunchKernelGGL((decode_split_kernel<T, D, G, NW, true>), dim3(p.n_blocks), dim3(64 * NW), 0, st, p);
    return tl_launch_status();
  }
  // One workgroup per resident slot (occupancy x compute units), never more
  // than the shares of min_share positions a full cache would hold.
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_split_kernel<T, D, G, 4, false>, kThreads, 0) !=
            hipSuccess ||
        n <= 0)
      n = 1;
    per_cu = n;
  }
  const int64_t most = ((int64_t)p.batch * p.n_pairs * p.max_ctx + p.min_share - 1) / p.min_share;
  const int64_t slots = (int64_t)per_cu * tl_device_cus();
  p.n_blocks = (int)(most < slots ? most : slots);
  hipLaunchKernelGGL((decode_split_kernel<T, D, G, 4, false>), dim3(p.n_blocks), dim3(kThreads), 0, st, p);
  int e = tl_launch_status();
  if (e) return e;
  hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3(p.n_head, p.batch), dim3(64), 0, st, p);
  return tl_launch_status();
}

template <typename T, int D>
int launch_decode_d(DecodeParams& p, hipStream_t st) {
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
int launch_decode_t(DecodeParams& p, int d_k, hipStream_t st) {
  switch (d_k) {
    case 64: return launch_decode_d<T, 64>(p, st);
    case 128: return launch_decode_d<T, 128>(p, st);
    default: return TL_ERR_UNSUPPORTED;
  }
}

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// The new token of tl_attention_decode_append.
struct AppendArgs {
  const void* k_new;
  const void* v_new;
  const float* cos_t;
  const float* sin_t;
  int rope_rows;
  const int64_t* k_new_strides;
  const int64_t* v_new_strides;
};

int decode_entry(const void* q, const void* k_cache, const void* v_cache,
                 const int32_t* cache_lens, int len_add, void* o, void* workspace,
                 size_t workspace_bytes, int batch, int n_head, int n_kv_head, int max_ctx,
                 int d_k, const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                 int split_size, int dtype, void* stream, bool check_only = false,
                 const AppendArgs* ap = nullptr);


}  // namespace

// ---- Scratch of the entry point that allocates nothing --------------------
// tl_attention_decode_noalloc keeps the split partials in this file-scope
// device array instead of a caller's workspace.  Every GPU the library runs
// on holds its own copy, at its own address, until the process ends.  In
// host code the name `scratch` is only a stand-in for the symbol, never a
// device address: the per-device address comes from hipGetSymbolAddress
// (noalloc_scratch below) and only that pointer reaches kernels.  The
// partials need no initial contents (each call's combine reads only the
// slots its own split pass wrote), so nothing is cleared; calls that
// overlap in time on one GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[TL_DECODE_NOALLOC_SCRATCH_BYTES];
extern "C" const size_t tl_decode_noalloc_scratch_bytes = sizeof(scratch);

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device with
// that device current.
int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return TL_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return TL_ERR_UNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

int tl_decode_split_size(int batch, int n_kv_head, int max_ctx) {
  // Minimum positions per workgroup share.  The split kernel shares the
  // cached positions evenly over the resident workgroups; this floor keeps a
  // share at least one 64-position iteration when the caches are short, and
  // bounds the partial slots one (sequence, head) can need, hence the
  // workspace.  Picked so a full-length cache would give about 16384 shares.
  const int64_t rows = (int64_t)(batch > 0 ? batch : 1) * (n_kv_head > 0 ? n_kv_head : 1) * (max_ctx > 0 ? max_ctx : 1);
  int split = 64;
  while (split < 4096 && rows > (int64_t)split * 16384) split *= 2;
  return split;
}

size_t tl_attention_decode_workspace_bytes(int batch, int n_head, int max_ctx,
                                           int d_k, int split_size) {
  if (batch <= 0 || n_head <= 0 || max_ctx <= 0 || d_k <= 0 || split_size <= 0) return 0;
  // A (sequence, head) covers at most ceil(max_ctx / split) + 1 workgroup
  // shares (every share holds at least split positions).
  const size_t splits = (size_t)((max_ctx + split_size - 1) / split_size) + 1;
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
  return decode_entry(q, k_cache, v_cache, cache_lens, len_add, o, workspace, workspace_bytes,
                      batch, n_head, n_kv_head, max_ctx, d_k, q_strides, k_strides, v_strides,
                      o_strides, sm_scale, split_size, dtype, stream);
}

int tl_attention_decode_append(void* q, const void* k_new, const void* v_new, void* k_cache,
                               void* v_cache, const int32_t* cache_lens, const float* cos_table,
                               const float* sin_table, int rope_rows, void* o, void* workspace,
                               size_t workspace_bytes, int batch, int n_head, int n_kv_head, int max_ctx,
                               int d_k, const int64_t* q_strides, const int64_t* k_new_strides,
                               const int64_t* v_new_strides, const int64_t* k_strides,
                               const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                               int split_size, int dtype, void* stream) {
  if (batch == 0 || n_head == 0) return 0;
  if (!k_new || !v_new || !cache_lens || !k_new_strides || !v_new_strides) return TL_ERR_INVALID;
  if ((cos_table == nullptr) != (sin_table == nullptr)) return TL_ERR_INVALID;
  if (cos_table && rope_rows < 0) return TL_ERR_INVALID;
  const AppendArgs ap{k_new, v_new, cos_table, sin_table, rope_rows, k_new_strides, v_new_strides};
  return decode_entry(q, k_cache, v_cache, cache_lens, 1, o, workspace, workspace_bytes, batch, n_head, n_kv_head,
                      max_ctx, d_k, q_strides, k_strides, v_strides, o_strides, sm_scale, split_size, dtype, stream,
                      false, &ap);
}

int tl_attention_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* cache_lens, int len_add, void* o, int batch,
                                int n_head, int n_kv_head, int max_ctx, int d_k,
                                const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides,
                                float sm_scale, int split_size, int dtype, void* stream) {
  if (batch == 0 || n_head == 0) return 0;
  if (batch < 0 || n_head < 0 || n_kv_head < 1 || max_ctx < 1) return TL_ERR_INVALID;
  if (split_size == 0) split_size = tl_decode_split_size(batch, n_kv_head, max_ctx);
  if (split_size < 16 || split_size % 16 != 0) return TL_ERR_INVALID;
  // Larger problems than the static scratch holds are refused before any
  // device work (the caller should use tl_attention_decode with a workspace).
  if (tl_attention_decode_workspace_bytes(batch, n_head, max_ctx, d_k, split_size) >
      (size_t)TL_DECODE_NOALLOC_SCRATCH_BYTES)
    return TL_ERR_INVALID;
  // every other argument check first, against a stand-in workspace address
  // (only its null-ness and alignment are checked), so an invalid call
  // returns before any HIP call
  int st = decode_entry(q, k_cache, v_cache, cache_lens, len_add, o, (void*)(uintptr_t)256,
                        (size_t)TL_DECODE_NOALLOC_SCRATCH_BYTES, batch, n_head, n_kv_head, max_ctx, d_k,
                        q_strides, k_strides, v_strides, o_strides, sm_scale, split_size, dtype, stream,
                        /*check_only=*/true);
  if (st != 0) return st;
  void* ws = nullptr;
  st = noalloc_scratch(&ws);
  if (st != 0) return st;
  return decode_entry(q, k_cache, v_cache, cache_lens, len_add, o, ws,
                      (size_t)TL_DECODE_NOALLOC_SCRATCH_BYTES, batch, n_head, n_kv_head, max_ctx,
                      d_k, q_strides, k_strides, v_strides, o_strides, sm_scale, split_size, dtype,
                      stream);
}

}  // extern "C"

namespace {

int decode_entry(const void* q, const void* k_cache, const void* v_cache,
                 const int32_t* cache_lens, int len_add, void* o, void* workspace,
                 size_t workspace_bytes, int batch, int n_head, int n_kv_head, int max_ctx,
                 int d_k, const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                 int split_size, int dtype, void* stream, bool check_only, const AppendArgs* ap) {
  if (batch == 0 || n_head == 0) return 0;
  if (!q || !k_cache || !v_cache || !o || !workspace || batch < 0 ||
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
  p.min_share = split_size;
  p.max_slots = (max_ctx + split_size - 1) / split_size + 1;
  p.heads_per_pair = p.group < 8 ? p.group : 8;
  p.n_pairs = n_kv_head * ((p.group + p.heads_per_pair - 1) / p.heads_per_pair);

  const size_t rows = (size_t)batch * n_head * p.max_slots;
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
  // Each lane loads d_k/16 contiguous elements (d_k/8 for 16-bit d_k 64
  // with at most 4 heads per pair in pair mode: lanes_per_row) with one
  // vector load, so every row start must be aligned to that slice;
  // positions are addressed with 32-bit byte offsets from the (b, head)
  // base.
  const int esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  const bool lanes8 = pair_mode(p, d_k, esize) && d_k * esize == 128 && p.heads_per_pair <= 4;
  const int64_t slice = lanes8 ? d_k / 8 : d_k / 16;
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
  if (check_only) return 0;  // every argument check passed; nothing launched
  if (ap) {
    if (pair_mode(p, d_k, esize)) {
      // small caches: each workgroup appends its pair's token itself
      p.append = 1;
      p.kn = ap->k_new;
      p.vn = ap->v_new;
      p.cos_t = ap->cos_t;
      p.sin_t = ap->sin_t;
      p.rope_rows = ap->rope_rows;
      p.kn_sb = ap->k_new_strides[0];
      p.kn_sh = ap->k_new_strides[1];
      p.vn_sb = ap->v_new_strides[0];
      p.vn_sh = ap->v_new_strides[1];
      p.k_ss = k_strides[2];
      p.v_ss = v_strides[2];
    } else {
      // shared positions: the token goes in first, by its own launch
      const int64_t qs[3] = {q_strides[0], 0, q_strides[1]};
      const int64_t ks[3] = {ap->k_new_strides[0], 0, ap->k_new_strides[1]};
      const int64_t vs[3] = {ap->v_new_strides[0], 0, ap->v_new_strides[1]};
      const int st = tl_rope_kv_append(const_cast<void*>(q), ap->k_new, ap->v_new, const_cast<void*>(k_cache),
                                       const_cast<void*>(v_cache), cache_lens, ap->cos_t, ap->sin_t, ap->rope_rows,
                                       batch, 1, n_head, n_kv_head, max_ctx, d_k, qs, ks, vs, k_strides, v_strides,
                                       dtype, stream);
      if (st != 0) return st;
    }
  }
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: return launch_decode_t<F32>(p, d_k, st);
    case TL_DTYPE_F16: return launch_decode_t<F16>(p, d_k, st);
    default: return launch_decode_t<BF16>(p, d_k, st);
  }
}

}  // namespace
