// Next-token sampling on the device, so the logits never leave the GPU.
//
// Reference behaviour being replaced: SmolLM2._sample (smollm2_triton/
// model.py:566-584), run on the host after a full logits download:
//   * temperature <= 1e-6: np.argmax(logits), the first index of the maximum
//     (a NaN counts as the maximum);
//   * otherwise p = exp(x / T - max(x / T)) (fp32 exp, then fp64); with
//     0 < top_k < V only the top_k largest are kept; the token is
//     np.random.choice(V, p=p / sum(p)), which takes one uniform u in [0, 1)
//     and returns the first index whose cumulative probability exceeds u.
// Here u comes in as an argument (one fp64 per row), so the token is a
// deterministic function of (logits, T, top_k, u) and the host keeps the
// random stream; the Python wrapper draws u from the same NumPy stream
// np.random.choice would.  The C entry point takes temperature <= 0 as greedy
// (the wrapper applies the reference's 1e-6 cut-off in double precision).
//
// A row is read by many workgroups at once: one CU keeps too few misses in
// flight to stream a 200-500 KB row quickly (~10 GB/s measured), so each row
// is cut into segments of 2048 entries, one 256-thread workgroup per segment
// (grid = segments x rows), each entry read from HBM exactly once:
//   * every segment records its maximum and first index;
//   * without top_k it also records its mass at its own maximum,
//     sum exp(x / T - m_seg / T) (fp64);
//   * with top_k it keeps its own top_k (every entry >= its k-th largest, by
//     a radix select on an order-preserving 32-bit key, 8 bits per step,
//     counted with LDS atomics) as candidates, written in index order.  The row's k-th
//     largest is >= each segment's k-th largest, so the candidates hold every
//     entry the row keeps.
// A second kernel, one workgroup per row, finishes each row (the kernel
// boundary publishes the segments' results; no fences or counters):
//   * greedy: the argmax of the segment maxima;
//   * without top_k: segment masses rescaled to the row maximum locate the
//     segment holding target = u * total, which is rescanned with the exact
//     p = exp(x / T - max / T);
//   * with top_k: the k-th largest candidate (radix select; candidates staged
//     in LDS when they fit), then the inverse CDF over the kept candidates.
// Every scan gives thread t the interval [lo_t, hi_t) of cumulative mass with
// hi_t the same double as lo_{t+1}, so exactly one thread holds target.
// Every entry >= the k-th largest logit is kept: ties with the k-th are all
// kept, where argpartition keeps exactly k of them in an arbitrary order.
// A row whose maximum is not finite (a NaN or +inf logit, all logits -inf)
// gets token -1 when sampling; np.random.choice raises ValueError there.
#include "tl_common.h"

#include <limits.h>
#include <math.h>

namespace {

constexpr int kBT = 256;                    // threads per workgroup
constexpr int kBW = kBT / 64;               // waves per workgroup
constexpr int kPer = 8;                     // entries per thread in a segment
constexpr int kSeg = kBT * kPer;            // entries per segment
constexpr int kMaxSeg = 128;                // segments per row (2 per lane of one wave)
constexpr int kMaxVocab = kMaxSeg * kSeg;   // 262144
constexpr int kLdsCand = 6144;              // candidates the finishing workgroup stages in LDS
constexpr int kMaxRows = 65535;             // grid.y

struct Ws {
  double* mass;    // [rows][G] segment mass at the segment maximum
  float* smax;     // [rows][G] segment maximum
  int* sarg;       // [rows][G] its first index
  int* count;      // [rows][G] candidates kept by the segment
  float* cx;       // [rows][vocab] candidate logits, segment g's list at g * kSeg
  int* ci;         // [rows][vocab] their indices
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }
int n_segments(int vocab) { return (vocab + kSeg - 1) / kSeg; }

// Workspace layout; base == nullptr only sizes it.
size_t ws_layout(int rows, int vocab, char* base, Ws* ws) {
  const size_t R = (size_t)rows, G = (size_t)n_segments(vocab), V = (size_t)vocab;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  char* mass = take(R * G * 8);
  char* smax = take(R * G * 4);
  char* sarg = take(R * G * 4);
  char* count = take(R * G * 4);
  char* cx = take(R * V * 4);
  char* ci = take(R * V * 4);
  if (ws) *ws = Ws{(double*)mass, (float*)smax, (int*)sarg, (int*)count, (float*)cx, (int*)ci};
  return off;
}

template <typename T>
__device__ __forceinline__ float logit(const void* row, int i) {
  return to_f32<T>(((const typename T::bits*)row)[i]);
}

// np.argmax order: NaN above everything, then larger value, then lower index.
__device__ __forceinline__ bool beats(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na != nb) return na;
  if (na) return ia < ib;
  return va > vb || (va == vb && ia < ib);
}

// Unsigned key with the order of the float value (-inf lowest, +inf highest;
// -0 and +0 share a key, as they compare equal).
__device__ __forceinline__ unsigned order_key(float x) {
  const unsigned b = x == 0.f ? 0u : __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ double wave_incl_scan_d(double v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double y = __shfl_up(v, d);
    if (lane >= d) v += y;
  }
  return v;
}

__device__ __forceinline__ int wave_incl_scan_i(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(v, d);
    if (lane >= d) v += y;
  }
  return v;
}

struct LdsSeg {
  float m[kBW];
  int a[kBW];
  double d[kBW];
  int i[kBW];
  unsigned hist[256];
  unsigned sel[3];
};

struct LdsFin : LdsSeg {
  int pick;
  double pick_lo;
  double target;
  int off[kMaxSeg + 1];
  float cx[kLdsCand];
  int ci[kLdsCand];
};

// (max, first index) over the workgroup; every thread gets the result.
__device__ __forceinline__ void block_argmax(float& m, int& a, LdsSeg& s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float om = __shfl_xor(m, off);
    const int oa = __shfl_xor(a, off);
    if (beats(om, oa, m, a)) {
      m = om;
      a = oa;
    }
  }
  __syncthreads();  // earlier readers of s.m / s.a are done
  if (lane == 0) {
    s.m[wave] = m;
    s.a[wave] = a;
  }
  __syncthreads();
  m = s.m[0];
  a = s.a[0];
#pragma unroll
  for (int w = 1; w < kBW; ++w)
    if (beats(s.m[w], s.a[w], m, a)) {
      m = s.m[w];
      a = s.a[w];
    }
}

// Workgroup scan of v: [lo, hi) is this thread's interval, total the sum.  The
// wave offsets are summed in one order by every thread, so the hi of one
// thread is the lo of the next bit for bit, and the last hi is total.
__device__ __forceinline__ void block_scan_d(double v, double& lo, double& hi, double& total, LdsSeg& s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const double incl = wave_incl_scan_d(v, lane);
  double excl = __shfl_up(incl, 1);
  if (lane == 0) excl = 0.0;
  __syncthreads();  // earlier readers of s.d are done
  if (lane == 63) s.d[wave] = incl;
  __syncthreads();
  double base = 0.0;
  total = 0.0;
#pragma unroll
  for (int w = 0; w < kBW; ++w) {
    if (w == wave) base = total;
    total += s.d[w];
  }
  lo = base + excl;
  hi = base + incl;
}

// Key of the need-th largest entry (1 <= need <= number of entries): radix
// select from the top byte down.  each(f) calls f(key) for every entry this
// thread holds.  A step counts the byte under the current prefix into 256
// LDS bins; wave 0 finds the largest byte D whose suffix still holds `need`
// entries.  It stops early when D's bin holds exactly the entries still to
// take: then every entry >= the prefix (lower bits zero) is in the top need.
template <class Each>
__device__ __forceinline__ unsigned kth_key(Each&& each, unsigned need, LdsSeg& s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned prefix = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    const unsigned hmask = shift == 24 ? 0u : ~0u << (shift + 8);
    for (int b = threadIdx.x; b < 256; b += kBT) s.hist[b] = 0u;
    __syncthreads();
    each([&](unsigned key) {
      if ((key & hmask) == prefix) atomicAdd(&s.hist[(key >> shift) & 255u], 1u);
    });
    __syncthreads();
    if (wave == 0) {
      unsigned c[4], lsum = 0;  // lane l: bins 4l .. 4l+3
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = s.hist[4 * lane + q];
        lsum += c[q];
      }
      unsigned v = lsum;  // entries in lanes >= l
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const unsigned y = __shfl_down(v, d);
        if (lane + d < 64) v += y;
      }
      // lane 0's suffix is every entry under the prefix, which holds `need`
      const int L = __popcll(__ballot(v >= need)) - 1;
      if (lane == L) {
        unsigned suf = v - lsum;  // entries in lanes > L
        int q = 3;
        for (;; --q) {
          suf += c[q];
          if (suf >= need || q == 0) break;
        }
        s.sel[0] = (unsigned)(4 * L + q);
        s.sel[1] = need - (suf - c[q]);
        s.sel[2] = c[q];
      }
    }
    __syncthreads();
    prefix |= s.sel[0] << shift;
    const bool settled = shift == 0 || s.sel[2] == s.sel[1];
    need = s.sel[1];
    if (settled) break;
    // The next step clears s.hist only after wave 0 has read it (the barrier
    // above), and writes s.sel only after its second barrier, which every
    // thread reaches after reading s.sel here.
  }
  return prefix;
}

// One segment of one row: grid (segments, rows).
template <typename T>
__global__ __launch_bounds__(kBT) void segment_kernel(const void* logits, int64_t row_stride, int vocab,
                                                      float temperature, int top_k, Ws ws) {
  __shared__ LdsSeg s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.x, r = blockIdx.y, G = gridDim.x;
  const void* row = (const char*)logits + (int64_t)r * row_stride * T::size;
  const bool greedy = !(temperature > 0.f);
  const bool filter = !greedy && top_k > 0 && top_k < vocab;
  const int s0 = g * kSeg;
  const int nseg = min(kSeg, vocab - s0);
  const int i0 = s0 + tid * kPer;  // this thread's kPer consecutive entries
  const size_t pi = (size_t)r * G + g;

  // ---- this segment ----
  float x[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) x[j] = i0 + j < vocab ? logit<T>(row, i0 + j) : -INFINITY;
  float m = -INFINITY;
  int a = INT_MAX;
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (i0 + j < vocab && beats(x[j], i0 + j, m, a)) {
      m = x[j];
      a = i0 + j;
    }
  block_argmax(m, a, s);
  if (tid == 0) {
    ws.smax[pi] = m;
    ws.sarg[pi] = a;
  }
  if (!greedy && !filter) {
    double v = 0.0;
    if (m > -INFINITY && m < INFINITY) {
      const float ms = m / temperature;
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (i0 + j < vocab) v += (double)expf(x[j] / temperature - ms);
    }
    double lo, hi, tot;
    block_scan_d(v, lo, hi, tot, s);
    if (tid == 0) ws.mass[pi] = tot;
  }
  if (filter) {
    unsigned thr = 0u;  // keep the whole segment when it has at most top_k entries
    if (top_k < nseg)
      thr = kth_key(
          [&](auto&& f) {
#pragma unroll
            for (int j = 0; j < kPer; ++j)
              if (i0 + j < vocab) f(order_key(x[j]));
          },
          (unsigned)top_k, s);
    int c = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) c += (i0 + j < vocab && order_key(x[j]) >= thr) ? 1 : 0;
    const int incl = wave_incl_scan_i(c, lane);
    __syncthreads();
    if (lane == 63) s.i[wave] = incl;
    __syncthreads();
    int pos = incl - c, n_kept = 0;
#pragma unroll
    for (int w = 0; w < kBW; ++w) {
      if (w < wave) pos += s.i[w];
      n_kept += s.i[w];
    }
    const size_t base = (size_t)r * vocab + s0;
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (i0 + j < vocab && order_key(x[j]) >= thr) {
        ws.cx[base + pos] = x[j];
        ws.ci[base + pos] = i0 + j;
        ++pos;
      }
    if (tid == 0) ws.count[pi] = n_kept;
  }

}

// The rest of each row, one workgroup per row, after segment_kernel.
template <typename T>
__global__ __launch_bounds__(kBT) void finish_kernel(const void* logits, int64_t row_stride, int vocab,
                                                     float temperature, int top_k, const double* uniforms,
                                                     double uniform, int32_t* out, Ws ws, int G) {
  __shared__ LdsFin s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = blockIdx.x;
  const void* row = (const char*)logits + (int64_t)r * row_stride * T::size;
  const bool greedy = !(temperature > 0.f);
  const bool filter = !greedy && top_k > 0 && top_k < vocab;

  float M = -INFINITY;
  int A = INT_MAX;
  if (tid < G) {
    M = ws.smax[(size_t)r * G + tid];
    A = ws.sarg[(size_t)r * G + tid];
  }
  block_argmax(M, A, s);
  if (tid == 0) out[r] = greedy ? A : -1;  // sampling: replaced below by the thread holding the draw
  if (greedy || !(M > -INFINITY && M < INFINITY)) return;
  const float Ms = M / temperature;
  const double u = fmin(fmax(uniforms ? uniforms[r] : uniform, 0.0), 1.0);

  if (!filter) {
    // segment weights: mass at the segment maximum rescaled to the row's
    if (wave == 0) {
      double wv[2], mine = 0.0;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int gg = 2 * lane + q;
        wv[q] = 0.0;
        if (gg < G) {
          const float mg = ws.smax[(size_t)r * G + gg];
          if (mg > -INFINITY) wv[q] = ws.mass[(size_t)r * G + gg] * exp((double)(mg / temperature) - (double)Ms);
        }
        mine += wv[q];
      }
      const double incl = wave_incl_scan_d(mine, lane);
      double excl = __shfl_up(incl, 1);
      if (lane == 0) excl = 0.0;
      const double total = __shfl(incl, 63);
      const double target = u * total;
      const uint64_t claim = __ballot(excl < incl && excl <= target && (target < incl || incl >= total));
      int gsel = -1;
      double clo = excl;
      if (claim) {
        const int owner = __ffsll((unsigned long long)claim) - 1;
        double acc = excl, lo_hit = excl, lo_last = excl;
        int q_hit = -1, q_last = 0;
#pragma unroll
        for (int q = 0; q < 2; ++q)
          if (wv[q] > 0.0) {
            q_last = q;
            lo_last = acc;
            const double next = acc + wv[q];
            if (q_hit < 0 && next > target) {
              q_hit = q;
              lo_hit = acc;
            }
            acc = next;
          }
        const int q = q_hit >= 0 ? q_hit : q_last;
        gsel = 2 * owner + __shfl(q, owner);
        clo = __shfl(q_hit >= 0 ? lo_hit : lo_last, owner);
      }
      if (lane == 0) {
        s.pick = gsel;
        s.pick_lo = clo;
        s.target = target;
      }
    }
    __syncthreads();
    const int gs = s.pick;
    const double clo = s.pick_lo, target = s.target;
    if (gs < 0) return;  // not reachable: the weights tile [0, total]
    const int e0 = gs * kSeg + tid * kPer;
    float p[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) p[j] = e0 + j < vocab ? logit<T>(row, e0 + j) : -INFINITY;
    double mine = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      p[j] = e0 + j < vocab ? expf(p[j] / temperature - Ms) : 0.f;
      mine += (double)p[j];
    }
    double lo, hi, tot;
    block_scan_d(mine, lo, hi, tot, s);
    lo += clo;
    hi += clo;
    const double end = clo + tot;
    if (lo < hi && lo <= target && (target < hi || hi >= end)) {
      double acc = lo;
      int tok = -1, last = -1;
#pragma unroll
      for (int j = 0; j < kPer; ++j)
        if (p[j] > 0.f) {
          last = e0 + j;
          acc += (double)p[j];
          if (tok < 0 && acc > target) tok = e0 + j;
        }
      out[r] = tok >= 0 ? tok : last;
    }
    return;
  }

  // ---- top_k: the candidates of all segments, in index order ----
  if (wave == 0) {
    const int g0 = 2 * lane, g1 = 2 * lane + 1;
    const int c0 = g0 < G ? ws.count[(size_t)r * G + g0] : 0;
    const int c1 = g1 < G ? ws.count[(size_t)r * G + g1] : 0;
    const int incl = wave_incl_scan_i(c0 + c1, lane);
    if (g0 < G) s.off[g0] = incl - c0 - c1;
    if (g1 < G) s.off[g1] = incl - c1;
    if (lane == 63) s.off[G] = incl;
  }
  __syncthreads();
  const int C = s.off[G];
  const bool staged = C <= kLdsCand;
  // position in the workspace of flat candidate f: the last segment whose
  // list starts at or before f (empty lists share their start with the next)
  auto locate = [&](int f) -> size_t {
    int lo = 0, hi = G - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s.off[mid] <= f)
        lo = mid;
      else
        hi = mid - 1;
    }
    return (size_t)r * vocab + (size_t)lo * kSeg + (size_t)(f - s.off[lo]);
  };
  if (staged) {
    // kStage loads per thread in flight: up to 4096 candidates in one round trip
    constexpr int kStage = 16;
    for (int f0 = tid; f0 < C; f0 += kStage * kBT) {
      size_t at[kStage];
      float vx[kStage];
      int vi[kStage];
#pragma unroll
      for (int q = 0; q < kStage; ++q) at[q] = f0 + q * kBT < C ? locate(f0 + q * kBT) : 0;
#pragma unroll
      for (int q = 0; q < kStage; ++q)
        if (f0 + q * kBT < C) {
          vx[q] = ws.cx[at[q]];
          vi[q] = ws.ci[at[q]];
        }
#pragma unroll
      for (int q = 0; q < kStage; ++q)
        if (f0 + q * kBT < C) {
          s.cx[f0 + q * kBT] = vx[q];
          s.ci[f0 + q * kBT] = vi[q];
        }
    }
    __syncthreads();
  }
  auto cand_x = [&](int f) -> float { return staged ? s.cx[f] : ws.cx[locate(f)]; };
  auto cand_i = [&](int f) -> int { return staged ? s.ci[f] : ws.ci[locate(f)]; };

  // the row's k-th largest key among the candidates (C >= top_k: every
  // segment kept min(top_k, its size) or more)
  const unsigned thr = kth_key(
      [&](auto&& fn) {
        for (int f = tid; f < C; f += kBT) fn(order_key(cand_x(f)));
      },
      (unsigned)top_k, s);

  // inverse CDF over the kept candidates, contiguous runs per thread
  const int run = (C + kBT - 1) / kBT;
  const int f0 = min(C, tid * run), f1 = min(C, f0 + run);
  double mine = 0.0;
  for (int f = f0; f < f1; ++f) {
    const float xv = cand_x(f);
    if (order_key(xv) >= thr) mine += (double)expf(xv / temperature - Ms);
  }
  double lo, hi, total;
  block_scan_d(mine, lo, hi, total, s);
  const double target = u * total;
  if (lo < hi && lo <= target && (target < hi || hi >= total)) {
    double acc = lo;
    int tok = -1, last = -1;
    for (int f = f0; f < f1; ++f) {
      const float xv = cand_x(f);
      if (order_key(xv) < thr) continue;
      const float pv = expf(xv / temperature - Ms);
      if (pv > 0.f) {
        last = f;
        acc += (double)pv;
        if (tok < 0 && acc > target) tok = f;
      }
    }
    out[r] = cand_i(tok >= 0 ? tok : last);
  }
}

template <typename T>
void launch(const void* logits, int rows, int vocab, int64_t row_stride, float temperature, int top_k,
            const double* uniforms, double uniform, int32_t* tokens, const Ws& ws, hipStream_t st) {
  const int G = n_segments(vocab);
  hipLaunchKernelGGL((segment_kernel<T>), dim3((unsigned)G, (unsigned)rows), dim3(kBT), 0, st, logits, row_stride,
                     vocab, temperature, top_k, ws);
  hipLaunchKernelGGL((finish_kernel<T>), dim3((unsigned)rows), dim3(kBT), 0, st, logits, row_stride, vocab,
                     temperature, top_k, uniforms, uniform, tokens, ws, G);
}

}  // namespace

extern "C" {

int tl_sample_max_vocab(void) { return kMaxVocab; }

size_t tl_sample_workspace_bytes(int rows, int vocab) {
  if (rows <= 0 || rows > kMaxRows || vocab <= 0 || vocab > kMaxVocab) return 0;
  return ws_layout(rows, vocab, nullptr, nullptr);
}

}  // extern "C"

namespace {

int sample_impl(const void* logits, int rows, int vocab, int64_t row_stride, float temperature, int top_k,
                const double* uniforms, double uniform, int32_t* tokens, void* workspace, size_t workspace_bytes,
                int dtype, void* stream) {
  if (rows < 0 || rows > kMaxRows || vocab <= 0 || vocab > kMaxVocab || row_stride < vocab || top_k < 0)
    return TL_ERR_INVALID;
  if (dtype != TL_DTYPE_F32 && dtype != TL_DTYPE_F16 && dtype != TL_DTYPE_BF16) return TL_ERR_INVALID;
  if (rows == 0) return 0;
  if (!logits || !tokens || !workspace) return TL_ERR_INVALID;
  Ws ws;
  if (workspace_bytes < ws_layout(rows, vocab, (char*)workspace, &ws)) return TL_ERR_INVALID;
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32:
      launch<F32>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, uniform, tokens, ws, st);
      break;
    case TL_DTYPE_F16:
      launch<F16>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, uniform, tokens, ws, st);
      break;
    default: launch<BF16>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, uniform, tokens, ws, st);
  }
  return tl_launch_status();
}

}  // namespace

extern "C" {

int tl_sample(const void* logits, int rows, int vocab, int64_t row_stride, float temperature, int top_k,
              const double* uniforms, int32_t* tokens, void* workspace, size_t workspace_bytes, int dtype,
              void* stream) {
  if (temperature > 0.f && !uniforms) return TL_ERR_INVALID;
  return sample_impl(logits, rows, vocab, row_stride, temperature, top_k, uniforms, 0.0, tokens, workspace,
                     workspace_bytes, dtype, stream);
}

int tl_sample_row(const void* logits, int vocab, float temperature, int top_k, double uniform, int32_t* token,
                  void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  return sample_impl(logits, 1, vocab, vocab, temperature, top_k, nullptr, uniform, token, workspace,
                     workspace_bytes, dtype, stream);
}

}  // extern "C"
