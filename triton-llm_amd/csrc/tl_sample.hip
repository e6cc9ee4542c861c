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
// One workgroup of 1024 threads per row; every pass over the row is a
// coalesced strided sweep with 16 loads in flight per thread (the row stays
// in L2 after the first):
//   1. row maximum and its first index (and the first radix digits);
//   2. top_k: radix select of the k-th largest logit on an order-preserving
//      32-bit key, 4 bits per pass from the top.  Each thread counts digits
//      in packed 8-bit fields (two 64-bit words), a wave sums them as 16-bit
//      fields, wave 0 picks the digit.  The select stops early once the
//      chosen digit's bin holds exactly the entries still to take.  Every
//      logit >= the k-th is kept, so all ties with the k-th are kept where
//      argpartition keeps exactly k of them in an arbitrary order;
//   3. p = exp(x / T - max / T) for the kept entries; the mass of each chunk
//      of 1024 consecutive entries (fp64) goes to LDS; wave 0 scans the chunk
//      masses for the chunk holding target = u * total, then scans that
//      chunk's entries.  Each scan gives lane l the interval [lo_l, hi_l) with
//      hi_l the same double as lo_{l+1}, so exactly one lane holds target.
// A row whose mass is not a positive finite number (a NaN or +inf logit, all
// logits -inf) gets token -1; np.random.choice raises ValueError there.
#include "tl_common.h"

#include <limits.h>
#include <math.h>

namespace {

constexpr int kSThreads = 1024;
constexpr int kSWaves = kSThreads / 64;
constexpr int kChunk = 1024;                  // entries per chunk of the inverse CDF
constexpr int kPerLane = kChunk / 64;         // a lane's run inside a chunk
constexpr int kMaxChunks = 256;               // wave 0 holds 4 chunk masses per lane
constexpr int kMaxVocab = 255 * kSThreads;    // per-thread radix counts fit 8 bits
constexpr int kSweep = 16;                    // loads in flight per thread in a sweep

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

// f(x, i) for every entry of the row, thread t taking i = t + 1024 j.  Each
// thread issues kSweep loads before it uses any, so a sweep waits for memory
// once per kSweep * 1024 entries instead of once per 1024.
template <typename T, typename F>
__device__ __forceinline__ void sweep(const void* row, int vocab, F&& f) {
  for (int base = threadIdx.x; base < vocab; base += kSweep * kSThreads) {
    float v[kSweep];
#pragma unroll
    for (int u = 0; u < kSweep; ++u) {
      const int i = base + u * kSThreads;
      v[u] = i < vocab ? logit<T>(row, i) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kSweep; ++u)
      if (base + u * kSThreads < vocab) f(v[u], base + u * kSThreads);
  }
}

// Count the 4-bit digit of key at shift: digits 0-7 in lo8, 8-15 in hi8,
// 8 bits per digit.
__device__ __forceinline__ void add_digit(unsigned key, int shift, uint64_t& lo8, uint64_t& hi8) {
  const unsigned d = (key >> shift) & 15u;
  const uint64_t inc = 1ull << ((d & 7u) * 8u);
  if (d < 8u)
    lo8 += inc;
  else
    hi8 += inc;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ double wave_incl_scan_d(double v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double y = __shfl_up(v, d);
    if (lane >= d) v += y;
  }
  return v;
}

template <typename T>
__global__ __launch_bounds__(kSThreads) void sample_kernel(const void* logits, int64_t row_stride, int vocab,
                                                           float temperature, int top_k, const double* uniforms,
                                                           int32_t* out) {
  __shared__ float s_max[kSWaves];
  __shared__ int s_arg[kSWaves];
  __shared__ unsigned s_hist[kSWaves][16];
  __shared__ unsigned s_sel[3];
  __shared__ double s_chunk[kMaxChunks];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const void* row = (const char*)logits + (int64_t)blockIdx.x * row_stride * T::size;

  // 1. maximum and its first index; with a top_k filter the same sweep
  //    counts the first (top 4 bits) radix digits
  const bool filter = temperature > 0.f && top_k > 0 && top_k < vocab;
  float bm = -INFINITY;
  int bi = INT_MAX;
  uint64_t lo8 = 0, hi8 = 0;  // digit counts of this thread, 8 bits each
  sweep<T>(row, vocab, [&](float x, int i) {
    if (beats(x, i, bm, bi)) {
      bm = x;
      bi = i;
    }
    if (filter) add_digit(order_key(x), 28, lo8, hi8);
  });
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float om = __shfl_xor(bm, off);
    const int oi = __shfl_xor(bi, off);
    if (beats(om, oi, bm, bi)) {
      bm = om;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_max[wave] = bm;
    s_arg[wave] = bi;
  }
  __syncthreads();
  bm = s_max[0];
  bi = s_arg[0];
  for (int w = 1; w < kSWaves; ++w)
    if (beats(s_max[w], s_arg[w], bm, bi)) {
      bm = s_max[w];
      bi = s_arg[w];
    }
  if (!(temperature > 0.f)) {
    if (tid == 0) out[blockIdx.x] = bi;
    return;
  }

  // 2. key of the k-th largest logit (0 keeps everything)
  unsigned thr = 0u;
  if (filter) {
    unsigned prefix = 0u, need = (unsigned)top_k;
    for (int shift = 28; shift >= 0; shift -= 4) {
      if (shift != 28) {  // the top digit was counted with the maximum
        const unsigned hmask = ~0u << (shift + 4);
        lo8 = hi8 = 0;
        sweep<T>(row, vocab, [&](float x, int) {
          const unsigned key = order_key(x);
          if ((key & hmask) == prefix) add_digit(key, shift, lo8, hi8);
        });
      }
      // 16-bit fields for the wave sum (at most 64 * 255 per digit)
      uint64_t w16[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t src = q < 2 ? lo8 : hi8;
        uint64_t v = 0;
#pragma unroll
        for (int f = 0; f < 4; ++f) v |= ((src >> (8 * ((q & 1) * 4 + f))) & 0xFFull) << (16 * f);
        w16[q] = v;
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
        for (int q = 0; q < 4; ++q) w16[q] += __shfl_xor(w16[q], off);
      if (lane == 0)
#pragma unroll
        for (int d = 0; d < 16; ++d) s_hist[wave][d] = (unsigned)((w16[d >> 2] >> (16 * (d & 3))) & 0xFFFFull);
      __syncthreads();
      if (wave == 0) {
        unsigned cnt = 0;
        if (lane < 16)
          for (int w = 0; w < kSWaves; ++w) cnt += s_hist[w][lane];
        unsigned suf = cnt;  // lane d: entries whose digit is >= d
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
          const unsigned y = __shfl_down(suf, d);
          if (lane + d < 16) suf += y;
        }
        // the largest digit whose suffix still holds `need` entries (digit 0
        // always does: its suffix is every entry under the prefix)
        const int D = __popcll(__ballot(lane < 16 && suf >= need)) - 1;
        const unsigned above = __shfl(suf, D + 1);  // lane 16 holds 0
        const unsigned inbin = __shfl(cnt, D);
        if (lane == 0) {
          s_sel[0] = (unsigned)D;
          s_sel[1] = need - above;
          s_sel[2] = inbin;
        }
      }
      __syncthreads();
      prefix |= s_sel[0] << shift;
      thr = prefix;
      if (s_sel[2] == s_sel[1]) break;  // the whole bin is kept: lower bits do not matter
      need = s_sel[1];
    }
  }

  // 3. chunk masses, then the inverse CDF in wave 0
  const float ms = bm / temperature;
  auto prob_of = [&](float x) -> float { return order_key(x) >= thr ? expf(x / temperature - ms) : 0.f; };
  const int n_chunks = (vocab + kChunk - 1) / kChunk;
  for (int c = wave; c < n_chunks; c += kSWaves) {
    float v[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int i = c * kChunk + j * 64 + lane;
      v[j] = i < vocab ? logit<T>(row, i) : 0.f;
    }
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (c * kChunk + j * 64 + lane < vocab) s += (double)prob_of(v[j]);
    s = wave_sum_d(s);
    if (lane == 0) s_chunk[c] = s;
  }
  __syncthreads();
  if (wave != 0) return;

  // lane l: chunks 4l .. 4l+3
  double cm[4], mine = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = 4 * lane + q;
    cm[q] = c < n_chunks ? s_chunk[c] : 0.0;
    mine += cm[q];
  }
  double incl = wave_incl_scan_d(mine, lane);
  double excl = __shfl_up(incl, 1);
  if (lane == 0) excl = 0.0;
  const double total = __shfl(incl, 63);
  if (!(total > 0.0) || !(total < INFINITY)) {
    if (lane == 0) out[blockIdx.x] = -1;
    return;
  }
  const double u = fmin(fmax(uniforms[blockIdx.x], 0.0), 1.0);
  const double target = u * total;
  // The lane whose interval holds target; when rounding leaves target at
  // total, the last lane with mass (its hi is total).
  uint64_t claim = __ballot(excl < incl && excl <= target && (target < incl || incl >= total));
  if (!claim) {  // not reachable: the intervals tile [0, total]
    if (lane == 0) out[blockIdx.x] = -1;
    return;
  }
  int owner = __ffsll((unsigned long long)claim) - 1;
  int cq = -1, lastq = 0;
  double acc = excl, clo = excl, clo_last = excl;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (cm[q] > 0.0) {
      lastq = q;
      clo_last = acc;
      const double next = acc + cm[q];
      if (cq < 0 && next > target) {
        cq = q;
        clo = acc;
      }
      acc = next;
    }
  }
  if (cq < 0) {
    cq = lastq;
    clo = clo_last;
  }
  const int chunk = 4 * __shfl(lane, owner) + __shfl(cq, owner);
  clo = __shfl(clo, owner);

  // lane l: entries chunk * 1024 + 16 l .. + 15
  const int e0 = chunk * kChunk + lane * kPerLane;
  float pr[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) pr[j] = e0 + j < vocab ? logit<T>(row, e0 + j) : 0.f;
  mine = 0.0;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    pr[j] = e0 + j < vocab ? prob_of(pr[j]) : 0.f;
    mine += (double)pr[j];
  }
  incl = wave_incl_scan_d(mine, lane);
  excl = __shfl_up(incl, 1);
  if (lane == 0) excl = 0.0;
  const double lo = clo + excl, hi = clo + incl, end = clo + __shfl(incl, 63);
  claim = __ballot(lo < hi && lo <= target && (target < hi || hi >= end));
  if (!claim) {  // not reachable: the chunk was chosen for holding mass at target
    if (lane == 0) out[blockIdx.x] = -1;
    return;
  }
  owner = __ffsll((unsigned long long)claim) - 1;
  if (lane == owner) {
    int tok = -1, last = -1;
    acc = lo;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      if (pr[j] > 0.f) {
        last = e0 + j;
        acc += (double)pr[j];
        if (tok < 0 && acc > target) tok = e0 + j;
      }
    }
    out[blockIdx.x] = tok >= 0 ? tok : last;
  }
}

template <typename T>
void launch(const void* logits, int rows, int vocab, int64_t row_stride, float temperature, int top_k,
            const double* uniforms, int32_t* tokens, hipStream_t st) {
  hipLaunchKernelGGL((sample_kernel<T>), dim3((unsigned)rows), dim3(kSThreads), 0, st, logits, row_stride, vocab,
                     temperature, top_k, uniforms, tokens);
}

}  // namespace

extern "C" {

int tl_sample_max_vocab(void) { return kMaxVocab; }

int tl_sample(const void* logits, int rows, int vocab, int64_t row_stride, float temperature, int top_k,
              const double* uniforms, int32_t* tokens, int dtype, void* stream) {
  if (rows < 0 || vocab <= 0 || vocab > kMaxVocab || row_stride < vocab || top_k < 0) return TL_ERR_INVALID;
  if (dtype != TL_DTYPE_F32 && dtype != TL_DTYPE_F16 && dtype != TL_DTYPE_BF16) return TL_ERR_INVALID;
  if (rows == 0) return 0;
  if (!logits || !tokens || (temperature > 0.f && !uniforms)) return TL_ERR_INVALID;
  hipStream_t st = tl_resolve_stream(stream);
  switch (dtype) {
    case TL_DTYPE_F32: launch<F32>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, tokens, st); break;
    case TL_DTYPE_F16: launch<F16>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, tokens, st); break;
    default: launch<BF16>(logits, rows, vocab, row_stride, temperature, top_k, uniforms, tokens, st);
  }
  return tl_launch_status();
}

}  // extern "C"
