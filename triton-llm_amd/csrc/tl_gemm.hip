// Dense projections of the model step: C = A . B on the library stream.
//
// Reference behaviour being replaced: triton_llm/kernels/gemm.py:14-108, a
// Triton fp32 tile GEMM (64 x 64 x 32 blocks, tl.dot) used for every
// projection of the model (q/k/v/o, gate/up/down, lm_head).
//
// Two regimes:
//   * a prompt (m > kSkinnyMaxM rows) is a compute-bound GEMM on the matrix
//     cores: gemm_mfma_kernel (128 x 128 tiles, LDS-DMA staging, fp32
//     accumulation); shapes whose rows are not 16-byte aligned take the
//     simple fp32-FMA gemm_simple_kernel.  A batch of decoded tokens (a few
//     dozen rows) has too few tiles to fill the device: K is split into
//     slices with fp32 partials and a reduce pass, and up to 64 rows take
//     64-row tiles;
//   * a decoded token (m <= kSkinnyMaxM rows) reads every weight once for a
//     handful of multiply-adds per element: an HBM-bound skinny product,
//     where rocBLAS measured 0.4-0.7 TB/s.  skinny_partial_kernel cuts B
//     into (64-column x TK-row) tiles, about a thousand of them, so enough
//     weight bytes are in flight to stream at HBM speed; each tile's
//     partial sums go to the workspace and skinny_reduce_kernel adds the
//     K-slices and rounds to the output type.
#include "tl_common.h"

namespace {

constexpr int kSkinnyMaxM = 8;     // rows of A handled by the skinny path
constexpr int kMaxSmallSplit = 32; // K-slices at most for few-row MFMA products
// 64-row tiles for at most 64 rows: half the padding MFMA work of 128-row
// tiles (Llama-3.2-3B layer at 9-64 rows: fp32 286-300 -> 169-189 us, bf16
// 84.5 -> 73.7 us at 9 rows); 16-bit keeps 64 k per stage in two stages
// (32 k in four measured 3-5% slower).
constexpr int kNarrowMaxM = 64;
constexpr int kNarrowBkb16 = 128;
constexpr int kNarrowNst16 = 2;
// fp32 MFMA kernels, k per LDS stage: 16, except 32 for the 64-row tiles a
// prompt takes by the occupancy model below (72 KiB in three stages, still
// two workgroups per CU; SmolLM2-360M's fp32 prompt layer 387 -> 380 us).
// Few rows keep 16 (a Llama-3.2-3B layer at 64 rows: 183 against 194 us
// with 32), and so do 128-row tiles (32 would need 96 KiB: one workgroup
// per CU).
constexpr int kF32Bk = 16;
constexpr int kF32BkDeep = 32;
constexpr int kSkThreads = 256;    // 4 waves
constexpr int kSkUnroll = 16;      // row loads in flight per lane
constexpr int kSkMaxTk = 1024;     // rows per K-slice at most (A's slice is staged in LDS)
constexpr int kSkRowsPerStep = 16; // rows one workgroup load instruction round covers
constexpr int kSkTargetTiles = 1024;
constexpr int kAuxNt = 2;          // buffer-load cache policy: nontemporal (weights are read once)

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

// Products that share A (q/k/v, gate/up): C_g = A . B_g, B_g (k x n_g), for
// g < count, run as one tile space in one launch.  tile0[g] is group g's
// first tile in that space (tile0[count] = all tiles); col0[g] its first
// column in the concatenated width (the split-K partials).
constexpr int kMaxGroups = 4;
struct GemmGroups {
  int count;
  const void* b[kMaxGroups];
  void* c[kMaxGroups];
  int n[kMaxGroups];
  int64_t ldb[kMaxGroups], ldc[kMaxGroups];
  int tile0[kMaxGroups + 1];
  int col0[kMaxGroups + 1];
};

// The group whose tiles (or columns, with col0) include t.
__device__ __forceinline__ int find_group(const int (&first)[kMaxGroups + 1], int count, int t) {
  int g = 0;
#pragma unroll
  for (int i = 1; i < kMaxGroups; ++i)
    if (i < count && t >= first[i]) g = i;
  return g;
}

SkinnyPlan skinny_plan(const GemmGroups& G, int k, int esize) {
  SkinnyPlan s;
  s.cols = 256 / esize;
  s.n_tiles = 0;
  for (int g = 0; g < G.count; ++g) s.n_tiles += (G.n[g] + s.cols - 1) / s.cols;
  const int step = kSkRowsPerStep;
  const int ks_target = kSkTargetTiles / s.n_tiles > 1 ? kSkTargetTiles / s.n_tiles : 1;
  int tk = (k + ks_target - 1) / ks_target;
  tk = (tk + step - 1) / step * step;
  tk = tk < kSkMaxTk ? tk : kSkMaxTk;
  s.tk = tk;
  s.ks = (k + tk - 1) / tk;
  return s;
}

size_t skinny_workspace_bytes(int m, const GemmGroups& G, int k, int esize) {
  const SkinnyPlan s = skinny_plan(G, k, esize);
  if (s.ks == 1) return 0;  // single K-slice: stored to C directly
  size_t ntot = 0;
  for (int g = 0; g < G.count; ++g) ntot += (size_t)G.n[g];
  return (size_t)s.ks * m * ntot * sizeof(float);
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
// blockIdx.x of the groups' tile space.  Lane (wave w, row group r = lane / 16, chunk c = lane % 16)
// reads 16 bytes of row k0 + 16 i + 4 w + r, columns chunk c; its MT x CPC
// sums cover the rows it read.  The four row groups of a wave, then the four
// waves, are added up and the slice's partial product is stored.
// With a single K-slice (gridDim.y == 1) the sums are the result: they are
// rounded and stored to C directly, and no reduce pass follows.
template <typename T, int MT>
__global__ __launch_bounds__(kSkThreads) void skinny_partial_kernel(const void* __restrict__ a, GemmGroups G,
                                                                     float* __restrict__ ws, int m, int k, int64_t lda,
                                                                     int ntot, int tk) {
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
  const int grp = find_group(G.tile0, G.count, blockIdx.x);
  const void* b = G.b[grp];
  const int n = G.n[grp];
  const int64_t ldb = G.ldb[grp];
  // The tile's rows of B as one buffer that ends at the last row's last
  // column inside the matrix: loads of rows past the slice read zeros with no
  // memory access.  (Chunks past column n of earlier rows read the next
  // row's data; those columns are never stored.)
  const int tile_col0 = (blockIdx.x - G.tile0[grp]) * COLS;
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
    const int col = tile_col0 + cc;
    if (mi < m && col < n) {
      const float v = s_sum[0][mi][cc] + s_sum[1][mi][cc] + s_sum[2][mi][cc] + s_sum[3][mi][cc];
      if (gridDim.y == 1)
        ((Bits*)G.c[grp])[(int64_t)mi * G.ldc[grp] + col] = from_f32<T>(v);
      else
        ws[((int64_t)blockIdx.y * m + mi) * ntot + G.col0[grp] + col] = v;
    }
  }
}

// C_g[mi][col] = sum over K-slices of the partials, rounded to T, for every
// column of the concatenated width.  The sum is latency-bound: up to
// kReduceBatch slices' loads are in flight at once (one round trip for the
// usual 4-24 slices), added in slice order.
constexpr int kReduceBatch = 32;  // measured: SmolLM2-360M one-token layer 41.0 -> 37.5 us against 8
template <typename T>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ ws, GemmGroups G, int m, int ntot,
                                                            int ks) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)m * ntot) return;
  const int mi = (int)(idx / ntot), colg = (int)(idx % ntot);
  const int grp = find_group(G.col0, G.count, colg);
  const int64_t stride = (int64_t)m * ntot;
  float s = 0.f;
  for (int q0 = 0; q0 < ks; q0 += kReduceBatch) {
    float v[kReduceBatch];
#pragma unroll
    for (int j = 0; j < kReduceBatch; ++j) v[j] = q0 + j < ks ? ws[(int64_t)(q0 + j) * stride + idx] : 0.f;
#pragma unroll
    for (int j = 0; j < kReduceBatch; ++j) s += v[j];
  }
  ((typename T::bits*)G.c[grp])[(int64_t)mi * G.ldc[grp] + (colg - G.col0[grp])] = from_f32<T>(s);
}

template <typename T>
int launch_skinny(const void* a, GemmGroups G, int m, int k, int64_t lda, void* ws, hipStream_t st) {
  const SkinnyPlan s = skinny_plan(G, k, T::size);
  int ntot = 0;
  G.tile0[0] = 0;
  G.col0[0] = 0;
  for (int g = 0; g < G.count; ++g) {
    G.tile0[g + 1] = G.tile0[g] + (G.n[g] + s.cols - 1) / s.cols;
    G.col0[g + 1] = G.col0[g] + G.n[g];
    ntot += G.n[g];
  }
  dim3 grid((unsigned)s.n_tiles, (unsigned)s.ks);
  float* w = (float*)ws;
  if (m <= 1)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 1>), grid, dim3(kSkThreads), 0, st, a, G, w, m, k, lda, ntot, s.tk);
  else if (m <= 2)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 2>), grid, dim3(kSkThreads), 0, st, a, G, w, m, k, lda, ntot, s.tk);
  else if (m <= 4)
    hipLaunchKernelGGL((skinny_partial_kernel<T, 4>), grid, dim3(kSkThreads), 0, st, a, G, w, m, k, lda, ntot, s.tk);
  else
    hipLaunchKernelGGL((skinny_partial_kernel<T, 8>), grid, dim3(kSkThreads), 0, st, a, G, w, m, k, lda, ntot, s.tk);
  int e = tl_launch_status();
  if (e || s.ks == 1) return e;
  const int64_t outs = (int64_t)m * ntot;
  hipLaunchKernelGGL((skinny_reduce_kernel<T>), dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, st,
                     (const float*)ws, G, m, ntot, s.ks);
  return tl_launch_status();
}

// ---------------------------------------------------------------------------
// Prompt-sized products on the matrix cores (m > kSkinnyMaxM).
//
// Workgroup tile 128 x 128 of C, 4 waves in 2 x 2, each wave 64 x 64 (2 x 2
// blocks of 32 x 32).  K is walked in LDS stages (16-bit: 64 k in two
// stages; fp32: 16 k in three, 32 k for the 64-row prompt plans), every
// tile moved global -> LDS by LDS-DMA
// (buffer_load ... lds: no register round trip), every wave loading a
// quarter.  Each wave computes the transposed block C^T = B^T . A^T with
// the MFMA, so a lane ends up owning one row of C and 4 consecutive columns
// per accumulator group: stores are 8 (16-bit) or 16 (fp32) contiguous bytes.
//
// Operand layouts in LDS (rows unpadded, 16-byte chunks XOR-swizzled so that
// every operand read is conflict-free):
//   A stage: 128 rows (m) x BKB bytes (k), chunk c of row r at slot
//            c ^ a_swz(r).  A fragment: lane (l % 32, h = l / 32) reads
//            one 16-byte chunk of row l % 32 of its block: 8 consecutive k
//            (16-bit) or 4 (fp32).
//   B stage, 16-bit: 64 rows (k) x 256 bytes (n), chunk c of row r at slot
//            c ^ (4 (r % 4)).  The MFMA wants 8 consecutive k of one column
//            per lane, i.e. B read down a column: two ds_read_b64_tr_b16.
//            That instruction transposes within each 16-lane group: output
//            lane j, element e is element j % 4 of what lane 4 e + j / 4 of
//            the group read.  So lane 4 e + p of group g reads row
//            8 (g / 2) + 4 t + e, columns n0 + 16 (g % 2) + 4 p .. + 3, and
//            lane 16 g + j receives column n0 + 16 (g % 2) + j, rows
//            8 (g / 2) + 4 t + 0..3 (t = 0, 1: the two reads).
//   B stage, fp32: 16 rows (k) x 512 bytes (n), chunk c of row r at slot
//            c ^ (8 ((r >> 2) & 1)); a lane reads one float of its column.
// fp32 uses v_mfma_f32_32x32x2f32 with the k order permuted: in k-group q
// (8 k), step s, lane half h uses k = 8 q + 4 h + s, so one 16-byte A read
// feeds 4 steps.
// ---------------------------------------------------------------------------
constexpr int kGmTile = 128;
constexpr int kGmThreads = 256;

struct GemmParams {
  const void* a;
  int m, k;
  int64_t lda;
  GemmGroups G;   // tile0 counts 128 x 128 tiles of C
  int tiles_m, per_xcd;
  int vec_store;  // bit g: C_g's rows and base allow 4-column vector stores
  // Split K (ksplit > 1): item (slice s, tile t) covers stages
  // [s kt_per, (s + 1) kt_per) and stores its fp32 partial tile at
  // ws + ws_off[g] + (s m + row) n_g + col; split_reduce_kernel sums them.
  int ksplit, kt_per;
  float* ws;
  int64_t ws_off[kMaxGroups];
};

// Work item of workgroup L: each XCD (workgroups are dealt to the 8 XCDs in
// turn) takes a contiguous run of items, row tiles fastest, so the
// workgroups an XCD runs at once share their B column tiles and A row tiles
// in its L2; items are slice-major (all tiles of K-slice 0, then slice 1).
__device__ __forceinline__ bool gemm_tile(const GemmParams& p, int& grp, int& tm, int& tn, int& ks) {
  const int L = blockIdx.x;
  const int it = (L % 8) * p.per_xcd + L / 8;
  const int tiles = p.G.tile0[p.G.count];
  if (it >= tiles * p.ksplit) return false;
  ks = it / tiles;
  const int t = it - ks * tiles;
  grp = find_group(p.G.tile0, p.G.count, t);
  const int local = t - p.G.tile0[grp];
  tm = local % p.tiles_m;
  tn = local / p.tiles_m;
  return true;
}

// BKB: bytes of k per A row per stage (64 or 128); NST: stages in LDS; MBW:
// 32-row blocks per wave along m (1: 64 x 128 tiles for few rows, 2: 128 x
// 128 tiles, 4: 256 x 128 tiles, where each B fragment a wave reads feeds
// four MFMAs instead of two); NWV: waves (4, or 8 for 16-bit 256 x 256 tiles:
// two along m by four along n, B staged as 512-byte rows, one workgroup per
// CU, half the operand bytes staged per MFMA of two 256 x 128 workgroups).
template <typename T, int BKB, int NST, int MBW, int NWV = 4>
__global__ __launch_bounds__(64 * NWV, NWV == 8 ? 1 : 2) void gemm_mfma_kernel(GemmParams p) {
  constexpr bool F32 = T::size == 4;
  constexpr int TM = 64 * MBW;                // rows of C per tile
  constexpr int BK = BKB / T::size;           // k per stage
  constexpr int ACH = BKB / 16;               // 16-byte chunks per A row (4 or 8)
  constexpr int TN = 32 * NWV;               // columns of C per tile (128 or 256)
  constexpr int BROW = TN * T::size;          // bytes per B row in LDS
  constexpr int NQ = F32 ? BK / 8 : BK / 16;  // fp32 k-groups / 16-bit k-steps per stage
  constexpr int kGmStages = NST;
  constexpr int kGmStageA = TM * BKB;         // bytes of one A stage
  constexpr int kGmStageB = BK * BROW;        // bytes of one B stage
  static_assert(kGmStageA % (1024 * NWV) == 0 && kGmStageB % (1024 * NWV) == 0, "every wave loads whole 1 KiB regions");
  static_assert(NWV == 4 || !F32, "eight waves: 16-bit only");
  using Bits = typename T::bits;
  __shared__ __attribute__((aligned(1024))) char smem[kGmStages * (kGmStageA + kGmStageB)];

  // 16 lanes read one chunk of 16 consecutive A rows: the XOR spreads them
  // over all 16 four-bank groups (64-byte rows: bits 2-3 of the row; 128-byte
  // rows: bits 1-3).
  auto a_swz = [](int row) __attribute__((always_inline)) {
    return ACH == 4 ? (row >> 2) & 3 : (row >> 1) & 7;
  };
  int grp, tm, tn, ks;
  if (!gemm_tile(p, grp, tm, tn, ks)) return;
  const int pn = p.G.n[grp];
  const int64_t pldb = p.G.ldb[grp], pldc = p.G.ldc[grp];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int wm = wave & 1, wn = wave >> 1;  // this wave's (32 MBW) x 64 block
  const int m_tile = tm * TM, n_tile = tn * TN;
  __attribute__((address_space(3))) char* const lds_base = (__attribute__((address_space(3))) char*)smem;
  const uint32_t lds0 = (uint32_t)(size_t)lds_base;
  const uint32_t lds_a = lds0, lds_b = lds0 + kGmStages * kGmStageA;

  // Buffer resources over all of A (rows < m) and B (rows < k): rows past
  // them read as zeros with no memory access.
  const uint32_t lda2 = (uint32_t)(p.lda * T::size), ldb2 = (uint32_t)(pldb * T::size);
  const i32x4 ra = uniform_rsrc(p.a, (uint32_t)((uint64_t)p.m * lda2));
  const i32x4 rb = uniform_rsrc(p.G.b[grp], (uint32_t)((uint64_t)p.k * ldb2));
  auto dma = [&](const i32x4& rs, uint32_t voff, uint32_t la) __attribute__((always_inline)) {
    lds_dma16(rs, voff, la);
  };
  // DMA lane offsets (bytes, stage k0 = 0).  A: region R (1 KiB: 1024 / BKB
  // rows) is filled by wave R % 4; lane i -> row R * (1024 / BKB) + i / ACH,
  // slot i % ACH.  The slot swizzle (see a_swz) depends on bits of the row
  // that the region step 4 j does not change, so one offset serves every
  // region of this wave.
  constexpr int A_RPR = 1024 / BKB;
  const int a_row0 = A_RPR * wave + lane / ACH;
  const uint32_t a_off = (uint32_t)(m_tile + a_row0) * lda2 + (uint32_t)(((lane % ACH) ^ a_swz(a_row0)) * 16);
  static_assert(NWV == 4 || BKB == 64, "eight waves: 64-byte A rows (the swizzle bits survive a 128-row step)");
  // B, 16-bit: regions of 4 rows of 256 bytes, lane i -> row 4 R + i / 16,
  // slot i % 16 (swizzle 4 (row % 4) = 4 (i / 16)).  fp32: regions of 2 rows
  // of 512 bytes, lane i -> row 2 R + i / 32, slot i % 32 (swizzle
  // 8 ((row >> 2) & 1) = 8 ((R >> 1) & 1), and R = wave + 4 j keeps that bit).
  uint32_t b_off;
  if constexpr (!F32 && NWV == 8)  // 512-byte rows: regions of 2 rows, lane i -> row 2 R + i / 32
    b_off = (uint32_t)(2 * wave + lane / 32) * ldb2 + (uint32_t)(n_tile * 2) +
            (uint32_t)(((lane % 32) ^ (4 * ((2 * wave + lane / 32) & 3))) * 16);
  else if constexpr (!F32)
    b_off = (uint32_t)(4 * wave + lane / 16) * ldb2 + (uint32_t)(n_tile * 2) +
            (uint32_t)(((lane % 16) ^ (4 * (lane / 16))) * 16);
  else
    b_off = (uint32_t)(2 * wave + lane / 32) * ldb2 + (uint32_t)(n_tile * 4) +
            (uint32_t)(((lane % 32) ^ (8 * ((wave >> 1) & 1))) * 16);
  constexpr int A_REG = kGmStageA / 1024 / NWV;  // regions per wave per stage
  constexpr int B_REG = kGmStageB / 1024 / NWV;
  constexpr int B_RPR = 1024 / BROW;           // B rows per region
  auto load_stage = [&](int kt, int buf) __attribute__((always_inline)) {
    const uint32_t ka = (uint32_t)(kt * BK * T::size);  // A: column bytes of the stage
    const uint32_t kb = (uint32_t)(kt * BK) * ldb2;     // B: row offset of the stage
#pragma unroll
    for (int j = 0; j < A_REG; ++j)
      dma(ra, a_off + ka + (uint32_t)(NWV * A_RPR * j) * lda2, lds_a + buf * kGmStageA + (wave + NWV * j) * 1024);
#pragma unroll
    for (int j = 0; j < B_REG; ++j)
      dma(rb, b_off + kb + (uint32_t)(NWV * B_RPR * j) * ldb2, lds_b + buf * kGmStageB + (wave + NWV * j) * 1024);
  };

  f32x16 acc[MBW][2];  // [m block][n block], C^T layout
#pragma unroll
  for (int i = 0; i < MBW; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Operand read offsets inside a stage.
  const int lq = lane & 31, h = lane >> 5;
  // A: row 32 MBW wm + 32 mb + lq, chunk c at slot c ^ a_swz(row).
  auto a_addr = [&](int mb, int c) __attribute__((always_inline)) {
    const int row = 32 * MBW * wm + 32 * mb + lq;
    return row * BKB + ((c ^ a_swz(row)) << 4);
  };
  const int n_kt = (p.k + BK - 1) / BK;
  const int k_rem = p.k - (n_kt - 1) * BK;  // valid k of the last stage
  const int kt_lo = ks * p.kt_per;          // this item's stages
  const int kt_hi = min(n_kt, kt_lo + p.kt_per);

#pragma unroll
  for (int s = 0; s < kGmStages - 1; ++s)
    if (kt_lo + s < kt_hi) load_stage(kt_lo + s, (kt_lo + s) % kGmStages);

  for (int kt = kt_lo; kt < kt_hi; ++kt) {
    // stage kt has landed (this wave's loads; the barrier covers the others'):
    // the stages issued after it, up to NST - 2 of them, may stay in flight
    constexpr int PER = A_REG + B_REG;
    if constexpr (NST >= 4) {
      if (kt + 2 < kt_hi) wait_vmcnt<2 * PER>();
      else if (kt + 1 < kt_hi) wait_vmcnt<PER>();
      else wait_vmcnt<0>();
    } else if constexpr (NST == 3) {
      if (kt + 1 < kt_hi) wait_vmcnt<PER>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    if (kt + kGmStages - 1 < kt_hi) load_stage(kt + kGmStages - 1, (kt + kGmStages - 1) % kGmStages);
    const int buf = kt % kGmStages;
    const char* sa = smem + buf * kGmStageA;
    const char* sb = smem + kGmStages * kGmStageA + buf * kGmStageB;
    const bool tail = kt == n_kt - 1 && k_rem < BK;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if constexpr (!F32) {
        // k-step q: k = 16 q + 8 h + 0..7 of the stage.
        bf16x8 af[MBW];
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) {
          u32x4 raw = *(const u32x4*)(sa + a_addr(mb, 2 * q + h));
          if (tail) {
            uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (16 * q + 8 * h + e >= k_rem) w[e / 2] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
            raw = u32x4{w[0], w[1], w[2], w[3]};
          }
          af[mb] = __builtin_bit_cast(bf16x8, raw);
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          // lane 16 g + 4 e + p reads row 16 q + 8 (g / 2) + 4 t + e, column
          // chunk of n = 64 wn + 32 nb + 16 (g % 2) + 4 p.
          const int g = lane >> 4, e = (lane >> 2) & 3, pp = lane & 3;
          const int row = 16 * q + 8 * (g >> 1) + e;
          const int n = 64 * wn + 32 * nb + 16 * (g & 1) + 4 * pp;
          const int addr = row * BROW + ((((n >> 3)) ^ (4 * (row & 3))) << 4) + 8 * ((n >> 2) & 1);
          typedef short v4s __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) v4s lds_v4s;
          const int boff = kGmStages * kGmStageA + buf * kGmStageB + addr;
          const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds_base + boff));
          const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds_base + boff + 4 * BROW));
          const u32x4 braw = u32x4{__builtin_bit_cast(u32x2, lo).x, __builtin_bit_cast(u32x2, lo).y,
                                   __builtin_bit_cast(u32x2, hi).x, __builtin_bit_cast(u32x2, hi).y};
#pragma unroll
          for (int mb = 0; mb < MBW; ++mb)
            acc[mb][nb] = Mfma<T>::mma(__builtin_bit_cast(typename Mfma<T>::frag, braw),
                                       __builtin_bit_cast(typename Mfma<T>::frag, af[mb]), acc[mb][nb]);
        }
      } else {
        // k-group q: k = 8 q + 4 h + s, s = 0..3.
        f32x4 af[MBW];
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) {
          f32x4 v = *(const f32x4*)(sa + a_addr(mb, 2 * q + h));
          if (tail) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
              if (8 * q + 4 * h + s >= k_rem) v[s] = 0.f;
          }
          af[mb] = v;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int row = 8 * q + 4 * h + s;
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) {
            const int byte = (64 * wn + 32 * nb + lq) * 4;
            const float bv = *(const float*)(sb + row * BROW + (byte ^ (128 * ((row >> 2) & 1))));
#pragma unroll
            for (int mb = 0; mb < MBW; ++mb)
              acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv, af[mb][s], acc[mb][nb], 0, 0, 0);
          }
        }
      }
    }
  }
  wait_vmcnt<0>();

  // lane (lq, h) holds row m = m_tile + 32 MBW wm + 32 mb + lq and, for
  // a = 0..3, columns n = n_tile + 64 wn + 32 nb + 8 a + 4 h + 0..3.
  if (p.ksplit > 1) {
    // fp32 partial of this K-slice; n_g is a multiple of 4 on this path, so
    // every 4-column run is whole and 16-byte aligned
    float* wsb = p.ws + p.ws_off[grp] + (int64_t)ks * p.m * pn;
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb) {
      const int m = m_tile + 32 * MBW * wm + 32 * mb + lq;
      if (m >= p.m) continue;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const int n = n_tile + 64 * wn + 32 * nb + 8 * a + 4 * h;
          if (n < pn)
            *(f32x4*)(wsb + (int64_t)m * pn + n) =
                f32x4{acc[mb][nb][4 * a], acc[mb][nb][4 * a + 1], acc[mb][nb][4 * a + 2], acc[mb][nb][4 * a + 3]};
        }
    }
    return;
  }
  Bits* cbase = (Bits*)p.G.c[grp];
  const bool vec = (p.vec_store >> grp) & 1;
#pragma unroll
  for (int mb = 0; mb < MBW; ++mb) {
    const int m = m_tile + 32 * MBW * wm + 32 * mb + lq;
    if (m >= p.m) continue;
    Bits* crow = cbase + (int64_t)m * pldc;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int n = n_tile + 64 * wn + 32 * nb + 8 * a + 4 * h;
        const float v[4] = {acc[mb][nb][4 * a], acc[mb][nb][4 * a + 1], acc[mb][nb][4 * a + 2],
                            acc[mb][nb][4 * a + 3]};
        if (vec && n + 3 < pn) {
          if constexpr (F32) {
            *(f32x4*)(crow + n) = f32x4{v[0], v[1], v[2], v[3]};
          } else {
            const float x0[2] = {v[0], v[1]}, x1[2] = {v[2], v[3]};
            *(u32x2*)(crow + n) = u32x2{pack2<T>(x0), pack2<T>(x1)};
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < pn) crow[n + e] = from_f32<T>(v[e]);
        }
      }
  }
}

// Split-K finish: C_g = sum over the K-slices of the fp32 partial tiles
// (slice 0 first, so the result does not depend on timing), rounded to T.
// One 4-column run per thread, grid-stride; blockIdx.y = group.
template <typename T>
__global__ __launch_bounds__(256) void split_reduce_kernel(GemmParams p) {
  using Bits = typename T::bits;
  const int g = blockIdx.y;
  const int n = p.G.n[g];
  const int q4 = n / 4;
  const int runs = p.m * q4;
  const float* w = p.ws + p.ws_off[g];
  const int64_t slice = (int64_t)p.m * n;
  Bits* c = (Bits*)p.G.c[g];
  const int64_t ldc = p.G.ldc[g];
  const bool vec = (p.vec_store >> g) & 1;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < runs; i += gridDim.x * 256) {
    const int r = i / q4;
    const int col = (i - r * q4) * 4;
    f32x4 sum = *(const f32x4*)(w + (int64_t)r * n + col);
    for (int ks = 1; ks < p.ksplit; ++ks) sum += *(const f32x4*)(w + ks * slice + (int64_t)r * n + col);
    Bits* dst = c + (int64_t)r * ldc + col;
    if constexpr (T::size == 4) {
      if (vec) {
        *(f32x4*)dst = sum;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(sum[e]);
      }
    } else {
      const float x0[2] = {sum[0], sum[1]}, x1[2] = {sum[2], sum[3]};
      if (vec) {
        *(u32x2*)dst = u32x2{pack2<T>(x0), pack2<T>(x1)};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = from_f32<T>(sum[e]);
      }
    }
  }
}

// Any shape and alignment (the MFMA kernel needs 16-byte aligned rows):
// 64 x 64 tiles of C_g (g = blockIdx.z), 256 threads with 4 x 4 outputs
// each, fp32 FMA over 16-deep K slices staged in LDS with bounds checks.
// Used for small or odd shapes only.
template <typename T>
__global__ __launch_bounds__(256) void gemm_simple_kernel(GemmParams p) {
  using Bits = typename T::bits;
  __shared__ float sa[16][65];
  __shared__ float sb[16][65];
  const int grp = blockIdx.z;
  const int n_g = p.G.n[grp];
  const Bits* bg = (const Bits*)p.G.b[grp];
  const int64_t ldb = p.G.ldb[grp];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  if (n0 >= n_g) return;  // the grid spans the widest group
  float acc[4][4] = {};
  for (int k0 = 0; k0 < p.k; k0 += 16) {
    for (int i = threadIdx.x; i < 16 * 64; i += 256) {
      const int kk = i / 64, mm = i % 64;
      const int m = m0 + mm, k = k0 + kk;
      sa[kk][mm] = (m < p.m && k < p.k) ? to_f32<T>(((const Bits*)p.a)[(int64_t)m * p.lda + k]) : 0.f;
      const int n = n0 + mm;
      sb[kk][mm] = (n < n_g && k < p.k) ? to_f32<T>(bg[(int64_t)k * ldb + n]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(sa[kk][ty * 4 + i], sb[kk][tx * 4 + j], acc[i][j]);
    __syncthreads();
  }
  Bits* cg = (Bits*)p.G.c[grp];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m < p.m && n < n_g) cg[(int64_t)m * p.G.ldc[grp] + n] = from_f32<T>(acc[i][j]);
    }
}

// How a prompt-sized product runs on the MFMA kernel: tile height and K split.
struct PromptPlan {
  bool huge;      // 16-bit 256 x 256 tiles (eight waves)
  bool narrow;    // 64 x 128 tiles (few rows: half the padding of 128-row tiles)
  bool f32_deep;  // fp32 64-row tiles with 32-k stages (prompts)
  int tiles_m, tiles;
  int ksplit, kt_per;
  size_t ws_bytes;  // fp32 partials when split
};

// 16-bit: 256 x 256 tiles (eight waves, one workgroup per CU; each B
// fragment feeds four MFMAs) where they still give every CU two: at a
// 2048-row Llama-3.2-3B prompt gate/up 206-209 -> 191 us, the layer
// 456-462 -> 442 us.  Fewer, larger tiles leave CUs idle on the narrower
// products (q/k/v, o and down keep 128 x 128).  (A 256 x 128 tile, taken
// at four or more per CU, measured gate/up 226 -> 219 us; every shape with
// four such tiles per CU has at least two 256 x 256 ones, so it was never
// reached once those existed, and it was removed.)
//
// K split (fp32): a CU's time is set by the items it runs, and a whole tile
// is the unit, so 384 tiles on 256 CUs cost two tiles' time where 1.5 would
// do.  Splitting K in S slices makes the unit 1 / S of a tile at the price of
// a reduce pass over S fp32 partials; S (1..4, at least 4 stages per slice)
// is the one with the least modelled time, and a split must win by 3%.
// Measured at a 2048-row Llama-3.2-3B prompt, fp32: q/k/v 583 -> 520, o
// 403 -> 317, down 1061 -> 805 us (S = 2).  16-bit products are not split:
// at their speed the partials' traffic cost more than the balance gained
// (bf16 down 118 -> 127 us with S = 2).
PromptPlan prompt_plan(int m, int k, const GemmGroups& G, int esize) {
  PromptPlan P{};
  const int cus = tl_device_cus();
  int64_t ncols = 0;
  for (int g = 0; g < G.count; ++g) ncols += G.n[g];
  int huge_tiles = 0;
  for (int g = 0; g < G.count; ++g)
    huge_tiles += ((m + 2 * kGmTile - 1) / (2 * kGmTile)) * ((G.n[g] + 2 * kGmTile - 1) / (2 * kGmTile));
  P.huge = esize == 2 && huge_tiles >= 2 * cus;
  P.narrow = !P.huge && m <= kNarrowMaxM;
  const int tm = P.huge ? 2 * kGmTile : (P.narrow ? kGmTile / 2 : kGmTile);
  P.tiles_m = (m + tm - 1) / tm;
  P.tiles = 0;
  const int tn = P.huge ? 2 * kGmTile : kGmTile;
  for (int g = 0; g < G.count; ++g) P.tiles += P.tiles_m * ((G.n[g] + tn - 1) / tn);
  // k per LDS stage of the kernel used
  const int bk = esize == 2 ? (P.huge ? 32 : (P.narrow ? kNarrowBkb16 / 2 : 64)) : kF32Bk;
  int n_kt = (k + bk - 1) / bk;
  // modelled seconds: the product at a sustained rate, scaled by the busiest
  // CU's share of items; the reduce as HBM traffic plus a launch
  const double rate = esize == 2 ? 9.0e14 : 1.3e14;
  const double t1 = 2.0 * m * (double)k * (double)ncols / rate;
  auto busiest = [&](int S) { return (double)((P.tiles * (int64_t)S + cus - 1) / cus) / S; };
  auto reduce_t = [&](int S) { return ((double)S * 4 + esize) * m * (double)ncols / 5.0e12 + 3e-6; };
  double best = t1;
  P.ksplit = 1;
  // Few rows (a batch of decoded tokens): the product streams B, and a few
  // dozen tiles of C, each walking all of K, leave most CUs idle (a
  // workgroup streams only tens of GB/s).  Split K until about one item per
  // CU runs for 16-bit products and two for fp32 ones (measured, Llama-3.2-3B
  // layer at 9-64 rows: bf16 74-91 us with two per CU against 67-81 us with
  // one; fp32 168-184 us against 198-208), while the fp32 partials stay
  // under half of B's bytes (which rules out large m) and every slice keeps
  // two stages.
  if (P.tiles < 2 * cus) {
    const int64_t by_traffic = (int64_t)k * esize / (2 * 4 * (int64_t)m);
    const int per_cu = esize == 2 ? 1 : 2;
    int64_t S = (per_cu * cus + P.tiles - 1) / P.tiles;
    S = S < by_traffic ? S : by_traffic;
    S = S < n_kt / 2 ? S : n_kt / 2;
    S = S < kMaxSmallSplit ? S : kMaxSmallSplit;
    if (S >= 2) {
      P.ksplit = (int)S;
      P.kt_per = (n_kt + P.ksplit - 1) / P.ksplit;
      P.ws_bytes = (size_t)P.ksplit * m * ncols * sizeof(float);
      return P;
    }
  }
  for (int S = 2; S <= 4 && esize == 4; ++S) {
    if (n_kt < 4 * S) break;
    const double t = t1 * busiest(S) / busiest(1) + reduce_t(S);
    if (t < 0.97 * best) {
      best = t;
      P.ksplit = S;
    }
  }
  if (esize == 4 && !P.narrow) {
    // fp32 with 64-row tiles instead, when a model of the busiest CU's items
    // says they win by 3%.  A CU runs two items at once at the sustained
    // rate; a lone item runs at about 0.7 of it (one 128 x 128 fp32
    // workgroup alone on a CU reaches 58% of the CU's MFMA peak, two
    // together 82%), and a 64-row tile does its FLOPs at about 0.865 of a
    // 128-row tile's rate (Llama-3.2-3B o at 2048 rows, K split in 2 either
    // way: 321 against 316 us).  More items of 64 rows fill the CUs that a
    // few 128-row tiles leave with one item or none (SmolLM2-360M at 2048
    // rows: grouped q/k/v 78 -> 73 us, gate/up 191 -> 166 us).
    const double r2 = rate / cus, r1 = r2 * (0.58 / 0.82);
    auto model = [&](int ctm, int S) {
      int64_t ctiles = 0;
      for (int g = 0; g < G.count; ++g) ctiles += (int64_t)((m + ctm - 1) / ctm) * ((G.n[g] + kGmTile - 1) / kGmTile);
      const int64_t per_cu = (ctiles * S + cus - 1) / cus;
      const double w = 2.0 * ctm * kGmTile * (double)k / S / (ctm < kGmTile ? 0.865 : 1.0);
      return (double)(per_cu - per_cu % 2) * w / r2 + (double)(per_cu % 2) * w / r1 + (S > 1 ? reduce_t(S) : 0.0);
    };
    const double t_cur = model(kGmTile, P.ksplit);
    double t_best = 0.97 * t_cur;
    int best_s = 0;
    const int n_kt64 = (k + kF32BkDeep - 1) / kF32BkDeep;
    for (int S = 1; S <= 4; ++S) {
      if (S > 1 && n_kt64 < 4 * S) break;
      const double t = model(kGmTile / 2, S);
      if (t < t_best) {
        t_best = t;
        best_s = S;
      }
    }
    if (best_s) {
      P.narrow = true;
      P.tiles_m = (m + kGmTile / 2 - 1) / (kGmTile / 2);
      P.tiles = 0;
      for (int g = 0; g < G.count; ++g) P.tiles += P.tiles_m * ((G.n[g] + kGmTile - 1) / kGmTile);
      P.ksplit = best_s;
      P.f32_deep = true;
      n_kt = n_kt64;
    }
  }
  P.kt_per = (n_kt + P.ksplit - 1) / P.ksplit;
  P.ws_bytes = P.ksplit > 1 ? (size_t)P.ksplit * m * ncols * sizeof(float) : 0;
  return P;
}

template <typename T>
int launch_gemm(const void* a, const GemmGroups& G, int m, int k, int64_t lda, void* workspace,
                size_t workspace_bytes, hipStream_t st) {
  GemmParams p{};
  p.a = a;
  p.m = m;
  p.k = k;
  p.lda = lda;
  p.G = G;
  const int64_t esize = T::size;
  const int64_t vec = 16 / esize;  // elements per 16-byte chunk
  // Every operand's rows must be 16-byte aligned for the LDS-DMA staging, and
  // all of A and each B addressable with 32-bit offsets (stage reads run up
  // to one stage past the last row / k).
  bool aligned = lda % vec == 0 && ((uintptr_t)a % 16) == 0 &&
                 ((int64_t)m + 2 * kGmTile + 1) * lda * esize < ((int64_t)1 << 32);
  int widest = 0;
  for (int g = 0; g < G.count; ++g) {
    aligned = aligned && G.ldb[g] % vec == 0 && G.n[g] % vec == 0 && ((uintptr_t)G.b[g] % 16) == 0 &&
              ((int64_t)k + 64 + 1) * G.ldb[g] * esize < ((int64_t)1 << 32);
    widest = G.n[g] > widest ? G.n[g] : widest;
  }
  if (aligned) {
    const PromptPlan P = prompt_plan(m, k, G, (int)esize);
    p.tiles_m = P.tiles_m;
    p.G.tile0[0] = 0;
    p.vec_store = 0;
    for (int g = 0; g < G.count; ++g) {
      const int tn = P.huge ? 2 * kGmTile : kGmTile;
      p.G.tile0[g + 1] = p.G.tile0[g] + p.tiles_m * ((G.n[g] + tn - 1) / tn);
      if (G.ldc[g] % 4 == 0 && ((uintptr_t)G.c[g] % (4 * esize)) == 0) p.vec_store |= 1 << g;
    }
    // the split needs its partials' workspace; without it the product runs whole
    const bool split = P.ksplit > 1 && workspace && workspace_bytes >= P.ws_bytes && ((uintptr_t)workspace % 16) == 0;
    p.ksplit = split ? P.ksplit : 1;
    p.kt_per = split ? P.kt_per : (k + 15) / 16 + 1;  // whole: one slice covers every stage
    p.ws = (float*)workspace;
    int64_t off = 0;
    for (int g = 0; g < G.count; ++g) {
      p.ws_off[g] = off;
      off += (int64_t)p.ksplit * m * G.n[g];
    }
    p.per_xcd = (p.G.tile0[G.count] * p.ksplit + 7) / 8;
    // Measured at the models' prompt shapes (2048 rows): 16-bit runs best
    // with 64 k per stage in two stages (729 against 645 TFLOP/s with 32 k
    // in three, 691 with 32 k in four, 507 with 64 k in three); fp32 is
    // within 1% across those and keeps 16 k in three stages, except the
    // 64-row tiles a prompt takes by the occupancy model (kF32BkDeep).
    const dim3 grid((unsigned)(8 * p.per_xcd));
    if constexpr (T::size == 2) {
      if (P.huge)
        hipLaunchKernelGGL((gemm_mfma_kernel<T, 64, 3, 4, 8>), grid, dim3(512), 0, st, p);
      else if (P.narrow)
        hipLaunchKernelGGL((gemm_mfma_kernel<T, kNarrowBkb16, kNarrowNst16, 1>), grid, dim3(kGmThreads), 0, st, p);
      else
        hipLaunchKernelGGL((gemm_mfma_kernel<T, 128, 2, 2>), grid, dim3(kGmThreads), 0, st, p);
    } else {
      if (P.narrow && P.f32_deep)
        hipLaunchKernelGGL((gemm_mfma_kernel<T, 4 * kF32BkDeep, 3, 1>), grid, dim3(kGmThreads), 0, st, p);
      else if (P.narrow)
        hipLaunchKernelGGL((gemm_mfma_kernel<T, 4 * kF32Bk, 3, 1>), grid, dim3(kGmThreads), 0, st, p);
      else
        hipLaunchKernelGGL((gemm_mfma_kernel<T, 4 * kF32Bk, 3, 2>), grid, dim3(kGmThreads), 0, st, p);
    }
    int e = tl_launch_status();
    if (e || p.ksplit == 1) return e;
    int64_t runs = 0;
    for (int g = 0; g < G.count; ++g) runs = (int64_t)m * (G.n[g] / 4) > runs ? (int64_t)m * (G.n[g] / 4) : runs;
    const unsigned rb = (unsigned)((runs + 255) / 256 < 4096 ? (runs + 255) / 256 : 4096);
    hipLaunchKernelGGL((split_reduce_kernel<T>), dim3(rb, G.count), dim3(256), 0, st, p);
    return tl_launch_status();
  }
  dim3 grid((unsigned)((widest + 63) / 64), (unsigned)((m + 63) / 64), (unsigned)G.count);
  hipLaunchKernelGGL((gemm_simple_kernel<T>), grid, dim3(256), 0, st, p);
  return tl_launch_status();
}

// Checks shared by both entry points; fills the group table.
int make_groups(GemmGroups& G, int count, const void* const* b, void* const* c, const int* n, const int64_t* ldb,
                const int64_t* ldc) {
  if (count < 1 || count > kMaxGroups || !b || !c || !n || !ldb || !ldc) return TL_ERR_INVALID;
  G = GemmGroups{};
  G.count = count;
  for (int g = 0; g < count; ++g) {
    G.b[g] = b[g];
    G.c[g] = c[g];
    G.n[g] = n[g];
    G.ldb[g] = ldb[g];
    G.ldc[g] = ldc[g];
  }
  return 0;
}

int gemm_groups(const void* a, const GemmGroups& G, int m, int k, int64_t lda, void* workspace,
                size_t workspace_bytes, int dtype, void* stream) {
  if (m < 0 || k < 0) return TL_ERR_INVALID;
  if (dtype != TL_DTYPE_F32 && dtype != TL_DTYPE_F16 && dtype != TL_DTYPE_BF16) return TL_ERR_INVALID;
  if (m == 0) return 0;
  for (int g = 0; g < G.count; ++g) {
    if (G.n[g] < 0) return TL_ERR_INVALID;
    if (G.n[g] == 0) continue;
    if (!G.c[g] || G.ldc[g] < G.n[g] || (k > 0 && (!G.b[g] || G.ldb[g] < G.n[g]))) return TL_ERR_INVALID;
    if (!fits_int(G.ldb[g]) || !fits_int(G.ldc[g])) return TL_ERR_UNSUPPORTED;
  }
  if (k > 0 && (!a || lda < k)) return TL_ERR_INVALID;
  if (!fits_int(lda)) return TL_ERR_UNSUPPORTED;
  const size_t esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  hipStream_t st = tl_resolve_stream(stream);
  // Groups with no columns take no part.
  GemmGroups live{};
  for (int g = 0; g < G.count; ++g) {
    if (G.n[g] == 0) continue;
    const int i = live.count++;
    live.b[i] = G.b[g];
    live.c[i] = G.c[g];
    live.n[i] = G.n[g];
    live.ldb[i] = G.ldb[g];
    live.ldc[i] = G.ldc[g];
  }
  if (live.count == 0) return 0;
  if (k == 0) {  // empty sum: zeros, row by row when C is a strided view
    for (int g = 0; g < live.count; ++g) {
      if (live.ldc[g] == live.n[g]) {
        const int e = tl_fill_bytes(live.c[g], 0, (size_t)m * live.n[g] * esize, st);
        if (e) return e;
        continue;
      }
      for (int r = 0; r < m; ++r) {
        const int e = tl_fill_bytes((char*)live.c[g] + (size_t)r * live.ldc[g] * esize, 0,
                                    (size_t)live.n[g] * esize, st);
        if (e) return e;
      }
    }
    return 0;
  }
  if (m <= kSkinnyMaxM) {
    bool ok = true;
    const int cpc = 16 / (int)esize;
    for (int g = 0; g < live.count; ++g)
      ok = ok && live.n[g] % cpc == 0 && live.ldb[g] % cpc == 0 && ((uintptr_t)live.b[g] % 16) == 0 &&
           (int64_t)(k - 1) * live.ldb[g] * (int64_t)esize < INT32_MAX;
    if (ok) {
      const size_t need = skinny_workspace_bytes(m, live, k, (int)esize);
      if (need && (!workspace || workspace_bytes < need)) return TL_ERR_INVALID;
      switch (dtype) {
        case TL_DTYPE_F32: return launch_skinny<F32>(a, live, m, k, lda, workspace, st);
        case TL_DTYPE_F16: return launch_skinny<F16>(a, live, m, k, lda, workspace, st);
        default: return launch_skinny<BF16>(a, live, m, k, lda, workspace, st);
      }
    }
  }
  switch (dtype) {
    case TL_DTYPE_F32: return launch_gemm<F32>(a, live, m, k, lda, workspace, workspace_bytes, st);
    case TL_DTYPE_F16: return launch_gemm<F16>(a, live, m, k, lda, workspace, workspace_bytes, st);
    default: return launch_gemm<BF16>(a, live, m, k, lda, workspace, workspace_bytes, st);
  }
}

size_t groups_workspace_bytes(int m, int k, const GemmGroups& G, int dtype) {
  if (m <= 0 || k <= 0) return 0;
  GemmGroups live{};
  for (int g = 0; g < G.count; ++g)
    if (G.n[g] > 0) live.n[live.count++] = G.n[g];
  if (live.count == 0) return 0;
  const int esize = dtype == TL_DTYPE_F32 ? 4 : 2;
  // few rows: the K-slice partials; more: the MFMA kernel's split-K partials
  // (if its plan splits; a product that falls back to the simple kernel
  // uses none of it)
  if (m <= kSkinnyMaxM) return skinny_workspace_bytes(m, live, k, esize);
  return prompt_plan(m, k, live, esize).ws_bytes;
}

}  // namespace

extern "C" {

size_t tl_gemm_workspace_bytes(int m, int n, int k, int dtype) {
  GemmGroups G{};
  G.count = 1;
  G.n[0] = n;
  return groups_workspace_bytes(m, k, G, dtype);
}

int tl_gemm(const void* a, const void* b, void* c, int m, int n, int k, int64_t lda, int64_t ldb, int64_t ldc,
            void* workspace, size_t workspace_bytes, int dtype, void* stream) {
  if (n < 0) return TL_ERR_INVALID;
  GemmGroups G{};
  const int st = make_groups(G, 1, &b, &c, &n, &ldb, &ldc);
  if (st) return st;
  return gemm_groups(a, G, m, k, lda, workspace, workspace_bytes, dtype, stream);
}

size_t tl_gemm_grouped_workspace_bytes(int m, int k, int count, const int* n, int dtype) {
  if (count < 1 || count > kMaxGroups || !n) return 0;
  GemmGroups G{};
  G.count = count;
  for (int g = 0; g < count; ++g) G.n[g] = n[g];
  return groups_workspace_bytes(m, k, G, dtype);
}

int tl_gemm_grouped(const void* a, int m, int k, int64_t lda, int count, const void* const* b, void* const* c,
                    const int* n, const int64_t* ldb, const int64_t* ldc, void* workspace, size_t workspace_bytes,
                    int dtype, void* stream) {
  GemmGroups G{};
  const int st = make_groups(G, count, b, c, n, ldb, ldc);
  if (st) return st;
  return gemm_groups(a, G, m, k, lda, workspace, workspace_bytes, dtype, stream);
}

}  // extern "C"
