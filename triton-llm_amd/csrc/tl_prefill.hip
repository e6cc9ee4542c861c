// Attention forward for prefill (any seq_q x seq_k, MHA and GQA, causal or
// not) on gfx950 matrix cores.
//
// Reference semantics (triton_llm/kernels/attention_gqa.py:21-146): query row
// i of head h attends to keys j of KV head h / group with j <= i + (Sk - Sq)
// when causal; scores are (q . k) * sm_scale; online softmax over key tiles;
// output = acc / row_sum.  The reference runs one program per (row, head)
// with vector multiply-reduce; these kernels are flash-style tiled kernels on
// MFMA: each wave owns 32 query rows of one query head and walks key tiles
// staged through LDS (16-bit kernel: 8 waves = 256 rows per workgroup in two
// ping-pong groups, 128-key tiles; fp32 kernel: 4 waves = 128 rows, 64-key
// tiles).
//
// It computes the TRANSPOSED products  S^T = K . Q^T  and  O^T = V^T . P^T
// with 32x32 MFMA tiles.  In the 32x32 accumulator layout lane l holds
// column n = l % 32 and 16 rows; with the transposed products column n is a
// query row, so every lane owns exactly one query row: the row max needs one
// exchange between lane l and l ^ 32, the row sum is kept per lane and merged
// once at the end, and the O rescale is a per-lane scalar.
//
// MFMA operand layouts used (gfx950, wave64):
//   32x32x16 (f16/bf16): A lane l = A[l%32][8*(l/32) + 0..7],
//                        B lane l = B[8*(l/32) + 0..7][l%32],
//                        C lane l, reg r = C[8*(r/4) + 4*(l/32) + r%4][l%32].
//   32x32x2  (f32):      A lane l = A[l%32][l/32], B lane l = B[l/32][l%32],
//                        same C layout.
// The reduction index of one MFMA may be any permutation as long as A and B
// agree; the P^T operand is taken straight from the S^T accumulator
// registers (lane half h holds keys 8a + 4h + b, b < 4, of each 32-key
// block) and the V^T operand is read with the matching key permutation.
//
// Kernels: vt_pack_kernel + flash_fwd_16 (f16 / bf16, d_k 64 / 128), flash_fwd_f32
// (fp32, d_k 64 / 128), attn_generic_kernel (any d_k <= 256).
#include "tl_prefill.h"

#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <stddef.h>
#include <atomic>
#include <chrono>
#include <mutex>
#include <random>
#include <type_traits>

namespace {

using namespace tlp;

constexpr int BM = 128;  // query rows per workgroup
constexpr int BN = 64;   // keys per tile
constexpr int kThreads = 256;



__device__ __forceinline__ float xor32(float x) { return __shfl_xor(x, 32); }

// Map the linear block id so that each XCD (blocks are dealt round-robin to
// the 8 XCDs) receives a contiguous range of work items, i.e. the same KV
// head, and inside it the longest causal rows first.
__device__ __forceinline__ void decode_block(const FlashParams& p, int& b, int& hq, int& qt) {
  const int L = blockIdx.x;
  const int N = gridDim.x;
  const int w = (N % 8 == 0) ? (L % 8) * (N / 8) + L / 8 : L;
  // w = ((b * n_kv + hkv) * n_qt + (n_qt - 1 - qt)) * group + g
  const int g = w % p.group;
  int rest = w / p.group;
  const int qt_rev = rest % p.n_qt;
  rest /= p.n_qt;
  const int hkv = rest % p.n_kv;
  b = rest / p.n_kv;
  qt = p.n_qt - 1 - qt_rev;
  hq = hkv * p.group + g;
}

// ---------------------------------------------------------------------------
// 16-bit (f16 / bf16) kernel, d_k 64 / 128.
//
// Workgroup = 8 waves = 2 groups of 4, one workgroup per CU; each wave owns
// 32 query rows, group g rows [128 g, 128 g + 128) of a 256-row query tile.
// Both groups walk the same 128-key K / V^T tiles.  Per key tile t a wave
// runs
//     G(t): O^T += V^T_{t-1} . P^T_{t-1} and S^T_t = K_t . Q^T   (64 MFMAs)
//     A(t): masked online softmax of S_t -> P_t                   (VALU)
// group 0 in the order G(t), A(t) and group 1 in the order A(t-1), G(t), so
// on every SIMD (one wave of each group) one wave issues MFMAs while the
// other does its softmax.  One workgroup barrier per t publishes the next K
// and V^T tiles (loaded by group 0 with LDS-DMA during G(t), waited for at
// the end of A(t)) and frees the buffers the following loads overwrite; two
// buffers each for K and V^T (128 KiB at d_k 128).
//
// S^T accumulators are seeded with -m_run (Q is pre-scaled by
// sm_scale * log2 e), so P = exp2(S) directly.  The row sum: at d_k 128
// (MFMA-bound) it is kept in fp32 per lane with VALU adds (v_dot2 would not
// co-execute with the other wave's MFMAs); at d_k 64 the softmax VALU work is
// the limit and the MFMA pipe has slack, so the row sum is one more MFMA per
// 16 keys, ones . P^T, in the G phase -- the sum of the rounded P that the
// PV product uses.  The
// running offset m_run is raised (and O rescaled) only when a tile's max
// exceeds it by more than kRescaleLog2 (log2 units), which bounds P by
// 2^kRescaleLog2.
//
// V is read from a key-major copy V^T [b][kv][d][Sk_pad] written once per
// call by vt_pack_kernel, with each 16-key group stored in the order the
// MFMA's k-index permutation wants (see vt_pack_kernel), so the 8 keys a lane
// feeds into one PV MFMA are one contiguous 16 bytes: ds_read_b128, the same
// fast LDS path as the K operand.  (A transposing LDS read of natural V,
// ds_read_b64_tr_b16, measured ~3x lower LDS throughput per byte on gfx950.)
//
// LDS rows are unpadded; the 16-byte chunk c of row r lives in slot
// c ^ lds_swz(r) (lds_swz<D> for K and Q rows, lds_swz<128> for the 256-byte
// V^T rows), which makes every operand read conflict-free.
// ---------------------------------------------------------------------------





// ---------------------------------------------------------------------------
// Persistence: one workgroup per CU walks a static list of query tiles.
//
// Tiles (b, hq, qt) form n_queues lists -- one per XCD when the query heads,
// cut into q_split parts by qt % q_split, deal evenly into 8 lists, so that
// a list covers a few consecutive heads and the K/V tiles it reads stay in
// one XCD's L2 (the dispatcher hands workgroups to XCDs round-robin, so
// workgroup L serves list L % n_queues) -- each ordered by qt descending,
// i.e. by causal cost.  Workgroup j of a list takes ranks j, then by rounds
// of q_machines in alternating direction (a round pair then sums to the same
// cost for every workgroup when costs fall linearly with rank); with an odd
// number of rounds the first three use a balanced-triple order whose rank
// sums differ by at most one.
//
// Tile switches do not wait for memory.  The last G step, G(n_kt), only
// finishes the PV of the last key tile (no S), so K_{n_kt} is never loaded:
// in G(n_kt - 1) group 0 loads its own next Q rows into that K buffer, and
// in G(n_kt) the next tile's first K tile (into the K buffer the next tile
// starts from) and group 1's next Q rows (into the V^T buffer no later step
// reads).  At the switch each wave copies its next Q from LDS, then stages
// its output in the same buffer; the output stores drain in the background.
// ---------------------------------------------------------------------------

// SCALE_S: Q is used as stored and each score is scaled in fp32 in the
// softmax (one FMA per score: s * scale_log2 - m_run) instead of Q being
// pre-scaled and rounded back to 16 bits.  Taken for fp16 when
// |sm_scale * log2 e| > 1, where the pre-scaled Q could exceed the fp16
// range (bf16 has fp32's range; the reference scales q in fp32).
template <typename T, int D, bool CAUSAL, bool SCALE_S = false>
__global__ __launch_bounds__(K16_THREADS, 2) void flash_fwd_16(FlashParams p) {
  using M = Mfma<T>;
  using frag = typename M::frag;
  using Bits = typename T::bits;
  constexpr int BN = K16_BN;
  constexpr int ROWB = D * 2;          // bytes per K / Q row in LDS
  constexpr int VROWB = BN * 2;        // bytes per V^T row in LDS (256)
  // d_k 64 reads V in its natural layout (no V^T copy): its softmax VALU
  // work, not LDS, limits a step, so the PV operand's transposing LDS reads
  // (two ds_read_b64_tr_b16 per fragment) are affordable there.
  constexpr bool VNAT = D == 64;
  constexpr int TILEB = BN * ROWB;     // bytes per K, V^T or 128-row Q tile
  constexpr int NSL = ROWB / 16;       // 16-byte slots per K row
  constexpr int RPR = 1024 / ROWB;     // K rows per 1 KiB region
  constexpr int NREG = TILEB / 1024;   // 1 KiB regions per tile
  constexpr int RPW = NREG / 4;        // regions per loading wave per tile
  constexpr int NDB = D / 32;          // 32-row blocks of O^T
  constexpr int NKS = D / 16;          // k-steps of S^T
  constexpr int NMB = BN / 32;         // 32-key blocks of S^T
  constexpr int NG = NMB * NKS;        // MFMA jobs per product
  static_assert(BN / 16 * NDB == NG, "S and PV job counts must match");
  static_assert(2 * RPW <= NG / 2, "every tile load needs an issue slot");
  static_assert(BN == 128 && K16_BM == 256, "a group's 128 Q rows fill one K-sized buffer");

  // K0 K1 V0 V1 (128 KiB at d_k 128)
  __shared__ __attribute__((aligned(1024))) char smem[4 * TILEB];

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // wave-uniform: phase branches are scalar
  const int group = wave >> 2;
  const int wq = wave & 3;
  const int off = p.seq_k - p.seq_q;  // bottom-right causal offset
  const int queue = blockIdx.x % p.n_queues;
  const int mach = blockIdx.x / p.n_queues;

  // ---- lane offsets (recomputed from fresh_lane() where used) ----------------
  // K and Q: region R holds rows R * RPR + l / NSL, slot l % NSL = chunk
  // (l % NSL) ^ swz(row).  V^T: region R holds rows 4 R + l / 16 (256-byte
  // rows), slot l % 16 = chunk (l % 16) ^ swz128(row).  Wave wq of the loading
  // group fills regions wq + 4 i; the swizzle term does not depend on i, so
  // one lane offset per tensor serves every region (region steps are added).
  // 32-bit products: the shape check bounds 128 rows of K / Q and a head's
  // V^T copy below 2^32 bytes.
  auto kq_off = [&](int ln, int64_t ss) __attribute__((always_inline)) {
    const int row = wq * RPR + ln / NSL;
    return ((uint32_t)row * (uint32_t)ss + (uint32_t)(((ln % NSL) ^ lds_swz<D>(row)) * 8)) * 2u;
  };
  auto v_off = [&](int ln) __attribute__((always_inline)) {
    const int row = 4 * wq + ln / 16;
    return ((uint32_t)row * (uint32_t)p.sk_pad + (uint32_t)(((ln % 16) ^ lds_swz<128>(row)) * 8)) * 2u;
  };
  // Natural V rows (VNAT): like K rows, chunk c of key row r at slot
  // c ^ vnat_swz(r), vnat_swz(r) = 2 ((r >> 1) & 1).  A transposing read
  // covers 4 consecutive rows of a 16-lane group (4 lanes per row, 8 bytes
  // each); rows 2 apart share banks, and the XOR moves one of them by 32
  // bytes, so the group's 16 reads hit 32 distinct banks.
  auto vnat_swz = [](int r) __attribute__((always_inline)) { return 2 * ((r >> 1) & 1); };
  auto vnat_off = [&](int ln) __attribute__((always_inline)) {
    const int row = wq * RPR + ln / NSL;
    return ((uint32_t)row * (uint32_t)p.v_ss + (uint32_t)(((ln % NSL) ^ vnat_swz(row)) * 8)) * 2u;
  };
  // Operand reads: lane (lq, h) reads row lq, chunk (2 ks + h) ^ swz(lq).
  auto k_lane_of = [&](int ln) __attribute__((always_inline)) {
    const int lq = ln & 31, h = ln >> 5;
    return lq * ROWB + ((h ^ lds_swz<D>(lq)) << 4);
  };
  auto v_lane_of = [&](int ln) __attribute__((always_inline)) {
    const int lq = ln & 31, h = ln >> 5;
    return lq * VROWB + ((h ^ lds_swz<128>(lq)) << 4);
  };
  const uint32_t wave_lds = __builtin_amdgcn_readfirstlane((uint32_t)wq * 1024u);
  const uint32_t lds_k0 = (uint32_t)(size_t)(__attribute__((address_space(3))) char*)smem;
  const uint32_t lds_v0 = lds_k0 + 2 * TILEB;
  const uint32_t k_ss2 = (uint32_t)p.k_ss * 2u;
  const uint32_t q_ss2 = (uint32_t)p.q_ss * 2u;
  const uint32_t k_step = 4u * RPR * k_ss2;                // bytes of 4 regions of K rows
  const uint32_t q_step = 4u * RPR * q_ss2;                // bytes of 4 regions of Q rows
  const uint32_t v_step = VNAT ? 4u * RPR * (uint32_t)p.v_ss * 2u    // bytes of 4 regions of V rows
                                : 16u * (uint32_t)p.sk_pad * 2u;     // bytes of 16 V^T rows

  // ---- tile state --------------------------------------------------------------
  // Code of list entry e, read from the kernel-argument segment (p is the
  // kernel's only argument, at offset 0) with a scalar load.
  auto entry_code = [&](int e) __attribute__((always_inline)) {
    typedef const __attribute__((address_space(4))) uint32_t kword;
    kword* tab = (kword*)((const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr() +
                          offsetof(FlashParams, e_code));
    return (int)((tab[e >> 2] >> (8 * (e & 3))) & 0xffu);
  };
  // Key-split parts exist only for causal calls (the host plans no split
  // otherwise); non-causal instances carry none of their code.
  constexpr bool kSplit = CAUSAL;
  // A key-split part covers K tiles [kt0, kt0 + n_kt) of its tile: the
  // lower part [0, h), the upper [h, n_kt of the whole tile), h = min(half
  // the tile's K tiles, (first query row + off) / BN), so every query row of
  // the tile (first row >= BM, off >= 0: the host splits no other tile) has
  // keys in both parts.
  struct Tile {
    int b, hq, qt, n_kt, k_rows, kt0, kpart, sidx;
    const char* kg;  // K rows from key kt0 * BN on
    const char* vg;  // natural V rows from key kt0 * BN on (VNAT)
  };
  auto make_tile = [&](int rank) __attribute__((always_inline)) {
    Tile tl;
    tl.kpart = 0;
    tl.sidx = 0;
    if (kSplit && p.n_entries)
      decode_item(p, queue, rank, entry_code(rank / p.q_parts), tl.b, tl.hq, tl.qt, tl.kpart, tl.sidx);
    else
      decode_tile(p, queue, rank, tl.b, tl.hq, tl.qt);
    const int q_last = min(p.seq_q, tl.qt * K16_BM + K16_BM) - 1;
    int k_end = p.seq_k;
    if (CAUSAL) k_end = max(0, min(p.seq_k, q_last + off + 1));
    tl.n_kt = (k_end + BN - 1) / BN;  // K tiles the workgroup loads
    tl.kt0 = 0;
    if (kSplit && tl.kpart) {
      const int h = min(tl.n_kt / 2, (tl.qt * K16_BM + off) / BN);
      tl.kt0 = tl.kpart == 1 ? 0 : h;
      tl.n_kt = tl.kpart == 1 ? h : tl.n_kt - h;
    }
    tl.k_rows = min(p.seq_k - tl.kt0 * BN, tl.n_kt * BN);  // keys the workgroup reads
    tl.kg = (const char*)((const Bits*)p.k + tl.b * p.k_sb + (tl.hq / p.group) * p.k_sh + (int64_t)tl.kt0 * BN * p.k_ss);
    tl.vg = (const char*)((const Bits*)p.v + tl.b * p.v_sb + (tl.hq / p.group) * p.v_sh + (int64_t)tl.kt0 * BN * p.v_ss);
    return tl;
  };

  using rsrc_t = i32x4;
  auto dma = [&](const rsrc_t& rsrc, uint32_t voff, uint32_t la) __attribute__((always_inline)) {
    lds_dma16(rsrc, voff, la);
  };
  auto rsrc_of = [&](const char* base, uint32_t bytes) __attribute__((always_inline)) {
    return uniform_rsrc(base, bytes);
  };
  // K tile tk of a tile: rows past its k_rows read as zeros, no traffic.
  auto k_rsrc = [&](const Tile& tl, int tk) __attribute__((always_inline)) {
    const int rows = min(max(tl.k_rows - tk * BN, 0), BN);
    return rsrc_of(tl.kg + (int64_t)tk * BN * k_ss2, (uint32_t)rows * k_ss2);
  };
  // V^T tile tv of a tile (nothing past its last K tile); with VNAT the
  // tile's natural V rows, bounded like K's.
  auto v_rsrc = [&](const Tile& tl, int tv) __attribute__((always_inline)) {
    if constexpr (VNAT) {
      const uint32_t v_ss2 = (uint32_t)p.v_ss * 2u;
      const int rows = min(max(tl.k_rows - tv * BN, 0), BN);
      return rsrc_of(tl.vg + (int64_t)tv * BN * v_ss2, (uint32_t)rows * v_ss2);
    } else {
      const char* vg = (const char*)((const Bits*)p.vt + ((int64_t)tl.b * p.n_kv + tl.hq / p.group) * D * p.sk_pad);
      return rsrc_of(vg + (int64_t)(tl.kt0 + tv) * BN * 2, tv < tl.n_kt ? (uint32_t)D * (uint32_t)p.sk_pad * 2u : 0u);
    }
  };
  // Q rows [128 g, 128 g + 128) of a tile (rows past seq_q read as zeros).
  auto q_rsrc = [&](const Tile& tl, int g) __attribute__((always_inline)) {
    const int r0 = tl.qt * K16_BM + 128 * g;
    const int rows = min(max(p.seq_q - r0, 0), 128);
    const char* qg = (const char*)((const Bits*)p.q + tl.b * p.q_sb + tl.hq * p.q_sh + (int64_t)r0 * p.q_ss);
    return rsrc_of(qg, (uint32_t)rows * q_ss2);
  };

  // ---- registers -------------------------------------------------------------------
  frag qf[NKS];  // Q pre-scaled by sm_scale * log2 e
  f32x16 o_acc[NDB];
  float m_run, l4[4];
  constexpr bool kMfmaRowSum = D == 64;  // row sums on the matrix cores
  f32x16 l_acc;                           // every register: the lane's row sum
  const frag ones = __builtin_bit_cast(
      frag, u32x4{T::one_pair, T::one_pair, T::one_pair, T::one_pair});
  bool fresh;
  f32x16 s_init;
  f32x16 s[NMB];      // S_t (relative scores)
  u32x4 pw[BN / 16];  // P_t packed 16-bit

  auto scale_q = [&]() __attribute__((always_inline)) {
    if constexpr (SCALE_S) return;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const u32x4 raw = __builtin_bit_cast(u32x4, qf[ks]);
      uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo, hi;
        unpack2<T>(w[i], lo, hi);
        const float x[2] = {lo * p.scale_log2, hi * p.scale_log2};
        w[i] = pack2<T>(x);  // hardware convert, round to nearest even
      }
      qf[ks] = __builtin_bit_cast(frag, u32x4{w[0], w[1], w[2], w[3]});
    }
  };
  // Cold tile start: K_0 into K buffer kb by all eight waves and this wave's
  // Q rows from global memory; waits for both.
  auto cold_start = [&](const Tile& tl, int kb) __attribute__((always_inline)) {
    const int ln = fresh_lane();
    const int h = ln >> 5;
    const rsrc_t rk = k_rsrc(tl, 0);
    const uint32_t kvo = kq_off(ln, p.k_ss);
#pragma unroll
    for (int i = group; i < RPW; i += 2) dma(rk, kvo + (uint32_t)i * k_step, lds_k0 + kb * TILEB + i * 4096 + wave_lds);
    const int qi = tl.qt * K16_BM + 128 * group + 32 * wq + (ln & 31);
    const Bits* qrow = (const Bits*)p.q + tl.b * p.q_sb + tl.hq * p.q_sh + (int64_t)min(qi, p.seq_q - 1) * p.q_ss;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      u32x4 raw = *(const u32x4*)(qrow + 16 * ks + 8 * h);
      if (qi >= p.seq_q) raw = u32x4{0u, 0u, 0u, 0u};
      qf[ks] = __builtin_bit_cast(frag, raw);
    }
    wait_vmcnt<0>();
    scale_q();
  };

  constexpr int kPrefetch = 2;
  static_assert(NMB == 4, "S jobs are ordered for four key blocks");
  constexpr auto s_mb = [](int g) { return 2 * (g / (2 * NKS)) + (g & 1); };
  constexpr auto s_ks = [](int g) { return (g % (2 * NKS)) >> 1; };

  int r = 0;
  int rank = sched_rank(p, mach, 0);
  if (rank >= p.q_tiles) return;
  Tile cur = make_tile(rank);
  int tb = 0;  // K / V^T buffer parity of the tile's K_0
  cold_start(cur, tb);
  lds_barrier();

  for (;;) {
    const int nrank = sched_rank(p, mach, r + 1);
    const bool has_next = nrank < p.q_tiles;
    const Tile nxt = make_tile(has_next ? nrank : rank);  // wave-uniform (SGPRs)
    const int n_kt = cur.n_kt;
    const int q0 = cur.qt * K16_BM + 128 * group + 32 * wq;  // first row of this wave
    int wave_k_end = p.seq_k;
    if (CAUSAL) wave_k_end = max(0, min(p.seq_k, min(q0 + 31, p.seq_q - 1) + off + 1));
    if (q0 >= p.seq_q) wave_k_end = 0;  // no rows: no compute
    // Key positions relative to the part's first key (a key-split part
    // starts at K tile kt0): the softmax compares t * BN with these.
    const int kshift = kSplit ? cur.kt0 * BN : 0;
    const int seq_k_rel = p.seq_k - kshift;
    const int off_rel = off - kshift;
    const int wave_k_end_rel = wave_k_end - kshift;

#pragma unroll
    for (int i = 0; i < NDB; ++i)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o_acc[i][rr] = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) s_init[rr] = 0.f;
    m_run = 0.f;
    fresh = true;
#pragma unroll
    for (int k = 0; k < 4; ++k) l4[k] = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) l_acc[rr] = 0.f;

    // G(t): job g = PV job g of tile t-1 (keys 16 (g / NDB).., d-block
    // g % NDB; none for t = 0) and S job g of tile t.  S jobs fill key blocks
    // in pairs (0 1, then 2 3), alternating the pair, so only half of S is
    // live while the first half of P is consumed.  Every G phase runs both
    // products: the P of a tile a wave does not use is zero (its PV adds
    // nothing) and the S of such a tile is never read, which keeps one
    // straight-line MFMA stream per group.  Group 0 loads, one every other
    // job, K_{t+1} then V^T_t -- for t = n_kt the next tile's K_0 and group
    // 1's next Q rows instead.
    auto g_phase = [&](int t, auto dma_tag, auto pv_tag, auto s_tag) __attribute__((always_inline)) {
      constexpr bool DO_DMA = decltype(dma_tag)::value;
      constexpr bool DO_PV = decltype(pv_tag)::value;
      constexpr bool DO_S = decltype(s_tag)::value;
      const int ln = fresh_lane();
      rsrc_t rk = {0, 0, 0, 0}, rv = {0, 0, 0, 0};
      uint32_t kvo = 0, vvo = 0, kstep = k_step, vstep = v_step;
      if constexpr (DO_DMA) {
        // K slot: K_{t+1}; at t = n_kt - 1 group 0's next Q rows (K_{n_kt}
        // is never used: G(n_kt) computes no S); at t = n_kt the next K_0.
        // V slot: V^T_t; at t = n_kt group 1's next Q rows.
        const rsrc_t none = rsrc_of(cur.kg, 0u);
        if (t < n_kt - 1) {
          rk = k_rsrc(cur, t + 1);
          kvo = kq_off(ln, p.k_ss);
        } else if (t == n_kt - 1) {
          rk = has_next ? q_rsrc(nxt, 0) : none;
          kvo = kq_off(ln, p.q_ss);
          kstep = q_step;
        } else {
          rk = has_next ? k_rsrc(nxt, 0) : none;
          kvo = kq_off(ln, p.k_ss);
        }
        if (t < n_kt) {
          rv = v_rsrc(cur, t);
          vvo = VNAT ? vnat_off(ln) : v_off(ln);
        } else {
          rv = has_next ? q_rsrc(nxt, 1) : none;
          vvo = kq_off(ln, p.q_ss);
          vstep = q_step;
        }
      }
      const int kbuf = (tb + t + 1) & 1;  // K_{t+1} (or a next Q / K_0)
      const int vbuf = (tb + t) & 1;      // V^T_t (or group 1's next Q)
      int kb_lane = k_lane_of(ln) + ((tb + t) & 1) * TILEB;              // K_t
      int vb_lane = v_lane_of(ln) + (2 + ((tb + t + 1) & 1)) * TILEB;   // V^T_{t-1}
      // VNAT: lane 16 g + 4 e + q reads 8 bytes of key row 16 tt + 4 h + e
      // (and + 8), columns 32 db + 16 (g % 2) + 4 q .. + 3 (h = g / 2); the
      // transposing read hands lane l column 32 db + l % 32, keys 16 tt +
      // 4 h + 0..3 (and + 8 ..): the PV operand's key order.
      int vn_lane = 0;
      if constexpr (VNAT) {
        const int g16 = ln >> 4, e = (ln >> 2) & 3, q = ln & 3;
        const int c0 = 2 * (g16 & 1) + (q >> 1);
        vn_lane = (2 + ((tb + t + 1) & 1)) * TILEB + (4 * (g16 >> 1) + e) * ROWB +
                  ((c0 ^ vnat_swz(e)) << 4) + 8 * (q & 1);
      }
      u32x4 kfr[NG], vfr[NG];
      auto fetch = [&](int g) __attribute__((always_inline)) {
        if constexpr (DO_PV) {
          const int tt = g / NDB, db = g % NDB;
          if constexpr (VNAT) {
            typedef short v4s __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4s lds_v4s;
            __attribute__((address_space(3))) char* lds = (__attribute__((address_space(3))) char*)smem;
            const int off = vn_lane + tt * 16 * ROWB + db * 64;
            const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds + off));
            const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(lds + off + 8 * ROWB));
            vfr[g] = u32x4{__builtin_bit_cast(u32x2, lo).x, __builtin_bit_cast(u32x2, lo).y,
                           __builtin_bit_cast(u32x2, hi).x, __builtin_bit_cast(u32x2, hi).y};
          } else {
            vfr[g] = *(const u32x4*)(smem + (vb_lane ^ (tt << 5)) + 32 * db * VROWB);
          }
        }
        if constexpr (DO_S) {
          const int ks = s_ks(g), mb = s_mb(g);
          kfr[g] = *(const u32x4*)(smem + (kb_lane ^ (ks << 5)) + 32 * mb * ROWB);
        }
      };
      // G phases issue at raised priority, so a G phase's MFMAs win over the
      // other group's softmax -- except group 1's G(0), which runs beside
      // group 0's G(0): it yields, so group 0 finishes its first S sooner and
      // its first softmax overlaps group 1's MFMAs.
      if (group == 1 && t == 0)
        __builtin_amdgcn_s_setprio(0);
      else
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int g = 0; g < kPrefetch; ++g) fetch(g);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if (g + kPrefetch < NG) fetch(g + kPrefetch);
        if constexpr (DO_PV) {
          const int tt = g / NDB, db = g % NDB;
          o_acc[db] = M::mma(__builtin_bit_cast(frag, vfr[g]), __builtin_bit_cast(frag, pw[tt]), o_acc[db]);
          if constexpr (kMfmaRowSum) {
            if (db == 0) l_acc = M::mma(ones, __builtin_bit_cast(frag, pw[tt]), l_acc);
          }
        }
        if constexpr (DO_S) {
          const int ks = s_ks(g), mb = s_mb(g);
          s[mb] = M::mma(__builtin_bit_cast(frag, kfr[g]), qf[ks], ks == 0 ? s_init : s[mb]);
        }
        if constexpr (DO_DMA) {
          if (g % 2 == 1 && g / 2 < RPW) {
            const int i = g / 2;
            dma(rk, kvo + (uint32_t)i * kstep, lds_k0 + kbuf * TILEB + i * 4096 + wave_lds);
          }
          if (g % 2 == 1 && g / 2 >= RPW && g / 2 < 2 * RPW) {
            const int i = g / 2 - RPW;
            dma(rv, vvo + (uint32_t)i * vstep, lds_v0 + vbuf * TILEB + i * 4096 + wave_lds);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
    };

    // A(t): masked softmax of S_t -> P_t.  key = kb + 32 mb + 8 (r/4) + 4 h + r % 4;
    // a tile the wave does not use yields P = 0.
    auto a_phase = [&](int t) __attribute__((always_inline)) {
      const int kb = t * BN;  // first key of the tile, relative to the part's first key
      if (t >= n_kt || kb >= wave_k_end_rel) {
#pragma unroll
        for (int tt = 0; tt < BN / 16; ++tt) pw[tt] = u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        return;
      }
      if constexpr (SCALE_S) {
        // raw scores -> log2 domain relative to m_run (s_init stays 0)
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) s[mb][rr] = fmaf(s[mb][rr], p.scale_log2, -m_run);
      }
      const bool need_mask = (kb + BN > seq_k_rel) || (CAUSAL && kb + BN - 1 > q0 + off_rel);
      if (need_mask) {
        const int ln = fresh_lane();
        const int h = ln >> 5;
        int lim = seq_k_rel - 1 - kb - 4 * h;
        if (CAUSAL) lim = min(lim, q0 + (ln & 31) + off_rel - kb - 4 * h);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int kl = 32 * mb + 8 * (rr >> 2) + (rr & 3);
            s[mb][rr] = kl <= lim ? s[mb][rr] : -INFINITY;
          }
      }
      // Row max over the tile: IEEE maximum (NaN-propagating) maps to
      // v_maximum3_f32 with no input canonicalisation, unlike fmaxf.
      auto mx3 = [](float x, float y, float z) { return __builtin_elementwise_maximum(__builtin_elementwise_maximum(x, y), z); };
      float mq[NMB];
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const f32x16& v = s[mb];
        const float a0 = mx3(v[0], v[1], v[2]), a1 = mx3(v[3], v[4], v[5]), a2 = mx3(v[6], v[7], v[8]);
        const float a3 = mx3(v[9], v[10], v[11]), a4 = mx3(v[12], v[13], v[14]);
        mq[mb] = __builtin_elementwise_maximum(mx3(a0, a1, a2), mx3(a3, a4, v[15]));
      }
      const float mxl = __builtin_elementwise_maximum(mx3(mq[0], mq[1], mq[2]), mq[3]);
      const float mx = max_xor32(mxl);
      const bool grow = fresh ? (mx != -INFINITY) : (mx > kRescaleLog2);
      if (__any(grow)) {
        const float delta = fresh ? (mx == -INFINITY ? 0.f : mx) : fmaxf(mx, 0.f);
        const float alpha = fresh ? 1.f : fast_exp2(-delta);  // fresh: nothing to scale, 2^-mx may overflow
        m_run += delta;
        fresh = fresh && (mx == -INFINITY);
#pragma unroll
        for (int k = 0; k < 4; ++k) l4[k] *= alpha;
        if constexpr (kMfmaRowSum) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) l_acc[rr] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) o_acc[i][rr] *= alpha;
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) s[mb][rr] -= delta;
        if constexpr (!SCALE_S) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) s_init[rr] = -m_run;
        }
      }
      // P chunk tt (keys 16 tt..) = s[tt / 2][8 (tt % 2) + 0..7]; fp32 row sums
      // (v_dot2 does not co-execute with the partner's MFMAs).
#pragma unroll
      for (int tt = 0; tt < BN / 16; ++tt)
#pragma unroll
        for (int j2 = 0; j2 < 4; ++j2) {
          float pr2[2] = {fast_exp2(s[tt >> 1][8 * (tt & 1) + 2 * j2]),
                          fast_exp2(s[tt >> 1][8 * (tt & 1) + 2 * j2 + 1])};
          pw[tt][j2] = pack2<T>(pr2);
          if constexpr (!kMfmaRowSum) l4[j2] += pr2[0] + pr2[1];
        }
      __builtin_amdgcn_sched_barrier(0);
    };

    // This wave's next Q rows out of LDS: group 0's in K buffer
    // (tb + n_kt) & 1, group 1's in V^T buffer (tb + n_kt) & 1 (each group
    // stages its output there too).
    const int qbuf = (group == 0 ? 0 : 2 * TILEB) + ((tb + n_kt) & 1) * TILEB;
    auto read_next_q = [&]() __attribute__((always_inline)) {
      const int ql = qbuf + 32 * wq * ROWB + k_lane_of(fresh_lane());
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) qf[ks] = __builtin_bit_cast(frag, *(const u32x4*)(smem + (ql ^ (ks << 5))));
      scale_q();
    };

    // ---- group 0 runs G(t), A(t); group 1 runs A(t-1), G(t), for t = 0 .. n_kt.
    // One barrier per t, after group 0's A(t) (which waits for the loads it
    // issued in G(t)) and group 1's G(t): G(t+1) then finds K_{t+1} and
    // V^T_t in LDS, and the buffers G(t+1)'s loads overwrite (K_{t-1}'s,
    // V^T_{t-1}'s) were last read in G(t).  Between barriers the groups are
    // not forced to alternate; G phases run at raised priority, so the MFMA
    // work of one group overlaps the other's softmax. -------------------------------
    if (n_kt > 0) {
      using Y = std::true_type;
      using N = std::false_type;
      if (group == 0) {
        g_phase(0, Y{}, N{}, Y{});
        a_phase(0);
        wait_vmcnt<0>();
        lds_barrier();
        for (int t = 1; t < n_kt; ++t) {
          g_phase(t, Y{}, Y{}, Y{});
          a_phase(t);
          wait_vmcnt<0>();
          lds_barrier();
        }
        g_phase(n_kt, Y{}, Y{}, N{});  // PV of the last tile; no S
        // Its next Q rows (loaded in G(n_kt - 1), published by the last
        // barrier) while group 1 still runs its last softmax and G phase.
        if (has_next) read_next_q();
        wait_vmcnt<0>();
        lds_barrier();
      } else {
        g_phase(0, N{}, N{}, Y{});
        lds_barrier();
        for (int t = 1; t < n_kt; ++t) {
          a_phase(t - 1);
          g_phase(t, N{}, Y{}, Y{});
          lds_barrier();
        }
        a_phase(n_kt - 1);
        g_phase(n_kt, N{}, Y{}, N{});
        lds_barrier();
      }
    }

    // ---- tile switch ---------------------------------------------------------------
    // 1. Every wave of group 1 copies its next Q rows out of LDS (group 0 did
    //    in its last step; after a tile that ran no phase, every wave loads
    //    them cold).  2. Each wave stages its output rows, normalised and
    //    rounded, in the rows of its group's Q buffer it just read its Q from
    //    (so no barrier is needed between the two) and stores them
    //    row-contiguously (16 lanes per 256-byte row), so each store
    //    instruction writes whole cache lines.  The stores are not waited
    //    for here.
    float l_row = kMfmaRowSum ? l_acc[0] : sum_xor32((l4[0] + l4[1]) + (l4[2] + l4[3]));
    const int ntb = (tb + n_kt + 1) & 1;  // where the next K_0 went
    if (has_next) {
      if (n_kt == 0)
        cold_start(nxt, ntb);  // no phase ran to prefetch it
      else if (group == 1)
        read_next_q();
    }
    // 3. A key-split part: each wave merges with the same wave of the tile's
    //    other part, which holds the same 32 query rows.  The wave stores its
    //    partial (O^T unnormalised, and per row m, l) in its part's slot,
    //    waits until the stores have completed, then one lane swaps the
    //    call's tag into the wave's arrival word.  The wave that finds the tag
    //    already there arrived second: it loads the other partial, merges the
    //    two in part order (so the result does not depend on which arrived
    //    first), clears the word for the next call and writes the output;
    //    the first wave writes nothing.  Nothing waits on another workgroup.
    //    Stores and loads of partials and the word are device-coherent (sc1
    //    stores and loads, a device-scope swap), which orders them across
    //    XCDs without a cache write-back or invalidate.
    bool write_out = true;
    if constexpr (kSplit) {
      if (cur.kpart) {
        constexpr uint32_t kWaveBytes = NDB * 4 * 1024 + 512;  // O^T (NDB x 4 float4 per lane), then (m, l)
        constexpr uint32_t kSlotBytes = 8 * kWaveBytes;
        constexpr int kSc1 = 16;                               // cache-policy bit sc1
        const int ln = fresh_lane();
        char* ws = (char*)p.split_ws;
        const uint32_t words = ((uint32_t)p.n_split_tiles * 64u + 255u) & ~255u;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(ws + words, (short)0, (int)p.split_part_bytes, kBufRsrcWord3);
        const uint32_t mine = ((uint32_t)cur.sidx * 2u + (uint32_t)(cur.kpart - 1)) * kSlotBytes + (uint32_t)wave * kWaveBytes;
        const uint32_t theirs = ((uint32_t)cur.sidx * 2u + (uint32_t)(2 - cur.kpart)) * kSlotBytes + (uint32_t)wave * kWaveBytes;
        const float m_row = fresh ? -INFINITY : m_run;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const f32x4 v = {o_acc[db][4 * rq], o_acc[db][4 * rq + 1], o_acc[db][4 * rq + 2], o_acc[db][4 * rq + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs,
                                                   (int)(mine + (uint32_t)(((db * 4 + rq) * 64 + ln) * 16)), 0, kSc1);
          }
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(m_row), __float_as_uint(l_row)}, rs,
                                              (int)(mine + NDB * 4 * 1024u + (uint32_t)ln * 8u), 0, kSc1);
        wait_vmcnt<0>();
        unsigned long long* word = (unsigned long long*)ws + (int64_t)cur.sidx * 8 + wave;
        unsigned long long old = 0;
        if (ln == 0) old = __hip_atomic_exchange(word, (unsigned long long)p.split_token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = ((unsigned long long)(uint32_t)__builtin_amdgcn_readfirstlane((int)(old >> 32)) << 32) |
              (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)old);
        write_out = old == p.split_token;
        if (write_out) {
          const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(theirs + NDB * 4 * 1024u + (uint32_t)ln * 8u), 0, kSc1);
          const float m_o = __uint_as_float(ml.x), l_o = __uint_as_float(ml.y);
          const bool lower = cur.kpart == 1;
          const float m_a = lower ? m_row : m_o, m_b = lower ? m_o : m_row;
          const float m = fmaxf(m_a, m_b);
          const float w_a = fast_exp2(m_a - m), w_b = fast_exp2(m_b - m);
          // O = O_a w_a + O_b w_b, l likewise (a: the lower part), the same
          // operations whichever part merges
          const float l_a = lower ? l_row : l_o, l_b = lower ? l_o : l_row;
          l_row = fmaf(l_a, w_a, l_b * w_b);
          constexpr int kChunk = NDB < 2 ? NDB : 2;  // d-blocks of the other partial in registers at once
#pragma unroll
          for (int d0 = 0; d0 < NDB; d0 += kChunk) {
            u32x4 t[kChunk][4];
#pragma unroll
            for (int db = 0; db < kChunk; ++db)
#pragma unroll
              for (int rq = 0; rq < 4; ++rq)
                t[db][rq] = __builtin_amdgcn_raw_buffer_load_b128(
                    rs, (int)(theirs + (uint32_t)((((d0 + db) * 4 + rq) * 64 + ln) * 16)), 0, kSc1);
#pragma unroll
            for (int db = 0; db < kChunk; ++db)
#pragma unroll
              for (int rq = 0; rq < 4; ++rq)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const float x_m = o_acc[d0 + db][4 * rq + e], x_t = __uint_as_float(t[db][rq][e]);
                  const float x_a = lower ? x_m : x_t, x_b = lower ? x_t : x_m;
                  o_acc[d0 + db][4 * rq + e] = fmaf(x_a, w_a, x_b * w_b);
                }
          }
          if (ln == 0) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    const float inv = 1.f / l_row;
    if (write_out) {
      const int ln = fresh_lane();
      const int lq = ln & 31, h = ln >> 5;
      const int wbase = qbuf + 32 * wq * ROWB;  // this wave's 32 rows
      // O^T lane (lq, h) holds row lq, d = 32 db + 8 rq + 4 h + 0..3: 16-byte
      // chunk 4 db + rq, half h.
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const float x0[2] = {o_acc[db][4 * rq + 0] * inv, o_acc[db][4 * rq + 1] * inv};
          const float x1[2] = {o_acc[db][4 * rq + 2] * inv, o_acc[db][4 * rq + 3] * inv};
          const int c = 4 * db + rq;
          *(u32x2*)(smem + wbase + lq * ROWB + ((c ^ lds_swz<D>(lq)) << 4) + 8 * h) = u32x2{pack2<T>(x0), pack2<T>(x1)};
        }
      // This wave's 32 output rows through one buffer resource that ends at
      // row seq_q (stores past it are dropped: no per-row branch), 32-bit
      // offsets (the shape check bounds 32 rows of o), all LDS reads first.
      const uint64_t oa = (uint64_t)(uintptr_t)((Bits*)p.o + cur.b * p.o_sb + cur.hq * p.o_sh + (int64_t)q0 * p.o_ss);
      const uint32_t o_ss2 = (uint32_t)p.o_ss * 2u;
      // every field wave-uniform (read from the first lane), so the resource
      // lives in SGPRs and the store needs no per-lane loop
      char* obase = (char*)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(oa >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)oa));
      const int o_bytes = __builtin_amdgcn_readfirstlane((int)((uint32_t)min(max(p.seq_q - q0, 0), 32) * o_ss2));
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(obase, (short)0, o_bytes, kBufRsrcWord3);
      u32x4 val[32 / RPR];
#pragma unroll
      for (int i = 0; i < 32 / RPR; ++i) {
        const int rr = i * RPR + ln / NSL, cc = ln % NSL;
        val[i] = *(const u32x4*)(smem + wbase + rr * ROWB + ((cc ^ lds_swz<D>(rr)) << 4));
      }
#pragma unroll
      for (int i = 0; i < 32 / RPR; ++i) {
        const int rr = i * RPR + ln / NSL, cc = ln % NSL;
        const uint32_t voff = (uint32_t)rr * o_ss2 + (uint32_t)cc * 16u;
        __builtin_amdgcn_raw_buffer_store_b128(val[i], ro, (int)voff, 0, 0);
      }
    }
    lds_barrier();  // the staging buffers are reused by the next tile's first loads
    if (!has_next) break;
    cur = nxt;
    rank = nrank;
    tb = ntb;
    ++r;
  }
  wait_vmcnt<0>();  // no LDS-DMA may land after the workgroup has left its LDS
}

// ---------------------------------------------------------------------------
// fp32 kernel (v_mfma_f32_32x32x2_f32).  K-step mapping for S^T: lane half h
// covers d = h*D/2 + 4c + i for step (c, i), so both K (LDS) and Q (global)
// are read as 16-byte chunks.
// ---------------------------------------------------------------------------
// d_k = 128 keeps 64 fp32 Q values per lane, so it runs at one wave per SIMD.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, D == 128 ? 1 : 2) void flash_fwd_f32(FlashParams p) {
  constexpr int KROW = D * 4 + 16;
  constexpr int VROW = D * 4 + 32;
  constexpr int CPR = D * 4 / 16;
  constexpr int CHUNKS = BN * CPR / kThreads;
  constexpr int NDB = D / 32;
  constexpr int NC = D / 8;  // 16-byte chunks per lane half
  static_assert(CHUNKS * kThreads == BN * CPR, "tile split");

  __shared__ __attribute__((aligned(16))) char smem[BN * KROW + BN * VROW];
  char* Ks = smem;
  char* Vs = smem + BN * KROW;

  int b, hq, qt;
  decode_block(p, b, hq, qt);
  const int hkv = hq / p.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lq = lane & 31;
  const int h = lane >> 5;
  const int off = p.seq_k - p.seq_q;

  const int q_first = qt * BM;
  const int q_last = min(p.seq_q, q_first + BM) - 1;
  int k_end = p.seq_k;
  if (CAUSAL) k_end = max(0, min(p.seq_k, q_last + off + 1));
  const int n_kt = (k_end + BN - 1) / BN;
  const int q0 = q_first + wave * 32;
  const int qi = q0 + lq;
  int wave_k_end = p.seq_k;
  if (CAUSAL) wave_k_end = max(0, min(p.seq_k, min(q0 + 31, p.seq_q - 1) + off + 1));

  f32x4 qf[NC];
  {
    const float* qrow = (const float*)p.q + b * p.q_sb + hq * p.q_sh + (int64_t)qi * p.q_ss;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
      qf[cc] = qi < p.seq_q ? *(const f32x4*)(qrow + h * (D / 2) + 4 * cc) : z;
    }
  }

  f32x16 o_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.f;
  float m_run = -INFINITY;
  float l_run = 0.f;

  const float* kbase = (const float*)p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = (const float*)p.v + b * p.v_sb + hkv * p.v_sh;
  f32x4 kreg[CHUNKS], vreg[CHUNKS];

  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int cidx = tid + kThreads * i;
      const int row = cidx / CPR;
      const int col = cidx % CPR;
      const int key = kt * BN + row;
      f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const bool ok = key < p.seq_k;
      kreg[i] = ok ? *(const f32x4*)(kbase + (int64_t)key * p.k_ss + col * 4) : z;
      vreg[i] = ok ? *(const f32x4*)(vbase + (int64_t)key * p.v_ss + col * 4) : z;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int cidx = tid + kThreads * i;
      const int row = cidx / CPR;
      const int col = cidx % CPR;
      *(f32x4*)(Ks + row * KROW + col * 16) = kreg[i];
      *(f32x4*)(Vs + row * VROW + col * 16) = vreg[i];
    }
  };

  const float c = p.scale_log2;
  if (n_kt > 0) load_tile(0);
  for (int kt = 0; kt < n_kt; ++kt) {
    if (kt > 0) __syncthreads();
    store_tile();
    __syncthreads();
    if (kt + 1 < n_kt) load_tile(kt + 1);

    const int kb = kt * BN;
    if (kb >= wave_k_end) continue;

    f32x16 s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[mb][r] = 0.f;
      const char* krow = Ks + (32 * mb + lq) * KROW + h * (D / 2) * 4;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const f32x4 a = *(const f32x4*)(krow + 16 * cc);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          s[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], qf[cc][i], s[mb], 0, 0, 0);
      }
    }

    const bool need_mask = (kb + BN > p.seq_k) || (CAUSAL && kb + BN - 1 > q0 + off);
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[mb][r] * c;
        if (need_mask) {
          const int key = kb + 32 * mb + 8 * (r >> 2) + 4 * h + (r & 3);
          const bool ok = key < p.seq_k && (!CAUSAL || key <= qi + off);
          x = ok ? x : -INFINITY;
        }
        s[mb][r] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx);
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - base);
    m_run = m_new;
    if (__any(alpha != 1.f)) {
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;
    }
    float psum = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(s[mb][r] - base);
        s[mb][r] = e;
        psum += e;
      }
    l_run += psum;

    // O^T += V^T . P^T: step (mb, r) uses key 32mb + 8(r/4) + 4h + r%4 in
    // lane half h, i.e. MFMA k = h.
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 32 * mb + 8 * (r >> 2) + 4 * h + (r & 3);
        const char* vrow = Vs + key * VROW + lq * 4;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const float a = *(const float*)(vrow + 128 * db);
          o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, s[mb][r], o_acc[db], 0, 0, 0);
        }
      }
  }

  const float l_tot = l_run + xor32(l_run);
  const float inv = 1.f / l_tot;
  if (qi < p.seq_q) {
    float* orow = (float*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)qi * p.o_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = 32 * db + 8 * rq + 4 * h;
        f32x4 v = {o_acc[db][4 * rq] * inv, o_acc[db][4 * rq + 1] * inv,
                   o_acc[db][4 * rq + 2] * inv, o_acc[db][4 * rq + 3] * inv};
        *(f32x4*)(orow + d0) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// fp32 kernel for small problems: the key range of a 32-row block split over
// the waves of a workgroup.  With few query blocks (GPT-2's 128-token
// prompt: 12 heads x 128 rows), flash_fwd_f32 runs a few dozen waves, each a
// serial chain of fp32 MFMAs over every key (v_mfma_f32_32x32x2f32 is 64
// cycles): latency, not throughput.  Here workgroup (b, hq, row block) runs
// 4 waves; wave w takes the 32-key chunks w, w + 4, ... of the block's keys,
// with K and V read from global memory straight into MFMA operand layout
// (no LDS tiles), and keeps its own online softmax state; at the end the
// four states are merged through LDS (m* = max m_w, O = sum 2^(m_w - m*)
// O_w / sum 2^(m_w - m*) l_w) and the block's rows are stored.
// ---------------------------------------------------------------------------
constexpr int KS_ROWS = 32;  // query rows per workgroup
constexpr int KS_KEYS = 32;  // keys per chunk
#ifndef KS_SMALL_GRID
#define KS_SMALL_GRID 64
#endif
template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads) void flash_fwd_f32_ks(FlashParams p) {
  constexpr int NDB = D / 32;
  constexpr int NC = D / 8;  // 16-byte chunks per lane half
  __shared__ float s_ml[4][2][KS_ROWS];
  __shared__ float s_o[3][NDB][16][64];  // waves 1..3's O^T accumulators, lane-minor (no bank conflicts)

  const int n_rb = (p.seq_q + KS_ROWS - 1) / KS_ROWS;
  const int rb = n_rb - 1 - (int)(blockIdx.x % n_rb);  // longest blocks first
  const int hq = (int)(blockIdx.x / n_rb) % p.n_head;
  const int b = (int)(blockIdx.x / n_rb) / p.n_head;
  const int hkv = hq / p.group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31;
  const int h = lane >> 5;
  const int off = p.seq_k - p.seq_q;
  const int q0 = rb * KS_ROWS;
  const int qi = q0 + lq;
  int k_end = p.seq_k;
  if (CAUSAL) k_end = max(0, min(p.seq_k, min(q0 + KS_ROWS - 1, p.seq_q - 1) + off + 1));
  const int n_ch = (k_end + KS_KEYS - 1) / KS_KEYS;

  f32x4 qf[NC];
  {
    const float* qrow = (const float*)p.q + b * p.q_sb + hq * p.q_sh + (int64_t)min(qi, p.seq_q - 1) * p.q_ss;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      qf[cc] = qi < p.seq_q ? *(const f32x4*)(qrow + h * (D / 2) + 4 * cc) : z;
    }
  }
  f32x16 o_acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const float* kbase = (const float*)p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = (const float*)p.v + b * p.v_sb + hkv * p.v_sh;
  const float c = p.scale_log2;
  for (int ch = wave; ch < n_ch; ch += 4) {
    const int kb = ch * KS_KEYS;
    // K^T operand: lane (lq, h) holds key kb + lq, d = h D/2 + 4 cc + i;
    // V^T operand of step r: key kb + 8 (r / 4) + 4 h + r % 4, d = 32 db + lq.
    f32x4 kf[NC];
    float vf[16][NDB];
    {
      const int key = kb + lq;
      const float* krow = kbase + (int64_t)min(key, p.seq_k - 1) * p.k_ss + h * (D / 2);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        kf[cc] = key < p.seq_k ? *(const f32x4*)(krow + 4 * cc) : z;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kv = kb + 8 * (r >> 2) + 4 * h + (r & 3);
        const float* vrow = vbase + (int64_t)min(kv, p.seq_k - 1) * p.v_ss + lq;
#pragma unroll
        for (int db = 0; db < NDB; ++db) vf[r][db] = kv < p.seq_k ? vrow[32 * db] : 0.f;
      }
    }
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[cc][i], qf[cc][i], s, 0, 0, 0);
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb + 8 * (r >> 2) + 4 * h + (r & 3);
      const bool ok = key < p.seq_k && (!CAUSAL || key <= qi + off);
      const float x = ok ? s[r] * c : -INFINITY;
      s[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx);
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - base);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < NDB; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = fast_exp2(s[r] - base);
      s[r] = e;
      l_run += e;
    }
    // O^T += V^T . P^T: step r uses key 8 (r / 4) + 4 h + r % 4 of the chunk
    // in lane half h (MFMA k = h), so P^T is the lane's own S value.
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int db = 0; db < NDB; ++db) o_acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[r][db], s[r], o_acc[db], 0, 0, 0);
  }

  // Merge the four waves' states (a wave with no chunk has m = -inf, l = 0).
  const float l_row = l_run + xor32(l_run);  // both lane halves hold the row's max
  if (h == 0) {
    s_ml[wave][0][lq] = m_run;
    s_ml[wave][1][lq] = l_row;
  }
  if (wave > 0) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) s_o[wave - 1][db][r][lane] = o_acc[db][r];
  }
  __syncthreads();
  if (wave != 0) return;
  float mw[4];
  float ms = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = s_ml[w][0][lq];
    ms = fmaxf(ms, mw[w]);
  }
  const float mb = (ms == -INFINITY) ? 0.f : ms;
  float wt[4], lsum = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    wt[w] = fast_exp2(mw[w] - mb);
    lsum += wt[w] * s_ml[w][1][lq];
  }
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    f32x16 a = o_acc[db];
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] *= wt[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
#pragma unroll
      for (int r = 0; r < 16; ++r) a[r] += wt[w] * s_o[w - 1][db][r][lane];
    }
    o_acc[db] = a;
  }
  const float inv = 1.f / lsum;
  if (qi < p.seq_q) {
    float* orow = (float*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)qi * p.o_ss;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const int d0 = 32 * db + 8 * rq + 4 * h;
        const f32x4 v = {o_acc[db][4 * rq] * inv, o_acc[db][4 * rq + 1] * inv, o_acc[db][4 * rq + 2] * inv,
                         o_acc[db][4 * rq + 3] * inv};
        *(f32x4*)(orow + d0) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// V (b, kv, s, d) -> V^T (b, kv, d, s_pad), s_pad a multiple of 128, keys past
// seq_k zero-filled.  Within each group of 16 keys the stored order is
//     position 16 u + 8 h + j  <-  key 16 u + 8 (j / 4) + 4 h + (j % 4)
// which is the key order of the PV MFMA's k-index for lane half h (the S^T
// accumulator layout puts keys 8 a + 4 h + b, b < 4, in lane half h), so a
// lane's 8 keys are contiguous.
//
// Tiles of 64 keys of one (b, kv head), numbered key tile fastest; workgroup
// w takes tiles w, w + gridDim.x, ...  A tile goes global -> registers ->
// LDS -> (transposed) global; the next tile's loads are issued before the
// current one is transposed, and the two LDS buffers alternate, so each
// workgroup keeps a tile of loads in flight (the copy is otherwise bound by
// load latency, one tile per workgroup).  In LDS the 16-byte chunk c of key
// row r sits at slot c ^ f(r), f(r) = ((r >> 4) & 3) | (((r >> 2) & 1) << 2):
// the 8 keys one transposing read instruction covers (16 u + 4 h + const)
// then fall in 8 different slots, 32 distinct banks for 64 lanes.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void vt_pack_kernel(const uint16_t* __restrict__ v,
                                                      uint16_t* __restrict__ vt, int seq_k,
                                                      int sk_pad, int n_kv, int n_tiles, int64_t v_sb,
                                                      int64_t v_sh, int64_t v_ss) {
  constexpr int PER = 64 * D / 8 / 256;  // 16-byte chunks each thread loads per tile
  constexpr int CPR = D / 8;             // chunks per key row
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][64 * D];
  const int kts = sk_pad / 64;
  auto swz = [](int r) { return ((r >> 4) & 3) | (((r >> 2) & 1) << 2); };
  auto load = [&](int t, u32x4 (&val)[PER]) {
    const int kt = t % kts, bh = t / kts;
    const uint16_t* src = v + (bh / n_kv) * v_sb + (bh % n_kv) * v_sh;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int r = c / CPR, col = c % CPR;
      const int key = kt * 64 + r;
      val[i] = key < seq_k ? *(const u32x4*)(src + (int64_t)key * v_ss + col * 8) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  u32x4 val[PER];
  int t = blockIdx.x;
  if (t >= n_tiles) return;
  load(t, val);
  for (int buf = 0; t < n_tiles; t += gridDim.x, buf ^= 1) {
    uint16_t* tl = tile[buf];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int r = c / CPR, col = c % CPR;
      *(u32x4*)(tl + r * D + ((col ^ swz(r)) << 3)) = val[i];
    }
    if (t + (int)gridDim.x < n_tiles) load(t + gridDim.x, val);
    __syncthreads();
    const int kt = t % kts, bh = t / kts;
    uint16_t* dst = vt + (int64_t)bh * D * sk_pad + kt * 64;
    for (int c = threadIdx.x; c < D * 8; c += 256) {
      const int d = c / 8, ch = c % 8;
      const int u = ch >> 1, h = ch & 1;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const int k0 = 16 * u + 8 * (j / 4) + 4 * h + (j % 4);
        const int e0 = k0 * D + (((d >> 3) ^ swz(k0)) << 3) + (d & 7);
        const int e1 = (k0 + 1) * D + (((d >> 3) ^ swz(k0 + 1)) << 3) + (d & 7);
        w[j / 2] = (uint32_t)tl[e0] | ((uint32_t)tl[e1] << 16);
      }
      *(u32x4*)(dst + (int64_t)d * sk_pad + ch * 8) = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

// ---------------------------------------------------------------------------
// Generic kernel for what the MFMA kernels do not cover: any power-of-two d_k
// up to kGenericMaxD (the reference accepts any power of two), strides that
// are not 16-byte multiples, and fp16 with a scale that would overflow a
// pre-scaled Q.  One wave per (query row, head), keys in tiles of 64 with
// the reference's online softmax, all in fp32.  The scaled query row and the
// output accumulator live in LDS (2 * d_k floats, dynamic), lane l owning
// accumulator entries l, l + 64, ...
// ---------------------------------------------------------------------------
constexpr int kGenericMaxD = 4096;

template <typename T>
__global__ __launch_bounds__(64) void attn_generic_kernel(FlashParams p, int D, int causal) {
  using Bits = typename T::bits;
  extern __shared__ float gsm[];
  float* qs = gsm;       // [D]
  float* acc = gsm + D;  // [D]
  __shared__ float ps[64];
  const int qi = blockIdx.x;
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int hkv = hq / p.group;
  const int lane = threadIdx.x;
  const Bits* qrow = (const Bits*)p.q + b * p.q_sb + hq * p.q_sh + (int64_t)qi * p.q_ss;
  for (int d = lane; d < D; d += 64) {
    qs[d] = to_f32<T>(qrow[d]);
    acc[d] = 0.f;
  }
  __syncthreads();
  const Bits* kb = (const Bits*)p.k + b * p.k_sb + hkv * p.k_sh;
  const Bits* vb = (const Bits*)p.v + b * p.v_sb + hkv * p.v_sh;
  const int limit = causal ? min(p.seq_k, qi + (p.seq_k - p.seq_q) + 1) : p.seq_k;
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;
  for (int k0 = 0; k0 < p.seq_k; k0 += 64) {
    const int key = k0 + lane;
    float s = -INFINITY;
    if (key < limit) {
      const Bits* kr = kb + (int64_t)key * p.k_ss;
      float d = 0.f;
      for (int e = 0; e < D; ++e) d = fmaf(qs[e], to_f32<T>(kr[e]), d);
      s = d * c;
    }
    float mx = s;
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float m_new = fmaxf(m_run, mx);
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - base);
    const float pk = fast_exp2(s - base);
    float sum = pk;
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    l_run = l_run * alpha + sum;
    m_run = m_new;
    __syncthreads();
    ps[lane] = pk;
    __syncthreads();
    const int n = min(64, p.seq_k - k0);
    for (int d = lane; d < D; d += 64) {
      float a = acc[d] * alpha;
      for (int kk = 0; kk < n; ++kk) {
        const float pw = ps[kk];
        if (pw != 0.f) a = fmaf(pw, to_f32<T>(vb[(int64_t)(k0 + kk) * p.v_ss + d]), a);
      }
      acc[d] = a;
    }
  }
  Bits* orow = (Bits*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)qi * p.o_ss;
  const float inv = 1.f / l_run;
  for (int d = lane; d < D; d += 64) orow[d] = from_f32<T>(acc[d] * inv);
}

inline bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Keys per V^T row: seq_k rounded up to a multiple of 128.
inline int64_t vt_row_keys(int64_t seq_k) { return (seq_k + 127) / 128 * 128; }

// Bytes of the key-major V^T copy.
size_t vt_bytes(int batch, int n_kv, int seq_k, int d_k) {
  return (size_t)batch * n_kv * d_k * (size_t)vt_row_keys(seq_k) * 2;
}

// ---- schedule planning (host) ----------------------------------------------------
// Partial slot of one key-split part: per wave, O^T unnormalised (D / 2
// floats per lane) and (m, l) per lane.
static size_t split_slot_bytes(int D) { return 8u * ((size_t)(D / 32) * 4 * 1024 + 512); }
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// K tiles a whole query tile qt reads (causal: up to its last row's diagonal).
static int tile_k_tiles(const FlashParams& p, int qt, bool causal) {
  int k_end = p.seq_k;
  if (causal) {
    const int q_last = min(p.seq_q, qt * K16_BM + K16_BM) - 1;
    k_end = max(0, min(p.seq_k, q_last + (p.seq_k - p.seq_q) + 1));
  }
  return (k_end + K16_BN - 1) / K16_BN;
}

static void set_rounds(FlashParams& p, int cus) {
  p.q_machines = min((cus + p.n_queues - 1) / p.n_queues, p.q_tiles);
  const int rounds = p.q_tiles / p.q_machines;
  p.q_triple = (p.q_tiles % p.q_machines == 0 && rounds % 2 == 1 && rounds >= 3 && p.q_machines % 2 == 0) ? 1 : 0;
}

// Modelled time of the busiest workgroup, in K steps: a whole tile of n K
// tiles costs n + kTileOvh (its steps and its tile switch, first G phase and
// first softmax, which do not overlap), a key-split part its own K tiles +
// kTileOvh + kMergeOvh (the same and the merge); items are dealt as the
// kernel deals them (decode_item, sched_rank).  The two constants were
// fitted by timing Llama-3.2-3B-shaped prompts (1024-4096 tokens, 16, 24
// and 32 query heads) under five settings: (2, 1.5) was best or tied on
// every shape, e.g. 40.9 against 43.4 us at 2048 tokens with (1, 0.5).
constexpr double kTileOvh = 2.0;
constexpr double kMergeOvh = 1.5;

static double busiest_cost(const FlashParams& p) {
  const double ovh = kTileOvh;
  const int off = p.seq_k - p.seq_q;
  double worst = 0.0;
  for (int queue = 0; queue < p.n_queues; ++queue)
    for (int j = 0; j < p.q_machines; ++j) {
      double sum = 0.0;
      for (int r = 0;; ++r) {
        const int i = sched_rank(p, j, r);
        if (i >= p.q_tiles) break;
        int b, hq, qt, kpart = 0;
        if (p.n_entries) {
          int sidx;
          decode_item(p, queue, i, p.e_code[i / p.q_parts], b, hq, qt, kpart, sidx);
        } else {
          decode_tile(p, queue, i, b, hq, qt);
        }
        const int n = tile_k_tiles(p, qt, true);
        if (kpart == 0) {
          sum += n + ovh;
        } else {
          const int h = min(n / 2, (qt * K16_BM + off) / K16_BN);
          sum += (kpart == 1 ? h : n - h) + ovh + kMergeOvh;
        }
      }
      worst = fmax(worst, sum);
    }
  return worst;
}

// Tile lists and rounds of flash_fwd_16, and its key split: causal calls
// (seq_k >= seq_q) with fewer tiles than a few rounds of the machine may cut
// the key range of their s costliest levels in two (one list entry per
// part), the s that minimises the modelled busiest workgroup, when that
// beats no split by 5% and the split region (arrival words, then two
// partial slots per split tile) fits in split_room bytes.  Returns the split
// region's size (0: no split).
static size_t plan_flash_16_uncached(FlashParams& p, int D, bool causal, size_t split_room, int cus) {
  p.n_qt = (p.seq_q + K16_BM - 1) / K16_BM;
  // Tile lists: one per XCD when the query heads' tiles deal evenly into 8
  // lists of whole parts (q_split parts per head, each n_qt / q_split tiles);
  // otherwise one list.
  const int heads = p.batch * p.n_head;
  p.n_queues = 1;
  p.q_split = 1;
  if (!tl_overrides.prefill_one_list) {
    for (int s = 1; s <= 8; s *= 2) {
      if ((int64_t)heads * s % 8 == 0 && p.n_qt % s == 0) {
        p.n_queues = 8;
        p.q_split = s;
        break;
      }
    }
  }
  p.q_parts = (int)((int64_t)heads * p.q_split / p.n_queues);
  int levels = p.n_qt / p.q_split;
  p.q_tiles = p.q_parts * levels;
  p.n_entries = 0;
  p.n_split_levels = 0;
  p.n_split_tiles = 0;
  p.split_part_bytes = 0;
  set_rounds(p, cus);
  if (!causal || p.seq_k < p.seq_q || tl_overrides.prefill_no_split) return 0;
  // Splits are planned on one list of whole heads (kept only if a split is
  // worth it) at d_k 64, and wherever the per-XCD lists cut each head into
  // as many parts as it has tiles, which leaves one cost level and nothing
  // to split (SmolLM2-135M at batch 1: 9 heads, 8 parts each).  Measured
  // against splits planned on the per-XCD lists: config 3 33.1 against 34.9
  // us (unsplit there), SmolLM2-360M heads at batch 2 29.4 against 33.3 us;
  // at d_k 128 the per-XCD lists were as fast or faster (Llama-3.2-3B at
  // 1024 and 2048 tokens: 25.8 / 40.6 against 26.5 / 41.2 us).
  const FlashParams lists = p;
  if ((levels < 2 || D == 64) && p.n_queues > 1 && p.n_qt >= 2) {
    p.n_queues = 1;
    p.q_split = 1;
    p.q_parts = heads;
    levels = p.n_qt;
    p.q_tiles = p.q_parts * levels;
    set_rounds(p, cus);
  }
  if (levels < 2 || levels > kMaxEntries / 2 || (int64_t)p.q_tiles * p.n_queues > 4 * (int64_t)cus) {
    p = lists;
    return 0;
  }
  const double base = busiest_cost(p);
  const double ovh = kTileOvh;
  FlashParams best = p;
  double best_cost = base;
  size_t best_bytes = 0;
  // level lvl holds qt = j + q_split (levels - 1 - lvl): every level but the
  // last has qt >= 1, whose parts both reach every query row
  for (int s = 1; s < levels; ++s) {
    FlashParams c = p;
    const int tiles = p.n_queues * s * p.q_parts;
    const size_t part_bytes = (size_t)tiles * 2 * split_slot_bytes(D);
    const size_t bytes = align256((size_t)tiles * 64) + part_bytes;
    if (bytes > split_room || part_bytes >= ((size_t)1 << 31)) break;
    // entries: (mean cost, level, part); ordered by cost descending
    struct Ent { double cost; int lvl, kpart; };
    Ent ent[kMaxEntries];
    int n = 0;
    for (int lvl = 0; lvl < levels; ++lvl) {
      double whole = 0.0, lo = 0.0, hi = 0.0;
      for (int j = 0; j < p.q_split; ++j) {
        const int qt = j + p.q_split * (levels - 1 - lvl);
        const int k = tile_k_tiles(p, qt, true);
        const int h = min(k / 2, (qt * K16_BM + p.seq_k - p.seq_q) / K16_BN);
        whole += k + ovh;
        lo += h + ovh + kMergeOvh;
        hi += (k - h) + ovh + kMergeOvh;
      }
      if (lvl < s) {
        ent[n++] = {lo / p.q_split, lvl, 1};
        ent[n++] = {hi / p.q_split, lvl, 2};
      } else {
        ent[n++] = {whole / p.q_split, lvl, 0};
      }
    }
    std::stable_sort(ent, ent + n, [](const Ent& a, const Ent& b) { return a.cost > b.cost; });
    for (int e = 0; e < n; ++e) c.e_code[e] = (uint8_t)(ent[e].lvl | ent[e].kpart << 6);  // lvl < 32
    c.n_entries = n;
    c.n_split_levels = s;
    c.n_split_tiles = tiles;
    c.split_part_bytes = (uint32_t)part_bytes;
    c.q_tiles = p.q_parts * n;
    set_rounds(c, cus);
    const double cost = busiest_cost(c);
    if (cost < best_cost) {
      best = c;
      best_cost = cost;
      best_bytes = bytes;
    }
  }
  if (best_cost > 0.95 * base) {
    p = lists;
    return 0;
  }
  p = best;
  return best_bytes;
}

// plan_flash_16_uncached, memoised: a call's plan depends only on the key
// below (the overrides included), and simulating the candidate
// splits costs tens of microseconds of host time, more than a short launch.
static size_t plan_flash_16(FlashParams& p, int D, bool causal, size_t split_room) {
  struct Key {
    int batch, n_head, seq_q, seq_k, D, causal, cus, one_list, no_split;
    size_t room;
    bool operator==(const Key& o) const {
      return batch == o.batch && n_head == o.n_head && seq_q == o.seq_q && seq_k == o.seq_k && D == o.D &&
             causal == o.causal && cus == o.cus && one_list == o.one_list && no_split == o.no_split &&
             room == o.room;
    }
  };
  struct Entry {
    Key key;
    FlashParams plan;
    size_t bytes;
  };
  static std::mutex mu;
  static Entry cache[16];
  static int n_cached = 0, next_slot = 0;
  const int cus = tl_device_cus();
  const Key key{p.batch,  p.n_head, p.seq_q, p.seq_k, D, causal ? 1 : 0, cus, tl_overrides.prefill_one_list,
                tl_overrides.prefill_no_split, split_room};
  auto take = [&p](const FlashParams& c) {  // the schedule fields only
    p.n_qt = c.n_qt;
    p.n_queues = c.n_queues;
    p.q_split = c.q_split;
    p.q_parts = c.q_parts;
    p.q_tiles = c.q_tiles;
    p.q_machines = c.q_machines;
    p.q_triple = c.q_triple;
    p.n_entries = c.n_entries;
    p.n_split_levels = c.n_split_levels;
    p.n_split_tiles = c.n_split_tiles;
    p.split_part_bytes = c.split_part_bytes;
    for (int e = 0; e < kMaxEntries; ++e) p.e_code[e] = c.e_code[e];
  };
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < n_cached; ++i)
      if (cache[i].key == key) {
        take(cache[i].plan);
        return cache[i].bytes;
      }
  }
  FlashParams c = p;
  const size_t bytes = plan_flash_16_uncached(c, D, causal, split_room, cus);
  take(c);
  std::lock_guard<std::mutex> lock(mu);
  cache[next_slot] = Entry{key, c, bytes};
  next_slot = (next_slot + 1) % 16;
  n_cached = min(n_cached + 1, 16);
  return bytes;
}

// This call's arrival tag: a per-process random base plus a call count, so a
// word left in a reused workspace by an earlier call (or holding unrelated
// data) is not mistaken for it.  Never 0, the value a merge leaves behind.
static uint64_t next_split_token() {
  static const uint64_t base = [] {
    uint64_t b = (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count() * 0x9e3779b97f4a7c15ull ^
                 (uint64_t)(uintptr_t)&b;
    try {  // no exception may leave the C ABI
      std::random_device rd;
      b ^= ((uint64_t)rd() << 32) ^ (uint64_t)rd();
    } catch (...) {
    }
    return b;
  }();
  static std::atomic<uint64_t> count{0};
  const uint64_t t = base + 2 * (count.fetch_add(1, std::memory_order_relaxed) + 1);
  return t ? t : 1;
}

template <typename T, int D>
int launch_flash_16(FlashParams& p, void* ws, size_t ws_bytes, bool causal, hipStream_t st) {
  // fp16 Q pre-scaled by |sm_scale log2 e| > 1 could overflow: scale scores instead
  const bool scale_s = std::is_same<T, F16>::value && fabsf(p.scale_log2) > 1.f;
  p.vt = ws;
  // d_k 128 with 64 query rows per wave (tl_prefill_w64.hip): on request
  // only (TRITON_LLM_HIP_PREFILL_W64); it measures about 8% slower than this
  // kernel on config 5a.  Not when the scores must be scaled in fp32 (fp16,
  // large scale); it addresses a wave's 64 output rows with 32-bit offsets.
  const bool w64 = D == 128 && !scale_s && tl_overrides.prefill_w64 && (64 * p.o_ss + D) * 2 < ((int64_t)1 << 32);
  const size_t vt_need = D == 64 ? 0 : vt_bytes(p.batch, p.n_kv, p.seq_k, D);
  const size_t room = ws && aligned16(ws) && ws_bytes > align256(vt_need) ? ws_bytes - align256(vt_need) : 0;
  p.split_ws = nullptr;
  p.split_token = 0;
  if (plan_flash_16(p, D, causal, w64 ? 0 : room)) {
    p.split_ws = (char*)ws + align256(vt_need);
    p.split_token = next_split_token();
  }
  if constexpr (D != 64) {  // d_k 64 reads V in place
    const int vt_tiles = p.sk_pad / 64 * p.n_kv * p.batch;
    const int vt_grid = min(vt_tiles, 2 * tl_device_cus());
    hipLaunchKernelGGL(vt_pack_kernel<D>, dim3(vt_grid), dim3(256), 0, st, (const uint16_t*)p.v, (uint16_t*)ws,
                       p.seq_k, p.sk_pad, p.n_kv, vt_tiles, p.v_sb, p.v_sh, p.v_ss);
    const int e = tl_launch_status();
    if (e) return e;
  }
  if (w64) return launch_flash_w64(p, T::code, causal, st);
  dim3 grid((unsigned)(p.q_machines * p.n_queues));
  if constexpr (std::is_same<T, F16>::value) {
    if (scale_s) {
      if (causal)
        hipLaunchKernelGGL((flash_fwd_16<T, D, true, true>), grid, dim3(K16_THREADS), 0, st, p);
      else
        hipLaunchKernelGGL((flash_fwd_16<T, D, false, true>), grid, dim3(K16_THREADS), 0, st, p);
      return tl_launch_status();
    }
  }
  if (causal)
    hipLaunchKernelGGL((flash_fwd_16<T, D, true>), grid, dim3(K16_THREADS), 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_16<T, D, false>), grid, dim3(K16_THREADS), 0, st, p);
  return tl_launch_status();
}

template <int D>
int launch_flash_f32(FlashParams& p, bool causal, hipStream_t st) {
  p.n_qt = (p.seq_q + BM - 1) / BM;
  const int64_t blocks = (int64_t)p.n_qt * p.n_head * p.batch;
  if (blocks < KS_SMALL_GRID) {
    // few 128-row blocks: split each 32-row block's keys over 4 waves
    dim3 g((unsigned)((int64_t)((p.seq_q + KS_ROWS - 1) / KS_ROWS) * p.n_head * p.batch));
    if (causal)
      hipLaunchKernelGGL((flash_fwd_f32_ks<D, true>), g, dim3(kThreads), 0, st, p);
    else
      hipLaunchKernelGGL((flash_fwd_f32_ks<D, false>), g, dim3(kThreads), 0, st, p);
    return tl_launch_status();
  }
  dim3 grid((unsigned)blocks);
  if (causal)
    hipLaunchKernelGGL((flash_fwd_f32<D, true>), grid, dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL((flash_fwd_f32<D, false>), grid, dim3(kThreads), 0, st, p);
  return tl_launch_status();
}

template <typename T>
int launch_generic(FlashParams& p, int d_k, bool causal, hipStream_t st) {
  dim3 grid(p.seq_q, p.n_head, p.batch);
  hipLaunchKernelGGL(attn_generic_kernel<T>, grid, dim3(64), 2 * d_k * sizeof(float), st, p, d_k, causal ? 1 : 0);
  return tl_launch_status();
}

bool mfma_shape_ok(const FlashParams& p, int d_k, int dtype) {
  if (d_k != 64 && d_k != 128) return false;
  const int64_t vec = dtype == TL_DTYPE_F32 ? 4 : 8;  // elements per 16 bytes
  const int64_t s[] = {p.q_sb, p.q_sh, p.q_ss, p.k_sb, p.k_sh, p.k_ss,
                       p.v_sb, p.v_sh, p.v_ss, p.o_sb, p.o_sh, p.o_ss};
  for (int64_t x : s)
    if (x < 0 || x % vec) return false;
  if (dtype != TL_DTYPE_F32) {
    // The 16-bit kernel addresses a K or Q tile (128 rows), a wave's 32
    // output rows and a head's V^T copy with 32-bit byte offsets, and bounds
    // a K or Q tile's reads and an output block's stores by its row count
    // times the row stride (rows must not overlap).
    const int64_t sk_pad = vt_row_keys(p.seq_k);
    if (p.k_ss < d_k || (128 * p.k_ss + d_k) * 2 >= ((int64_t)1 << 32) || p.q_ss < d_k ||
        p.o_ss < d_k || (32 * p.o_ss + d_k) * 2 >= ((int64_t)1 << 32) ||
        (128 * p.q_ss + d_k) * 2 >= ((int64_t)1 << 32) || (int64_t)d_k * sk_pad * 2 >= ((int64_t)1 << 32))
      return false;
    // d_k 64 reads V tiles in place, bounded like K's
    if (d_k == 64 && (p.v_ss < d_k || (128 * p.v_ss + d_k) * 2 >= ((int64_t)1 << 32))) return false;
  }
  return aligned16(p.q) && aligned16(p.k) && aligned16(p.v) && aligned16(p.o);
}

}  // namespace

extern "C" {

size_t tl_attention_fwd_workspace_bytes(int batch, int n_kv_head, int seq_k, int d_k,
                                        int dtype) {
  // 16-bit MFMA path at d_k 128: the permuted key-major V^T copy.  d_k 64,
  // fp32 and the generic kernel read V in place.
  if (dtype == TL_DTYPE_F32 || batch <= 0 || n_kv_head <= 0 || seq_k <= 0 || d_k != 128)
    return 0;
  return vt_bytes(batch, n_kv_head, seq_k, d_k);
}

size_t tl_attention_fwd_workspace_bytes_split(int batch, int n_head, int n_kv_head, int seq_q, int seq_k,
                                              int d_k, int causal, int dtype) {
  const size_t base = tl_attention_fwd_workspace_bytes(batch, n_kv_head, seq_k, d_k, dtype);
  if ((dtype != TL_DTYPE_BF16 && dtype != TL_DTYPE_F16) || (d_k != 64 && d_k != 128) || !causal ||
      batch <= 0 || n_head <= 0 || n_kv_head <= 0 || n_head % n_kv_head || seq_q <= 0 || seq_k <= 0)
    return base;
  FlashParams p{};
  p.batch = batch;
  p.n_head = n_head;
  p.n_kv = n_kv_head;
  p.group = n_head / n_kv_head;
  p.seq_q = seq_q;
  p.seq_k = seq_k;
  const size_t split = plan_flash_16(p, d_k, true, SIZE_MAX);
  return split ? align256(base) + split : base;
}

int tl_attention_fwd(const void* q, const void* k, const void* v, void* o, void* workspace,
                     size_t workspace_bytes, int batch, int n_head, int n_kv_head,
                     int seq_q, int seq_k, int d_k, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* v_strides,
                     const int64_t* o_strides, float sm_scale, int causal, int dtype,
                     void* stream) {
  if (batch == 0 || n_head == 0 || seq_q == 0) return 0;
  if (!q || !k || !v || !o || batch < 0 || n_head < 0 || n_kv_head < 1 ||
      n_head % n_kv_head != 0 || seq_q < 0 || seq_k < 1 || d_k < 1 ||
      !q_strides || !k_strides || !v_strides || !o_strides)
    return TL_ERR_INVALID;
  if (d_k > kGenericMaxD) return TL_ERR_UNSUPPORTED;
  FlashParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.batch = batch;
  p.n_head = n_head;
  p.n_kv = n_kv_head;
  p.group = n_head / n_kv_head;
  p.seq_q = seq_q;
  p.seq_k = seq_k;
  p.n_qt = (seq_q + BM - 1) / BM;
  p.sk_pad = (int)vt_row_keys(seq_k);
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  hipStream_t st = tl_resolve_stream(stream);
  const bool cz = causal != 0;
  if (mfma_shape_ok(p, d_k, dtype)) {
    if (dtype == TL_DTYPE_F32) {
      return d_k == 64 ? launch_flash_f32<64>(p, cz, st) : launch_flash_f32<128>(p, cz, st);
    }
    const size_t need = tl_attention_fwd_workspace_bytes(batch, n_kv_head, seq_k, d_k, dtype);
    if (need && (!workspace || !aligned16(workspace) || workspace_bytes < need)) return TL_ERR_INVALID;
    if (dtype == TL_DTYPE_BF16)
      return d_k == 64 ? launch_flash_16<BF16, 64>(p, workspace, workspace_bytes, cz, st)
                       : launch_flash_16<BF16, 128>(p, workspace, workspace_bytes, cz, st);
    if (dtype == TL_DTYPE_F16)
      return d_k == 64 ? launch_flash_16<F16, 64>(p, workspace, workspace_bytes, cz, st)
                       : launch_flash_16<F16, 128>(p, workspace, workspace_bytes, cz, st);
    return TL_ERR_INVALID;
  }
  switch (dtype) {
    case TL_DTYPE_F32: return launch_generic<F32>(p, d_k, cz, st);
    case TL_DTYPE_F16: return launch_generic<F16>(p, d_k, cz, st);
    case TL_DTYPE_BF16: return launch_generic<BF16>(p, d_k, cz, st);
    default: return TL_ERR_INVALID;
  }
}

}  // extern "C"
