// Causal / non-causal prefill attention at d_k 128 (bf16 / fp16) with 64
// query rows per wave: flash_fwd_w64.  Same semantics, layouts, V^T copy
// (vt_pack_kernel) and persistent tile schedule as flash_fwd_16 in
// tl_prefill.hip (reference: triton_llm/kernels/attention_gqa.py:21-146).
// It runs when TRITON_LLM_HIP_PREFILL_W64 is set: on config 5a it measures
// about 0.92x flash_fwd_16 (gfx950, 1080-1118 against 1179-1225 TFLOP/s on
// the same boxes), so flash_fwd_16 stays the default.
//
// Why a second kernel.  In flash_fwd_16 a wave owns 32 query rows, so each K
// or V^T fragment it reads from LDS feeds one 32x32x16 MFMA: 1 KiB of LDS
// reads per 32-cycle MFMA.  Here a wave owns 64 rows as two 32-row query
// blocks, so every fragment feeds two MFMAs: half the LDS bytes per MFMA.
// The price is one wave per SIMD, whose own instruction stream must keep
// the matrix core busy.  Measured on gfx950 with one wave per SIMD: 32
// MFMAs take 1024 cycles; every MFMA also takes about 9 cycles of the
// VALU issue port, an exp2 8, a simple VALU op about 4.5 and a 3-operand op
// about 5, so an iteration's softmax work (32 exp2, 32 adds, 16 max3, 16
// packs) and its 32 MFMAs just fit in about 1100 cycles.  The kernel's
// iterations take about 1480 (no loads) to 1930 cycles (with the tile
// loads): the gap to the MFMA bound is where its time goes.
//
// Registers (512 per lane at one wave per SIMD).  O^T, 128 fp32 per lane
// (64 rows x 128 d), and the Q^T fragments (64) live in AGPRs: every
// definition of them is an AGPR output of an asm statement, and the MFMAs
// that use them are inline asm.  This file is compiled with the MFMA
// builtins in VGPR form (-mllvm -amdgpu-mfma-vgpr-form=1).  VGPRs hold S
// of two 32-key blocks (64), the S seeds (32), P of two blocks (32) and the
// K / V^T fragments in flight.
//
// Pipeline.  Keys go in blocks u of 32.  Iteration u runs
//     PV(u-1) MFMAs (db 0..3, kk 0)   | max and lazy-rescale test of S(u)
//     -- branch: rescale bookkeeping (rare) --
//     S(u+1) MFMAs, PV(u-1) (kk 1)    | exp2 / pack / row sums of S(u) -> P(u)
//     -- branch: O *= alpha (rare, after PV(u-1) has completed) --
// so S(u+1) is seeded with the running maximum the softmax of block u has
// just settled (its accumulators start at -m_run), and P(u) feeds PV(u) in
// iteration u + 1.  Q is pre-scaled by sm_scale * log2 e, so P = exp2(S).
//
// LDS (160 KiB).  K and V^T come in tiles of 64 keys (two blocks) through
// rings of three buffers each; Q rows of the next query tile are staged in
// 64 KiB.  Block pair (tile) t of a query tile reads K_t, K_{t+1}, V_{t-1}
// and V_t; during it the workgroup loads K_{t+2} and V_{t+1} (LDS-DMA, eight
// 1 KiB loads per wave) into the buffers K_{t-1} and V_{t-2} left, waits for
// them at its end and passes one barrier.  The stream of tiles runs on into
// the next query tile of the schedule, so a query tile starts with its
// first two K tiles and first V tile already in LDS; each wave also loads
// its own 64 rows of the next query tile's Q during the first tile, and
// stages its output rows in the same 64 rows once that Q is in registers.
//
// Hazards the compiler cannot see in the inline-asm MFMAs are handled here:
// a VALU result read by an asm MFMA is at least two instructions old (an
// s_nop at each iteration start separates the previous iteration's P
// packing from the first PV MFMA); O is read or written by VALU code only
// after s_nop waits that pass through the asm as AGPR operands (so no
// access can be moved ahead of them); S is read by VALU code only an MFMA
// or more after the S MFMAs that wrote it, or after the same kind of wait
// (the tile's first block, and the masking of diagonal / tail blocks that
// runs just after the previous iteration's last S MFMA).
#include "tl_prefill.h"

#include <type_traits>

namespace {

using namespace tlp;

constexpr int W_THREADS = 256;                // 4 waves, one per SIMD
constexpr int W_D = 128;                      // head size
constexpr int W_KT = 64;                      // keys per K / V^T tile
constexpr int W_KTILE = W_KT * W_D * 2;       // 16 KiB: 64 key rows of 256 B
constexpr int W_VTILE = W_D * W_KT * 2;       // 16 KiB: 128 d-rows of 128 B
constexpr int W_QSTAGE = K16_BM * W_D * 2;    // 64 KiB: 256 query rows
constexpr int W_LDS = 3 * W_KTILE + 3 * W_VTILE + W_QSTAGE;
static_assert(W_LDS == 160 * 1024, "the whole LDS of a CU");

// V^T rows in LDS are 128 bytes (64 keys, 8 chunks of 16 bytes): chunk c of
// d-row r sits at slot c ^ vswz(r).  The 16 rows of a 16-lane read group
// share a chunk index; rows r and r + 1 fill one 256-byte bank line and
// vswz spreads the 8 row pairs over the 8 slots: 16 distinct bank groups.
__device__ __forceinline__ int vswz(int r) { return (r >> 1) & 7; }

// O^T += V^T . P^T with the accumulator in AGPRs.
// zero(c) sets c = 0 . 0 + 0 with the same instruction, so that every
// definition of an accumulator is an AGPR output of an asm statement: were
// it set to zero by ordinary code, its live range would not be tied to the
// AGPR file and the compiler would copy it in and out around every MFMA.
template <typename T>
struct PvMfma;
template <>
struct PvMfma<BF16> {
  static __device__ __forceinline__ void run(f32x16& c, const u32x4& a, const u32x4& b) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ void zero(f32x16& c, const u32x4& z) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(c) : "v"(z));
  }
};
template <>
struct PvMfma<F16> {
  static __device__ __forceinline__ void run(f32x16& c, const u32x4& a, const u32x4& b) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  static __device__ __forceinline__ void zero(f32x16& c, const u32x4& z) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %1, 0" : "=a"(c) : "v"(z));
  }
};

// S^T = K . Q^T + C with Q^T (the B operand) in AGPRs and C, S^T in VGPRs:
// first() starts a chain from the seed c (S is written to registers apart
// from c, which stays live), acc() continues it.
template <typename T>
struct SMfma;
template <>
struct SMfma<BF16> {
  static __device__ __forceinline__ void first(f32x16& s, const u32x4& k, const u32x4& q, const f32x16& c) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(s) : "v"(k), "a"(q), "v"(c));
  }
  static __device__ __forceinline__ void acc(f32x16& s, const u32x4& k, const u32x4& q) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s) : "v"(k), "a"(q));
  }
};
template <>
struct SMfma<F16> {
  static __device__ __forceinline__ void first(f32x16& s, const u32x4& k, const u32x4& q, const f32x16& c) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %3" : "=&v"(s) : "v"(k), "a"(q), "v"(c));
  }
  static __device__ __forceinline__ void acc(f32x16& s, const u32x4& k, const u32x4& q) {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(s) : "v"(k), "a"(q));
  }
};

// The same wait for S accumulators written by asm MFMAs before VALU code
// reads them.
__device__ __forceinline__ void wait_s(f32x16 (&s)[2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(s[0]), "+v"(s[1]));
}

// Wait until every issued asm MFMA has written its accumulator (the longest
// XDL write-to-VALU-read distance is 19 wait states; this gives 24) before
// VALU code reads or writes o; the accumulators pass through the asm so no
// such access can be scheduled ahead of it.
__device__ __forceinline__ void wait_o(f32x16 (&o)[4][2]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[1][0]), "+a"(o[1][1]), "+a"(o[2][0]), "+a"(o[2][1]),
                 "+a"(o[3][0]), "+a"(o[3][1]));
}

template <typename T, bool CAUSAL>
__global__ __launch_bounds__(W_THREADS, 1) void flash_fwd_w64(FlashParams p) {
  using Bits = typename T::bits;
  constexpr int NKS = W_D / 16;  // k-steps of S^T = K . Q^T
  constexpr int NDB = W_D / 32;  // 32-row d-blocks of O^T

  __shared__ __attribute__((aligned(1024))) char smem[W_LDS];
  const uint32_t lds0 = (uint32_t)(size_t)(__attribute__((address_space(3))) char*)smem;
  const uint32_t lds_k = lds0;                    // K ring: 3 x 16 KiB
  const uint32_t lds_v = lds0 + 3 * W_KTILE;      // V^T ring: 3 x 16 KiB
  const uint32_t lds_q = lds_v + 3 * W_VTILE;     // Q staging: 256 rows
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int off = p.seq_k - p.seq_q;  // bottom-right causal offset
  const int queue = blockIdx.x % p.n_queues;
  const int mach = blockIdx.x / p.n_queues;
  const uint32_t k_ss2 = (uint32_t)p.k_ss * 2u, q_ss2 = (uint32_t)p.q_ss * 2u;
  const uint32_t vt_row2 = (uint32_t)p.sk_pad * 2u;  // bytes per V^T d-row in global memory

  // ---- tiles ---------------------------------------------------------------
  struct Tile {
    int b, hq, qt, n_kt, k_rows;
    const char* kg;  // K rows of the tile's (batch, kv head)
    const char* vg;  // its V^T copy
  };
  auto make_tile = [&](int rank) __attribute__((always_inline)) {
    Tile tl;
    decode_tile(p, queue, rank, tl.b, tl.hq, tl.qt);
    const int q_last = min(p.seq_q, tl.qt * K16_BM + K16_BM) - 1;
    int k_end = p.seq_k;
    if (CAUSAL) k_end = max(0, min(p.seq_k, q_last + off + 1));
    // At least two K tiles, so the load stream never reaches past the next
    // query tile (tiles past k_end are loaded and never computed on).
    tl.n_kt = max(2, (k_end + W_KT - 1) / W_KT);
    tl.k_rows = min(p.seq_k, tl.n_kt * W_KT);
    const int hkv = tl.hq / p.group;
    tl.kg = (const char*)((const Bits*)p.k + tl.b * p.k_sb + hkv * p.k_sh);
    tl.vg = (const char*)((const Bits*)p.vt + ((int64_t)tl.b * p.n_kv + hkv) * W_D * p.sk_pad);
    return tl;
  };

  // ---- LDS-DMA of K / V^T tiles and Q rows ------------------------------------
  // K tile j: 16 regions of 4 rows; wave w loads regions w + 4 i.  Lane l of
  // region R covers row 4 R + l / 16, slot l % 16 = chunk (l % 16) ^
  // lds_swz<128>(row); row & 3 = l / 16 and (row >> 2) & 3 = w for every i.
  const int ln0 = fresh_lane();
  const uint32_t k_dma_lane =
      (uint32_t)(4 * wave + ln0 / 16) * k_ss2 + (uint32_t)(((ln0 % 16) ^ (4 * (ln0 / 16) + wave)) * 16);
  // V^T tile j: 16 regions of 8 d-rows of 128 bytes; lane l of region R covers
  // d-row 8 R + l / 8, slot l % 8 = chunk (l % 8) ^ vswz(row), and vswz(row) =
  // (4 (R & 1) + l / 16) & 7 with R & 1 = w & 1 for R = w + 4 i.
  const uint32_t v_dma_lane = (uint32_t)(8 * wave + ln0 / 8) * vt_row2 +
                              (uint32_t)(((ln0 % 8) ^ ((4 * (wave & 1) + ln0 / 16) & 7)) * 16);
  auto k_tile_dma = [&](const Tile& tl, int j, int slot) __attribute__((always_inline)) {
    const int rows = min(max(tl.k_rows - j * W_KT, 0), W_KT);
    const i32x4 rs = uniform_rsrc(tl.kg + (int64_t)j * W_KT * k_ss2, (uint32_t)rows * k_ss2);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lds_dma16(rs, k_dma_lane + (uint32_t)(16 * i) * k_ss2, lds_k + slot * W_KTILE + (wave + 4 * i) * 1024);
  };
  auto v_tile_dma = [&](const Tile& tl, int j, int slot) __attribute__((always_inline)) {
    const i32x4 rs = uniform_rsrc(tl.vg + (int64_t)j * W_KT * 2, (uint32_t)(W_D * p.sk_pad * 2 - j * W_KT * 2));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lds_dma16(rs, v_dma_lane + (uint32_t)(32 * i) * vt_row2, lds_v + slot * W_VTILE + (wave + 4 * i) * 1024);
  };
  // This wave's 64 Q rows of a tile: 16 regions of 4 rows at staging rows
  // 64 w + 4 i (rows past seq_q read as zeros).
  auto q_dma = [&](const Tile& tl) __attribute__((always_inline)) {
    const int r0 = tl.qt * K16_BM + 64 * wave;
    const int rows = min(max(p.seq_q - r0, 0), 64);
    const char* qg = (const char*)((const Bits*)p.q + tl.b * p.q_sb + tl.hq * p.q_sh + (int64_t)r0 * p.q_ss);
    const i32x4 rs = uniform_rsrc(qg, (uint32_t)rows * q_ss2);
    const int ln = fresh_lane();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 4 * i + ln / 16;
      const uint32_t vo = (uint32_t)row * q_ss2 + (uint32_t)(((ln % 16) ^ lds_swz<W_D>(row)) * 16);
      lds_dma16(rs, vo, lds_q + (64 * wave + 4 * i) * 256);
    }
  };

  // The same 16 loads as jobs 8..23 of an iteration (one per slot in slots
  // 8-23; none without a next tile).
  auto q_dma_job = [&](const Tile& tl, bool has) __attribute__((always_inline)) {
    const int r0 = tl.qt * K16_BM + 64 * wave;
    const int rows = has ? min(max(p.seq_q - r0, 0), 64) : 0;
    const char* qg = (const char*)((const Bits*)p.q + tl.b * p.q_sb + tl.hq * p.q_sh + (int64_t)r0 * p.q_ss);
    const i32x4 rs = uniform_rsrc(qg, (uint32_t)rows * q_ss2);
    const uint32_t lq0 = lds_q + 64 * wave * 256;
    return [=](int job) __attribute__((always_inline)) {
      if (job < 8) return;
      const int i = job - 8;
      const int row = 4 * i + ln0 / 16;
      const uint32_t vo = (uint32_t)row * q_ss2 + (uint32_t)(((ln0 % 16) ^ lds_swz<W_D>(row)) * 16);
      lds_dma16(rs, vo, lq0 + 4 * i * 256);
    };
  };

  // ---- registers ---------------------------------------------------------------
  u32x4 qf[2][NKS];          // Q^T fragments [query block][k-step], pre-scaled (AGPRs)
  f32x16 o[NDB][2];          // O^T [d-block][query block], AGPRs
  f32x16 s0[2], s1[2];       // S of the even / odd 32-key block [query block]
  u32x4 pwb[2][2][2];        // P of the last two blocks [parity of u][query block][16 keys]
  float m_run[2], l4[2][2];  // running max and two partial row sums per query block
  f32x16 seed[2];            // -m_run in every element: the S accumulators' initial value
  bool fresh[2];

  // Q of this wave from staging into registers, pre-scaled by sm_scale log2 e
  // and rounded to T (round to nearest even).
  auto load_q = [&]() __attribute__((always_inline)) {
    const int ln = fresh_lane();
    const int lq = ln & 31, h = ln >> 5;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int row = 64 * wave + 32 * qb + lq;
        const u32x4 raw = *(const u32x4*)(smem + 3 * W_KTILE + 3 * W_VTILE + row * 256 +
                                          (((2 * ks + h) ^ lds_swz<W_D>(lq)) << 4));
        uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float lo, hi;
          unpack2<T>(w[i], lo, hi);
          const float x[2] = {lo * p.scale_log2, hi * p.scale_log2};
          w[i] = pack2<T>(x);
        }
        // defined as an AGPR output, so the fragments live in AGPRs between tiles
        asm volatile("" : "=a"(qf[qb][ks]) : "0"(u32x4{w[0], w[1], w[2], w[3]}));
      }
  };

  // Fragment reads.  K (S^T A operand, 32 keys x 16 d): lane (lq, h) reads
  // key row 32 half + lq of the tile, chunk 2 ks + h.  V^T (O^T A operand,
  // 32 d x 16 keys): d-row 32 db + lq, chunk 4 half + 2 kk + h (16-key group
  // 2 half + kk of the tile).  One VGPR per operand holds the lane's
  // swizzled base (chunk h); a read XORs the chunk bits in and adds the ring
  // slot (a scalar); rows and d-blocks go into the offset field.
  const uint32_t kx0 = (uint32_t)((ln0 & 31) * 256 + (((ln0 >> 5) ^ lds_swz<W_D>(ln0 & 31)) << 4));
  const uint32_t vx0 = (uint32_t)((ln0 & 31) * 128 + (((ln0 >> 5) ^ vswz(ln0 & 31)) << 4));
  auto k_frag = [&](int slot, int half, int ks) __attribute__((always_inline)) {
    const uint32_t a = (kx0 ^ (uint32_t)(ks << 5)) + (uint32_t)__builtin_amdgcn_readfirstlane(slot * W_KTILE);
    return *(const u32x4*)(smem + a + half * 32 * 256);
  };
  auto v_frag = [&](int slot, int half, int db, int kk) __attribute__((always_inline)) {
    const uint32_t a = (vx0 ^ (uint32_t)((4 * half + 2 * kk) << 4)) + (uint32_t)__builtin_amdgcn_readfirstlane(slot * W_VTILE);
    return *(const u32x4*)(smem + 3 * W_KTILE + a + db * 32 * 128);
  };

  // ---- one iteration of the block pipeline ----------------------------------------
  // PAR: parity of u (S(u) in s0 / s1 by parity, S(u+1) in the other); DS:
  // compute S(u+1) from K slot ks_slot, tile rows 32 hs ..; DPV: PV(u-1)
  // from V^T slot vs_slot, tile keys 32 hv ..; DSM: softmax of S(u).
  //
  // A wave issues in order and its next MFMA waits for the matrix core, so
  // the instruction stream alternates: one MFMA per slot, then the slot's
  // share of the softmax (run while that MFMA executes), with every LDS
  // operand read at least eight slots ahead.
  //   slots 0-7   PV(u-1) of the block's first 16 keys (d-block s/2, query
  //               block s%2) | row max of S(u) | tile loads (LDS-DMA jobs
  //               0-7) | rescale test (a branch)
  //   slots 8-31  PV(u-1) of its last 16 keys (slots 8, 10, .. 22: d-block,
  //               query block) between S(u+1)'s 16 MFMAs | softmax jobs of
  //               S(u): exp2 of two scores, their pack into P(u) and row sums
  //               (16 jobs over slots 8-30) | Q loads of the next query tile
  //               (jobs 8-23, tile pair 0 only)
  // P(u) goes to the other buffer of pwb than P(u-1), which the PV MFMAs of
  // this iteration still read.
  // vnext carries the V^T fragments of the next iteration's first 16 keys, read
  // during this one.  Returns whether O must be rescaled by alpha (after
  // PV(u-1)).
  auto iteration = [&](auto par_tag, auto ds_tag, auto dpv_tag, auto dsm_tag, int u, int q0, int ks_slot, int hs,
                       int vs_slot, int hv, int vs_next, int hv_next, u32x4 (&vnext)[NDB], float (&alpha)[2],
                       auto&& dma) __attribute__((always_inline)) {
    constexpr int PAR = decltype(par_tag)::value;
    constexpr bool DS = decltype(ds_tag)::value;
    constexpr bool DPV = decltype(dpv_tag)::value;
    constexpr bool DSM = decltype(dsm_tag)::value;
    f32x16(&s_cur)[2] = PAR ? s1 : s0;
    f32x16(&s_nxt)[2] = PAR ? s0 : s1;
    u32x4(&pw)[2][2] = pwb[PAR ^ 1];    // P(u-1), read by PV(u-1)
    u32x4(&pnew)[2][2] = pwb[PAR];      // P(u), written here
    alpha[0] = alpha[1] = 1.f;

    if constexpr (DSM) {
      const int kb = 32 * u;
      const bool need_mask = (kb + 32 > p.seq_k) || (CAUSAL && kb + 31 > q0 + off);
      if (need_mask) {
        wait_s(s_cur);  // the last S MFMAs of the previous iteration are a few instructions back
        const int ln = fresh_lane();
        const int h = ln >> 5;
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          int lim = p.seq_k - 1 - kb - 4 * h;
          if (CAUSAL) lim = min(lim, q0 + 32 * qb + (ln & 31) + off - kb - 4 * h);
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            const int kl = 8 * (rr >> 2) + (rr & 3);
            s_cur[qb][rr] = kl <= lim ? s_cur[qb][rr] : -INFINITY;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- slots 0-7 ----
    u32x4 vf[NDB];  // V^T fragments of the first 16 keys
    u32x4 vg[NDB];  // V^T fragments of the last 16 keys
    u32x4 kf[NKS];  // K fragments of S(u+1)
    if constexpr (DPV) {
      asm volatile("s_nop 1");  // P(u-1) was packed by VALU: two wait states before an MFMA reads it
#pragma unroll
      for (int db = 0; db < NDB; ++db) vf[db] = vnext[db];
    }
    auto mx3 = [](float x, float y, float z) {
      return __builtin_elementwise_maximum(__builtin_elementwise_maximum(x, y), z);
    };
    float part[2][2], mxv[2] = {0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) {
      const int db = sl / 2, qb = sl % 2;
      // Every LDS operand is read at least eight slots (about 250 cycles)
      // before the MFMA that uses it: here V^T of the last 16 keys (used
      // from slot 8) and the first two K fragments of S(u+1) (slots 9, 13)
      if constexpr (DPV) {
        if (sl == 0) vg[0] = v_frag(vs_slot, hv, 0, 1);
        if (sl >= 2 && sl < 5) vg[sl - 1] = v_frag(vs_slot, hv, sl - 1, 1);
        PvMfma<T>::run(o[db][qb], vf[db], pw[qb][0]);
      }
      if constexpr (DS) {
        if (sl == 1) kf[0] = k_frag(ks_slot, hs, 0);
        if (sl == 5) kf[1] = k_frag(ks_slot, hs, 1);
      }
      dma(sl);  // LDS-DMA job sl of this iteration, if any
      if constexpr (DSM) {
        // row max of query block sl / 4 in four steps
        const int mq = sl / 4, st = sl % 4;
        const f32x16& v = s_cur[mq];
        if (st == 0) part[mq][0] = mx3(mx3(v[0], v[1], v[2]), v[3], v[4]);
        if (st == 1) part[mq][1] = mx3(mx3(v[5], v[6], v[7]), v[8], v[9]);
        if (st == 2) part[mq][0] = mx3(mx3(v[10], v[11], v[12]), v[13], part[mq][0]);
        if (st == 3) {
          float m = max_xor32(mx3(mx3(v[14], v[15], part[mq][1]), part[mq][0], part[mq][0]));
          asm volatile("" : "+v"(m));  // computed in this slot (see the P packing below)
          mxv[mq] = m;
        }
      }
      // one scheduling region per slot: its asm MFMA (volatile, so in program
      // order), then its VALU and LDS work
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x102, 32, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    bool rescale = false;
    if constexpr (DSM) {
      // m_run moves (and O is rescaled) only when the block's max exceeds it
      // by more than kRescaleLog2, or on the first block with a finite score
      // (S(u) is relative to m_run: its accumulators were seeded with -m_run)
      const bool g0 = fresh[0] ? (mxv[0] != -INFINITY) : (mxv[0] > kRescaleLog2);
      const bool g1 = fresh[1] ? (mxv[1] != -INFINITY) : (mxv[1] > kRescaleLog2);
      if (__any(g0 || g1)) {
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const float mx = mxv[qb];
          float delta = 0.f;
          if (fresh[qb]) {
            // first finite score (alpha 1: nothing accumulated; 2^-mx may overflow)
            if (mx != -INFINITY) delta = mx;
            fresh[qb] = mx == -INFINITY;
          } else if (mx > 0.f) {
            delta = mx;
            alpha[qb] = fast_exp2(-mx);
#pragma unroll
            for (int k = 0; k < 2; ++k) l4[qb][k] *= alpha[qb];
          }
          m_run[qb] += delta;
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) {
            s_cur[qb][rr] -= delta;
            seed[qb][rr] = -m_run[qb];
          }
        }
        rescale = __any(alpha[0] != 1.f || alpha[1] != 1.f);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- slots 8-31 ----
#pragma unroll
    for (int sl = 8; sl < 32; ++sl) {
      const int i = sl - 8;
      // MFMA of the slot: PV at even i < 16 (d-block i / 4, query block
      // (i % 4) / 2), S on the others (a PV slot stays empty without PV)
      const bool pv_slot = i % 2 == 0 && i < 16;
      if constexpr (DPV) {
        if (pv_slot) {
          const int db = i / 4, qb = (i % 4) / 2;
          PvMfma<T>::run(o[db][qb], vg[db], pw[qb][1]);
        }
      }
      if constexpr (DS) {
        // the remaining K fragments, eight slots before their S MFMAs (slots
        // 17, 21, 24, 26, 28, 30)
        if (i == 1) kf[2] = k_frag(ks_slot, hs, 2);
        if (i == 5) kf[3] = k_frag(ks_slot, hs, 3);
        if (i >= 8 && i < 16 && i % 2 == 0) kf[4 + (i - 8) / 2] = k_frag(ks_slot, hs, 4 + (i - 8) / 2);
        if (!pv_slot) {
          // S job number: slots 8-23 carry S on odd i, slots 24-31 on every i
          const int sj = i < 16 ? (i / 2) : (8 + (i - 16));
          const int ks = sj / 2, qb = sj % 2;
          if (ks == 0) SMfma<T>::first(s_nxt[qb], kf[ks], qf[qb][ks], seed[qb]);
          else SMfma<T>::acc(s_nxt[qb], kf[ks], qf[qb][ks]);
        }
      }
      if (i < 16) dma(8 + i);  // LDS-DMA job 8 + i, if any
      // V^T of the next iteration's first 16 keys (its slots 0-7)
      if (sl >= 23 && sl < 23 + NDB) vnext[sl - 23] = v_frag(vs_next, hv_next, sl - 23, 0);
      if constexpr (DSM) {
        // softmax job j (two scores: exp2, pack into P(u), row sums) in
        // slot i = 3j / 2: jobs 0..15 in slots 8..30, none where i % 3 == 2
        if (i < 23 && i % 3 != 2) {
          const int j = (2 * i + 1) / 3;
          const int qb = j / 8, r = 2 * (j % 8);
          float x[2] = {fast_exp2(s_cur[qb][r]), fast_exp2(s_cur[qb][r + 1])};
          uint32_t w = pack2<T>(x);
          float l = l4[qb][j % 2] + (x[0] + x[1]);
          asm volatile("" : "+v"(w), "+v"(l));  // computed in this slot
          pnew[qb][r / 8][(r % 8) / 2] = w;
          l4[qb][j % 2] = l;
        }
      }
      // one scheduling region per slot: its asm MFMA (volatile, so in program
      // order), then its VALU and LDS work
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x102, 32, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    return rescale;
  };

  // O *= alpha (per lane and query block) once every issued PV MFMA has
  // completed; the next PV MFMA is two wait states away (the s_nop waits).
  auto rescale_o = [&](const float (&alpha)[2]) __attribute__((always_inline)) {
    wait_o(o);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) o[db][qb][rr] *= alpha[qb];
        asm volatile("" : "+a"(o[db][qb]));  // back into AGPRs now: one accumulator at a time in VGPRs
        __builtin_amdgcn_sched_barrier(0);
      }
    wait_o(o);
  };

  using Y = std::true_type;
  using N = std::false_type;
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // Every wave runs every iteration of the workgroup's tile pairs in full:
  // the waves meet at one barrier per tile pair anyway, so the diagonal
  // blocks a wave's rows do not reach cost no time.  Their scores are
  // masked to -inf (P = 0, row max -inf), as are keys past seq_k.  Only
  // u = 0 (no P(-1) yet: a V^T buffer may hold another tile's data, and 0 x
  // a NaN there would not be 0) and the drain u = 2 n_kt (no S(u+1), no
  // softmax) leave work out.
  u32x4 vnext[NDB];  // V^T fragments of the next iteration's first 16 keys
  auto step = [&](auto par_tag, auto ds, auto dpv, auto dsm, int u, int q0, int ks_slot, int hs, int vs_slot, int hv,
                  int vs_next, int hv_next, auto&& dma) __attribute__((always_inline)) {
    float alpha[2];
    if (iteration(par_tag, ds, dpv, dsm, u, q0, ks_slot, hs, vs_slot, hv, vs_next, hv_next, vnext, alpha, dma))
      rescale_o(alpha);
  };
  auto no_dma = [](int) {};

  // ---- the persistent loop --------------------------------------------------------------
  int r = 0;
  int rank = sched_rank(p, mach, 0);
  if (rank >= p.q_tiles) return;
  Tile cur = make_tile(rank);
  int kbase = 0, vbase = 0;  // ring slots of the tile's K_0 and V_0
  // cold start: K_0, K_1, V_0 and this wave's Q rows
  k_tile_dma(cur, 0, 0);
  k_tile_dma(cur, 1, 1);
  v_tile_dma(cur, 0, 0);
  q_dma(cur);
  wait_vmcnt<0>();
  lds_barrier();
  load_q();

  for (;;) {
    const int nrank = sched_rank(p, mach, r + 1);
    const bool has_next = nrank < p.q_tiles;
    const Tile nxt = make_tile(has_next ? nrank : rank);  // wave-uniform (SGPRs)
    const int n_kt = cur.n_kt;
    const int q0 = cur.qt * K16_BM + 64 * wave;  // this wave's first row

    {
      const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) PvMfma<T>::zero(o[db][qb], z);
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      m_run[qb] = 0.f;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) seed[qb][rr] = 0.f;
      fresh[qb] = true;
#pragma unroll
      for (int k = 0; k < 2; ++k) l4[qb][k] = 0.f;
    }

    // S(0) from K_0 (in LDS since the previous tile pair's barrier)
    {
#pragma unroll
      for (int j = 0; j < NKS; ++j) {
        const u32x4 kf = k_frag(kbase, 0, j);
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          if (j == 0) SMfma<T>::first(s0[qb], kf, qf[qb][j], seed[qb]);
          else SMfma<T>::acc(s0[qb], kf, qf[qb][j]);
        }
      }
      wait_s(s0);  // read by VALU code next (iteration 0 issues no MFMA before its row max)
    }

    // Tile pair t: ring slots K_t, K_{t+1}, K_{t+2} (loaded now) and V_{t-1},
    // V_t, V_{t+1} (loaded now); the loads of the stream run on into the next
    // query tile.  u = 2t: S(2t+1) from K_t rows 32.., PV(2t-1) from V_{t-1}
    // keys 32..; u = 2t+1: S(2t+2) from K_{t+1} rows 0.., PV(2t) from V_t
    // keys 0.. (S(2 n_kt) of the last pair reads a buffer it never uses).
    // Pair 0 is peeled off the loop (its u = 0 runs no PV): a branch between
    // the two variants inside the loop makes the register allocator keep O
    // in two AGPR sets and copy all 128 registers between them.
    int kt0 = kbase, vtm = vbase == 0 ? 2 : vbase - 1;
    // The loads of tile pair t: K_{t+2} into ring slot kt2 and V_{t+1} into
    // vt1, from this query tile or the next one (a missing tile is a
    // resource of zero bytes: its loads fetch nothing).  Eight 1 KiB loads
    // per wave, jobs 0-7 of the pair's first iteration: one per slot in
    // slots 0-7, whose VALU share (the row max) is the lightest (measured:
    // the same loads among the exp2 slots cost about 3% more kernel time).
    auto pair_dma = [&](int t, int kt2, int vt1) __attribute__((always_inline)) {
      const bool kc = t + 2 < n_kt, vc = t + 1 < n_kt;
      const Tile& ktl = kc ? cur : nxt;
      const Tile& vtl = vc ? cur : nxt;
      const int kj = kc ? t + 2 : t + 2 - n_kt, vj = vc ? t + 1 : 0;
      const int krows = (kc || has_next) ? min(max(ktl.k_rows - kj * W_KT, 0), W_KT) : 0;
      const i32x4 rk = uniform_rsrc(ktl.kg + (int64_t)kj * W_KT * k_ss2, (uint32_t)krows * k_ss2);
      const i32x4 rv = uniform_rsrc(vtl.vg + (int64_t)vj * W_KT * 2,
                                    (vc || has_next) ? (uint32_t)(W_D * p.sk_pad * 2 - vj * W_KT * 2) : 0u);
      const uint32_t lk = lds_k + kt2 * W_KTILE + wave * 1024, lv = lds_v + vt1 * W_VTILE + wave * 1024;
      return [=](int i) __attribute__((always_inline)) {
        if (i < 4) lds_dma16(rk, k_dma_lane + (uint32_t)(16 * i) * k_ss2, lk + i * 4096);
        if (i >= 4 && i < 8) lds_dma16(rv, v_dma_lane + (uint32_t)(32 * (i - 4)) * vt_row2, lv + (i - 4) * 4096);
      };
    };
    {
      const int kt1 = kt0 == 2 ? 0 : kt0 + 1, kt2 = kt1 == 2 ? 0 : kt1 + 1;
      const int vt0 = vtm == 2 ? 0 : vtm + 1, vt1 = vt0 == 2 ? 0 : vt0 + 1;
      step(P0{}, Y{}, N{}, Y{}, 0, q0, kt0, 1, vtm, 1, vt0, 0, pair_dma(0, kt2, vt1));
      step(P1{}, Y{}, Y{}, Y{}, 1, q0, kt1, 0, vt0, 0, vt0, 1, q_dma_job(nxt, has_next));
      // the 16 Q loads just issued may stay in flight until the end of tile
      // pair 1 (loads complete in issue order, so the K / V^T loads of this
      // pair, issued before them, have landed)
      wait_vmcnt<16>();
      lds_barrier();
      kt0 = kt1;
      vtm = vt0;
    }
    for (int t = 1; t < n_kt; ++t) {
      const int kt1 = kt0 == 2 ? 0 : kt0 + 1, kt2 = kt1 == 2 ? 0 : kt1 + 1;
      const int vt0 = vtm == 2 ? 0 : vtm + 1, vt1 = vt0 == 2 ? 0 : vt0 + 1;
      step(P0{}, Y{}, Y{}, Y{}, 2 * t, q0, kt0, 1, vtm, 1, vt0, 0, pair_dma(t, kt2, vt1));
      step(P1{}, Y{}, Y{}, Y{}, 2 * t + 1, q0, kt1, 0, vt0, 0, vt0, 1, no_dma);
      wait_vmcnt<0>();
      lds_barrier();
      kt0 = kt1;
      vtm = vt0;
    }
    // u = 2 n_kt: PV(2 n_kt - 1) from V_{n_kt-1} keys 32..
    step(P0{}, N{}, Y{}, N{}, 2 * n_kt, q0, kt0, 1, vtm, 1, vtm, 1, no_dma);

    // The next tile's Q rows into registers first: this wave's 64 staging
    // rows then take its output tile.
    if (has_next) load_q();

    // ---- output: O^T / l, rounded to T, through LDS ------------------------------
    // O^T lane (lq, h) of o[db][qb] holds row 32 qb + lq, d = 32 db + 8 rq + 4 h + 0..3:
    // eight bytes of 32 different rows per register group.  Written to the
    // staging rows (chunk c of row r at slot c ^ lds_swz(r)) and read back
    // row-contiguous, the tile leaves in 16 stores of four whole rows each.
    {
      float inv[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) inv[qb] = 1.f / sum_xor32(l4[qb][0] + l4[qb][1]);
      wait_o(o);
      const int ln = fresh_lane();
      const int lq = ln & 31, h = ln >> 5;
      char* stage = smem + 3 * W_KTILE + 3 * W_VTILE + 64 * wave * 256;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int rq = 0; rq < 4; ++rq) {
            const float x0[2] = {o[db][qb][4 * rq + 0] * inv[qb], o[db][qb][4 * rq + 1] * inv[qb]};
            const float x1[2] = {o[db][qb][4 * rq + 2] * inv[qb], o[db][qb][4 * rq + 3] * inv[qb]};
            const int r = 32 * qb + lq, c = 4 * db + rq;
            *(u32x2*)(stage + r * 256 + ((c ^ lds_swz<W_D>(r)) << 4) + h * 8) = u32x2{pack2<T>(x0), pack2<T>(x1)};
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      // this wave's 64 output rows through one resource that ends at row
      // seq_q (stores past it are dropped)
      const char* ob = (const char*)((const Bits*)p.o + cur.b * p.o_sb + cur.hq * p.o_sh + (int64_t)q0 * p.o_ss);
      const uint32_t o_ss2 = (uint32_t)p.o_ss * 2u;
      const uint64_t oa = (uint64_t)(uintptr_t)ob;
      char* obase = (char*)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(oa >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)oa));
      const int o_bytes = __builtin_amdgcn_readfirstlane((int)((uint32_t)min(max(p.seq_q - q0, 0), 64) * o_ss2));
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(obase, (short)0, o_bytes, kBufRsrcWord3);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 4 * i + ln / 16, sl = ln % 16;
        const u32x4 v = *(const u32x4*)(stage + r * 256 + sl * 16);
        const uint32_t voff = (uint32_t)r * o_ss2 + (uint32_t)((sl ^ lds_swz<W_D>(r)) * 16);
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, (int)voff, 0, 0);
      }
    }
    if (!has_next) break;
    kbase = (kbase + n_kt) % 3;
    vbase = (vbase + n_kt) % 3;
    cur = nxt;
    rank = nrank;
    ++r;
  }
  wait_vmcnt<0>();
}

}  // namespace

namespace tlp {

int launch_flash_w64(FlashParams& p, int dtype, bool causal, hipStream_t st) {
  const dim3 grid((unsigned)(p.q_machines * p.n_queues));
  if (dtype == TL_DTYPE_BF16) {
    if (causal)
      hipLaunchKernelGGL((flash_fwd_w64<BF16, true>), grid, dim3(W_THREADS), 0, st, p);
    else
      hipLaunchKernelGGL((flash_fwd_w64<BF16, false>), grid, dim3(W_THREADS), 0, st, p);
  } else {
    if (causal)
      hipLaunchKernelGGL((flash_fwd_w64<F16, true>), grid, dim3(W_THREADS), 0, st, p);
    else
      hipLaunchKernelGGL((flash_fwd_w64<F16, false>), grid, dim3(W_THREADS), 0, st, p);
  }
  return tl_launch_status();
}

}  // namespace tlp
