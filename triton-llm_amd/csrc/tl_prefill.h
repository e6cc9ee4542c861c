// Internal header of the prefill kernels (tl_prefill.hip, tl_prefill_w64.hip):
// the launch parameters, the persistent tile schedule and the LDS swizzles
// they share.  Not part of the C ABI.
#pragma once

#include "tl_common.h"

namespace tlp {

constexpr int kMaxEntries = 64;  // list entries of a key-split schedule

struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  const void* vt;  // key-major V^T copy (16-bit path), see vt_pack_kernel
  void* o;
  int batch, n_head, n_kv, group, seq_q, seq_k, n_qt, sk_pad;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  float scale_log2;
  // Static tile schedule of the persistent 16-bit kernel (see flash_fwd_16).
  int n_queues;    // 8 (one tile list per XCD) or 1
  int q_split;     // parts per query head: part j holds its tiles with qt % q_split == j
  int q_parts;     // parts per list
  int q_tiles;     // tiles per list: q_parts * n_qt / q_split
  int q_machines;  // workgroups per list
  int q_triple;    // first three rounds use the balanced-triple order
  // Key split (causal flash_fwd_16 only; n_entries 0: none).  A list is a
  // sequence of n_entries entries of q_parts items each: entry e holds level
  // lvl = e_code[e] & 63's tiles whole (part e_code[e] >> 6 = 0) or the lower
  // (1) or upper (2) part of their key tiles.  The split levels are the
  // costliest, 0 .. n_split_levels - 1.  The parts of one tile merge through
  // split_ws (see flash_fwd_16's tile switch).  The kernel reads e_code from
  // the kernel-argument segment (entry_code): indexing the by-value argument
  // would copy the array into registers.
  int n_entries;
  int n_split_levels;
  int n_split_tiles;         // n_queues * n_split_levels * q_parts
  uint32_t split_part_bytes; // partial region bytes (2 slots per split tile)
  uint64_t split_token;      // this call's arrival tag (never 0)
  void* split_ws;            // arrival words (8 per split tile), then the partial slots
  uint8_t e_code[kMaxEntries];
};

// 16-bit kernels: query rows per tile (both flash_fwd_16 and flash_fwd_w64)
// and the lazy-rescale threshold of the online softmax.
constexpr int K16_BM = 256;       // query rows per tile
constexpr int K16_BN = 128;       // keys per K / V^T tile
constexpr int K16_THREADS = 512;  // 8 waves
constexpr float kRescaleLog2 = 8.0f;

// Slot swizzle of LDS rows of D 16-bit elements: 16 consecutive rows read
// the same 16-byte chunk of their row in one operand load, so the chunk is
// XORed with bits of the row index that spread those rows over all banks.
template <int D>
__device__ __forceinline__ int lds_swz(int r) {
  if constexpr (D == 128) return 4 * (r & 3) + ((r >> 2) & 3);
  else return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}

__device__ __forceinline__ float max_xor32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_xor32(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The lane index, read afresh at each use (an opaque read that cannot be
// hoisted), so that lane-derived offsets are recomputed where they are used
// instead of occupying registers across the tile loop.
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Tile i of list `queue` of the persistent schedule.  The query heads of the
// call, (batch, kv head) unit by unit, are cut into q_split parts each (part
// j: the head's query tiles with qt % q_split == j), and list x holds parts
// [x q_parts, (x + 1) q_parts): a few consecutive heads, hence few (batch,
// kv head) units, whose K / V then stay in one XCD's L2.  A list is ordered
// by qt descending (causal cost): the lvl-th costliest tile of every part,
// parts in order, then the next level.
__host__ __device__ inline void decode_tile(const FlashParams& p, int queue, int i, int& b, int& hq, int& qt) {
  const int lvl = i / p.q_parts;
  const int part = queue * p.q_parts + (i - lvl * p.q_parts);
  const int hs = part / p.q_split;  // query head (b, hkv, g) as (b * n_kv + hkv) * group + g
  const int j = part - hs * p.q_split;
  const int u = hs / p.group;
  const int hkv = u % p.n_kv;
  b = u / p.n_kv;
  hq = hkv * p.group + (hs - u * p.group);
  qt = j + p.q_split * (p.n_qt / p.q_split - 1 - lvl);
}

// Item i of list `queue` of a key-split schedule (p.n_entries > 0) whose
// entry e = i / q_parts has code `code`: the tile as decode_tile gives it
// for the entry's level, its key part (0 whole, 1 lower, 2 upper) and, for a
// part, the tile's split index (< n_split_tiles).
__host__ __device__ inline void decode_item(const FlashParams& p, int queue, int i, int code, int& b, int& hq,
                                            int& qt, int& kpart, int& sidx) {
  const int e = i / p.q_parts;
  const int within = i - e * p.q_parts;
  const int lvl = code & 63;
  decode_tile(p, queue, lvl * p.q_parts + within, b, hq, qt);
  kpart = code >> 6;
  sidx = (queue * p.n_split_levels + lvl) * p.q_parts + within;
}

// Rank (position in its list) of workgroup j's r-th tile; >= q_tiles: none.
__host__ __device__ inline int sched_rank(const FlashParams& p, int j, int r) {
  const int m = p.q_machines;
  if (p.q_triple && r < 3) {
    const int hm = m / 2;
    if (r == 0) return j;
    if (r == 1) return m + (j < hm ? m - 1 - 2 * j : 2 * m - 2 - 2 * j);
    return 2 * m + (j < hm ? hm + j : j - hm);
  }
  const int rr = p.q_triple ? r - 3 : r;
  return r * m + ((rr & 1) ? m - 1 - j : j);
}

// d_k 128 16-bit prefill with 64 query rows per wave (tl_prefill_w64.hip);
// expects p.vt to hold the vt_pack copy of V and the schedule fields set.
int launch_flash_w64(FlashParams& p, int dtype, bool causal, hipStream_t st);

}  // namespace tlp
