// Shared device/host helpers for the gfx950 attention library.
//
// Element types are tagged by the same integer codes the C ABI uses
// (TL_DTYPE_F32 / TL_DTYPE_F16 / TL_DTYPE_BF16).  All arithmetic that feeds
// softmax or accumulation runs in fp32; 16-bit types are storage formats.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/triton_llm_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource, dword 3 for CDNA (32-bit data format, no swizzle).
constexpr int kBufRsrcWord3 = 0x00020000;

// Storage type tags.  `bits` is the raw 16/32-bit pattern type.
struct F32 {
  using bits = uint32_t;
  static constexpr int code = TL_DTYPE_F32;
  static constexpr int size = 4;
};
struct F16 {
  using bits = uint16_t;
  static constexpr int code = TL_DTYPE_F16;
  static constexpr int size = 2;
  static constexpr uint32_t one_pair = 0x3C003C00u;  // two 1.0 values in one word
};
struct BF16 {
  using bits = uint16_t;
  static constexpr int code = TL_DTYPE_BF16;
  static constexpr int size = 2;
  static constexpr uint32_t one_pair = 0x3F803F80u;  // two 1.0 values in one word
};

// ---- scalar conversions -------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// fp32 -> bf16 with round-to-nearest-even on the bit pattern.  NaN maps to a
// quiet NaN that keeps the sign (0x7FC0 | sign), the convention the host
// oracle uses, so stores of rounded values are bit-exact against it.
__device__ __forceinline__ uint32_t f32_to_bf16_bits_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7FC0u;
  uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return (u + bias) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
  return (float)h;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32, round-to-nearest-even
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

template <typename T>
__device__ __forceinline__ float to_f32(typename T::bits b);
template <>
__device__ __forceinline__ float to_f32<F32>(uint32_t b) { return __uint_as_float(b); }
template <>
__device__ __forceinline__ float to_f32<F16>(uint16_t b) { return f16_bits_to_f32(b); }
template <>
__device__ __forceinline__ float to_f32<BF16>(uint16_t b) { return bf16_bits_to_f32(b); }

template <typename T>
__device__ __forceinline__ typename T::bits from_f32(float f);
template <>
__device__ __forceinline__ uint32_t from_f32<F32>(float f) { return __float_as_uint(f); }
template <>
__device__ __forceinline__ uint16_t from_f32<F16>(float f) { return (uint16_t)f32_to_f16_bits(f); }
template <>
__device__ __forceinline__ uint16_t from_f32<BF16>(float f) { return (uint16_t)f32_to_bf16_bits_rne(f); }

// RoPE of one half-split pair (x_i, x_{i+d/2}) at one position: each product
// and the sum / difference rounded separately in fp32, as NumPy evaluates
// the same expression (hipcc would otherwise contract a*b - c*d into an FMA).
__device__ __forceinline__ void rope_rotate_pair(float xe, float xo, float c, float s, float& oe, float& oo) {
#pragma clang fp contract(off)
  const float a = xe * c, b = xo * s, d = xe * s, e = xo * c;
  oe = a - b;
  oo = d + e;
}

// Unpack a 32-bit word holding two 16-bit values (low half first).
template <typename T>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi);
template <>
__device__ __forceinline__ void unpack2<BF16>(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xFFFF0000u);
}
template <>
__device__ __forceinline__ void unpack2<F16>(uint32_t w, float& lo, float& hi) {
  lo = f16_bits_to_f32(w & 0xFFFFu);
  hi = f16_bits_to_f32(w >> 16);
}

// ---- DPP cross-lane helpers (rows of 16 lanes) --------------------------
// dpp_ctrl encodings (GCN/CDNA DPP): row_ror:n = 0x120 + n.

// Written as update_dpp with old = 0 and bound_ctrl so the compiler can fold
// the move into the consuming VALU op (v_add_f32_dpp); row rotations never
// read an invalid lane, so the result equals a plain DPP move.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the sum.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_mov<0x128>(x);  // row_ror:8
  x += dpp_mov<0x124>(x);  // row_ror:4
  x += dpp_mov<0x122>(x);  // row_ror:2
  x += dpp_mov<0x121>(x);  // row_ror:1
  return x;
}

// Sum over each group of 8 lanes (half a DPP row); every lane of the group
// receives the sum: quad sums by two quad permutations, then the mirrored
// lane of the other quad (row_half_mirror maps lane i to 7 - i).
__device__ __forceinline__ float row8_sum(float x) {
  x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);  // row_half_mirror
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Status returned by launch wrappers: the HIP error of the launch (0 = ok).
static inline int tl_launch_status() { return (int)hipGetLastError(); }

// Resolve the stream argument of an entry point: NULL means the library stream.
hipStream_t tl_resolve_stream(void* stream);

// Fill nbytes at dst with value on stream st by a kernel (capturable in a
// HIP graph as a kernel node).
int tl_fill_bytes(void* dst, unsigned char value, size_t nbytes, hipStream_t st);

// Test-only overrides.  tl_init reads them from the environment on every
// call (so a test re-reads them by calling tl_init again); launches read only
// these fields, never the environment.
//   max_cus        TRITON_LLM_HIP_MAX_CUS: caps the compute units the
//                  persistent and equal-share schedules plan for (0: none),
//                  so small problems take multi-round schedules;
//   decode_shares  TRITON_LLM_HIP_DECODE_SHARES nonzero: small-cache decode
//                  takes the equal-share path instead of pair mode;
//   prefill_w64    TRITON_LLM_HIP_PREFILL_W64 nonzero: 16-bit d_k 128
//                  prefill runs flash_fwd_w64 (64 query rows per wave)
//                  instead of flash_fwd_16, so tests and A/B timing can
//                  run both;
//   prefill_one_list  TRITON_LLM_HIP_PREFILL_ONE_LIST nonzero: flash_fwd_16
//                  deals every tile from one list instead of one per XCD;
//   prefill_no_split  TRITON_LLM_HIP_PREFILL_NO_SPLIT nonzero: flash_fwd_16
//                  splits no tile's key range over two workgroups (and
//                  tl_attention_fwd_workspace_bytes_split asks for no
//                  split region).
struct TlOverrides {
  int max_cus;
  int decode_shares;
  int prefill_w64;
  int prefill_one_list;
  int prefill_no_split;
};
extern TlOverrides tl_overrides;

// Compute units of the current device (cached per device), capped by
// tl_overrides.max_cus when set.
int tl_device_cus();

// ---- matrix-core and LDS helpers shared by the MFMA kernels -------------

// 32x32x16 MFMA (fp32 accumulation) for the 16-bit storage types.
template <typename T>
struct Mfma;

template <>
struct Mfma<BF16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag pack(const float* x) {
    frag r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (__bf16)x[i];
    return r;
  }
};

template <>
struct Mfma<F16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ frag pack(const float* x) {
    frag r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)x[i];
    return r;
  }
};

// Two fp32 values -> one 32-bit word of two 16-bit values (low half first),
// rounded to nearest even.
template <typename T>
__device__ __forceinline__ uint32_t pack2(const float (&x)[2]);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(const float (&x)[2]) {
  const bf16x2 v = {(__bf16)x[0], (__bf16)x[1]};
  return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(const float (&x)[2]) {
  const f16x2 v = {(_Float16)x[0], (_Float16)x[1]};
  return __builtin_bit_cast(uint32_t, v);
}

// Buffer resource over `bytes` bytes at `base` (raw, no stride) as the four
// SGPR words an LDS-DMA takes: reads past the end return zeros with no
// memory access.  Every word is taken from the first lane (callers pass
// wave-uniform values), so the resource lives in SGPRs.
__device__ __forceinline__ i32x4 uniform_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
               __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu)),
               __builtin_amdgcn_readfirstlane((int)bytes), kBufRsrcWord3};
}

// Global -> LDS copy (buffer_load_dwordx4 ... lds, "LDS-DMA"): lane i's 16
// bytes at byte offset voff of the resource land at LDS byte address
// lds_addr + 16 i, with no register round trip.  lds_addr is wave-uniform
// (an SGPR); the instruction takes it from m0.
//
// Inline assembly, not __builtin_amdgcn_raw_ptr_buffer_load_lds: with the
// builtin the compiler waits for every outstanding LDS-DMA (vmcnt(0))
// before each later LDS read it cannot prove disjoint from the DMA target,
// which here includes every ds_read_b64_tr_b16.  That serialises the
// prefetch of the next key tile behind the current tile's operand reads
// (measured: the d_k 64 prefill, config 3, fell from 543 to 342 TFLOP/s).
// So the kernels order the DMAs themselves: each issuing wave waits with
// wait_vmcnt<0>() before the barrier that publishes the tile.  The compiler
// does not count these loads, which only makes its own vmcnt waits wait
// longer (loads return in order), never shorter.  m0 is written here and
// cannot be declared clobbered (it is a reserved register); the library
// build (triton_llm/_build.py) therefore rejects any kernel that issues
// these DMAs and in which compiler-generated code reads or writes m0.
__device__ __forceinline__ void lds_dma16(const i32x4& rsrc, uint32_t voff, uint32_t lds_addr) {
  const uint32_t la = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_addr);  // wave-uniform by contract
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(la), "v"(voff), "s"(rsrc)
               : "memory");
}

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier that orders LDS only (global prefetches stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

