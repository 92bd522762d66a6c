// Device-side building blocks shared by the gfx950 INT4 kernels.
//
// Nibble unpack.  The packing convention (reference kernelforge/quantize.py:12-24)
// stores k offsets (0,2,4,6,1,3,5,7) at nibble positions 0..7, so
// (w >> 4i) & 0x000F000F holds u(k 2i) in bits 0-3 and u(k 2i+1) in bits 16-19.
// OR-ing 0x6400 into each 16-bit half forms the fp16 number 1024 + u exactly
// (fp16 spacing is 1 on [1024, 2048)), and one packed fp16 subtraction of
// 1032 = 1024 + 8 yields (q[2i], q[2i+1]) exactly.  On gfx950 this is one
// v_and_or_b32 and one v_pk_add_f16 per pair (plus a shift for i > 0).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kf {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename To, typename From>
__device__ __forceinline__ To bit_cast(const From& v) {
  static_assert(sizeof(To) == sizeof(From), "bit_cast size mismatch");
  return __builtin_bit_cast(To, v);
}

// q pair (k 2i, k 2i+1) of a packed word as exact fp16 integers.  Nibble pair I sits at bits
// 4I (low half) and 16 + 4I (high half).  A nibble u at mantissa bits 0-3 under exponent 2^10
// (0x6400) reads 1024 + u; at mantissa bits 4-7 under exponent 2^6 (0x5400) it reads
// 64 + 16u / 16 = 64 + u.  So pairs 0 and 1 come from the word itself and pairs 2 and 3 from the
// word shifted by 8, one shift per word instead of three; q = u - 8 = v - 1032 or v - 72, exact.
template <int I>
__device__ __forceinline__ half2_t nibble_pair(uint32_t w) {
  const uint32_t src = I >= 2 ? (w >> 8) : w;
  const uint32_t v = (I & 1) ? ((src & 0x00F000F0u) | 0x54005400u) : ((src & 0x000F000Fu) | 0x64006400u);
  const half_t b = (I & 1) ? (half_t)72.0f : (half_t)1032.0f;
  const half2_t bias = {b, b};
  return bit_cast<half2_t>(v) - bias;
}

// All 8 weights of a word as fp16 integers in k order: (k0,k1),(k2,k3),(k4,k5),(k6,k7).
__device__ __forceinline__ void unpack8(uint32_t w, half2_t (&q)[4]) {
  q[0] = nibble_pair<0>(w);
  q[1] = nibble_pair<1>(w);
  q[2] = nibble_pair<2>(w);
  q[3] = nibble_pair<3>(w);
}

// fp16_rne(q * s) for the 8 weights of a word: the dequantized W_hat the
// reference feeds to its tensor cores (dequant_gemm_tc_kernel.cuh:100-112,
// quantize.py:112-113).  q * s is exact before the single rounding because
// |q| <= 8 has at most 4 significant bits.
__device__ __forceinline__ half8_t dequant8(uint32_t w, half2_t s2) {
  half2_t q[4];
  unpack8(w, q);
  const half2_t p0 = q[0] * s2, p1 = q[1] * s2, p2 = q[2] * s2, p3 = q[3] * s2;
  half8_t out = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  return out;
}

// The same unpack with its masks and magic numbers held in registers.  gfx9 VOP3 encodings take
// no literal operand and at most one SGPR, so without this the compiler splits every
// v_and_or_b32 into v_and_b32 + v_or_b32.  With them a word costs 13 VALU ops: one shift, four
// v_and_or_b32, four packed subtracts and four packed scale multiplies (15 when every pair
// needed its own shift).  The constants come from opaque moves, made once per kernel, that the
// compiler cannot fold.
struct UnpackConsts {
  uint32_t mask;      // 0x000F000F, in an SGPR
  uint32_t mask_hi;   // 0x00F000F0, in an SGPR
  uint32_t magic;     // 0x64006400, in a VGPR
  uint32_t magic_hi;  // 0x54005400, in a VGPR
};
__device__ __forceinline__ UnpackConsts unpack_consts() {
  UnpackConsts c;
  asm("s_mov_b32 %0, 0x000f000f" : "=s"(c.mask));
  asm("s_mov_b32 %0, 0x00f000f0" : "=s"(c.mask_hi));
  asm("v_mov_b32 %0, 0x64006400" : "=v"(c.magic));
  asm("v_mov_b32 %0, 0x54005400" : "=v"(c.magic_hi));
  return c;
}

// nibble_pair<I>(w) with one v_and_or_b32 per pair (see above for the two encodings).
template <int I>
__device__ __forceinline__ half2_t nibble_pair(uint32_t w, const UnpackConsts& c) {
  uint32_t v;
  const uint32_t src = I >= 2 ? (w >> 8) : w;
  if constexpr (I & 1)
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(v) : "v"(src), "s"(c.mask_hi), "v"(c.magic_hi));
  else
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(v) : "v"(src), "s"(c.mask), "v"(c.magic));
  const half_t b = (I & 1) ? (half_t)72.0f : (half_t)1032.0f;
  const half2_t bias = {b, b};
  return bit_cast<half2_t>(v) - bias;
}

__device__ __forceinline__ half8_t dequant8(uint32_t w, half2_t s2, const UnpackConsts& c) {
  const half2_t p0 = nibble_pair<0>(w, c) * s2, p1 = nibble_pair<1>(w, c) * s2;
  const half2_t p2 = nibble_pair<2>(w, c) * s2, p3 = nibble_pair<3>(w, c) * s2;
  half8_t out = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  return out;
}

// Sum over each 32-lane half of a wave64 with DPP row ops: lane 31 ends with the total of
// lanes 0-31 and lane 63 with that of lanes 32-63.
//   quad_perm [1,0,3,2] and [2,3,0,1]: every lane holds its quad's sum
//   row_shr:4, row_shr:8: lane 15 of each 16-lane row holds the row sum
//   row_bcast:15 into rows 1 and 3: lanes 31 and 63 hold their half's total
__device__ __forceinline__ float half_sum_lanes31_63(float v) {
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0xB1, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x4E, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x114, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x118, 0xF, 0xF, false);
  v += __builtin_amdgcn_update_dpp(0.0f, v, 0x142, 0xA, 0xF, false);
  return v;
}

// Waits until at most N vector-memory operations of this wavefront are outstanding.  LDS-DMA
// copies (global_load_lds_*) are issued from inline assembly, which the compiler neither tracks
// nor orders against its own waits, so the kernels wait for a copy with a counted wait: N is the
// number of vector-memory instructions the kernel issues after that copy (the GEMV's first-pass
// weight and scale loads; the GEMM's next stage of DMAs).  That count holds only while the
// compiler emits exactly those instructions in between; a different count would let a wavefront
// read LDS before its copy lands.  Built with KF_DMA_WAIT_ALL defined (KF_DMA_WAIT_ALL=1 in the
// environment of kernelforge/build.py), every such wait is vmcnt(0) instead: slower, and
// correct whatever the compiler emits.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
#ifdef KF_DMA_WAIT_ALL
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#else
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#endif
}

__device__ __forceinline__ u32x4 load_u32x4(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Streaming (non-temporal) 16-byte load for data read exactly once.
__device__ __forceinline__ u32x4 load_u32x4_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

}  // namespace kf
