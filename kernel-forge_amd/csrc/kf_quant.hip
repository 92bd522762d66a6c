// On-device INT4 quantize + pack: the format producer of kernelforge/quantize.py:61-105,
// bit-exact with it (and with the oracle that restates it).
//
// Per group of G consecutive k of one row:
//   absmax = max |w|                                   (w converted to fp32 exactly)
//   scale  = fp16_rne(max(fl32(absmax / 7), 2^-14)),   1 for an all-zero group
//   q      = clamp(rint(fl32(w / fp32(scale))), -8, 7) (ties to even)
//   u      = q + 8 packed 8 per int32, nibble position p holding k offset (0,2,4,6,1,3,5,7)[p]
// The results are those of IEEE fp32 divisions (hipcc's default correctly rounded division),
// the scalar division by 7 included: the reference quantizes on the CPU, where torch divides
// by the scalar 7.0 (its GPU kernels would multiply by a rounded 1/7 instead).  The division by
// the scale goes through a reciprocal wherever that provably gives the same integer
// (pack_word).
//
// One thread per packed word (8 consecutive k): it loads its 8 values with vector loads
// (16 or 32 bytes), the G/8 threads of a group combine their maxima with DPP (a group never
// straddles a wavefront: G/8 divides 64 and every row holds whole groups), each thread writes
// its word and the group's first thread writes the scale.  HBM-bound once the arithmetic per
// value is a handful of instructions: 4 (fp32) or 2 (fp16/bf16) bytes read and 0.5 + 2/G bytes
// written per weight.
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

constexpr int kQuantThreads = 256;

// Max over aligned runs of L lanes (L = 8 or 16), returned to every lane of the run: DPP quad
// swaps, then the 8- and 16-lane mirrors.  The inputs are >= 0, and non-negative floats order
// as their bit patterns do, so the maxima are taken on integers (one v_max_u32 with DPP each).
template <int L>
__device__ __forceinline__ float run_max(float mf) {
  static_assert(L == 8 || L == 16, "a group is 8 or 16 words");
  uint32_t m = __float_as_uint(mf);
  m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0xB1, 0xF, 0xF, true));   // quad_perm 1,0,3,2
  m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x4E, 0xF, 0xF, true));   // quad_perm 2,3,0,1
  m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x141, 0xF, 0xF, true));  // row_half_mirror
  if constexpr (L == 16) m = max(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x140, 0xF, 0xF, true));  // row_mirror
  return __uint_as_float(m);
}

__device__ __forceinline__ float absmax8(const float (&v)[8]) {
  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
  return m;
}

// fp16 scale of a group with absmax m: fp16_rne(max(fl32(m / 7), 2^-14)), 1 for m == 0.
__device__ __forceinline__ half_t group_scale(float m) {
  half_t s16 = (half_t)fmaxf(m / 7.0f, 6.103515625e-05f);  // 2^-14, the smallest normal fp16
  if (m == 0.0f) s16 = (half_t)1.0f;
  return s16;
}

// The packed word of 8 values with scale s: nibble (k & 1) * 4 + k / 2 holds
// clamp(rint(fl32(v[k] / s)), -8, 7) + 8.
//
// The division only matters near a rounding boundary.  A group's values satisfy
// |v / s| <= 7 / (1 - 2^-11) < 8 (s is absmax / 7 rounded to fp16, or larger).  With
// r = rcp(s) (v_rcp_f32, within 1 ulp) the product P = v * r is within 2^-23 * 8 = 2^-20 of
// v / s, y = fl32(P) within 2^-21 of P, and fl32(v / s) within 2^-21 of v / s.  q = rint(y) is
// the reference's integer whenever |P - q| < 1/2 - 2^-17: then
// |fl32(v / s) - q| < 1/2 - 2^-17 + 2^-21 + 2^-21 + 2^-20 + 2^-21 < 1/2, so fl32(v / s) rounds
// to q whatever the tie rule.  The test holds for |P - q| computed rounded or fused (the error
// of that one rounding is far below the margin), and the margin also covers an rcp error of a
// few ulps.  A lane with any value past the test (about 2^-16 of values) redoes its word with
// the divisions.  s = inf (an overflowed scale) gives r = 0 and q = 0, as the division does.
__device__ __forceinline__ uint32_t pack_word(const float (&v)[8], float s) {
  const float r = __builtin_amdgcn_rcpf(s);
  float q[8];
  bool near = false;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float y = v[k] * r;
    q[k] = __builtin_rintf(y);
    near |= fabsf(y - q[k]) >= 0.5f - 0x1p-17f;
  }
  if (near) {
#pragma unroll
    for (int k = 0; k < 8; ++k) q[k] = __builtin_rintf(v[k] / s);
  }
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k)  // the clamp on integers (v_cvt_i32_f32 saturates)
    word |= (uint32_t)(min(max((int)q[k], -8), 7) + 8) << (4 * ((k & 1) * 4 + (k >> 1)));
  return word;
}

// One thread per word; dead threads (past the end) load the last word and store nothing.  The
// scale of word i is entry i / GW: every row holds whole groups, so the row-major scale index
// row * (K / G) + column / G equals the word index over GW.
template <int DT, int GW>  // GW = G / 8 threads per group
__global__ __launch_bounds__(kQuantThreads) void quantize_kernel(const void* __restrict__ w,
                                                                  uint32_t* __restrict__ packed,
                                                                  half_t* __restrict__ scales, long total_words) {
  const long t = (long)blockIdx.x * kQuantThreads + threadIdx.x;
  const bool live = t < total_words;
  const long i = live ? t : total_words - 1;
  float v[8];
  if constexpr (DT == kQuantF32) {
    // Two 16-byte loads per lane, 32 bytes apart between lanes: measured faster than a layout in
    // which each load instruction reads whole lines (two lanes per word), whose pairs then
    // exchange halves.
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(w) + i * 8);
    const u32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = bit_cast<float>(a[j]);
      v[4 + j] = bit_cast<float>(b[j]);
    }
  } else {
    // Plain loads: the non-temporal form measured slower for 2-byte weights.
    const u32x4 a = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + i * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (DT == kQuantF16) {
        v[2 * j] = (float)bit_cast<half_t>((uint16_t)(a[j] & 0xFFFFu));
        v[2 * j + 1] = (float)bit_cast<half_t>((uint16_t)(a[j] >> 16));
      } else {  // bf16: the top half of an fp32
        v[2 * j] = bit_cast<float>(a[j] << 16);
        v[2 * j + 1] = bit_cast<float>(a[j] & 0xFFFF0000u);
      }
    }
  }
  const half_t s16 = group_scale(run_max<GW>(absmax8(v)));
  const uint32_t word = pack_word(v, (float)s16);
  if (live) {
    packed[i] = word;
    if ((i & (GW - 1)) == 0) scales[i / GW] = s16;
  }
}

typedef void (*QuantFn)(const void*, uint32_t*, half_t*, long);

template <int DT>
QuantFn quant_fn(int group_size) {
  return group_size == 128 ? quantize_kernel<DT, 16> : quantize_kernel<DT, 8>;
}

}  // namespace

hipError_t quantize_launch(const void* w, int dtype, void* packed, void* scales, int N, int K, int group_size,
                           hipStream_t stream) {
  const long total = (long)N * (K / 8);
  const QuantFn fn = dtype == kQuantF32 ? quant_fn<kQuantF32>(group_size)
                                        : (dtype == kQuantF16 ? quant_fn<kQuantF16>(group_size)
                                                              : quant_fn<kQuantBF16>(group_size));
  const long blocks = (total + kQuantThreads - 1) / kQuantThreads;
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(kQuantThreads), 0, stream, w, static_cast<uint32_t*>(packed),
                     static_cast<half_t*>(scales), total);
  return hipGetLastError();
}

}  // namespace kf
