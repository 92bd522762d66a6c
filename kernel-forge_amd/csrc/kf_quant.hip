// On-device INT4 quantize + pack: the format producer of kernelforge/quantize.py:61-105,
// bit-exact with it (and with the oracle that restates it).
//
// Per group of G consecutive k of one row:
//   absmax = max |w|                                   (w converted to fp32 exactly)
//   scale  = fp16_rne(max(fl32(absmax / 7), 2^-14)),   1 for an all-zero group
//   q      = clamp(rint(fl32(w / fp32(scale))), -8, 7) (ties to even)
//   u      = q + 8 packed 8 per int32, nibble position p holding k offset (0,2,4,6,1,3,5,7)[p]
// Divisions are IEEE fp32 divisions (hipcc's default correctly rounded division), the scalar
// division by 7 included: the reference quantizes on the CPU, where torch divides by the
// scalar 7.0 (its GPU kernels would multiply by a rounded 1/7 instead).
//
// One thread per packed word (8 consecutive k): it loads its 8 values with vector loads
// (16 or 32 bytes), the G/8 threads of a group combine their maxima with lane shuffles
// (a group never straddles a wavefront: G/8 divides 64 and every row holds whole groups),
// each thread writes its word and the group's first thread writes the scale.  HBM-bound:
// 4 (fp32) or 2 (fp16/bf16) bytes read and 0.5 + 2/G bytes written per weight.
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

constexpr int kQuantThreads = 256;

template <int DT>
__device__ __forceinline__ void load8(const void* base, size_t idx, float (&v)[8]) {
  if constexpr (DT == kQuantF32) {
    const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + idx);
    const u32x4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = bit_cast<float>(a[j]);
      v[4 + j] = bit_cast<float>(b[j]);
    }
  } else {
    const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(base) + idx));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = a[j] & 0xFFFFu, hi = a[j] >> 16;
      if constexpr (DT == kQuantF16) {
        v[2 * j] = (float)bit_cast<half_t>((uint16_t)lo);
        v[2 * j + 1] = (float)bit_cast<half_t>((uint16_t)hi);
      } else {  // bf16: the top half of an fp32
        v[2 * j] = bit_cast<float>(lo << 16);
        v[2 * j + 1] = bit_cast<float>(hi << 16);
      }
    }
  }
}

template <int DT, int GW>  // GW = G / 8 threads per group
__global__ __launch_bounds__(kQuantThreads) void quantize_kernel(const void* __restrict__ w,
                                                                  uint32_t* __restrict__ packed,
                                                                  half_t* __restrict__ scales, long total_words,
                                                                  int words_per_row) {
  const long t = (long)blockIdx.x * kQuantThreads + threadIdx.x;
  // Threads past the end take the last word (whole groups only, since every row holds
  // whole groups and total_words is a multiple of GW) and store nothing.
  const bool live = t < total_words;
  const long i = live ? t : total_words - 1;
  float v[8];
  load8<DT>(w, (size_t)i * 8, v);

  float m = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
#pragma unroll
  for (int off = 1; off < GW; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 64));

  half_t s16 = (half_t)fmaxf(m / 7.0f, 6.103515625e-05f);  // 2^-14, the smallest normal fp16
  if (m == 0.0f) s16 = (half_t)1.0f;
  const float s = (float)s16;

  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float q = fminf(fmaxf(__builtin_rintf(v[k] / s), -8.0f), 7.0f);
    const uint32_t u = (uint32_t)((int)q + 8);
    word |= u << (4 * ((k & 1) * 4 + (k >> 1)));  // k offset k sits at nibble (k & 1) * 4 + k / 2
  }
  if (live) {
    packed[i] = word;
    const long row = i / words_per_row;
    const int wd = (int)(i - row * words_per_row);
    if (wd % GW == 0) scales[row * (words_per_row / GW) + wd / GW] = s16;
  }
}

typedef void (*QuantFn)(const void*, uint32_t*, half_t*, long, int);

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
                     static_cast<half_t*>(scales), total, K / 8);
  return hipGetLastError();
}

}  // namespace kf
