// Auxiliary kernels: the fp16 dequantization exported for bit-exactness checks,
// the streaming HBM ceiling kernels the roofline fractions are quoted against, and
// the greedy step of a graph-captured decode loop (argmax + position bookkeeping).
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

// One thread per packed word: the 8 weights of word i become fp16_rne(q * s),
// using the same dequant8 the GEMM uses to fill its LDS tiles.
__global__ __launch_bounds__(256) void dequant_fp16_kernel(const uint32_t* __restrict__ packed,
                                                            const half_t* __restrict__ scales,
                                                            half_t* __restrict__ out, size_t total_words,
                                                            int words_per_row, int groups_per_row,
                                                            int log2_group) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total_words; i += (size_t)gridDim.x * 256) {
    const size_t n = i / words_per_row;
    const int k0 = (int)(i - n * words_per_row) * 8;
    const half_t s = scales[n * groups_per_row + (k0 >> log2_group)];
    const half2_t s2 = {s, s};
    *reinterpret_cast<half8_t*>(out + 8 * i) = dequant8(packed[i], s2);
  }
}

__global__ __launch_bounds__(256) void bw_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                       size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Folds everything it reads into one word per thread; the store is taken only
// when that word equals an unlikely constant, so the loads cannot be removed
// but almost nothing is written.
__global__ __launch_bounds__(256) void bw_read_kernel(const u32x4* __restrict__ src, uint32_t* __restrict__ sink,
                                                       size_t n) {
  uint32_t acc = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// bw_read_kernel plus the stores of a decode GEMV: lanes 31 and 63 of every wavefront store one
// fp16 each (2 bytes, 4 per wavefront, wavefronts' values adjacent), unconditionally, so the
// kernel ends with the small scattered stores the GEMV's outputs make.
__global__ __launch_bounds__(256) void bw_read_store_kernel(const u32x4* __restrict__ src, uint16_t* __restrict__ out,
                                                             size_t n) {
  uint32_t acc = 0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if ((threadIdx.x & 31) == 31) out[((size_t)blockIdx.x * 256 + threadIdx.x) >> 5] = (uint16_t)acc;
}

__global__ __launch_bounds__(256) void bw_write_kernel(u32x4* __restrict__ dst, size_t n) {
  const u32x4 v = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    __builtin_nontemporal_store(v, dst + i);
}

// Greedy decode step.  One workgroup: every thread keeps the best (value, index) of the
// elements it reads, then the wavefront and the workgroup combine them.  "Best" is torch's
// argmax order: NaN above every number, larger values above smaller ones, and among equals
// (NaN included, +0 and -0 equal) the smaller index.  Thread 0 then advances the position and
// records the token: p = pos + 1; pos = p; token = idx; history[p] = idx and mask[p] = 0 when
// p < max_seq (a position past the cache records nothing: every write stays in bounds).
constexpr int kArgmaxThreads = 1024;

// (v, i) replaced by (w, j) when (w, j) comes first in that order.
__device__ __forceinline__ void take_better(float& v, int& i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  const bool take = vn != wn ? wn : ((!vn && v != w) ? w > v : j < i);
  v = take ? w : v;
  i = take ? j : i;
}

__global__ __launch_bounds__(kArgmaxThreads) void decode_argmax_kernel(const half_t* __restrict__ logits, int n,
                                                                      int64_t* token, int64_t* pos, int64_t* history,
                                                                      int max_seq, half_t* mask, int vec) {
  const int tid = threadIdx.x;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  if (vec) {  // 16-byte aligned logits: 8 values per load, the tail one by one
    const int n8 = n >> 3;
    for (int v = tid; v < n8; v += kArgmaxThreads) {
      const u32x4 h = *reinterpret_cast<const u32x4*>(logits + 8 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const half2_t pr = bit_cast<half2_t>(h[e]);
        take_better(bv, bi, (float)pr[0], 8 * v + 2 * e);
        take_better(bv, bi, (float)pr[1], 8 * v + 2 * e + 1);
      }
    }
    for (int i = 8 * n8 + tid; i < n; i += kArgmaxThreads) take_better(bv, bi, (float)logits[i], i);
  } else {
    for (int i = tid; i < n; i += kArgmaxThreads) take_better(bv, bi, (float)logits[i], i);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    take_better(bv, bi, ov, oi);
  }
  __shared__ float wave_v[kArgmaxThreads / 64];
  __shared__ int wave_i[kArgmaxThreads / 64];
  if ((tid & 63) == 0) {
    wave_v[tid >> 6] = bv;
    wave_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float rv = wave_v[0];
    int ri = wave_i[0];
    for (int w = 1; w < kArgmaxThreads / 64; ++w) take_better(rv, ri, wave_v[w], wave_i[w]);
    const int64_t idx = ri;
    const int64_t p = *pos + 1;
    *pos = p;
    *token = idx;
    if (p >= 0 && p < max_seq) {
      history[p] = idx;
      if (mask) mask[p] = (half_t)0.0f;
    }
  }
}

}  // namespace

hipError_t decode_argmax_launch(const void* logits, int n, void* token, void* pos, void* history, int max_seq,
                                void* mask, hipStream_t stream) {
  const int vec = ((uintptr_t)logits & 15) == 0;
  hipLaunchKernelGGL(decode_argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, stream,
                     static_cast<const half_t*>(logits), n, static_cast<int64_t*>(token), static_cast<int64_t*>(pos),
                     static_cast<int64_t*>(history), max_seq, static_cast<half_t*>(mask), vec);
  return hipGetLastError();
}

hipError_t dequant_fp16_launch(const void* packed, const void* scales, void* w_hat, int N, int K, int group_size,
                               hipStream_t stream) {
  const size_t total = (size_t)N * (K / 8);
  size_t blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(dequant_fp16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const uint32_t*>(packed), static_cast<const half_t*>(scales),
                     static_cast<half_t*>(w_hat), total, K / 8, K / group_size, group_size == 128 ? 7 : 6);
  return hipGetLastError();
}

hipError_t bw_copy_launch(const void* src, void* dst, size_t bytes, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(bw_copy_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4*>(src),
                     static_cast<u32x4*>(dst), bytes / 16);
  return hipGetLastError();
}

hipError_t bw_read_launch(const void* src, void* sink, size_t bytes, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(bw_read_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4*>(src),
                     static_cast<uint32_t*>(sink), bytes / 16);
  return hipGetLastError();
}

hipError_t bw_read_store_launch(const void* src, void* out, size_t bytes, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(bw_read_store_kernel, dim3(grid), dim3(256), 0, stream, static_cast<const u32x4*>(src),
                     static_cast<uint16_t*>(out), bytes / 16);
  return hipGetLastError();
}

hipError_t bw_write_launch(void* dst, size_t bytes, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(bw_write_kernel, dim3(grid), dim3(256), 0, stream, static_cast<u32x4*>(dst), bytes / 16);
  return hipGetLastError();
}

}  // namespace kf
