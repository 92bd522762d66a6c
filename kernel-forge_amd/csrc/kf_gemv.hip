// Fused INT4 dequant GEMV for decode (M in [1, 8]) on gfx950.
//
// Computes y[m, n] = fp16( sum_c s[n, c/(G/32)] * sum_{k in chunk c} x[m, k] * q[n, k] )
// with fp32 accumulation, the arithmetic of the reference's
// dequant_gemv_kernel<M> (csrc/gemm/dequant_gemv_kernel.cuh:38-109): the scale
// is applied once per 32-k chunk (32 divides G), so W_hat is never rounded.
//
// Mapping (bandwidth-first, no LDS, no MFMA):
//   * A "chunk" is 32 consecutive k of one row: 16 B of packed words (one
//     dwordx4), 64 B of x and exactly one scale.
//   * Each wavefront owns R consecutive output rows.  Lane l handles chunks
//     l, l+64, l+128, ... of every one of its rows, so one wavefront-wide
//     dwordx4 instruction streams 1 KiB of a row contiguously.
//   * U chunk iterations (U*R dwordx4 weight loads per lane) are issued before
//     any arithmetic so enough bytes are in flight to cover HBM latency.
//     Out-of-range chunks are clamped to the row's last chunk (always in
//     bounds) and masked out of the sum.
//   * The q unpack is done once per (chunk, row) and reused for all M rows
//     of x; x is re-read per m from L1/L2 (a few KiB shared by all waves).
//   * Each lane accumulates M*R fp32 partials; a DPP wave reduction puts the
//     totals in lane 63, which rounds to fp16 (RNE) and stores them.
//   * Rows past N are clamped to row N-1 for loading and never stored.
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

template <int M, int R, int U>
__global__ __launch_bounds__(256) void gemv_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed,
                                                   const half_t* __restrict__ scales, half_t* __restrict__ y,
                                                   int N, int K, int scale_shift) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int row0 = (blockIdx.x * waves + wave) * R;
  if (row0 >= N) return;

  const int chunks = K >> 5;               // 32-k chunks per row
  const int words = K >> 3;                // packed words per row
  const int groups = chunks >> scale_shift;  // scales per row

  const uint32_t* prow[R];
  const half_t* srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(row0 + r, N - 1);
    prow[r] = packed + (size_t)n * words;
    srow[r] = scales + (size_t)n * groups;
  }

  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int c0 = lane; c0 < chunks; c0 += 64 * U) {
    u32x4 wv[U][R];
    half_t sv[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = min(c0 + 64 * u, chunks - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        wv[u][r] = load_u32x4_stream(prow[r] + 4 * c);
        sv[u][r] = srow[r][c >> scale_shift];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + 64 * u;
      if (c < chunks) {
        half2_t q[R][16];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t w = wv[u][r][j];
            q[r][4 * j + 0] = nibble_pair<0>(w);
            q[r][4 * j + 1] = nibble_pair<1>(w);
            q[r][4 * j + 2] = nibble_pair<2>(w);
            q[r][4 * j + 3] = nibble_pair<3>(w);
          }
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const u32x4* xp = reinterpret_cast<const u32x4*>(x + (size_t)m * K + 32 * c);
          u32x4 xv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[j] = xp[j];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float part = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                part = __builtin_amdgcn_fdot2(q[r][4 * j + i], bit_cast<half2_t>(xv[j][i]), part, false);
            acc[m][r] = fmaf((float)sv[u][r], part, acc[m][r]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = wave_sum_lane63(acc[m][r]);

  if (lane == 63) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (row0 + r < N) y[(size_t)m * N + row0 + r] = (half_t)acc[m][r];
  }
}

typedef void (*GemvFn)(const half_t*, const uint32_t*, const half_t*, half_t*, int, int, int);

// Instantiated (R, U) shapes; the plan only ever picks one of these.
constexpr int kRs[3] = {1, 2, 4};
constexpr int kUs[4] = {1, 2, 3, 4};

template <int M, int R>
GemvFn pick_u(int U) {
  switch (U) {
    case 1: return gemv_kernel<M, R, 1>;
    case 2: return gemv_kernel<M, R, 2>;
    case 3: return gemv_kernel<M, R, 3>;
    default: return gemv_kernel<M, R, 4>;
  }
}

template <int M>
GemvFn pick_r(int R, int U) {
  switch (R) {
    case 1: return pick_u<M, 1>(U);
    case 2: return pick_u<M, 2>(U);
    default: return pick_u<M, 4>(U);
  }
}

GemvFn pick(int M, int R, int U) {
  switch (M) {
    case 1: return pick_r<1>(R, U);
    case 2: return pick_r<2>(R, U);
    case 3: return pick_r<3>(R, U);
    case 4: return pick_r<4>(R, U);
    case 5: return pick_r<5>(R, U);
    case 6: return pick_r<6>(R, U);
    case 7: return pick_r<7>(R, U);
    default: return pick_r<8>(R, U);
  }
}

}  // namespace

GemvPlan gemv_plan(int M, int N, int K, int cu_count) {
  (void)kRs;
  (void)kUs;
  GemvPlan p;
  const int chunks = K / 32;
  const int passes_one = ceil_div(chunks, 64);  // chunk iterations per lane
  // Keep every lane's weight loads of a row in one pass when registers allow.
  const int u_max = M <= 2 ? 4 : (M <= 4 ? 2 : 1);
  p.unroll = passes_one < u_max ? passes_one : u_max;
  // Rows per wave: as many as still leave >= 4 wavefronts per CU.
  const int target_waves = 4 * (cu_count > 0 ? cu_count : 256);
  p.rows_per_wave = 1;
  if (M <= 4) {
    if (ceil_div(N, 4) >= target_waves) p.rows_per_wave = 4;
    else if (ceil_div(N, 2) >= target_waves) p.rows_per_wave = 2;
  } else if (ceil_div(N, 2) >= target_waves) {
    p.rows_per_wave = 2;
  }
  p.waves_per_block = 4;
  return p;
}

hipError_t gemv_launch(const GemvPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       int M, int N, int K, int group_size, hipStream_t stream) {
  const int scale_shift = group_size == 128 ? 2 : 1;  // chunks per group = G / 32
  const int waves = ceil_div(N, p.rows_per_wave);
  const int blocks = ceil_div(waves, p.waves_per_block);
  GemvFn fn = pick(M, p.rows_per_wave, p.unroll);
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(64 * p.waves_per_block), 0, stream,
                     static_cast<const half_t*>(x), static_cast<const uint32_t*>(packed),
                     static_cast<const half_t*>(scales), static_cast<half_t*>(y), N, K, scale_shift);
  return hipGetLastError();
}

}  // namespace kf
