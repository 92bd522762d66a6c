// "Skinny" INT4 GEMM for small M (M <= 32) on gfx950: a weight stream with matrix-core math.
//
// y[M, N] = x[M, K] @ W_hat^T with W_hat = fp16_rne(q * s) (the same operand the tiled GEMM
// and the reference's tensor-core kernel use, dequant_gemm_tc_kernel.cuh:100-112), fp32
// accumulation, fp16 RNE output.
//
// At small M the weights are the traffic: the tiled GEMM re-stages them through LDS per
// M-tile and splits K through a global workspace, and the GEMV spends 4 dot2 per 8 weights
// per row of x.  Here every weight is read from HBM exactly once and dequantized once, and
// all rows of x share it through v_mfma_f32_16x16x32_f16:
//   * A workgroup owns CB blocks of 16 output columns (weight rows n0..n0+16 CB-1) and splits K
//     over its KS wavefronts; wavefront w takes a contiguous run of 128-k "super-steps" of every
//     block, so each x fragment it holds feeds CB blocks.
//   * Lane l serves column n0 + l%16 and k-quarter g = l/16 of each super-step: one dwordx4
//     of packed words per lane covers k = 128s + 32g .. +31 of its column, so a wavefront
//     instruction streams 16 columns x 128 k = 1 KiB.
//   * MFMA sub-step t (0..3) of super-step s gives lane l the k range 128s + 32g + 8t .. +7
//     for both operands: B = dequant8(word t) of its column, A = 8 consecutive x values of
//     row (16*mt + l%16).  Since A and B agree on which k each (lane group, slot) holds, the
//     MFMA sums exactly the 128 k of the super-step.
//   * Weight loads of UU super-steps are issued before their math (one round trip per pass).
//   * x: a wavefront's fragments are rows 0..15 (x 16 B each) of its own k range, and every
//     workgroup needs all of x, so per-lane loads from L2 moved 4x the weight bytes through the
//     load path (a timing-only copy without them ran 30-40% faster).  Two column blocks per
//     workgroup halve that traffic where N leaves enough workgroups to fill the GPU
//     (SkinnyPlan::col_blocks).  When the plan allows
//     (SkinnyPlan::x_lds), each wavefront first copies its k range of the M real rows into a
//     region of LDS of its own with LDS-DMA (no registers, no duplicate rows), waits for it with
//     its first weights, and reads the fragments from there; otherwise the lanes load x from L2.
//   * The KS partial 16 x 16*MT tiles are summed in fixed wavefront order through LDS
//     (deterministic) and written as fp16.  Rows past M read row M-1 and are never stored;
//     columns past N read row N-1 and are never stored.
//   * Two weight layouts, the same arithmetic (bit-identical results):
//       - row-major (the public packed format): a wavefront load touches 16 rows x 64 B;
//       - MFMA-16 blocks (kf_int4_reorder_mfma16): for each 16 columns and 128-k super-step,
//         the 64 lanes' 16-byte pieces stored contiguously in lane order, so a wavefront load
//         is one contiguous 1 KiB; scales as [N/16][K/G][16].  Measured 7-15% faster at
//         M = 1..32 on the TinyLlama / Qwen2.5 shapes.
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

__device__ __forceinline__ void dma_16B(uint32_t lds, const void* src) {
  asm volatile("global_load_lds_dwordx4 %1, off" ::"{m0}"(lds), "v"(src) : "memory");
}

// LDS layout of the x copy (XL): wavefront w's region holds rows 0..M-1 of its k range, each row
// `cpr` 16-byte chunk slots (16 per super-step, for the longest range of any wavefront); chunk c of
// row r sits at slot c ^ (r & 15), so the 16 lanes of a fragment-read phase (16 rows, one chunk)
// hit 16 different bank groups.  Regions are whole LDS-DMA instructions (64 slots) long.
__host__ __device__ inline int skinny_x_cpr(int nss, int ks) { return 16 * ((nss + ks - 1) / ks); }
__host__ __device__ inline int skinny_x_region_slots(int M, int cpr) { return (M * cpr + 63) & ~63; }

template <int MT, int U, bool BLOCKED, bool XL, int CB>
__global__ __launch_bounds__(1024) void skinny_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed,
                                                      const half_t* __restrict__ scales, half_t* __restrict__ y,
                                                      int M, int N, int K, int log2_group) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [KS][CB * MT * 256], then (XL) the x regions
  const int ks_waves = blockDim.x >> 6;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * 16 * CB;
  const int col = lane & 15;
  const int g = lane >> 4;
  const int nss = K >> 7;  // 128-k super-steps
  const int ss_begin = (wave * nss) / ks_waves;
  const int ss_end = ((wave + 1) * nss) / ks_waves;

  // Per-lane weight pointers at super-step 0 (one per column block) and their stride per
  // super-step (words); per-lane scale pointers and stride per scale group (halves).  A block
  // past the last (never on the GEMM path, where N % 64 == 0) would re-read the last block and
  // not be stored.
  const uint32_t* wrow[CB];
  const half_t* srow[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const int blk = min(blockIdx.x * CB + cb, (N + 15) / 16 - 1);
    const int n = min(16 * blk + col, N - 1);
    wrow[cb] = BLOCKED ? packed + (size_t)blk * nss * 256 + 4 * lane : packed + (size_t)n * (K >> 3) + 4 * g;
    srow[cb] = BLOCKED ? scales + (size_t)blk * (K >> log2_group) * 16 + col : scales + (size_t)n * (K >> log2_group);
  }
  constexpr int W_STEP = BLOCKED ? 256 : 16;
  constexpr int S_STEP = BLOCKED ? 16 : 1;
  const half_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = x + (size_t)min(16 * mt + col, M - 1) * K + 32 * g;

  float4_t acc[CB][MT];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[cb][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  // XL: this wavefront's k range of x rows 0..M-1 into its LDS region (see skinny_x_cpr).  Slots
  // past the last row (the region's rounding) re-load row M-1; chunks past K re-load the last one.
  const int cpr = skinny_x_cpr(nss, ks_waves);
  const unsigned char* xw = reinterpret_cast<const unsigned char*>(red) + ks_waves * CB * MT * 1024 +
                            wave * skinny_x_region_slots(M, cpr) * 16;
  if constexpr (XL) {
    const uint32_t base = (uint32_t)(uintptr_t)xw;
    const int slots = skinny_x_region_slots(M, cpr);
    for (int i0 = 0; i0 < slots; i0 += 64) {
      const int q = i0 + lane;
      const int r = min(q / cpr, M - 1), p = q % cpr;
      const int c = min(16 * ss_begin + (p ^ (r & 15)), (K >> 3) - 1);
      dma_16B(__builtin_amdgcn_readfirstlane(base + 16 * i0), x + (size_t)r * K + 8 * c);
    }
  }

  for (int ss = ss_begin; ss < ss_end; ss += U) {
    u32x4 wv[U][CB];
    half_t sv[U][CB];
    half8_t xa[U][MT][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = min(ss + u, ss_end - 1);  // in range; repeats are masked below
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        wv[u][cb] = load_u32x4_stream(wrow[cb] + W_STEP * s);
        sv[u][cb] = srow[cb][S_STEP * ((128 * s + 32 * g) >> log2_group)];
      }
      if constexpr (!XL) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < 4; ++t) xa[u][mt][t] = *reinterpret_cast<const half8_t*>(xrow[mt] + 128 * s + 8 * t);
      }
    }
    if constexpr (XL) {
      // The x copy (issued before the first pass) and this pass's weights have landed; the copy
      // is not tracked by the compiler, hence the explicit wait.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p0 = 16 * (min(ss + u, ss_end - 1) - ss_begin) + 4 * g;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int r = min(16 * mt + col, M - 1);
#pragma unroll
          for (int t = 0; t < 4; ++t)
            xa[u][mt][t] = *reinterpret_cast<const half8_t*>(xw + 16 * (r * cpr + ((p0 + t) ^ (r & 15))));
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (ss + u < ss_end) {  // uniform
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const half2_t s2 = {sv[u][cb], sv[u][cb]};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const half8_t b = dequant8(wv[u][cb][t], s2);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[cb][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u][mt][t], b, acc[cb][mt], 0, 0, 0);
          }
        }
      }
    }
  }

  // Fixed-order reduction of the KS partial tiles.  MFMA result layout: lane l,
  // element r holds row 4*(l/16)+r of the 16-row tile, column l%16.
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<float4_t*>(&red[wave * (CB * MT * 256) + (cb * MT + mt) * 256 + 4 * lane]) = acc[cb][mt];
  __syncthreads();
  for (int i = threadIdx.x; i < CB * MT * 256; i += blockDim.x) {
    float sum = 0.0f;
    for (int w = 0; w < ks_waves; ++w) sum += red[w * (CB * MT * 256) + i];
    const int bt = i >> 8, l = (i >> 2) & 63, r = i & 3;
    const int cb = bt / MT, mt = bt - cb * MT;
    const int row = 16 * mt + 4 * (l >> 4) + r;
    const int c = n0 + 16 * cb + (l & 15);
    if (row < M && c < N) y[(size_t)row * N + c] = (half_t)sum;
  }
}

typedef void (*SkinnyFn)(const half_t*, const uint32_t*, const half_t*, half_t*, int, int, int, int);

template <bool B, bool XL, int CB>
SkinnyFn skinny_fn_cb(int mt, int u) {
  switch (mt) {
    case 1:
      return u >= 4 ? skinny_kernel<1, 4, B, XL, CB>
                    : (u == 2 ? skinny_kernel<1, 2, B, XL, CB> : skinny_kernel<1, 1, B, XL, CB>);
    default: return u >= 2 ? skinny_kernel<2, 2, B, XL, CB> : skinny_kernel<2, 1, B, XL, CB>;
  }
}

template <bool B, bool XL>
SkinnyFn skinny_fn(int mt, int u, int cb) {
  return cb == 2 ? skinny_fn_cb<B, XL, 2>(mt, u) : skinny_fn_cb<B, XL, 1>(mt, u);
}

// MFMA-16 block layout: one thread per 16-byte piece of the output (grid-stride).  Piece
// o = ((nb * nss) + s) * 64 + lane holds words 16 s + 4 g .. + 3 of row min(16 nb + lane % 16,
// N - 1), g = lane / 16; the rows past N repeat row N - 1 (their columns are never stored).
__global__ __launch_bounds__(256) void reorder_mfma16_kernel(const u32x4* __restrict__ packed,
                                                             const half_t* __restrict__ scales,
                                                             u32x4* __restrict__ packed_r, half_t* __restrict__ scales_r,
                                                             int N, int K, int groups) {
  const int nss = K >> 7;
  const int nblk = (N + 15) >> 4;
  const size_t pieces = (size_t)nblk * nss * 64;
  for (size_t o = (size_t)blockIdx.x * 256 + threadIdx.x; o < pieces; o += (size_t)gridDim.x * 256) {
    const int lane = (int)(o & 63);
    const size_t bs = o >> 6;
    const int s = (int)(bs % nss);
    const int nb = (int)(bs / nss);
    const int n = min(16 * nb + (lane & 15), N - 1);
    packed_r[o] = packed[(size_t)n * (K >> 5) + 4 * s + (lane >> 4)];
  }
  const size_t nscales = (size_t)nblk * groups * 16;
  for (size_t o = (size_t)blockIdx.x * 256 + threadIdx.x; o < nscales; o += (size_t)gridDim.x * 256) {
    const int col = (int)(o & 15);
    const size_t bj = o >> 4;
    const int j = (int)(bj % groups);
    const int nb = (int)(bj / groups);
    scales_r[o] = scales[(size_t)min(16 * nb + col, N - 1) * groups + j];
  }
}

}  // namespace

int skinny_col_blocks(int N, int cu_count) {
  const int cus = cu_count > 0 ? cu_count : 256;
  return 2 * ceil_div(ceil_div(N, 32), cus) <= ceil_div(ceil_div(N, 16), cus) ? 2 : 1;
}

SkinnyPlan skinny_plan(int M, int N, int K, int cu_count) {
  SkinnyPlan p;
  p.m_tiles = ceil_div(M, 16);
  // The K split depends on K (and M) only, never on N: a column's result is then the same
  // whatever other rows share the launch, so concatenating q|k|v or gate|up rows is
  // bit-identical to separate calls.  At least two 128-k super-steps per wavefront, at
  // most 16 wavefronts, and a reduction buffer of at most 32 KiB of LDS.
  const int nss = K / 128;
  int ks = nss / 2;
  if (ks > 16) ks = 16;
  if (ks < 1) ks = 1;
  while (ks * p.m_tiles > 32) --ks;
  p.ks_waves = ks;
  // Super-steps whose weight loads are in flight together; x fragments cost 16 VGPRs per
  // 16-row tile per super-step, so fewer for more rows.
  const int per_wave = ceil_div(nss, ks);
  const int u_max = p.m_tiles == 1 ? 4 : (p.m_tiles == 2 ? 2 : 1);
  int u = per_wave < u_max ? per_wave : u_max;
  if (u == 3) u = 2;
  p.unroll = u < 1 ? 1 : u;
  // x through LDS (row-major weights only, see skinny_launch) when its copy fits, the grid still
  // runs in one round at the workgroups per CU that LDS then allows (Qwen2.5 gate/up at M = 16,
  // 560 workgroups of 55 KiB, would need two: 5% slower), and K >= 2048 or the grid has at least
  // one workgroup per CU.  Measured on the public layout, M = 4..32: TinyLlama's 4 layer shapes
  // 5-20% faster, Qwen2.5 gate/up and down up to 10% faster, Qwen2.5 q/o and k/v (K = 1536, 96 and
  // 16 workgroups) 3-9% slower with the copy, hence the last condition.
  // Two 16-column blocks per workgroup halve the copies (or L2 loads) of x per weight byte, each
  // x fragment feeding two blocks, but double the work of a workgroup: taken when the busiest
  // CU's share (workgroups per CU, rounded up, times blocks per workgroup) does not grow.
  // Measured on MI355X: TinyLlama gate/up (352 -> 176 workgroups) M = 8 / 16 with the MFMA-16
  // copy 4.90 -> 4.37 / 6.30 -> 4.85 us, on the public layout 5.57 -> 5.37 / 6.53 -> 5.92 us;
  // Qwen2.5 gate/up (560 -> 280) M = 2..16 up to 15% slower, N = 2048 (128 -> 64) 14-34% slower.
  const long cus = cu_count > 0 ? cu_count : 256;
  p.col_blocks = skinny_col_blocks(N, cu_count);
  const int red = ks * p.m_tiles * p.col_blocks * 1024;
  const long xb = (long)ks * skinny_x_region_slots(M, skinny_x_cpr(nss, ks)) * 16;
  const long lds = red + xb;
  const long wgs = ceil_div(N, 16 * p.col_blocks);
  p.x_lds = lds <= kSkinnyMaxLds && wgs <= cus * (kSkinnyMaxLds / lds) && (K >= 2048 || wgs >= cus);
  p.lds_bytes = (int)(p.x_lds ? lds : red);
  return p;
}

hipError_t skinny_launch(const SkinnyPlan& p, const void* x, const void* packed, const void* scales, void* y, int M,
                         int N, int K, int group_size, bool blocked, hipStream_t stream) {
  const int log2_group = group_size == 128 ? 7 : 6;
  // The x copy pays only with the row-major weights: with the MFMA-16 blocks the weight loads are
  // contiguous and the lanes' x loads are not what the kernel waits on (M = 4..16: 5% slower).
  const bool xl = p.x_lds && !blocked;
  const size_t lds = xl ? (size_t)p.lds_bytes : (size_t)p.ks_waves * p.m_tiles * p.col_blocks * 1024;
  const SkinnyFn fn = blocked ? skinny_fn<true, false>(p.m_tiles, p.unroll, p.col_blocks)
                              : (xl ? skinny_fn<false, true>(p.m_tiles, p.unroll, p.col_blocks)
                                    : skinny_fn<false, false>(p.m_tiles, p.unroll, p.col_blocks));
  if (lds > 65536) {  // dynamic LDS beyond 64 KiB is opted into per kernel
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, kSkinnyMaxLds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(ceil_div(N, 16 * p.col_blocks)), dim3(64 * p.ks_waves), lds, stream,
                     static_cast<const half_t*>(x), static_cast<const uint32_t*>(packed),
                     static_cast<const half_t*>(scales), static_cast<half_t*>(y), M, N, K, log2_group);
  return hipGetLastError();
}

size_t mfma16_packed_words(int N, int K) { return (size_t)ceil_div(N, 16) * 16 * (K / 8); }
size_t mfma16_scale_count(int N, int K, int group_size) { return (size_t)ceil_div(N, 16) * 16 * (K / group_size); }

hipError_t reorder_mfma16_launch(const void* packed, const void* scales, void* packed_r, void* scales_r, int N, int K,
                                 int group_size, hipStream_t stream) {
  const size_t pieces = mfma16_packed_words(N, K) / 4;
  size_t blocks = (pieces + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(reorder_mfma16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const u32x4*>(packed), static_cast<const half_t*>(scales),
                     static_cast<u32x4*>(packed_r), static_cast<half_t*>(scales_r), N, K, K / group_size);
  return hipGetLastError();
}

}  // namespace kf
