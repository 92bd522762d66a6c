// INT4 dequant GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x32_f16).
//
// y[M, N] = x[M, K] @ W_hat^T with W_hat = fp16_rne(q * s) exactly as the
// reference's tensor-core path dequantizes (dequant_gemm_tc_kernel.cuh:100-112),
// fp32 accumulation, fp16 RNE output.  Optional split-K writes fp32 partials
// that kf::splitk_reduce sums in fixed split order (deterministic), the
// behaviour of the reference's splitk_reduce (dequant_gemm_tc_kernel.cuh:156-162).
//
// Block tile BM x BN x 64 with 256 threads (4 wavefronts as WM x WN); each
// wavefront owns a (BM/WM) x (BN/WN) accumulator tile of 16x16 MFMA blocks.
// Per k-tile of 64 (64 <= G, so one scale per row and k-tile):
//   global -> registers: x tile as dwordx4 (rows >= M zero-filled) and the
//     packed tile as dwordx4 (32 B per weight row; rows >= N clamped to N-1);
//   registers -> LDS: x stored as is; weights unpacked and scaled to fp16
//     W_hat once per block (not once per wavefront) and stored row-major;
//   LDS -> MFMA: lane l reads 8 consecutive k of row (l % 16) for both A (x)
//     and B (W_hat) fragments, 16 B each, from rows padded to 72 halves.
// The next k-tile's global loads are issued before the current tile's MFMAs.
#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // halves per LDS row (144 B, 16 B aligned)
constexpr int kXcds = 8;

template <int BM, int BN, int WM, int WN, bool XCD_ORDER>
__global__ __launch_bounds__(256) void gemm_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed,
                                                   const half_t* __restrict__ scales, half_t* __restrict__ y,
                                                   float* __restrict__ ws, int M, int N, int K, int log2_group,
                                                   int kt_per_split, int tiles_n, int tiles_total) {
  static_assert(WM * WN == 4, "256 threads = 4 wavefronts");
  constexpr int TM = BM / WM / 16;
  constexpr int TN = BN / WN / 16;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 16x16 block");
  constexpr int A_VECS = BM * (BK / 8);  // dwordx4 per x tile
  constexpr int B_VECS = BN * (BK / 32); // dwordx4 per packed tile
  constexpr int A_PER_T = (A_VECS + 255) / 256;
  constexpr int B_PER_T = (B_VECS + 255) / 256;

  __shared__ __attribute__((aligned(16))) half_t As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) half_t Bs[BN * LDS_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  // Tile of this workgroup.  Consecutive workgroup ids rotate over the 8 XCDs;
  // with XCD_ORDER each XCD takes a contiguous run of tiles (M-major), so the
  // x rows and weight columns it touches stay in that XCD's L2.
  const int bid = blockIdx.x;
  int tile = bid;
  if (XCD_ORDER) {
    const int per_xcd = (tiles_total + kXcds - 1) / kXcds;
    tile = (bid % kXcds) * per_xcd + bid / kXcds;
  }
  if (tile >= tiles_total) return;
  const int tm = tile / tiles_n;
  const int n0 = (tile - tm * tiles_n) * BN;
  const int m0 = tm * BM;
  const int nkt = K / BK;
  const int kt_begin = blockIdx.y * kt_per_split;
  const int kt_end = min(nkt, kt_begin + kt_per_split);
  const int words_per_row = K >> 3;
  const int groups_per_row = K >> log2_group;

  u32x4 areg[A_PER_T];
  u32x4 breg[B_PER_T];
  half_t sreg[B_PER_T];

  auto load_tile = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < A_PER_T; ++j) {
      const int i = tid + 256 * j;
      if (A_VECS % 256 == 0 || i < A_VECS) {
        const int row = i >> 3, c = i & 7;
        const int m = m0 + row;
        if (m < M) {
          areg[j] = load_u32x4(x + (size_t)m * K + k0 + 8 * c);
        } else {
          areg[j] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
#pragma unroll
    for (int j = 0; j < B_PER_T; ++j) {
      const int i = tid + 256 * j;
      if (B_VECS % 256 == 0 || i < B_VECS) {
        const int row = i >> 1, h = i & 1;
        const int n = min(n0 + row, N - 1);
        breg[j] = load_u32x4_stream(packed + (size_t)n * words_per_row + (k0 >> 3) + 4 * h);
        sreg[j] = scales[(size_t)n * groups_per_row + (k0 >> log2_group)];
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < A_PER_T; ++j) {
      const int i = tid + 256 * j;
      if (A_VECS % 256 == 0 || i < A_VECS) {
        const int row = i >> 3, c = i & 7;
        *reinterpret_cast<u32x4*>(&As[row * LDS_STRIDE + 8 * c]) = areg[j];
      }
    }
#pragma unroll
    for (int j = 0; j < B_PER_T; ++j) {
      const int i = tid + 256 * j;
      if (B_VECS % 256 == 0 || i < B_VECS) {
        const int row = i >> 1, h = i & 1;
        const half2_t s2 = {sreg[j], sreg[j]};
#pragma unroll
        for (int w = 0; w < 4; ++w)
          *reinterpret_cast<half8_t*>(&Bs[row * LDS_STRIDE + 32 * h + 8 * w]) = dequant8(breg[j][w], s2);
      }
    }
  };

  float4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;

  if (kt_begin < kt_end) load_tile(kt_begin);
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    __syncthreads();  // every wavefront is done reading the previous tile
    store_tile();
    __syncthreads();
    if (kt + 1 < kt_end) load_tile(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      half8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const half8_t*>(
            &As[((wm * TM + i) * 16 + frag_row) * LDS_STRIDE + 32 * ks + frag_k]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const half8_t*>(
            &Bs[((wn * TN + j) * 16 + frag_row) * LDS_STRIDE + 32 * ks + frag_k]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // 16x16 MFMA result layout: lane l, element r holds row 4*(l/16)+r, column l%16.
  const int out_col = lane & 15;
  const int out_row = (lane >> 4) * 4;
  float* part = ws ? ws + (size_t)blockIdx.y * M * N : nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int col = n0 + (wn * TN + j) * 16 + out_col;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + (wm * TM + i) * 16 + out_row + r;
        if (row < M) {
          if (part)
            part[(size_t)row * N + col] = acc[i][j][r];
          else
            y[(size_t)row * N + col] = (half_t)acc[i][j][r];
        }
      }
    }
}

__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ ws, half_t* __restrict__ y,
                                                      size_t mn, int splits) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < mn; i += (size_t)gridDim.x * 256) {
    float s = 0.0f;
    for (int z = 0; z < splits; ++z) s += ws[(size_t)z * mn + i];
    y[i] = (half_t)s;
  }
}

struct TileCfg {
  int bm, bn;
  bool xcd;
};
// Tile table: index = GemmPlan::tile.
constexpr TileCfg kTiles[] = {{16, 128, false}, {32, 128, false}, {64, 128, false}, {128, 128, false},
                              {128, 128, true}, {64, 128, true}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

typedef void (*GemmFn)(const half_t*, const uint32_t*, const half_t*, half_t*, float*, int, int, int, int, int, int,
                       int);

GemmFn gemm_fn(int tile) {
  switch (tile) {
    case 0: return gemm_kernel<16, 128, 1, 4, false>;
    case 1: return gemm_kernel<32, 128, 1, 4, false>;
    case 2: return gemm_kernel<64, 128, 2, 2, false>;
    case 3: return gemm_kernel<128, 128, 2, 2, false>;
    case 4: return gemm_kernel<128, 128, 2, 2, true>;
    default: return gemm_kernel<64, 128, 2, 2, true>;
  }
}

}  // namespace

int gemm_num_tiles() { return kNumTiles; }

GemmPlan gemm_plan_with_tile(int M, int N, int K, int cu_count, int tile) {
  GemmPlan p;
  p.skinny = false;
  p.sk = SkinnyPlan{0, 0, 0};
  p.tile = tile;
  p.block_m = kTiles[tile].bm;
  p.block_n = kTiles[tile].bn;
  const int nkt = K / BK;
  const long tiles = (long)ceil_div(N, p.block_n) * ceil_div(M, p.block_m);
  const long want = 2L * (cu_count > 0 ? cu_count : 256);
  int splits = 1;
  if (tiles < want) {
    splits = (int)((want + tiles - 1) / tiles);
    const int max_splits = nkt / 4 > 0 ? nkt / 4 : 1;  // at least 4 k-tiles per split
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
  }
  p.kt_per_split = ceil_div(nkt, splits);
  p.splits = ceil_div(nkt, p.kt_per_split);  // no empty splits
  return p;
}

GemmPlan gemm_plan(int M, int N, int K, int cu_count) {
  if (M <= kSkinnyMaxM && K % 128 == 0) {
    GemmPlan p = gemm_plan_with_tile(M, N, K, cu_count, 0);
    p.skinny = true;
    p.splits = 1;
    p.sk = skinny_plan(M, N, K, cu_count);
    return p;
  }
  const int tile = M <= 16 ? 0 : (M <= 32 ? 1 : (M <= 64 ? 2 : 3));
  return gemm_plan_with_tile(M, N, K, cu_count, tile);
}

size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N) {
  return !p.skinny && p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

hipError_t gemm_launch(const GemmPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       void* ws, int M, int N, int K, int group_size, hipStream_t stream) {
  if (p.skinny) return skinny_launch(p.sk, x, packed, scales, y, M, N, K, group_size, stream);
  const int log2_group = group_size == 128 ? 7 : 6;
  const int tiles_n = ceil_div(N, p.block_n);
  const int tiles_total = tiles_n * ceil_div(M, p.block_m);
  const int grid_x = kTiles[p.tile].xcd ? ceil_div(tiles_total, kXcds) * kXcds : tiles_total;
  float* part = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
  hipLaunchKernelGGL(gemm_fn(p.tile), dim3(grid_x, p.splits), dim3(256), 0, stream, static_cast<const half_t*>(x),
                     static_cast<const uint32_t*>(packed), static_cast<const half_t*>(scales),
                     static_cast<half_t*>(y), part, M, N, K, log2_group, p.kt_per_split, tiles_n, tiles_total);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.splits == 1) return err;
  const size_t mn = (size_t)M * N;
  size_t blocks = (mn + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const float*>(ws),
                     static_cast<half_t*>(y), mn, p.splits);
  return hipGetLastError();
}

}  // namespace kf
