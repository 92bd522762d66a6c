// INT4 dequant GEMM on the CDNA4 matrix cores (v_mfma_f32_16x16x32_f16).
//
// y[M, N] = x[M, K] @ W_hat^T with W_hat = fp16_rne(q * s) exactly as the reference's
// tensor-core path dequantizes (dequant_gemm_tc_kernel.cuh:100-112), fp32 accumulation,
// fp16 RNE output.  Optional split-K writes fp32 partials that kf::splitk_reduce sums in
// fixed split order (deterministic), the behaviour of the reference's splitk_reduce
// (dequant_gemm_tc_kernel.cuh:156-162).
//
// Three kernel families share one tile table (kTiles below; gemm_plan picks an entry and a
// split-K factor with a fitted cost model):
//   * gemm_kernel<TileCfg>: register-staged LDS tiles, 64 x 128 down to 16 x 64;
//   * gemm_dma_kernel<KW>: 128 x 128 tiles fed by LDS-DMA, 2 (4 wavefronts) or 4 (8 wavefronts)
//     k-groups; see the comment above the kernel;
//   * gemm_wide_kernel: 192 x 256 tiles fed by LDS-DMA, 8 wavefronts, one workgroup per CU, for
//     grids of about one tile per CU (half the L2 -> LDS bytes per output of the 128 x 128 tiles).
//
// Design of gemm_kernel (gfx950: 4 SIMDs per CU, ~2 VALU ops hide under one 16x16x32 MFMA,
// LDS reads ~150-200 B/clk per CU):
//   * Workgroup tile BM x BN; WGM x WGN wavefronts tile it, and WK such groups split each
//     stage's k range (in-block split-K, summed in fixed order through LDS at the end).
//   * A stage covers SK = 64 * WK k.  x is staged in LDS as fp16; the weights stay PACKED
//     in LDS (4 bits per weight: 4x less LDS traffic than an fp16 W_hat tile).  Each
//     wavefront dequantizes only its own columns, with one scale per column and stage, so
//     a weight is dequantized once per (workgroup, M-wavefront row); with WGM = 1 that is
//     once per workgroup.
//   * Global -> registers two stages ahead, registers -> LDS one stage ahead, LDS double
//     buffered: one barrier per stage.
//   * LDS layouts are XOR-swizzled so every fragment read and tile write is free of bank
//     conflicts on gfx950's 64-bank LDS: x rows are 16-byte chunks c stored at slot
//     c ^ f(row); packed rows are 8-byte units u stored at u ^ f'(row).
//   * MFMA operands: lane l serves row / column l % 16 and k-group g = l / 16.  In sub-step
//     t (0, 1) of k-group kw it supplies k = 64 kw + 16 g + 8 t .. +7 for both A (one
//     16-byte x chunk) and B (one packed word, dequantized with dequant8), so one 8-byte
//     LDS read gives a lane both sub-steps' weights.
//   * Tiles are ordered in bands of group_m M-tiles (all N-tiles of a band before the next
//     band); the (split, tile) jobs of a launch, split-major, are dealt to the 8 XCDs in
//     contiguous runs of equal length, so the x rows an XCD uses stay in its L2, each weight
//     tile is fetched once per band, and no XCD holds more jobs than another (a 1-D grid: the
//     hardware deals workgroup i to XCD i % 8).
#include <algorithm>
#include <type_traits>

#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

constexpr int kXcds = 8;

// Job of this workgroup in a 1-D grid of ceil(jobs / 8) * 8 workgroups: XCD x (= blockIdx.x % 8)
// takes jobs x * per_xcd .. + per_xcd - 1.  Job j = split * tiles + tile.  False: no job.
__device__ __forceinline__ bool gemm_job(int tiles, int splits, int& split, int& tile) {
  const int jobs = tiles * splits;
  const int per_xcd = (jobs + kXcds - 1) / kXcds;
  const int j = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (j >= jobs) return false;
  split = j / tiles;
  tile = j - split * tiles;
  return true;
}

template <int BM_, int BN_, int WGM_, int WGN_, int WK_, int WAVES_PER_SIMD_ = 2>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_, WK = WK_;
  // Occupancy target: 2 wavefronts per SIMD leave 256 registers per lane, 1 leaves 512.
  static constexpr int WAVES_PER_SIMD = WAVES_PER_SIMD_;
  static constexpr int THREADS = 64 * WGM * WGN * WK;
  static constexpr int SK = 64 * WK;                  // k per stage
  static constexpr int A_ROW = 2 * SK;                // bytes per x row in LDS
  static constexpr int A_CHUNKS_ROW = SK / 8;         // 16-byte chunks per x row
  static constexpr int B_ROW = SK / 2;                // bytes per packed row in LDS
  static constexpr int B_CHUNKS_ROW = SK / 32;        // 16-byte chunks per packed row
  static constexpr int B_UNITS_ROW = SK / 16;         // 8-byte units per packed row
  static constexpr int A_STAGE = BM * A_ROW;
  static constexpr int B_STAGE = BN * B_ROW;
  static constexpr int S_STAGE = WK * BN * 2;         // fp16 scales [WK][BN]
  static constexpr int STAGE = A_STAGE + B_STAGE + S_STAGE;
  static constexpr int A_CHUNKS = BM * A_CHUNKS_ROW;
  static constexpr int B_CHUNKS = BN * B_CHUNKS_ROW;
  static constexpr int A_PER_T = A_CHUNKS / THREADS;
  static constexpr int B_PER_T = (B_CHUNKS + THREADS - 1) / THREADS;
  static constexpr int TM = BM / WGM / 16;            // 16x16 blocks per wavefront along M
  static constexpr int TN = BN / WGN / 16;            // ... along N
  static constexpr int RED = (WK - 1) * WGM * WGN * TM * TN * 256 * 4;  // bytes of k-group partials
  static_assert(A_CHUNKS % THREADS == 0, "x tile must split evenly over the threads");
  static_assert(TM >= 1 && TN >= 1 && BM % (16 * WGM) == 0 && BN % (16 * WGN) == 0, "wave tile");
  static_assert(16 % B_UNITS_ROW == 0, "packed-row swizzle needs 4, 8 or 16 units per row");
  static_assert(STAGE % 16 == 0, "stage alignment");
  static_assert(RED <= 2 * STAGE, "k-group reduction must fit in the stage buffers");
  static_assert(2 * STAGE <= 160 * 1024, "LDS");
};

// Swizzle of 8-byte units in packed row `row`: rows that a 16-lane phase of an 8-byte read
// touches land on distinct banks.
template <class C>
__device__ __forceinline__ int b_swizzle(int row) {
  return (row / (16 / C::B_UNITS_ROW)) & (C::B_UNITS_ROW - 1);
}

template <class C>
struct StageRegs {
  u32x4 a[C::A_PER_T];
  u32x4 b[C::B_PER_T];
  half_t s[C::B_PER_T];
};

template <class C>
__global__ __launch_bounds__(C::THREADS) __attribute__((amdgpu_waves_per_eu(C::WAVES_PER_SIMD, C::WAVES_PER_SIMD)))
void gemm_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed, const half_t* __restrict__ scales,
                 half_t* __restrict__ y, float* __restrict__ ws, int M, int N, int K, int log2_group,
                 int stages_per_split, int splits, int tiles_m, int tiles_n, int group_m) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * C::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave / (C::WGM * C::WGN);
  const int wmn = wave - kw * (C::WGM * C::WGN);
  const int wm = wmn / C::WGN;
  const int wn = wmn - wm * C::WGN;
  const int g = lane >> 4;
  const int l16 = lane & 15;

  // Split and tile of this workgroup (see the header comment for the order).
  int split, t;
  if (!gemm_job(tiles_m * tiles_n, splits, split, t)) return;
  const int band = group_m * tiles_n;
  const int bi = t / band;
  const int tb = t - bi * band;
  const int gm = min(group_m, tiles_m - bi * group_m);
  const int mt = bi * group_m + tb % gm;
  const int nt = tb / gm;
  const int m0 = mt * C::BM;
  const int n0 = nt * C::BN;

  const int nst = K / C::SK;
  const int st_begin = split * stages_per_split;
  const int st_end = min(nst, st_begin + stages_per_split);
  const int ns = st_end - st_begin;
  const int words_per_row = K >> 3;
  const int groups_per_row = K >> log2_group;

  // Global -> registers.  Rows of x past M are clamped (they only feed output rows that
  // are never stored); weight rows past N are clamped the same way.  Every thread loads
  // every stage unconditionally (stage indices are clamped instead), which keeps the
  // compiler's per-register load tracking exact: a wait covers only the stage it needs.
  const half_t* a_src[C::A_PER_T];
#pragma unroll
  for (int j = 0; j < C::A_PER_T; ++j) {
    const int i = tid + C::THREADS * j;
    const int row = i / C::A_CHUNKS_ROW, c = i % C::A_CHUNKS_ROW;
    a_src[j] = x + (size_t)min(m0 + row, M - 1) * K + 8 * c;
  }
  const uint32_t* b_src[C::B_PER_T];
  const half_t* s_src[C::B_PER_T];
#pragma unroll
  for (int j = 0; j < C::B_PER_T; ++j) {
    const int i = min(tid + C::THREADS * j, C::B_CHUNKS - 1);
    const int row = i / C::B_CHUNKS_ROW, h = i % C::B_CHUNKS_ROW;
    const int n = min(n0 + row, N - 1);
    b_src[j] = packed + (size_t)n * words_per_row + 4 * h;
    s_src[j] = scales + (size_t)n * groups_per_row;
  }
  auto load = [&](StageRegs<C>& R, int st) {
    const int k0 = st * C::SK;
#pragma unroll
    for (int j = 0; j < C::A_PER_T; ++j) R.a[j] = load_u32x4(a_src[j] + k0);
#pragma unroll
    for (int j = 0; j < C::B_PER_T; ++j) {
      const int h = (tid + C::THREADS * j) % C::B_CHUNKS_ROW;
      R.b[j] = load_u32x4(b_src[j] + (k0 >> 3));
      R.s[j] = s_src[j][(k0 + 32 * (h & ~1)) >> log2_group];
    }
  };

  // x tile: 16-byte chunk c of row r sits at slot c ^ a_swizzle(r).  Sixteen consecutive
  // rows (one 16-lane phase of a 16-byte read) then cover all 64 banks.
  auto a_slot = [](int row, int c) {
    constexpr int RSH = C::A_ROW >= 256 ? 0 : 1;  // rows per 256-byte bank window: 1 or 2
    return c ^ ((row >> RSH) & (C::A_CHUNKS_ROW - 1));
  };

  // Registers -> LDS stage buffer (swizzled).
  auto store = [&](const StageRegs<C>& R, unsigned char* st) {
#pragma unroll
    for (int j = 0; j < C::A_PER_T; ++j) {
      const int i = tid + C::THREADS * j;
      const int row = i / C::A_CHUNKS_ROW, c = i % C::A_CHUNKS_ROW;
      *reinterpret_cast<u32x4*>(st + row * C::A_ROW + 16 * a_slot(row, c)) = R.a[j];
    }
#pragma unroll
    for (int j = 0; j < C::B_PER_T; ++j) {
      const int i = tid + C::THREADS * j;
      if (C::B_CHUNKS % C::THREADS == 0 || i < C::B_CHUNKS) {
        const int row = i / C::B_CHUNKS_ROW, h = i % C::B_CHUNKS_ROW;
        const int sw = b_swizzle<C>(row);
        unsigned char* rb = st + C::A_STAGE + row * C::B_ROW;
        *reinterpret_cast<uint2*>(rb + 8 * ((2 * h) ^ sw)) = uint2{R.b[j].x, R.b[j].y};
        *reinterpret_cast<uint2*>(rb + 8 * ((2 * h + 1) ^ sw)) = uint2{R.b[j].z, R.b[j].w};
        if ((h & 1) == 0)
          reinterpret_cast<half_t*>(st + C::A_STAGE + C::B_STAGE)[(h >> 1) * C::BN + row] = R.s[j];
      }
    }
  };

  float4_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Packed words (both sub-steps) and scales of this wave's columns for one stage.
  uint2 bw[C::TN];
  half2_t s2[C::TN];
  auto read_b = [&](const unsigned char* st) {
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int row = (wn * C::TN + j) * 16 + l16;
      const int u = 4 * kw + g;
      bw[j] = *reinterpret_cast<const uint2*>(st + C::A_STAGE + row * C::B_ROW + 8 * (u ^ b_swizzle<C>(row)));
      const half_t sc = reinterpret_cast<const half_t*>(st + C::A_STAGE + C::B_STAGE)[kw * C::BN + row];
      s2[j] = half2_t{sc, sc};
    }
  };
  auto read_a = [&](const unsigned char* st, int sub, half8_t (&a)[C::TM]) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int row = (wm * C::TM + i) * 16 + l16;
      a[i] = *reinterpret_cast<const half8_t*>(st + row * C::A_ROW + 16 * a_slot(row, 8 * kw + 2 * g + sub));
    }
  };
  auto mfma_sub = [&](const half8_t (&a)[C::TM], const uint32_t (&w)[C::TN], const half2_t (&sc)[C::TN]) {
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const half8_t b = dequant8(w[j], sc[j]);
#pragma unroll
      for (int i = 0; i < C::TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a[i], acc[i][j], 0, 0, 0);
    }
  };

  // Software pipeline, one barrier per stage.  Stage s lives in LDS buffer s % 2 and is
  // computed in two sub-steps; the LDS reads for the next sub-step are issued before the
  // MFMAs of the current one, and the barrier sits between the two sub-steps:
  //   read x(sub 1) | MFMA sub 0 | write stage s+1 to the other buffer, load stage s+3 |
  //   barrier | read words, scales, x(sub 0) of stage s+1 | MFMA sub 1
  // Registers R[(s+1) % 2] carry stage s+1 from global memory to LDS (loaded two stages
  // ahead).  Stage indices past the split's end are clamped to its last stage; those
  // duplicate loads, writes and reads are never used.
  unsigned char* const L0 = smem;
  unsigned char* const L1 = smem + C::STAGE;
  const int last = st_end - 1;
  auto stage_at = [&](int i) { return min(st_begin + i, last); };
  StageRegs<C> R0, R1;
  half8_t a0[C::TM], a1[C::TM];
  if (ns > 0) {
    load(R0, stage_at(0));
    load(R1, stage_at(1));
    store(R0, L0);
    load(R0, stage_at(2));
    __syncthreads();
    read_b(L0);
    read_a(L0, 0, a0);

    auto half_iter = [&](auto cur_c, int s) {
      constexpr int CUR = decltype(cur_c)::value;
      unsigned char* const cur = CUR ? L1 : L0;
      unsigned char* const nxt = CUR ? L0 : L1;
      StageRegs<C>& Rn = CUR ? R0 : R1;
      uint32_t w0[C::TN], w1[C::TN];
      half2_t sc[C::TN];
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        w0[j] = bw[j].x;
        w1[j] = bw[j].y;
        sc[j] = s2[j];
      }
      read_a(cur, 1, a1);
      mfma_sub(a0, w0, sc);
      store(Rn, nxt);
      load(Rn, stage_at(s + 3));
      __syncthreads();
      read_b(nxt);
      read_a(nxt, 0, a0);
      mfma_sub(a1, w1, sc);
    };
    for (int s = 0; s < ns; s += 2) {
      half_iter(std::integral_constant<int, 0>(), s);
      if (s + 1 >= ns) break;
      half_iter(std::integral_constant<int, 1>(), s + 1);
    }
  }
  __syncthreads();

  // In-block split-K: k-groups 1.. hand their partial tiles to k-group 0 through LDS (the
  // stage buffers are free after the barrier above) and it adds them in fixed order.
  if constexpr (C::WK > 1) {
    float* red = reinterpret_cast<float*>(smem);
    constexpr int WAVE_FLOATS = C::TM * C::TN * 256;
    if (kw > 0) {
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          *reinterpret_cast<float4_t*>(
              &red[((kw - 1) * C::WGM * C::WGN + wmn) * WAVE_FLOATS + (i * C::TN + j) * 256 + 4 * lane]) = acc[i][j];
    }
    __syncthreads();
    if (kw > 0) return;
#pragma unroll
    for (int q = 1; q < C::WK; ++q)
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
          acc[i][j] += *reinterpret_cast<const float4_t*>(
              &red[((q - 1) * C::WGM * C::WGN + wmn) * WAVE_FLOATS + (i * C::TN + j) * 256 + 4 * lane]);
  }

  // The MFMAs take the weights as their first operand, so each 16 x 16 block comes out transposed:
  // lane l, element r holds y row l%16, column 4*(l/16)+r.  A lane stores its four consecutive
  // columns at once (8 bytes of y or 16 of fp32 partials); N % 64 == 0 keeps them inside the row.
  float* part = ws ? ws + (size_t)split * M * N : nullptr;
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int row = m0 + (wm * C::TM + i) * 16 + l16;
    if (row >= M) continue;
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      const int col = n0 + (wn * C::TN + j) * 16 + 4 * g;
      if (col >= N) continue;
      if (part) {
        *reinterpret_cast<float4_t*>(part + (size_t)row * N + col) = acc[i][j];
      } else {
        const half2_t lo = {(half_t)acc[i][j][0], (half_t)acc[i][j][1]};
        const half2_t hi = {(half_t)acc[i][j][2], (half_t)acc[i][j][3]};
        *reinterpret_cast<u32x2*>(y + (size_t)row * N + col) = u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
      }
    }
  }
}

// ---- DMA-fed kernel: 128 x 128 tile, KW k-groups (KW = 2: 4 wavefronts, 64-k stages;
// KW = 4: 8 wavefronts, 128-k stages) ------------------------------------------------
//
// Every byte of a stage goes global -> LDS through the gfx950 LDS-DMA loads
// (global_load_lds_dwordx4 / _ushort: lane l's data lands at M0 + 16 l, or M0 + 4 l for
// 16-bit loads, zero-extended), so staging costs no registers and no VALU/LDS-write
// instructions, and the 128 accumulators per lane of a 128 x 64 wave tile fit with two
// wavefronts per SIMD.  A 128 x 64 wave tile makes one dequantized weight fragment feed 8
// MFMAs (the VALU work stays under the MFMA shadow) and one x fragment feed 4 (LDS reads
// stay well under the LDS bandwidth).
//
// Wavefront (kw, wn): column half wn (64 columns) and k-group kw, which takes k 32 kw ..
// 32 kw + 31 of every stage; the k-groups' accumulators are summed in fixed order through LDS
// at the end (in-block split-K).  KW = 2 gives four wave tasks per 128 x 128 tile, enough to
// spread evenly over the 1024 SIMDs when the grid has several tiles per CU; KW = 4 gives one
// workgroup of two wavefronts per SIMD when the grid has about one tile per CU.
//
// The DMA loads are issued from inline assembly with a "memory" clobber: the compiler
// neither tracks them nor moves LDS accesses across them, and the loop contains no
// compiler-tracked global loads, so its own waits never cover the prefetches.  Each
// wavefront issues exactly kDmaPerStage loads per stage (stage indices are clamped, never
// skipped), so "s_waitcnt vmcnt(kDmaPerStage)" means: the older stage has landed, the
// newer one may still be in flight.
//
// LDS stage layout (bytes): x rows of A_ROW = 2 BK bytes with 16-byte chunk c at slot
// c ^ a_swz(row); packed rows of BK / 2 bytes with 16-byte chunk h at h ^ b_swz(row).  Every
// read phase of the MFMA fragments is free of bank conflicts.  Three stages rotate.  Scales:
// with KW = 2 a stage lies inside one group (G >= 64 = BK), so they live in their own ring of
// three slabs of 4-byte slots, one slab per group, fetched by the k-group 0 wavefronts with
// the first stage of the group (that stage costs those two wavefronts one more DMA, and their
// wait count for it is one higher); with KW = 4 each stage carries the slabs of its one or two
// groups, fetched by the first one or two k-groups with every stage.
// Constants of the DMA-fed kernel with KW k-groups (KW = 2: 4 wavefronts, 64-k stages;
// KW = 4: 8 wavefronts, 128-k stages).  Every wavefront owns a 128 x 64 wave tile over a 32-k
// slice of each stage, so the VALU/MFMA and LDS/MFMA ratios are the same for both; KW = 4 puts
// two wavefronts per SIMD into one workgroup per CU, for grids with about one tile per CU.
template <int KW>
struct DmaCfg {
  static constexpr int BM = 128, BN = 128, BK = 32 * KW, NS = 3, WAVES = 2 * KW, THREADS = 64 * WAVES;
  static constexpr int TM = 8, TN = 4;
  static constexpr int A_ROW = BK * 2;               // bytes of x per row and stage (128 / 256)
  static constexpr int A_CH = BK / 8;                // 16-byte chunks per x row (8 / 16)
  static constexpr int A_RSH = A_ROW >= 256 ? 0 : 1; // rows per 256-byte bank window: 1 or 2
  static constexpr int A_BYTES = BM * A_ROW;
  static constexpr int B_OFF = A_BYTES;
  static constexpr int B_ROW = BK / 2;               // bytes of packed weights per row and stage
  static constexpr int B_CH = BK / 32;               // 16-byte chunks per packed row (2 / 4)
  static constexpr int B_BYTES = BN * B_ROW;
  // Scales.  KW = 2: a stage lies inside one group (G >= 64 = BK), so the scales live in a ring
  // of NS per-group slabs after the stages and are fetched once per group.  KW = 4: a stage
  // holds one (G = 128) or two (G = 64) groups, fetched with the stage into its own slabs.
  static constexpr bool STAGE_SCALES = KW == 4;
  static constexpr int S_SLAB = BN * 4;              // [BN] 4-byte slots
  static constexpr int S_OFF = B_OFF + B_BYTES;      // per-stage slabs (KW = 4): [2][BN]
  static constexpr int STAGE = STAGE_SCALES ? S_OFF + 2 * S_SLAB : S_OFF;
  static constexpr int S_RING = NS * STAGE;          // per-group ring (KW = 2): [NS][BN]
  static constexpr int RING_END = S_RING + (STAGE_SCALES ? 0 : NS * S_SLAB);
  static constexpr int OUT_ROW = BN * 2 + 16;        // epilogue fp16 tile row stride (bytes), padded
  static constexpr int WAVE_TILE = TM * TN * 256 * 4;  // fp32 partial tile of one wavefront
  static constexpr int RED_BYTES = (KW / 2) * 2 * WAVE_TILE;  // k-group partials staged at once
  static constexpr int SMEM = RING_END > RED_BYTES ? (RING_END > BM * OUT_ROW ? RING_END : BM * OUT_ROW)
                                                   : (RED_BYTES > BM * OUT_ROW ? RED_BYTES : BM * OUT_ROW);
  static constexpr int kDmaPerStage = 5;             // per wavefront: 4 x, 1 packed (+1 scales, see below)
  static_assert(A_BYTES == 4 * 1024 * WAVES && B_BYTES == 1024 * WAVES, "4 x and 1 packed DMA per wavefront");
  static_assert(SMEM <= 160 * 1024, "LDS");
};

__device__ __forceinline__ void dma_16B(uint32_t lds, const void* src) {
  asm volatile("global_load_lds_dwordx4 %1, off" ::"{m0}"(lds), "v"(src) : "memory");
}
__device__ __forceinline__ void dma_u16(uint32_t lds, const void* src) {
  asm volatile("global_load_lds_ushort %1, off" ::"{m0}"(lds), "v"(src) : "memory");
}

template <int KW>
__global__ __launch_bounds__(DmaCfg<KW>::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_dma_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed,
                     const half_t* __restrict__ scales, half_t* __restrict__ y, float* __restrict__ ws, int M, int N,
                     int K, int log2_group, int stages_per_split, int splits, int tiles_m, int tiles_n,
                     int group_m) {
  using C = DmaCfg<KW>;
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, NS = C::NS, THREADS = C::THREADS, TM = C::TM, TN = C::TN;
  constexpr int A_ROW = C::A_ROW, B_ROW = C::B_ROW, B_OFF = C::B_OFF, STAGE = C::STAGE, OUT_ROW = C::OUT_ROW;
  constexpr int kDmaPerStage = C::kDmaPerStage;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 1;
  const int kw = wave >> 1;
  const int g = lane >> 4;
  const int l16 = lane & 15;

  int split, t;
  if (!gemm_job(tiles_m * tiles_n, splits, split, t)) return;
  const int band = group_m * tiles_n;
  const int bi = t / band;
  const int tb = t - bi * band;
  const int gm = min(group_m, tiles_m - bi * group_m);
  const int m0 = (bi * group_m + tb % gm) * BM;
  const int n0 = (tb / gm) * BN;

  const int nst = K / BK;
  const int st_begin = split * stages_per_split;
  const int last = min(nst, st_begin + stages_per_split) - 1;
  const int ns = last + 1 - st_begin;

  // XOR swizzles: x chunk c of row r at slot c ^ a_swz(r); packed chunk h of row r at h ^ b_swz(r).
  auto a_swz = [](int row) { return (row >> C::A_RSH) & (C::A_CH - 1); };
  auto b_swz = [](int row) { return (row / (16 / C::B_CH)) & (C::B_CH - 1); };

  // Per-lane DMA sources at k = 0 (advanced by the stage's k offset).  x: this wave's 4
  // instructions of 1 KiB cover 1024 / A_ROW rows each; packed: one instruction of 1 KiB.
  constexpr int A_RPI = 1024 / A_ROW, A_LPR = A_ROW / 16;  // rows per instruction, lanes per row
  constexpr int B_RPI = 1024 / B_ROW, B_LPR = B_ROW / 16;
  const half_t* a_src[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = A_RPI * (4 * wave + q) + lane / A_LPR;
    a_src[q] = x + (size_t)min(m0 + row, M - 1) * K + 8 * ((lane % A_LPR) ^ a_swz(row));
  }
  const int brow = B_RPI * wave + lane / B_LPR;
  const uint32_t* b_src =
      packed + (size_t)min(n0 + brow, N - 1) * (K >> 3) + 4 * ((lane % B_LPR) ^ b_swz(brow));
  const int groups = K >> log2_group;
  const half_t* s_src = scales + (size_t)min(n0 + 64 * wn + lane, N - 1) * groups;
  const uint32_t smem_base = (uint32_t)(uintptr_t)smem;

  // KW = 2, per-group scale ring: split-local stage i (clamped) starts a scale group when
  // i == 0 or its k0 is a multiple of G; groups are numbered from the split's first stage.
  // The clamped repeats of the last stage past the split's end never start one.
  const int log2_spg = log2_group - 6;  // log2(stages per group), KW = 2
  auto starts_group = [&](int i) {
    const int st = st_begin + i;
    return i == 0 || (st <= last && (st & ((1 << log2_spg) - 1)) == 0);
  };
  auto group_of = [&](int i) {  // split-local group index of split-local stage i (i <= ns - 1)
    return ((st_begin + i) >> log2_spg) - (st_begin >> log2_spg);
  };
  // KW = 4, per-stage scales: a stage holds gps = BK / G groups (1 or 2); k-group kw < gps
  // fetches group gps * st + kw for its wavefronts' 64 columns, and k-group kw reads slab
  // (32 kw) >> log2_group.
  const int gps = BK >> log2_group;
  const bool stage_scale_loader = C::STAGE_SCALES && kw < gps;
  // DMA of split-local stage i (clamped) into buffer i % NS, plus scales.  Returns whether
  // this wavefront issued a scale load (one more outstanding load).
  auto issue = [&](int i, int buf) {  // buf == i % NS
    const int st = min(st_begin + i, last);
    const int k0 = st * BK;
    const uint32_t base = __builtin_amdgcn_readfirstlane(smem_base + (uint32_t)(buf * STAGE));
#pragma unroll
    for (int q = 0; q < 4; ++q) dma_16B(base + 1024 * (4 * wave + q), a_src[q] + k0);
    dma_16B(base + B_OFF + 1024 * wave, b_src + (k0 >> 3));
    if constexpr (C::STAGE_SCALES) {
      if (stage_scale_loader) {
        dma_u16(__builtin_amdgcn_readfirstlane(base + (uint32_t)(C::S_OFF + kw * C::S_SLAB + 256 * wn)),
                s_src + gps * st + kw);
      }
      return stage_scale_loader;
    } else {
      const bool sc = kw == 0 && starts_group(i);
      if (sc) {
        const uint32_t sbase = __builtin_amdgcn_readfirstlane(
            smem_base + (uint32_t)(C::S_RING + (group_of(i) % NS) * C::S_SLAB + 256 * wn));
        dma_u16(sbase, s_src + (k0 >> log2_group));
      }
      return sc;
    }
  };
  auto wait_older = [&](bool newer_has_scales) {  // all but the newest stage's loads landed
    if (newer_has_scales)
      wait_vmcnt<kDmaPerStage + 1>();
    else
      wait_vmcnt<kDmaPerStage>();
  };

  float4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Lane-dependent LDS offsets inside a stage.  x: row l16 (+16 per block), chunk 4 kw + g.
  // packed: row 64 wn + 16 j + l16, dword 4 kw + g.  scales: column 64 wn + 16 j + l16.
  const int a_off = l16 * A_ROW + 16 * ((4 * kw + g) ^ a_swz(l16));
  const int b_off = B_OFF + (64 * wn + l16) * B_ROW + 16 * (kw ^ b_swz(l16)) + 4 * g;
  const int s_off = 4 * (64 * wn + l16) + (C::STAGE_SCALES ? C::S_OFF + ((32 * kw) >> log2_group) * C::S_SLAB : 0);

  const UnpackConsts uc = unpack_consts();
  half8_t a[TM];
  uint32_t w[TN];
  half2_t s2[TN];
  auto read_frags = [&](int i, int buf) {  // buf == i % NS, a compile-time constant at the call
    const unsigned char* st = smem + buf * STAGE;
    const unsigned char* slab = C::STAGE_SCALES ? st : smem + C::S_RING + (group_of(i) % NS) * C::S_SLAB;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      w[j] = *reinterpret_cast<const uint32_t*>(st + b_off + 16 * B_ROW * j);
      const half_t sc = *reinterpret_cast<const half_t*>(slab + s_off + 64 * j);
      s2[j] = half2_t{sc, sc};
    }
#pragma unroll
    for (int q = 0; q < TM; ++q) a[q] = *reinterpret_cast<const half8_t*>(st + a_off + 16 * A_ROW * q);
  };

  // Stage i: DMA issued at iteration i - 2 into buffer i % NS; at iteration i - 1 each
  // wavefront waits for its own loads of it and the barrier publishes it; at iteration i
  // its fragments are read and its MFMAs run.  The DMA of stage i + 2 (iteration i)
  // overwrites the buffer of stage i - 1, whose reads completed before the barrier of
  // iteration i - 1 (lgkmcnt(0) precedes every barrier).  Likewise (KW = 2) the scale slab
  // of group q is fetched with q's first stage i (iteration i - 2) into the slab of group
  // q - 3, last read at a stage <= i - 3 (groups span >= 1 stage), before that barrier.
  // The loop is unrolled by NS so every buffer offset is a compile-time immediate.
  issue(0, 0);
  wait_older(issue(1, 1));
  __syncthreads();
  auto step = [&](auto buf_c, int s) {  // stage s, held in buffer CUR == s % NS
    constexpr int CUR = decltype(buf_c)::value;
    read_frags(s, CUR);
    wait_older(issue(s + 2, (CUR + 2) % NS));  // stage s + 1 landed
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const half8_t b = dequant8(w[j], s2[j], uc);
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a[i], acc[i][j], 0, 0, 0);
    }
  };
  static_assert(NS == 3, "the unrolled loop below assumes three stages");
  for (int s = 0; s < ns; s += NS) {
    step(std::integral_constant<int, 0>(), s);
    if (s + 1 >= ns) break;
    step(std::integral_constant<int, 1>(), s + 1);
    if (s + 2 >= ns) break;
    step(std::integral_constant<int, 2>(), s + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped tail loads, before LDS is reused
  __syncthreads();

  // The k-groups' partial tiles are added in fixed order through LDS: KW = 2: a0 + a1;
  // KW = 4: (a0 + a2) + (a1 + a3).  Round r hands k-group giver's tile to k-group taker through
  // slot h (one 2 x wave-tile region per slot); straight-line code keeps acc in registers.
  float* red = reinterpret_cast<float*>(smem);
  constexpr int ROUNDS = KW == 4 ? 2 : 1;
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const bool last_round = r == ROUNDS - 1;
    const bool give = last_round ? kw == 1 : kw >= 2;
    const bool take = last_round ? kw == 0 : kw < 2;
    const int h = last_round ? 0 : (kw & 1);
    float* base = red + ((h * 2 + wn) * TM * TN) * 256 + 4 * lane;
    if (r > 0) __syncthreads();  // the previous round's tiles have been read
    if (give) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) *reinterpret_cast<float4_t*>(base + (i * TN + j) * 256) = acc[i][j];
    }
    __syncthreads();
    if (take) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] += *reinterpret_cast<const float4_t*>(base + (i * TN + j) * 256);
    }
  }

  // The MFMAs take the weights as their first operand, so each 16 x 16 block comes out
  // transposed: lane l, element r holds y row l%16, column 4*(l/16)+r (four consecutive columns:
  // one 8-byte LDS write per block in the epilogue; same products, same order, same bits).
  if (ws) {
    if (kw == 0) {
      float* part = ws + (size_t)split * M * N;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int row = m0 + 16 * i + l16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int col = n0 + 64 * wn + 16 * j + 4 * g + r;
            if (row < M && col < N) part[(size_t)row * N + col] = acc[i][j][r];
          }
        }
    }
    return;
  }
  // fp16 tile through LDS, then 16-byte row-major stores by all wavefronts.
  __syncthreads();  // the partial tiles have been read
  if (kw == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const half2_t lo = {(half_t)acc[i][j][0], (half_t)acc[i][j][1]};
        const half2_t hi = {(half_t)acc[i][j][2], (half_t)acc[i][j][3]};
        *reinterpret_cast<u32x2*>(smem + (16 * i + l16) * OUT_ROW + 2 * (64 * wn + 16 * j + 4 * g)) =
            u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
      }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < BM * BN / 8 / THREADS; ++q) {
    const int c = tid + THREADS * q;
    const int row = c >> 4, chunk = c & 15;
    const int gr = m0 + row, gc = n0 + 8 * chunk;
    if (gr < M && gc < N)
      *reinterpret_cast<u32x4*>(y + (size_t)gr * N + gc) = *reinterpret_cast<const u32x4*>(smem + row * OUT_ROW + 16 * chunk);
  }
}

// Wide DMA-fed tile: 192 x 256 per workgroup, 8 wavefronts as 2 x 4 wave tiles of 96 x 64, every
// wavefront over the whole 64-k stage (no k split, no partial-tile reduction), one workgroup per
// CU (99 KiB of stages and scale ring).  Per 64-k stage a CU moves 32 KiB from L2 into LDS for
// 192 x 256 outputs, against 40 KiB for the two 128 x 128 tiles of gemm_dma_kernel<2> (half the
// outputs): x, fp16 and the larger operand, is re-read from L2 once per 256 columns instead of
// once per 128.  Stage pipeline, swizzles, scale ring and counted waits are those of
// gemm_dma_kernel<2>.  MI355X, M = 2048, N = 5632, K = 2048 (242 tiles, one per CU): 52 us = 906
// TFLOPS against 56 us for the 128 x 128 tiles.  A tile alone on its CU takes 44 us (K = 2048), so
// the tile pays only where its count fills whole rounds of 256; gemm_plan weighs that.
struct WideCfg {
  static constexpr int BM = 192, BN = 256, BK = 64, NS = 3, WM = 2, WN = 4, WAVES = WM * WN, THREADS = 64 * WAVES;
  static constexpr int TM = 6, TN = 4;               // 16 x 16 blocks per wavefront
  static constexpr int A_ROW = BK * 2;               // 128 bytes of x per row and stage
  static constexpr int A_CH = BK / 8;                // 8 chunks of 16 bytes
  static constexpr int A_BYTES = BM * A_ROW;         // 24 KiB
  static constexpr int B_OFF = A_BYTES;
  static constexpr int B_ROW = BK / 2;               // 32 bytes of packed weights per row and stage
  static constexpr int B_CH = BK / 32;               // 2 chunks
  static constexpr int B_BYTES = BN * B_ROW;         // 8 KiB
  static constexpr int STAGE = B_OFF + B_BYTES;
  static constexpr int S_SLAB = BN * 4;              // [BN] 4-byte slots
  static constexpr int S_RING = NS * STAGE;
  static constexpr int RING_END = S_RING + NS * S_SLAB;
  static constexpr int OUT_ROW = BN * 2 + 16;
  static constexpr int SMEM = RING_END > BM * OUT_ROW ? RING_END : BM * OUT_ROW;
  static constexpr int A_DMA = A_BYTES / 1024 / WAVES;  // 3 x instructions per wavefront and stage
  static constexpr int kDmaPerStage = A_DMA + 1;        // + 1 packed
  static_assert(A_DMA * 1024 * WAVES == A_BYTES && B_BYTES == 1024 * WAVES, "DMA split");
  static_assert(SMEM <= 160 * 1024, "LDS");
};

__global__ __launch_bounds__(WideCfg::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_wide_kernel(const half_t* __restrict__ x, const uint32_t* __restrict__ packed,
                      const half_t* __restrict__ scales, half_t* __restrict__ y, float* __restrict__ ws, int M, int N,
                      int K, int log2_group, int stages_per_split, int splits, int tiles_m, int tiles_n,
                      int group_m) {
  using C = WideCfg;
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, NS = C::NS, THREADS = C::THREADS, TM = C::TM, TN = C::TN;
  constexpr int A_ROW = C::A_ROW, B_ROW = C::B_ROW, B_OFF = C::B_OFF, STAGE = C::STAGE, OUT_ROW = C::OUT_ROW;
  constexpr int kDmaPerStage = C::kDmaPerStage, A_DMA = C::A_DMA;
  __shared__ __attribute__((aligned(16))) unsigned char smem[C::SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave & 3;
  const int wm = wave >> 2;
  const int g = lane >> 4;
  const int l16 = lane & 15;

  int split, t;
  if (!gemm_job(tiles_m * tiles_n, splits, split, t)) return;
  const int band = group_m * tiles_n;
  const int bi = t / band;
  const int tb = t - bi * band;
  const int gm = min(group_m, tiles_m - bi * group_m);
  const int m0 = (bi * group_m + tb % gm) * BM;
  const int n0 = (tb / gm) * BN;

  const int nst = K / BK;
  const int st_begin = split * stages_per_split;
  const int last = min(nst, st_begin + stages_per_split) - 1;
  const int ns = last + 1 - st_begin;

  // XOR swizzles: x chunk c of row r at slot c ^ a_swz(r); packed chunk h of row r at h ^ b_swz(r).
  auto a_swz = [](int row) { return (row >> 1) & (C::A_CH - 1); };
  auto b_swz = [](int row) { return (row >> 3) & (C::B_CH - 1); };

  // DMA sources at k = 0.  x: A_DMA instructions of 1 KiB (8 rows) per wavefront; packed: one
  // of 1 KiB (32 rows).
  const half_t* a_src[A_DMA];
#pragma unroll
  for (int q = 0; q < A_DMA; ++q) {
    const int row = 8 * (A_DMA * wave + q) + (lane >> 3);
    a_src[q] = x + (size_t)min(m0 + row, M - 1) * K + 8 * ((lane & 7) ^ a_swz(row));
  }
  const int brow = 32 * wave + (lane >> 1);
  const uint32_t* b_src = packed + (size_t)min(n0 + brow, N - 1) * (K >> 3) + 4 * ((lane & 1) ^ b_swz(brow));
  const int groups = K >> log2_group;
  const half_t* s_src = scales + (size_t)min(n0 + 64 * wn + lane, N - 1) * groups;
  const uint32_t smem_base = (uint32_t)(uintptr_t)smem;

  const int log2_spg = log2_group - 6;  // log2(stages per group)
  auto starts_group = [&](int i) {
    const int st = st_begin + i;
    return i == 0 || (st <= last && (st & ((1 << log2_spg) - 1)) == 0);
  };
  auto group_of = [&](int i) { return ((st_begin + i) >> log2_spg) - (st_begin >> log2_spg); };
  auto issue = [&](int i, int buf) {
    const int st = min(st_begin + i, last);
    const int k0 = st * BK;
    const uint32_t base = __builtin_amdgcn_readfirstlane(smem_base + (uint32_t)(buf * STAGE));
#pragma unroll
    for (int q = 0; q < A_DMA; ++q) dma_16B(base + 1024 * (A_DMA * wave + q), a_src[q] + k0);
    dma_16B(base + B_OFF + 1024 * wave, b_src + (k0 >> 3));
    const bool sc = wm == 0 && starts_group(i);
    if (sc) {
      const uint32_t sbase = __builtin_amdgcn_readfirstlane(
          smem_base + (uint32_t)(C::S_RING + (group_of(i) % NS) * C::S_SLAB + 256 * wn));
      dma_u16(sbase, s_src + (k0 >> log2_group));
    }
    return sc;
  };
  auto wait_older = [&](bool newer_has_scales) {
    if (newer_has_scales)
      wait_vmcnt<kDmaPerStage + 1>();
    else
      wait_vmcnt<kDmaPerStage>();
  };

  float4_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Lane offsets: x row 96 wm + l16 (+16 per block), chunk 4 kk + g; packed row 64 wn + 16 j + l16,
  // chunk kk, dword g; scales column 64 wn + 16 j + l16.
  const int a_row0 = 96 * wm + l16;
  const int a_off0 = a_row0 * A_ROW + 16 * ((0 + g) ^ a_swz(a_row0));
  const int a_off1 = a_row0 * A_ROW + 16 * ((4 + g) ^ a_swz(a_row0));
  const int b_row0 = 64 * wn + l16;
  const int b_off0 = B_OFF + b_row0 * B_ROW + 16 * (0 ^ b_swz(b_row0)) + 4 * g;
  const int b_off1 = B_OFF + b_row0 * B_ROW + 16 * (1 ^ b_swz(b_row0)) + 4 * g;
  const int s_off = 4 * (64 * wn + l16);

  const UnpackConsts uc = unpack_consts();
  half8_t a[2][TM];
  uint32_t w[2][TN];
  half2_t s2[TN];
  auto read_frags = [&](int i, int buf) {
    const unsigned char* st = smem + buf * STAGE;
    const unsigned char* slab = smem + C::S_RING + (group_of(i) % NS) * C::S_SLAB;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      w[0][j] = *reinterpret_cast<const uint32_t*>(st + b_off0 + 16 * B_ROW * j);
      w[1][j] = *reinterpret_cast<const uint32_t*>(st + b_off1 + 16 * B_ROW * j);
      const half_t sc = *reinterpret_cast<const half_t*>(slab + s_off + 64 * j);
      s2[j] = half2_t{sc, sc};
    }
#pragma unroll
    for (int q = 0; q < TM; ++q) {
      a[0][q] = *reinterpret_cast<const half8_t*>(st + a_off0 + 16 * A_ROW * q);
      a[1][q] = *reinterpret_cast<const half8_t*>(st + a_off1 + 16 * A_ROW * q);
    }
  };

  issue(0, 0);
  wait_older(issue(1, 1));
  __syncthreads();
  // Stage pipeline of gemm_dma_kernel: stage i's fragments (both 32-k steps) are read at
  // iteration i, before the barrier after which stage i + 2's DMA may overwrite stage i - 1's
  // buffer; the scheduling barrier keeps the next stage's reads out of this stage's MFMAs.
  auto step = [&](auto buf_c, int s) {
    constexpr int CUR = decltype(buf_c)::value;
    __builtin_amdgcn_sched_barrier(0);
    read_frags(s, CUR);
    wait_older(issue(s + 2, (CUR + 2) % NS));
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const half8_t b = dequant8(w[kk][j], s2[j], uc);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a[kk][i], acc[i][j], 0, 0, 0);
      }
  };
  // Whole rounds of NS stages, then the remaining one or two: an exit in the middle of the
  // unrolled round made the compiler copy the accumulators between its copies of the round and
  // spill (256 VGPRs + 111 spilled against 236 without).
  static_assert(NS == 3, "the unrolled loop below assumes three stages");
  int s = 0;
  for (; s + NS <= ns; s += NS) {
    step(std::integral_constant<int, 0>(), s);
    step(std::integral_constant<int, 1>(), s + 1);
    step(std::integral_constant<int, 2>(), s + 2);
  }
  if (s < ns) step(std::integral_constant<int, 0>(), s);
  if (s + 1 < ns) step(std::integral_constant<int, 1>(), s + 1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // fp16 tile through LDS, then 16-byte row-major stores by all wavefronts (no split-K: ws unused).
  // The MFMAs take the weights as their first operand, so block (i, j) comes out transposed: lane
  // (g, l16) holds y[row 16 i + l16][columns 16 j + 4 g .. + 3], four consecutive fp16 that go to
  // LDS in one 8-byte write (a quarter of the writes of the row-per-element layout; the sums are
  // the same products added in the same order: bit-identical, 51.8 -> 50.6 us at M = 2048,
  // N = 5632, K = 2048).  Storing those 8 bytes straight to y instead measured 54.6 us.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const half2_t lo = {(half_t)acc[i][j][0], (half_t)acc[i][j][1]};
      const half2_t hi = {(half_t)acc[i][j][2], (half_t)acc[i][j][3]};
      *reinterpret_cast<u32x2*>(smem + (96 * wm + 16 * i + l16) * OUT_ROW + 2 * (64 * wn + 16 * j + 4 * g)) =
          u32x2{bit_cast<uint32_t>(lo), bit_cast<uint32_t>(hi)};
    }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < BM * BN / 8 / THREADS; ++q) {
    const int c = tid + THREADS * q;
    const int row = c >> 5, chunk = c & 31;
    const int gr = m0 + row, gc = n0 + 8 * chunk;
    if (gr < M && gc < N)
      *reinterpret_cast<u32x4*>(y + (size_t)gr * N + gc) = *reinterpret_cast<const u32x4*>(smem + row * OUT_ROW + 16 * chunk);
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

typedef void (*GemmFn)(const half_t*, const uint32_t*, const half_t*, half_t*, float*, int, int, int, int, int, int,
                       int, int, int);

struct TileEntry {
  int bm, bn, sk, threads;  // tile, k per stage, workgroup size
  // Cost terms of the dispatcher (see gemm_plan): workgroups resident per CU, and the time of
  // one round of resident workgroups, us_per_gmac * 1e-9 * BM * BN * k + us_fixed microseconds
  // for k = the split's k range.  0 blocks_per_cu: never chosen by the cost model.
  int blocks_per_cu;
  double us_per_gmac, us_fixed;
  GemmFn fn;
};

template <class C>
TileEntry entry(int blocks_per_cu, double us_per_gmac, double us_fixed) {
  return TileEntry{C::BM, C::BN, C::SK, C::THREADS, blocks_per_cu, us_per_gmac, us_fixed, gemm_kernel<C>};
}

// Tile table: index = GemmPlan::tile.  Cost terms: weighted least-squares fit (relative error)
// of the model in gemm_plan to graph-replayed timings of every tile and split count 1..12 over
// the TinyLlama and Qwen2.5 layer shapes, M = 48 .. 4096, weights rotated through more than
// twice the MALL, on MI355X (4,172 points, rms error 7.7%).  Over those shapes the plan's
// choices take 1.0074x the time of the best measured (tile, split) per shape (1.0122x without
// the 192 x 256 tile).
const TileEntry kTiles[] = {
    entry<TileCfg<64, 128, 1, 4, 1>>(0, 0.0, 0.0),         // 0: 64 x 128, 4 waves; 64-k stages (any K)
    entry<TileCfg<64, 128, 1, 4, 2>>(1, 702.21, 2.867),    // 1: 64 x 128, 8 waves (2 k-groups)
    TileEntry{128, 128, DmaCfg<2>::BK, DmaCfg<2>::THREADS, 2, 557.73, 5.918, gemm_dma_kernel<2>},  // 2: DMA 128 x 128
    entry<TileCfg<32, 128, 1, 4, 2>>(1, 999.91, 1.977),    // 3: 32 x 128, 8 waves (2 k-groups)
    entry<TileCfg<32, 64, 1, 2, 4>>(1, 1081.97, 2.779),    // 4: 32 x 64, 8 waves (4 k-groups, 256-k stages)
    entry<TileCfg<16, 64, 1, 2, 4>>(1, 1831.66, 2.117),    // 5: 16 x 64, 8 waves (4 k-groups, 256-k stages)
    TileEntry{128, 128, DmaCfg<4>::BK, DmaCfg<4>::THREADS, 1, 388.59, 7.265, gemm_dma_kernel<4>},  // 6: DMA, 8 waves
    TileEntry{192, 256, WideCfg::BK, WideCfg::THREADS, 1, 387.22, 4.351, gemm_wide_kernel},  // 7: DMA 192 x 256
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);
constexpr int kTile64 = 0, kDmaTile = 2, kWideTile = 7;
// Split-K costs one more launch plus the fp32 partials: kSplitUs + kSplitUsPerElem * splits * M * N
// (same fit), and is taken only when the model predicts it at least 10% faster.
constexpr double kSplitUs = 4.352, kSplitUsPerElem = 1.3750e-6, kSplitMargin = 0.9;
constexpr int kMaxSplits = 12;  // the largest split count the fit was measured on

GemmPlan plan_for(int K, int tile, int splits) {
  GemmPlan p;
  p.skinny = false;
  p.sk = SkinnyPlan{0, 0, 0, false, 0, 1};
  p.tile = tile;
  p.block_m = kTiles[tile].bm;
  p.block_n = kTiles[tile].bn;
  const int nst = K / kTiles[tile].sk;
  p.kt_per_split = ceil_div(nst, splits);
  p.splits = ceil_div(nst, p.kt_per_split);  // no empty splits
  return p;
}

}  // namespace

int gemm_num_tiles() { return kNumTiles; }

GemmPlan gemm_plan_with_tile(int M, int N, int K, int cu_count, int tile) {
  if (K % kTiles[tile].sk != 0) tile = kTile64;  // its 64-k stage divides every K here
  const int nst = K / kTiles[tile].sk;
  const long tiles = (long)ceil_div(N, kTiles[tile].bn) * ceil_div(M, kTiles[tile].bm);
  const long want = cu_count > 0 ? cu_count : 256;
  int splits = 1;
  if (tiles < want) {
    splits = (int)((want + tiles - 1) / tiles);
    const int max_splits = nst / 4 > 0 ? nst / 4 : 1;  // at least 4 stages per split
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
  }
  return plan_for(K, tile, splits);
}

// Kernel choice.
//   * The skinny kernel (one weight stream, K split inside the workgroup) for M <= 8, for
//     M <= 16 when K <= 4096, and up to M = 32 for small matrices (N*K <= 4.2M: TinyLlama q/o
//     and k/v) or grids of at most one workgroup per CU (TinyLlama gate/up, whose workgroups
//     take two column blocks, M = 20..32: 7.3 -> 6.0-7.0 us; q|k|v fused 7.1 -> 5.1-6.0 us; Qwen2.5
//     gate/up at 560 workgroups and TinyLlama gate|up fused at 704 stay faster tiled).  The rule
//     depends on N only through those last two clauses, so concatenated q|k|v or gate|up rows
//     take the same kernel as the separate layers for M <= 16 (bit-identical columns).
//   * Otherwise the tile and split-K factor that minimise a fitted cost: each XCD runs its
//     share of the tiles x splits workgroups in rounds of blocks_per_cu * cu_count / 8; a round
//     costs the tile entry's us_per_gmac * 1e-9 * BM * BN * (K / splits) + us_fixed, and
//     splitting adds its own cost (see kSplitUs).  Measured effect: small tiles (16 x 64,
//     32 x 64) at medium M and for narrow N (k/v projections), the DMA tile once it fills the
//     GPU, split-K only for long K.
GemmPlan gemm_plan(int M, int N, int K, int cu_count) {
  const int cus = cu_count > 0 ? cu_count : 256;
  const bool k128 = K % 128 == 0;
  const bool one_round = (long)ceil_div(N, 16 * skinny_col_blocks(N, cus)) <= cus;
  if (M <= kSkinnyMaxM && k128 && (M <= 8 || (K <= 4096 && (M <= 16 || (long)N * K <= 4200000L || one_round)))) {
    GemmPlan p = plan_for(K, kTile64, 1);
    p.skinny = true;
    p.sk = skinny_plan(M, N, K, cu_count);
    return p;
  }
  if (!k128) {  // K % 64 == 0 only: the 64-k-stage kernels
    const long dma_tiles = (long)ceil_div(M, 128) * ceil_div(N, 128);
    return gemm_plan_with_tile(M, N, K, cu_count, dma_tiles >= cus ? kDmaTile : kTile64);
  }
  int best_tile = kDmaTile, best_splits = 1;
  double best = 1e300;
  for (int tile = 0; tile < kNumTiles; ++tile) {
    const TileEntry& e = kTiles[tile];
    if (e.blocks_per_cu == 0 || K % e.sk != 0) continue;
    const int nst = K / e.sk;
    const long tiles = (long)ceil_div(M, e.bm) * ceil_div(N, e.bn);
    // >= 4 stages per split; the 192 x 256 tile never splits (its kernel writes no partials)
    const int max_splits = tile == kWideTile ? 1 : std::min(kMaxSplits, std::max(1, nst / 4));
    int prev = 0;
    for (int s = 1; s <= max_splits; ++s) {
      const int splits = ceil_div(nst, ceil_div(nst, s));
      if (splits == prev) continue;
      prev = splits;
      // Jobs are dealt evenly to the XCDs (gemm_job); each XCD runs its share in rounds.
      const long per_xcd = (tiles * splits + kXcds - 1) / kXcds;
      const long slots = std::max(1L, (long)e.blocks_per_cu * cus / kXcds);
      const long rounds = (per_xcd + slots - 1) / slots;
      double cost = rounds * (e.us_per_gmac * 1e-9 * e.bm * e.bn * ((double)K / splits) + e.us_fixed);
      if (splits > 1) cost = (cost + kSplitUs + kSplitUsPerElem * splits * (double)M * N) / kSplitMargin;
      if (cost < best) {
        best = cost;
        best_tile = tile;
        best_splits = splits;
      }
    }
  }
  return plan_for(K, best_tile, best_splits);
}

size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N) {
  return !p.skinny && p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

hipError_t gemm_launch(const GemmPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       void* ws, int M, int N, int K, int group_size, hipStream_t stream, const void* packed_r,
                       const void* scales_r) {
  if (p.skinny) {
    const bool blocked = packed_r != nullptr && scales_r != nullptr;
    return skinny_launch(p.sk, x, blocked ? packed_r : packed, blocked ? scales_r : scales, y, M, N, K, group_size,
                         blocked, stream);
  }
  const TileEntry& e = kTiles[p.tile];
  const int log2_group = group_size == 128 ? 7 : 6;
  const int tiles_m = ceil_div(M, e.bm);
  const int tiles_n = ceil_div(N, e.bn);
  const int grid_x = ceil_div(tiles_m * tiles_n * p.splits, kXcds) * kXcds;
  // Bands of M-tiles: one band per XCD when the M-tiles divide evenly, else single rows.
  int group_m = tiles_m / kXcds;
  if (group_m < 1) group_m = 1;
  float* part = p.splits > 1 ? static_cast<float*>(ws) : nullptr;
  hipLaunchKernelGGL(e.fn, dim3(grid_x), dim3(e.threads), 0, stream, static_cast<const half_t*>(x),
                     static_cast<const uint32_t*>(packed), static_cast<const half_t*>(scales),
                     static_cast<half_t*>(y), part, M, N, K, log2_group, p.kt_per_split, p.splits, tiles_m, tiles_n,
                     group_m);
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
