// Fused INT4 dequant GEMV for decode (M in [1, 8]) on gfx950, single- or multi-problem.
//
// y[m, n] = fp16( sum_c s[n, c/(G/32)] * sum_{k in chunk c} x[m, k] * q[n, k] ), fp32
// accumulation: the arithmetic of the reference's dequant_gemv_kernel<M>
// (csrc/gemm/dequant_gemv_kernel.cuh:38-109).  The scale is applied once per
// 32-k chunk (32 divides G), so W_hat is never rounded to fp16 here.
//
// One launch serves up to kMaxGemvGroup independent problems (x_p, W_p, y_p,
// N_p, K_p) with a common M and G (gemv_grouped_kernel), or one problem
// (gemv_kernel).  On MI355X an empty launch already costs ~1.6 us, longer than
// streaming a 2 MB layer, so independent decode linears should share a launch.
// A wavefront lives for one or a few memory round trips, so whatever it must
// read before its first weight load is on the critical path: the single-problem
// kernel takes every argument as a preloaded scalar, and the grouped kernel
// finds its problem from a preloaded header and then reads that problem's
// descriptor in one round of scalar loads (a problem lookup through two
// dependent scalar loads cost 0.3-0.5 us per launch).
//
// Mapping (bandwidth-first, no MFMA):
//   * A "chunk" is 32 consecutive k of one row: 16 B of packed words (one
//     dwordx4), 64 B of x and exactly one scale.
//   * x: every lane needs the 64 B of x of its chunk per 16 B of weights per
//     row, so per-lane x loads would move more bytes through the texture path
//     than the weights do.  When M*K fp16 values fit 20 KiB, each workgroup
//     copies x into LDS once with LDS-DMA (issued before the weight loads) and
//     the lanes read their x from there; otherwise every lane loads its own.
//   * Each wavefront owns R consecutive rows of one problem (R = 1 or 2; a
//     grouped launch that would not fit one resident round gives its largest
//     problems 3).  Lane l handles chunks l, l+64, ... of its rows, so a
//     wavefront-wide dwordx4 streams 1 KiB of a row contiguously.  Large
//     grouped launches at M = 1 also use flat rows (K = 1024 / 1536: several
//     short rows per full load, gemv_rows_flat) and deep rows (two long rows,
//     five blocks per round trip, gemv_rows_deep); both give every row the
//     bits gemv_rows gives it.
//   * A pass covers UU (1..4) consecutive 64-chunk blocks; UU is picked per
//     pass from the chunks left in the row, so a K=5632 row is one pass of
//     3 blocks and a K=2048 row one pass of 1, in the same launch.  Every load
//     of a pass (UU*R weight dwordx4, UU*R scales, x of the first XM rows) is
//     issued before any arithmetic: one memory round trip per pass.
//   * Unpack without magic numbers: a word masked with 0x000F000F holds the
//     nibble pair (k0, k1) as two fp16 subnormals u * 2^-24; masked with
//     0x00F000F0 the pair (k2, k3) becomes u * 2^-20; the word shifted right
//     by 8 gives (k4, k5) and (k6, k7) the same way.  v_dot2_f32_f16 on these
//     (exact products, fp32 sums) yields sum u*x up to a power of two, and
//     sum q*x = sum u*x - 8 * sum x, with sum x per chunk shared by all rows
//     of the wave.  5 bit operations and 4 dot2 per 8 weights per x row; the
//     accumulators stay scaled by 2^-24 until the final store.
//   * A DPP wave reduction (both rows of a two-row wave at once, after a
//     permlane32 swap) leaves the totals in lanes 31 / 63, which round to
//     fp16 (RNE) and store them.  Rows past N_p are clamped to row N_p - 1
//     for loading and never stored.
#include <limits.h>
#include <stddef.h>

#include "kf_device.h"
#include "kf_launch.h"

namespace kf {
namespace {

// x rows prefetched with the weights; larger M reads x per m inside the pass.
template <int M>
struct XPrefetch {
  static constexpr int value = M < 2 ? M : 2;
};

// Sum of the 32 x values of a chunk (fp32).
__device__ __forceinline__ float chunk_xsum(const u32x4 (&xv)[4]) {
  const half2_t one = {(half_t)1.0f, (half_t)1.0f};
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s0 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(xv[j][0]), one, s0, false);
    s1 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(xv[j][1]), one, s1, false);
    s0 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(xv[j][2]), one, s0, false);
    s1 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(xv[j][3]), one, s1, false);
  }
  return s0 + s1;
}

// The four masked forms of each word of a chunk: nibble pairs as fp16 subnormals.
struct ChunkNibbles {
  uint32_t t[4][4];  // [word][pair slot]: slots 0,2 hold u * 2^-24, slots 1,3 hold u * 2^-20
};

__device__ __forceinline__ void split_chunk(const u32x4& wv, ChunkNibbles& nb) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = wv[j], w8 = w >> 8;
    nb.t[j][0] = w & 0x000F000Fu;   // (k0, k1)
    nb.t[j][1] = w & 0x00F000F0u;   // (k2, k3) * 16
    nb.t[j][2] = w8 & 0x000F000Fu;  // (k4, k5)
    nb.t[j][3] = w8 & 0x00F000F0u;  // (k6, k7) * 16
  }
}

// 2^-24 * sum_{k in chunk} q[k] * x[k] for one row and one x row, in fp32, given
// xs8 = -8 * 2^-24 * sum x.  The dot products of the 2^-24-scaled pairs (k0,k1), (k4,k5)
// accumulate on top of xs8 and those of the 2^-20-scaled pairs (k2,k3), (k6,k7) separately,
// so A + B/16 = 2^-24 * (sum u*x - 8 * sum x) with q = u - 8.  The row accumulators stay in
// this 2^-24 domain (all values far above fp32's normal range limit) and are scaled by 2^24,
// exactly, before rounding to fp16.
__device__ __forceinline__ float chunk_dot(const ChunkNibbles& nb, const u32x4 (&xv)[4], float xs8) {
  float a = xs8, b = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a = __builtin_amdgcn_fdot2(bit_cast<half2_t>(nb.t[j][0]), bit_cast<half2_t>(xv[j][0]), a, false);
    b = __builtin_amdgcn_fdot2(bit_cast<half2_t>(nb.t[j][1]), bit_cast<half2_t>(xv[j][1]), b, false);
    a = __builtin_amdgcn_fdot2(bit_cast<half2_t>(nb.t[j][2]), bit_cast<half2_t>(xv[j][2]), a, false);
    b = __builtin_amdgcn_fdot2(bit_cast<half2_t>(nb.t[j][3]), bit_cast<half2_t>(xv[j][3]), b, false);
  }
  return fmaf(b, 0.0625f, a);
}

constexpr float kTwoPow24 = 16777216.0f;
constexpr float kMinus8TwoPowMinus24 = -4.76837158203125e-07f;  // -8 * 2^-24

// The workgroup's LDS copy of x (dynamic shared memory, sized per launch; plan.x_lds only).
extern __shared__ __attribute__((aligned(1024))) u32x4 gemv_x_lds[];

// Copies x (n16 16-byte pieces) into gemv_x_lds with LDS-DMA: wavefront w of a WPB-wavefront
// workgroup moves 1 KiB blocks w, w + WPB, ... straight from global memory to LDS, no registers.
// Lanes past the end re-read the last piece into the tail of the last block (inside the
// allocation, which the launcher rounds up to whole 1 KiB blocks).  Completion is awaited
// with vmcnt in gemv_pass.  `off`: byte offset of the destination in the LDS allocation.
template <int WPB = kGemvWavesPerBlock>
__device__ __forceinline__ void stage_x_lds(const half_t* x, int n16, int lane, uint32_t off = 0) {
  const uint32_t base = (uint32_t)(uintptr_t)gemv_x_lds + off;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blocks = (n16 + 63) >> 6;
  for (int b = wave; b < blocks; b += WPB) {
    const int idx = min(64 * b + lane, n16 - 1);
    asm volatile("global_load_lds_dwordx4 %1, off" ::"{m0}"(__builtin_amdgcn_readfirstlane(base + 1024u * b)),
                 "v"(x + 8 * idx)
                 : "memory");
  }
}

// Bytes of LDS one row of x takes (whole 1 KiB blocks, as the copy writes them).
__device__ __forceinline__ uint32_t x_row_lds_bytes(int K) { return (uint32_t)((2 * K + 1023) & ~1023); }

// Logical workgroup of this hardware workgroup.  The hardware deals workgroups to the 8 XCDs
// round robin (workgroup b runs on XCD b % 8); the logical ids give each XCD runs of kXcdRun
// consecutive workgroups, so consecutive rows - and each 128-byte line of y they store - stay
// in one XCD's L2 (7 TinyLlama linears at M = 1: 5.73 -> 5.66 us, Qwen2.5: 7.05 -> 6.85 us on
// MI355X; every problem still spreads evenly over the XCDs).  Launches pad their grid to whole
// runs of all XCDs (kXcdGrid workgroups); padded workgroups get ids past the real ones.
constexpr int kXcdRun = 8;
constexpr int kXcdGrid = 8 * kXcdRun;
__device__ __forceinline__ int xcd_run_block() {
  const int hb = blockIdx.x, j = hb >> 3;
  return (j / kXcdRun) * kXcdGrid + (hb & 7) * kXcdRun + (j % kXcdRun);
}

// Sum over the 64 lanes, returned to every lane: lanes i and i + 32 paired by permlane32_swap,
// then the DPP half-wave sum, read from lane 31.
__device__ __forceinline__ float wave_sum(float v) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float t = half_sum_lanes31_63(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 31));
}

// Fused prologues (one row of x, K halves), run by the whole workgroup on its LDS copies once
// they have landed; they end with a barrier.  LDS layout in 16-byte units, xb = one row's blocks:
// [0, xb) x, written here; [xb, 2 xb) the row copied in (x for RMSNorm, gate for SwiGLU);
// [2 xb, 3 xb) the second input (RMSNorm weight, up).  Writing x to its own region lets every
// wavefront read the whole input row while others already write, so one barrier suffices.
//   RMSNorm: x = fp16((x * rsqrt(sum(x^2) / K + eps)) * w); every wavefront sums the whole row in
//            the same order (per lane with v_dot2_f32_f16 on pairs, fp32, then across the
//            wavefront), so all agree.
//   SwiGLU:  x = fp16(float(fp16(silu(gate))) * up), silu(g) = g * rcp(1 + exp(-g)) with the
//            hardware exp and reciprocal (about 1 ulp of fp32 each, far below the fp16 rounding
//            that follows), and torch's two fp16 roundings of silu(gate) * up.
template <int PRO, int WPB>
__device__ __forceinline__ void x_prologue(int K, float eps) {
  const int tid = threadIdx.x;
  const int k8 = K >> 3;
  const int xb = (int)(x_row_lds_bytes(K) >> 4);
  const u32x4* in = gemv_x_lds + xb;
  const u32x4* in2 = gemv_x_lds + 2 * xb;
  if constexpr (PRO == kGemvProRmsNorm) {
    // Squares of pairs with dot2 (products exact in fp32): a quarter of the VALU of converting and
    // multiplying each element, and every wavefront of every workgroup repeats this sum.
    float s0 = 0.0f, s1 = 0.0f;
    for (int p = tid & 63; p < k8; p += 64) {
      const u32x4 v = in[p];
      s0 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(v[0]), bit_cast<half2_t>(v[0]), s0, false);
      s1 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(v[1]), bit_cast<half2_t>(v[1]), s1, false);
      s0 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(v[2]), bit_cast<half2_t>(v[2]), s0, false);
      s1 = __builtin_amdgcn_fdot2(bit_cast<half2_t>(v[3]), bit_cast<half2_t>(v[3]), s1, false);
    }
    const float rstd = rsqrtf(wave_sum(s0 + s1) / (float)K + eps);
    for (int p = tid; p < k8; p += 64 * WPB) {
      const u32x4 v = in[p], g = in2[p];
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t h = bit_cast<half2_t>(v[j]), gw = bit_cast<half2_t>(g[j]);
        const half2_t r = {(half_t)(((float)h[0] * rstd) * (float)gw[0]), (half_t)(((float)h[1] * rstd) * (float)gw[1])};
        o[j] = bit_cast<uint32_t>(r);
      }
      gemv_x_lds[p] = o;
    }
  } else {
    static_assert(PRO == kGemvProSwiGLU, "prologue kind");
    for (int p = tid; p < k8; p += 64 * WPB) {
      const u32x4 gv = in[p], uv = in2[p];
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t g = bit_cast<half2_t>(gv[j]), u = bit_cast<half2_t>(uv[j]);
        half2_t r;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float gf = (float)g[e];
          const half_t sh = (half_t)(gf * __builtin_amdgcn_rcpf(1.0f + __expf(-gf)));
          r[e] = (half_t)((float)sh * (float)u[e]);
        }
        o[j] = bit_cast<uint32_t>(r);
      }
      gemv_x_lds[p] = o;
    }
  }
  __syncthreads();
}

// RoPE + KV-cache epilogue (GemvRope).  tot: after the two-row reduction, lane 31 holds row
// row0's sum and lane 63 row row0 + step's (2^-24 domain); p is the token's position (PosLoad).
// For a q or k head, rows row0 and row0 + step are dims j and j + d/2; each is rounded to fp16
// and rotated with the roundings of torch's x * cos + swap_halves(x) * sin on fp16 tensors:
// fp16(fp16(x * cos) + partner * sin).  v rows are stored as they are.  A position outside the cache writes no cache entry and rotates
// with the tables' row 0 (the read stays in bounds).
__device__ __forceinline__ void rope_epilogue(float tot, int lane, int row0, int step, int N, half_t* y,
                                              const GemvRope& rc, int64_t p) {
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 31));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 63));
  if ((lane & 31) != 31) return;
  const int hi = lane >> 5;  // 0: row row0, 1: row row0 + step
  const int n = row0 + hi * step;
  if (n >= N) return;
  const int d = rc.head_dim;
  const int nrope = (rc.heads + rc.kv_heads) * d;
  const bool in_cache = p >= 0 && p < rc.max_seq;
  const size_t prow = (size_t)(in_cache ? p : 0) * d;
  if (row0 < nrope) {
    const int head = row0 / d;
    const int dim = row0 - head * d + hi * (d >> 1);
    const half_t self = (half_t)((hi ? b : a) * kTwoPow24), other = (half_t)((hi ? a : b) * kTwoPow24);
    const half_t c = static_cast<const half_t*>(rc.cos)[prow + dim], s = static_cast<const half_t*>(rc.sin)[prow + dim];
    const half_t t = (half_t)((float)self * (float)c);
    const half_t o = (half_t)((float)t + (float)other * (float)s);
    y[n] = o;
    if (head >= rc.heads && in_cache)
      static_cast<half_t*>(rc.cache_k)[((size_t)(head - rc.heads) * d + dim) * rc.max_seq + p] = o;
  } else {
    const half_t o = (half_t)((hi ? b : a) * kTwoPow24);
    y[n] = o;
    const int r = n - nrope, kvh = r / d;
    if (in_cache) static_cast<half_t*>(rc.cache_v)[((size_t)kvh * rc.max_seq + p) * d + (r - kvh * d)] = o;
  }
}

template <int R>
struct RowSet {
  const char* prow[R];  // packed row bases
  const char* srow[R];  // scale row bases
  const half_t* x;
  int K;
  int chunks;
  int scale_shift;
  float eps;  // RMSNorm prologue only
};

// The RoPE epilogue's position, read with a scalar load (it is constant during the launch) right
// after the first pass has issued its weight loads, so it arrives while the wavefront waits for
// the x copy instead of being a memory round trip before the epilogue's table reads (q|k|v with
// RMSNorm and RoPE 3.43 -> 3.33 us on MI355X; reading the cos / sin entries there as well measured
// 3.39).  The opaque move keeps the load from being hoisted to the start of the kernel, where the
// wait for it would hold back the weight loads.
struct PosLoad {
  const void* ptr;
  int64_t value;
  __device__ __forceinline__ void issue() {
    uintptr_t pp = (uintptr_t)ptr;
    asm volatile("" : "+s"(pp));
    value = *(const __attribute__((address_space(4))) int64_t*)pp;
  }
};

// One pass over UU consecutive 64-chunk blocks starting at chunk base cb (uniform).  With
// XLDS, x comes from the workgroup's LDS copy; the first pass waits for that copy: the only
// vector-memory loads issued after the copy are this pass's UU * R weight and UU * R scale
// loads, so vmcnt(2 * UU * R) means the copy has landed, and the barrier makes every
// wavefront's share visible to all.  pos (RoPE launches): issued there, see PosLoad.
template <int M, int R, int UU, bool XLDS, int PRO = kGemvProNone, int WPB = kGemvWavesPerBlock>
__device__ __forceinline__ void gemv_pass(const RowSet<R>& rs, int cb, int lane, float (&acc)[M][R], bool first,
                                          PosLoad* pos = nullptr) {
  constexpr int XM = XPrefetch<M>::value;
  u32x4 wv[UU][R];
  half_t sv[UU][R];
  u32x4 xv[UU][XM][4];
#pragma unroll
  for (int u = 0; u < UU; ++u) {
    // Clamped to the row's last chunk: always in bounds and one basic block
    // for all loads; lanes past the end re-read one line and are masked below.
    const uint32_t c = (uint32_t)min(cb + lane + 64 * u, rs.chunks - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      wv[u][r] = load_u32x4_stream(rs.prow[r] + 16u * c);
      sv[u][r] = *reinterpret_cast<const half_t*>(rs.srow[r] + 2u * (c >> rs.scale_shift));
    }
    if constexpr (!XLDS) {
#pragma unroll
      for (int m = 0; m < XM; ++m) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(rs.x + (size_t)m * rs.K + 32 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[u][m][j] = xp[j];
      }
    }
  }
  if constexpr (XLDS) {
    if (first) {
      if (pos) {  // a scalar load: vmcnt still counts only this pass's loads after the copy
        __builtin_amdgcn_sched_barrier(0);
        pos->issue();
      }
      wait_vmcnt<2 * UU * R>();
      __syncthreads();
      if constexpr (PRO != kGemvProNone) x_prologue<PRO, WPB>(rs.K, rs.eps);
    }
#pragma unroll
    for (int u = 0; u < UU; ++u) {
      const int xi = 4 * min(cb + lane + 64 * u, rs.chunks - 1);
#pragma unroll
      for (int m = 0; m < XM; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[u][m][j] = gemv_x_lds[m * (rs.K >> 3) + xi + j];
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep every load of the pass ahead of the math
  // With x in LDS, the chunk sums of x need nothing from the weight loads: computed here, ahead
  // of the first weight use, they run while those loads are in flight instead of after the
  // wait for them (same operations in the same order, so the same bits).  M <= 2 only: above
  // that the extra live sums cost occupancy in the unrolled kernels.  (A table of the sums
  // built once per workgroup in LDS does 4x less VALU work but costs a second barrier, and
  // measured slower: 7 TinyLlama linears 5.72 -> 5.79 us.)
  constexpr bool kEarlyXsum = XLDS && M <= 2;
  float xs8_early[UU][XM];
  if constexpr (kEarlyXsum) {
#pragma unroll
    for (int u = 0; u < UU; ++u)
#pragma unroll
      for (int m = 0; m < XM; ++m) xs8_early[u][m] = chunk_xsum(xv[u][m]) * kMinus8TwoPowMinus24;
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = 0; u < UU; ++u) {
    const int c = cb + lane + 64 * u;
    if (c < rs.chunks) {
      ChunkNibbles nb[R];
#pragma unroll
      for (int r = 0; r < R; ++r) split_chunk(wv[u][r], nb[r]);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        u32x4 xm[4];
        if (m < XM) {
#pragma unroll
          for (int j = 0; j < 4; ++j) xm[j] = xv[u][m < XM ? m : 0][j];
        } else if constexpr (XLDS) {
          const int xi = m * (rs.K >> 3) + 4 * c;
#pragma unroll
          for (int j = 0; j < 4; ++j) xm[j] = gemv_x_lds[xi + j];
        } else {
          const u32x4* xp = reinterpret_cast<const u32x4*>(rs.x + (size_t)m * rs.K + 32 * c);
#pragma unroll
          for (int j = 0; j < 4; ++j) xm[j] = xp[j];
        }
        const float xs8 = kEarlyXsum && m < XM ? xs8_early[u][m < XM ? m : 0] : chunk_xsum(xm) * kMinus8TwoPowMinus24;
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = fmaf((float)sv[u][r], chunk_dot(nb[r], xm, xs8), acc[m][r]);
      }
    }
  }
}

// Rows row0 .. row0 + R - 1 of one problem (the body both entry kernels share, so a problem
// gives the same bits whichever kernel runs it).  Rows past N are clamped to N - 1 for
// loading and never stored.
template <int M, int R, int UMAX, bool XLDS, int PRO = kGemvProNone, bool ROPE = false,
          int WPB = kGemvWavesPerBlock>
__device__ __forceinline__ void gemv_rows(const half_t* x, const uint32_t* packed, const half_t* scales,
                                          half_t* y, int N, int K, int scale_shift, int row0, int lane,
                                          const half_t* res = nullptr, const half_t* aux = nullptr,
                                          float eps = 0.0f, int row_step = 1, const GemvRope* rope = nullptr) {
  PosLoad posl{ROPE ? rope->pos : nullptr, 0};
  PosLoad* pos = ROPE ? &posl : nullptr;
  static_assert(PRO == kGemvProNone || (XLDS && M == 1), "fused prologues work on one row of x in LDS");
  static_assert(!ROPE || XLDS, "the position is read in the first pass's wait for the x copy");
  if constexpr (XLDS) {
    // The copies come before any other vector-memory load.
    if constexpr (PRO == kGemvProNone) {
      stage_x_lds(x, (M * K) >> 3, lane);
    } else {  // the row and the second input go past the x region, which the prologue writes
      stage_x_lds<WPB>(x, K >> 3, lane, x_row_lds_bytes(K));
      stage_x_lds<WPB>(aux, K >> 3, lane, 2 * x_row_lds_bytes(K));
    }
    // The first pass counts its own weight and scale loads as the only ones issued after the
    // copy.  Loads through __restrict__ arguments could legally be moved past the copy's
    // wait (into the lanes-in-range branch, after the barrier); passing the bases through
    // an opaque move makes them ordinary pointers, which stay ahead of the "memory" clobber,
    // and the casts restate that they address global memory (global_load, not flat_load).
    uintptr_t pa = (uintptr_t)packed, sa = (uintptr_t)scales;
    asm volatile("" : "+s"(pa), "+s"(sa));
    packed = (const uint32_t*)(const __attribute__((address_space(1))) uint32_t*)pa;
    scales = (const half_t*)(const __attribute__((address_space(1))) half_t*)sa;
  }
  RowSet<R> rs;
  rs.x = x;
  rs.K = K;
  rs.chunks = K >> 5;
  rs.scale_shift = scale_shift;
  rs.eps = eps;
  const size_t row_bytes = (size_t)K >> 1;
  const size_t srow_bytes = (size_t)(rs.chunks >> scale_shift) * 2;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const size_t n = (size_t)min(row0 + r * row_step, N - 1);
    rs.prow[r] = reinterpret_cast<const char*>(packed) + n * row_bytes;
    rs.srow[r] = reinterpret_cast<const char*>(scales) + n * srow_bytes;
  }

  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int cb = 0; cb < rs.chunks;) {
    const int left = rs.chunks - cb;  // uniform
    const bool first = cb == 0;
    if (UMAX >= 4 && left > 192) {
      gemv_pass<M, R, (UMAX >= 4 ? 4 : 1), XLDS, PRO, WPB>(rs, cb, lane, acc, first, pos);
      cb += 256;
    } else if (UMAX >= 3 && left > 128) {
      gemv_pass<M, R, (UMAX >= 3 ? 3 : 1), XLDS, PRO, WPB>(rs, cb, lane, acc, first, pos);
      cb += 192;
    } else if (UMAX >= 2 && left > 64) {
      gemv_pass<M, R, (UMAX >= 2 ? 2 : 1), XLDS, PRO, WPB>(rs, cb, lane, acc, first, pos);
      cb += 128;
    } else {
      gemv_pass<M, R, 1, XLDS, PRO, WPB>(rs, cb, lane, acc, first, pos);
      cb += 64;
    }
  }

  // Two rows in one reduction: v_permlane32_swap leaves (row a lanes 0-31, row b lanes 0-31) in
  // one register and (row a lanes 32-63, row b lanes 32-63) in the other, so their sum holds row
  // a in lanes 0-31 and row b in lanes 32-63, and lanes 31 and 63 end with the totals.  A
  // one-row wave pairs its row with itself, which adds in the same order, so a problem gives
  // the same bits for R = 1 and R = 2.
  // A third row is reduced on its own, paired with itself, and stored from lane 31.
  static_assert(R >= 1 && R <= 3, "rows per wave");
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[m][0]),
                                                     __float_as_uint(acc[m][R >= 2 ? 1 : 0]), false, false);
    acc[m][0] = half_sum_lanes31_63(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
    if constexpr (R == 3) {
      const auto s2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[m][2]), __float_as_uint(acc[m][2]), false,
                                                       false);
      acc[m][2] = half_sum_lanes31_63(__uint_as_float(s2[0]) + __uint_as_float(s2[1]));
    }
  }
  if constexpr (ROPE) {
    static_assert(M == 1 && R == 2, "the RoPE epilogue pairs two rows of one x row");
    rope_epilogue(acc[0][0], lane, row0, row_step, N, y, *rope, posl.value);
    return;
  }
  if ((lane & 31) == 31 && (R >= 2 || lane == 31)) {
    const int n = row0 + (lane >> 5);
    // With a residual: fp16(residual + fp16(result)), the two roundings of adding fp16 tensors.
    if (n < N) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        half_t o = (half_t)(acc[m][0] * kTwoPow24);
        if (res) o = (half_t)((float)res[(size_t)m * N + n] + (float)o);
        y[(size_t)m * N + n] = o;
      }
    }
    if (R == 3 && lane == 31 && row0 + 2 < N) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        half_t o = (half_t)(acc[m][R - 1] * kTwoPow24);
        if (res) o = (half_t)((float)res[(size_t)m * N + row0 + 2] + (float)o);
        y[(size_t)m * N + row0 + 2] = o;
      }
    }
  }
}

// Flat rows (M = 1, x in LDS): rows of C = K / 32 < 64 chunks, E = 64 - C dividing C
// (gemv_flat_rows).  The wavefront owns F = L + 1 rows row0 .. row0 + L, L = C / E, and issues L
// full 64-lane loads: load j holds row row0 + j in lanes 0 .. C - 1 (chunk = lane, as in
// gemv_rows) and chunks E j .. E j + E - 1 of the last row in lanes C .. 63.  Every lane computes
// fmaf(s, dot, 0) per chunk, the value gemv_rows' single pass leaves in that chunk's lane; the
// last row's values are then moved to lane = chunk (ds_bpermute) and each row is reduced with
// gemv_rows' two-row tree, so a row's result has the same bits as in gemv_rows.  A wavefront
// thus moves 1 KiB per load instead of 2 C * 8 bytes, and a K = 1536 problem needs a quarter
// fewer wavefronts than at three rows each.  Rows past N are clamped for loading, never stored.
template <int C>
__device__ __forceinline__ void gemv_rows_flat(const half_t* x, const uint32_t* packed, const half_t* scales,
                                               half_t* y, int N, int scale_shift, int row0, int lane) {
  constexpr int E = 64 - C, L = C / E, F = L + 1, K = 32 * C;
  static_assert(E * L == C && F % 2 == 0 && L <= 3 && (E & (E - 1)) == 0, "flat rows: E, a power of two, divides C");
  stage_x_lds(x, K >> 3, lane);
  // As in gemv_rows: the weight and scale bases pass through an opaque move so their loads
  // stay after the copy, which the wait below counts on.
  uintptr_t pa = (uintptr_t)packed, sa = (uintptr_t)scales;
  asm volatile("" : "+s"(pa), "+s"(sa));
  const char* pk = (const char*)(const __attribute__((address_space(1))) char*)pa;
  const char* sc = (const char*)(const __attribute__((address_space(1))) char*)sa;

  const bool extra = lane >= C;  // lanes carrying the last row
  const int ce = lane - C;       // their chunk offset within each load's E chunks
  const size_t srow_bytes = (size_t)(C >> scale_shift) * 2;
  const int nlast = min(row0 + L, N - 1);
  u32x4 wv[L];
  half_t sv[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    const size_t n = (size_t)(extra ? nlast : min(row0 + j, N - 1));
    const uint32_t c = (uint32_t)(extra ? E * j + ce : lane);
    wv[j] = load_u32x4_stream(pk + n * (16 * C) + 16u * c);
    sv[j] = *reinterpret_cast<const half_t*>(sc + n * srow_bytes + 2u * (c >> scale_shift));
  }
  wait_vmcnt<2 * L>();  // the x copy has landed (only this wavefront's 2 L loads follow it)
  __syncthreads();

  // x of a lane's chunk: lanes below C see chunk `lane` in every load, the extra lanes chunk
  // E j + ce of load j, read into the same registers under their own mask.
  u32x4 xm[4];
  {
    const int xi = 4 * (extra ? ce : lane);
#pragma unroll
    for (int q = 0; q < 4; ++q) xm[q] = gemv_x_lds[xi + q];
  }
  // Chunk sums: lane t < C sums chunk t, once; in load j > 0 the extra lanes take the sum of
  // their chunk E j + ce from lane E j + ce (the same value, fetched instead of recomputed:
  // Qwen2.5's 7 linears 6.57 -> 6.39 us on MI355X).
  const float xs_own = chunk_xsum(xm) * kMinus8TwoPowMinus24;
  float prod[L];
#pragma unroll
  for (int j = 0; j < L; ++j) {
    float xs8 = xs_own;
    if (j > 0) {
      const float moved =
          __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (E * j + (ce & (E - 1))), __float_as_int(xs_own)));
      if (extra) {
        xs8 = moved;
        const int xi = 4 * (E * j + ce);
#pragma unroll
        for (int q = 0; q < 4; ++q) xm[q] = gemv_x_lds[xi + q];
      }
    }
    ChunkNibbles nb;
    split_chunk(wv[j], nb);
    prod[j] = fmaf((float)sv[j], chunk_dot(nb, xm, xs8), 0.0f);
  }

  // Row values in chunk order: rows 0 .. L - 1 in lanes 0 .. C - 1 as loaded; the last row's
  // chunk t comes from load t / E, lane C + t % E.  Lanes C .. 63 hold 0 for every row, as the
  // lanes past a row's chunks do in gemv_rows.
  float v[F];
#pragma unroll
  for (int j = 0; j < L; ++j) v[j] = extra ? 0.0f : prod[j];
  {
    const int src = 4 * (C + lane % E);
    const int jl = lane / E;
    float last = 0.0f;
#pragma unroll
    for (int j = 0; j < L; ++j) {
      const float moved = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(prod[j])));
      if (jl == j) last = moved;
    }
    v[L] = extra ? 0.0f : last;
  }
#pragma unroll
  for (int p = 0; p < F / 2; ++p) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2 * p]), __float_as_uint(v[2 * p + 1]),
                                                     false, false);
    const float tot = half_sum_lanes31_63(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
    const int n = row0 + 2 * p + (lane >> 5);
    if ((lane & 31) == 31 && n < N) y[n] = (half_t)(tot * kTwoPow24);
  }
}

// Deep rows (M = 1, x in LDS): rows row0 and row0 + 1, of B = ceil(K / 2048) 64-chunk blocks each,
// as 2 B (row, block) items - the first row's blocks, then the second's - loaded P at a time,
// every load of a pass issued before its math.  A pass holds its weights and scales (5
// registers per item) and one chunk of x at a time.  Each row's chunks are added in gemv_rows'
// order (lane l: chunks l, l + 64, ..., each as fmaf(s, dot, acc)) and the pair is reduced with
// its two-row tree, so every row has the bits gemv_rows gives it.  Two rows per wavefront halve
// the workgroups, and with them the copies of x (17.5 KiB each at K = 8960), against one row
// per wavefront for the same two round trips (Qwen2.5's 7 linears 6.46-6.51 -> 6.31-6.34 us on
// MI355X; three rows per wavefront in two or three passes measured slower).
template <int P>
__device__ __forceinline__ void gemv_rows_deep(const half_t* x, const uint32_t* packed, const half_t* scales,
                                               half_t* y, int N, int K, int scale_shift, int row0, int lane) {
  stage_x_lds(x, K >> 3, lane);
  uintptr_t pa = (uintptr_t)packed, sa = (uintptr_t)scales;  // see gemv_rows
  asm volatile("" : "+s"(pa), "+s"(sa));
  const char* pk = (const char*)(const __attribute__((address_space(1))) char*)pa;
  const char* sc = (const char*)(const __attribute__((address_space(1))) char*)sa;
  const int chunks = K >> 5;
  const int nb = (chunks + 63) >> 6;
  const int items = 2 * nb;
  const size_t srow_bytes = (size_t)((chunks >> scale_shift) * 2);
  const size_t na = (size_t)min(row0, N - 1), nr = (size_t)min(row0 + 1, N - 1);  // past N: clamped, not stored
  const char* prow0 = pk + na * (size_t)(K >> 1);
  const char* prow1 = pk + nr * (size_t)(K >> 1);
  const char* srow0 = sc + na * srow_bytes;
  const char* srow1 = sc + nr * srow_bytes;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int i0 = 0; i0 < items; i0 += P) {  // uniform
    u32x4 wv[P];
    half_t sv[P];
#pragma unroll
    for (int u = 0; u < P; ++u) {
      // Items past the end load the last item again (masked below), so every pass issues P
      // loads of each kind: the first pass's wait counts on that.
      const int it = min(i0 + u, items - 1);
      const bool second = it >= nb;
      const uint32_t c = (uint32_t)min(64 * (second ? it - nb : it) + lane, chunks - 1);
      wv[u] = load_u32x4_stream((second ? prow1 : prow0) + 16u * c);
      sv[u] = *reinterpret_cast<const half_t*>((second ? srow1 : srow0) + 2u * (c >> scale_shift));
    }
    if (i0 == 0) {
      wait_vmcnt<2 * P>();  // the x copy has landed (only this pass's 2 P loads follow it)
      __syncthreads();
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the pass ahead of the math
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int it = i0 + u;
      const bool second = it >= nb;
      const int c = 64 * (second ? it - nb : it) + lane;
      const int xi = 4 * min(c, chunks - 1);
      u32x4 xm[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) xm[q] = gemv_x_lds[xi + q];
      const float xs8 = chunk_xsum(xm) * kMinus8TwoPowMinus24;
      // Every lane computes (past the row's end on its clamped chunk) and keeps the sum only in
      // range, with selects: a branch here would let a pass end with loads never waited for, and
      // the compiler would then wait for all loads, the x copy included, before the next pass's
      // first weights.
      ChunkNibbles nbl;
      split_chunk(wv[u], nbl);
      const bool in_range = it < items && c < chunks;
      const float next = fmaf((float)sv[u], chunk_dot(nbl, xm, xs8), second ? acc1 : acc0);
      acc0 = in_range && !second ? next : acc0;
      acc1 = in_range && second ? next : acc1;
    }
  }
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc0), __float_as_uint(acc1), false, false);
  const float tot = half_sum_lanes31_63(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
  const int n = row0 + (lane >> 5);
  if ((lane & 31) == 31 && n < N) y[n] = (half_t)(tot * kTwoPow24);
}

// One problem: every argument is a scalar kernel argument, preloaded into SGPRs, so a
// wavefront issues its weight loads without waiting on any scalar memory access.  With
// XLDS every wavefront takes part in the x copy and its barrier, so none leaves early.
template <int M, int R, int UMAX, bool XLDS>
__global__ __launch_bounds__(64 * kGemvWavesPerBlock) void gemv_kernel(const half_t* __restrict__ x,
                                                                     const uint32_t* __restrict__ packed,
                                                                     const half_t* __restrict__ scales,
                                                                     half_t* __restrict__ y, int N, int K,
                                                                     int scale_shift) {
  const int lane = threadIdx.x & 63;
  const int lb = xcd_run_block();
  if (lb * kGemvWavesPerBlock * R >= N) return;  // a padded workgroup: all of its wavefronts leave
  const int row0 = (lb * kGemvWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  if (!XLDS && row0 >= N) return;  // past the last row
  gemv_rows<M, R, UMAX, XLDS>(x, packed, scales, y, N, K, scale_shift, row0, lane);
}

// One problem at M = 1 with a prologue on x (GemvPrologue) and/or a residual: gemv_kernel with
// x in LDS, whose copy the prologue transforms before the first product.  y may alias res.
// Workgroups of gemv_fused_waves_per_block(PRO) wavefronts.
template <int R, int UMAX, int PRO>
__global__ __launch_bounds__(64 * gemv_fused_waves_per_block(PRO)) void gemv_fused_kernel(
    const half_t* __restrict__ x, const uint32_t* __restrict__ packed, const half_t* __restrict__ scales, half_t* y,
    int N, int K, int scale_shift, const half_t* res, const half_t* __restrict__ aux, float eps) {
  constexpr int WPB = gemv_fused_waves_per_block(PRO);
  const int lane = threadIdx.x & 63;
  const int lb = xcd_run_block();
  if (lb * WPB * R >= N) return;  // a padded workgroup: all of its wavefronts leave
  const int row0 = (lb * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  gemv_rows<1, R, UMAX, true, PRO, false, WPB>(x, packed, scales, y, N, K, scale_shift, row0, lane, res, aux, eps);
}

// The q|k|v decode GEMV with the RoPE + KV-cache epilogue (GemvRope), optionally an RMSNorm
// prologue.  Wavefront w < (heads + kv_heads) * d / 2 owns dims j, j + d / 2 of head w / (d / 2);
// the rest own two consecutive v rows.  Workgroups of gemv_fused_waves_per_block(PRO) wavefronts.
template <int UMAX, int PRO>
__global__ __launch_bounds__(64 * gemv_fused_waves_per_block(PRO)) void gemv_qkv_rope_kernel(
    const half_t* __restrict__ x, const uint32_t* __restrict__ packed, const half_t* __restrict__ scales, half_t* y,
    int N, int K, int scale_shift, const half_t* __restrict__ aux, float eps, const GemvRope rope) {
  constexpr int WPB = gemv_fused_waves_per_block(PRO);
  const int lane = threadIdx.x & 63;
  const int lb = xcd_run_block();
  if (lb * WPB * 2 >= N) return;  // a padded workgroup: all of its wavefronts leave
  const int w = lb * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half_d = rope.head_dim >> 1;
  const int nwr = (rope.heads + rope.kv_heads) * half_d;
  int row0, step;
  if (w < nwr) {
    const int head = w / half_d;
    row0 = head * rope.head_dim + (w - head * half_d);
    step = half_d;
  } else {
    row0 = 2 * nwr + 2 * (w - nwr);
    step = 1;
  }
  gemv_rows<1, 2, UMAX, true, PRO, true, WPB>(x, packed, scales, y, N, K, scale_shift, row0, lane, nullptr, aux,
                                              eps, step, &rope);
}

// Several problems.  b1 .. b8: first global wavefront of problems 1 .. 8 (ascending; the
// total after the last problem, then INT_MAX), so the problem index is the number of bounds
// at or below the wavefront's index: eight subtract-and-shift steps on preloaded SGPRs.  The
// problem's slot (pointers, sizes, first wavefront) is then read in one round of scalar
// loads; the pointers are global memory, which the casts state so the loads stay global_load
// rather than flat_load.  With XLDS the launcher starts every problem on a workgroup
// boundary, so a workgroup serves one problem and one x.
template <int M, int R, int UMAX, bool XLDS>
__global__ __launch_bounds__(64 * kGemvWavesPerBlock) void gemv_grouped_kernel(int count, int scale_shift, int b1,
                                                                             int b2, int b3, int b4, int b5, int b6,
                                                                             int b7, int b8,
                                                                             const GemvTable table) {
  const int lane = threadIdx.x & 63;
  const int gwave = xcd_run_block() * kGemvWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // gwave - b >> 31 is 1 exactly when gwave < b (both in [0, 2^31)); padded workgroups lie past
  // the last problem's waves.
  const unsigned g = (unsigned)gwave;
  const int p = kMaxGemvGroup - (int)(((g - b1) >> 31) + ((g - b2) >> 31) + ((g - b3) >> 31) + ((g - b4) >> 31) +
                                      ((g - b5) >> 31) + ((g - b6) >> 31) + ((g - b7) >> 31) + ((g - b8) >> 31));
  if (p >= count) return;  // past the last problem's waves (whole workgroups)

  typedef unsigned long long u64x4 __attribute__((ext_vector_type(4)));
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  static_assert(sizeof(GemvSlot) == 48 && offsetof(GemvSlot, N) == 32 && offsetof(GemvSlot, wave0) == 40,
                "slot layout");
  const char* desc = reinterpret_cast<const char*>(&table.slot[p]);
  const u64x4 ptr = *reinterpret_cast<const u64x4*>(desc);  // x, packed, scales, y
  const i32x4 nkw = *reinterpret_cast<const i32x4*>(desc + 32);  // N, K, wave0, rows per wave
  typedef const __attribute__((address_space(1))) half_t* gh_t;
  typedef const __attribute__((address_space(1))) uint32_t* gu_t;
  typedef __attribute__((address_space(1))) half_t* gy_t;
  if constexpr (R == kGemvRowsMixed || R == kGemvRowsShaped) {
    // Mixed launch: each problem carries its own rows per wavefront (2 or 3; in the shaped
    // launch also flat or deep rows) in the slot.
    if constexpr (R == kGemvRowsShaped) {
      static_assert(M == 1 && XLDS, "flat and deep rows: one row of x in LDS");
      if (nkw.w > kGemvFlat) {
        if (nkw.y == 32 * 48)
          gemv_rows_flat<48>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y, (const half_t*)(gh_t)ptr.z,
                             (half_t*)(gy_t)ptr.w, nkw.x, scale_shift, (gwave - nkw.z) * 4, lane);
        else
          gemv_rows_flat<32>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y, (const half_t*)(gh_t)ptr.z,
                             (half_t*)(gy_t)ptr.w, nkw.x, scale_shift, (gwave - nkw.z) * 2, lane);
        return;
      }
      if (nkw.w == kGemvDeep) {
        gemv_rows_deep<kGemvDeepPass>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y,
                                      (const half_t*)(gh_t)ptr.z, (half_t*)(gy_t)ptr.w, nkw.x, nkw.y, scale_shift,
                                      (gwave - nkw.z) * 2, lane);
        return;
      }
    }
    if (nkw.w == 3)
      gemv_rows<M, 3, UMAX, XLDS>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y,
                                  (const half_t*)(gh_t)ptr.z, (half_t*)(gy_t)ptr.w, nkw.x, nkw.y, scale_shift,
                                  (gwave - nkw.z) * 3, lane);
    else
      gemv_rows<M, 2, UMAX, XLDS>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y,
                                  (const half_t*)(gh_t)ptr.z, (half_t*)(gy_t)ptr.w, nkw.x, nkw.y, scale_shift,
                                  (gwave - nkw.z) * 2, lane);
  } else {
    gemv_rows<M, R, UMAX, XLDS>((const half_t*)(gh_t)ptr.x, (const uint32_t*)(gu_t)ptr.y,
                                (const half_t*)(gh_t)ptr.z, (half_t*)(gy_t)ptr.w, nkw.x, nkw.y, scale_shift,
                                (gwave - nkw.z) * R, lane);
  }
}

typedef void (*GemvFn)(const half_t*, const uint32_t*, const half_t*, half_t*, int, int, int);
typedef void (*GemvGroupedFn)(int, int, int, int, int, int, int, int, int, int, const GemvTable);

template <int M, int R, int U, bool XLDS>
struct GemvKernels {
  static constexpr GemvFn single = gemv_kernel<M, R, U, XLDS>;
  static constexpr GemvGroupedFn grouped = gemv_grouped_kernel<M, R, U, XLDS>;
};

template <bool GROUPED, bool XLDS, int M, int R>
void* pick_u(int U) {
  switch (U) {
    case 1: return GROUPED ? (void*)GemvKernels<M, R, 1, XLDS>::grouped : (void*)GemvKernels<M, R, 1, XLDS>::single;
    case 2: return GROUPED ? (void*)GemvKernels<M, R, 2, XLDS>::grouped : (void*)GemvKernels<M, R, 2, XLDS>::single;
    case 3: return GROUPED ? (void*)GemvKernels<M, R, 3, XLDS>::grouped : (void*)GemvKernels<M, R, 3, XLDS>::single;
    default: return GROUPED ? (void*)GemvKernels<M, R, 4, XLDS>::grouped : (void*)GemvKernels<M, R, 4, XLDS>::single;
  }
}

// Grouped launch with 2 or 3 rows per wavefront per problem (M <= 2 only).
template <bool XLDS, int M>
void* pick_mixed(int U) {
  constexpr int RM = kGemvRowsMixed;
  switch (U) {
    case 1: return (void*)gemv_grouped_kernel<M, RM, 1, XLDS>;
    case 2: return (void*)gemv_grouped_kernel<M, RM, 2, XLDS>;
    case 3: return (void*)gemv_grouped_kernel<M, RM, 3, XLDS>;
    default: return (void*)gemv_grouped_kernel<M, RM, 4, XLDS>;
  }
}

template <bool GROUPED, bool XLDS, int M>
void* pick_r(int R, int U) {
  if (R == kGemvRowsMixed) {
    if constexpr (GROUPED && M <= 2) return pick_mixed<XLDS, M>(U);
    return nullptr;  // the plan never asks for it
  }
  if (R == kGemvRowsShaped) {  // the plan gives it unroll 1, M = 1 and x in LDS only
    if constexpr (GROUPED && M == 1 && XLDS) return (void*)gemv_grouped_kernel<1, kGemvRowsShaped, 1, true>;
    return nullptr;
  }
  return R == 1 ? pick_u<GROUPED, XLDS, M, 1>(U) : pick_u<GROUPED, XLDS, M, 2>(U);
}

template <bool GROUPED, bool XLDS>
void* pick_m(int M, int R, int U) {
  switch (M) {
    case 1: return pick_r<GROUPED, XLDS, 1>(R, U);
    case 2: return pick_r<GROUPED, XLDS, 2>(R, U);
    case 3: return pick_r<GROUPED, XLDS, 3>(R, U);
    case 4: return pick_r<GROUPED, XLDS, 4>(R, U);
    case 5: return pick_r<GROUPED, XLDS, 5>(R, U);
    case 6: return pick_r<GROUPED, XLDS, 6>(R, U);
    case 7: return pick_r<GROUPED, XLDS, 7>(R, U);
    default: return pick_r<GROUPED, XLDS, 8>(R, U);
  }
}

template <bool GROUPED>
void* pick(int M, const GemvPlan& plan) {
  return plan.x_lds ? pick_m<GROUPED, true>(M, plan.rows_per_wave, plan.unroll)
                    : pick_m<GROUPED, false>(M, plan.rows_per_wave, plan.unroll);
}

// Dynamic LDS of the x copy: whole 1 KiB blocks of M * K fp16 values.
size_t x_lds_bytes(int M, int K) { return (size_t)ceil_div(M * K * 2, 1024) * 1024; }

// A grid of `blocks` workgroups padded to whole XCD runs (see xcd_run_block).
int xcd_grid(int blocks) { return ceil_div(blocks, kXcdGrid) * kXcdGrid; }

typedef void (*GemvFusedFn)(const half_t*, const uint32_t*, const half_t*, half_t*, int, int, int, const half_t*,
                            const half_t*, float);

template <int R, int PRO>
GemvFusedFn pick_fused_u(int U) {
  switch (U) {
    case 1: return gemv_fused_kernel<R, 1, PRO>;
    case 2: return gemv_fused_kernel<R, 2, PRO>;
    case 3: return gemv_fused_kernel<R, 3, PRO>;
    default: return gemv_fused_kernel<R, 4, PRO>;
  }
}

template <int PRO>
GemvFusedFn pick_fused_r(int R, int U) {
  return R == 1 ? pick_fused_u<1, PRO>(U) : (R == 2 ? pick_fused_u<2, PRO>(U) : pick_fused_u<3, PRO>(U));
}

GemvFusedFn pick_fused(int prologue, int R, int U) {
  switch (prologue) {
    case kGemvProRmsNorm: return pick_fused_r<kGemvProRmsNorm>(R, U);
    case kGemvProSwiGLU: return pick_fused_r<kGemvProSwiGLU>(R, U);
    default: return pick_fused_r<kGemvProNone>(R, U);
  }
}

typedef void (*GemvRopeFn)(const half_t*, const uint32_t*, const half_t*, half_t*, int, int, int, const half_t*, float,
                           const GemvRope);

template <int PRO>
GemvRopeFn pick_rope_u(int U) {
  switch (U) {
    case 1: return gemv_qkv_rope_kernel<1, PRO>;
    case 2: return gemv_qkv_rope_kernel<2, PRO>;
    case 3: return gemv_qkv_rope_kernel<3, PRO>;
    default: return gemv_qkv_rope_kernel<4, PRO>;
  }
}

// Dynamic LDS of the fused kernel: x, plus the prologue's two inputs.
size_t fused_lds_bytes(int K, int prologue) {
  const size_t xb = x_lds_bytes(1, K);
  return prologue == kGemvProNone ? xb : 3 * xb;
}

}  // namespace

GemvPlan gemv_plan(int M, const int* N, const int* K, int count, int cu_count) {
  GemvPlan p;
  const long cus = cu_count > 0 ? cu_count : 256;
  long rows = 0;
  int max_chunks = 0, max_k = 0;
  for (int i = 0; i < count; ++i) {
    rows += N[i];
    if (K[i] / 32 > max_chunks) max_chunks = K[i] / 32;
    if (K[i] > max_k) max_k = K[i];
  }
  // Two rows per wave once that still leaves >= 8 wavefronts per CU
  // (measured on MI355X: q/o 2048x2048 alone prefers one row, gate 5632x2048
  // and every grouped decode set prefer two; four is always slower).
  p.rows_per_wave = (rows + 1) / 2 >= 8 * cus ? 2 : 1;
  const long waves = (rows + p.rows_per_wave - 1) / p.rows_per_wave;
  // Deep passes (several 64-chunk blocks per round trip) pay off only when
  // the launch has few wavefronts: down 2048x5632 alone is fastest with 3
  // blocks per pass, the 7-layer group with 1 (the registers of a deep pass
  // cost more occupancy than the extra memory parallelism returns).
  const int blocks = ceil_div(max_chunks, 64);
  const int u_max = M <= 2 ? 4 : (M <= 4 ? 2 : 1);
  p.unroll = waves >= 12 * cus ? 1 : (blocks < u_max ? blocks : u_max);
  // Per-lane x loads move 64 bytes of x through the texture path for every 16 bytes of a
  // row; one LDS copy per workgroup removes that traffic (7 TinyLlama linears at M = 1:
  // 6.9 -> 6.3 us on MI355X) wherever x fits the LDS budget.  The budget is what leaves every
  // workgroup of the launch resident: 20 KiB for launches of eight or more workgroups per CU,
  // the CU's 160 KiB shared among fewer.  The larger copies take M = 2-8 rows of long x into
  // LDS in single-problem launches (same bits; MI355X, TinyLlama down M = 2 / 3 / 4:
  // 5.24 / 6.41 / 7.64 -> 3.86 / 5.26 / 6.11 us, Qwen2.5 down 7.66 / 9.37 / 11.58 -> 5.67 /
  // 7.20 / 8.54 us, q/o and gate at M = 8 -25%).
  const long wgs_per_cu = ((waves + kGemvWavesPerBlock - 1) / kGemvWavesPerBlock + cus - 1) / cus;
  const long budget = std::max<long>(kGemvMaxLdsX, kLdsPerCu / wgs_per_cu / 1024 * 1024);
  const size_t xb = x_lds_bytes(M, max_k);
  p.x_lds = xb <= (size_t)budget;
  for (int i = 0; i < count; ++i) p.rows[i] = p.rows_per_wave;
  // Large grouped launches (two rows per wavefront) shape each problem's rows:
  //   * M = 1, x in LDS: K = 1024 / 1536 problems take flat rows (full 1 KiB loads), and rows
  //     longer than one 64-chunk block deep rows (two per wavefront, kGemvDeepPass blocks per
  //     round trip), if the launch then still fits the wave slots (Qwen2.5's 7 linears at
  //     M = 1: 6.85 -> 6.31 us on MI355X; TinyLlama's do not fit, and keep their plan).
  //   * A launch whose wavefronts outnumber the wave slots (8 per SIMD) runs its last
  //     wavefronts in a second round, a full memory round trip after the others.  The largest
  //     two-row problems then take three rows per wavefront, just enough of them for the grid
  //     to fit (7 TinyLlama linears: 8,960 two-row wavefronts for 8,192 slots).
  if (p.rows_per_wave == 2 && count > 1 && M <= 2) {
    auto waves_of = [&](int i) {
      const int r = gemv_entry_rows(p.rows[i]);
      long w = (N[i] + r - 1) / r;
      if (p.x_lds) w = (w + kGemvWavesPerBlock - 1) / kGemvWavesPerBlock * kGemvWavesPerBlock;
      return w;
    };
    auto total_waves = [&]() {
      long t = 0;
      for (int i = 0; i < count; ++i) t += waves_of(i);
      return t;
    };
    if (M == 1 && p.x_lds) {
      for (int i = 0; i < count; ++i) {
        const int f = gemv_flat_rows(K[i]);
        if (f > 0) p.rows[i] = kGemvFlat + f;
      }
      bool deep = false;
      for (int i = 0; i < count; ++i)
        if (K[i] > 2048 && p.rows[i] == 2) {
          p.rows[i] = kGemvDeep;
          deep = true;
        }
      if (deep && total_waves() > 32L * cus) {
        for (int i = 0; i < count; ++i)
          if (p.rows[i] == kGemvDeep) p.rows[i] = 2;
      }
    }
    long slots = 32L * cus;
    if (!p.x_lds && M == 2 && xb <= (size_t)kLdsPerCu / 2) {
      // x past the default budget (M = 2 with K > 5120): in LDS after all when the launch, with
      // three rows per wavefront for every two-row problem, fits the workgroups the LDS holds;
      // the shaping below then aims at that many wave slots (TinyLlama's 7 linears: 22 KiB of x,
      // seven workgroups per CU by LDS).  The mixed M = 2 kernel this selects holds only five
      // 4-wavefront workgroups per CU by its registers (85 VGPRs, 5 waves per SIMD), so such a
      // launch runs in about 1.4 rounds (TinyLlama: 7,088 wavefronts, 5,120 resident); measured on
      // MI355X it is still faster than per-lane x loads in one round (8.63 -> 7.42 us).
      const long lds_slots = (long)(kLdsPerCu / xb) * kGemvWavesPerBlock * cus;
      long w3 = 0;
      for (int i = 0; i < count; ++i) {
        const long r = p.rows[i] == 2 ? 3 : gemv_entry_rows(p.rows[i]);
        w3 += ((N[i] + r - 1) / r + kGemvWavesPerBlock - 1) / kGemvWavesPerBlock * kGemvWavesPerBlock;
      }
      if (w3 <= lds_slots) {
        p.x_lds = true;
        slots = lds_slots;
      }
    }
    long total = total_waves();
    bool three = false;
    while (total > slots) {  // two-row problems (plain or flat) to three rows, largest first
      int best = -1;
      for (int i = 0; i < count; ++i)
        if ((p.rows[i] == 2 || p.rows[i] == kGemvFlat + 2) && (best < 0 || N[i] > N[best])) best = i;
      if (best < 0) break;
      total -= waves_of(best);
      p.rows[best] = 3;
      total += waves_of(best);
      three = true;
    }
    bool shaped = false;
    for (int i = 0; i < count; ++i) shaped = shaped || p.rows[i] == kGemvDeep || p.rows[i] > kGemvFlat;
    if (shaped) {
      p.rows_per_wave = kGemvRowsShaped;
      p.unroll = 1;
    } else if (three) {
      p.rows_per_wave = kGemvRowsMixed;
    }
  }
  return p;
}

hipError_t gemv_launch(const GemvPlan& plan, const GemvProblem* problems, int count, int M, int group_size,
                       hipStream_t stream) {
  const int shift = group_size == 128 ? 2 : 1;  // log2(G / 32)
  if (count == 1) {
    const GemvProblem& q = problems[0];
    const int blocks = xcd_grid(ceil_div(ceil_div(q.N, plan.rows_per_wave), kGemvWavesPerBlock));
    const size_t lds = plan.x_lds ? x_lds_bytes(M, q.K) : 0;
    void* fn = pick<false>(M, plan);
    if (lds > 65536) {  // dynamic LDS beyond 64 KiB is opted into per kernel
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPerCu);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(reinterpret_cast<GemvFn>(fn), dim3(blocks), dim3(64 * kGemvWavesPerBlock),
                       lds, stream, static_cast<const half_t*>(q.x), static_cast<const uint32_t*>(q.packed),
                       static_cast<const half_t*>(q.scales), static_cast<half_t*>(q.y), q.N, q.K, shift);
    return hipGetLastError();
  }
  // Longest rows first: their waves carry the most bytes, so they are
  // dispatched before the short ones (outputs do not depend on the order).
  int order[kMaxGemvGroup];
  for (int i = 0; i < count; ++i) order[i] = i;
  for (int i = 1; i < count; ++i)
    for (int j = i; j > 0 && problems[order[j]].K > problems[order[j - 1]].K; --j) {
      const int t = order[j];
      order[j] = order[j - 1];
      order[j - 1] = t;
    }
  GemvTable table = {};
  int bounds[kMaxGemvGroup];  // first wave of problems 1 .., then the total, then INT_MAX
  int waves = 0, max_k = 0;
  for (int i = 0; i < kMaxGemvGroup; ++i) {
    if (i < count) {
      const GemvProblem& q = problems[order[i]];
      const int rows = plan.rows[order[i]];
      table.slot[i] = GemvSlot{q.x, q.packed, q.scales, q.y, q.N, q.K, waves, rows};
      int w = ceil_div(q.N, gemv_entry_rows(rows));
      if (plan.x_lds) w = ceil_div(w, kGemvWavesPerBlock) * kGemvWavesPerBlock;  // whole workgroups
      waves += w;
      bounds[i] = waves;
      if (q.K > max_k) max_k = q.K;
    } else {
      bounds[i] = INT_MAX;
    }
  }
  const int blocks = xcd_grid(ceil_div(waves, kGemvWavesPerBlock));
  const size_t lds = plan.x_lds ? x_lds_bytes(M, max_k) : 0;
  void* fn = pick<true>(M, plan);
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsPerCu);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(reinterpret_cast<GemvGroupedFn>(fn), dim3(blocks),
                     dim3(64 * kGemvWavesPerBlock), lds, stream, count, shift, bounds[0], bounds[1], bounds[2],
                     bounds[3], bounds[4], bounds[5], bounds[6], bounds[7], table);
  return hipGetLastError();
}

hipError_t gemv_qkv_rope_launch(const GemvProblem& q, const GemvFused& f, const GemvRope& rope, int unroll,
                                int group_size, hipStream_t stream) {
  const int shift = group_size == 128 ? 2 : 1;  // log2(G / 32)
  const int wpb = gemv_fused_waves_per_block(f.prologue);
  const int blocks = xcd_grid(ceil_div(ceil_div(q.N, 2), wpb));
  const GemvRopeFn fn = f.prologue == kGemvProRmsNorm ? pick_rope_u<kGemvProRmsNorm>(unroll)
                                                      : pick_rope_u<kGemvProNone>(unroll);
  hipLaunchKernelGGL(fn, dim3(blocks), dim3(64 * wpb), fused_lds_bytes(q.K, f.prologue), stream,
                     static_cast<const half_t*>(q.x), static_cast<const uint32_t*>(q.packed),
                     static_cast<const half_t*>(q.scales), static_cast<half_t*>(q.y), q.N, q.K, shift,
                     static_cast<const half_t*>(f.aux), f.eps, rope);
  return hipGetLastError();
}

hipError_t gemv_fused_launch(const GemvPlan& plan, const GemvProblem& q, const GemvFused& f, int group_size,
                             hipStream_t stream) {
  const int shift = group_size == 128 ? 2 : 1;  // log2(G / 32)
  // One problem: never the mixed launch.  With a prologue every workgroup makes a second LDS copy
  // of an input row, so large N takes three rows per wavefront, a third fewer workgroups and copies
  // (measured: TinyLlama gate|up with RMSNorm 5.50 -> 5.21 us, Qwen2.5's 6.28 -> 5.89 us); the
  // third row's sums are added in the same order, so the bits do not change.
  int rows = plan.rows_per_wave == 1 ? 1 : 2;
  if (rows == 2 && f.prologue != kGemvProNone && q.N >= 8192) rows = 3;
  const int wpb = gemv_fused_waves_per_block(f.prologue);
  const int blocks = xcd_grid(ceil_div(ceil_div(q.N, rows), wpb));
  hipLaunchKernelGGL(pick_fused(f.prologue, rows, plan.unroll), dim3(blocks), dim3(64 * wpb),
                     fused_lds_bytes(q.K, f.prologue), stream, static_cast<const half_t*>(q.x),
                     static_cast<const uint32_t*>(q.packed), static_cast<const half_t*>(q.scales),
                     static_cast<half_t*>(q.y), q.N, q.K, shift, static_cast<const half_t*>(f.residual),
                     static_cast<const half_t*>(f.aux), f.eps);
  return hipGetLastError();
}

}  // namespace kf
