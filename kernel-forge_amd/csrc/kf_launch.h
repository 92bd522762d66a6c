// Host-side launch interfaces between the C ABI (kf_abi.hip) and the kernel
// translation units.  All launchers are asynchronous on `stream`, assume the
// arguments were validated by the ABI layer, and return hipSuccess or the
// launch error.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kf {

// ---- GEMV (M in [1, 8]), one or several independent problems per launch ----
constexpr int kMaxGemvGroup = 8;

struct GemvProblem {
  const void* x;       // fp16 [M, K]
  const void* packed;  // int32 [N, K/8]
  const void* scales;  // fp16 [N, K/G]
  void* y;             // fp16 [M, N]
  int N;
  int K;
};

// One problem as the grouped kernel reads it: the problem plus the index of its first
// wavefront in the launch.
struct GemvSlot {
  const void* x;
  const void* packed;
  const void* scales;
  void* y;
  int N;
  int K;
  int wave0;
  int rows;  // rows per wavefront of this problem (2 or 3), kGemvFlat + F or kGemvDeep
};

// The grouped kernel's arguments: the lookup header as ten scalar arguments (preloaded into
// SGPRs at wave launch), then this table by value.  A wavefront finds its problem from the
// header without memory traffic and then fetches that problem's 48-byte slot in one round of
// scalar loads (see kf_gemv.hip).
struct GemvTable {
  GemvSlot slot[kMaxGemvGroup];
};

constexpr int kGemvWavesPerBlock = 4;  // 256-thread workgroups
// Largest x (M * K fp16 values, in bytes) a workgroup copies into LDS; 20 KiB keeps eight
// workgroups (32 wavefronts) per CU within the 160 KiB of LDS.
constexpr int kGemvMaxLdsX = 20480;
// A launch with fewer workgroups per CU gives each a larger copy: the CU's 160 KiB over the
// workgroups it holds (beyond 64 KiB the launch opts into the larger dynamic LDS).
constexpr int kLdsPerCu = 160 * 1024;

// GemvPlan::rows_per_wave of a grouped launch whose problems take 2 or 3 rows per wavefront
// each (GemvPlan::rows, GemvSlot::rows); also the grouped kernel's template rows for it.
constexpr int kGemvRowsMixed = 3;

// Flat rows (M = 1, grouped launches): a row of K = 32 C with C < 64 leaves E = 64 - C lanes of
// every 64-chunk load idle.  When E divides C and C / E <= 3 (K = 1024: C = 32; K = 1536: C = 48)
// one wavefront owns F = C / E + 1 rows in C / E full loads (gemv_rows_flat in kf_gemv.hip).  Such
// a problem's GemvPlan::rows / GemvSlot::rows entry is kGemvFlat + F.  Returns F, or 0.
constexpr int kGemvFlat = 16;
inline int gemv_flat_rows(int K) {
  if (K % 32 != 0 || K >= 2048) return 0;
  const int c = K / 32, e = 64 - c;
  return (e <= c && c % e == 0 && c / e <= 3) ? c / e + 1 : 0;
}
// Deep rows (M = 1, grouped launches with wavefront slots to spare): two long rows per
// wavefront, their 64-chunk blocks loaded kGemvDeepPass at a time per memory round trip
// (gemv_rows_deep in kf_gemv.hip).
constexpr int kGemvDeep = 8;
// GemvPlan::rows_per_wave of a grouped launch (M = 1, x in LDS) with flat or deep rows among its
// problems.  Its kernel is an instantiation of its own, so launches without such rows keep the
// mixed kernel's code and registers.  kGemvDeepPass: (row, block) loads per pass of a deep
// wavefront, as many as keep the kernel at 8 wavefronts per SIMD (kernelforge/build.py checks
// it): a K = 8960 row pair is two passes of five.
constexpr int kGemvRowsShaped = 4;
constexpr int kGemvDeepPass = 5;
// Rows one wavefront owns for a GemvPlan::rows / GemvSlot::rows entry.
inline int gemv_entry_rows(int entry) {
  return entry == kGemvDeep ? 2 : (entry > kGemvFlat ? entry - kGemvFlat : entry);
}

struct GemvPlan {
  int rows_per_wave;   // R: output rows one wavefront owns, or kGemvRowsMixed
  int unroll;          // U: 64-chunk blocks (64 lanes x 32 k) whose loads one pass keeps in flight
  bool x_lds;          // each workgroup copies x into LDS once (else every lane loads its x)
  int rows[kMaxGemvGroup];  // per problem (caller's order): rows per wavefront, kGemvFlat + F or kGemvDeep
};
GemvPlan gemv_plan(int M, const int* N, const int* K, int count, int cu_count);
hipError_t gemv_launch(const GemvPlan& p, const GemvProblem* problems, int count, int M, int group_size,
                       hipStream_t stream);

// ---- fused decode GEMV (M = 1): a transform of x before the product, a residual after it ----
// The product is the GEMV's (same kernel body, same bits); the transform runs on the
// workgroup's LDS copy of x, the residual is added to the fp16 result before its store.
enum GemvPrologue {
  kGemvProNone = 0,     // x as given
  kGemvProRmsNorm = 1,  // x * rsqrt(mean(x^2) + eps) * weight (aux: fp16 weight [K])
  kGemvProSwiGLU = 2,   // fp16(fp16(silu(gate)) * up) (x: gate [K], aux: up [K])
};
constexpr int kGemvFusedMaxK = kGemvMaxLdsX / 2;  // x of the one row fits the LDS budget
// Workgroup size of the fused launches.  With a prologue every workgroup copies two input rows
// into LDS and transforms them before its first product; eight wavefronts per workgroup halve
// those copies and that work (MI355X, TinyLlama decode shapes: gate|up with RMSNorm
// 5.16 -> 4.93 us, down with SwiGLU and residual 4.26 -> 3.51, q|k|v with RMSNorm and RoPE
// 3.89 -> 3.48; sixteen are slower than four).  Without a prologue the plain GEMV's four stay
// faster.
constexpr int kGemvWavesPerBlockPrologue = 8;
constexpr int gemv_fused_waves_per_block(int prologue) {
  return prologue == kGemvProNone ? kGemvWavesPerBlock : kGemvWavesPerBlockPrologue;
}
struct GemvFused {
  int prologue;          // GemvPrologue
  const void* aux;       // prologue input (see GemvPrologue), else nullptr
  float eps;             // RMSNorm epsilon
  const void* residual;  // fp16 [N]: y = fp16(residual + fp16(x @ W_hat^T)); nullptr: no residual
};
hipError_t gemv_fused_launch(const GemvPlan& p, const GemvProblem& problem, const GemvFused& f, int group_size,
                             hipStream_t stream);

// RoPE + KV-cache epilogue of the q|k|v decode GEMV: rows = heads q heads, kv_heads k heads, then
// kv_heads v heads of head_dim rows each.  A wavefront owns dims j and j + head_dim / 2 of one q or
// k head, rotates the pair with the position's cos / sin rows, stores it to y (natural order)
// and, for k, into the key cache; v rows go to y and the value cache.
struct GemvRope {
  const void* cos;     // fp16 [max_seq, head_dim]
  const void* sin;     // fp16 [max_seq, head_dim], rotate-half sign folded in (-sin on the first half)
  const void* pos;     // int64: the token's position (device memory)
  void* cache_k;       // fp16 [kv_heads, head_dim, max_seq] (K transposed)
  void* cache_v;       // fp16 [kv_heads, max_seq, head_dim]
  int heads, kv_heads, head_dim, max_seq;
};
hipError_t gemv_qkv_rope_launch(const GemvProblem& problem, const GemvFused& f, const GemvRope& rope, int unroll,
                                int group_size, hipStream_t stream);

// ---- skinny MFMA GEMM (M <= 32, K % 128 == 0): one weight stream, K split in-block ----
// gemm_plan (kf_gemm.hip) picks it for small M by the measured rule stated there.
constexpr int kSkinnyMaxM = 32;
struct SkinnyPlan {
  int m_tiles;    // 16-row tiles of M (1..2)
  int ks_waves;   // wavefronts per workgroup, each a contiguous run of 128-k super-steps
  int unroll;     // super-steps whose weight loads are in flight together
  bool x_lds;     // x fragments from each wavefront's LDS copy of its k range (else from L2)
  int lds_bytes;  // dynamic LDS per workgroup
  int col_blocks; // 16-column blocks per workgroup (1..2)
};
constexpr int kSkinnyMaxLds = 160 * 1024;  // LDS of a gfx950 CU
SkinnyPlan skinny_plan(int M, int N, int K, int cu_count);
// 16-column blocks per skinny workgroup for N on cu_count CUs (SkinnyPlan::col_blocks).
int skinny_col_blocks(int N, int cu_count);
hipError_t skinny_launch(const SkinnyPlan& p, const void* x, const void* packed, const void* scales, void* y, int M,
                         int N, int K, int group_size, bool blocked, hipStream_t stream);
// MFMA-16 block copy of packed / scales (kf_skinny.hip): sizes in int32 words and fp16 scales.
size_t mfma16_packed_words(int N, int K);
size_t mfma16_scale_count(int N, int K, int group_size);
hipError_t reorder_mfma16_launch(const void* packed, const void* scales, void* packed_r, void* scales_r, int N, int K,
                                 int group_size, hipStream_t stream);

// ---- MFMA GEMM (any M, N % 64 == 0) --------------------------------------
struct GemmPlan {
  bool skinny;     // true: the skinny kernel (fields below unused except sk)
  SkinnyPlan sk;
  int tile;        // index into the tile table (kf_gemm.hip)
  int block_m;     // BM
  int block_n;     // BN
  int splits;      // split-K factor (1 = no workspace)
  int kt_per_split;// k stages (of the tile's stage depth) per split
};
GemmPlan gemm_plan(int M, int N, int K, int cu_count);
// Plan with an explicit tile-table entry and the fill-the-CUs split rule (the K % 128 != 0
// fallback of gemm_plan, and tuning).
GemmPlan gemm_plan_with_tile(int M, int N, int K, int cu_count, int tile);
int gemm_num_tiles();
size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N);
// packed_r / scales_r: the MFMA-16 block copy, read where the skinny kernel runs (may be null).
hipError_t gemm_launch(const GemmPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       void* ws, int M, int N, int K, int group_size, hipStream_t stream,
                       const void* packed_r = nullptr, const void* scales_r = nullptr);

// ---- on-device quantize + pack (kf_quant.hip) -------------------------------
constexpr int kQuantF32 = 0, kQuantF16 = 1, kQuantBF16 = 2;  // == KF_DTYPE_* of the C ABI
hipError_t quantize_launch(const void* w, int dtype, void* packed, void* scales, int N, int K, int group_size,
                           hipStream_t stream);

// ---- auxiliary kernels ----------------------------------------------------
hipError_t dequant_fp16_launch(const void* packed, const void* scales, void* w_hat, int N, int K, int group_size,
                               hipStream_t stream);
hipError_t bw_copy_launch(const void* src, void* dst, size_t bytes, int grid, hipStream_t stream);
hipError_t bw_read_launch(const void* src, void* sink, size_t bytes, int grid, hipStream_t stream);
hipError_t bw_read_store_launch(const void* src, void* out, size_t bytes, int grid, hipStream_t stream);
hipError_t bw_write_launch(void* dst, size_t bytes, int grid, hipStream_t stream);
hipError_t decode_argmax_launch(const void* logits, int n, void* token, void* pos, void* history, int max_seq,
                                void* mask, hipStream_t stream);

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace kf
