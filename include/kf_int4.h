/*
 * C ABI of the MI355X (gfx950) INT4 weight-only linear library, libkf_int4.so.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*; NULL is the legacy default stream).  Nothing here
 * allocates device memory, synchronizes, or reads device memory from the
 * host, so every call is asynchronous and safe under hipGraph stream capture.
 * Outputs and the split-K workspace are owned by the caller.
 *
 * Data layout (the reference's packing convention, kernelforge/quantize.py:12-24):
 *   x       fp16  [M, K]    row-major, contiguous
 *   packed  int32 [N, K/8]  row-major; word j of row n holds u = q + 8 for
 *                           k = 8j..8j+7 with nibble p (bits 4p..4p+3) = k offset
 *                           (0,2,4,6,1,3,5,7)[p]
 *   scales  fp16  [N, K/G]  row-major
 *   y       fp16  [M, N]    row-major
 * y[m, n] = fp16_rne( sum_k x[m, k] * W_hat[n, k] ) with fp32 accumulation,
 * W_hat = fp16_rne(q * s) (GEMM path) or q * s folded per 32-k chunk (GEMV).
 *
 * Return value: KF_OK (0) or one of the KF_ERR_* codes; kf_last_error()
 * returns a thread-local message describing the most recent failure.
 */
#ifndef KF_INT4_H_
#define KF_INT4_H_

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_ABI_VERSION 1

enum kf_status {
  KF_OK = 0,
  KF_ERR_INVALID_ARG = 1,   /* null pointer, misaligned pointer, bad M/N/K/G */
  KF_ERR_UNSUPPORTED = 2,   /* valid arguments outside this kernel's domain */
  KF_ERR_WORKSPACE = 3,     /* split-K workspace missing or too small */
  KF_ERR_HIP = 4,           /* HIP runtime error (launch failure, bad device) */
};

/* Version of this ABI (KF_ABI_VERSION). No reference counterpart. */
int kf_abi_version(void);

/* Message for the most recent non-zero status on the calling thread.
 * Replaces the reference's exception text (csrc/common/check.cuh:8-24,
 * TORCH_CHECK in csrc/gemm/dequant_gemv.cu:5-19). */
const char* kf_last_error(void);

/* Largest N one launch accepts (for a grouped GEMV: the sum of N over its
 * problems).  At one row per wavefront this keeps a launch below 2^31
 * work-items; larger N returns KF_ERR_UNSUPPORTED.  No reference counterpart. */
#define KF_MAX_ROWS ((1 << 25) - 64)

/* Fused dequant GEMV for M in [1, 8], N in [1, KF_MAX_ROWS], K % G == 0, G in {64, 128}.
 * x and packed must be 16-byte aligned.
 * Replaces kf::gemv::dispatch (csrc/gemm/dequant_gemv_kernel.cuh:120-142)
 * and the pybind entry _C.int4_gemv (csrc/bindings.cpp:24-25,
 * csrc/gemm/dequant_gemv.cu:21-36). */
int kf_int4_gemv(const void* x, const void* packed, const void* scales, void* y,
                 int M, int N, int K, int group_size, void* stream);

/* One problem of a grouped GEMV launch: y = x @ W_hat^T with x fp16 [M, K],
 * packed int32 [N, K/8], scales fp16 [N, K/G], y fp16 [M, N]. */
typedef struct kf_gemv_problem {
  const void* x;
  const void* packed;
  const void* scales;
  void* y;
  int N;
  int K;
} kf_gemv_problem;

#define KF_GEMV_MAX_GROUP 8

/* Up to KF_GEMV_MAX_GROUP independent GEMVs (common M in [1, 8] and G) in
 * ONE launch; each output equals what kf_int4_gemv computes for that problem,
 * bit for bit.  The problems array is read on the host during the call (it
 * is passed to the kernel by value), so it may live on the caller's stack.
 * No reference counterpart as an entry point: it is the multi-problem launch
 * of the reference's GEMV (csrc/gemm/dequant_gemv_kernel.cuh:38-142), for
 * decode linears that are independent (q|k|v on one x, gate|up on one x, or
 * separate layers), since on MI355X a launch's fixed cost (~1.5 us) exceeds
 * the time to stream a whole small layer. */
int kf_int4_gemv_grouped(const kf_gemv_problem* problems, int count, int M, int group_size, void* stream);

/* The launch plan of kf_int4_gemv (count = 1) or kf_int4_gemv_grouped for these shapes, on a
 * GPU with cu_count compute units (<= 0: the current device's).  *kernel: KF_GEMV_KERNEL_*;
 * rows[i] (count entries): output rows per wavefront of problem i (1, 2 or 3), KF_GEMV_FLAT + F
 * (F rows of K = 1024 or 1536 per wavefront, their chunks packed into full 64-lane loads) or
 * KF_GEMV_DEEP (two long rows per wavefront, five 64-chunk blocks per memory round trip);
 * *unroll: 64-chunk blocks per pass of the other rows; *x_lds: 1 when each workgroup stages x in
 * LDS.  Any output pointer may be NULL.  Host code only (no launch, no device access when
 * cu_count > 0).  For diagnostics and tests; no reference counterpart. */
#define KF_GEMV_KERNEL_ROWS1 1   /* one row per wavefront */
#define KF_GEMV_KERNEL_ROWS2 2   /* two rows per wavefront */
#define KF_GEMV_KERNEL_MIXED 3   /* grouped: two or three rows per problem */
#define KF_GEMV_KERNEL_SHAPED 4  /* grouped, M = 1: also flat and deep rows */
#define KF_GEMV_DEEP 8
#define KF_GEMV_FLAT 16
int kf_int4_gemv_plan(int M, const int* N, const int* K, int count, int cu_count, int* kernel, int* rows,
                      int* unroll, int* x_lds);

#define KF_PROLOGUE_NONE 0     /* x as given */
#define KF_PROLOGUE_RMSNORM 1  /* x * rsqrt(mean(x^2) + eps) * aux, aux = fp16 norm weight [K] */
#define KF_PROLOGUE_SWIGLU 2   /* fp16(fp16(silu(x)) * aux): x = gate [K], aux = up [K] */
#define KF_GEMV_FUSED_MAX_K 10240

/* Decode GEMV (M = 1, K <= KF_GEMV_FUSED_MAX_K) with the work either side of a decoder linear
 * fused in: a prologue transforms x before the product (RMSNorm with weight aux and eps, or
 * SwiGLU of gate x and up aux, computed on the workgroup's LDS copy of x), and a non-NULL
 * residual (fp16 [N], may equal y) is added to the fp16 result:
 * y = fp16(residual + fp16(prologue(x) @ W_hat^T)).  The product is kf_int4_gemv's, bit for bit;
 * with the residual the output equals torch's residual + int4_linear(x) bit for bit, and the
 * SwiGLU prologue rounds like torch's silu(gate) * up on fp16 tensors.  aux must be 16-byte
 * aligned.  No reference counterpart: it fuses the RMSNorm, SiLU-multiply and residual adds
 * that surround the reference's int4_linear in a decoder layer into the GEMV launch. */
int kf_int4_gemv_fused(const void* x, const void* packed, const void* scales, void* y, int M, int N, int K,
                       int group_size, int prologue, const void* aux, float eps, const void* residual, void* stream);

/* Attention inputs the q|k|v decode GEMV writes directly (kf_int4_gemv_qkv_rope). */
typedef struct kf_rope_cache {
  const void* cos;  /* fp16 [max_seq, head_dim] */
  const void* sin;  /* fp16 [max_seq, head_dim], rotate-half sign folded in: -sin on the first half */
  const void* pos;  /* int64 in device memory: the token's position (read by the kernel) */
  void* cache_k;    /* fp16 [kv_heads, head_dim, max_seq]: K transposed */
  void* cache_v;    /* fp16 [kv_heads, max_seq, head_dim] */
  int heads;
  int kv_heads;
  int head_dim;     /* even */
  int max_seq;
} kf_rope_cache;

/* The q|k|v projection of one decode token (M = 1, K <= KF_GEMV_FUSED_MAX_K) with RoPE and the
 * KV-cache writes in its epilogue, optionally the input RMSNorm in its prologue (norm_weight
 * non-NULL, as KF_PROLOGUE_RMSNORM).  Rows of packed / scales: heads q heads, kv_heads k heads,
 * kv_heads v heads, head_dim rows each (N = (heads + 2 kv_heads) * head_dim), i.e. the weights of
 * q|k|v concatenated.  y [N] receives q and k rotated, v as is, in that order; k is also stored
 * at cache_k[h][:][pos], v at cache_v[h][pos][:].  A pos outside [0, max_seq) writes no cache entry
 * and rotates q and k in y with row 0 of the tables (no table row exists for it).
 * Rotation: fp16(fp16(x * cos) + x_partner * sin), the roundings of x * cos + swap_halves(x) * sin
 * on fp16 tensors.  No reference counterpart: it fuses the RoPE and cache update that follow the
 * q|k|v int4_linear calls in a decoder's attention. */
int kf_int4_gemv_qkv_rope(const void* x, const void* packed, const void* scales, void* y, int N, int K,
                          int group_size, const void* norm_weight, float eps, const kf_rope_cache* rope,
                          void* stream);

/* Bytes of fp32 split-K workspace kf_int4_gemm needs for this problem on the
 * current device (0 when the chosen plan has no split-K).
 * Replaces kf::gemm_tc::workspace_floats (dequant_gemm_tc_kernel.cuh:179-183),
 * which counted floats instead of bytes. */
size_t kf_int4_gemm_workspace_bytes(int M, int N, int K, int group_size);

/* The kernel kf_int4_gemm() runs for (M, N, K, G) on the current device: *kernel is
 * KF_GEMM_SKINNY or a tile-table index in [0, *num_kernels), *splits the split-K factor
 * (1 = no workspace), *block_m x *block_n the output tile (0 x 0 for the skinny kernel).
 * Any output pointer may be NULL.  For diagnostics and tests; no reference counterpart. */
#define KF_GEMM_SKINNY (-1)
int kf_int4_gemm_plan(int M, int N, int K, int group_size, int* kernel, int* num_kernels,
                      int* splits, int* block_m, int* block_n);

/* MFMA dequant GEMM, any M >= 1, N % 64 == 0 and N <= KF_MAX_ROWS, K % G == 0, G in {64, 128}.
 * x, packed and y 16-byte aligned (its epilogues store y in 8- and 16-byte vectors; the GEMV
 * entry points need only 2-byte aligned y).
 * ws may be NULL when kf_int4_gemm_workspace_bytes() returned 0.
 * Replaces kf::gemm_tc::run (dequant_gemm_tc_kernel.cuh:203-211) and the
 * pybind entry _C.int4_gemm (csrc/bindings.cpp:26-27,
 * csrc/gemm/dequant_gemm_tc.cu:7-28). */
int kf_int4_gemm(const void* x, const void* packed, const void* scales, void* y,
                 void* ws, size_t ws_bytes, int M, int N, int K, int group_size, void* stream);

/* Bytes of split-K scratch kf_int4_gemm_noalloc holds per GPU (a device array in the library). */
#define KF_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* kf_int4_gemm without a workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The split-K partials go to a device array of
 * KF_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on until the process ends;
 * the call itself allocates nothing (no hipMalloc / hipFree).  Same plan, kernels and results
 * as kf_int4_gemm, bit for bit.  A problem whose plan needs more partials than the scratch holds
 * (kf_int4_gemm_workspace_bytes() > KF_NOALLOC_SCRATCH_BYTES) returns KF_ERR_WORKSPACE without
 * launching.  All calls on one GPU share its scratch: calls that overlap on that GPU (other
 * streams, other threads) race; serialize them.  The first call on a device looks up the scratch
 * address (hipGetSymbolAddress) with that device current. */
int kf_int4_gemm_noalloc(const void* x, const void* packed, const void* scales, void* y, int M, int N, int K,
                         int group_size, void* stream);

/* MFMA-16 block copy of a packed weight (an internal layout; the public packed format is
 * unchanged): for every 16 rows of W and 128-k super-step, the 64 lanes' 16-byte pieces of
 * the MFMA fragments stored contiguously in lane order (lane l: row 16b + l%16, words
 * 16s + 4(l/16) .. +3), rows padded to a multiple of 16 by repeating row N-1; scales as
 * [ceil(N/16)][K/G][16].  K must be a multiple of 128.  Sizes of the two buffers: */
int kf_int4_mfma16_sizes(int N, int K, int group_size, size_t* packed_bytes, size_t* scales_bytes);

/* Writes the MFMA-16 copy of (packed, scales) into (packed_r, scales_r); a pure permutation.
 * The weight copy behind the op that the reference names as its next GEMM step
 * (docs/phase4-notes.md:59, docs/references.md:26); no reference function. */
int kf_int4_reorder_mfma16(const void* packed, const void* scales, void* packed_r, void* scales_r,
                           int N, int K, int group_size, void* stream);

/* kf_int4_gemm with the MFMA-16 copy of the same weight: where the skinny kernel runs it
 * streams packed_r / scales_r (contiguous 1 KiB wavefront loads, 7-15% faster), elsewhere
 * packed / scales.  Results are bit-identical to kf_int4_gemm.  Same requirements, plus
 * K % 128 == 0.  No reference counterpart (see kf_int4_reorder_mfma16). */
int kf_int4_gemm_mfma16(const void* x, const void* packed, const void* scales, const void* packed_r,
                        const void* scales_r, void* y, void* ws, size_t ws_bytes,
                        int M, int N, int K, int group_size, void* stream);

/* W_hat = fp16_rne(q * s) as fp16 [N, K]: the dequantization the GEMM feeds
 * to the matrix cores, exported so it can be compared bit for bit with the
 * reference's dequantize(qw, torch.float16) (kernelforge/quantize.py:108-113). */
int kf_int4_dequant_fp16(const void* packed, const void* scales, void* w_hat,
                         int N, int K, int group_size, void* stream);

/* Element types of a weight matrix handed to kf_int4_quantize. */
#define KF_DTYPE_F32 0
#define KF_DTYPE_F16 1
#define KF_DTYPE_BF16 2

/* Quantize and pack a weight matrix w [N, K] (row-major, dtype one of KF_DTYPE_*,
 * 16-byte aligned, finite values) into packed int32 [N, K/8] and fp16 scales [N, K/G],
 * bit for bit what quantize_weight() produces on the CPU: scale = fp16(max(absmax/7, 2^-14))
 * (1 for an all-zero group), q = clamp(rint(w / scale), -8, 7), nibble order of
 * pack_int4.  Replaces quantize_int4 + pack_int4 + quantize_weight
 * (kernelforge/quantize.py:61-105), which run as torch elementwise ops. */
int kf_int4_quantize(const void* w, int dtype, void* packed, void* scales,
                     int N, int K, int group_size, void* stream);

/* Streaming HBM ceilings with dwordx4 accesses: dst[i] = src[i] (copy),
 * a checksum of src folded into sink[0..grid) (read), dst[i] = pattern
 * (write).  bytes must be a multiple of 16.  grid_blocks <= 0 picks a default.
 * Replace the reference's measurement kernels (csrc/micro/bandwidth.cu:17-42). */
int kf_bw_copy(const void* src, void* dst, size_t bytes, int grid_blocks, void* stream);
int kf_bw_read(const void* src, void* sink, size_t bytes, int grid_blocks, void* stream);
int kf_bw_write(void* dst, size_t bytes, int grid_blocks, void* stream);

/* kf_bw_read that also stores, as a decode GEMV does: 2 fp16 values per wavefront of 64 threads
 * (lanes 31 and 63) into out, adjacent across wavefronts, so out needs 16 * grid_blocks bytes.
 * The same-size read with and without these stores bounds what a one-launch GEMV step that must
 * write its outputs can reach.  No reference counterpart (a measurement kernel beside
 * csrc/micro/bandwidth.cu:17-42's). */
int kf_bw_read_store(const void* src, void* out, size_t bytes, int grid_blocks, void* stream);

/* The greedy step of a graph-captured decode loop, one launch: idx = argmax(logits[0..n)) over
 * fp16 logits in torch.argmax's order (NaN above every number; among equal values the smallest
 * index), then p = *pos + 1; *pos = p; *token = idx; and, when 0 <= p < max_seq,
 * history[p] = idx and (mask non-NULL) mask[p] = 0 (fp16), so the next step's additive mask
 * admits its own position.  token, pos, history: int64 on the device; every write stays inside
 * history[0, max_seq) and mask[0, max_seq).  Replaces torch's argmax, fp32 cast and the
 * index / copy / add kernels of the decoder's step (kernelforge/tinyllama.py, config 5 of the
 * benchmark); no reference counterpart (the reference's harness does these in torch,
 * bench/e2e_model.py:85-141). */
int kf_decode_argmax_step(const void* logits, int n, void* token, void* pos, void* history, int max_seq,
                          void* mask, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KF_INT4_H_ */
