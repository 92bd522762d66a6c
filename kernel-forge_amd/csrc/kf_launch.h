// Host-side launch interfaces between the C ABI (kf_abi.hip) and the kernel
// translation units.  All launchers are asynchronous on `stream`, assume the
// arguments were validated by the ABI layer, and return hipSuccess or the
// launch error.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kf {

// ---- GEMV (M in [1, 8]) -------------------------------------------------
struct GemvPlan {
  int rows_per_wave;   // R: output rows one wavefront owns
  int unroll;          // U: 32-k chunks per lane kept in flight per pass
  int waves_per_block; // W: wavefronts per workgroup
};
GemvPlan gemv_plan(int M, int N, int K, int cu_count);
hipError_t gemv_launch(const GemvPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       int M, int N, int K, int group_size, hipStream_t stream);

// ---- MFMA GEMM (any M, N % 64 == 0) --------------------------------------
struct GemmPlan {
  int tile;        // index into the tile table (kf_gemm.hip)
  int block_m;     // BM
  int block_n;     // BN
  int splits;      // split-K factor (1 = no workspace)
  int kt_per_split;// k-tiles of 64 per split
};
GemmPlan gemm_plan(int M, int N, int K, int cu_count);
size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N);
hipError_t gemm_launch(const GemmPlan& p, const void* x, const void* packed, const void* scales, void* y,
                       void* ws, int M, int N, int K, int group_size, hipStream_t stream);

// ---- auxiliary kernels ----------------------------------------------------
hipError_t dequant_fp16_launch(const void* packed, const void* scales, void* w_hat, int N, int K, int group_size,
                               hipStream_t stream);
hipError_t bw_copy_launch(const void* src, void* dst, size_t bytes, int grid, hipStream_t stream);
hipError_t bw_read_launch(const void* src, void* sink, size_t bytes, int grid, hipStream_t stream);
hipError_t bw_write_launch(void* dst, size_t bytes, int grid, hipStream_t stream);

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace kf
