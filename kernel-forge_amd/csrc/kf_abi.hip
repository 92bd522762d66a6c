// extern "C" entry points of libkf_int4.so (declared in include/kf_int4.h).
//
// This layer validates arguments (the checks of the reference's
// int4_check_inputs, csrc/gemm/dequant_gemv.cu:5-19, and of
// csrc/gemm/dequant_gemm_tc.cu:9-14), maps failures to status codes plus a
// thread-local message, and launches on the caller's stream.  It never
// allocates, synchronizes, or reads device memory, so it is safe inside
// hipGraph stream capture.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "kf_int4.h"
#include "kf_launch.h"

static_assert(KF_DTYPE_F32 == kf::kQuantF32 && KF_DTYPE_F16 == kf::kQuantF16 && KF_DTYPE_BF16 == kf::kQuantBF16,
              "dtype codes of the C ABI and the kernels differ");
static_assert(KF_GEMV_MAX_GROUP == kf::kMaxGemvGroup, "header and kernels disagree on the group limit");
static_assert(KF_PROLOGUE_NONE == kf::kGemvProNone && KF_PROLOGUE_RMSNORM == kf::kGemvProRmsNorm &&
                  KF_PROLOGUE_SWIGLU == kf::kGemvProSwiGLU,
              "prologue codes of the C ABI and the kernels differ");
static_assert(KF_GEMV_FUSED_MAX_K == kf::kGemvFusedMaxK, "header and kernels disagree on the fused K limit");

namespace {

thread_local char g_error[512] = "";

int fail(int status, const char* fmt, ...) {
  char buf[sizeof(g_error)];  // the message may quote the previous one
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  memcpy(g_error, buf, sizeof(g_error));
  return status;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return KF_OK;
  return fail(KF_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(err), hipGetErrorString(err));
}

// Compute-unit count of the current device, queried once per device.
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count(int* out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(KF_ERR_HIP, "device ordinal %d out of range", dev);
  int cus = g_cu_count[dev].load(std::memory_order_relaxed);
  if (cus <= 0) {
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return hip_status(err, "hipDeviceGetAttribute(MultiprocessorCount)");
    g_cu_count[dev].store(cus, std::memory_order_relaxed);
  }
  *out = cus;
  return KF_OK;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Checks shared by the GEMV and the GEMM (order and wording follow
// kernelforge/ops.py:171-182 and csrc/gemm/dequant_gemv.cu:5-19).  The sizes come before the
// pointers: an empty tensor's data pointer is null, and its size is the error worth naming.
int check_common(const void* x, const void* packed, const void* scales, const void* y, int M, int N, int K,
                 int group_size) {
  if (M < 1 || N < 1 || K < 1) return fail(KF_ERR_INVALID_ARG, "M, N, K must be positive, got M=%d N=%d K=%d", M, N, K);
  if (!x || !packed || !scales || !y) return fail(KF_ERR_INVALID_ARG, "x, packed, scales and y must be non-null");
  if (N > KF_MAX_ROWS) return fail(KF_ERR_UNSUPPORTED, "N=%d exceeds the %d rows one launch supports", N, KF_MAX_ROWS);
  if (group_size != 64 && group_size != 128)
    return fail(KF_ERR_INVALID_ARG, "group_size must be one of (64, 128), got %d", group_size);
  if (K % group_size != 0)
    return fail(KF_ERR_INVALID_ARG, "K=%d is not a multiple of group_size=%d", K, group_size);
  if (!aligned(x, 16) || !aligned(packed, 16))
    return fail(KF_ERR_INVALID_ARG, "x and packed must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(y, 2)) return fail(KF_ERR_INVALID_ARG, "scales and y must be 2-byte aligned");
  return KF_OK;
}

// ---- Scratch of kf_int4_gemm_noalloc --------------------------------------------------------
// The split-K partials of the entry point that allocates nothing live in this file-scope device
// array instead of a caller's workspace.  On the host, `scratch` names a host-side stand-in, not
// a device address: host code never passes it to a kernel or a copy.  The device address of each
// GPU's copy comes from hipGetSymbolAddress, called once per device with that device current
// (scratch_ptr), and only that address is handed to the kernels.  Every call on a GPU shares the
// GPU's copy, so calls that overlap on one GPU race; each call's split-K kernels overwrite every
// element of the partials they later read, so nothing has to start at zero.
constexpr size_t kScratchBytes = KF_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];
static_assert(kScratchBytes % 256 == 0, "scratch size");

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// Device address of the current device's scratch array, looked up on the first call per device.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(KF_ERR_HIP, "device ordinal %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess) return hip_status(err, "hipGetSymbolAddress(scratch)");
      if (!p) return fail(KF_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address on device %d", dev);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KF_OK;
}

// kf_int4_gemm, kf_int4_gemm_mfma16 and kf_int4_gemm_noalloc: validation, plan, workspace check,
// launch.  With use_scratch the split-K partials go to this device's scratch array (ws is ignored).
int gemm_entry(const void* x, const void* packed, const void* scales, const void* packed_r, const void* scales_r,
               void* y, void* ws, size_t ws_bytes, int M, int N, int K, int group_size, void* stream,
               bool use_scratch = false) {

  int st = check_common(x, packed, scales, y, M, N, K, group_size);
  if (st) return st;
  if (N % 64 != 0) return fail(KF_ERR_UNSUPPORTED, "int4_gemm needs N to be a multiple of 64, got N=%d", N);
  if (K % 64 != 0) return fail(KF_ERR_UNSUPPORTED, "int4_gemm needs K to be a multiple of 64, got K=%d", K);
  // The GEMM epilogues store y as 8- and 16-byte vectors (N % 64 == 0 keeps every row's start on
  // a 16-byte boundary once y's is).
  if (!aligned(y, 16)) return fail(KF_ERR_INVALID_ARG, "int4_gemm needs y to be 16-byte aligned");
  int cus = 0;
  if ((st = cu_count(&cus))) return st;
  const kf::GemmPlan plan = kf::gemm_plan(M, N, K, cus);
  // One workgroup (<= 512 threads) per output tile and split, all in grid dimension x.
  const long long tiles = (long long)((M + plan.block_m - 1) / plan.block_m) * ((N + plan.block_n - 1) / plan.block_n);
  if (!plan.skinny && (tiles * plan.splits + 8) * 512 > 0x7FFFFFFFLL)
    return fail(KF_ERR_UNSUPPORTED, "M=%d, N=%d exceed the grid limit for %dx%d tiles", M, N, plan.block_m,
                plan.block_n);
  const size_t need = kf::gemm_workspace_bytes(plan, M, N);
  if (use_scratch) {
    ws = nullptr;
    if (need > kScratchBytes)
      return fail(KF_ERR_WORKSPACE,
                  "int4_gemm_noalloc: M=%d N=%d K=%d needs %zu bytes of split-K partials, more than the %zu-byte "
                  "scratch it holds; call kf_int4_gemm with a workspace",
                  M, N, K, need, kScratchBytes);
    if (need > 0 && (st = scratch_ptr(&ws))) return st;
  } else if (need > 0) {
    if (!ws) return fail(KF_ERR_WORKSPACE, "split-K workspace of %zu bytes required, got NULL", need);
    if (ws_bytes < need) return fail(KF_ERR_WORKSPACE, "split-K workspace of %zu bytes required, got %zu", need, ws_bytes);
    if (!aligned(ws, 16)) return fail(KF_ERR_INVALID_ARG, "workspace must be 16-byte aligned");
  }
  return hip_status(kf::gemm_launch(plan, x, packed, scales, y, ws, M, N, K, group_size,
                                    static_cast<hipStream_t>(stream), packed_r, scales_r),
                    "int4_gemm launch");
}

}  // namespace

extern "C" {

int kf_abi_version(void) { return KF_ABI_VERSION; }

const char* kf_last_error(void) { return g_error; }

int kf_int4_gemv(const void* x, const void* packed, const void* scales, void* y, int M, int N, int K,
                 int group_size, void* stream) {
  int st = check_common(x, packed, scales, y, M, N, K, group_size);
  if (st) return st;
  if (M > 8) return fail(KF_ERR_INVALID_ARG, "int4_gemv handles M in [1, 8], got M=%d", M);
  int cus = 0;
  if ((st = cu_count(&cus))) return st;
  const kf::GemvProblem prob = {x, packed, scales, y, N, K};
  const kf::GemvPlan plan = kf::gemv_plan(M, &N, &K, 1, cus);
  return hip_status(kf::gemv_launch(plan, &prob, 1, M, group_size, static_cast<hipStream_t>(stream)),
                    "int4_gemv launch");
}

int kf_int4_gemv_grouped(const kf_gemv_problem* problems, int count, int M, int group_size, void* stream) {
  if (!problems) return fail(KF_ERR_INVALID_ARG, "problems must be non-null");
  if (count < 1 || count > KF_GEMV_MAX_GROUP)
    return fail(KF_ERR_INVALID_ARG, "count must be in [1, %d], got %d", KF_GEMV_MAX_GROUP, count);
  if (M < 1 || M > 8) return fail(KF_ERR_INVALID_ARG, "int4_gemv handles M in [1, 8], got M=%d", M);
  kf::GemvProblem probs[KF_GEMV_MAX_GROUP];
  int ns[KF_GEMV_MAX_GROUP], ks[KF_GEMV_MAX_GROUP];
  long rows = 0;
  for (int i = 0; i < count; ++i) {
    const kf_gemv_problem& p = problems[i];
    int st = check_common(p.x, p.packed, p.scales, p.y, M, p.N, p.K, group_size);
    if (st) return fail(st, "problem %d: %s", i, kf_last_error());
    probs[i] = {p.x, p.packed, p.scales, p.y, p.N, p.K};
    ns[i] = p.N;
    ks[i] = p.K;
    rows += p.N;
  }
  if (rows > KF_MAX_ROWS)
    return fail(KF_ERR_UNSUPPORTED, "the problems have %ld rows in total, more than the %d one launch supports", rows,
                KF_MAX_ROWS);
  int cus = 0;
  int st = cu_count(&cus);
  if (st) return st;
  const kf::GemvPlan plan = kf::gemv_plan(M, ns, ks, count, cus);
  return hip_status(kf::gemv_launch(plan, probs, count, M, group_size, static_cast<hipStream_t>(stream)),
                    "int4_gemv_grouped launch");
}

int kf_int4_gemv_plan(int M, const int* N, const int* K, int count, int cus_given, int* kernel, int* rows,
                      int* unroll, int* x_lds) {
  static_assert(KF_GEMV_FLAT == kf::kGemvFlat && KF_GEMV_DEEP == kf::kGemvDeep &&
                    KF_GEMV_KERNEL_MIXED == kf::kGemvRowsMixed && KF_GEMV_KERNEL_SHAPED == kf::kGemvRowsShaped,
                "plan codes");
  if (!N || !K) return fail(KF_ERR_INVALID_ARG, "N and K must be non-null");
  if (count < 1 || count > KF_GEMV_MAX_GROUP)
    return fail(KF_ERR_INVALID_ARG, "count must be in [1, %d], got %d", KF_GEMV_MAX_GROUP, count);
  if (M < 1 || M > 8) return fail(KF_ERR_INVALID_ARG, "int4_gemv handles M in [1, 8], got M=%d", M);
  for (int i = 0; i < count; ++i)
    if (N[i] < 1 || K[i] < 64 || K[i] % 64)
      return fail(KF_ERR_INVALID_ARG, "problem %d: N >= 1 and K a positive multiple of 64, got N=%d K=%d", i, N[i],
                  K[i]);
  int cus = cus_given;
  if (cus <= 0) {
    const int st = cu_count(&cus);
    if (st) return st;
  }
  const kf::GemvPlan p = kf::gemv_plan(M, N, K, count, cus);
  if (kernel) *kernel = p.rows_per_wave;
  if (rows)
    for (int i = 0; i < count; ++i) rows[i] = p.rows[i];
  if (unroll) *unroll = p.unroll;
  if (x_lds) *x_lds = p.x_lds ? 1 : 0;
  return KF_OK;
}

int kf_int4_gemv_fused(const void* x, const void* packed, const void* scales, void* y, int M, int N, int K,
                       int group_size, int prologue, const void* aux, float eps, const void* residual, void* stream) {
  int st = check_common(x, packed, scales, y, M, N, K, group_size);
  if (st) return st;
  if (M != 1) return fail(KF_ERR_UNSUPPORTED, "int4_gemv_fused handles M = 1 (decode), got M=%d", M);
  if (prologue < KF_PROLOGUE_NONE || prologue > KF_PROLOGUE_SWIGLU)
    return fail(KF_ERR_INVALID_ARG, "prologue must be KF_PROLOGUE_NONE, _RMSNORM or _SWIGLU, got %d", prologue);
  if (prologue != KF_PROLOGUE_NONE && (!aux || !aligned(aux, 16)))
    return fail(KF_ERR_INVALID_ARG, "the prologue's aux input must be non-null and 16-byte aligned");
  if (prologue == KF_PROLOGUE_RMSNORM && !(eps >= 0.0f && eps <= 3.0e38f))
    return fail(KF_ERR_INVALID_ARG, "eps must be finite and >= 0, got %g", (double)eps);
  if (residual && !aligned(residual, 2)) return fail(KF_ERR_INVALID_ARG, "residual must be 2-byte aligned");
  if (K > KF_GEMV_FUSED_MAX_K)
    return fail(KF_ERR_UNSUPPORTED, "int4_gemv_fused needs K <= %d (x in LDS), got K=%d", KF_GEMV_FUSED_MAX_K, K);
  int cus = 0;
  if ((st = cu_count(&cus))) return st;
  const kf::GemvProblem prob = {x, packed, scales, y, N, K};
  const kf::GemvPlan plan = kf::gemv_plan(1, &N, &K, 1, cus);
  if (!plan.x_lds) return fail(KF_ERR_UNSUPPORTED, "int4_gemv_fused: x of K=%d does not fit LDS", K);
  const kf::GemvFused fused = {prologue, aux, eps, residual};
  return hip_status(kf::gemv_fused_launch(plan, prob, fused, group_size, static_cast<hipStream_t>(stream)),
                    "int4_gemv_fused launch");
}

int kf_int4_gemv_qkv_rope(const void* x, const void* packed, const void* scales, void* y, int N, int K,
                          int group_size, const void* norm_weight, float eps, const kf_rope_cache* rope,
                          void* stream) {
  int st = check_common(x, packed, scales, y, 1, N, K, group_size);
  if (st) return st;
  if (!rope) return fail(KF_ERR_INVALID_ARG, "rope must be non-null");
  const kf_rope_cache& r = *rope;
  if (!r.cos || !r.sin || !r.pos || !r.cache_k || !r.cache_v)
    return fail(KF_ERR_INVALID_ARG, "rope: cos, sin, pos, cache_k and cache_v must be non-null");
  if (!aligned(r.cos, 2) || !aligned(r.sin, 2) || !aligned(r.cache_k, 2) || !aligned(r.cache_v, 2) ||
      !aligned(r.pos, 8))
    return fail(KF_ERR_INVALID_ARG, "rope: fp16 tables and caches must be 2-byte, pos 8-byte aligned");
  if (r.heads < 1 || r.kv_heads < 1 || r.head_dim < 2 || r.head_dim % 2 || r.max_seq < 1)
    return fail(KF_ERR_INVALID_ARG, "rope: need heads, kv_heads, max_seq >= 1 and an even head_dim, got %d, %d, %d, %d",
                r.heads, r.kv_heads, r.max_seq, r.head_dim);
  if ((long long)(r.heads + 2LL * r.kv_heads) * r.head_dim != N)
    return fail(KF_ERR_INVALID_ARG, "N=%d is not (heads + 2 kv_heads) * head_dim = %lld", N,
                (long long)(r.heads + 2LL * r.kv_heads) * r.head_dim);
  if (norm_weight && !aligned(norm_weight, 16)) return fail(KF_ERR_INVALID_ARG, "norm_weight must be 16-byte aligned");
  if (norm_weight && !(eps >= 0.0f && eps <= 3.0e38f))
    return fail(KF_ERR_INVALID_ARG, "eps must be finite and >= 0, got %g", (double)eps);
  if (K > KF_GEMV_FUSED_MAX_K)
    return fail(KF_ERR_UNSUPPORTED, "int4_gemv_qkv_rope needs K <= %d (x in LDS), got K=%d", KF_GEMV_FUSED_MAX_K, K);
  int cus = 0;
  if ((st = cu_count(&cus))) return st;
  const kf::GemvPlan plan = kf::gemv_plan(1, &N, &K, 1, cus);
  const kf::GemvProblem prob = {x, packed, scales, y, N, K};
  const kf::GemvFused fused = {norm_weight ? KF_PROLOGUE_RMSNORM : KF_PROLOGUE_NONE, norm_weight, eps, nullptr};
  const kf::GemvRope gr = {r.cos, r.sin, r.pos, r.cache_k, r.cache_v, r.heads, r.kv_heads, r.head_dim, r.max_seq};
  return hip_status(kf::gemv_qkv_rope_launch(prob, fused, gr, plan.unroll, group_size, static_cast<hipStream_t>(stream)),
                    "int4_gemv_qkv_rope launch");
}

size_t kf_int4_gemm_workspace_bytes(int M, int N, int K, int group_size) {
  if (M < 1 || N < 1 || K < 64 || K % 64 || (group_size != 64 && group_size != 128)) return 0;
  int cus = 0;
  if (cu_count(&cus)) return 0;
  return kf::gemm_workspace_bytes(kf::gemm_plan(M, N, K, cus), M, N);
}

int kf_int4_gemm_plan(int M, int N, int K, int group_size, int* kernel, int* num_kernels, int* splits, int* block_m,
                      int* block_n) {
  if (M < 1 || N < 1 || K < 64 || K % 64)
    return fail(KF_ERR_INVALID_ARG, "gemm plan needs M, N >= 1 and K a positive multiple of 64, got M=%d N=%d K=%d", M,
                N, K);
  if (group_size != 64 && group_size != 128)
    return fail(KF_ERR_INVALID_ARG, "group_size must be one of (64, 128), got %d", group_size);
  int cus = 0;
  const int st = cu_count(&cus);
  if (st) return st;
  const kf::GemmPlan p = kf::gemm_plan(M, N, K, cus);
  if (kernel) *kernel = p.skinny ? KF_GEMM_SKINNY : p.tile;
  if (num_kernels) *num_kernels = kf::gemm_num_tiles();
  if (splits) *splits = p.skinny ? 1 : p.splits;
  if (block_m) *block_m = p.skinny ? 0 : p.block_m;
  if (block_n) *block_n = p.skinny ? 0 : p.block_n;
  return KF_OK;
}

int kf_int4_gemm(const void* x, const void* packed, const void* scales, void* y, void* ws, size_t ws_bytes, int M,
                 int N, int K, int group_size, void* stream) {
  return gemm_entry(x, packed, scales, nullptr, nullptr, y, ws, ws_bytes, M, N, K, group_size, stream);
}

int kf_int4_gemm_noalloc(const void* x, const void* packed, const void* scales, void* y, int M, int N, int K,
                         int group_size, void* stream) {
  return gemm_entry(x, packed, scales, nullptr, nullptr, y, nullptr, 0, M, N, K, group_size, stream, true);
}

int kf_int4_mfma16_sizes(int N, int K, int group_size, size_t* packed_bytes, size_t* scales_bytes) {
  if (N < 1 || K < 128 || K % 128 || (group_size != 64 && group_size != 128))
    return fail(KF_ERR_INVALID_ARG, "MFMA-16 layout needs N >= 1, K a multiple of 128 and G in (64, 128), got N=%d K=%d G=%d",
                N, K, group_size);
  if (packed_bytes) *packed_bytes = kf::mfma16_packed_words(N, K) * 4;
  if (scales_bytes) *scales_bytes = kf::mfma16_scale_count(N, K, group_size) * 2;
  return KF_OK;
}

int kf_int4_reorder_mfma16(const void* packed, const void* scales, void* packed_r, void* scales_r, int N, int K,
                           int group_size, void* stream) {
  if (!packed || !scales || !packed_r || !scales_r)
    return fail(KF_ERR_INVALID_ARG, "packed, scales, packed_r and scales_r must be non-null");
  int st = kf_int4_mfma16_sizes(N, K, group_size, nullptr, nullptr);
  if (st) return st;
  if (!aligned(packed, 16) || !aligned(packed_r, 16)) return fail(KF_ERR_INVALID_ARG, "packed and packed_r must be 16-byte aligned");
  if (!aligned(scales, 2) || !aligned(scales_r, 2)) return fail(KF_ERR_INVALID_ARG, "scales and scales_r must be 2-byte aligned");
  return hip_status(kf::reorder_mfma16_launch(packed, scales, packed_r, scales_r, N, K, group_size,
                                              static_cast<hipStream_t>(stream)),
                    "reorder_mfma16 launch");
}

int kf_int4_gemm_mfma16(const void* x, const void* packed, const void* scales, const void* packed_r,
                        const void* scales_r, void* y, void* ws, size_t ws_bytes, int M, int N, int K, int group_size,
                        void* stream) {
  if (!packed_r || !scales_r) return fail(KF_ERR_INVALID_ARG, "packed_r and scales_r must be non-null");
  int st = kf_int4_mfma16_sizes(N, K, group_size, nullptr, nullptr);
  if (st) return st;
  if (!aligned(packed_r, 16) || !aligned(scales_r, 2)) return fail(KF_ERR_INVALID_ARG, "packed_r / scales_r misaligned");
  return gemm_entry(x, packed, scales, packed_r, scales_r, y, ws, ws_bytes, M, N, K, group_size, stream);
}

int kf_int4_quantize(const void* w, int dtype, void* packed, void* scales, int N, int K, int group_size,
                     void* stream) {
  if (!w || !packed || !scales) return fail(KF_ERR_INVALID_ARG, "w, packed and scales must be non-null");
  if (N < 1 || K < 1) return fail(KF_ERR_INVALID_ARG, "N, K must be positive, got N=%d K=%d", N, K);
  if (group_size != 64 && group_size != 128)
    return fail(KF_ERR_INVALID_ARG, "group_size must be one of (64, 128), got %d", group_size);
  if (K % group_size != 0)
    return fail(KF_ERR_INVALID_ARG, "K=%d is not a multiple of group_size=%d. Pad K or pick another group size.", K,
                group_size);
  if (dtype != KF_DTYPE_F32 && dtype != KF_DTYPE_F16 && dtype != KF_DTYPE_BF16)
    return fail(KF_ERR_INVALID_ARG, "dtype must be KF_DTYPE_F32, KF_DTYPE_F16 or KF_DTYPE_BF16, got %d", dtype);
  if (!aligned(w, 16)) return fail(KF_ERR_INVALID_ARG, "w must be 16-byte aligned");
  if (!aligned(packed, 4) || !aligned(scales, 2)) return fail(KF_ERR_INVALID_ARG, "packed / scales misaligned");
  return hip_status(kf::quantize_launch(w, dtype, packed, scales, N, K, group_size, static_cast<hipStream_t>(stream)),
                    "int4_quantize launch");
}

int kf_int4_dequant_fp16(const void* packed, const void* scales, void* w_hat, int N, int K, int group_size,
                         void* stream) {
  if (!packed || !scales || !w_hat) return fail(KF_ERR_INVALID_ARG, "packed, scales and w_hat must be non-null");
  if (N < 1 || K < 1) return fail(KF_ERR_INVALID_ARG, "N, K must be positive, got N=%d K=%d", N, K);
  if (group_size != 64 && group_size != 128)
    return fail(KF_ERR_INVALID_ARG, "group_size must be one of (64, 128), got %d", group_size);
  if (K % group_size != 0)
    return fail(KF_ERR_INVALID_ARG, "K=%d is not a multiple of group_size=%d", K, group_size);
  if (!aligned(packed, 4) || !aligned(scales, 2) || !aligned(w_hat, 16))
    return fail(KF_ERR_INVALID_ARG, "packed must be 4-byte, scales 2-byte and w_hat 16-byte aligned");
  return hip_status(kf::dequant_fp16_launch(packed, scales, w_hat, N, K, group_size,
                                            static_cast<hipStream_t>(stream)),
                    "dequant_fp16 launch");
}

static int bw_args(const void* a, size_t bytes, int* grid) {
  if (!a) return fail(KF_ERR_INVALID_ARG, "buffer must be non-null");
  if (bytes == 0 || bytes % 16) return fail(KF_ERR_INVALID_ARG, "bytes must be a positive multiple of 16");
  if (!aligned(a, 16)) return fail(KF_ERR_INVALID_ARG, "buffers must be 16-byte aligned");
  if (*grid <= 0) {
    int cus = 0;
    int st = cu_count(&cus);
    if (st) return st;
    *grid = 8 * cus;
  }
  return KF_OK;
}

int kf_bw_copy(const void* src, void* dst, size_t bytes, int grid_blocks, void* stream) {
  int st = bw_args(src, bytes, &grid_blocks);
  if (st) return st;
  if (!dst || !aligned(dst, 16)) return fail(KF_ERR_INVALID_ARG, "dst must be non-null and 16-byte aligned");
  return hip_status(kf::bw_copy_launch(src, dst, bytes, grid_blocks, static_cast<hipStream_t>(stream)), "bw_copy");
}

int kf_bw_read(const void* src, void* sink, size_t bytes, int grid_blocks, void* stream) {
  int st = bw_args(src, bytes, &grid_blocks);
  if (st) return st;
  if (!sink) return fail(KF_ERR_INVALID_ARG, "sink must be non-null (4 bytes per block)");
  return hip_status(kf::bw_read_launch(src, sink, bytes, grid_blocks, static_cast<hipStream_t>(stream)), "bw_read");
}

int kf_bw_read_store(const void* src, void* out, size_t bytes, int grid_blocks, void* stream) {
  int st = bw_args(src, bytes, &grid_blocks);
  if (st) return st;
  if (!out || !aligned(out, 2)) return fail(KF_ERR_INVALID_ARG, "out must be non-null and 2-byte aligned");
  return hip_status(kf::bw_read_store_launch(src, out, bytes, grid_blocks, static_cast<hipStream_t>(stream)),
                    "bw_read_store");
}

int kf_decode_argmax_step(const void* logits, int n, void* token, void* pos, void* history, int max_seq, void* mask,
                          void* stream) {
  if (!logits || !token || !pos || !history)
    return fail(KF_ERR_INVALID_ARG, "logits, token, pos and history must be non-null");
  if (n < 1 || max_seq < 1) return fail(KF_ERR_INVALID_ARG, "n and max_seq must be positive, got n=%d max_seq=%d", n,
                                        max_seq);
  if (!aligned(logits, 2) || (mask && !aligned(mask, 2)))
    return fail(KF_ERR_INVALID_ARG, "logits and mask must be 2-byte aligned");
  if (!aligned(token, 8) || !aligned(pos, 8) || !aligned(history, 8))
    return fail(KF_ERR_INVALID_ARG, "token, pos and history must be 8-byte aligned");
  return hip_status(kf::decode_argmax_launch(logits, n, token, pos, history, max_seq, mask,
                                             static_cast<hipStream_t>(stream)),
                    "decode_argmax_step launch");
}

int kf_bw_write(void* dst, size_t bytes, int grid_blocks, void* stream) {
  int st = bw_args(dst, bytes, &grid_blocks);
  if (st) return st;
  return hip_status(kf::bw_write_launch(dst, bytes, grid_blocks, static_cast<hipStream_t>(stream)), "bw_write");
}

}  // extern "C"
