// Torch-free correctness workload for libkf_int4.so (test infrastructure).
//
// The counterpart of the reference's csrc/micro/sanitize_gemm.cu:31-95: the reference's LCG
// inputs (restated in oracle/kf_oracle.c), the host packer, a double-precision reference, the
// GEMV at every M <= 8 and the GEMM at every M (with split-K on these small grids), all through
// the C ABI of include/kf_int4.h with plain HIP device memory: no torch, no Python.  It is
// built twice by the package build: plainly and with AddressSanitizer on this host code.
//
// Checks: max|y - ref| <= 2e-3 * max|ref| (the reference's tolerance, tests/test_gemm.py:17),
// bit-exact GPU dequantization, the ABI's status codes on bad arguments, and that a guard band
// around y is never written.  Exit status 0 on success; one line per case on stdout.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kf_int4.h"

extern "C" {
void kfo_lcg_workload(int group, int n, int k, const int* ms, int nms, int8_t* q, uint16_t* scales, int32_t* packed,
                      uint16_t* xcat);
void kfo_dequant_fp16(const int32_t* packed, const uint16_t* scales, int n, int k, int group, uint16_t* out);
void kfo_ref_f64(const uint16_t* x, const int32_t* packed, const uint16_t* scales, int m, int n, int k, int group,
                 double* y);
float kfo_f16_to_f32(uint16_t h);
uint16_t kfo_f32_to_f16(float f);
double kfo_max_rel_err_f16(const uint16_t* y, const double* ref, size_t n);
}

namespace {

int g_failures = 0;

void check(bool ok, const char* what) {
  if (!ok) {
    ++g_failures;
    std::printf("FAIL %s\n", what);
  }
}

bool hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    ++g_failures;
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
    return false;
  }
  return true;
}

// RAII device allocation (the role of the reference's DeviceBuffer, csrc/common/cuda_utils.cuh:18-50).
class DeviceBuffer {
 public:
  explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
    if (bytes_ && hipMalloc(&ptr_, bytes_) != hipSuccess) ptr_ = nullptr;
  }
  ~DeviceBuffer() {
    if (ptr_) (void)hipFree(ptr_);
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  void* get() const { return ptr_; }
  size_t bytes() const { return bytes_; }
  bool upload(const void* src, size_t n) { return hipMemcpy(ptr_, src, n, hipMemcpyHostToDevice) == hipSuccess; }
  bool download(void* dst, size_t n) const { return hipMemcpy(dst, ptr_, n, hipMemcpyDeviceToHost) == hipSuccess; }

 private:
  void* ptr_ = nullptr;
  size_t bytes_;
};

// RAII hipEvent pair timing one region on a stream (the role of the reference's GpuTimer,
// csrc/common/timer.cuh:14-75).
class EventTimer {
 public:
  explicit EventTimer(hipStream_t s) : s_(s) {
    (void)hipEventCreate(&a_);
    (void)hipEventCreate(&b_);
    (void)hipEventRecord(a_, s_);
  }
  ~EventTimer() {
    (void)hipEventDestroy(a_);
    (void)hipEventDestroy(b_);
  }
  float stop_us() {
    float ms = 0.f;
    (void)hipEventRecord(b_, s_);
    (void)hipEventSynchronize(b_);
    (void)hipEventElapsedTime(&ms, a_, b_);
    return ms * 1e3f;
  }

 private:
  hipStream_t s_;
  hipEvent_t a_{}, b_{};
};

constexpr uint16_t kGuard = 0x7E11;  // an fp16 NaN pattern the kernels never produce
constexpr int kGuardElems = 64;

// The pass rule's ratio from the C oracle (kfo_max_rel_err_f16, pinned by tests/test_oracle.py):
// NaN for a NaN output, so "err <= 2e-3" fails on it.
double max_rel_err(const std::vector<uint16_t>& y, const std::vector<double>& ref) {
  if (y.size() < ref.size()) return NAN;
  return kfo_max_rel_err_f16(y.data(), ref.data(), ref.size());
}

void run_group(int group, hipStream_t stream) {
  const int n = 128, k = 1024;  // the reference's sizes (sanitize_gemm.cu:33-34)
  const int ms[] = {1, 3, 8, 9, 16, 17, 33, 64, 65};
  const int nms = sizeof(ms) / sizeof(ms[0]);
  int msum = 0;
  for (int m : ms) msum += m;
  std::vector<int8_t> q((size_t)n * k);
  std::vector<uint16_t> scales((size_t)n * (k / group)), xcat((size_t)msum * k);
  std::vector<int32_t> packed((size_t)n * (k / 8));
  kfo_lcg_workload(group, n, k, ms, nms, q.data(), scales.data(), packed.data(), xcat.data());

  DeviceBuffer d_packed(packed.size() * 4), d_scales(scales.size() * 2);
  if (!d_packed.get() || !d_scales.get()) return check(false, "hipMalloc weights");
  check(d_packed.upload(packed.data(), d_packed.bytes()) && d_scales.upload(scales.data(), d_scales.bytes()),
        "upload weights");

  // Dequantization, bit for bit.
  {
    std::vector<uint16_t> want((size_t)n * k), got((size_t)n * k);
    kfo_dequant_fp16(packed.data(), scales.data(), n, k, group, want.data());
    DeviceBuffer d_w(got.size() * 2);
    const int st = kf_int4_dequant_fp16(d_packed.get(), d_scales.get(), d_w.get(), n, k, group, stream);
    check(st == KF_OK, kf_last_error());
    hip_ok(hipStreamSynchronize(stream), "dequant sync");
    check(d_w.download(got.data(), got.size() * 2), "download w_hat");
    const bool same = std::memcmp(got.data(), want.data(), got.size() * 2) == 0;
    std::printf("G=%d dequant_fp16 bit-exact=%d\n", group, (int)same);
    check(same, "dequant_fp16 bit-exact");
  }

  size_t off = 0;
  for (int m : ms) {
    const uint16_t* x = xcat.data() + off;
    off += (size_t)m * k;
    std::vector<double> ref((size_t)m * n);
    kfo_ref_f64(x, packed.data(), scales.data(), m, n, k, group, ref.data());
    DeviceBuffer d_x((size_t)m * k * 2), d_y(((size_t)m * n + 2 * kGuardElems) * 2);
    check(d_x.upload(x, d_x.bytes()), "upload x");
    std::vector<uint16_t> guard((size_t)m * n + 2 * kGuardElems, kGuard);
    uint16_t* y = static_cast<uint16_t*>(d_y.get()) + kGuardElems;

    for (int path = 0; path < 2; ++path) {  // 0: GEMV (M <= 8), 1: GEMM
      if (path == 0 && m > 8) continue;
      check(d_y.upload(guard.data(), d_y.bytes()), "upload guard");
      int st;
      float us;
      size_t ws_bytes = 0;
      {
        const size_t need = path ? kf_int4_gemm_workspace_bytes(m, n, k, group) : 0;
        DeviceBuffer ws(need);
        ws_bytes = need;
        EventTimer t(stream);
        st = path ? kf_int4_gemm(d_x.get(), d_packed.get(), d_scales.get(), y, ws.get(), need, m, n, k, group, stream)
                  : kf_int4_gemv(d_x.get(), d_packed.get(), d_scales.get(), y, m, n, k, group, stream);
        us = t.stop_us();
        hip_ok(hipStreamSynchronize(stream), "kernel sync");
      }
      check(st == KF_OK, kf_last_error());
      std::vector<uint16_t> all(guard.size());
      check(d_y.download(all.data(), all.size() * 2), "download y");
      bool guard_ok = true;
      for (int i = 0; i < kGuardElems; ++i)
        guard_ok &= all[i] == kGuard && all[all.size() - 1 - i] == kGuard;
      std::vector<uint16_t> out(all.begin() + kGuardElems, all.end() - kGuardElems);
      const double err = max_rel_err(out, ref);
      std::printf("G=%d M=%d %s err=%.3e guard=%d ws=%zu time=%.1fus\n", group, m, path ? "gemm" : "gemv", err,
                  (int)guard_ok, ws_bytes, us);
      check(err <= 2e-3, "tolerance");
      check(guard_ok, "guard band");
    }
  }
}

uint16_t h16(double v) { return kfo_f32_to_f16((float)v); }
double f64(uint16_t v) { return (double)kfo_f16_to_f32(v); }

// The fused decode entry points on one token of the same workload: the residual bit for bit
// against kf_int4_gemv plus a host fp16 add; the RMSNorm and SwiGLU prologues against the
// double-precision reference fed the prologue computed on the host; the q|k|v launch against a
// host rotation of kf_int4_gemv's output, with exactly the cache entries it must write.
void run_fused(int group, hipStream_t stream) {
  const int n = 128, k = 1024;
  const int ms[] = {1, 1};  // x, and a second row (up, norm weight, residual source)
  std::vector<int8_t> q((size_t)n * k);
  std::vector<uint16_t> scales((size_t)n * (k / group)), xcat((size_t)2 * k);
  std::vector<int32_t> packed((size_t)n * (k / 8));
  kfo_lcg_workload(group, n, k, ms, 2, q.data(), scales.data(), packed.data(), xcat.data());
  const uint16_t* x = xcat.data();
  const uint16_t* u = xcat.data() + k;
  std::vector<uint16_t> w(k), r(n);
  for (int i = 0; i < k; ++i) w[i] = h16(std::fabs(f64(u[i])) + 0.5);
  for (int i = 0; i < n; ++i) r[i] = h16(0.5 * ((i * 37) % 17) - 4.0);
  DeviceBuffer d_packed(packed.size() * 4), d_scales(scales.size() * 2), d_x(k * 2), d_u(k * 2), d_w(k * 2),
      d_r(n * 2), d_y(n * 2), d_y0(n * 2);
  check(d_packed.upload(packed.data(), d_packed.bytes()) && d_scales.upload(scales.data(), d_scales.bytes()) &&
            d_x.upload(x, k * 2) && d_u.upload(u, k * 2) && d_w.upload(w.data(), k * 2) && d_r.upload(r.data(), n * 2),
        "upload fused inputs");
  std::vector<uint16_t> y0(n), y(n);
  int st = kf_int4_gemv(d_x.get(), d_packed.get(), d_scales.get(), d_y0.get(), 1, n, k, group, stream);
  check(st == KF_OK, kf_last_error());
  hip_ok(hipStreamSynchronize(stream), "gemv sync");
  check(d_y0.download(y0.data(), n * 2), "download y0");

  // residual: fp16(r + fp16(x W^T)), bit for bit
  st = kf_int4_gemv_fused(d_x.get(), d_packed.get(), d_scales.get(), d_y.get(), 1, n, k, group, KF_PROLOGUE_NONE,
                          nullptr, 0.0f, d_r.get(), stream);
  check(st == KF_OK, kf_last_error());
  hip_ok(hipStreamSynchronize(stream), "fused sync");
  check(d_y.download(y.data(), n * 2), "download y");
  bool same = true;
  for (int i = 0; i < n; ++i) same &= y[i] == kfo_f32_to_f16(kfo_f16_to_f32(r[i]) + kfo_f16_to_f32(y0[i]));
  std::printf("G=%d fused residual bit-exact=%d\n", group, (int)same);
  check(same, "fused residual bit-exact");

  // prologues
  for (int pro : {KF_PROLOGUE_RMSNORM, KF_PROLOGUE_SWIGLU}) {
    std::vector<uint16_t> xp(k);
    if (pro == KF_PROLOGUE_RMSNORM) {
      double ss = 0.0;
      for (int i = 0; i < k; ++i) ss += f64(x[i]) * f64(x[i]);
      const double rstd = 1.0 / std::sqrt(ss / k + 1e-5);
      for (int i = 0; i < k; ++i) xp[i] = h16(f64(x[i]) * rstd * f64(w[i]));
    } else {
      for (int i = 0; i < k; ++i) {
        const double g = f64(x[i]);
        xp[i] = h16(f64(h16(g / (1.0 + std::exp(-g)))) * f64(u[i]));
      }
    }
    std::vector<double> ref(n);
    kfo_ref_f64(xp.data(), packed.data(), scales.data(), 1, n, k, group, ref.data());
    st = kf_int4_gemv_fused(d_x.get(), d_packed.get(), d_scales.get(), d_y.get(), 1, n, k, group, pro,
                            pro == KF_PROLOGUE_RMSNORM ? d_w.get() : d_u.get(), 1e-5f, nullptr, stream);
    check(st == KF_OK, kf_last_error());
    hip_ok(hipStreamSynchronize(stream), "fused prologue sync");
    check(d_y.download(y.data(), n * 2), "download y");
    const double err = max_rel_err(y, ref);
    std::printf("G=%d fused %s err=%.3e\n", group, pro == KF_PROLOGUE_RMSNORM ? "rmsnorm" : "swiglu", err);
    check(err <= 2e-3, "fused prologue tolerance");
  }
  st = kf_int4_gemv_fused(d_x.get(), d_packed.get(), d_scales.get(), d_y.get(), 2, n, k, group, KF_PROLOGUE_NONE,
                          nullptr, 0.0f, nullptr, stream);
  check(st == KF_ERR_UNSUPPORTED, "fused M = 2 rejected");

  // q|k|v with RoPE and the cache writes: 2 q heads, 1 k head, 1 v head of 32 dims (N = 128).
  const int heads = 2, kvh = 1, d = 32, smax = 8, pos = 3;
  std::vector<uint16_t> cs((size_t)smax * d), sn((size_t)smax * d);
  for (int p = 0; p < smax; ++p)
    for (int j = 0; j < d / 2; ++j) {
      const double a = p * std::pow(10000.0, -2.0 * j / d);
      cs[(size_t)p * d + j] = cs[(size_t)p * d + j + d / 2] = h16(std::cos(a));
      sn[(size_t)p * d + j] = h16(-std::sin(a));
      sn[(size_t)p * d + j + d / 2] = h16(std::sin(a));
    }
  const int64_t pos64 = pos;
  std::vector<uint16_t> ck((size_t)kvh * d * smax, kGuard), cv((size_t)kvh * smax * d, kGuard);
  DeviceBuffer d_cs(cs.size() * 2), d_sn(sn.size() * 2), d_pos(8), d_ck(ck.size() * 2), d_cv(cv.size() * 2);
  check(d_cs.upload(cs.data(), cs.size() * 2) && d_sn.upload(sn.data(), sn.size() * 2) && d_pos.upload(&pos64, 8) &&
            d_ck.upload(ck.data(), ck.size() * 2) && d_cv.upload(cv.data(), cv.size() * 2),
        "upload rope inputs");
  const kf_rope_cache rc = {d_cs.get(), d_sn.get(), d_pos.get(), d_ck.get(), d_cv.get(), heads, kvh, d, smax};
  st = kf_int4_gemv_qkv_rope(d_x.get(), d_packed.get(), d_scales.get(), d_y.get(), n, k, group, nullptr, 0.0f, &rc,
                             stream);
  check(st == KF_OK, kf_last_error());
  hip_ok(hipStreamSynchronize(stream), "qkv rope sync");
  check(d_y.download(y.data(), n * 2) && d_ck.download(ck.data(), ck.size() * 2) &&
            d_cv.download(cv.data(), cv.size() * 2),
        "download rope outputs");
  double dmax = 0.0, rmax = 0.0;
  const int nrope = (heads + kvh) * d;
  for (int hh = 0; hh < heads + kvh; ++hh)
    for (int dim = 0; dim < d; ++dim) {
      const int partner = dim < d / 2 ? dim + d / 2 : dim - d / 2;
      const double t = f64(h16(f64(y0[hh * d + dim]) * f64(cs[(size_t)pos * d + dim])));
      const double want = f64(h16(t + f64(y0[hh * d + partner]) * f64(sn[(size_t)pos * d + dim])));
      dmax = std::fmax(dmax, std::fabs(f64(y[hh * d + dim]) - want));
      rmax = std::fmax(rmax, std::fabs(want));
    }
  bool v_same = true, cache_ok = true;
  for (int i = nrope; i < n; ++i) v_same &= y[i] == y0[i];
  for (int dim = 0; dim < d; ++dim)
    for (int p = 0; p < smax; ++p) {
      const uint16_t kw = ck[(size_t)dim * smax + p], vw = cv[(size_t)p * d + dim];
      cache_ok &= p == pos ? (kw == y[heads * d + dim] && vw == y[nrope + dim]) : (kw == kGuard && vw == kGuard);
    }
  std::printf("G=%d qkv rope max|diff|=%.3e (max|ref| %.3e) v bit-exact=%d cache=%d\n", group, dmax, rmax,
              (int)v_same, (int)cache_ok);
  check(dmax <= 2e-3 * rmax, "qkv rope tolerance");
  check(v_same, "qkv rope v rows bit-exact");
  check(cache_ok, "qkv rope cache entries");
}

void run_rejections(hipStream_t stream) {
  DeviceBuffer a(1 << 16), b(1 << 16), c(1 << 16), d(1 << 16);
  int st = kf_int4_gemv(nullptr, b.get(), c.get(), d.get(), 1, 64, 256, 128, stream);
  check(st == KF_ERR_INVALID_ARG, "null x rejected");
  st = kf_int4_gemv(a.get(), b.get(), c.get(), d.get(), 1, 64, 256, 96, stream);
  check(st == KF_ERR_INVALID_ARG && std::strstr(kf_last_error(), "group_size") != nullptr, "group 96 rejected");
  st = kf_int4_gemm(a.get(), b.get(), c.get(), d.get(), nullptr, 0, 16, 100, 256, 128, stream);
  check(st == KF_ERR_UNSUPPORTED, "gemm N % 64 rejected");
  st = kf_int4_quantize(a.get(), 7, b.get(), c.get(), 16, 256, 128, stream);
  check(st == KF_ERR_INVALID_ARG, "quantize dtype rejected");
  std::printf("rejections checked\n");
}

}  // namespace

int main() {
  if (kf_abi_version() != KF_ABI_VERSION) {
    std::printf("FAIL ABI version %d != %d\n", kf_abi_version(), KF_ABI_VERSION);
    return 1;
  }
  hipStream_t stream;
  if (!hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) return 1;
  run_group(64, stream);
  run_group(128, stream);
  run_fused(64, stream);
  run_fused(128, stream);
  run_rejections(stream);
  (void)hipStreamDestroy(stream);
  std::printf("%s (%d failures)\n", g_failures ? "FAILED" : "OK", g_failures);
  return g_failures ? 1 : 0;
}
