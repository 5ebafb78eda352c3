// GPU check of the C ABI from plain C++, with no torch: buffers from hipMalloc, a stream from
// hipStreamCreate, the workspace sized by the library's own query.  It runs
// velograd_rmsnorm_residual_fwd and velograd_rmsnorm_residual_bwd (saved = h) on a bf16 case with
// a ragged row count and compares them with a double-precision restatement of the reference's
// fused.py:28-66 computed here from the same bf16 inputs:
//   h bit-exact (one fp32 add rounded to bf16); y within 1 bf16 ulp of the double value plus a
//   float32 term; inv_rms within 1e-5 relative; dx within 1 bf16 ulp plus the operand-scaled
//   floor 2^-20 * (|r gw| + |r xhat| mean|gw xhat|); dweight within 1e-3 of max(|ref|, rms(ref)).
// Also: an argument error comes back as a negative status with a message.  Prints "c_abi ok".
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "velograd_kernels.h"

#define HIP_OK(call)                                                              \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #call,               \
              hipGetErrorString(e_));                                             \
      return 1;                                                                   \
    }                                                                             \
  } while (0)

static float bf16_to_f(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f_to_bf16(float f) {  // round to nearest even (inputs here are finite)
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static double ulp_bf16(double v) {  // spacing of bf16 values around |v|
  const double a = fabs(v) > 1e-30 ? fabs(v) : 1e-30;
  return ldexp(1.0, ilogb(a) - 7);
}

// A fixed-seed generator of N(0, 1) values (Box-Muller over a 64-bit LCG).
struct Gauss {
  uint64_t s;
  double next_u() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return ((s >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  }
  double next() {
    const double u = next_u(), v = next_u();
    return sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v);
  }
};

int main() {
  const int64_t rows = 301, dim = 4096;
  const size_t n = (size_t)(rows * dim);
  const float eps = 1e-5f;
  Gauss g{12345};
  std::vector<uint16_t> x(n), r(n), w(dim), gy(n);
  for (auto& v : x) v = f_to_bf16((float)g.next());
  for (auto& v : r) v = f_to_bf16((float)g.next());
  for (auto& v : gy) v = f_to_bf16((float)g.next());
  for (auto& v : w) v = f_to_bf16((float)(1.0 + 0.1 * g.next()));

  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  void *dx_, *dr, *dw, *dy, *dh, *dg, *ddx, *dinv, *ddw, *ws;
  const size_t ws_bytes = velograd_rmsnorm_residual_bwd_workspace_bytes(rows, dim, dev);
  HIP_OK(hipMalloc(&dx_, n * 2));
  HIP_OK(hipMalloc(&dr, n * 2));
  HIP_OK(hipMalloc(&dw, dim * 2));
  HIP_OK(hipMalloc(&dy, n * 2));
  HIP_OK(hipMalloc(&dh, n * 2));
  HIP_OK(hipMalloc(&dg, n * 2));
  HIP_OK(hipMalloc(&ddx, n * 2));
  HIP_OK(hipMalloc(&dinv, rows * 4));
  HIP_OK(hipMalloc(&ddw, dim * 4));
  HIP_OK(hipMalloc(&ws, ws_bytes));
  HIP_OK(hipMemcpy(dx_, x.data(), n * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dr, r.data(), n * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dw, w.data(), dim * 2, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(dg, gy.data(), n * 2, hipMemcpyHostToDevice));

  int32_t rc = velograd_rmsnorm_residual_fwd(dx_, dr, dw, dy, dh, (float*)dinv, rows, dim, dim,
                                             dim, dim, dim, VELOGRAD_DTYPE_BF16,
                                             VELOGRAD_DTYPE_BF16, eps, st);
  if (rc != 0) {
    fprintf(stderr, "fwd: %d %s\n", rc, velograd_kernels_last_error());
    return 1;
  }
  rc = velograd_rmsnorm_residual_bwd(dg, dh, 1, dw, (const float*)dinv, nullptr, ddx, nullptr,
                                     (float*)ddw, ws, ws_bytes, rows, dim, dim, dim, dim, dim,
                                     dim, VELOGRAD_DTYPE_BF16, VELOGRAD_DTYPE_BF16, st);
  if (rc != 0) {
    fprintf(stderr, "bwd: %d %s\n", rc, velograd_kernels_last_error());
    return 1;
  }
  HIP_OK(hipStreamSynchronize(st));
  std::vector<uint16_t> y(n), h(n), dxo(n);
  std::vector<float> inv(rows), dwo(dim);
  HIP_OK(hipMemcpy(y.data(), dy, n * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(h.data(), dh, n * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(dxo.data(), ddx, n * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(inv.data(), dinv, rows * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(dwo.data(), ddw, dim * 4, hipMemcpyDeviceToHost));

  int bad = 0;
  std::vector<double> dwref(dim, 0.0);
  for (int64_t i = 0; i < rows; ++i) {
    // forward (fused.py:39-46), h from the fp32 add as the kernel forms it
    std::vector<double> hh(dim);
    double ss = 0.0;
    for (int64_t j = 0; j < dim; ++j) {
      const float hf = bf16_to_f(x[i * dim + j]) + bf16_to_f(r[i * dim + j]);
      if (h[i * dim + j] != f_to_bf16(hf)) ++bad;
      hh[j] = hf;
      ss += hh[j] * hh[j];
    }
    const double rr = 1.0 / sqrt(ss / dim + (double)eps);
    if (fabs(inv[i] - rr) > 1e-5 * rr) ++bad;
    for (int64_t j = 0; j < dim; ++j) {
      const double yr = hh[j] * rr * bf16_to_f(w[j]);
      if (fabs(bf16_to_f(y[i * dim + j]) - yr) > ulp_bf16(yr) + 1e-6 * fabs(yr)) ++bad;
    }
    // backward (fused.py:58-65) with the device's h and inv_rms, as the kernel receives them
    const double r32 = inv[i];
    double m = 0.0, mabs = 0.0;
    std::vector<double> gw(dim), xh(dim);
    for (int64_t j = 0; j < dim; ++j) {
      gw[j] = (double)bf16_to_f(gy[i * dim + j]) * bf16_to_f(w[j]);
      xh[j] = (double)bf16_to_f(h[i * dim + j]) * r32;
      m += gw[j] * xh[j];
      mabs += fabs(gw[j] * xh[j]);
      dwref[j] += (double)bf16_to_f(gy[i * dim + j]) * xh[j];
    }
    m /= dim;
    mabs /= dim;
    for (int64_t j = 0; j < dim; ++j) {
      const double d = r32 * (gw[j] - xh[j] * m);
      const double floor = ldexp(1.0, -20) * (fabs(r32 * gw[j]) + fabs(r32 * xh[j]) * mabs);
      if (fabs(bf16_to_f(dxo[i * dim + j]) - d) > ulp_bf16(d) + floor) ++bad;
    }
  }
  double rms = 0.0;
  for (double v : dwref) rms += v * v;
  rms = sqrt(rms / dim);
  for (int64_t j = 0; j < dim; ++j) {
    const double sc = fabs(dwref[j]) > rms ? fabs(dwref[j]) : rms;
    if (fabs(dwo[j] - dwref[j]) > 1e-3 * sc) ++bad;
  }

  // an argument error: negative status, message, nothing launched
  rc = velograd_rmsnorm_residual_fwd(dx_, dr, dw, dy, dh, (float*)dinv, rows, -1, dim, dim, dim,
                                     dim, VELOGRAD_DTYPE_BF16, VELOGRAD_DTYPE_BF16, eps, st);
  if (rc >= 0 || strlen(velograd_kernels_last_error()) == 0) ++bad;

  for (void* p : {dx_, dr, dw, dy, dh, dg, ddx, dinv, ddw, ws}) HIP_OK(hipFree(p));
  HIP_OK(hipStreamDestroy(st));
  if (bad) {
    fprintf(stderr, "c_abi: %d mismatches\n", bad);
    return 1;
  }
  printf("c_abi ok (%s)\n", velograd_kernels_version());
  return 0;
}
