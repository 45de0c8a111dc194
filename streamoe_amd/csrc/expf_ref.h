// expf_ref.h — the router softmax's exponential, bit for bit the one the
// reference's CPU path calls.
//
// moe_router.rs:64 computes `(*v - max_val).exp()`, i.e. the platform
// libm's expf. On Linux that is glibc's (sysdeps/ieee754/flt-32/e_expf.c,
// the published ARM optimized-routines method by Szabolcs Nagy): with
// N = 32, x * N / ln2 = k + r rounded to nearest by the 1.5 * 2^52 shift,
// 2^(k/N) = T[k mod N] with k / N added to the exponent field, and
// 2^(r/N) ~ C0 r^3 + C1 r^2 + C2 r + 1, all in double, rounded once to
// float. The x86-64 build selected on FMA hardware contracts every
// multiply-add, which is what is written here (explicit fma).
//
// T[i] is the double nearest 2^(i/32) with i << 47 subtracted from its bit
// pattern, computed to 60 digits and rounded; C0..C2 are the method's
// published minimax coefficients. The device's own expf differs from
// glibc's in the last bit on part of the range (and glibc's is not
// correctly rounded: 97,052 of the 1,120,927,745 floats in [-104, 0]), so
// a softmax that must reproduce the reference's probabilities bit for bit
// uses this one. It is checked against glibc's expf on every float in
// [-0x1.9fe368p6, 0] on the CPU (tests/test_expf_ref.py) and on the GPU
// (tests/test_gpu_softmax.py).
//
// Usable from host and device code: the lookup of T is a parameter (the
// device kernels take it from a register table by lane permute).
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define SMOE_HD __host__ __device__
#else
#define SMOE_HD
#endif

namespace smoe {

static constexpr uint64_t kExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

#if defined(__HIPCC__) || defined(__HIP__)
// The table in device memory, for lookups by index (expf_ref_dev).
static __device__ const uint64_t kExpTabDev[32] = {
    kExpTab[0],  kExpTab[1],  kExpTab[2],  kExpTab[3],  kExpTab[4],  kExpTab[5],  kExpTab[6],  kExpTab[7],
    kExpTab[8],  kExpTab[9],  kExpTab[10], kExpTab[11], kExpTab[12], kExpTab[13], kExpTab[14], kExpTab[15],
    kExpTab[16], kExpTab[17], kExpTab[18], kExpTab[19], kExpTab[20], kExpTab[21], kExpTab[22], kExpTab[23],
    kExpTab[24], kExpTab[25], kExpTab[26], kExpTab[27], kExpTab[28], kExpTab[29], kExpTab[30], kExpTab[31]};
#endif

SMOE_HD inline double expref_asd(uint64_t u) {
  double d;
  memcpy(&d, &u, 8);
  return d;
}
SMOE_HD inline uint64_t expref_asu(double d) {
  uint64_t u;
  memcpy(&u, &d, 8);
  return u;
}

// exp(x) as glibc's expf computes it. `lookup(i)` returns kExpTab[i]
// (0 <= i < 32) and is called exactly once, unconditionally, so a device
// lookup by lane permute sees every lane active. Branch-free: the special
// cases of glibc (|x| >= 88 or NaN) are selected at the end.
template <typename Lookup>
SMOE_HD inline float expf_ref(float x, Lookup lookup) {
#pragma clang fp contract(off)
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  const double kShift = 0x1.8p+52;
  const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = expref_asu(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = lookup((uint32_t)(ki & 31u)) + (ki << 47);
  const double s = expref_asd(t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  float res = (float)y;
  // glibc's special cases: abstop = top 12 bits of |x| >= those of 88.0f.
  uint32_t ux;
  memcpy(&ux, &x, 4);
  if (((ux >> 20) & 0x7ffu) >= 0x42bu) {
    if (ux == 0xff800000u) res = 0.0f;               // -inf
    else if (((ux >> 20) & 0x7ffu) >= 0x7f8u) res = x + x;  // +inf, NaN
    else if (x > 0x1.62e42ep6f) res = __builtin_inff();      // overflow
    else if (x < -0x1.9fe368p6f) res = 0.0f;                 // underflow
  }
  return res;
}

#if defined(__HIPCC__) || defined(__HIP__)
// expf_ref with the table read from device memory (one load per call, any
// lanes active).
__device__ inline float expf_ref_dev(float x) {
  return expf_ref(x, [](uint32_t i) { return kExpTabDev[i]; });
}

// The reference's sigmoid, 1 / (1 + exp(-x)) (cpu_ops.rs:22-25), with
// glibc's expf and a correctly rounded division.
__device__ inline float sigmoid_ref(float x) { return __fdiv_rn(1.0f, 1.0f + expf_ref_dev(-x)); }
#endif

}  // namespace smoe
