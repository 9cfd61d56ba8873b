// smp_math.hpp -- bit-exact binary64 exp/log, SplitMix64 mixing and the
// token-keyed Gumbel noise of YASAKANI's sampler, as gfx950 device code.
//
// The algorithms must produce the same bits as the reference's portable
// math (crates/yskn-ref/src/portable_math.rs:224-364, itself the fdlibm
// e_exp.c / e_log.c method) and hash (output_head_sampler.rs:214-228).
// The operation order is therefore fixed by the reference; every binary64
// multiply, add and divide below is a separately rounded IEEE operation.
// The translation unit is compiled with -ffp-contract=off so that no
// multiply/add pair is fused, and division is IEEE correctly rounded.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yskn {

__device__ __forceinline__ double pm_hilo(uint32_t hi, uint32_t lo) {
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | (uint64_t)lo));
}
__device__ __forceinline__ uint64_t pm_bits(double x) { return (uint64_t)__double_as_longlong(x); }

// exp(value) in binary64; portable_math.rs:224-283.
__device__ __forceinline__ double exp_d_inline(double value) {
  const uint64_t b = pm_bits(value);
  const uint32_t hi = (uint32_t)(b >> 32), lo = (uint32_t)b;
  const bool neg = (hi >> 31) != 0;
  const uint32_t ahi = hi & 0x7fffffffu;
  if (ahi >= 0x40862e42u) {
    if (ahi >= 0x7ff00000u) {
      if (((ahi & 0x000fffffu) | lo) != 0) return value + value;
      return neg ? 0.0 : value;
    }
    if (value > pm_hilo(0x40862e42u, 0xfefa39efu)) return __longlong_as_double(0x7ff0000000000000ll);
    if (value < pm_hilo(0xc0874910u, 0xd52d3051u)) return 0.0;
  }
  const double ln2_hi = pm_hilo(0x3fe62e42u, 0xfee00000u);
  const double ln2_lo = pm_hilo(0x3dea39efu, 0x35793c76u);
  double h = 0.0, l = 0.0, r = value;
  int32_t k = 0;
  if (ahi > 0x3fd62e42u) {
    if (ahi < 0x3ff0a2b2u) {
      h = value - (neg ? -ln2_hi : ln2_hi);
      l = neg ? -ln2_lo : ln2_lo;
      k = neg ? -1 : 1;
    } else {
      double t = pm_hilo(0x3ff71547u, 0x652b82feu) * value;
      t = t + (neg ? -0.5 : 0.5);
      k = (int32_t)t;  // truncation toward zero; |t| < 1100 here
      const double kf = (double)k;
      const double kh = kf * ln2_hi;
      h = value - kh;
      l = kf * ln2_lo;
    }
    r = h - l;
  } else if (ahi < 0x3e300000u) {
    return 1.0 + value;
  }
  const double s = r * r;
  double p = s * pm_hilo(0x3e663769u, 0x72bea4d0u);
  p = pm_hilo(0xbebbbd41u, 0xc5d26bf1u) + p;
  p = s * p;
  p = pm_hilo(0x3f11566au, 0xaf25de2cu) + p;
  p = s * p;
  p = pm_hilo(0xbf66c16cu, 0x16bebd93u) + p;
  p = s * p;
  p = pm_hilo(0x3fc55555u, 0x5555553eu) + p;
  const double sp = s * p;
  const double c = r - sp;
  const double rc = r * c;
  if (k == 0) {
    const double q = rc / (c - 2.0);
    return 1.0 - (q - r);
  }
  const double q = rc / (2.0 - c);
  const double y = 1.0 - ((l - q) - h);
  const int32_t adj = (k >= -1021) ? k : k + 1000;
  const uint64_t yb = pm_bits(y);
  const uint32_t yhi = (uint32_t)(yb >> 32) + (uint32_t)adj * 1048576u;
  const double scaled = pm_hilo(yhi, (uint32_t)yb);
  if (k >= -1021) return scaled;
  return scaled * pm_hilo(0x01700000u, 0u);
}

// log(value) in binary64 without a zero special case; portable_math.rs:297-364.
__device__ __forceinline__ double log_d_inline(double value) {
  int32_t hx = (int32_t)(uint32_t)(pm_bits(value) >> 32);
  int32_t k = 0;
  if (hx < 0x00100000) {
    value = value * pm_hilo(0x43500000u, 0u);
    k = -54;
    hx = (int32_t)(uint32_t)(pm_bits(value) >> 32);
  }
  k += (hx >> 20) - 1023;
  hx &= 0x000fffff;
  const int32_t i = (hx + 0x00095f64) & 0x00100000;
  value = pm_hilo((uint32_t)(hx | (i ^ 0x3ff00000)), (uint32_t)pm_bits(value));
  k += i >> 20;
  const double ln2_hi = pm_hilo(0x3fe62e42u, 0xfee00000u);
  const double ln2_lo = pm_hilo(0x3dea39efu, 0x35793c76u);
  const double f = value - 1.0;
  const double dk = (double)k;
  if ((0x000fffff & (2 + hx)) < 3) {
    if (f == 0.0) {
      if (k == 0) return 0.0;
      const double a = dk * ln2_hi;
      const double b2 = dk * ln2_lo;
      return a + b2;
    }
    const double ff = f * f;
    double t = pm_hilo(0x3fd55555u, 0x55555555u) * f;
    t = 0.5 - t;
    const double R = ff * t;
    if (k == 0) return f - R;
    const double a = dk * ln2_hi;
    const double b2 = dk * ln2_lo;
    return a - ((R - b2) - f);
  }
  const double s = f / (2.0 + f);
  const double z = s * s;
  const double w = z * z;
  const int32_t j = (hx - 0x0006147a) | (0x0006b851 - hx);
  double t2 = w * pm_hilo(0x3fc39a09u, 0xd078c69fu);
  t2 = pm_hilo(0x3fcc71c5u, 0x1d8e78afu) + t2;
  t2 = w * t2;
  t2 = pm_hilo(0x3fd99999u, 0x9997fa04u) + t2;
  t2 = w * t2;
  double t1 = w * pm_hilo(0x3fc2f112u, 0xdf3e5244u);
  t1 = pm_hilo(0x3fc74664u, 0x96cb03deu) + t1;
  t1 = w * t1;
  t1 = pm_hilo(0x3fd24924u, 0x94229359u) + t1;
  t1 = w * t1;
  t1 = pm_hilo(0x3fe55555u, 0x55555593u) + t1;
  t1 = z * t1;
  const double R = t1 + t2;
  if (j > 0) {
    double hfsq = 0.5 * f;
    hfsq = hfsq * f;
    double u = hfsq + R;
    u = s * u;
    if (k == 0) {
      u = hfsq - u;
      return f - u;
    }
    const double b2 = dk * ln2_lo;
    u = u + b2;
    u = hfsq - u;
    u = u - f;
    const double a = dk * ln2_hi;
    return a - u;
  }
  double u = f - R;
  u = s * u;
  if (k == 0) return f - u;
  const double b2 = dk * ln2_lo;
  u = u - b2;
  u = u - f;
  const double a = dk * ln2_hi;
  return a - u;
}

// Out-of-line copies for the block-wide paths (code size); the per-wave
// draw inlines the bodies above.
__device__ __noinline__ double exp_d(double value) { return exp_d_inline(value); }
__device__ __noinline__ double log_d(double value) { return log_d_inline(value); }

// SplitMix64 finaliser; output_head_sampler.rs:214-219.
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Token-keyed Gumbel noise given the per-(seed, position) hash
// b = mix64(mix64(seed) ^ position); output_head_sampler.rs:221-228.
template <bool INLINE = false>
__device__ __forceinline__ double gumbel_from_key(uint64_t b, uint32_t token) {
  const uint64_t h = mix64(b ^ ((uint64_t)token * 0xd6e8feb86659fd93ull));
  double u = (double)(h >> 11) + 0.5;
  u = u * (1.0 / 9007199254740992.0);
  if (INLINE) return -log_d_inline(-log_d_inline(u));
  return -log_d(-log_d(u));
}

__device__ __forceinline__ uint64_t position_key(uint64_t seed, uint64_t position) {
  return mix64(mix64(seed) ^ position);
}

// e^z for z <= 0 within 2^-46 (relative): Cody-Waite reduction by ln 2 with
// fused multiply-adds, a degree-11 Taylor polynomial on |r| <= 0.35
// (truncation below 2^-47; 2^-46.7 is the largest error over 2e7
// arguments), then ldexp. Not the reference's exp_d: used only where its
// error is bounded above (the certified dense tail of smp_kernels.hip).
__device__ __forceinline__ double exp_approx(double z) {
  z = z >= -700.0 ? z : -700.0;  // (a NaN, from a padding lane, too: every value below stays defined)
  const double t = __builtin_rint(z * 1.4426950408889634);
  double r = __builtin_fma(-t, 0.6931471805599453, z);
  r = __builtin_fma(-t, 2.3190468138462996e-17, r);
  double p = 2.505210838544172e-08;                // 1/11!
  p = __builtin_fma(p, r, 2.755731922398589e-07);  // 1/10!
  p = __builtin_fma(p, r, 2.7557319223985893e-06); // 1/9!
  p = __builtin_fma(p, r, 2.48015873015873e-05);   // 1/8!
  p = __builtin_fma(p, r, 0.0001984126984126984);  // 1/7!
  p = __builtin_fma(p, r, 0.001388888888888889);   // 1/6!
  p = __builtin_fma(p, r, 0.008333333333333333);   // 1/5!
  p = __builtin_fma(p, r, 0.041666666666666664);   // 1/4!
  p = __builtin_fma(p, r, 0.16666666666666666);    // 1/3!
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  return __builtin_amdgcn_ldexp(p, (int)t);
}

// z + g of the version-3 draw (z = (l - M) / T, g the Gumbel noise of
// gumbel_from_key) in binary32 arithmetic, within 1e-4 of the binary64 value
// for |z| <= 40 and every uniform below 1: z to ~5e-6; -log u to ~1e-6
// relative (from 1 - u, exact in binary64, by a series when u is near 1,
// else from log of u); the outer log adds ~3e-6. 2.7e-6 is the largest
// error over 2e7 uniforms, the endpoints included. At the uniform's upper
// endpoint u = 1 both are +inf, so such an entry is never filtered out.
__device__ __forceinline__ float score_approx(float zf, uint64_t pk, uint32_t token) {
  const uint64_t h = mix64(pk ^ ((uint64_t)token * 0xd6e8feb86659fd93ull));
  const double u = ((double)(h >> 11) + 0.5) * (1.0 / 9007199254740992.0);  // the reference's uniform
  const float d = (float)(1.0 - u);  // exact for u >= 1/2
  float l1;
  if (d < 0.0625f) {
    l1 = d * (1.0f + d * (0.5f + d * (0.33333334f + d * (0.25f + d * 0.2f))));
  } else {
    l1 = -logf((float)u);
  }
  return zf - logf(l1);
}

// Version-2 uniform; output_head_sampler.rs:196-197 (no +0.5).
__device__ __forceinline__ double uniform_v2(uint64_t seed, uint64_t position) {
  return (double)(position_key(seed, position) >> 11) * (1.0 / 9007199254740992.0);
}

// Correctly rounded binary32 square root from an integer square root. The
// reference fixes the result (portable_math.rs:61-106: round to nearest,
// independent of a platform math library), not the method. A normalised
// radicand m in [2^46, 2^48) with an even exponent has r = floor(sqrt(m)) of
// 24 bits (or 2^24 after rounding up); m - r^2 > r decides round-to-nearest,
// since m = (r + 1/2)^2 is impossible for an integer m.
__host__ __device__ __forceinline__ float sqrt_rn_f32(float value) {
  uint32_t b;
  __builtin_memcpy(&b, &value, 4);
  if ((b & 0x7fffffffu) == 0u || b == 0x7f800000u) return value;  // +-0, +inf
  if ((b & 0x80000000u) || (b & 0x7f800000u) == 0x7f800000u) return __builtin_nanf("");
  uint64_t sig;
  int e;  // value = sig * 2^e
  if ((b >> 23) == 0u) {
    sig = b & 0x007fffffu;
    e = -149;
  } else {
    sig = (uint64_t)((b & 0x007fffffu) | 0x00800000u);
    e = (int)(b >> 23) - 150;
  }
  const int top = 63 - __builtin_clzll(sig);
  int shift = 46 - top;
  int ee = e - shift;
  if (ee & 1) {
    shift += 1;
    ee -= 1;
  }
  uint64_t m = sig << shift;
  // bit-by-bit integer square root
  uint64_t r = 0, bit = 1ull << 46;
  while (bit > m) bit >>= 2;
  uint64_t rem = m;
  while (bit) {
    if (rem >= r + bit) {
      rem -= r + bit;
      r = (r >> 1) + bit;
    } else {
      r >>= 1;
    }
    bit >>= 2;
  }
  if (rem > r) r += 1;
  int ex = ee / 2;
  if (r == (1ull << 24)) {
    r >>= 1;
    ex += 1;
  }
  const uint32_t out = ((uint32_t)(ex + 23 + 127) << 23) | ((uint32_t)r & 0x007fffffu);
  float f;
  __builtin_memcpy(&f, &out, 4);
  return f;
}

// 1 / sqrt_rn(value), the division separately rounded (portable_math.rs:108-111).
__device__ __forceinline__ float rsqrt_rn_f32(float value) { return __fdiv_rn(1.0f, sqrt_rn_f32(value)); }

}  // namespace yskn
