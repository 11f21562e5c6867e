// Shared device helpers for the MI355X (gfx950) GPTQ calibration solver.
//
// Every encoder here reproduces, bit for bit, the fp32 arithmetic of the
// reference quantization grids (mlx_gptq/grid.py). The library is compiled
// with -ffp-contract=off so `a * b + c` stays two IEEE roundings exactly as
// torch evaluates `q * s + b`, and fp32 division is IEEE (hipcc default).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e8m0_thresholds.h"

namespace mgq {

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };
enum Mode : int { kAffine = 0, kMxfp4 = 1, kMxfp8 = 2 };

constexpr int kMxGroup = 32;  // MX_GROUP_SIZE (grid.py:21)

// Bit casts usable on host and device (HIP's __float_as_uint is device-only).
__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------------------
// 16-bit float conversions (round to nearest even).
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return u2f(static_cast<uint32_t>(h) << 16);
}

__host__ __device__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ inline float round_to_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

__device__ inline float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ inline uint16_t f32_to_f16_rne(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));  // IEEE RNE
}
__device__ inline float round_to_f16(float f) { return f16_to_f32(f32_to_f16_rne(f)); }

// Round a float32 value to the storage dtype and back (torch `.to(dt).float()`).
__device__ inline float round_to_storage(float f, int storage) {
  if (storage == kBF16) return round_to_bf16(f);
  if (storage == kF16) return round_to_f16(f);
  return f;
}

__device__ inline void store_storage(void* base, int64_t i, float v, int storage) {
  if (storage == kBF16) {
    static_cast<uint16_t*>(base)[i] = f32_to_bf16_rne(v);
  } else if (storage == kF16) {
    static_cast<uint16_t*>(base)[i] = f32_to_f16_rne(v);
  } else {
    static_cast<float*>(base)[i] = v;
  }
}

__device__ inline float load_storage(const void* base, int64_t i, int storage) {
  if (storage == kBF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  if (storage == kF16) return f16_to_f32(static_cast<const uint16_t*>(base)[i]);
  return static_cast<const float*>(base)[i];
}

__device__ inline float load_any(const void* base, int64_t i, int dtype) {
  return load_storage(base, i, dtype);
}

// 1/d for d > 0: v_rcp_f64 refined by two Newton-Raphson steps
// y <- y + y (1 - d y), each of which squares the relative error.
__device__ inline double recip_f64(double d) {
  double y = __builtin_amdgcn_rcp(d);
  double e = fma(-d, y, 1.0);
  y = fma(y, e, y);
  e = fma(-d, y, 1.0);
  return fma(y, e, y);
}

// ---------------------------------------------------------------------------
// E8M0 shared scale (grid.py:61-79).
// exponent = clamp(round_half_even(fp32(log2(max_abs / fmax))), -127, 127),
// 0 when max_abs == 0; inf/NaN land on -127 (the int cast of inf/NaN is
// INT_MIN before the clamp). Evaluated with the exact per-binade threshold
// table instead of a device log2.
// ---------------------------------------------------------------------------
__device__ inline int e8m0_exponent(float max_abs, float fmax) {
  if (max_abs == 0.0f) return 0;
  const float y = max_abs / fmax;
  const uint32_t u = __float_as_uint(y);
  if (!(u < 0x7f800000u)) return -127;  // inf or NaN (y is non-negative)
  if (u < 0x00800000u) return u >= kE8m0Threshold[0] ? -126 : -127;
  const int e = static_cast<int>(u >> 23) - 127;  // floor(log2 y), in [-126, 127]
  int r = e + (u >= kE8m0Threshold[e + 1 + 126] ? 1 : 0);
  return r > 127 ? 127 : r;
}

// 2^k for k in [-127, 127] (exact; 2^-127 is subnormal), like torch.pow(2, k):
// one v_ldexp_f32 (fp32 denormals are kept in this build's float mode).
__device__ inline float exp2_int(int k) { return __builtin_amdgcn_ldexpf(1.0f, k); }

// ---------------------------------------------------------------------------
// E2M1 (grid.py:82-105): saturating round-half-even onto
// {0, .5, 1, 1.5, 2, 3, 4, 6}; sign bit only for x < 0 (so -0 and NaN -> 0).
// ---------------------------------------------------------------------------
__host__ __device__ inline uint32_t e2m1_code(float x) {
  const float ax = fabsf(x);
  uint32_t m = (ax > 5.0f)    ? 7u
               : (ax >= 3.5f) ? 6u
               : (ax > 2.5f)  ? 5u
               : (ax >= 1.75f) ? 4u
               : (ax > 1.25f) ? 3u
               : (ax >= 0.75f) ? 2u
               : (ax > 0.25f) ? 1u
                              : 0u;
  return m | (x < 0.0f ? 8u : 0u);
}

// _E2M1_VALUES[code] (grid.py:23-40).
__host__ __device__ inline float e2m1_value(uint32_t code) {
  const uint32_t m = code & 7u;
  // magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6 as fp32 bit patterns
  constexpr uint32_t kMag[8] = {0x00000000u, 0x3f000000u, 0x3f800000u, 0x3fc00000u,
                                0x40000000u, 0x40400000u, 0x40800000u, 0x40c00000u};
  uint32_t b = kMag[0];
#pragma unroll
  for (uint32_t i = 1; i < 8; ++i) b = (m == i) ? kMag[i] : b;
  return u2f(b | ((code & 8u) << 28));
}

// ---------------------------------------------------------------------------
// E4M3 (torch float8_e4m3fn cast after clamp to +-448, grid.py:118-121).
// Round-half-even onto the e4m3fn grid with subnormals (step 2^-9); NaN keeps
// its sign bit (0x7f / 0xff); -0 -> 0x80.
// ---------------------------------------------------------------------------
__device__ inline uint32_t e4m3_code_clamped(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t ua = u & 0x7fffffffu;
  if (ua > 0x7f800000u) return sign | 0x7fu;
  float a = __uint_as_float(ua);
  a = fminf(a, 448.0f);
  uint32_t mag;
  if (a < 0.015625f) {  // below 2^-6: subnormal grid, a * 2^9 is exact
    mag = static_cast<uint32_t>(rintf(a * 512.0f));
  } else {
    const uint32_t b = __float_as_uint(a);
    const uint32_t r = (b + 0x7ffffu + ((b >> 20) & 1u)) >> 20;
    mag = r - ((127u - 7u) << 3);
  }
  return sign | mag;
}

__device__ inline float e4m3_value(uint32_t code) {
  const uint32_t sign = (code & 0x80u) << 24;
  const uint32_t e = (code >> 3) & 0xfu;
  const uint32_t m = code & 7u;
  if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7fc00000u);
  float v;
  if (e == 0u) {
    v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9, exact
  } else {
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(v) | sign);
}

// clamp(x, -448, 448) keeps NaN (torch.clamp semantics).
__device__ inline float clamp448(float x) {
  if (x != x) return x;
  return fminf(fmaxf(x, -448.0f), 448.0f);
}

// One MXFP element: normalized = w / scale, code, dq = value(code) * scale
// (grid.py:108-124), each an IEEE fp32 operation as in torch.
__device__ inline uint32_t mx_quant(float w, float scale, int mode, float* dq) {
  const float n = w / scale;
  uint32_t code;
  float v;
  if (mode == kMxfp4) {
    code = e2m1_code(n);
    v = e2m1_value(code);
  } else {
    code = e4m3_code_clamped(clamp448(n));
    v = e4m3_value(code);
  }
  *dq = v * scale;
  return code;
}

// ---------------------------------------------------------------------------
// Solver fast path: the same values as mx_quant, computed arithmetically.
// Because every MXFP scale is a power of two, w / scale == w * (1/scale)
// exactly (both are the correctly rounded w * 2^-e, and 2^-e is
// representable for e in [-127, 127]). These produce exactly mx_quant's dq
// (same grid value, same sign rule, same product with the scale) without
// materialising the code; the solver uses them to score scale candidates.
// ---------------------------------------------------------------------------

// Quantization error of MXFP4 in units of the scale: (dq - w) / scale with
// dq = value(code(n)) * scale, n = w * inv_scale, for scoring scale
// candidates. n is rounded half-even to the E2M1 step of its binade (1/2
// below 2, 1 on [2,4), 2 from 4) by adding and subtracting
// 1.5 * 2^(22+k), k = clamp(binade, 0, 2), whose ulp is that step (symmetric
// in the sign of n), then clamped to +-6. q - n is exact when q is the
// rounding of n (it is n's discarded low bits) and is the reference's single
// fp32 rounding when q saturates, so (q - n) * scale is the reference's
// dq - w whenever that product stays normal. Equal to
// e2m1_value(e2m1_code(n)) - n for every fp32 n (checked for all 2^32
// inputs; NaN in, NaN out).
__host__ __device__ inline float mx4_err(float w, float inv_scale) {
  const float n = w * inv_scale;
  uint32_t eb = (f2u(n) >> 23) & 0xffu;
  eb = eb < 127u ? 127u : (eb > 129u ? 129u : eb);
  const float magic = u2f((eb << 23) + ((22u << 23) | 0x400000u));
  float q = (n + magic) - magic;
  q = fminf(fmaxf(q, -6.0f), 6.0f);
  return q - n;
}

// Exact MXFP4 encoding of n = w * inv_scale without a compare chain: the
// magnitude comes from the same half-even rounding as mx4_err, and the code
// from its bit pattern (f2u(m) >> 22 is 0 for 0, 252 for 0.5 and 254..259 for
// 1, 1.5, 2, 3, 4, 6). Code and dq equal e2m1_code(n) and
// e2m1_value(code) * scale for every fp32 n, NaN and -0 included (checked
// for all 2^32 inputs).
__host__ __device__ inline uint32_t mx4_encode(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  const uint32_t ua = f2u(n) & 0x7fffffffu;
  uint32_t eb = ua >> 23;
  eb = eb < 127u ? 127u : (eb > 129u ? 129u : eb);
  const float magic = u2f((eb << 23) + ((22u << 23) | 0x400000u));
  float m = fminf((u2f(ua) + magic) - magic, 6.0f);
  m = (n == n) ? m : 0.0f;
  const uint32_t t = f2u(m) >> 22;
  const uint32_t mag = t >= 254u ? t - 252u : (t != 0u ? 1u : 0u);
  const bool neg = n < 0.0f;
  *dq = (neg ? -m : m) * scale;
  return mag | (neg ? 8u : 0u);
}

// E4M3 value of clamp(n, +-448) rounded half-even onto the e4m3fn grid,
// sign preserved, NaN stays NaN.
__device__ inline float e4m3_round(float n) {
  const uint32_t u = __float_as_uint(n);
  const uint32_t sign = u & 0x80000000u;
  uint32_t ua = u & 0x7fffffffu;
  if (ua > 0x7f800000u) return __uint_as_float(sign | 0x7fc00000u);
  if (ua > 0x43e00000u) ua = 0x43e00000u;  // 448
  float m;
  if (ua < 0x3c800000u) {  // below 2^-6: subnormal step 2^-9
    m = rintf(__uint_as_float(ua) * 512.0f) * 0.001953125f;
  } else {
    m = __uint_as_float((ua + 0x7ffffu + ((ua >> 20) & 1u)) & 0xfff00000u);
  }
  return __uint_as_float(__float_as_uint(m) | sign);
}

__device__ inline float mx8_dq(float w, float inv_scale, float scale) {
  return e4m3_round(w * inv_scale) * scale;
}

// ---------------------------------------------------------------------------
// Small helpers.
// ---------------------------------------------------------------------------
__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace mgq
