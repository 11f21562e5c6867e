// MXFP element arithmetic on gfx950's scaled MX conversion instructions
// (v_cvt_scalef32_pk_{fp4,fp8}_f32 and their decodes), equal to the exact
// software encoders of mgq_common.h:
//
//   - the encoders round half-even onto the E2M1 / E4M3 grids with the
//     reference's saturation (E2M1 saturates to +-6 in hardware; E4M3 is
//     clamped to +-448 first, as grid.py:118-121 does, because the hardware
//     turns overflow into NaN);
//   - the conversion to FP4/FP8 divides by the scale operand and the decode
//     multiplies by it; only the scale's exponent field is used, so 2^-127
//     (an fp32 subnormal) acts as the E8M0 value 2^-127;
//   - the reference encodes -0 and NaN as code 0 (its sign bit is set for
//     x < 0 only), E4M3 NaN as sign | 0x7f; the hardware differs there and
//     the encoders below patch those inputs.
//
// Checked on the GPU against mx4_encode / mx4_err / e4m3_code_clamped /
// e4m3_round for every fp32 input at a spread of scale exponents
// (tests/native/check_mx_hw.hip). The candidate errors differ from mx4_err
// only where n = w / scale is below 2^-126 in magnitude (sign of zero or the
// last subnormal bit), which no fp32 objective can see.
//
// div_exact: a / d correctly rounded with Markstein's correction from a
// precomputed y = RN(1/d): q = a y, r = fma(-q, d, a) (exact),
// q' = fma(r, y, q). q' equals the IEEE quotient for every pair of
// significands (a, d in [1, 2): all 2^46 pairs checked on the GPU), hence for
// every a, d whose intermediates stay normal: d in [2^-24, 2^24] (the caller
// passes y = 0 otherwise) and 2^-100 <= |a| < 2^101. Other inputs (zero
// included) take the IEEE division.
#pragma once

#include "mgq_common.h"

namespace mgq {

typedef short mx_s16x2_t __attribute__((ext_vector_type(2)));

// A register whose prior contents do not matter (the conversions below merge
// into it byte- or word-wise and only the written parts are read back).
__device__ inline uint32_t mx_undef_u32() {
  uint32_t u;
  asm volatile("" : "=v"(u));
  return u;
}

// Quantization errors in units of the scale, (q - n) with n = w / 2^e, for
// eight weights: the FP4 codes come straight from w with the scale folded
// into the conversion (four pairs into the four bytes of one register), and
// fma(w, -2^-e, q) is q - n rounded once (n is exact).
__device__ inline void mx4_cand_err8(const float (&w)[8], float scale, float inv_scale, float (&e)[8]) {
  uint32_t c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(mx_undef_u32(), w[0], w[1], scale, 0);
  c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(c, w[2], w[3], scale, 1);
  c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(c, w[4], w[5], scale, 2);
  c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(c, w[6], w[7], scale, 3);
  const auto q0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 0);
  const auto q1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 1);
  const auto q2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 2);
  const auto q3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 3);
  const float q[8] = {q0[0], q0[1], q1[0], q1[1], q2[0], q2[1], q3[0], q3[1]};
#pragma unroll
  for (int j = 0; j < 8; ++j) e[j] = fmaf(w[j], -inv_scale, q[j]);
}

// E4M3 counterpart for four weights; lim = min(448 * 2^e, FLT_MAX) clamps w
// so that w / 2^e is clamp(n, +-448) exactly (and inf stays finite for the
// conversion).
__device__ inline void mx8_cand_err4(const float (&w)[4], float scale, float inv_scale, float lim,
                                     float (&e)[4]) {
  float c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_fmed3f(w[j], -lim, lim);
  mx_s16x2_t p = __builtin_bit_cast(mx_s16x2_t, mx_undef_u32());
  p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, c[0], c[1], scale, false);
  p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(p, c[2], c[3], scale, true);
  const uint32_t u = __builtin_bit_cast(uint32_t, p);
  const auto q0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(u, 1.0f, false);
  const auto q1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(u, 1.0f, true);
  const float q[4] = {q0[0], q0[1], q1[0], q1[1]};
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = fmaf(w[j], -inv_scale, q[j]);
}

__device__ inline float mx8_clamp_limit(float scale) {
  return fminf(448.0f * scale, 3.40282347e38f);
}

// The encoders below take scale = 2^e, e in [-127, 127] (an E8M0 scale), and
// inv_scale = 2^-e. Their dq is the decode with the scale passed to the
// conversion, which equals value(code) * scale bit for bit for every code and
// every such scale (tests/test_gpu_mx_hw.py checks all of them).
//
// Exact MXFP4 code and dq = value(code) * scale of n = w * inv_scale
// (= mx4_encode for every fp32 w).
__device__ inline uint32_t mx4_encode_hw(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  uint32_t code = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, n, 0.0f, 1.0f, 0);
  code = (n == 0.0f || n != n) ? 0u : code;
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(code, scale, 0)[0];
  return code;
}

// mx4_encode_hw for every w whose n = w * inv_scale is not NaN, without the
// patch: n + 0 is n, except that -0 becomes +0 (the one non-NaN input whose
// hardware code, 8, differs from the reference's 0). A NaN n gives an
// unspecified code; the GPTQ recurrence's fast pass relies on that NaN
// reaching its last error, which sends the wave to the exact pass.
__device__ inline uint32_t mx4_encode_hw_nonan(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale + 0.0f;
  const uint32_t code = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, n, 0.0f, 1.0f, 0);
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(code, scale, 0)[0];
  return code;
}

// mx4_encode_hw_nonan written straight into byte k of `word` (one code per
// byte): the conversion stores the code and a zero code in that byte and
// keeps the other three, so no shift and merge is needed; dq is decoded from
// the same byte with the scale passed in. k must be a compile-time constant
// once the caller unrolls (the byte select is an immediate).
__device__ inline float mx4_encode_into(uint32_t& word, int k, float w, float inv_scale,
                                        float scale) {
  const float n = w * inv_scale + 0.0f;  // -0 -> +0, as mx4_encode_hw_nonan
  switch (k) {
    case 0:
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, n, 0.0f, 1.0f, 0);
      return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 0)[0];
    case 1:
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, n, 0.0f, 1.0f, 1);
      return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 1)[0];
    case 2:
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, n, 0.0f, 1.0f, 2);
      return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 2)[0];
    default:
      word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, n, 0.0f, 1.0f, 3);
      return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 3)[0];
  }
}

// Exact E4M3 code of clamp(n, +-448) and dq = value(code) * scale
// (= e4m3_code_clamped(clamp448(n)), e4m3_value(code) * scale).
__device__ inline uint32_t mx8_encode_hw(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  const float c = __builtin_amdgcn_fmed3f(n, -448.0f, 448.0f);
  const mx_s16x2_t p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(mx_s16x2_t{0, 0}, c, 0.0f, 1.0f, false);
  uint32_t code = __builtin_bit_cast(uint32_t, p);
  code = (n != n) ? (((f2u(n) >> 24) & 0x80u) | 0x7fu) : code;
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code, scale, false)[0];
  return code;
}

// mx8_encode_hw for every w whose n = w * inv_scale is not NaN (a NaN n
// gives an unspecified code, as in mx4_encode_hw_nonan).
__device__ inline uint32_t mx8_encode_hw_nonan(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  const float c = __builtin_amdgcn_fmed3f(n, -448.0f, 448.0f);
  const mx_s16x2_t p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(mx_s16x2_t{0, 0}, c, 0.0f, 1.0f, false);
  const uint32_t code = __builtin_bit_cast(uint32_t, p);
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code, scale, false)[0];
  return code;
}

__device__ inline float div_exact(float a, float d, float y) {
  const float q = a * y;
  const float r = fmaf(-q, d, a);
  float e = fmaf(r, y, q);
  const uint32_t ea = f2u(a) & 0x7f800000u;
  if (!(y != 0.0f) || (ea - (27u << 23)) > (200u << 23)) e = a / d;
  return e;
}

// y for div_exact: RN(1/d) where d is in [2^-24, 2^24], else 0.
__device__ inline float div_exact_recip(float d) {
  return (d >= 5.96046448e-8f && d <= 16777216.0f) ? 1.0f / d : 0.0f;
}

}  // namespace mgq
