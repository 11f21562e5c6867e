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
#pragma once

#include "mgq_common.h"

namespace mgq {

typedef short mx_s16x2_t __attribute__((ext_vector_type(2)));

// Quantization errors in units of the scale, (q - n) with n = w / 2^e, for two
// weights: the FP4 code comes straight from w with the scale folded into the
// conversion, and fma(w, -2^-e, q) is q - n rounded once (n is exact).
__device__ inline void mx4_cand_err2(float w0, float w1, float scale, float inv_scale, float& e0,
                                     float& e1) {
  const uint32_t c = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, w0, w1, scale, 0);
  const auto q = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(c, 1.0f, 0);
  e0 = fmaf(w0, -inv_scale, q[0]);
  e1 = fmaf(w1, -inv_scale, q[1]);
}

// E4M3 counterpart; lim = min(448 * 2^e, FLT_MAX) clamps w so that w / 2^e
// is clamp(n, +-448) exactly (and inf stays finite for the conversion).
__device__ inline void mx8_cand_err2(float w0, float w1, float scale, float inv_scale, float lim,
                                     float& e0, float& e1) {
  const float c0 = __builtin_amdgcn_fmed3f(w0, -lim, lim);
  const float c1 = __builtin_amdgcn_fmed3f(w1, -lim, lim);
  const mx_s16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(mx_s16x2_t{0, 0}, c0, c1, scale, false);
  const auto q = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(__builtin_bit_cast(uint32_t, c), 1.0f, false);
  e0 = fmaf(w0, -inv_scale, q[0]);
  e1 = fmaf(w1, -inv_scale, q[1]);
}

__device__ inline float mx8_clamp_limit(float scale) {
  return fminf(448.0f * scale, 3.40282347e38f);
}

// Exact MXFP4 code and dq = value(code) * scale of n = w * inv_scale
// (= mx4_encode for every fp32 w).
__device__ inline uint32_t mx4_encode_hw(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  uint32_t code = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(0u, n, 0.0f, 1.0f, 0);
  code = (n == 0.0f || n != n) ? 0u : code;
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(code, 1.0f, 0)[0] * scale;
  return code;
}

// Exact E4M3 code of clamp(n, +-448) and dq = value(code) * scale
// (= e4m3_code_clamped(clamp448(n)), e4m3_value(code) * scale).
__device__ inline uint32_t mx8_encode_hw(float w, float inv_scale, float scale, float* dq) {
  const float n = w * inv_scale;
  const float c = __builtin_amdgcn_fmed3f(n, -448.0f, 448.0f);
  const mx_s16x2_t p = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(mx_s16x2_t{0, 0}, c, 0.0f, 1.0f, false);
  uint32_t code = __builtin_bit_cast(uint32_t, p);
  code = (n != n) ? (((f2u(n) >> 24) & 0x80u) | 0x7fu) : code;
  *dq = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(code, 1.0f, false)[0] * scale;
  return code;
}

}  // namespace mgq
