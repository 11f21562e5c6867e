// Exhaustive GPU check of the solver's hardware MX conversion forms
// (csrc/mx_hw.h) against the exact software encoders (csrc/mgq_common.h,
// which tests/native/check_mx4_projection.hip pins against the threshold
// chain of grid.py:82-105), for every fp32 weight w at one scale exponent e.
//
// counts[k] after mgq_hwcheck_mx(e, counts):
//   0  mx4_encode_hw code != mx4_encode code
//   1  mx4_encode_hw dq   != mx4_encode dq           (bits; NaN == NaN)
//   2  mx8_encode_hw code != e4m3_code_clamped(clamp448(n))
//   3  mx8_encode_hw dq   != e4m3_value(code) * scale (bits; NaN == NaN)
//   4  mx4_cand_err2      != mx4_err                  (bits, NaN == NaN; both
//                                                      below 2^-126 when n is)
//   5  mx8_cand_err2      != e4m3_round(n) - n        (same rule)
//   6  MXFP4 error not exact in bf16 although w is a bf16 value and
//      2^-126 <= |n| < 512
//   7  MXFP8 error not exact in bf16 although w is a bf16 value and
//      2^-126 <= |n| < 16384
#include <hip/hip_runtime.h>

#include "mx_hw.h"

using namespace mgq;

namespace {

constexpr int kKinds = 8;

__device__ inline bool same_bits(float a, float b) { return f2u(a) == f2u(b) || (a != a && b != b); }
__device__ inline bool tiny(float x) { return !(fabsf(x) >= 1.17549435e-38f) && x == x; }
__device__ inline bool bf16_exact(float x) { return (f2u(x) & 0xffffu) == 0u; }

__global__ void check_kernel(int e, unsigned long long* counts) {
  unsigned loc[kKinds] = {};
  const float inv = exp2_int(-e), scale = exp2_int(e);
  const float lim = mx8_clamp_limit(scale);
  // 2^24 threads x 128 iterations x 2 weights = 2^32 inputs
  for (int it = 0; it < 128; ++it) {
    const unsigned long long t = static_cast<unsigned long long>(it) * (1ull << 24) +
                                 static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t u0 = static_cast<uint32_t>(2ull * t);
    const float w[2] = {u2f(u0), u2f(u0 + 1u)};
    float e4[2], e8[2];
    mx4_cand_err2(w[0], w[1], scale, inv, e4[0], e4[1]);
    mx8_cand_err2(w[0], w[1], scale, inv, lim, e8[0], e8[1]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float n = w[j] * inv;
      float dq_hw, dq_ref;
      const uint32_t c_hw = mx4_encode_hw(w[j], inv, scale, &dq_hw);
      const uint32_t c_ref = mx4_encode(w[j], inv, scale, &dq_ref);
      loc[0] += c_hw != c_ref;
      loc[1] += !same_bits(dq_hw, dq_ref);
      const uint32_t k_hw = mx8_encode_hw(w[j], inv, scale, &dq_hw);
      const uint32_t k_ref = e4m3_code_clamped(clamp448(n));
      loc[2] += k_hw != k_ref;
      loc[3] += !same_bits(dq_hw, e4m3_value(k_ref) * scale);
      const float r4 = mx4_err(w[j], inv);
      const float r8 = e4m3_round(n) - n;
      const bool small = tiny(n);
      loc[4] += !(same_bits(e4[j], r4) || (small && tiny(e4[j]) && tiny(r4)));
      loc[5] += !(same_bits(e8[j], r8) || (small && tiny(e8[j]) && tiny(r8)));
      const float an = fabsf(n);
      const bool w_bf16 = bf16_exact(w[j]);
      loc[6] += (w_bf16 && !small && an < 512.0f && !bf16_exact(e4[j]));
      loc[7] += (w_bf16 && !small && an < 16384.0f && !bf16_exact(e8[j]));
    }
  }
#pragma unroll
  for (int k = 0; k < kKinds; ++k)
    if (loc[k]) atomicAdd(&counts[k], static_cast<unsigned long long>(loc[k]));
}

}  // namespace

// Runs the check for scale exponent e in [-127, 127]; counts: host array of 8.
extern "C" int mgq_hwcheck_mx(int e, unsigned long long* counts) {
  if (e < -127 || e > 127) return -1;
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, kKinds * sizeof(unsigned long long)) != hipSuccess) return -2;
  hipMemset(d, 0, kKinds * sizeof(unsigned long long));
  check_kernel<<<(1u << 24) / 256, 256>>>(e, d);
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpy(counts, d, kKinds * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(d);
  return err == hipSuccess ? 0 : -3;
}
