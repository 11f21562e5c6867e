// GPU checks of the solver's hardware-instruction arithmetic (csrc/mx_hw.h)
// against the exact software forms (csrc/mgq_common.h, which
// tests/native/check_mx4_projection.hip pins against the threshold chain of
// grid.py:82-105) and against IEEE division.
//
// mgq_hwcheck_mx(e, counts): every fp32 weight w at scale exponent e;
// counts[k]:
//   0  mx4_encode_hw code != mx4_encode code
//   1  mx4_encode_hw dq   != mx4_encode dq           (bits; NaN == NaN)
//   2  mx8_encode_hw code != e4m3_code_clamped(clamp448(n))
//   3  mx8_encode_hw dq   != e4m3_value(code) * scale (bits; NaN == NaN)
//   4  mx4_cand_err8      != mx4_err                  (bits, NaN == NaN; both
//                                                      below 2^-126 when n is)
//   5  mx8_cand_err4      != e4m3_round(n) - n        (same rule)
//   6  MXFP4 error not exact in bf16 although w is a bf16 value and
//      2^-126 <= |n| < 512
//   7  MXFP8 error not exact in bf16 although w is a bf16 value and
//      2^-126 <= |n| < 16384
//   8  mx4_encode_into (the NaN-free encode written into one byte of a
//      word) != mx4_encode in code or dq bits, or a neighbouring byte
//      changed, for every w whose n is not NaN
//   9  mx8_encode_hw_nonan != mx8_encode_hw in code or dq bits, for every w
//      whose n is not NaN
//
// mgq_hwcheck_scaled_decode(counts): the scaled decodes with the scale
// folded in against the decode at scale 1 times the scale, bit for bit
// (NaN == NaN), for every byte value in every byte position and every
// E8M0 scale 2^e, e in [-127, 127]:
//   counts[0]: v_cvt_scalef32_pk_f32_fp4 (both values of the byte)
//   counts[1]: v_cvt_scalef32_pk_f32_fp8 (both halves)
//
// mgq_hwcheck_div(stride_log, counts): div_exact(a, d, div_exact_recip(d))
// against a / d, bit for bit:
//   counts[0]: a, d over all significands in [1, 2), d every 2^stride_log-th
//              (stride_log = 0: all 2^46 pairs);
//   counts[1]: 2^12 pseudo-random significand pairs at every exponent pair
//              ea in [-130, 127], ed in [-30, 30] (both guards' edges and
//              the fallback side), signs mixed, plus a = 0.
#include <hip/hip_runtime.h>

#include "mx_hw.h"

using namespace mgq;

namespace {

constexpr int kKinds = 10;

__device__ inline bool same_bits(float a, float b) { return f2u(a) == f2u(b) || (a != a && b != b); }
__device__ inline bool tiny(float x) { return !(fabsf(x) >= 1.17549435e-38f) && x == x; }
__device__ inline bool bf16_exact(float x) { return (f2u(x) & 0xffffu) == 0u; }

__global__ void check_kernel(int e, unsigned long long* counts) {
  unsigned loc[kKinds] = {};
  const float inv = exp2_int(-e), scale = exp2_int(e);
  const float lim = mx8_clamp_limit(scale);
  // 2^22 threads x 128 iterations x 8 consecutive weights = 2^32 inputs
  for (int it = 0; it < 128; ++it) {
    const unsigned long long t = static_cast<unsigned long long>(it) * (1ull << 22) +
                                 static_cast<unsigned long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint32_t u0 = static_cast<uint32_t>(8ull * t);
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = u2f(u0 + j);
    float e4[8], e8[8];
    mx4_cand_err8(w, scale, inv, e4);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x[4] = {w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]};
      float t8[4];
      mx8_cand_err4(x, scale, inv, lim, t8);
#pragma unroll
      for (int j = 0; j < 4; ++j) e8[4 * h + j] = t8[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
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
      if (n == n) {
        // byte j % 4 of a word whose other bytes hold a marker
        const int k = j & 3;
        uint32_t word = 0xa5a5a5a5u;
        const float dq_in = mx4_encode_into(word, k, w[j], inv, scale);
        const uint32_t byte = (word >> (8 * k)) & 0xffu;
        const uint32_t rest = word | (0xffu << (8 * k));
        loc[8] += (byte != c_ref) || !same_bits(dq_in, dq_ref) ||
                  rest != (0xa5a5a5a5u | (0xffu << (8 * k)));
        float dq8_nn, dq8;
        const uint32_t k_nn = mx8_encode_hw_nonan(w[j], inv, scale, &dq8_nn);
        const uint32_t k_ex = mx8_encode_hw(w[j], inv, scale, &dq8);
        loc[9] += (k_nn != k_ex) || !same_bits(dq8_nn, dq8);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kKinds; ++k)
    if (loc[k]) atomicAdd(&counts[k], static_cast<unsigned long long>(loc[k]));
}

// one d significand per thread, every a significand
__global__ void div_pairs_kernel(uint32_t d0, uint32_t stride, unsigned long long* counts) {
  const uint32_t id = d0 + (blockIdx.x * blockDim.x + threadIdx.x) * stride;
  if (id >= (1u << 23)) return;
  const float d = u2f(0x3f800000u | id);
  const float y = div_exact_recip(d);
  unsigned n = 0;
  for (uint32_t ia = 0; ia < (1u << 23); ++ia) {
    const float a = u2f(0x3f800000u | ia);
    n += f2u(div_exact(a, d, y)) != f2u(a / d);
  }
  if (n) atomicAdd(&counts[0], static_cast<unsigned long long>(n));
}

__device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// blockIdx.x = exponent pair, 256 threads x 16 samples each
__global__ void div_ranges_kernel(unsigned long long* counts) {
  const int ea = static_cast<int>(blockIdx.x % 258) - 130;
  const int ed = static_cast<int>(blockIdx.x / 258) - 30;
  unsigned n = 0;
  for (int s = 0; s < 16; ++s) {
    const uint32_t h = mix32(blockIdx.x * 4096u + threadIdx.x * 16u + s);
    const uint32_t h2 = mix32(h ^ 0x9e3779b9u);
    float a = u2f(0x3f800000u | (h & 0x7fffffu)) * exp2_int(ea < -127 ? -127 : ea);
    if (ea < -127) a = a * exp2_int(ea + 127);  // subnormal (or zero) a
    if (s == 0 && threadIdx.x == 0) a = 0.0f;
    if (h & 0x80000000u) a = -a;
    const float d = u2f(0x3f800000u | (h2 & 0x7fffffu)) * exp2_int(ed);
    n += f2u(div_exact(a, d, div_exact_recip(d))) != f2u(a / d);
  }
  if (n) atomicAdd(&counts[1], static_cast<unsigned long long>(n));
}

}  // namespace

// Block e + 127, thread = byte value b, replicated into all four bytes.
__global__ void scaled_decode_kernel(unsigned long long* counts) {
  const int e = static_cast<int>(blockIdx.x) - 127;
  const float scale = exp2_int(e);
  const uint32_t word = threadIdx.x * 0x01010101u;
  unsigned long long bad4 = 0, bad8 = 0;
#define MGQ_CHECK4(k)                                                           \
  {                                                                             \
    const auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, k);   \
    const auto b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, 1.0f, k);    \
    bad4 += !same_bits(a[0], b[0] * scale) + !same_bits(a[1], b[1] * scale);   \
  }
  MGQ_CHECK4(0) MGQ_CHECK4(1) MGQ_CHECK4(2) MGQ_CHECK4(3)
#undef MGQ_CHECK4
#define MGQ_CHECK8(h)                                                           \
  {                                                                             \
    const auto a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, scale, h);   \
    const auto b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, 1.0f, h);    \
    bad8 += !same_bits(a[0], b[0] * scale) + !same_bits(a[1], b[1] * scale);   \
  }
  MGQ_CHECK8(false) MGQ_CHECK8(true)
#undef MGQ_CHECK8
  if (bad4) atomicAdd(&counts[0], bad4);
  if (bad8) atomicAdd(&counts[1], bad8);
}

// Runs the MX check for scale exponent e in [-127, 127]; counts: host array of 10.
extern "C" int mgq_hwcheck_mx(int e, unsigned long long* counts) {
  if (e < -127 || e > 127) return -1;
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, kKinds * sizeof(unsigned long long)) != hipSuccess) return -2;
  hipMemset(d, 0, kKinds * sizeof(unsigned long long));
  check_kernel<<<(1u << 22) / 256, 256>>>(e, d);
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpy(counts, d, kKinds * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(d);
  return err == hipSuccess ? 0 : -3;
}

// Runs the scaled-decode check; counts: host array of 2.
extern "C" int mgq_hwcheck_scaled_decode(unsigned long long* counts) {
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, 2 * sizeof(unsigned long long)) != hipSuccess) return -2;
  hipMemset(d, 0, 2 * sizeof(unsigned long long));
  scaled_decode_kernel<<<255, 256>>>(d);
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpy(counts, d, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(d);
  return err == hipSuccess ? 0 : -3;
}

// Runs the division check; counts: host array of 2.
extern "C" int mgq_hwcheck_div(int stride_log, unsigned long long* counts) {
  if (stride_log < 0 || stride_log > 23) return -1;
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, 2 * sizeof(unsigned long long)) != hipSuccess) return -2;
  hipMemset(d, 0, 2 * sizeof(unsigned long long));
  const uint32_t stride = 1u << stride_log;
  const uint32_t n_d = (1u << 23) >> stride_log;  // d significands checked
  const uint32_t per = 1u << 18;                  // per launch
  hipError_t err = hipSuccess;
  for (uint32_t k = 0; k < n_d && err == hipSuccess; k += per) {
    const uint32_t cnt = n_d - k < per ? n_d - k : per;
    div_pairs_kernel<<<(cnt + 255) / 256, 256>>>(k * stride, stride, d);
    err = hipDeviceSynchronize();
  }
  if (err == hipSuccess) {
    div_ranges_kernel<<<258 * 61, 256>>>(d);
    err = hipDeviceSynchronize();
  }
  if (err == hipSuccess) err = hipMemcpy(counts, d, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  hipFree(d);
  return err == hipSuccess ? 0 : -3;
}
