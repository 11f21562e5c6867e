// Quantization grids: E8M0 scale choice, E2M1 / E4M3 encoders, MXFP RTN and
// dequant, affine MSE clip search with storage-rounded params, affine RTN.
// Element-parallel, HBM-bound kernels; the hot solver kernels reuse the same
// device encoders from mgq_common.h.
#include <string.h>

#include "mgq_capi.h"
#include "mgq_common.h"
#include "mx_hw.h"

namespace mgq {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxShrinks = 128;

struct Shrinks {
  int n;
  float p_over_maxq[kMaxShrinks];  // float32(p / maxq)
  float p[kMaxShrinks];            // float32(p)
};

// grid.py:185-192: maxq = float(2**bits - 1); p_i = 1.0 - max_shrink*i/grid_steps
// evaluated in double exactly as Python does, then cast to fp32 the way torch
// casts a Python scalar operand.
int make_shrinks(int bits, int method, int grid_steps, double max_shrink, Shrinks* out) {
  const double maxq = static_cast<double>((1 << bits) - 1);
  if (method == MGQ_CLIP_MINMAX) {
    out->n = 1;
    out->p_over_maxq[0] = static_cast<float>(1.0 / maxq);
    out->p[0] = 1.0f;
    return MGQ_OK;
  }
  MGQ_REQUIRE(grid_steps >= 1 && grid_steps < kMaxShrinks, MGQ_ERR_VALUE,
              "grid_steps must be in [1, %d), got %d", kMaxShrinks, grid_steps);
  out->n = grid_steps + 1;
  for (int i = 0; i <= grid_steps; ++i) {
    const double p = 1.0 - max_shrink * static_cast<double>(i) / static_cast<double>(grid_steps);
    out->p_over_maxq[i] = static_cast<float>(p / maxq);
    out->p[i] = static_cast<float>(p);
  }
  return MGQ_OK;
}

// NaN-propagating max / min (torch amax / amin semantics).
__device__ inline float nan_max(float m, float a) { return (a > m || a != a) ? a : m; }
__device__ inline float nan_min(float m, float a) { return (a < m || a != a) ? a : m; }

__device__ inline float affine_q(float w, float b, float s_safe, float maxq) {
  float q = rintf((w - b) / s_safe);
  if (q != q) return q;
  return fminf(fmaxf(q, 0.0f), maxq);
}

// ---------------------------------------------------------------------------
__global__ void choose_mxfp_scale_kernel(const float* __restrict__ w, int64_t n_groups,
                                         int64_t len, float fmax, uint8_t* __restrict__ bytes,
                                         float* __restrict__ scales) {
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < n_groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    const float* p = w + g * len;
    float m = fabsf(p[0]);
    for (int64_t i = 1; i < len; ++i) m = nan_max(m, fabsf(p[i]));
    const int e = e8m0_exponent(m, fmax);
    bytes[g] = static_cast<uint8_t>(e + 127);
    scales[g] = exp2_int(e);
  }
}

__global__ void quantize_mxfp_kernel(const float* __restrict__ w, const float* __restrict__ scales,
                                     int64_t n, int64_t len, int mode, uint8_t* __restrict__ q,
                                     float* __restrict__ dq) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float d;
    q[i] = static_cast<uint8_t>(mx_quant(w[i], scales[i / len], mode, &d));
    dq[i] = d;
  }
}

__device__ inline float scale_from_byte(uint32_t b) {
  // torch.pow(2, byte - 127) in fp32: 2^128 overflows to inf.
  const int e = static_cast<int>(b) - 127;
  return e > 127 ? __uint_as_float(0x7f800000u) : exp2_int(e);
}

__global__ void dequantize_mxfp_kernel(const uint8_t* __restrict__ q,
                                       const uint8_t* __restrict__ bytes, int64_t n, int mode,
                                       float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float s = scale_from_byte(bytes[i / kMxGroup]);
    const uint32_t c = q[i];
    const float v = (mode == kMxfp4) ? e2m1_value(c & 15u) : e4m3_value(c);
    out[i] = v * s;
  }
}

// One thread per 32-value group: scale choice + projection (grid.py:142-151).
__global__ void rtn_mxfp_kernel(const void* __restrict__ W, int dtype, int64_t n_groups,
                                int mode, uint8_t* __restrict__ q, uint8_t* __restrict__ bytes,
                                float* __restrict__ dq) {
  const float fmax = (mode == kMxfp4) ? 6.0f : 448.0f;
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < n_groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    float v[kMxGroup];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kMxGroup; ++i) {
      v[i] = load_any(W, g * kMxGroup + i, dtype);
      m = (i == 0) ? fabsf(v[i]) : nan_max(m, fabsf(v[i]));
    }
    const int e = e8m0_exponent(m, fmax);
    const float s = exp2_int(e);
    bytes[g] = static_cast<uint8_t>(e + 127);
#pragma unroll
    for (int i = 0; i < kMxGroup; ++i) {
      float d;
      q[g * kMxGroup + i] = static_cast<uint8_t>(mx_quant(v[i], s, mode, &d));
      dq[g * kMxGroup + i] = d;
    }
  }
}

// The same for 16-byte aligned W, q and dq: one thread per group with
// 16-byte loads and stores, and the hardware MX encoders (mx_hw.h, equal to
// mx_quant for every input: w / s == w * (1/s) for power-of-two s).
template <typename TIn, bool IS_F16>
__global__ void rtn_mxfp_vec_kernel(const TIn* __restrict__ W, int64_t n_groups, int mode,
                                    uint8_t* __restrict__ q, uint8_t* __restrict__ bytes,
                                    float* __restrict__ dq) {
  const float fmax = (mode == kMxfp4) ? 6.0f : 448.0f;
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < n_groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    float v[kMxGroup];
    if constexpr (sizeof(TIn) == 4) {
      const float4* p = reinterpret_cast<const float4*>(W + g * kMxGroup);
#pragma unroll
      for (int i = 0; i < kMxGroup / 4; ++i) {
        const float4 x = p[i];
        v[4 * i] = x.x, v[4 * i + 1] = x.y, v[4 * i + 2] = x.z, v[4 * i + 3] = x.w;
      }
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(W + g * kMxGroup);
#pragma unroll
      for (int i = 0; i < kMxGroup / 8; ++i) {
        const uint4 x = p[i];
        const uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint16_t lo = static_cast<uint16_t>(d[k] & 0xffffu), hi = static_cast<uint16_t>(d[k] >> 16);
          v[8 * i + 2 * k] = IS_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
          v[8 * i + 2 * k + 1] = IS_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
        }
      }
    }
    float m = fabsf(v[0]);
#pragma unroll
    for (int i = 1; i < kMxGroup; ++i) m = nan_max(m, fabsf(v[i]));
    const int e = e8m0_exponent(m, fmax);
    const float s = exp2_int(e), inv = exp2_int(-e);
    bytes[g] = static_cast<uint8_t>(e + 127);
    uint32_t codes[kMxGroup / 4];
    float d[kMxGroup];
#pragma unroll
    for (int i = 0; i < kMxGroup / 4; ++i) codes[i] = 0u;
#pragma unroll
    for (int i = 0; i < kMxGroup; ++i) {
      const uint32_t c = (mode == kMxfp4) ? mx4_encode_hw(v[i], inv, s, &d[i])
                                          : mx8_encode_hw(v[i], inv, s, &d[i]);
      codes[i / 4] |= c << (8 * (i % 4));
    }
    uint4* qp = reinterpret_cast<uint4*>(q + g * kMxGroup);
    qp[0] = make_uint4(codes[0], codes[1], codes[2], codes[3]);
    qp[1] = make_uint4(codes[4], codes[5], codes[6], codes[7]);
    float4* op = reinterpret_cast<float4*>(dq + g * kMxGroup);
#pragma unroll
    for (int i = 0; i < kMxGroup / 4; ++i) op[i] = make_float4(d[4 * i], d[4 * i + 1], d[4 * i + 2], d[4 * i + 3]);
  }
}

__global__ void dequantize_affine_kernel(const uint8_t* __restrict__ q, const void* scales,
                                         const void* biases, int storage, int64_t n, int64_t len,
                                         float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = i / len;
    out[i] = static_cast<float>(q[i]) * load_storage(scales, g, storage) +
             load_storage(biases, g, storage);
  }
}

// grid.py:167-212 for one group. Returns the chosen (s, b) in fp32 (already
// rounded to the storage dtype).
__device__ inline void choose_qparams_group(const float* __restrict__ p, int64_t len, float maxq,
                                            int storage, const Shrinks& sh, float* s_out,
                                            float* b_out) {
  float wmin = p[0], wmax = p[0];
  for (int64_t i = 1; i < len; ++i) {
    wmin = nan_min(wmin, p[i]);
    wmax = nan_max(wmax, p[i]);
  }
  const float range = wmax - wmin;
  float best_err = 0.0f, best_s = 0.0f, best_b = 0.0f;
  for (int c = 0; c < sh.n; ++c) {
    const float s = round_to_storage(range * sh.p_over_maxq[c], storage);
    const float b = round_to_storage(wmin * sh.p[c], storage);
    const float s_safe = (fabsf(s) < 1e-12f) ? 1.0f : s;
    float err = 0.0f;
    for (int64_t i = 0; i < len; ++i) {
      const float q = affine_q(p[i], b, s_safe, maxq);
      const float d = q * s + b - p[i];
      err += d * d;
    }
    if (c == 0 || err < best_err) {
      best_err = err;
      best_s = s;
      best_b = b;
    }
  }
  *s_out = best_s;
  *b_out = best_b;
}

__global__ void choose_qparams_kernel(const float* __restrict__ w, int64_t n_groups, int64_t len,
                                      float maxq, int storage, Shrinks sh, void* s_store,
                                      void* b_store, float* __restrict__ s32,
                                      float* __restrict__ b32) {
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < n_groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    float s, b;
    choose_qparams_group(w + g * len, len, maxq, storage, sh, &s, &b);
    store_storage(s_store, g, s, storage);
    store_storage(b_store, g, b, storage);
    s32[g] = s;
    b32[g] = b;
  }
}

__global__ void quantize_with_params_kernel(const float* __restrict__ w,
                                            const float* __restrict__ s32,
                                            const float* __restrict__ b32, int64_t n, int64_t len,
                                            float maxq, float* __restrict__ q,
                                            float* __restrict__ dq) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = i / len;
    const float s = s32[g], b = b32[g];
    const float s_safe = (fabsf(s) < 1e-12f) ? 1.0f : s;
    const float qq = affine_q(w[i], b, s_safe, maxq);
    q[i] = qq;
    dq[i] = qq * s + b;
  }
}

// rtn_quantize (grid.py:224-246) on an fp32 view [n_groups, len].
__global__ void rtn_affine_kernel(const float* __restrict__ W, int64_t n_groups, int len,
                                  float maxq, int storage, Shrinks sh, uint8_t* __restrict__ q,
                                  void* s_store, void* b_store, float* __restrict__ dq) {
  for (int64_t g = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; g < n_groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    const float* p = W + g * len;
    float s, b;
    choose_qparams_group(p, len, maxq, storage, sh, &s, &b);
    store_storage(s_store, g, s, storage);
    store_storage(b_store, g, b, storage);
    const float s_safe = (fabsf(s) < 1e-12f) ? 1.0f : s;
    for (int i = 0; i < len; ++i) {
      const float qq = affine_q(p[i], b, s_safe, maxq);
      q[g * len + i] = (qq == qq) ? static_cast<uint8_t>(qq) : 0;
      dq[g * len + i] = qq * s + b;
    }
  }
}

int check_mx_mode(int mode) {
  MGQ_REQUIRE(mode == kMxfp4 || mode == kMxfp8, MGQ_ERR_VALUE,
              "not a microscaling mode: %d", mode);
  return MGQ_OK;
}

int check_dtype(int dtype, const char* what) {
  MGQ_REQUIRE(dtype == kF32 || dtype == kBF16 || dtype == kF16, MGQ_ERR_VALUE,
              "%s: unsupported dtype code %d", what, dtype);
  return MGQ_OK;
}

int check_bits(int bits) {
  MGQ_REQUIRE(bits >= 1 && bits <= 8, MGQ_ERR_VALUE, "unsupported bits: %d", bits);
  return MGQ_OK;
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int mgq_choose_mxfp_scale(const float* w, int64_t n_groups, int64_t group_len,
                                     int mode, uint8_t* scale_bytes, float* scales,
                                     void* stream) {
  clear_error();
  if (int rc = check_mx_mode(mode)) return rc;
  MGQ_REQUIRE(n_groups >= 0 && group_len >= 1, MGQ_ERR_SHAPE, "bad shape [%lld, %lld]",
              (long long)n_groups, (long long)group_len);
  if (n_groups == 0) return MGQ_OK;
  choose_mxfp_scale_kernel<<<elementwise_blocks(n_groups, kThreads), kThreads, 0,
                             as_stream(stream)>>>(w, n_groups, group_len,
                                                  mode == kMxfp4 ? 6.0f : 448.0f, scale_bytes,
                                                  scales);
  return check_launch("choose_mxfp_scale");
}

extern "C" int mgq_quantize_mxfp_with_scale(const float* w, const float* scales,
                                            int64_t n_groups, int64_t group_len, int mode,
                                            uint8_t* q, float* dq, void* stream) {
  clear_error();
  if (int rc = check_mx_mode(mode)) return rc;
  MGQ_REQUIRE(n_groups >= 0 && group_len >= 1, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n = n_groups * group_len;
  if (n == 0) return MGQ_OK;
  quantize_mxfp_kernel<<<elementwise_blocks(n, kThreads), kThreads, 0, as_stream(stream)>>>(
      w, scales, n, group_len, mode, q, dq);
  return check_launch("quantize_mxfp_with_scale");
}

extern "C" int mgq_dequantize_mxfp(const uint8_t* q, const uint8_t* scale_bytes,
                                   int64_t n_groups, int mode, float* out, void* stream) {
  clear_error();
  if (int rc = check_mx_mode(mode)) return rc;
  MGQ_REQUIRE(n_groups >= 0, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n = n_groups * kMxGroup;
  if (n == 0) return MGQ_OK;
  dequantize_mxfp_kernel<<<elementwise_blocks(n, kThreads), kThreads, 0, as_stream(stream)>>>(
      q, scale_bytes, n, mode, out);
  return check_launch("dequantize_mxfp");
}

extern "C" int mgq_rtn_quantize_mxfp(const void* W, int w_dtype, int64_t rows, int64_t cols,
                                     int mode, uint8_t* q, uint8_t* scale_bytes, float* dq,
                                     void* stream) {
  clear_error();
  if (int rc = check_mx_mode(mode)) return rc;
  if (int rc = check_dtype(w_dtype, "rtn_quantize_mxfp")) return rc;
  MGQ_REQUIRE(cols % kMxGroup == 0, MGQ_ERR_VALUE, "columns %lld not divisible by %d",
              (long long)cols, kMxGroup);
  MGQ_REQUIRE(rows >= 0 && cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n_groups = rows * (cols / kMxGroup);
  if (n_groups == 0) return MGQ_OK;
  const bool aligned = ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(q) |
                         reinterpret_cast<uintptr_t>(dq)) & 15u) == 0;
  const unsigned blocks = elementwise_blocks(n_groups, kThreads);
  hipStream_t st = as_stream(stream);
  if (!aligned)
    rtn_mxfp_kernel<<<blocks, kThreads, 0, st>>>(W, w_dtype, n_groups, mode, q, scale_bytes, dq);
  else if (w_dtype == kF32)
    rtn_mxfp_vec_kernel<float, false><<<blocks, kThreads, 0, st>>>(
        static_cast<const float*>(W), n_groups, mode, q, scale_bytes, dq);
  else if (w_dtype == kBF16)
    rtn_mxfp_vec_kernel<uint16_t, false><<<blocks, kThreads, 0, st>>>(
        static_cast<const uint16_t*>(W), n_groups, mode, q, scale_bytes, dq);
  else
    rtn_mxfp_vec_kernel<uint16_t, true><<<blocks, kThreads, 0, st>>>(
        static_cast<const uint16_t*>(W), n_groups, mode, q, scale_bytes, dq);
  return check_launch("rtn_quantize_mxfp");
}

extern "C" int mgq_dequantize_affine(const uint8_t* q, const void* scales, const void* biases,
                                     int storage_dtype, int64_t n_groups, int64_t group_size,
                                     float* out, void* stream) {
  clear_error();
  if (int rc = check_dtype(storage_dtype, "dequantize_affine")) return rc;
  MGQ_REQUIRE(n_groups >= 0 && group_size >= 1, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n = n_groups * group_size;
  if (n == 0) return MGQ_OK;
  dequantize_affine_kernel<<<elementwise_blocks(n, kThreads), kThreads, 0,
                             as_stream(stream)>>>(q, scales, biases, storage_dtype, n,
                                                  group_size, out);
  return check_launch("dequantize_affine");
}

extern "C" int mgq_choose_qparams(const float* w, int64_t n_groups, int64_t group_len, int bits,
                                  int method, int storage_dtype, int grid_steps,
                                  double max_shrink, void* s_store, void* b_store, float* s32,
                                  float* b32, void* stream) {
  clear_error();
  if (int rc = check_bits(bits)) return rc;
  if (int rc = check_dtype(storage_dtype, "choose_qparams")) return rc;
  MGQ_REQUIRE(method == MGQ_CLIP_MINMAX || method == MGQ_CLIP_MSE, MGQ_ERR_VALUE,
              "unsupported clip method %d", method);
  MGQ_REQUIRE(n_groups >= 0 && group_len >= 1, MGQ_ERR_SHAPE, "bad shape");
  Shrinks sh;
  if (int rc = make_shrinks(bits, method, grid_steps, max_shrink, &sh)) return rc;
  if (n_groups == 0) return MGQ_OK;
  choose_qparams_kernel<<<elementwise_blocks(n_groups, kThreads), kThreads, 0,
                          as_stream(stream)>>>(w, n_groups, group_len,
                                               static_cast<float>((1 << bits) - 1),
                                               storage_dtype, sh, s_store, b_store, s32, b32);
  return check_launch("choose_qparams");
}

extern "C" int mgq_quantize_with_params(const float* w, const float* s32, const float* b32,
                                        int64_t n_groups, int64_t group_len, int bits, float* q,
                                        float* dq, void* stream) {
  clear_error();
  if (int rc = check_bits(bits)) return rc;
  MGQ_REQUIRE(n_groups >= 0 && group_len >= 1, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n = n_groups * group_len;
  if (n == 0) return MGQ_OK;
  quantize_with_params_kernel<<<elementwise_blocks(n, kThreads), kThreads, 0,
                                as_stream(stream)>>>(w, s32, b32, n, group_len,
                                                     static_cast<float>((1 << bits) - 1), q, dq);
  return check_launch("quantize_with_params");
}

extern "C" int mgq_rtn_quantize_affine(const void* W, int w_dtype, int64_t rows, int64_t cols,
                                       int bits, int group_size, int method, int storage_dtype,
                                       uint8_t* q, void* s_store, void* b_store, float* dq,
                                       void* stream) {
  clear_error();
  if (int rc = check_bits(bits)) return rc;
  if (int rc = check_dtype(w_dtype, "rtn_quantize")) return rc;
  if (int rc = check_dtype(storage_dtype, "rtn_quantize")) return rc;
  MGQ_REQUIRE(method == MGQ_CLIP_MINMAX || method == MGQ_CLIP_MSE, MGQ_ERR_VALUE,
              "unsupported clip method %d", method);
  MGQ_REQUIRE(group_size >= 1 && cols % group_size == 0, MGQ_ERR_SHAPE,
              "cols %lld not divisible by group size %d", (long long)cols, group_size);
  const int64_t n_groups = rows * (cols / group_size);
  if (n_groups == 0) return MGQ_OK;
  MGQ_REQUIRE(w_dtype == kF32, MGQ_ERR_VALUE,
              "rtn_quantize: convert W to float32 first (got dtype code %d)", w_dtype);
  Shrinks sh;
  if (int rc = make_shrinks(bits, method, 20, 0.2, &sh)) return rc;
  rtn_affine_kernel<<<elementwise_blocks(n_groups, kThreads), kThreads, 0, as_stream(stream)>>>(
      static_cast<const float*>(W), n_groups, group_size, static_cast<float>((1 << bits) - 1),
      storage_dtype, sh, q, s_store, b_store, dq);
  return check_launch("rtn_quantize");
}
