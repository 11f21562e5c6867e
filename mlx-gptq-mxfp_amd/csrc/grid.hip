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


// Range audit of one stored artifact against its source weights
// (validate_artifacts.py:15-68), fused into one pass: every element is
// dequantized in-register (dequantize_artifact, grid.py:154-164), and per
// 32-column group g the kernel forms smax = max|source|, amax = max|deq|,
// limit = max(fp64(smax) * 32, 2^-126) and ratio = fp64(amax) / limit.
// Results go to `stats` (zeroed by the caller) with one atomic per block:
//   u64[0] non-finite dequantized values, u64[1] groups with amax > limit,
//   u64[2] max ratio (bits of a non-negative fp64; NaN ratios skipped),
//   u64[3] max |source| (bits of a non-negative fp32), u64[4] max |deq|.
// The grid is capped (grid-stride loop), so the atomics stay few.
constexpr int kAuditBlocks = 2048;

__device__ inline float nanless_max(float a, float b) { return b > a ? b : a; }

struct AuditAcc {
  unsigned long long nonfinite = 0, exceed = 0;
  double rmax = 0.0;
  float smax = 0.0f, amax = 0.0f;
  // one group's maxima, held by its leading lane
  __device__ void group(float gs, float ga) {
    const double limit = fmax(static_cast<double>(gs) * 32.0, 0x1p-126);
    const double r = static_cast<double>(ga) / limit;
    if (static_cast<double>(ga) > limit) ++exceed;
    if (r == r) rmax = fmax(rmax, r);
    smax = nanless_max(smax, gs);
    amax = nanless_max(amax, ga);
  }
  // wave, then workgroup reduction; one atomic per block and field
  __device__ void flush(unsigned long long* stats) {
    __shared__ unsigned long long s_cnt[2][kThreads / 64];
    __shared__ double s_r[kThreads / 64];
    __shared__ float s_m[2][kThreads / 64];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      nonfinite += __shfl_xor(nonfinite, o);
      exceed += __shfl_xor(exceed, o);
      rmax = fmax(rmax, __shfl_xor(rmax, o));
      smax = nanless_max(smax, __shfl_xor(smax, o));
      amax = nanless_max(amax, __shfl_xor(amax, o));
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      s_cnt[0][w] = nonfinite, s_cnt[1][w] = exceed, s_r[w] = rmax;
      s_m[0][w] = smax, s_m[1][w] = amax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int k = 1; k < kThreads / 64; ++k) {
        s_cnt[0][0] += s_cnt[0][k], s_cnt[1][0] += s_cnt[1][k];
        s_r[0] = fmax(s_r[0], s_r[k]);
        s_m[0][0] = nanless_max(s_m[0][0], s_m[0][k]);
        s_m[1][0] = nanless_max(s_m[1][0], s_m[1][k]);
      }
      if (s_cnt[0][0]) atomicAdd(&stats[0], s_cnt[0][0]);
      if (s_cnt[1][0]) atomicAdd(&stats[1], s_cnt[1][0]);
      atomicMax(&stats[2], static_cast<unsigned long long>(__double_as_longlong(s_r[0])));
      atomicMax(&stats[3], static_cast<unsigned long long>(__float_as_uint(s_m[0][0])));
      atomicMax(&stats[4], static_cast<unsigned long long>(__float_as_uint(s_m[1][0])));
    }
  }
};

__device__ inline float audit_deq(uint32_t c, float sc, float bias, int mode) {
  if (mode == kAffine) return static_cast<float>(c) * sc + bias;
  return ((mode == kMxfp4) ? e2m1_value(c & 15u) : e4m3_value(c)) * sc;
}

// One element per lane (any alignment, any affine group size); the 32 lanes
// of a half-wave hold one group together (n and the stride are multiples
// of 32).
__global__ void __launch_bounds__(kThreads)
    range_audit_kernel(const void* __restrict__ src, int src_dtype, const uint8_t* __restrict__ q,
                       const void* __restrict__ scales, const void* __restrict__ biases,
                       int storage, int mode, int64_t group_size, int64_t n,
                       unsigned long long* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  AuditAcc acc;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i - (lane & 31) < n;
       i += stride) {
    const float sv = fabsf(load_any(src, i, src_dtype));
    float sc, bias = 0.0f;
    if (mode == kAffine) {
      const int64_t g = i / group_size;
      sc = load_storage(scales, g, storage);
      bias = load_storage(biases, g, storage);
    } else {
      sc = scale_from_byte(static_cast<const uint8_t*>(scales)[i / kMxGroup]);
    }
    const float v = audit_deq(q[i], sc, bias, mode);
    if (!isfinite(v)) ++acc.nonfinite;
    float gs = sv, ga = fabsf(v);
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
      gs = nanless_max(gs, __shfl_xor(gs, o));
      ga = nanless_max(ga, __shfl_xor(ga, o));
    }
    if ((lane & 31) == 0) acc.group(gs, ga);
  }
  acc.flush(stats);
}

// Eight elements per lane from 16-byte-aligned rows: 16 (bf16 / f16) or 32
// (f32) bytes of source and 8 code bytes per load; four lanes hold one
// 32-column group (n8 = n / 8 and the stride are multiples of 4). The
// affine group size is a multiple of 8, so a lane's eight values share one
// scale. Each lane issues the loads of kAuditUnroll grid-stride units
// before it evaluates any of them (2 and 4 measured no faster than 1; 4
// needs 102 VGPRs). For MXFP4 (MX4 = true) a lane needs no per-element
// dequantization: every value of a group is e2m1(c) * sc with one positive
// power-of-two scale, so max|deq| = e2m1(max(c & 7)) * sc (0 when every
// code is 0), and the values are non-finite exactly when sc is inf (E8M0
// byte 255). max|source| is taken on the bit patterns with the sign cleared
// (monotonic in |x|; NaN patterns count as 0, as the float path's compare
// skips NaN).
constexpr int kAuditUnroll = 1;

template <int SD>
__device__ inline float src_absmax(const uint4& a, const uint4& b) {
  if constexpr (SD == kF32) {
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t v = w[k] & 0x7fffffffu;
      m = max(m, v > 0x7f800000u ? 0u : v);
    }
    return __uint_as_float(m);
  } else {
    constexpr uint32_t kInf = (SD == kBF16) ? 0x7f80u : 0x7c00u;
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
    uint32_t m = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = w[k] & 0x7fffu, hi = (w[k] >> 16) & 0x7fffu;
      m = max(m, max(lo > kInf ? 0u : lo, hi > kInf ? 0u : hi));
    }
    return (SD == kBF16) ? __uint_as_float(m << 16) : f16_to_f32(static_cast<uint16_t>(m));
  }
}

template <int SD, bool MX4>
__global__ void __launch_bounds__(kThreads)
    range_audit_vec_kernel(const void* __restrict__ src, const uint8_t* __restrict__ q,
                           const void* __restrict__ scales, const void* __restrict__ biases,
                           int storage, int mode, int64_t group_size, int64_t n8,
                           unsigned long long* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  AuditAcc acc;
  for (int64_t t0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t0 - (lane & 3) < n8;
       t0 += stride * kAuditUnroll) {
    uint4 ra[kAuditUnroll], rb[kAuditUnroll];
    uint2 rc[kAuditUnroll];
    float sc[kAuditUnroll], bias[kAuditUnroll];
    bool on[kAuditUnroll];
#pragma unroll
    for (int u = 0; u < kAuditUnroll; ++u) {
      const int64_t t = t0 + u * stride;
      on[u] = t - (lane & 3) < n8;  // the same in the group's four lanes
      bias[u] = 0.0f;
      if (on[u]) {
        if constexpr (SD == kF32) {
          ra[u] = reinterpret_cast<const uint4*>(src)[2 * t];
          rb[u] = reinterpret_cast<const uint4*>(src)[2 * t + 1];
        } else {
          ra[u] = reinterpret_cast<const uint4*>(src)[t];
        }
        rc[u] = reinterpret_cast<const uint2*>(q)[t];
        if (mode == kAffine) {
          const int64_t g = (8 * t) / group_size;
          sc[u] = load_storage(scales, g, storage);
          bias[u] = load_storage(biases, g, storage);
        } else {
          sc[u] = scale_from_byte(static_cast<const uint8_t*>(scales)[t >> 2]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kAuditUnroll; ++u) {
      if (!on[u]) continue;
      if constexpr (MX4) {
        float gs = src_absmax<SD>(ra[u], rb[u]);
        const uint32_t x = rc[u].x & 0x07070707u, y = rc[u].y & 0x07070707u;
        uint32_t mc = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) mc = max(mc, max((x >> (8 * k)) & 7u, (y >> (8 * k)) & 7u));
        float ga = mc ? e2m1_value(mc) * sc[u] : 0.0f;
        if (isinf(sc[u])) acc.nonfinite += 8;
#pragma unroll
        for (int o = 2; o >= 1; o >>= 1) {
          gs = nanless_max(gs, __shfl_xor(gs, o));
          ga = nanless_max(ga, __shfl_xor(ga, o));
        }
        if ((lane & 3) == 0) acc.group(gs, ga);
        continue;
      }
      float sv[8];
      if constexpr (SD == kF32) {
        sv[0] = __uint_as_float(ra[u].x), sv[1] = __uint_as_float(ra[u].y);
        sv[2] = __uint_as_float(ra[u].z), sv[3] = __uint_as_float(ra[u].w);
        sv[4] = __uint_as_float(rb[u].x), sv[5] = __uint_as_float(rb[u].y);
        sv[6] = __uint_as_float(rb[u].z), sv[7] = __uint_as_float(rb[u].w);
      } else {
        const uint32_t w[4] = {ra[u].x, ra[u].y, ra[u].z, ra[u].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if constexpr (SD == kBF16) {
            sv[2 * k] = __uint_as_float(w[k] << 16);
            sv[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
          } else {
            sv[2 * k] = f16_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
            sv[2 * k + 1] = f16_to_f32(static_cast<uint16_t>(w[k] >> 16));
          }
        }
      }
      float gs = 0.0f, ga = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t c = ((k < 4 ? rc[u].x : rc[u].y) >> (8 * (k & 3))) & 0xffu;
        const float v = audit_deq(c, sc[u], bias[u], mode);
        if (!isfinite(v)) ++acc.nonfinite;
        gs = nanless_max(gs, fabsf(sv[k]));
        ga = nanless_max(ga, fabsf(v));
      }
#pragma unroll
      for (int o = 2; o >= 1; o >>= 1) {
        gs = nanless_max(gs, __shfl_xor(gs, o));
        ga = nanless_max(ga, __shfl_xor(ga, o));
      }
      if ((lane & 3) == 0) acc.group(gs, ga);
    }
  }
  acc.flush(stats);
}

template <bool MX4>
void launch_audit_vec(int sd, unsigned blocks, hipStream_t st, const void* src, const uint8_t* q,
                      const void* scales, const void* biases, int storage, int mode,
                      int64_t group_size, int64_t n8, unsigned long long* stats) {
  if (sd == kF32)
    range_audit_vec_kernel<kF32, MX4><<<blocks, kThreads, 0, st>>>(src, q, scales, biases, storage,
                                                                   mode, group_size, n8, stats);
  else if (sd == kBF16)
    range_audit_vec_kernel<kBF16, MX4><<<blocks, kThreads, 0, st>>>(src, q, scales, biases, storage,
                                                                    mode, group_size, n8, stats);
  else
    range_audit_vec_kernel<kF16, MX4><<<blocks, kThreads, 0, st>>>(src, q, scales, biases, storage,
                                                                   mode, group_size, n8, stats);
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

extern "C" int mgq_range_audit(const void* source, int source_dtype, const uint8_t* q,
                               const void* scales, const void* biases, int storage_dtype,
                               int mode, int64_t rows, int64_t cols, int64_t group_size,
                               unsigned long long* stats, void* stream) {
  clear_error();
  if (int rc = check_dtype(source_dtype, "range_audit")) return rc;
  MGQ_REQUIRE(mode == kAffine || mode == kMxfp4 || mode == kMxfp8, MGQ_ERR_VALUE,
              "unsupported mode %d", mode);
  MGQ_REQUIRE(rows >= 0 && cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(cols % kMxGroup == 0, MGQ_ERR_SHAPE, "columns %lld not divisible by %d",
              (long long)cols, kMxGroup);
  if (mode == kAffine) {
    if (int rc = check_dtype(storage_dtype, "range_audit")) return rc;
    MGQ_REQUIRE(group_size >= 1 && cols % group_size == 0, MGQ_ERR_SHAPE,
                "columns %lld not divisible by group %lld", (long long)cols,
                (long long)group_size);
    MGQ_REQUIRE(biases != nullptr, MGQ_ERR_VALUE, "affine artifacts need biases");
  } else {
    MGQ_REQUIRE(group_size == kMxGroup, MGQ_ERR_VALUE, "mxfp requires group size %d", kMxGroup);
  }
  MGQ_REQUIRE(stats != nullptr, MGQ_ERR_VALUE, "stats required");
  const int64_t n = rows * cols;
  if (n == 0) return MGQ_OK;
  hipStream_t st = as_stream(stream);
  const bool vec = ((reinterpret_cast<uintptr_t>(source) | reinterpret_cast<uintptr_t>(q)) & 15u) == 0 &&
                   (mode != kAffine || group_size % 8 == 0);
  const int64_t units = vec ? n / 8 : n;
  int64_t nb = (units + kThreads - 1) / kThreads;
  if (nb > kAuditBlocks) nb = kAuditBlocks;
  const unsigned blocks = static_cast<unsigned>(nb);
  if (!vec)
    range_audit_kernel<<<blocks, kThreads, 0, st>>>(source, source_dtype, q, scales, biases,
                                                    storage_dtype, mode, group_size, n, stats);
  else if (mode == kMxfp4)
    launch_audit_vec<true>(source_dtype, blocks, st, source, q, scales, biases, storage_dtype,
                           mode, group_size, units, stats);
  else
    launch_audit_vec<false>(source_dtype, blocks, st, source, q, scales, biases, storage_dtype,
                            mode, group_size, units, stats);
  return check_launch("range_audit");
}
