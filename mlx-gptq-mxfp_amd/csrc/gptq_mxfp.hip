// Fused MXFP GPTQ solver: gptq.py:69-180 (_gptq_quantize_mxfp_groupwise)
// plus the dead-column fix of gptq.py:216-222 and the rel_err of
// gptq.py:300-302, for MXFP4 (E2M1 + E8M0) and MXFP8 (E4M3 + E8M0).
//
// Every 32-column group of every row is independent: it sees only its own
// 32x32 Hessian block Hg and the block's upper Cholesky-inverse factor U
// (hinv32). One thread owns one (batch item, row, group): its 32 weights stay
// in registers through the whole recurrence, so nothing touches HBM between
// reading W and writing (q, W_dq, scale byte). All lanes of a workgroup share
// (b, g), so Hg and U are wave-uniform and are read with scalar loads.
//
// Per (row, group), in the reference's order:
//   1. scale choice: groupwise = round(log2(max|w|/fmax)) (E8M0); safe =
//      candidate exponents e0+off (clamped to [-127,127]) scored by the
//      quadratic form err^T Hg err, strict '<' so the first best wins;
//   2. 32-step GPTQ with the chosen fixed scale:
//        dq_c = Q(w_c);  err = (w_c - dq_c) / U[c,c];  w_j -= err * U[c,j] (j>c)
//      (sub, IEEE div, mul, sub: the exact torch op sequence);
//   3. safe search keeps the GPTQ result only if its objective <= the best
//      RTN candidate's;
//   4. range guard: every |dq| <= max(32 * max|orig|, 2^-126), else the RTN
//      baseline at the chosen scale.
// Objectives are fp32 sums in a fixed order (not torch's einsum order), so
// near-exact ties between candidates may resolve differently from the
// reference; every encoding itself is bit-exact.
#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {

int launch_hinv32(const float* H, int64_t B, int64_t C, float damp, int max_attempts, float* U,
                  int32_t* attempts, hipStream_t s);

namespace {

constexpr int kG = 32;
constexpr int kThreads = 256;
constexpr int kMaxOffsets = 8;

struct Offsets {
  int n;
  int v[kMaxOffsets];
};

// gptq.py:216-222: diag(H) <= 0 marks a dead column; its diagonal becomes 1
// (in place) and its weights are treated as 0.
__global__ void dead_fix_kernel(float* __restrict__ H, int64_t B, int64_t C,
                                uint8_t* __restrict__ dead) {
  const int64_t n = B * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / C, c = i % C;
    float* d = H + b * C * C + c * C + c;
    const bool is_dead = *d <= 0.0f;
    if (is_dead) *d = 1.0f;
    dead[i] = is_dead ? 1 : 0;
  }
}

template <int MODE>
__device__ inline float quant_dq(float w, float scale, uint32_t* code) {
  float dq;
  *code = mx_quant(w, scale, MODE, &dq);
  return dq;
}

// e^T Hg e. Hg row stride C; values are wave-uniform (scalar loads).
// Symmetric blocks use the upper triangle (H_ii e_i^2 + 2 sum_{j>i} H_ij e_i e_j
// as e_i * (H_ii e_i + 2 * sum_{j>i} H_ij e_j)); otherwise the full form.
__device__ inline float quad_form(const float (&e)[kG], const float* __restrict__ Hg, int64_t C,
                                  bool sym) {
  float obj = 0.0f;
  if (sym) {
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      float s = 0.0f;
#pragma unroll
      for (int j = i + 1; j < kG; ++j) s += Hg[i * C + j] * e[j];
      const float t = Hg[i * C + i] * e[i] + 2.0f * s;
      obj += e[i] * t;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      float t = 0.0f;
#pragma unroll
      for (int j = 0; j < kG; ++j) t += Hg[i * C + j] * e[j];
      obj += e[i] * t;
    }
  }
  return obj;
}

__device__ inline float nan_max(float m, float a) { return (a > m || a != a) ? a : m; }

template <typename T>
__device__ inline float load_w(const T* p, int i);
template <>
__device__ inline float load_w<float>(const float* p, int i) { return p[i]; }
template <>
__device__ inline float load_w<uint16_t>(const uint16_t* p, int i) { return bf16_to_f32(p[i]); }

struct F16Tag {};

template <typename TIn, bool IS_F16, int MODE, bool SAFE>
__global__ void __launch_bounds__(kThreads)
    mxfp_solve_kernel(const TIn* __restrict__ W, int64_t B, int64_t R, int64_t C,
                      const float* __restrict__ H, const float* __restrict__ U,
                      const uint8_t* __restrict__ dead, Offsets offs, uint8_t* __restrict__ q_out,
                      uint8_t* __restrict__ s_out, float* __restrict__ W_dq,
                      double* __restrict__ rel_part) {
  const int64_t G = C / kG;
  const int64_t chunks = (R + kThreads - 1) / kThreads;
  const int64_t bg = blockIdx.x / chunks;
  const int64_t chunk = blockIdx.x % chunks;
  const int64_t b = bg / G, g = bg % G;
  const int64_t r_raw = chunk * kThreads + threadIdx.x;
  const bool valid = r_raw < R;
  const int64_t r = valid ? r_raw : R - 1;

  const float* __restrict__ Hg = H + b * C * C + (g * kG) * C + g * kG;
  const float* __restrict__ Ug = U + (b * G + g) * kG * kG;
  const uint8_t* __restrict__ dd = dead + b * C + g * kG;
  const int64_t base = (b * R + r) * C + g * kG;
  const float fmax = (MODE == kMxfp4) ? 6.0f : 448.0f;

  // symmetric Hessian block? (uniform; exact bit equality)
  bool sym = true;
  if (SAFE) {
#pragma unroll
    for (int i = 0; i < kG; ++i)
#pragma unroll
      for (int j = i + 1; j < kG; ++j)
        sym = sym && (__float_as_uint(Hg[i * C + j]) == __float_as_uint(Hg[j * C + i]));
  }

  float raw[kG], orig[kG];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kG; ++i) {
    float v;
    if constexpr (IS_F16) {
      v = f16_to_f32(reinterpret_cast<const uint16_t*>(W)[base + i]);
    } else {
      v = load_w<TIn>(W + base, i);
    }
    raw[i] = v;
    orig[i] = dd[i] ? 0.0f : v;
    amax = (i == 0) ? fabsf(orig[i]) : nan_max(amax, fabsf(orig[i]));
  }

  // 1. scale choice
  const int e0 = e8m0_exponent(amax, fmax);
  int e_sel = e0;
  float best = 0.0f;
  if (SAFE) {
    float err[kG];
    for (int o = 0; o < offs.n; ++o) {
      int e = e0 + offs.v[o];
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      const float sc = exp2_int(e);
#pragma unroll
      for (int i = 0; i < kG; ++i) {
        uint32_t code;
        err[i] = quant_dq<MODE>(orig[i], sc, &code) - orig[i];
      }
      const float obj = quad_form(err, Hg, C, sym);
      if (o == 0 || obj < best) {
        best = obj;
        e_sel = e;
      }
    }
  }
  const float scale = exp2_int(e_sel);

  // 2. GPTQ recurrence with the fixed scale; w[c] becomes dq_c.
  float w[kG];
  uint32_t codes[kG / 4];
#pragma unroll
  for (int i = 0; i < kG; ++i) w[i] = orig[i];
#pragma unroll
  for (int i = 0; i < kG / 4; ++i) codes[i] = 0u;
#pragma unroll
  for (int c = 0; c < kG; ++c) {
    uint32_t code;
    const float dq = quant_dq<MODE>(w[c], scale, &code);
    const float err = (w[c] - dq) / Ug[c * kG + c];
#pragma unroll
    for (int j = c + 1; j < kG; ++j) w[j] = w[j] - err * Ug[c * kG + j];
    w[c] = dq;
    codes[c / 4] |= code << (8 * (c % 4));
  }

  // 3. GPTQ vs best RTN candidate (safe search only)
  bool use_gptq = true;
  if (SAFE) {
    float err[kG];
#pragma unroll
    for (int i = 0; i < kG; ++i) err[i] = w[i] - orig[i];
    use_gptq = quad_form(err, Hg, C, sym) <= best;
  }
  // 4. range guard on the selected result
  float limit = amax * 32.0f;
  const float floor_ = __uint_as_float(0x00800000u);  // 2^-126
  limit = (limit != limit) ? limit : fmaxf(limit, floor_);
  bool ok = use_gptq;
  if (use_gptq) {
#pragma unroll
    for (int i = 0; i < kG; ++i) ok = ok && (fabsf(w[i]) <= limit);
  }
  if (!ok) {  // RTN baseline at the chosen scale
#pragma unroll
    for (int i = 0; i < kG / 4; ++i) codes[i] = 0u;
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      uint32_t code;
      w[i] = quant_dq<MODE>(orig[i], scale, &code);
      codes[i / 4] |= code << (8 * (i % 4));
    }
  }

  double num = 0.0, den = 0.0;
  if (valid) {
    uint32_t* qp = reinterpret_cast<uint32_t*>(q_out + base);
#pragma unroll
    for (int i = 0; i < kG / 4; ++i) qp[i] = codes[i];
#pragma unroll
    for (int i = 0; i < kG; ++i) {
      W_dq[base + i] = w[i];
      const double d = static_cast<double>(w[i]) - static_cast<double>(raw[i]);
      num += d * d;
      den += static_cast<double>(raw[i]) * static_cast<double>(raw[i]);
    }
    s_out[(b * R + r) * G + g] = static_cast<uint8_t>(e_sel + 127);
  }
  if (rel_part) {
    // wave reduction, one (num, den) pair per wave
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      num += __shfl_xor(num, off);
      den += __shfl_xor(den, off);
    }
    if ((threadIdx.x & 63) == 0) {
      const int64_t waves = (R + 63) / 64;
      const int64_t wv = chunk * (kThreads / 64) + (threadIdx.x >> 6);
      if (wv < waves) {
        double* pp = rel_part + ((b * G + g) * waves + wv) * 2;
        pp[0] = num;
        pp[1] = den;
      }
    }
  }
}

// rel[b] = sqrt(sum num) / max(sqrt(sum den), 1e-12), partials summed in order.
__global__ void rel_err_kernel(const double* __restrict__ part, int64_t n_per_b, int64_t B,
                               float* __restrict__ rel) {
  const int64_t b = blockIdx.x;
  __shared__ double sn[256], sd[256];
  double n = 0.0, d = 0.0;
  for (int64_t i = threadIdx.x; i < n_per_b; i += blockDim.x) {
    n += part[(b * n_per_b + i) * 2];
    d += part[(b * n_per_b + i) * 2 + 1];
  }
  sn[threadIdx.x] = n;
  sd[threadIdx.x] = d;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      sn[threadIdx.x] += sn[threadIdx.x + s];
      sd[threadIdx.x] += sd[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float num = sqrtf(static_cast<float>(sn[0]));
    float den = sqrtf(static_cast<float>(sd[0]));
    den = den < 1e-12f ? 1e-12f : den;
    rel[b] = num / den;
  }
}

struct WsLayout {
  int64_t dead_off, u_off, rel_off, total;
};

WsLayout ws_layout(int64_t B, int64_t R, int64_t C) {
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t G = C / kG;
  WsLayout L;
  L.dead_off = 0;
  L.u_off = al(B * C);
  L.rel_off = L.u_off + al(B * G * kG * kG * 4);
  L.total = L.rel_off + al(B * G * ((R + 63) / 64) * 2 * 8);
  return L;
}

template <typename TIn, bool IS_F16>
int launch_solve(const void* W, int64_t B, int64_t R, int64_t C, const float* H, const float* U,
                 const uint8_t* dead, int mode, bool safe, const Offsets& offs, uint8_t* q,
                 uint8_t* s, float* W_dq, double* rel_part, hipStream_t st) {
  const int64_t G = C / kG;
  const int64_t blocks = B * G * ((R + kThreads - 1) / kThreads);
  const TIn* w = static_cast<const TIn*>(W);
#define MGQ_LAUNCH(MODE, SAFE)                                                              \
  mxfp_solve_kernel<TIn, IS_F16, MODE, SAFE><<<static_cast<unsigned>(blocks), kThreads, 0, st>>>( \
      w, B, R, C, H, U, dead, offs, q, s, W_dq, rel_part)
  if (mode == kMxfp4) {
    if (safe) MGQ_LAUNCH(kMxfp4, true); else MGQ_LAUNCH(kMxfp4, false);
  } else {
    if (safe) MGQ_LAUNCH(kMxfp8, true); else MGQ_LAUNCH(kMxfp8, false);
  }
#undef MGQ_LAUNCH
  return check_launch("mxfp solve");
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int64_t mgq_gptq_mxfp_workspace_size(int64_t B, int64_t R, int64_t C) {
  return ws_layout(B, R, C).total;
}

extern "C" int mgq_gptq_mxfp(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C,
                             float* H, int mode, int algorithm, float damp, int max_attempts,
                             const int32_t* offsets, int n_offsets, uint8_t* q_out,
                             uint8_t* scales_out, float* W_dq, float* rel_err,
                             int32_t* attempts, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  clear_error();
  MGQ_REQUIRE(mode == kMxfp4 || mode == kMxfp8, MGQ_ERR_VALUE, "not a microscaling mode: %d",
              mode);
  MGQ_REQUIRE(algorithm == 0 || algorithm == 1, MGQ_ERR_VALUE,
              "unsupported MXFP GPTQ algorithm code: %d", algorithm);
  MGQ_REQUIRE(w_dtype == kF32 || w_dtype == kBF16 || w_dtype == kF16, MGQ_ERR_VALUE,
              "unsupported weight dtype code %d", w_dtype);
  MGQ_REQUIRE(B >= 0 && R >= 0 && C >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(C % kG == 0, MGQ_ERR_SHAPE, "in_features %lld not divisible by group %d",
              (long long)C, kG);
  MGQ_REQUIRE(max_attempts >= 1, MGQ_ERR_VALUE, "max_attempts must be >= 1");
  Offsets offs{0, {0}};
  if (algorithm == 1) {
    MGQ_REQUIRE(offsets != nullptr && n_offsets >= 1 && n_offsets <= kMaxOffsets, MGQ_ERR_VALUE,
                "safe-scale-search needs 1..%d exponent offsets", kMaxOffsets);
    offs.n = n_offsets;
    for (int i = 0; i < n_offsets; ++i) offs.v[i] = offsets[i];
  }
  const WsLayout L = ws_layout(B, R, C);
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MGQ_ERR_WORKSPACE,
              "mxfp workspace %lld < %lld bytes", (long long)workspace_bytes,
              (long long)L.total);
  if (B == 0 || C == 0) return MGQ_OK;
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  uint8_t* dead = reinterpret_cast<uint8_t*>(ws + L.dead_off);
  float* U = reinterpret_cast<float*>(ws + L.u_off);
  double* rel_part = reinterpret_cast<double*>(ws + L.rel_off);

  dead_fix_kernel<<<elementwise_blocks(B * C, 256), 256, 0, st>>>(H, B, C, dead);
  if (int rc = check_launch("dead-column fix")) return rc;
  if (int rc = launch_hinv32(H, B, C, damp, max_attempts, U, attempts, st)) return rc;
  if (R == 0) return MGQ_OK;
  int rc;
  if (w_dtype == kF32) {
    rc = launch_solve<float, false>(W, B, R, C, H, U, dead, mode, algorithm == 1, offs, q_out,
                                    scales_out, W_dq, rel_err ? rel_part : nullptr, st);
  } else if (w_dtype == kBF16) {
    rc = launch_solve<uint16_t, false>(W, B, R, C, H, U, dead, mode, algorithm == 1, offs, q_out,
                                       scales_out, W_dq, rel_err ? rel_part : nullptr, st);
  } else {
    rc = launch_solve<uint16_t, true>(W, B, R, C, H, U, dead, mode, algorithm == 1, offs, q_out,
                                      scales_out, W_dq, rel_err ? rel_part : nullptr, st);
  }
  if (rc) return rc;
  if (rel_err) {
    const int64_t n_per_b = (C / kG) * ((R + 63) / 64);
    rel_err_kernel<<<static_cast<unsigned>(B), 256, 0, st>>>(rel_part, n_per_b, B, rel_err);
    if (int rc2 = check_launch("rel_err")) return rc2;
  }
  return MGQ_OK;
}
