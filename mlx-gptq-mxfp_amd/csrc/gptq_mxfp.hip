// Fused MXFP GPTQ solver: gptq.py:69-180 (_gptq_quantize_mxfp_groupwise)
// plus the dead-column fix of gptq.py:216-222 and the rel_err of
// gptq.py:300-302, for MXFP4 (E2M1 + E8M0) and MXFP8 (E4M3 + E8M0).
//
// Every 32-column group of every row is independent: it sees only its own
// 32x32 Hessian block Hg and the block's upper Cholesky-inverse factor U
// (hinv32). One thread owns one (batch item, row, group): its 32 weights sit
// in LDS and its codes and errors in registers through the whole solve, so
// nothing touches HBM between reading W and writing (q, packed q, W_dq,
// scale byte). All lanes of a workgroup share (b, g): Hg (as bf16 parts)
// and U (as V, each row scaled by its diagonal's reciprocal) are staged once
// per workgroup in LDS and read there with uniform addresses.
//
// Per (row, group), in the reference's order:
//   1. scale choice: groupwise = round(log2(max|w|/fmax)) (E8M0); safe =
//      candidate exponents e0+off (clamped to [-127,127]) scored by the
//      quadratic form err^T Hg err, strict '<' so the first best wins;
//   2. 32-step GPTQ with the chosen fixed scale:
//        dq_c = Q(w_c);  err = (w_c - dq_c) / U[c,c];  w_j -= err * U[c,j] (j>c)
//      computed as a_c = w_c - dq_c and w_j -= a_c * V[c,j] with
//      V[c,j] = U[c,j] * RN(1/U[c,c]) formed once per block, one fused
//      multiply-add per update (torch rounds err, the product and the
//      difference; the two agree to an ulp or two per term);
//   3. safe search keeps the GPTQ result only if its objective <= the best
//      RTN candidate's;
//   4. range guard: every |dq| <= max(32 * max|orig|, 2^-126), else the RTN
//      baseline at the chosen scale.
// Objectives have fp32 accuracy (exact bf16 x bf16 products of three-way
// split operands, fp32 accumulation) but a fixed summation order, not
// torch's einsum order, so ties within a few fp32 ulps between candidates
// may resolve differently from the reference; every encoding itself is
// bit-exact.
#include <type_traits>

#include "mgq_capi.h"
#include "mgq_common.h"
#include "mx_hw.h"

namespace mgq {

int launch_hinv32(float* H, int64_t B, int64_t C, float damp, int max_attempts, float* U,
                  int32_t* attempts, float* Hc, uint8_t* dead, hipStream_t s);

namespace {

constexpr int kG = 32;
// 512 threads (8 waves) per workgroup: the per-workgroup LDS (the weights'
// 64 KB plus Ut, the H split and ydiag, 74 KB in all) lets two workgroups
// share a CU, i.e. 4 waves per SIMD, which the kernel reaches in 128 VGPRs
// without spilling (amdgpu_waves_per_eu below). With 256 threads the fixed
// part would hold the CU to 3 workgroups, 3 waves per SIMD.
constexpr int kThreads = 512;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dealt round-robin
constexpr int kMaxOffsets = 8;

struct Offsets {
  int n;
  int v[kMaxOffsets];
};

// Exact reference projection of one element (code and dq), w / scale done
// as w * inv_scale (identical for power-of-two scales), on the hardware MX
// conversions. NONAN: exact only where w * inv_scale is not NaN (the
// recurrence's fast pass, which a NaN sends to the exact pass anyway).
template <int MODE, bool NONAN = false>
__device__ inline uint32_t quant_exact(float w, float inv_scale, float scale, float* dq) {
  if constexpr (MODE == kMxfp4)
    return NONAN ? mx4_encode_hw_nonan(w, inv_scale, scale, dq) : mx4_encode_hw(w, inv_scale, scale, dq);
  else
    return NONAN ? mx8_encode_hw_nonan(w, inv_scale, scale, dq) : mx8_encode_hw(w, inv_scale, scale, dq);
}

// (dq - w) / scale of eight weights for scoring a scale candidate.
template <int MODE>
__device__ inline void quant_err8(const float (&w)[8], float scale, float inv_scale, float lim,
                                  float* e) {
  if constexpr (MODE == kMxfp4) {
    float t[8];
    mx4_cand_err8(w, scale, inv_scale, t);
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = t[j];
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x[4] = {w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]};
      float t[4];
      mx8_cand_err4(x, scale, inv_scale, lim, t);
#pragma unroll
      for (int j = 0; j < 4; ++j) e[4 * h + j] = t[j];
    }
  }
}

// e^T Hg e on the matrix cores, for the 64 rows of a wave at once.
//
// P^T = Hg E^T is a 32x32 by 32x64 product: two 32-row blocks of E, each
// v_mfma_f32_32x32x16_bf16 over K = 32. Every fp32 operand is split into
// three bf16 parts, x = x1 + x2 + x3 exactly (each part holds the next 8
// significant bits; exact for |x| >= 2^-100), and the product is
// accumulated in fp32 from the partial products that carry more than 2^-24
// of the result: h1 e1, h1 e2, h2 e1, h1 e3, h2 e2, h3 e1 (each bf16 x bf16
// product is exact). The objective therefore has the accuracy of an fp32
// sum, as the reference's fp32 einsum (gptq.py:123-125,168); only its
// summation order differs.
// Layouts (32x32x16 bf16): A lane l = row l%32, k = 8(l/32)+0..7; B lane l =
// k = 8(l/32)+0..7, column l%32; D lane l register r = row 8(r/4)+4(l/32)+
// r%4, column l%32.
//   - A = Hg: lane l needs Hg[l%32][16kc + 8(l/32) + 0..7]; the three parts
//     of the workgroup's block are staged in LDS (HSplit) in exactly that
//     order, so each operand is one conflict-free 16-byte read per lane.
//   - B = E^T of a 32-row block: lane l needs row l%32 of the block, columns
//     16kc + 8(l/32) + 0..7. Each lane owns its own row's e[]; one
//     v_permlane32_swap of (e[16kc..+7], e[16kc+8..+15]) yields block 0's B
//     in the first result and block 1's in the second.
//   - D of block 0 (rows 0-31) and block 1 (rows 32-63) hold P[i][c] with
//     i = l%32 (+32) and c in S0 = {8(r/4)+r%4} on lanes < 32 or S1 = S0 + 4
//     on lanes >= 32; one more swap of (D0, D1) gives every lane its own row
//     for c in S0 (first) and S1 (second), so obj = sum_c e[c] P[c] is local.
// All 64 lanes of the wave must execute this together.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// The three bf16 parts of a 32x32 Hessian block in the A-operand order:
// part p, K-chunk kc, row c, half h = the 8 values Hg[c][16kc + 8h + 0..7].
struct HSplit {
  u32x4_t v[3][2][kG][2];
};

// Two values rounded to bf16 as one packed word (v_cvt_pk_bf16_f32), and the
// halves of such a word widened back to fp32.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2v_t));
}
__device__ inline float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ inline float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// The three-way split of eight values: x = a + b + c with a = RN_bf16(x),
// b = RN_bf16(x - a), c = x - a - b (each difference exact, and c exact in
// bf16), two values at a time: each part is rounded as a pair and widened
// back from the packed word.
__device__ inline void split3x8(const float* x, bf16x8_t& a, bf16x8_t& b, bf16x8_t& c) {
  u32x4_t pa, pb, pc;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t wa = pk_bf16(x[2 * p], x[2 * p + 1]);
    const float r0 = x[2 * p] - bf16_lo(wa), r1 = x[2 * p + 1] - bf16_hi(wa);  // exact
    const uint32_t wb = pk_bf16(r0, r1);
    const float s0 = r0 - bf16_lo(wb), s1 = r1 - bf16_hi(wb);  // exact, and exact in bf16
    pa[p] = wa;
    pb[p] = wb;
    pc[p] = pk_bf16(s0, s1);
  }
  a = __builtin_bit_cast(bf16x8_t, pa);
  b = __builtin_bit_cast(bf16x8_t, pb);
  c = __builtin_bit_cast(bf16x8_t, pc);
}

// Fill the workgroup's HSplit from the compact Hessian block (row-major
// 32x32 fp32); threads 0..127 each build one (kc, row, half) chunk.
__device__ inline void stage_hsplit(const float* __restrict__ Hg, HSplit* hs) {
  const int t = threadIdx.x;
  if (t < 2 * kG * 2) {
    const int kc = t / (2 * kG), c = (t / 2) % kG, h = t & 1;
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = Hg[c * kG + 16 * kc + 8 * h + j];
    bf16x8_t a, b, d;
    split3x8(x, a, b, d);
    hs->v[0][kc][c][h] = __builtin_bit_cast(u32x4_t, a);
    hs->v[1][kc][c][h] = __builtin_bit_cast(u32x4_t, b);
    hs->v[2][kc][c][h] = __builtin_bit_cast(u32x4_t, d);
  }
}

__device__ inline bf16x8_t h_part(const HSplit* hs, int p, int kc, int lane) {
  return __builtin_bit_cast(bf16x8_t, hs->v[p][kc][lane & 31][lane >> 5]);
}

// (x, y) -> ([x lanes 0-31 | y lanes 0-31], [x lanes 32-63 | y lanes 32-63])
__device__ inline void swap_halves(bf16x8_t& x, bf16x8_t& y) {
  u32x4_t a = __builtin_bit_cast(u32x4_t, x), b = __builtin_bit_cast(u32x4_t, y);
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const auto r = __builtin_amdgcn_permlane32_swap(a[w], b[w], false, false);
    a[w] = r[0];
    b[w] = r[1];
  }
  x = __builtin_bit_cast(bf16x8_t, a);
  y = __builtin_bit_cast(bf16x8_t, b);
}

// obj = sum_c e[c] P[c] from the two accumulator blocks
__device__ inline float objective_from(const float (&e)[kG], const f32x16_t& d0,
                                       const f32x16_t& d1) {
  float obj = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(d0[r]), __float_as_uint(d1[r]),
                                                     false, false);
    const int c0 = 8 * (r >> 2) + (r & 3);
    obj = fmaf(e[c0], __uint_as_float(sw[0]), obj);
    obj = fmaf(e[c0 + 4], __uint_as_float(sw[1]), obj);
  }
  return obj;
}

#define MGQ_MFMA2(A, X, Y)                                          \
  d0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16((A), (X), d0, 0, 0, 0); \
  d1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16((A), (Y), d1, 0, 0, 0)

__device__ inline float mfma_objective(const float (&e)[kG], const HSplit* hs, int lane) {
  f32x16_t d0, d1;
#pragma unroll
  for (int r = 0; r < 16; ++r) d0[r] = d1[r] = 0.0f;
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    bf16x8_t x1, x2, x3, y1, y2, y3;
    split3x8(e + 16 * kc, x1, x2, x3);
    split3x8(e + 16 * kc + 8, y1, y2, y3);
    swap_halves(x1, y1);
    swap_halves(x2, y2);
    swap_halves(x3, y3);
    const bf16x8_t h1 = h_part(hs, 0, kc, lane), h2 = h_part(hs, 1, kc, lane),
                   h3 = h_part(hs, 2, kc, lane);
    // the nonzero products in the order mfma_objective_x1 adds them when
    // e2 = e3 = 0 (h1 e1, h2 e1, h3 e1), so both give the same bits then
    MGQ_MFMA2(h1, x1, y1);
    MGQ_MFMA2(h1, x2, y2);
    MGQ_MFMA2(h2, x1, y1);
    MGQ_MFMA2(h1, x3, y3);
    MGQ_MFMA2(h2, x2, y2);
    MGQ_MFMA2(h3, x1, y1);
    // one K-chunk's split operands live at a time
    __builtin_amdgcn_sched_barrier(0);
  }
  return objective_from(e, d0, d1);
}

// The same objective when every e[c] is exactly a bf16 value (bf16 weights
// and candidate scales whose |w / scale| stays below 512 for MXFP4, 16384
// for MXFP8): E is one exact bf16 operand and only h1 e, h2 e, h3 e remain.
__device__ inline float mfma_objective_x1(const float (&e)[kG], const HSplit* hs, int lane) {
  f32x16_t d0, d1;
#pragma unroll
  for (int r = 0; r < 16; ++r) d0[r] = d1[r] = 0.0f;
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) {
    bf16x8_t x, y;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = static_cast<__bf16>(e[16 * kc + j]);
      y[j] = static_cast<__bf16>(e[16 * kc + 8 + j]);
    }
    swap_halves(x, y);
    MGQ_MFMA2(h_part(hs, 0, kc, lane), x, y);
    MGQ_MFMA2(h_part(hs, 1, kc, lane), x, y);
    MGQ_MFMA2(h_part(hs, 2, kc, lane), x, y);
  }
  return objective_from(e, d0, d1);
}
#undef MGQ_MFMA2

// An opaque zero that depends on `v`: addresses built from it cannot be
// computed before `v`, so the loads behind them are neither hoisted out of
// the loop nor scheduled far ahead of their use (without this the compiler
// lifts the V block out of the recurrence and runs out of registers).
__device__ inline int zero_after(float v) {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z) : "v"(v));
  return z;
}

typedef __attribute__((address_space(3))) float lds_f32;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x4_t lds_f32x4;

// The LDS address p, opaque to the compiler and ordered after `dep`: reads at
// small offsets from it use one base register (their immediate offsets fit),
// and they are not hoisted above the value they wait for.
__device__ inline const lds_f32* lds_after(const lds_f32* p, float dep) {
  uint32_t a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
  asm volatile("; lds_after %1" : "+v"(a) : "v"(dep));
  return reinterpret_cast<const lds_f32*>(static_cast<uintptr_t>(a));
}

// value(code) * scale of the code in byte k of `word` (one code per byte),
// on the hardware decode with the E8M0 scale passed in, which equals the
// decode at scale 1 times the scale bit for bit (k is a constant once the
// callers unroll).
template <int MODE>
__device__ inline float decode_code(uint32_t word, int k, float scale) {
  if constexpr (MODE == kMxfp4) {
    switch (k) {
      case 0: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 0)[0];
      case 1: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 1)[0];
      case 2: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 2)[0];
      default: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 3)[0];
    }
  } else {
    switch (k) {
      case 0: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, scale, false)[0];
      case 1: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, scale, false)[1];
      case 2: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, scale, true)[0];
      default: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, scale, true)[1];
    }
  }
}


__device__ inline float nan_max(float m, float a) { return (a > m || a != a) ? a : m; }

// The 32 weights of one (row, group), 16-byte loads, widened to fp32; for
// 16-bit weights also the loaded words (weights 2k, 2k+1 in word k).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <typename TIn, bool IS_F16>
__device__ inline void load_group(const TIn* __restrict__ W, int64_t base, float (&v)[kG],
                                  uint32_t (&raw)[kG / 2]) {
  if constexpr (sizeof(TIn) == 4) {
    const float4* p = reinterpret_cast<const float4*>(W + base);
#pragma unroll
    for (int i = 0; i < kG / 4; ++i) {
      const float4 x = p[i];
      v[4 * i] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(W + base);
#pragma unroll
    for (int i = 0; i < kG / 8; ++i) {
      const uint4 x = p[i];
      const uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        raw[4 * i + k] = d[k];
        const uint16_t lo = static_cast<uint16_t>(d[k] & 0xffffu);
        const uint16_t hi = static_cast<uint16_t>(d[k] >> 16);
        v[8 * i + 2 * k] = IS_F16 ? f16_to_f32(lo) : bf16_to_f32(lo);
        v[8 * i + 2 * k + 1] = IS_F16 ? f16_to_f32(hi) : bf16_to_f32(hi);
      }
    }
  }
}

// XERR: the candidate errors are exact in bf16 (bf16 weights, offsets within
// the bound the host checks), so their objective uses mfma_objective_x1.
template <typename TIn, bool IS_F16, int MODE, bool SAFE, bool XERR>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 4)))
    mxfp_solve_kernel(const TIn* __restrict__ W, int64_t B, int64_t R, int64_t C,
                      const float* __restrict__ Hc, const float* __restrict__ U,
                      const uint8_t* __restrict__ dead,
                      Offsets offs, uint8_t* __restrict__ q_out, uint8_t* __restrict__ s_out,
                      float* __restrict__ W_dq, double* __restrict__ rel_part,
                      uint32_t* __restrict__ packed_out) {
  static_assert(!XERR || (SAFE && sizeof(TIn) == 2 && !IS_F16), "XERR needs bf16 weights");
  const int64_t G = C / kG;
  const int64_t chunks = (R + kThreads - 1) / kThreads;
  // Work order: the group index is fastest, so the workgroups of groups
  // g, g+1, ... of the same rows are neighbours; and neighbours run on one
  // XCD: physical block p goes to XCD p % 8, so each XCD is given one
  // contiguous range of the work order. Two neighbouring groups share every
  // 128-byte line of W (bf16) and four share every line of q, which are then
  // fetched and written through one L2 instead of two.
  const int64_t n_blocks = static_cast<int64_t>(gridDim.x);
  const int64_t xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  const int64_t per = n_blocks / kXcds, extra = n_blocks % kXcds;
  const int64_t work = xcd * per + (xcd < extra ? xcd : extra) + slot;
  const int64_t g = work % G;
  const int64_t bc = work / G;
  const int64_t b = bc / chunks, chunk = bc % chunks;
  const int64_t r_raw = chunk * kThreads + threadIdx.x;
  const bool valid = r_raw < R;
  const int64_t r = valid ? r_raw : R - 1;

  // compact (post dead-column fix) Hessian block, written by hinv32
  const float* __restrict__ Hg = Hc + (b * G + g) * kG * kG;
  const int lane = threadIdx.x & 63;
  // V^T staged in LDS (Ut[c][k] = V[k][c] = U[k][c] * RN(1/U[k][k]); the
  // recurrence reads the entries k < c): one column of V per step with
  // broadcast LDS loads (uniform addresses).
  __shared__ float Ut[kG * kG];
  // RN(1/U[k][k]), or 0 where U[k][k] is outside [2^-24, 2^24]
  __shared__ float ydiag[kG];
  // the safe search's objective operand: Hg as three exact bf16 parts
  HSplit* hs = nullptr;
  if constexpr (SAFE) {
    __shared__ HSplit hsplit_s;
    hs = &hsplit_s;
  }
  {
    const float* Ub = U + (b * G + g) * kG * kG;
    if (threadIdx.x < kG) ydiag[threadIdx.x] = div_exact_recip(Ub[threadIdx.x * (kG + 1)]);
    if constexpr (SAFE) stage_hsplit(Hg, hs);
    __syncthreads();
    // V = U[k][c] * RN(1/U[k][k]); a divisor outside [2^-24, 2^24] divides
    constexpr int kPer = kG * kG / kThreads;
    float u[kPer], y[kPer];
    bool any_div = false;
#pragma unroll
    for (int i = 0; i < kPer; ++i) u[i] = Ub[threadIdx.x + i * kThreads];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      y[i] = ydiag[(threadIdx.x + i * kThreads) / kG];
      any_div |= y[i] == 0.0f;
    }
    if (any_div) {
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int k = (threadIdx.x + i * kThreads) / kG;
        if (y[i] == 0.0f) u[i] = u[i] / Ub[k * (kG + 1)];
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = threadIdx.x + i * kThreads;
      Ut[(e % kG) * kG + e / kG] = y[i] == 0.0f ? u[i] : u[i] * y[i];
    }
  }
  __syncthreads();
  const uint8_t* __restrict__ dd = dead + b * C + g * kG;
  const int64_t base = (b * R + r) * C + g * kG;
  const float fmax = (MODE == kMxfp4) ? 6.0f : 448.0f;

  // The group's 32 (dead-column-fixed) weights live in LDS as fp32, not in
  // registers, which leaves room for 4 waves per SIMD without spills.
  // Weights 2p and 2p+1 of thread t sit side by side at
  // so[p * 2 kThreads + 2t], so a pair is one 8-byte read and both pair and
  // single reads are conflict-free.
  __shared__ float so[kG * kThreads];
  float amax;
  // rel_err partials (gptq.py:300-302) against the caller's W as given:
  // den = sum w^2 and, for dead columns (whose W_dq is 0), their w^2.
  float den = 0.0f, dead_sq = 0.0f;
  {
    float v[kG];
    uint32_t raw[kG / 2];
    load_group<TIn, IS_F16>(W, base, v, raw);
    // dead columns (gptq.py:219-221) read as 0
    const uint4 m0 = reinterpret_cast<const uint4*>(dd)[0];
    const uint4 m1 = reinterpret_cast<const uint4*>(dd)[1];
    const uint32_t mw[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    const bool any_dead = (m0.x | m0.y | m0.z | m0.w | m1.x | m1.y | m1.z | m1.w) != 0u;  // uniform
    if (rel_part) {
      if constexpr (sizeof(TIn) == 2 && !IS_F16) {
        // bf16 pairs: both exact products and their sum in one instruction
#pragma unroll
        for (int k = 0; k < kG / 2; ++k) {
          const bf16x2_t x = __builtin_bit_cast(bf16x2_t, raw[k]);
          den = __builtin_amdgcn_fdot2_f32_bf16(x, x, den, false);
        }
      } else {
#pragma unroll
        for (int i = 0; i < kG; ++i) den = fmaf(v[i], v[i], den);
      }
      if (any_dead) {
#pragma unroll
        for (int i = 0; i < kG; ++i)
          if ((mw[i / 4] >> (8 * (i % 4))) & 0xffu) dead_sq = fmaf(v[i], v[i], dead_sq);
      }
    }
    if (any_dead) {
#pragma unroll
      for (int i = 0; i < kG; ++i)
        if ((mw[i / 4] >> (8 * (i % 4))) & 0xffu) v[i] = 0.0f;
    }
    // amax = max |v|, NaN when any v is NaN (grid.py's amax propagates it;
    // which NaN does not matter: e8m0_exponent and the range guard only
    // test for one): IEEE maximum propagates NaN, three operands at a time.
    amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kG; i += 2)
      amax = __builtin_elementwise_maximum(
          amax, __builtin_elementwise_maximum(fabsf(v[i]), fabsf(v[i + 1])));
#pragma unroll
    for (int p = 0; p < kG / 2; ++p)
      *reinterpret_cast<float2*>(so + p * 2 * kThreads + 2 * threadIdx.x) = make_float2(v[2 * p], v[2 * p + 1]);
  }
  const float* orig = so + 2 * threadIdx.x;
  // weights 2p and 2p+1
  auto orig_pair = [](const float* o, int p, float& a, float& c) __attribute__((always_inline)) {
    const float2 x = *reinterpret_cast<const float2*>(o + p * 2 * kThreads);
    a = x.x;
    c = x.y;
  };
  auto orig_at = [](const float* o, int i) __attribute__((always_inline)) -> float {
    return o[(i / 2) * 2 * kThreads + (i & 1)];
  };
#define ORIG(i) orig_at(orig, (i))
  // The selected result's codes, one per byte (codes[i / 4] byte i % 4),
  // kept in registers until the final store. The safe search, whose
  // candidate objectives need the registers, reads its dequantized values
  // back from them: value(code) * scale on the hardware decode, the same
  // product the encoder returned. The groupwise solve keeps them in
  // registers as they come.
  uint32_t codes[kG / 4];
  float dqr[SAFE ? 1 : kG];
  float dq_scale = 0.0f;  // the selected scale, set before the first read
  auto dq_get = [&](int i) __attribute__((always_inline)) -> float {
    if constexpr (!SAFE)
      return dqr[i];
    else
      return decode_code<MODE>(codes[i / 4], i % 4, dq_scale);
  };
  auto dq_set = [&](int i, float v) __attribute__((always_inline)) {
    if constexpr (!SAFE) dqr[i] = v;
  };
#define DQ(i) dq_get(i)

  // 1. scale choice
  const int e0 = e8m0_exponent(amax, fmax);
  int e_sel = e0;
  // Objectives are computed on errors in units of the candidate's scale and
  // multiplied by 2^(2 (e - e0)), which is exact: the comparisons are those
  // of the scaled objectives, without scaling every error.
  float best = 0.0f;
  if (SAFE) {
    float err[kG];
    for (int o = 0; o < offs.n; ++o) {
      int e = e0 + offs.v[o];
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      const float inv = exp2_int(-e), sc = exp2_int(e);
      const float lim = (MODE == kMxfp8) ? mx8_clamp_limit(sc) : 0.0f;
      // re-read the weights from LDS per candidate (an opaque offset keeps
      // the compiler from holding all 32 in registers across the loop)
      const float* og = orig + zero_after(inv);
      // four pairs at a time: the scheduler would otherwise run each op
      // over all 32 elements before the next and hold 4 x 32 temporaries
#pragma unroll
      for (int p0 = 0; p0 < kG / 2; p0 += 4) {
        float x[8];
#pragma unroll
        for (int p = 0; p < 4; ++p) orig_pair(og, p0 + p, x[2 * p], x[2 * p + 1]);
        quant_err8<MODE>(x, sc, inv, lim, err + 2 * p0);
        __builtin_amdgcn_sched_barrier(0);
      }
      const float raw = XERR ? mfma_objective_x1(err, hs, lane) : mfma_objective(err, hs, lane);
      const float obj = __builtin_amdgcn_ldexpf(raw, 2 * (e - e0));
      if (o == 0 || obj < best) {
        best = obj;
        e_sel = e;
      }
    }
  }
  const float scale = exp2_int(e_sel), inv_scale = exp2_int(-e_sel);
  dq_scale = scale;

  // 2. GPTQ recurrence with the fixed scale, column by column. The
  // reference updates all later columns after each step
  // (W[c+1:] -= err_c * U[c, c+1:], err_c = (w_c - dq_c) / U[c,c]); each
  // element therefore sees w_c = ((orig_c - err_0 U[0,c]) - err_1 U[1,c]) -
  // ... in that order. Forming w_c lazily keeps that order while keeping
  // only one value per column live: the numerator a_k = w_k - dq_k, with the
  // division moved onto the factor, err_k U[k,c] = a_k V[k,c] (V staged
  // above, each entry rounded once). Each step is one fused multiply-add,
  // where the reference rounds err_k, then err_k U[k,c], then the
  // difference: the terms agree to an ulp or two, and so do the codes on
  // practically every element.
  //
  // The fast pass (EXACT = false) encodes without the NaN patch; a NaN w_c
  // reaches the last numerator through every later column (NaN times V is
  // NaN, zero entries included), which sends the wave to the exact pass. A
  // zero numerator may come out as a zero of either sign, which no output
  // can see: numerators only feed the later columns' sums, and a zero sum of
  // either sign encodes to code 0 and decodes to +0.
  float errs[kG];
  auto recurrence = [&](auto exact_tag) __attribute__((always_inline)) -> bool {
    constexpr bool EXACT = decltype(exact_tag)::value;
#pragma unroll
    for (int i = 0; i < kG / 4; ++i) codes[i] = 0u;
    // Ut's base, passed from column to column through lds_after so that its
    // register is updated in place (no copy per column) and every column's
    // reads take immediate offsets from it
    const lds_f32* ubase = (const lds_f32*)Ut;
#pragma unroll
    for (int c = 0; c < kG; ++c) {
      // column c of V (row c of Ut, 16-byte aligned), read 4 values at a time
      if (c) ubase = lds_after(ubase, errs[c - 1]);
      const lds_f32* col = ubase + c * kG;
      float acc = ORIG(c);
#pragma unroll
      for (int k0 = 0; k0 < c; k0 += 4) {
        const f32x4_t u4 = *reinterpret_cast<const lds_f32x4*>(col + k0);
#pragma unroll
        for (int k = k0; k < c && k < k0 + 4; ++k) acc = fmaf(-errs[k], u4[k - k0], acc);
      }
      float dq;
      uint32_t code = 0u;
      if constexpr (MODE == kMxfp4 && !EXACT)
        dq = mx4_encode_into(codes[c / 4], c % 4, acc, inv_scale, scale);
      else
        code = quant_exact<MODE, !EXACT>(acc, inv_scale, scale, &dq);
      errs[c] = acc - dq;
      if constexpr (!(MODE == kMxfp4 && !EXACT)) codes[c / 4] |= code << (8 * (c % 4));
      dq_set(c, dq);
    }
    return errs[kG - 1] != errs[kG - 1];
  };
  if (__builtin_amdgcn_ballot_w64(recurrence(std::false_type{})) != 0)
    recurrence(std::true_type{});

  // 4's test first: the range guard on the GPTQ result, every |dq| <= limit;
  // and (safe search) the result's errors for step 3, from the same decode.
  // The dequantized values are not kept through the objective (they are
  // decoded again below), which keeps the objective's registers in budget.
  float limit = amax * 32.0f;
  const float floor_ = __uint_as_float(0x00800000u);  // 2^-126
  limit = (limit != limit) ? limit : fmaxf(limit, floor_);
  bool in_range = true;
  float err[SAFE ? kG : 1];
  if constexpr (SAFE) {
    // in units of the scale: the decode at scale 1 is dq / 2^e exactly, so
    // |dq| <= limit is |value| <= limit * 2^-e (exact: the product stays
    // normal or becomes inf for every reachable (amax, e)), and
    // err = (dq - w) * 2^-e = value - w * 2^-e, one fused multiply-add with
    // the same rounding as the difference scaled afterwards
    const float limit_u = limit * inv_scale;
#pragma unroll
    for (int i0 = 0; i0 < kG; i0 += 8) {
#pragma unroll
      for (int i = i0; i < i0 + 8; ++i) {
        const float v = decode_code<MODE>(codes[i / 4], i % 4, 1.0f);
        in_range = in_range & (fabsf(v) <= limit_u);  // no short-circuit branches
        err[i] = fmaf(ORIG(i), -inv_scale, v);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kG; ++i) in_range = in_range & (fabsf(DQ(i)) <= limit);
  }
  // 3. GPTQ vs best RTN candidate (safe search only)
  bool use_gptq = true;
  if constexpr (SAFE)
    use_gptq = __builtin_amdgcn_ldexpf(mfma_objective(err, hs, lane), 2 * (e_sel - e0)) <= best;
  const bool ok = use_gptq & in_range;
  if constexpr (SAFE) {
    // opaque to the compiler, so that the values are decoded again here
    // rather than kept from the loop above
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < kG / 4; ++i) asm volatile("" : "+v"(codes[i]));
  }
  float w[kG];
#pragma unroll
  for (int i = 0; i < kG; ++i) w[i] = DQ(i);
  if (!ok) {  // RTN baseline at the chosen scale
    // A NaN weight is the only input that the NaN-free encode gets wrong (its
    // n = w * inv_scale is NaN exactly when w is), and amax is NaN exactly
    // when a weight is: without one among this wave's fallback lanes, MXFP4
    // takes the encode that writes each code straight into its byte.
    if (MODE == kMxfp4 && __builtin_amdgcn_ballot_w64(amax != amax) == 0) {
#pragma unroll
      for (int i = 0; i < kG; ++i)
        w[i] = mx4_encode_into(codes[i / 4], i % 4, ORIG(i), inv_scale, scale);
    } else {
#pragma unroll
      for (int i = 0; i < kG / 4; ++i) codes[i] = 0u;
#pragma unroll
      for (int i = 0; i < kG; ++i) {
        float dq;
        const uint32_t code = quant_exact<MODE>(ORIG(i), inv_scale, scale, &dq);
        codes[i / 4] |= code << (8 * (i % 4));
        w[i] = dq;
      }
    }
  }

  double num = 0.0, den_d = 0.0;
  if (valid) {
    uint4* qp = reinterpret_cast<uint4*>(q_out + base);
    qp[0] = make_uint4(codes[0], codes[1], codes[2], codes[3]);
    qp[1] = make_uint4(codes[4], codes[5], codes[6], codes[7]);
    if (packed_out != nullptr) {
      // the codes in MLX's uint32 layout (packing.py:15-26: value j of a
      // word at bits width * j, LSB first): MXFP4 packs the 32 codes of the
      // group into words 4g..4g+3 of the row, MXFP8's words are its code
      // bytes as they are
      if constexpr (MODE == kMxfp4) {
        uint32_t pw[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // byte 0 of t = codes 0 | 1 << 4, byte 2 = codes 2 | 3 << 4
          const uint32_t t0 = codes[2 * p] | (codes[2 * p] >> 4);
          const uint32_t t1 = codes[2 * p + 1] | (codes[2 * p + 1] >> 4);
          pw[p] = __builtin_amdgcn_perm(t1, t0, 0x06040200u);
        }
        *reinterpret_cast<uint4*>(packed_out + (b * R + r) * (C / 8) + g * 4) =
            make_uint4(pw[0], pw[1], pw[2], pw[3]);
      } else {
        uint4* pp = reinterpret_cast<uint4*>(packed_out + (b * R + r) * (C / 4) + g * 8);
        pp[0] = make_uint4(codes[0], codes[1], codes[2], codes[3]);
        pp[1] = make_uint4(codes[4], codes[5], codes[6], codes[7]);
      }
    }
    float4* op = reinterpret_cast<float4*>(W_dq + base);
#pragma unroll
    for (int i = 0; i < kG / 4; ++i)
      op[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    s_out[(b * R + r) * G + g] = static_cast<uint8_t>(e_sel + 127);
    if (rel_part) {
      // live columns: (W_dq - w)^2 from the LDS copy (dead columns hold 0
      // there and in W_dq; their w^2 is dead_sq)
      float sq = dead_sq;
#pragma unroll
      for (int i = 0; i < kG; ++i) {
        const float d = w[i] - ORIG(i);
        sq = fmaf(d, d, sq);
      }
      num = sq;
      den_d = den;
    }
  }
  if (rel_part) {
    // wave reduction, one (num, den) pair per wave
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      num += __shfl_xor(num, off);
      den_d += __shfl_xor(den_d, off);
    }
    if ((threadIdx.x & 63) == 0) {
      const int64_t waves = (R + 63) / 64;
      const int64_t wv = chunk * (kThreads / 64) + (threadIdx.x >> 6);
      if (wv < waves) {
        double* pp = rel_part + ((b * G + g) * waves + wv) * 2;
        pp[0] = num;
        pp[1] = den_d;
      }
    }
  }
}

#undef ORIG
#undef DQ

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

// Partial sums of gptq.py:300-302's rel_err for the affine path: block
// (c, b) adds (W_dq - W)^2 and W^2 (in double) over elements
// [c * chunk, (c + 1) * chunk) of item b, reduced in a fixed order, into
// part[(b * nb + c) * 2 + {0, 1}] for rel_err_kernel. W is f32, bf16 or f16.
template <typename TIn, bool IS_F16>
__global__ void __launch_bounds__(256) rel_part_kernel(const float* __restrict__ W_dq,
                                                       const TIn* __restrict__ W, int64_t n,
                                                       int64_t chunk, double* __restrict__ part) {
  const int64_t b = blockIdx.y, c = blockIdx.x;
  const int64_t lo = c * chunk, hi = (lo + chunk < n) ? lo + chunk : n;
  const float* dq = W_dq + b * n;
  const TIn* w = W + b * n;
  double num = 0.0, den = 0.0;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    float x;
    if constexpr (sizeof(TIn) == 4)
      x = w[i];
    else
      x = IS_F16 ? f16_to_f32(w[i]) : bf16_to_f32(w[i]);
    const float d = dq[i] - x;
    num += static_cast<double>(d) * d;
    den += static_cast<double>(x) * x;
  }
  __shared__ double sn[256], sd[256];
  sn[threadIdx.x] = num;
  sd[threadIdx.x] = den;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (threadIdx.x < st) {
      sn[threadIdx.x] += sn[threadIdx.x + st];
      sd[threadIdx.x] += sd[threadIdx.x + st];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part[(b * gridDim.x + c) * 2] = sn[0];
    part[(b * gridDim.x + c) * 2 + 1] = sd[0];
  }
}

struct WsLayout {
  int64_t dead_off, u_off, hc_off, rel_off, total;
};

WsLayout ws_layout(int64_t B, int64_t R, int64_t C) {
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t G = C / kG;
  WsLayout L;
  L.dead_off = 0;
  L.u_off = al(B * C);
  L.hc_off = L.u_off + al(B * G * kG * kG * 4);
  L.rel_off = L.hc_off + al(B * G * kG * kG * 4);
  L.total = L.rel_off + al(B * G * ((R + 63) / 64) * 2 * 8);
  return L;
}

template <typename TIn, bool IS_F16, bool XERR>
int launch_solve(const void* W, int64_t B, int64_t R, int64_t C, const float* Hc, const float* U,
                 const uint8_t* dead, int mode, bool safe, const Offsets& offs, uint8_t* q,
                 uint8_t* s, float* W_dq, double* rel_part, uint32_t* packed, hipStream_t st) {
  const int64_t G = C / kG;
  const int64_t blocks = B * G * ((R + kThreads - 1) / kThreads);
  const TIn* w = static_cast<const TIn*>(W);
#define MGQ_LAUNCH(MODE, SAFE, X)                                                                    \
  mxfp_solve_kernel<TIn, IS_F16, MODE, SAFE, X><<<static_cast<unsigned>(blocks), kThreads, 0, st>>>( \
      w, B, R, C, Hc, U, dead, offs, q, s, W_dq, rel_part, packed)
  if constexpr (XERR) {
    if (mode == kMxfp4) MGQ_LAUNCH(kMxfp4, true, true); else MGQ_LAUNCH(kMxfp8, true, true);
  } else if (mode == kMxfp4) {
    if (safe) MGQ_LAUNCH(kMxfp4, true, false); else MGQ_LAUNCH(kMxfp4, false, false);
  } else {
    if (safe) MGQ_LAUNCH(kMxfp8, true, false); else MGQ_LAUNCH(kMxfp8, false, false);
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

extern "C" int mgq_gptq_mxfp_prepare(float* H, int64_t B, int64_t R, int64_t C, float damp,
                                     int max_attempts, int32_t* attempts, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  clear_error();
  MGQ_REQUIRE(B >= 0 && R >= 0 && C >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(C % kG == 0, MGQ_ERR_SHAPE, "in_features %lld not divisible by group %d",
              (long long)C, kG);
  MGQ_REQUIRE(max_attempts >= 1, MGQ_ERR_VALUE, "max_attempts must be >= 1");
  const WsLayout L = ws_layout(B, R, C);
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MGQ_ERR_WORKSPACE,
              "mxfp workspace %lld < %lld bytes", (long long)workspace_bytes,
              (long long)L.total);
  MGQ_REQUIRE((reinterpret_cast<uintptr_t>(H) & 15u) == 0, MGQ_ERR_SHAPE,
              "H must be 16-byte aligned");
  if (B == 0 || C == 0) return MGQ_OK;
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  uint8_t* dead = reinterpret_cast<uint8_t*>(ws + L.dead_off);
  float* U = reinterpret_cast<float*>(ws + L.u_off);
  float* Hcmp = reinterpret_cast<float*>(ws + L.hc_off);
  // the dead-column fix (gptq.py:216-222: diag(H) <= 0 marks a dead column,
  // its diagonal becomes 1 in place, its weights are treated as 0) runs in
  // the same launch, each 32x32 block fixing its own diagonal first
  return launch_hinv32(H, B, C, damp, max_attempts, U, attempts, Hcmp, dead, st);
}

namespace mgq {
namespace {

// mgq_gptq_mxfp_solve, and with packed_out != nullptr also the codes packed
// as pack_q (packing.py:15-26) packs them, by the solver itself.
int solve_entry(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C, int mode,
                int algorithm, const int32_t* offsets, int n_offsets, uint8_t* q_out,
                uint32_t* packed_out, uint8_t* scales_out, float* W_dq, float* rel_err,
                void* workspace, int64_t workspace_bytes, void* stream) {
  MGQ_REQUIRE(mode == kMxfp4 || mode == kMxfp8, MGQ_ERR_VALUE, "not a microscaling mode: %d",
              mode);
  MGQ_REQUIRE(algorithm == 0 || algorithm == 1, MGQ_ERR_VALUE,
              "unsupported MXFP GPTQ algorithm code: %d", algorithm);
  MGQ_REQUIRE(w_dtype == kF32 || w_dtype == kBF16 || w_dtype == kF16, MGQ_ERR_VALUE,
              "unsupported weight dtype code %d", w_dtype);
  MGQ_REQUIRE(B >= 0 && R >= 0 && C >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(C % kG == 0, MGQ_ERR_SHAPE, "in_features %lld not divisible by group %d",
              (long long)C, kG);
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
  MGQ_REQUIRE(rel_err == nullptr || static_cast<const void*>(W_dq) != W, MGQ_ERR_VALUE,
              "rel_err needs W_dq separate from W (in-place solves skip rel_err)");
  MGQ_REQUIRE((reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(W_dq) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(q_out) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(packed_out) & 15u) == 0,
              MGQ_ERR_SHAPE, "W, W_dq, q_out and packed_out must be 16-byte aligned");
  if (B == 0 || C == 0 || R == 0) return MGQ_OK;
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  const uint8_t* dead = reinterpret_cast<const uint8_t*>(ws + L.dead_off);
  const float* U = reinterpret_cast<const float*>(ws + L.u_off);
  const float* Hcmp = reinterpret_cast<const float*>(ws + L.hc_off);
  double* rel_part = reinterpret_cast<double*>(ws + L.rel_off);
  // Candidate errors are exact in bf16 for bf16 weights while every
  // |w / scale| stays below 512 (MXFP4) or 16384 (MXFP8): with e0 the
  // groupwise exponent, |w / 2^(e0+off)| <= fmax * 2^(0.5 - off), so offsets
  // >= -5 (MXFP4) or >= -4 (MXFP8) keep it there.
  int min_off = 0;
  for (int i = 0; i < offs.n; ++i) min_off = offs.v[i] < min_off ? offs.v[i] : min_off;
  const bool xerr = algorithm == 1 && w_dtype == kBF16 && min_off >= (mode == kMxfp4 ? -5 : -4);
  int rc;
  double* rp = rel_err ? rel_part : nullptr;
  if (w_dtype == kF32) {
    rc = launch_solve<float, false, false>(W, B, R, C, Hcmp, U, dead, mode, algorithm == 1, offs,
                                           q_out, scales_out, W_dq, rp, packed_out, st);
  } else if (w_dtype == kBF16 && xerr) {
    rc = launch_solve<uint16_t, false, true>(W, B, R, C, Hcmp, U, dead, mode, true, offs, q_out,
                                             scales_out, W_dq, rp, packed_out, st);
  } else if (w_dtype == kBF16) {
    rc = launch_solve<uint16_t, false, false>(W, B, R, C, Hcmp, U, dead, mode, algorithm == 1,
                                              offs, q_out, scales_out, W_dq, rp, packed_out, st);
  } else {
    rc = launch_solve<uint16_t, true, false>(W, B, R, C, Hcmp, U, dead, mode, algorithm == 1,
                                             offs, q_out, scales_out, W_dq, rp, packed_out, st);
  }
  if (rc) return rc;
  if (rel_err) {
    const int64_t n_per_b = (C / kG) * ((R + 63) / 64);
    rel_err_kernel<<<static_cast<unsigned>(B), 256, 0, st>>>(rel_part, n_per_b, B, rel_err);
    if (int rc2 = check_launch("rel_err")) return rc2;
  }
  return MGQ_OK;
}

}  // namespace
}  // namespace mgq

extern "C" int mgq_gptq_mxfp_solve(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C,
                                   int mode, int algorithm, const int32_t* offsets, int n_offsets,
                                   uint8_t* q_out, uint8_t* scales_out, float* W_dq,
                                   float* rel_err, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  clear_error();
  return solve_entry(W, w_dtype, B, R, C, mode, algorithm, offsets, n_offsets, q_out, nullptr,
                     scales_out, W_dq, rel_err, workspace, workspace_bytes, stream);
}

extern "C" int mgq_gptq_mxfp_solve_packed(const void* W, int w_dtype, int64_t B, int64_t R,
                                          int64_t C, int mode, int algorithm,
                                          const int32_t* offsets, int n_offsets, uint8_t* q_out,
                                          uint32_t* packed_out, uint8_t* scales_out, float* W_dq,
                                          float* rel_err, void* workspace,
                                          int64_t workspace_bytes, void* stream) {
  clear_error();
  MGQ_REQUIRE(packed_out != nullptr, MGQ_ERR_VALUE, "packed_out required");
  return solve_entry(W, w_dtype, B, R, C, mode, algorithm, offsets, n_offsets, q_out, packed_out,
                     scales_out, W_dq, rel_err, workspace, workspace_bytes, stream);
}

extern "C" int mgq_rel_err(const float* W_dq, const void* W, int w_dtype, int64_t B, int64_t n,
                           double* partials, int64_t n_partials, float* rel, void* stream) {
  clear_error();
  MGQ_REQUIRE(w_dtype == kF32 || w_dtype == kBF16 || w_dtype == kF16, MGQ_ERR_VALUE,
              "unsupported weight dtype code %d", w_dtype);
  MGQ_REQUIRE(B >= 0 && n >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(n_partials >= 1 && n_partials <= 65535, MGQ_ERR_VALUE,
              "n_partials %lld outside 1..65535", (long long)n_partials);
  if (B == 0) return MGQ_OK;
  MGQ_REQUIRE(B <= 65535, MGQ_ERR_SHAPE, "rel_err: batch %lld exceeds 65535", (long long)B);
  MGQ_REQUIRE(W_dq != nullptr && W != nullptr && partials != nullptr && rel != nullptr,
              MGQ_ERR_VALUE, "rel_err: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t chunk = (n + n_partials - 1) / n_partials;
  const dim3 grid(static_cast<unsigned>(n_partials), static_cast<unsigned>(B));
  if (w_dtype == kF32)
    rel_part_kernel<float, false><<<grid, 256, 0, st>>>(W_dq, static_cast<const float*>(W), n,
                                                        chunk, partials);
  else if (w_dtype == kBF16)
    rel_part_kernel<uint16_t, false><<<grid, 256, 0, st>>>(
        W_dq, static_cast<const uint16_t*>(W), n, chunk, partials);
  else
    rel_part_kernel<uint16_t, true><<<grid, 256, 0, st>>>(
        W_dq, static_cast<const uint16_t*>(W), n, chunk, partials);
  if (int rc = check_launch("rel_err partials")) return rc;
  rel_err_kernel<<<static_cast<unsigned>(B), 256, 0, st>>>(partials, n_partials, B, rel);
  return check_launch("rel_err");
}

extern "C" int mgq_gptq_mxfp(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C,
                             float* H, int mode, int algorithm, float damp, int max_attempts,
                             const int32_t* offsets, int n_offsets, uint8_t* q_out,
                             uint8_t* scales_out, float* W_dq, float* rel_err,
                             int32_t* attempts, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  clear_error();
  // argument checks of both halves before anything is launched
  MGQ_REQUIRE(mode == kMxfp4 || mode == kMxfp8, MGQ_ERR_VALUE, "not a microscaling mode: %d",
              mode);
  MGQ_REQUIRE(algorithm == 0 || algorithm == 1, MGQ_ERR_VALUE,
              "unsupported MXFP GPTQ algorithm code: %d", algorithm);
  MGQ_REQUIRE(w_dtype == kF32 || w_dtype == kBF16 || w_dtype == kF16, MGQ_ERR_VALUE,
              "unsupported weight dtype code %d", w_dtype);
  MGQ_REQUIRE(algorithm == 0 || (offsets != nullptr && n_offsets >= 1 && n_offsets <= kMaxOffsets),
              MGQ_ERR_VALUE, "safe-scale-search needs 1..%d exponent offsets", kMaxOffsets);
  MGQ_REQUIRE(rel_err == nullptr || static_cast<const void*>(W_dq) != W, MGQ_ERR_VALUE,
              "rel_err needs W_dq separate from W (in-place solves skip rel_err)");
  MGQ_REQUIRE((reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(W_dq) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(q_out) & 15u) == 0,
              MGQ_ERR_SHAPE, "W, W_dq and q_out must be 16-byte aligned");
  if (int rc = mgq_gptq_mxfp_prepare(H, B, R, C, damp, max_attempts, attempts, workspace,
                                     workspace_bytes, stream))
    return rc;
  return mgq_gptq_mxfp_solve(W, w_dtype, B, R, C, mode, algorithm, offsets, n_offsets, q_out,
                             scales_out, W_dq, rel_err, workspace, workspace_bytes, stream);
}
