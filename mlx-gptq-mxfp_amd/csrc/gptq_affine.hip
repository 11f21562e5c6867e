// Affine (MLX scale/bias) GPTQ: the lazy-block column loop of
// gptq.py:229-272 with the MSE clip search of grid.py:167-212.
//
// One wavefront owns one (batch item, row). For each block of `bs` columns
// (a multiple of the group size G) and each G-column group in it:
//   - lane t holds column j+t (and j+t+64 for G = 128); at the group start
//     the lane applies the earlier in-block updates
//         w <- w - err_k * U[k, col]   for k = block start .. j-1, in order,
//     which are exactly the element's updates in the reference's order;
//   - the clip search runs on those G values across lanes (wave min/max and
//     wave sums of squared errors, strict '<' over the shrink candidates);
//   - the G columns are then quantized one by one; the owner lane's error
//     err = (w - dq) / U[c, c] is broadcast and every later column applies
//     w <- w - err * U[c, col].
// After the block a separate kernel applies the deferred update
//     W[:, i2:] -= Err @ U[i1:i2, i2:]
// (the reference's bmm) as an fp32 GEMM.
#include <type_traits>

#include "mgq_capi.h"
#include "mgq_common.h"
#include "mx_hw.h"

namespace mgq {
namespace {

constexpr int kWaves = 4;
constexpr int kMaxBlock = 2048;  // errs of one block per wave in LDS: 32 KB
constexpr int kMaxShrinks = 128;
constexpr int kCand = 12;  // clip candidates scored per butterfly

struct Shrinks {
  int n;
  float p_over_maxq[kMaxShrinks];
  float p[kMaxShrinks];
};

__device__ inline float nan_max(float m, float a) { return (a > m || a != a) ? a : m; }
__device__ inline float nan_min(float m, float a) { return (a < m || a != a) ? a : m; }

// ---- cross-lane steps without LDS traffic --------------------------------
// A butterfly over the xor masks 32, 16, 8, 4, 2, 1 (in that order). xor 32
// and xor 16 go through gfx950's v_permlane32_swap / v_permlane16_swap: with
// both operands v, the swap leaves ([lo | lo], [hi | hi]) for 32 and (rows
// [r0 r0 r2 r2], [r1 r1 r3 r3]) for 16, so a lane's partner is one of the two
// results. xor 8 is a DPP rotation by 8 inside each 16-lane row. xor 2 and
// xor 1 are DPP quad permutations.
template <int CTRL>
__device__ inline float dpp_read(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppXor2 = 0x4e, kDppXor1 = 0xb1;

__device__ inline float2 swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ inline float2 swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// N wave sums (N a multiple of 4), each rounded like an xor butterfly with
// __shfl_xor (v <- v + partner for xor 32, 16, 8, 4, 2, 1), by recursive
// halving. The xor-32 step swaps v[i] with v[i + N/2], so lanes 0-31 keep
// sum i and lanes 32-63 sum i + N/2, both as lo + hi; the xor-16 step pairs
// those results the same way (row 2k + row 2k+1); the DPP steps then run on
// N/4 values. Because a + b == b + a bit for bit, after the 8 step a lane's
// value depends only on lane mod 8, so a rotation by 4 reads the value of
// lane ^ 4. Sum i + (N/4) r ends in u[i] of the lanes of row r (lanes 16r ..
// 16r + 15).
template <int N>
__device__ inline void wave_sum_halving(const float (&v)[N], float (&u)[N / 4]) {
  static_assert(N % 4 == 0, "N must be a multiple of 4");
  float w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]),
                                                    __float_as_uint(v[i + N / 2]), false, false);
    w[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[i]),
                                                    __float_as_uint(w[i + N / 4]), false, false);
    u[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) u[i] += dpp_read<kDppRor8>(u[i]);
#pragma unroll
  for (int i = 0; i < N / 4; ++i) u[i] += dpp_read<kDppRor4>(u[i]);
#pragma unroll
  for (int i = 0; i < N / 4; ++i) u[i] += dpp_read<kDppXor2>(u[i]);
#pragma unroll
  for (int i = 0; i < N / 4; ++i) u[i] += dpp_read<kDppXor1>(u[i]);
}

// wave_nan_min and wave_nan_max of two values in one xor butterfly, each
// lane applying f(own, partner). nan_min / nan_max are not symmetric in the
// sign of a zero, so every step reads the exact xor partner (xor 4 through
// __shfl_xor).
__device__ inline void wave_nan_minmax(float& lo, float& hi, int lane) {
  const bool lo32 = lane < 32, even16 = (lane & 16) == 0;
  {
    const float2 a = swap32(lo), b = swap32(hi);
    lo = nan_min(lo, lo32 ? a.y : a.x);
    hi = nan_max(hi, lo32 ? b.y : b.x);
  }
  {
    const float2 a = swap16(lo), b = swap16(hi);
    lo = nan_min(lo, even16 ? a.y : a.x);
    hi = nan_max(hi, even16 ? b.y : b.x);
  }
  {
    const float a = dpp_read<kDppRor8>(lo), b = dpp_read<kDppRor8>(hi);
    lo = nan_min(lo, a);
    hi = nan_max(hi, b);
  }
  {
    const float a = __shfl_xor(lo, 4), b = __shfl_xor(hi, 4);
    lo = nan_min(lo, a);
    hi = nan_max(hi, b);
  }
  {
    const float a = dpp_read<kDppXor2>(lo), b = dpp_read<kDppXor2>(hi);
    lo = nan_min(lo, a);
    hi = nan_max(hi, b);
  }
  {
    const float a = dpp_read<kDppXor1>(lo), b = dpp_read<kDppXor1>(hi);
    lo = nan_min(lo, a);
    hi = nan_max(hi, b);
  }
}

// ---- exact division by a positive divisor ----------------------------------
// a / d for d > 0 (or NaN), correctly rounded: Markstein's correction from
// y = div_exact_recip(d) (mx_hw.h); a zero numerator is returned as is (a / d
// keeps its sign for d > 0); outside the correction's range the IEEE
// division. Every divisor here is positive: the clip scale (range >= 0) and
// U's diagonal. div_fast is the correction, div_slow says when it is not
// exact (the operators are the non-short-circuit ones so that no branch is
// formed around the test).
__device__ inline float div_fast(float a, float d, float y) {
  const float q = a * y;
  const float r = fmaf(-q, d, a);
  return fmaf(r, y, q);
}
__device__ inline bool div_slow(float a, float y) {
  const uint32_t ea = f2u(a) & 0x7f800000u;
  return (a != 0.0f) & ((!(y != 0.0f)) | ((ea - (27u << 23)) > (200u << 23)));
}

__device__ inline float div_pos(float a, float d, float y) {
  float e = div_fast(a, d, y);
  const bool slow = div_slow(a, y);
  // the IEEE division only when some lane needs it: a wave-uniform branch
  // (the empty asm keeps the compiler from hoisting the division out of it)
  if (__builtin_amdgcn_ballot_w64(slow) != 0) {
    asm volatile("" ::: "memory");
    const float ref = a / d;
    e = slow ? ref : e;
  }
  return a == 0.0f ? a : e;
}

// grid.py:215-221 from a quotient (w - b) / s_safe: q = clamp(rne(quot), 0,
// maxq), NaN kept
__device__ inline float affine_round(float quot, float maxq) {
  const float q = rintf(quot);
  return q != q ? q : fminf(fmaxf(q, 0.0f), maxq);
}

// grid.py:215-221: q = clamp(rne((w - b) / s_safe), 0, maxq); ys = RN(1/s_safe)
__device__ inline float affine_q(float w, float b, float s_safe, float ys, float maxq) {
  return affine_round(div_pos(w - b, s_safe, ys), maxq);
}

// gptq.py:216-222 for the affine path: dead columns zeroed in W, H diag := 1.
__global__ void dead_fix_w_kernel(float* __restrict__ W, float* __restrict__ H, int64_t B,
                                  int64_t R, int64_t C) {
  const int64_t n = B * R * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / (R * C), c = i % C;
    if (H[b * C * C + c * C + c] <= 0.0f) W[i] = 0.0f;
  }
}

__global__ void dead_fix_h_kernel(float* __restrict__ H, int64_t B, int64_t C) {
  const int64_t n = B * C;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t b = i / C, c = i % C;
    float* d = H + b * C * C + c * C + c;
    if (*d <= 0.0f) *d = 1.0f;
  }
}

// Row k of U restricted to the group's columns: lane t holds U[k][j + t + 64 s]
// (0 past the group). LDSU: from the block's copy Ublk[(k - i1) * n + (col -
// i1)] in LDS, else from global memory. Lanes past the group read the
// group's first column, so the load needs no branch.
template <int CPL, bool LDSU>
__device__ inline void load_urow(const float* __restrict__ Ub, const float* Ublk, int64_t C,
                                 int64_t i1, int n, int64_t k, int64_t j, int lane,
                                 const bool (&act)[CPL], float (&u)[CPL]) {
  const float* Uk = LDSU ? Ublk + (k - i1) * n + (j - i1) : Ub + k * C + j;
#pragma unroll
  for (int s = 0; s < CPL; ++s) {
    const float v = Uk[act[s] ? lane + 64 * s : 0];
    u[s] = act[s] ? v : 0.0f;
  }
}

__device__ inline float lane_read(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Grid (ceil(R / 4), B): the four waves of a workgroup take rows of one
// batch item. LDSU (blocks of at most kLdsBlock columns): the workgroup first
// copies the block's U[i1:i1+n, i1:i1+n] to LDS, so the column loop and the
// in-block updates read U rows from LDS instead of all waves fetching the
// same row from L2 at once.
constexpr int kLdsBlock = 128;

template <int CPL, bool LDSU>
__global__ void __launch_bounds__(kWaves * 64)
    affine_block_kernel(float* __restrict__ W, const float* __restrict__ U, int64_t B, int64_t R,
                        int64_t C, int64_t i1, int n, int G, float maxq, int storage, Shrinks sh,
                        uint8_t* __restrict__ q_out, void* s_store, void* b_store,
                        float* __restrict__ Err) {
  // per-wave table [kWaves][max(G, 64)] (float4: the clip candidates, then
  // the column table), errs [kWaves][n], then (LDSU) Ublk [n][n]
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tab_n = G > 64 ? G : 64;
  float4* ctab = reinterpret_cast<float4*>(smem) + wave * tab_n;
  float* errs = smem + kWaves * 4 * tab_n + wave * n;
  float* Ublk = smem + kWaves * 4 * tab_n + kWaves * n;
  const int64_t b = blockIdx.y;
  const float* Ub = U + b * C * C;
  if constexpr (LDSU) {
    if ((n & 1) == 0 && (C & 1) == 0 && (i1 & 1) == 0) {
      // wave w copies rows w, w+4, ...: one 8-byte chunk per lane and row,
      // sixteen rows' loads in flight before their LDS stores
      const int half_n = n >> 1;
      const bool on = lane < half_n;
      for (int r0 = wave; r0 < n; r0 += kWaves * 16) {
        float2 v[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const int r = r0 + kWaves * t;
          v[t] = (on && r < n) ? *reinterpret_cast<const float2*>(Ub + (i1 + r) * C + i1 + 2 * lane)
                               : float2{0.0f, 0.0f};
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const int r = r0 + kWaves * t;
          if (on && r < n) *reinterpret_cast<float2*>(Ublk + r * n + 2 * lane) = v[t];
        }
      }
    } else {
      for (int e = threadIdx.x; e < n * n; e += kWaves * 64) {
        const int r = e / n, c = e % n;
        Ublk[e] = Ub[(i1 + r) * C + i1 + c];
      }
    }
    __syncthreads();
  }
  const int64_t r_in = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (r_in >= R) return;  // whole wave exits together (no block barriers below)
  // canonicalized once, so that the clamps in affine_round do not redo it
  maxq = __builtin_canonicalizef(maxq);
  const int64_t row = b * R + r_in;
  float* Wr = W + row * C;
  const int64_t ng = C / G;
  // the clip candidates' p / maxq and p, one per lane (batches of 64)
  const int n_batches = (sh.n + 63) / 64;
  for (int64_t j = i1; j < i1 + n; j += G) {
    float acc[CPL], dg[CPL], yd[CPL];
    bool act[CPL];
#pragma unroll
    for (int s = 0; s < CPL; ++s) {
      const int col = lane + 64 * s;
      act[s] = col < G;
      acc[s] = act[s] ? Wr[j + col] : 0.0f;
      // U's diagonal of the lane's column and its reciprocal for div_pos
      const int cc = act[s] ? col : 0;
      dg[s] = act[s] ? (LDSU ? Ublk[(j - i1 + cc) * (n + 1)] : Ub[(j + cc) * (C + 1)]) : 1.0f;
      yd[s] = div_exact_recip(dg[s]);
    }
    // earlier in-block updates, in column order; sixteen rows of U in flight
    {
      const int64_t kn = j - i1;  // a multiple of G
      int64_t k = 0;
      for (; k + 16 <= kn; k += 16) {
        float u[16][CPL];
#pragma unroll
        for (int t = 0; t < 16; ++t) load_urow<CPL, LDSU>(Ub, Ublk, C, i1, n, i1 + k + t, j, lane, act, u[t]);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const float e = errs[k + t];
#pragma unroll
          for (int s = 0; s < CPL; ++s) acc[s] = act[s] ? acc[s] - e * u[t][s] : acc[s];
        }
      }
      for (; k < kn; ++k) {
        float u[CPL];
        load_urow<CPL, LDSU>(Ub, Ublk, C, i1, n, i1 + k, j, lane, act, u);
        const float e = errs[k];
#pragma unroll
        for (int s = 0; s < CPL; ++s) acc[s] = act[s] ? acc[s] - e * u[s] : acc[s];
      }
    }
    // clip search (grid.py:167-212) on the group's current values
    float lo = act[0] ? acc[0] : __uint_as_float(0x7f800000u);
    float hi = act[0] ? acc[0] : __uint_as_float(0xff800000u);
#pragma unroll
    for (int s = 1; s < CPL; ++s)
      if (act[s]) {
        lo = nan_min(lo, acc[s]);
        hi = nan_max(hi, acc[s]);
      }
    wave_nan_minmax(lo, hi, lane);
    const float wmin = lo, wmax = hi;
    const float range = wmax - wmin;
    float best_err = 0.0f, s32 = 0.0f, b32 = 0.0f;
    for (int bt = 0; bt < n_batches; ++bt) {
      // lane l prepares candidate 64 bt + l: scale, bias, divisor and its
      // reciprocal, into the wave's table (one LDS read per candidate)
      {
        const int cl = 64 * bt + lane < sh.n ? 64 * bt + lane : sh.n - 1;
        const float sc_l = round_to_storage(range * sh.p_over_maxq[cl], storage);
        const float bi_l = round_to_storage(wmin * sh.p[cl], storage);
        const float ss_l = (fabsf(sc_l) < 1e-12f) ? 1.0f : sc_l;
        ctab[lane] = float4{sc_l, bi_l, ss_l, div_exact_recip(ss_l)};
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
      }
      // candidates kCand at a time, their error sums reduced in one
      // butterfly; slots past the batch score a copy of its last candidate
      // (an equal error never replaces the earlier best under strict '<').
      // The quotients of the whole batch take the exact-division correction;
      // the numerators' magnitudes (as in the column chain) and a zero
      // reciprocal send the batch's out-of-range quotients to the IEEE
      // division.
      const int nb = sh.n - 64 * bt < 64 ? sh.n - 64 * bt : 64;
      for (int c0 = 0; c0 < nb; c0 += kCand) {
        float sc[kCand], bi[kCand], ss[kCand], ys[kCand], part[kCand];
        float num[kCand][CPL], quo[kCand][CPL];
        uint32_t mag_lo = 0xffffffffu;
        float mag_hi = 0.0f;
        bool y_zero = false;
#pragma unroll
        for (int i = 0; i < kCand; ++i) {
          const int ci = c0 + i < nb ? c0 + i : nb - 1;
          const float4 pc = ctab[ci];
          sc[i] = pc.x, bi[i] = pc.y, ss[i] = pc.z, ys[i] = pc.w;
          y_zero |= !(ys[i] != 0.0f);
#pragma unroll
          for (int s = 0; s < CPL; ++s) {
            num[i][s] = acc[s] - bi[i];
            quo[i][s] = div_fast(num[i][s], ss[i], ys[i]);
            mag_lo = min(mag_lo, (f2u(num[i][s]) << 1) - 2u);
            mag_hi = fmaxf(mag_hi, fabsf(num[i][s]));
          }
        }
        const bool slow = y_zero | (mag_lo < (27u << 24) - 2u) | !(mag_hi < 0x1p101f);
        if (__builtin_amdgcn_ballot_w64(slow) != 0) {
          asm volatile("" ::: "memory");
#pragma unroll
          for (int i = 0; i < kCand; ++i)
#pragma unroll
            for (int s = 0; s < CPL; ++s)
              if (act[s] && div_slow(num[i][s], ys[i])) quo[i][s] = num[i][s] / ss[i];
        }
#pragma unroll
        for (int i = 0; i < kCand; ++i) {
          part[i] = 0.0f;
#pragma unroll
          for (int s = 0; s < CPL; ++s) {
            // a zero numerator's quotient is that zero (see the column chain);
            // the clamp need not keep a NaN: a NaN quotient comes only from a
            // NaN acc, which makes d NaN anyway
            const float qt = copysignf(quo[i][s], num[i][s]);
            const float d = fminf(fmaxf(rintf(qt), 0.0f), maxq) * sc[i] + bi[i] - acc[s];
            part[i] = act[s] ? part[i] + d * d : part[i];
          }
        }
        float sums[kCand / 4];
        wave_sum_halving<kCand>(part, sums);
#pragma unroll
        for (int i = 0; i < kCand; ++i) {
          const float pi = lane_read(sums[i % (kCand / 4)], 16 * (i / (kCand / 4)));
          if ((bt == 0 && c0 + i == 0) || pi < best_err) {
            best_err = pi;
            s32 = sc[i];
            b32 = bi[i];
          }
        }
      }
    }
    const int64_t gi = row * ng + j / G;
    if (lane == 0) {
      store_storage(s_store, gi, s32, storage);
      store_storage(b_store, gi, b32, storage);
    }
    const float s_safe = (fabsf(s32) < 1e-12f) ? 1.0f : s32;
    const float ysafe = div_exact_recip(s_safe);
    // Sequential columns of the group. wn is the current column's value: the
    // owner lane's value after the updates of every earlier column. Before
    // column c's update the wave reads lane c+1's value (updated through
    // column c-1) and U[c, c+1], and wn = pre - e * U[c, c+1] repeats lane
    // c+1's own update (the same two roundings), so no lane read waits for
    // the column's error. Every lane past c applies w <- w - e * U[c, col]
    // (lanes past the group too: their values are never read). A column's
    // lane is not updated after its own column, so at the group's end it
    // holds the value its column was quantized from.
    //
    // The two divisions of a column take Markstein's correction without a
    // branch (EXACT = false); the operands outside its exact range are only
    // recorded. If any occurred, the group is run again from its start values
    // with the guarded division (EXACT = true), so every quotient is the
    // correctly rounded one either way.
    float acc0[CPL];
#pragma unroll
    for (int s = 0; s < CPL; ++s) acc0[s] = acc[s];
    // A divisor whose reciprocal is 0 (outside [2^-24, 2^24]) sends the
    // group to the guarded division directly.
    bool y_zero = !(ysafe != 0.0f);
#pragma unroll
    for (int s = 0; s < CPL; ++s) y_zero |= act[s] & !(yd[s] != 0.0f);
    y_zero = __builtin_amdgcn_ballot_w64(y_zero) != 0;
    // the column table: U[c][c], RN(1 / U[c][c]) and U[c][c+1] for column
    // c, read by the whole wave with one LDS read per column
#pragma unroll
    for (int s = 0; s < CPL; ++s) {
      const int col = lane + 64 * s;
      if (act[s]) {
        const int cn = col + 1 < G ? col + 1 : col;
        const float u1 = col + 1 < G ? (LDSU ? Ublk[(j - i1 + col) * n + (j - i1 + cn)]
                                             : Ub[(j + col) * C + j + cn])
                                     : 0.0f;
        ctab[col] = float4{dg[s], yd[s], u1, 0.0f};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    auto run_columns = [&](auto exact_tag) __attribute__((always_inline)) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      // The numerators' smallest nonzero magnitude (as its bit pattern
      // shifted left by one, minus 2, so that a zero wraps to the top) and
      // their largest magnitude. The correction is exact when every nonzero
      // numerator has a biased exponent in [27, 227] (div_slow).
      uint32_t mag_lo = 0xffffffffu;
      float mag_hi = 0.0f;
      float wn = lane_read(acc[0], 0);
      // column c; c1 = c + 1 (c for the last column)
      auto column = [&](int c, int c1, const float (&uc)[CPL]) __attribute__((always_inline)) {
        const int owner1 = c1 & 63, slot1 = c1 >> 6;
        float pre_v = acc[0];
#pragma unroll
        for (int s = 1; s < CPL; ++s)
          if (s == slot1) pre_v = acc[s];
        const float4 ct = ctab[c];
        const float diag = ct.x, ydg = ct.y, u1 = ct.z;
        const float pre1 = lane_read(pre_v, owner1);
        float e;
        if constexpr (EXACT) {
          const float q = affine_q(wn, b32, s_safe, ysafe, maxq);
          const float dq = q * s32 + b32;
          e = div_pos(wn - dq, diag, ydg);
        } else {
          // a zero numerator's quotient is that zero: copysign turns the
          // correction's +0 into it (every other quotient has its sign)
          // NaN is not kept here: a NaN quotient means a NaN column value,
          // which reaches wn at the end of the group and sends the group to
          // the exact pass, whose rounding keeps it
          const float n1 = wn - b32;
          const float q =
              fminf(fmaxf(rintf(copysignf(div_fast(n1, s_safe, ysafe), n1)), 0.0f), maxq);
          const float dq = q * s32 + b32;
          const float n2 = wn - dq;
          e = copysignf(div_fast(n2, diag, ydg), n2);
          mag_lo = min(mag_lo, min((f2u(n1) << 1) - 2u, (f2u(n2) << 1) - 2u));
          mag_hi = fmaxf(mag_hi, fmaxf(fabsf(n1), fabsf(n2)));
        }
#pragma unroll
        for (int s = 0; s < CPL; ++s) acc[s] = lane + 64 * s > c ? acc[s] - e * uc[s] : acc[s];
        wn = pre1 - e * u1;
      };
      // Row c of the group's U block at urow + c * ust. Rows arrive eight
      // columns ahead (a slot is refilled once its column is done); the last
      // eight full columns load nothing, and the columns past the last
      // multiple of 8 load their own rows.
      const float* urow = LDSU ? Ublk + (j - i1) * n + (j - i1) : Ub + j * C + j;
      const int64_t ust = LDSU ? n : C;
      // (lanes past the group read the row's first entry: their values are
      // never read)
      auto load_row = [&](const float* p, float (&u)[CPL]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < CPL; ++s) u[s] = p[act[s] ? lane + 64 * s : 0];
      };
      const int G8 = G & ~7;
      float ring[8][CPL];
#pragma unroll
      for (int u = 0; u < 8; ++u) load_row(urow + (u < G ? u : G - 1) * ust, ring[u]);
      const float* unext = urow + 8 * ust;
      int c0 = 0;
      for (; c0 + 8 < G8; c0 += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          column(c0 + u, c0 + u + 1, ring[u]);
          load_row(unext, ring[u]);
          unext += ust;
        }
      }
      if (G8 > 0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int c = c0 + u;
          column(c, c + 1 < G ? c + 1 : c, ring[u]);
        }
      }
      for (int c = G8; c < G; ++c) {
        float uc[CPL];
        load_row(urow + c * ust, uc);
        column(c, c + 1 < G ? c + 1 : c, uc);
      }
      // nonzero numerators below 2^-100, any at or above 2^101, or a NaN
      // anywhere in the chain (it reaches the final wn through e)
      return (mag_lo < (27u << 24) - 2u) | !(mag_hi < 0x1p101f) | (wn != wn);
    };
    // every lane computed the same chain, so its verdict is wave-uniform
    if (y_zero || __builtin_amdgcn_ballot_w64(run_columns(std::false_type{})) != 0) {
#pragma unroll
      for (int s = 0; s < CPL; ++s) acc[s] = acc0[s];
      run_columns(std::true_type{});
    }
    // each lane's code, dequantized value and error, from the value its
    // column was quantized from (the same operations as the column step)
#pragma unroll
    for (int s = 0; s < CPL; ++s) {
      const float q = affine_q(acc[s], b32, s_safe, ysafe, maxq);
      const float dq = q * s32 + b32;
      const float e = div_pos(acc[s] - dq, dg[s], yd[s]);
      if (!act[s]) continue;
      const int col = lane + 64 * s;
      q_out[row * C + j + col] = (q == q) ? static_cast<uint8_t>(q) : 0;
      Wr[j + col] = dq;
      errs[j + col - i1] = e;
      Err[row * n + (j + col - i1)] = e;
    }
    // errs[] is read by every lane of this wave at the next group start
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

// W[row, i2 + m] -= sum_k Err[row, k] * U[b, i1 + k, i2 + m] (the reference's
// deferred bmm): 64x64 output tiles, each wave a 32x32 block on
// v_mfma_f32_32x32x2f32 (A[l%32][k], B[k][l%32] with k = l/32 per step; result
// register r of lane l = D[8(r/4) + 4(l/32) + r%4][l%32]). K goes in chunks of
// 64: the workgroup stages the chunk's Err rows and U columns (transposed) in
// LDS with 16-byte coalesced loads, then each lane reads four consecutive k
// of its Err row and of its U column with one 16-byte LDS read each; step t
// of an 8-k group takes k = group + 4(l/32) + t for both operands (the same
// permutation of k in every build of this kernel, so the sums round the same
// way). The tile's W values are loaded before the products and updated after
// them.
constexpr int kTm = 64, kTn = 64, kLzK = 64, kLzS = kLzK + 4;  // LDS row stride (floats)
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256)
    lazy_update_kernel(float* __restrict__ W, const float* __restrict__ U,
                       const float* __restrict__ Err, int64_t B, int64_t R, int64_t C, int64_t i1,
                       int n) {
  __shared__ __attribute__((aligned(16))) float sE[kTm][kLzS];  // Err[r0 + i][kc + k]
  __shared__ __attribute__((aligned(16))) float sU[kTn][kLzS];  // U[i1 + kc + k][m0 + j], as [j][k]
  const int64_t i2 = i1 + n;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t R0 = static_cast<int64_t>(blockIdx.y) * kTm;
  const int64_t M0 = i2 + static_cast<int64_t>(blockIdx.x) * kTn;
  const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
  const int li = lane & 31, g = lane >> 5;
  const int64_t m = M0 + wc + li;
  const bool mok = m < C;
  // this lane's 16 outputs: rows R0 + wr + 8(i/4) + 4g + i%4, column m
  float wv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t rr = R0 + wr + 8 * (i >> 2) + 4 * g + (i & 3);
    wv[i] = (rr < R && mok) ? W[(b * R + rr) * C + m] : 0.0f;
  }
  const float* Eb = Err + b * R * n;
  const float* Ub = U + b * C * C;
  const bool vec = (n & 3) == 0 && (C & 3) == 0 && (i2 & 3) == 0;
  f32x16_t acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  for (int kc = 0; kc < n; kc += kLzK) {
    // stage: thread t copies 16-byte pieces (row t / 16 + 16 p, k or column 4 (t % 16))
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int rr = tid / 16 + 16 * p, c4 = 4 * (tid % 16);
      // Err rows
      {
        const int64_t row = R0 + rr;
        const int k = kc + c4;
        float v[4];
        if (vec && row < R && k + 4 <= n) {
          const float4 q = *reinterpret_cast<const float4*>(Eb + row * n + k);
          v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = (row < R && k + t < n) ? Eb[row * n + k + t] : 0.0f;
        }
        *reinterpret_cast<float4*>(&sE[rr][c4]) = float4{v[0], v[1], v[2], v[3]};
      }
      // U row i1 + kc + rr, columns M0 + c4 .. + 3, stored transposed
      {
        const int k = kc + rr;
        const int64_t col = M0 + c4;
        float v[4];
        if (vec && k < n && col + 4 <= C) {
          const float4 q = *reinterpret_cast<const float4*>(Ub + (i1 + k) * C + col);
          v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t) v[t] = (k < n && col + t < C) ? Ub[(i1 + k) * C + col + t] : 0.0f;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) sU[c4 + t][rr] = v[t];
      }
    }
    __syncthreads();
#pragma unroll
    for (int k8 = 0; k8 < kLzK; k8 += 8) {
      const float4 a = *reinterpret_cast<const float4*>(&sE[wr + li][k8 + 4 * g]);
      const float4 u = *reinterpret_cast<const float4*>(&sU[wc + li][k8 + 4 * g]);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, u.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, u.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, u.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, u.w, acc, 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t rr = R0 + wr + 8 * (i >> 2) + 4 * g + (i & 3);
    if (rr < R && mok) W[(b * R + rr) * C + m] = wv[i] - acc[i];
  }
}

int make_shrinks(int bits, int method, int grid_steps, double max_shrink, Shrinks* out) {
  const double maxq = static_cast<double>((1 << bits) - 1);
  if (method == MGQ_CLIP_MINMAX) {
    out->n = 4;  // one candidate, padded to the kernel's batch of four
    for (int i = 0; i < 4; ++i) {
      out->p_over_maxq[i] = static_cast<float>(1.0 / maxq);
      out->p[i] = 1.0f;
    }
    return MGQ_OK;
  }
  MGQ_REQUIRE(grid_steps >= 1 && grid_steps < kMaxShrinks - 4, MGQ_ERR_VALUE,
              "grid_steps must be in [1, %d)", kMaxShrinks - 4);
  out->n = grid_steps + 1;
  for (int i = 0; i <= grid_steps; ++i) {
    const double p = 1.0 - max_shrink * static_cast<double>(i) / static_cast<double>(grid_steps);
    out->p_over_maxq[i] = static_cast<float>(p / maxq);
    out->p[i] = static_cast<float>(p);
  }
  // the kernel scores candidates four at a time: pad with copies of the last
  // one (an equal error never replaces the earlier best under strict '<')
  while (out->n % 4) {
    out->p_over_maxq[out->n] = out->p_over_maxq[out->n - 1];
    out->p[out->n] = out->p[out->n - 1];
    ++out->n;
  }
  return MGQ_OK;
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int mgq_dead_fix(float* W, int64_t B, int64_t R, int64_t C, float* H, void* stream) {
  clear_error();
  MGQ_REQUIRE(B >= 0 && R >= 0 && C >= 0, MGQ_ERR_SHAPE, "bad shape");
  if (B * C == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  if (W != nullptr && R > 0) {
    dead_fix_w_kernel<<<elementwise_blocks(B * R * C, 256), 256, 0, s>>>(W, H, B, R, C);
    if (int rc = check_launch("dead fix W")) return rc;
  }
  dead_fix_h_kernel<<<elementwise_blocks(B * C, 256), 256, 0, s>>>(H, B, C);
  return check_launch("dead fix H");
}

extern "C" int mgq_gptq_affine_block(float* W, const float* U, int64_t B, int64_t R, int64_t C,
                                     int64_t i1, int64_t n, int group_size, int bits, int method,
                                     int storage_dtype, int grid_steps, double max_shrink,
                                     uint8_t* q_out, void* s_store, void* b_store, float* Err,
                                     void* stream) {
  clear_error();
  MGQ_REQUIRE(bits >= 1 && bits <= 8, MGQ_ERR_VALUE, "unsupported bits: %d", bits);
  MGQ_REQUIRE(group_size >= 1 && group_size <= 128, MGQ_ERR_VALUE,
              "group size %d unsupported (1..128)", group_size);
  MGQ_REQUIRE(storage_dtype == kF32 || storage_dtype == kBF16 || storage_dtype == kF16,
              MGQ_ERR_VALUE, "bad storage dtype");
  MGQ_REQUIRE(method == MGQ_CLIP_MINMAX || method == MGQ_CLIP_MSE, MGQ_ERR_VALUE,
              "unsupported clip method %d", method);
  MGQ_REQUIRE(C % group_size == 0 && i1 % group_size == 0 && n % group_size == 0 &&
                  n >= 1 && n <= kMaxBlock && i1 + n <= C,
              MGQ_ERR_SHAPE, "bad block [%lld, %lld) for C=%lld, G=%d", (long long)i1,
              (long long)(i1 + n), (long long)C, group_size);
  Shrinks sh;
  if (int rc = make_shrinks(bits, method, grid_steps, max_shrink, &sh)) return rc;
  if (B * R == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  const dim3 blocks(static_cast<unsigned>(ceil_div(R, kWaves)), static_cast<unsigned>(B));
  const float maxq = static_cast<float>((1 << bits) - 1);
  const bool ldsu = n <= kLdsBlock;
  const size_t tab_n = group_size > 64 ? group_size : 64;
  const size_t lds = sizeof(float) * (kWaves * 4 * tab_n +
                                      kWaves * static_cast<size_t>(n) +
                                      (ldsu ? static_cast<size_t>(n) * n : 0));
#define AFFINE_LAUNCH(CPL_, LDSU_)                                                          \
  affine_block_kernel<CPL_, LDSU_><<<blocks, kWaves * 64, lds, s>>>(                        \
      W, U, B, R, C, i1, static_cast<int>(n), group_size, maxq, storage_dtype, sh, q_out,  \
      s_store, b_store, Err)
  if (group_size <= 64) {
    if (ldsu) AFFINE_LAUNCH(1, true); else AFFINE_LAUNCH(1, false);
  } else {
    if (ldsu) AFFINE_LAUNCH(2, true); else AFFINE_LAUNCH(2, false);
  }
#undef AFFINE_LAUNCH
  if (int rc = check_launch("affine block")) return rc;
  if (i1 + n < C) {
    dim3 grid(static_cast<unsigned>(ceil_div(C - i1 - n, kTn)),
              static_cast<unsigned>(ceil_div(R, kTm)), static_cast<unsigned>(B));
    lazy_update_kernel<<<grid, 256, 0, s>>>(W, U, Err, B, R, C, i1, static_cast<int>(n));
    if (int rc = check_launch("affine lazy update")) return rc;
  }
  return MGQ_OK;
}
