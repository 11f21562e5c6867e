// Damped Cholesky-inverse upper factors (gptq.py:27-66, _prepare_hinv).
//
// For every square diagonal block Hb of size n (n = 32: the per-group blocks
// of the MXFP solver, gptq.py:99-100) compute the upper-triangular U with
//     U^T U = (Hd)^-1,   Hd = Hb + lam I,   lam = damp * max(mean(diag Hb), 1e-8),
// escalating damp *= 10 (fp32, per block) until the factorisation succeeds,
// at most max_attempts times, exactly as the reference escalates failed batch
// items. Hd is formed in fp32 as the reference does and, like
// torch.linalg.cholesky_ex, only its lower triangle is read; the
// factorisation and inverse run in fp64 and are rounded to fp32 once, so U
// is the correctly rounded factor up to fp64 error.
//
// Method. Factor Hd = V V^T with V upper triangular (Cholesky in reverse
// index order); then (Hd)^-1 = V^-T V^-1 = W^T W with W = V^-1 upper, and by
// uniqueness of the Cholesky factor U = W. The reference's factor / invert /
// re-factor sequence becomes one sweep over j = n-1 .. 0 that does the
// factorisation step and the Gauss-Jordan step of the inverse together:
// with a = row j of the working matrix (a_k = A[j][k] for k < j, the lower
// triangle; a_j = d, the pivot; a_k = X[j][k] for k > j, the not yet scaled
// row j of the inverse) and c_i = a_i / d, every row i < j does
//     R[i][k] -= c_i a_k   (k != j),   R[i][j] = -c_i,
// which is the trailing update A[i][k] -= V[i][j] V[k][j] for k < j and the
// elimination X[i][k] -= V[i][j] X[j][k] / sqrt(d) for k >= j at once.
// Row j is final after its step; at the end row i is scaled by 1/sqrt(d_i).
// A pivot <= 0 or NaN fails the attempt (LAPACK potrf semantics).
//
// Layout: one wavefront per block, lanes as an 8 x 8 grid (p = lane / 8,
// q = lane % 8), lane (p, q) holding rows 4p..4p+3 x columns 4q..4q+3 in 16
// fp64 registers. Each step the 8 lanes that hold row j write it (256 bytes)
// to the wave's LDS slot and every lane reads back the 4 entries of its rows
// and the 4 of its columns. There is no workgroup barrier: the four waves
// of a workgroup work on different blocks and LDS operations of one wave
// complete in issue order.
#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

constexpr int kN = 32;
constexpr int kWaves = 4;  // blocks per workgroup, one wavefront each

typedef double f64x2_t __attribute__((ext_vector_type(2)));

__device__ inline double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// attempts[g*B + b]: 1..max_attempts on success, 0 if every attempt failed.
// Hc (optional): compact [B*G][32][32] copy of each undamped block.
// dead (optional): the dead-column fix of gptq.py:216-222 on the block's own
// diagonal first -- an entry <= 0 marks its column dead (dead[b*C + c] = 1)
// and becomes 1 in H, in place -- so the block is factored (and copied to
// Hc) as the reference factors it after the fix. Without dead, H is only
// read.
__global__ void __launch_bounds__(64 * kWaves)
    hinv32_kernel(float* H, int64_t B, int64_t C, float damp, int max_attempts,
                  float* __restrict__ U, int32_t* __restrict__ attempts, float* __restrict__ Hc,
                  uint8_t* __restrict__ dead) {
  __shared__ __attribute__((aligned(16))) double bcast[kWaves][kN];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t G = C / kN;
  const int64_t blk = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
  if (blk >= B * G) return;  // whole wavefront
  const int64_t b = blk / G, g = blk % G;
  const int p = lane >> 3, q = lane & 7;
  double* bc = bcast[wave];

  // the lane's 4x4 tile of the undamped block (rows 4p+r, columns 4q+c)
  float h[4][4];
  {
    float* src = H + b * C * C + (g * kN + 4 * p) * C + g * kN + 4 * q;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float4 v = *reinterpret_cast<const float4*>(src + r * C);
      h[r][0] = v.x, h[r][1] = v.y, h[r][2] = v.z, h[r][3] = v.w;
    }
    if (dead != nullptr && p == q) {  // this lane holds diagonal entries 4p..4p+3
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool is_dead = h[r][r] <= 0.0f;
        if (is_dead) {
          h[r][r] = 1.0f;
          src[r * C + r] = 1.0f;
        }
        dead[b * C + g * kN + 4 * p + r] = is_dead ? 1 : 0;
      }
    }
    if (Hc) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *reinterpret_cast<float4*>(Hc + blk * kN * kN + (4 * p + r) * kN + 4 * q) =
            float4{h[r][0], h[r][1], h[r][2], h[r][3]};
    }
  }
  // diag mean (fp64 sum, rounded once) clamped like torch .clamp(min=1e-8)
  double ds = 0.0;
  if (p == q) ds = (static_cast<double>(h[0][0]) + h[1][1]) + (static_cast<double>(h[2][2]) + h[3][3]);
  float dmean = static_cast<float>(wave_sum_f64(ds) / kN);
  dmean = (dmean < 1e-8f) ? 1e-8f : dmean;  // NaN stays NaN

  double R[4][4], piv[4];
  float cur = damp;
  int used = 0;
  for (int att = 1; att <= max_attempts; ++att) {
    const float lam = dmean * cur;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int i = 4 * p + r, k = 4 * q + c;
        const float v = (i == k) ? h[r][c] + lam : h[r][c];  // Hd in fp32
        R[r][c] = (k <= i) ? static_cast<double>(v) : 0.0;
      }
      piv[r] = 0.0;
    }
    bool ok = true;
    // j = 4 jp + jr: the row-group loop stays rolled (its predicates are
    // computed per iteration), the 4 rows of a group are unrolled so that
    // register indices are compile-time constants.
#pragma unroll 1
    for (int jp = kN / 4 - 1; jp >= 0; --jp) {
      const bool own_row = (p == jp), own_col = (q == jp);
#pragma unroll
      for (int jr = 3; jr >= 0; --jr) {
        const int j = 4 * jp + jr;
        if (own_row) {  // the 8 lanes holding row j publish it
          *reinterpret_cast<f64x2_t*>(bc + 4 * q) = f64x2_t{R[jr][0], R[jr][1]};
          *reinterpret_cast<f64x2_t*>(bc + 4 * q + 2) = f64x2_t{R[jr][2], R[jr][3]};
        }
        __builtin_amdgcn_wave_barrier();
        const f64x2_t a01 = *reinterpret_cast<const f64x2_t*>(bc + 4 * p);
        const f64x2_t a23 = *reinterpret_cast<const f64x2_t*>(bc + 4 * p + 2);
        const f64x2_t b01 = *reinterpret_cast<const f64x2_t*>(bc + 4 * q);
        const f64x2_t b23 = *reinterpret_cast<const f64x2_t*>(bc + 4 * q + 2);
        const double d = bc[j];
        __builtin_amdgcn_wave_barrier();
        ok = ok & (d > 0.0);
        const double rd = recip_f64(d);
        piv[jr] = own_row ? d : piv[jr];
        const double ai[4] = {a01.x, a01.y, a23.x, a23.y};
        const double ak[4] = {b01.x, b01.y, b23.x, b23.y};
        double cf[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) cf[r] = (4 * p + r < j) ? ai[r] * rd : 0.0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int c = 0; c < 4; ++c) R[r][c] = fma(-cf[r], ak[c], R[r][c]);
          // column j of the inverse: X[i][j] = -c_i (cf is 0 for rows i >= j,
          // whose entry the fma above left unchanged)
          if (4 * p + r < j) R[r][jr] = own_col ? -cf[r] : R[r][jr];
        }
      }
    }
    if (__builtin_amdgcn_readfirstlane(ok ? 1 : 0)) {  // d is the same in every lane
      used = att;
      break;
    }
    cur = cur * 10.0f;
  }
  float* Ub = U + blk * kN * kN;
  if (used == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<float4*>(Ub + (4 * p + r) * kN + 4 * q) = float4{0.f, 0.f, 0.f, 0.f};
    if (lane == 0) attempts[g * B + b] = 0;
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * p + r;
    const double rs = 1.0 / sqrt(piv[r]);  // meaningful where the tile holds column i
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = 4 * q + c;
      o[c] = (k > i) ? static_cast<float>(R[r][c] * rs) : (k == i ? static_cast<float>(rs) : 0.0f);
    }
    *reinterpret_cast<float4*>(Ub + i * kN + 4 * q) = float4{o[0], o[1], o[2], o[3]};
  }
  if (lane == 0) attempts[g * B + b] = used;
}

}  // namespace

// Launch helper shared with the MXFP solver (which passes dead, and so has
// H's dead diagonals fixed in place by this launch).
int launch_hinv32(float* H, int64_t B, int64_t C, float damp, int max_attempts, float* U,
                  int32_t* attempts, float* Hc, uint8_t* dead, hipStream_t s) {
  const int64_t n = B * (C / kN);
  if (n == 0) return MGQ_OK;
  hinv32_kernel<<<static_cast<unsigned>((n + kWaves - 1) / kWaves), 64 * kWaves, 0, s>>>(
      H, B, C, damp, max_attempts, U, attempts, Hc, dead);
  return check_launch("hinv32");
}

}  // namespace mgq

using namespace mgq;

extern "C" int mgq_prepare_hinv_blocks(const float* H, int64_t B, int64_t C, int64_t block,
                                       float damp, int max_attempts, float* U,
                                       int32_t* attempts, void* stream) {
  clear_error();
  MGQ_REQUIRE(block == kN, MGQ_ERR_VALUE, "block size %lld unsupported (32)", (long long)block);
  MGQ_REQUIRE(B >= 0 && C >= 0 && C % kN == 0, MGQ_ERR_SHAPE,
              "C=%lld not a multiple of the block size %d", (long long)C, kN);
  MGQ_REQUIRE(max_attempts >= 1, MGQ_ERR_VALUE, "max_attempts must be >= 1");
  MGQ_REQUIRE((reinterpret_cast<uintptr_t>(H) & 15u) == 0 && (reinterpret_cast<uintptr_t>(U) & 15u) == 0,
              MGQ_ERR_SHAPE, "H and U must be 16-byte aligned");
  // without dead the kernel only reads H
  return launch_hinv32(const_cast<float*>(H), B, C, damp, max_attempts, U, attempts, nullptr,
                       nullptr, as_stream(stream));
}
