// Full-matrix damped Cholesky-inverse upper factor (gptq.py:27-66 for the
// affine solver, which factors the whole [C, C] Hessian).
//
//   U (upper) with U^T U = (H + lam I)^-1,  lam = damp * max(mean(diag H), 1e-8)
//
// As in the 32x32 kernel, Hd = V V^T is factored with V upper triangular
// ("UL" Cholesky, i.e. Cholesky in reverse index order) and U = V^-1. The
// blocked algorithm walks diagonal blocks of nb = 64 from the bottom-right
// corner to the top-left; for the block at jb (A11 = A[0:jb,0:jb],
// A12 = A[0:jb, jb:jb+nb], A22 = the diagonal block):
//   1. A22 = V22 V22^T (one workgroup, fp64 in LDS), W22 = V22^-1;
//   2. V12 = A12 W22^T                                 (panel);
//   3. A11 -= V12 V12^T  (upper triangle)              (trailing update);
//   4. W[jb:jb+nb, jb+nb:] = -W22 V[jb:jb+nb, jb+nb:] W[jb+nb:, jb+nb:]
//      (the inverse grows upward with the factor: W = V^-1 is upper).
// Everything runs in fp64 (the factor of an fp32 matrix, rounded once), on
// a per-batch-item fp64 workspace. Items whose pivot fails are flagged and
// skipped by later steps; the host escalates their damping and reruns them,
// exactly like the reference retries only the failed batch items.
#include <algorithm>

#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

constexpr int kNb = 64;

// A = fp64(H + lam I) for items with active[b]; lam from fp32 ops as the
// reference forms Hd (diag_mean * damp, then diag += lam).
__global__ void build_hd_kernel(const float* __restrict__ H, int64_t C,
                                const float* __restrict__ damp, const uint8_t* __restrict__ active,
                                double* __restrict__ A) {
  const int64_t b = blockIdx.y;
  if (!active[b]) return;
  const float* Hb = H + b * C * C;
  double* Ab = A + b * C * C;
  // diag mean: fp64 sum, rounded once, clamped at 1e-8 (NaN stays NaN)
  __shared__ float s_lam;
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int64_t i = 0; i < C; ++i) s += static_cast<double>(Hb[i * C + i]);
    float dm = static_cast<float>(s / static_cast<double>(C));
    dm = dm < 1e-8f ? 1e-8f : dm;
    s_lam = dm * damp[b];
  }
  __syncthreads();
  const float lam = s_lam;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < C * C;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / C, j = e % C;
    float v = Hb[e];
    if (i == j) v = v + lam;
    Ab[e] = static_cast<double>(v);
  }
}

// Step 1: factor the diagonal block at jb (size n <= 64) in LDS; write V22
// into A's block and W22 = V22^-1 into W's block. A failed pivot sets
// failed[b].
__global__ void __launch_bounds__(256)
    diag_block_kernel(double* __restrict__ A, double* __restrict__ W, int64_t C, int64_t jb, int n,
                      const uint8_t* __restrict__ active, uint8_t* __restrict__ failed) {
  const int64_t b = blockIdx.x;
  if (!active[b] || failed[b]) return;
  __shared__ double S[kNb][kNb + 1];
  __shared__ double Wi[kNb][kNb + 1];
  __shared__ int s_fail;
  double* Ab = A + b * C * C;
  double* Wb = W + b * C * C;
  const int tid = threadIdx.x;
  for (int e = tid; e < n * n; e += blockDim.x) {
    const int i = e / n, j = e % n;
    S[i][j] = Ab[(jb + i) * C + jb + j];
  }
  if (tid == 0) s_fail = 0;
  __syncthreads();
  for (int j = n - 1; j >= 0; --j) {
    const double d = S[j][j];
    if (!(d > 0.0)) {
      if (tid == 0) s_fail = 1;
      break;  // uniform: every thread read the same pivot after the barrier
    }
    const double s = sqrt(d);
    __syncthreads();
    if (tid < j) S[tid][j] = S[tid][j] / s;
    if (tid == 0) S[j][j] = s;
    __syncthreads();
    for (int e = tid; e < j * j; e += blockDim.x) {
      const int i = e / j, k = e % j;
      if (i <= k) S[i][k] = S[i][k] - S[i][j] * S[k][j];
    }
    __syncthreads();
  }
  __syncthreads();
  if (s_fail) {
    if (tid == 0) failed[b] = 1;
    return;
  }
  // W22 = V22^-1 (upper), thread j back-substitutes column j
  if (tid < n) {
    const int j = tid;
    Wi[j][j] = 1.0 / S[j][j];
    for (int i = j - 1; i >= 0; --i) {
      double acc = 0.0;
      for (int k = i + 1; k <= j; ++k) acc += S[i][k] * Wi[k][j];
      Wi[i][j] = -acc / S[i][i];
    }
  }
  __syncthreads();
  for (int e = tid; e < n * n; e += blockDim.x) {
    const int i = e / n, j = e % n;
    Ab[(jb + i) * C + jb + j] = (i <= j) ? S[i][j] : 0.0;
    Wb[(jb + i) * C + jb + j] = (i <= j) ? Wi[i][j] : 0.0;
  }
}

// Step 2: V12 = A12 * W22^T, rows 0..jb-1, cols jb..jb+n-1 (in place in A).
// One thread per (row, col); the row of A12 is staged in registers first.
__global__ void panel_kernel(double* __restrict__ A, const double* __restrict__ W, int64_t C,
                             int64_t jb, int n, const uint8_t* __restrict__ active,
                             const uint8_t* __restrict__ failed) {
  const int64_t b = blockIdx.y;
  if (!active[b] || failed[b]) return;
  double* Ab = A + b * C * C;
  const double* Wb = W + b * C * C;
  __shared__ double Wt[kNb][kNb + 1];  // W22
  for (int e = threadIdx.x; e < n * n; e += blockDim.x) Wt[e / n][e % n] = Wb[(jb + e / n) * C + jb + e % n];
  __syncthreads();
  const int64_t rows_per_block = blockDim.x / kNb;
  const int64_t i = blockIdx.x * rows_per_block + threadIdx.x / kNb;
  const int c = threadIdx.x % kNb;
  __shared__ double Arow[4][kNb];
  const int slot = threadIdx.x / kNb;
  if (i < jb && c < n) Arow[slot][c] = Ab[i * C + jb + c];
  __syncthreads();
  if (i < jb && c < n) {
    // V12[i][c] = sum_k A12[i][k] * W22[c][k]  (W22 upper: k >= c)
    double acc = 0.0;
    for (int k = c; k < n; ++k) acc += Arow[slot][k] * Wt[c][k];
    Ab[i * C + jb + c] = acc;
  }
}

// Step 3: A11[i][k] -= sum_c V12[i][c] V12[k][c] for i <= k < jb. 64x64
// output tiles (upper-triangular tiles only), 4x4 outputs per thread, the
// two V12 row panels staged in LDS (K = n <= 64).
__global__ void __launch_bounds__(256)
    trailing_kernel(double* __restrict__ A, int64_t C, int64_t jb, int n,
                    const uint8_t* __restrict__ active, const uint8_t* __restrict__ failed) {
  const int64_t b = blockIdx.z;
  if (!active[b] || failed[b]) return;
  const int64_t ti = blockIdx.y, tk = blockIdx.x;
  if (tk < ti) return;  // upper tiles only
  double* Ab = A + b * C * C;
  __shared__ double Pi[kNb][kNb + 1], Pk[kNb][kNb + 1];  // [c][row]
  const int tid = threadIdx.x;
  for (int e = tid; e < kNb * kNb; e += 256) {
    const int r = e / kNb, c = e % kNb;
    const int64_t ri = ti * kNb + r, rk = tk * kNb + r;
    Pi[c][r] = (ri < jb && c < n) ? Ab[ri * C + jb + c] : 0.0;
    Pk[c][r] = (rk < jb && c < n) ? Ab[rk * C + jb + c] : 0.0;
  }
  __syncthreads();
  const int tx = tid % 16, ty = tid / 16;
  double acc[4][4] = {};
  for (int c = 0; c < n; ++c) {
    double pi[4], pk[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) pi[a] = Pi[c][ty * 4 + a];
#pragma unroll
    for (int a = 0; a < 4; ++a) pk[a] = Pk[c][tx * 4 + a];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int d = 0; d < 4; ++d) acc[a][d] += pi[a] * pk[d];
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t i = ti * kNb + ty * 4 + a;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int64_t k = tk * kNb + tx * 4 + d;
      if (i < jb && k < jb && i <= k) Ab[i * C + k] -= acc[a][d];
    }
  }
}

// Step 4: W[jb+r][m] = -sum_q W22[r][q] * T[q][m] for m >= jb+n, with
// T[q][m] = sum_{k=jb+n}^{m} V[jb+q][k] * W[k][m] (W upper: terms k > m are
// zero and are masked, since W's lower blocks are never written). One block
// per 64-column tile: T by a K-chunked LDS GEMM, then the 64x64 product
// with W22, 4x4 outputs per thread in both.
constexpr int kKc = 16;

__global__ void __launch_bounds__(256)
    wrow_kernel(const double* __restrict__ A, double* __restrict__ W, int64_t C, int64_t jb, int n,
                const uint8_t* __restrict__ active, const uint8_t* __restrict__ failed) {
  const int64_t b = blockIdx.y;
  if (!active[b] || failed[b]) return;
  const double* Ab = A + b * C * C;
  double* Wb = W + b * C * C;
  const int64_t m0 = jb + n + static_cast<int64_t>(blockIdx.x) * kNb;  // column tile
  if (m0 >= C) return;
  __shared__ double Vs[kKc][kNb + 1];  // [kk][q]
  __shared__ double Ws[kKc][kNb + 1];  // [kk][mm]
  __shared__ double T[kNb][kNb + 1];   // [q][mm]
  __shared__ double Wd[kNb][kNb + 1];  // W22 transposed: Wd[q][r] = W22[r][q]
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;
  const int64_t kend = (m0 + kNb < C) ? m0 + kNb : C;
  double acc[4][4] = {};
  for (int64_t k0 = jb + n; k0 < kend; k0 += kKc) {
    for (int e = tid; e < kKc * kNb; e += 256) {
      const int q = e / kKc, kk = e % kKc;
      const int64_t k = k0 + kk;
      Vs[kk][q] = (q < n && k < kend) ? Ab[(jb + q) * C + k] : 0.0;
    }
    for (int e = tid; e < kKc * kNb; e += 256) {
      const int kk = e / kNb, mm = e % kNb;
      const int64_t k = k0 + kk, m = m0 + mm;
      Ws[kk][mm] = (k < kend && m < C && k <= m) ? Wb[k * C + m] : 0.0;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kKc; ++kk) {
      double v[4], w[4];
#pragma unroll
      for (int a = 0; a < 4; ++a) v[a] = Vs[kk][ty * 4 + a];
#pragma unroll
      for (int a = 0; a < 4; ++a) w[a] = Ws[kk][tx * 4 + a];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[a][d] += v[a] * w[d];
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int d = 0; d < 4; ++d) T[ty * 4 + a][tx * 4 + d] = acc[a][d];
  for (int e = tid; e < kNb * kNb; e += 256) {
    const int r = e / kNb, q = e % kNb;
    Wd[q][r] = (r < n && q < n) ? Wb[(jb + r) * C + jb + q] : 0.0;
  }
  __syncthreads();
  double out[4][4] = {};
  for (int q = 0; q < n; ++q) {
    double wr[4], t[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) wr[a] = Wd[q][ty * 4 + a];
#pragma unroll
    for (int d = 0; d < 4; ++d) t[d] = T[q][tx * 4 + d];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int d = 0; d < 4; ++d) out[a][d] += wr[a] * t[d];
  }
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int r = ty * 4 + a;
    if (r >= n) continue;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int64_t m = m0 + tx * 4 + d;
      if (m < C) Wb[(jb + r) * C + m] = -out[a][d];
    }
  }
}

// U = fp32(W) (upper), zero below the diagonal, for items that succeeded.
__global__ void emit_u_kernel(const double* __restrict__ W, int64_t C,
                              const uint8_t* __restrict__ active,
                              const uint8_t* __restrict__ failed, float* __restrict__ U) {
  const int64_t b = blockIdx.y;
  if (!active[b] || failed[b]) return;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < C * C;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = e / C, j = e % C;
    U[b * C * C + e] = (i <= j) ? static_cast<float>(W[b * C * C + e]) : 0.0f;
  }
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int64_t mgq_hinv_full_workspace_size(int64_t B, int64_t C) {
  return 2 * B * C * C * 8 + 256;
}

// One factorisation pass for the items with active[b] != 0, using per-item
// damp[b]; failed[b] (device, cleared by the caller) reports pivot failure.
extern "C" int mgq_hinv_full_pass(const float* H, int64_t B, int64_t C, const float* damp,
                                  const uint8_t* active, uint8_t* failed, float* U,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  MGQ_REQUIRE(B >= 0 && C >= 1, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= mgq_hinv_full_workspace_size(B, C),
              MGQ_ERR_WORKSPACE, "hinv workspace too small");
  if (B == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  double* A = static_cast<double*>(workspace);
  double* W = A + B * C * C;
  const unsigned gb = static_cast<unsigned>(B);
  build_hd_kernel<<<dim3(elementwise_blocks(C * C, 256) / 8 + 1, gb), 256, 0, s>>>(H, C, damp,
                                                                                  active, A);
  if (int rc = check_launch("hinv build")) return rc;
  for (int64_t jb = ((C - 1) / kNb) * kNb; jb >= 0; jb -= kNb) {
    const int n = static_cast<int>(std::min<int64_t>(kNb, C - jb));
    diag_block_kernel<<<gb, 256, 0, s>>>(A, W, C, jb, n, active, failed);
    if (int rc = check_launch("hinv diag")) return rc;
    if (jb > 0) {
      panel_kernel<<<dim3(static_cast<unsigned>(ceil_div(jb, 4)), gb), 256, 0, s>>>(A, W, C, jb, n,
                                                                                   active, failed);
      if (int rc = check_launch("hinv panel")) return rc;
      const unsigned nt = static_cast<unsigned>(ceil_div(jb, kNb));
      trailing_kernel<<<dim3(nt, nt, gb), 256, 0, s>>>(A, C, jb, n, active, failed);
      if (int rc = check_launch("hinv trailing")) return rc;
    }
    if (jb + n < C) {
      const unsigned mt = static_cast<unsigned>(ceil_div(C - jb - n, kNb));
      wrow_kernel<<<dim3(mt, gb), 256, 0, s>>>(A, W, C, jb, n, active, failed);
      if (int rc = check_launch("hinv wrow")) return rc;
    }
  }
  emit_u_kernel<<<dim3(elementwise_blocks(C * C, 256) / 8 + 1, gb), 256, 0, s>>>(W, C, active,
                                                                                failed, U);
  return check_launch("hinv emit");
}
