// Full-matrix damped Cholesky-inverse upper factor (gptq.py:27-66 for the
// affine solver, which factors the whole [C, C] Hessian).
//
//   U (upper) with U^T U = (H + lam I)^-1,  lam = damp * max(mean(diag H), 1e-8)
//
// As in the 32x32 kernel, Hd = V V^T is factored with V upper triangular
// ("UL" Cholesky, i.e. Cholesky in reverse index order) and U = V^-1 = W.
// The factor and its inverse are built together by recursion over 64-row
// blocks [b0, b1), split at mid (top rows T = [b0, mid), bottom rows
// S = [mid, b1)):
//   1. (V_SS, W_SS) of A_SS                          (recursion, bottom first)
//   2. P = V_TS = A_TS W_SS^T                        (GEMM)
//   3. A_TT -= P P^T                                 (GEMM, upper tiles)
//   4. Q = P W_SS                                    (GEMM)
//   5. (V_TT, W_TT) of the updated A_TT              (recursion)
//   6. W_TS = -W_TT Q                                (GEMM)
// since V V^T = [[V_TT V_TT^T + V_TS V_TS^T, V_TS V_SS^T], [., V_SS V_SS^T]]
// and V^-1 = [[W_TT, -W_TT V_TS W_SS], [0, W_SS]]. A 64x64 leaf is factored
// and inverted by one workgroup with the block in registers. Everything runs
// in fp64 (the factor of an fp32 matrix, rounded to fp32 once). Items whose
// pivot fails are flagged and skipped by later steps; the host escalates
// their damping and reruns them, exactly like the reference retries only the
// failed batch items.
#include <algorithm>
#include <vector>

#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

constexpr int kNb = 64;  // leaf block

typedef double f64x2_t __attribute__((ext_vector_type(2)));

// lam[b] = fp32(max(mean(diag H_b), 1e-8) * damp[b]): fp64 diagonal sum
// rounded once, then the reference's fp32 clamp and product.
__global__ void __launch_bounds__(256)
    lam_kernel(const float* __restrict__ H, int64_t C, const float* __restrict__ damp,
               const uint8_t* __restrict__ active, float* __restrict__ lam) {
  const int64_t b = blockIdx.x;
  if (!active[b]) return;
  __shared__ double part[256];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < C; i += 256) s += static_cast<double>(H[b * C * C + i * C + i]);
  part[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float dm = static_cast<float>(part[0] / static_cast<double>(C));
    dm = dm < 1e-8f ? 1e-8f : dm;  // NaN stays NaN
    lam[b] = dm * damp[b];
  }
}

// A = fp64(H + lam I) (diagonal added in fp32, as the reference forms Hd);
// W = 0 (its blocks below the block diagonal must read as zero).
__global__ void build_kernel(const float* __restrict__ H, int64_t C, const float* __restrict__ lam,
                             const uint8_t* __restrict__ active, double* __restrict__ A,
                             double* __restrict__ W) {
  const int64_t b = blockIdx.y;
  if (!active[b]) return;
  const float l = lam[b];
  const float* Hb = H + b * C * C;
  double* Ab = A + b * C * C;
  double* Wb = W + b * C * C;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < C * C;
       e += (int64_t)gridDim.x * blockDim.x) {
    float v = Hb[e];
    if (e / C == e % C) v = v + l;
    Ab[e] = static_cast<double>(v);
    Wb[e] = 0.0;
  }
}

// Leaf: W = V^-1 for the n x n (n <= 64) diagonal block A_b = V V^T at r0
// (V upper). One workgroup of four waves per batch item. The sweep over
// j = 63 .. 0 does the factor step and the Gauss-Jordan step of the inverse
// at once (the 32 x 32 kernel of cholesky.hip does the same): with a = row j
// of the working matrix R (a_k = A[j][k] for k < j, a_j = d the pivot, a_k =
// unscaled row j of the inverse for k > j) and c_i = a_i / d, every row
// i < j does R[i][k] -= c_i a_k (k != j) and R[i][j] = -c_i. Row j is final
// after its step; at the end W[i][k] = R[i][k] / sqrt(d_i) for k > i and
// W[i][i] = 1 / sqrt(d_i). Wave w holds columns 16w..16w+15, its lanes an
// 8 x 8 grid (p = lane / 8, q = lane % 8): lane (p, q) holds rows 8p..8p+7 x
// columns 16w + 2q, 16w + 2q + 1 (16 fp64 registers). The steps go in pairs
// (j, j - 1), both rows in the same 8-row group: the lanes holding the two
// rows publish them through LDS (two alternating buffer pairs, so one
// workgroup barrier per pair), and every lane forms row j - 1 after step j
// from the two published rows itself, with the same operations the lanes
// holding row j - 1 apply to it (so the result is bitwise that of single
// steps). Each lane reads the entries of its 8 rows, its 2 columns and the
// pivots of both rows: 32 FMAs of update per lane and pair. The sweep is
// bound by instruction issue (one wave per SIMD), so the rows a step updates
// are selected by exec masks over two lane sets rather than by per-row
// selects, and rows at or past the pivot are not touched at all. Only the
// lower triangle of the block is read; rows past n are identity padding. A
// pivot <= 0 or NaN flags the item as failed.
__global__ void __launch_bounds__(256)
    leaf_kernel(const double* __restrict__ A, double* __restrict__ W, int64_t C, int64_t r0, int n,
                const uint8_t* __restrict__ active, uint8_t* __restrict__ failed) {
  const int64_t b = blockIdx.x;
  if (!active[b] || failed[b]) return;  // uniform over the workgroup
  __shared__ __attribute__((aligned(16))) double bc[4][kNb];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int p = lane >> 3, q = lane & 7;
  const int k0 = 16 * wave + 2 * q;  // this lane's two columns
  const double* Ab = A + b * C * C + r0 * C + r0;
  double R[8][2];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int i = 8 * p + r;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int k = k0 + c;
      R[r][c] = (i < n && k < n) ? (k <= i ? Ab[i * C + k] : 0.0) : (i == k ? 1.0 : 0.0);
    }
  }
  double piv[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) piv[r] = 1.0;
  bool ok = true;
#pragma unroll 1
  for (int jp = 7; jp >= 0; --jp) {
    const bool own_row = (p == jp);
#pragma unroll
    for (int jr = 7; jr >= 1; jr -= 2) {
      const int j = 8 * jp + jr;  // pivots j, then j - 1
      double* rj = bc[2 * ((jr >> 1) & 1)];
      double* rj1 = rj + kNb;
      if (own_row) {
        *reinterpret_cast<f64x2_t*>(rj + k0) = f64x2_t{R[jr][0], R[jr][1]};
        *reinterpret_cast<f64x2_t*>(rj1 + k0) = f64x2_t{R[jr - 1][0], R[jr - 1][1]};
      }
      __syncthreads();
      double ai[8], bi[8];
#pragma unroll
      for (int r = 0; r < 8; r += 2) {
        const f64x2_t u = *reinterpret_cast<const f64x2_t*>(rj + 8 * p + r);
        const f64x2_t v = *reinterpret_cast<const f64x2_t*>(rj1 + 8 * p + r);
        ai[r] = u.x, ai[r + 1] = u.y;
        bi[r] = v.x, bi[r + 1] = v.y;
      }
      const f64x2_t ak = *reinterpret_cast<const f64x2_t*>(rj + k0);
      const f64x2_t bk = *reinterpret_cast<const f64x2_t*>(rj1 + k0);
      const f64x2_t dj = *reinterpret_cast<const f64x2_t*>(rj + j - 1);  // {a_{j-1}, d}
      const double e = rj1[j - 1];
      const double d = dj.y;
      const double rd = recip_f64(d);
      const double cj = dj.x * rd;           // c_{j-1} of step j
      const double d1 = fma(-cj, dj.x, e);   // pivot of step j - 1
      ok = ok & (d > 0.0) & (d1 > 0.0);
      const double rd1 = recip_f64(d1);
      piv[jr] = own_row ? d : piv[jr];
      piv[jr - 1] = own_row ? d1 : piv[jr - 1];
      const bool col_j = (k0 == j - 1);  // this lane holds columns j - 1 and j
      // Row i = 8p + r takes step j when i < j: every row of a lane with
      // p < jp, the rows r < jr of the lanes with p == jp. The two lane sets
      // run as exec-masked blocks, so rows past the pivot are not touched
      // and no per-row select is needed; only the wave holding column j
      // enters the block that writes X[i][j] = -c_i.
      double cf[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) cf[r] = ai[r] * rd;
      if (p <= jp) {
#pragma unroll
        for (int r = 0; r < jr; ++r) {
          R[r][0] = fma(-cf[r], ak.x, R[r][0]);
          R[r][1] = fma(-cf[r], ak.y, R[r][1]);
        }
        if (col_j) {
#pragma unroll
          for (int r = 0; r < jr; ++r) R[r][1] = -cf[r];
        }
      }
      if (p < jp) {
#pragma unroll
        for (int r = jr; r < 8; ++r) {
          R[r][0] = fma(-cf[r], ak.x, R[r][0]);
          R[r][1] = fma(-cf[r], ak.y, R[r][1]);
        }
        if (col_j) {
#pragma unroll
          for (int r = jr; r < 8; ++r) R[r][1] = -cf[r];
        }
      }
      // row j - 1 after step j, at this lane's rows and columns
      double a1[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) a1[r] = fma(-cj, ai[r], bi[r]);
      const double ak1x = fma(-cj, ak.x, bk.x);
      const double ak1y = col_j ? -cj : fma(-cj, ak.y, bk.y);
      // step j - 1: rows i < j - 1
#pragma unroll
      for (int r = 0; r < 8; ++r) cf[r] = a1[r] * rd1;
      if (p <= jp) {
#pragma unroll
        for (int r = 0; r < jr - 1; ++r) {
          R[r][0] = fma(-cf[r], ak1x, R[r][0]);
          R[r][1] = fma(-cf[r], ak1y, R[r][1]);
        }
        if (col_j) {
#pragma unroll
          for (int r = 0; r < jr - 1; ++r) R[r][0] = -cf[r];
        }
      }
      if (p < jp) {
#pragma unroll
        for (int r = jr - 1; r < 8; ++r) {
          R[r][0] = fma(-cf[r], ak1x, R[r][0]);
          R[r][1] = fma(-cf[r], ak1y, R[r][1]);
        }
        if (col_j) {
#pragma unroll
          for (int r = jr - 1; r < 8; ++r) R[r][0] = -cf[r];
        }
      }
    }
  }
  if (!__builtin_amdgcn_readfirstlane(ok ? 1 : 0)) {  // d is the same in every lane
    if (threadIdx.x == 0) failed[b] = 1;
    return;
  }
  double* Wb = W + b * C * C + r0 * C + r0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int i = 8 * p + r;
    if (i >= n) continue;
    const double rs = 1.0 / sqrt(piv[r]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int k = k0 + c;
      if (k < n) Wb[i * C + k] = k > i ? R[r][c] * rs : (k == i ? rs : 0.0);
    }
  }
}

// C[m][n] = alpha * sum_k A[m][k] opB[k][n] + beta * C[m][n], opB = B or B^T
// (B stored [N][K]); row-major with leading dimensions, one matrix per batch
// item (item strides sA, sB, sC). fp64 MFMA (v_mfma_f64_16x16x4f64, whose
// operand layout is A[l%16][k], B[k][l%16] with k = l/16 per k-step, and
// result register r of lane l = D[l/16 + 4r][l%16]). A workgroup computes a
// 32 x 32 output tile as 2 x 2 MFMA blocks; its four waves split K in
// chunks of 16 (wave w takes chunks w, w+4, ...), each lane loading its four
// consecutive k of A and opB straight from global memory (the next chunk's
// loads in flight while the current one is multiplied; lane group l/16 of
// k-step t takes k = chunk + 4(l/16) + t, the same permutation of k for both
// operands). The four partial tiles are summed through LDS in wave order, so
// the result is deterministic. UPPER skips the tiles strictly below the
// 64-block diagonal (a leaf reads the lower triangle of its 64-block).
constexpr int kMt = 32;  // output tile edge
constexpr int kKc = 16;  // k per chunk and wave
typedef double f64x4_t __attribute__((ext_vector_type(4)));

// v[t] = p[t * stride] for t < cnt (0 past it); 16-byte loads where p allows
__device__ inline void load4(const double* __restrict__ p, int64_t stride, int cnt, double (&v)[4]) {
  if (cnt >= 4 && stride == 1 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    const f64x2_t lo = *reinterpret_cast<const f64x2_t*>(p);
    const f64x2_t hi = *reinterpret_cast<const f64x2_t*>(p + 2);
    v[0] = lo.x, v[1] = lo.y, v[2] = hi.x, v[3] = hi.y;
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = t < cnt ? p[t * stride] : 0.0;
  }
}

// One product's operands: C = alpha * A opB + beta * C, per batch item.
struct GemmArgs {
  const double* A;
  int64_t lda, sA;
  const double* B;
  int64_t ldb, sB;
  double* C;
  int64_t ldc, sC;
  int M, N, K;
  double alpha, beta;
};

// The 32 x 32 output tile at (m0, n0) of batch item `item`; red is the
// workgroup's LDS for the four waves' partial tiles.
template <bool TRANSB, bool UPPER>
__device__ inline void dgemm_tile(const GemmArgs& g, int m0, int n0, int64_t item,
                                  double (*red)[4][4][64]) {
  if (UPPER && (n0 >> 6) < (m0 >> 6)) return;  // uniform over the workgroup
  const double* Ab = g.A + item * g.sA;
  const double* Bb = g.B + item * g.sB;
  double* Cb = g.C + item * g.sC;
  const int M = g.M, N = g.N, K = g.K;
  const int64_t lda = g.lda, ldb = g.ldb, ldc = g.ldc;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 15, gq = lane >> 4;
  // this lane's A rows and opB columns; rows / columns past M / N read zeros
  const double* ap[2];
  const double* bp[2];
  bool aok[2], bok[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int m = m0 + 16 * h + li, n = n0 + 16 * h + li;
    aok[h] = m < M;
    bok[h] = n < N;
    ap[h] = Ab + static_cast<int64_t>(aok[h] ? m : 0) * lda;
    bp[h] = TRANSB ? Bb + static_cast<int64_t>(bok[h] ? n : 0) * ldb : Bb + (bok[h] ? n : 0);
  }
  auto load_chunk = [&](int kc, double (&a)[2][4], double (&b)[2][4]) {
    const int kb = kc + 4 * gq;
    const int cnt = K - kb < 0 ? 0 : (K - kb > 4 ? 4 : K - kb);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      load4(ap[h] + kb, 1, aok[h] ? cnt : 0, a[h]);
      if (TRANSB)
        load4(bp[h] + kb, 1, bok[h] ? cnt : 0, b[h]);
      else
        load4(bp[h] + static_cast<int64_t>(kb) * ldb, ldb, bok[h] ? cnt : 0, b[h]);
    }
  };
  f64x4_t acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f64x4_t{0.0, 0.0, 0.0, 0.0};
  int kc = wave * kKc;
  if (kc < K) {
    double a[2][4], b[2][4];
    load_chunk(kc, a, b);
    for (; kc < K; kc += 4 * kKc) {
      double na[2][4], nb[2][4];
      const bool more = kc + 4 * kKc < K;
      if (more) load_chunk(kc + 4 * kKc, na, nb);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[x][t], b[y][t], acc[x][y], 0, 0, 0);
      if (more) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int t = 0; t < 4; ++t) a[x][t] = na[x][t], b[x][t] = nb[x][t];
      }
    }
  }
  // red[wave][block (2x+y)][register][lane]
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][2 * x + y][r][lane] = acc[x][y][r];
  __syncthreads();
  // thread (part = wave, lane) finishes block part: rows l/16 + 4r, column l%16
  const int x = wave >> 1, y = wave & 1;
  const int n = n0 + 16 * y + li;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const double v = ((red[0][wave][r][lane] + red[1][wave][r][lane]) + red[2][wave][r][lane]) +
                     red[3][wave][r][lane];
    const int m = m0 + 16 * x + gq + 4 * r;
    if (m < M && n < N) {
      double* p = Cb + static_cast<int64_t>(m) * ldc + n;
      *p = g.beta == 0.0 ? g.alpha * v : g.alpha * v + g.beta * *p;
    }
  }
}

template <bool TRANSB, bool UPPER>
__global__ void __launch_bounds__(256)
    dgemm_kernel(GemmArgs g, const uint8_t* __restrict__ active,
                 const uint8_t* __restrict__ failed) {
  const int64_t item = blockIdx.z;
  if (!active[item] || failed[item]) return;
  __shared__ double red[4][4][4][64];
  dgemm_tile<TRANSB, UPPER>(g, static_cast<int>(blockIdx.y) * kMt,
                            static_cast<int>(blockIdx.x) * kMt, item, red);
}

// The two products of a recursion node that both follow P, in one launch:
// A_TT -= P P^T (upper tiles; workgroups [0, tiles0)) and Q = P W_SS (the
// rest). They read P and write disjoint memory.
__global__ void __launch_bounds__(256)
    dgemm_pair_kernel(GemmArgs g0, int nt0, int tiles0, GemmArgs g1, int nt1,
                      const uint8_t* __restrict__ active, const uint8_t* __restrict__ failed) {
  const int64_t item = blockIdx.z;
  if (!active[item] || failed[item]) return;
  __shared__ double red[4][4][4][64];
  const int t = static_cast<int>(blockIdx.x);
  if (t < tiles0)
    dgemm_tile<true, true>(g0, (t / nt0) * kMt, (t % nt0) * kMt, item, red);
  else
    dgemm_tile<false, false>(g1, ((t - tiles0) / nt1) * kMt, ((t - tiles0) % nt1) * kMt, item,
                             red);
}

// 64 x 64 output tiles for the large products (both edges >= kBigEdge): wave
// (wr, wc) computes its 32 x 32 quadrant as 2 x 2 MFMA blocks over the whole
// K, so there is no cross-wave reduction. Per 16-k chunk the workgroup stages
// A rows and op(B) columns (as rows, [n][k]) in LDS with 16-byte loads, the
// next chunk's loads in flight while the current one is multiplied (two LDS
// buffers, one barrier per chunk; a 32-k chunk is 32 MFMAs per wave, enough
// to cover the loads). Lane l of k-step (h, t) reads k = chunk + 16 h +
// 4(l/16) + t for both operands (t = 0..3), one 32-byte LDS read per
// operand row and h. The row stride of 34 doubles keeps eight consecutive
// rows on distinct banks.
constexpr int kBt = 64, kBk = 32, kBs = kBk + 2, kBigEdge = 768;

struct Big64Lds {
  double a[2][kBt][kBs];
  double b[2][kBt][kBs];
};

template <bool TRANSB, bool UPPER>
__device__ inline void dgemm64_tile(const GemmArgs& g, int m0, int n0, int64_t item,
                                    Big64Lds& s) {
  if (UPPER && (n0 >> 6) < (m0 >> 6)) return;  // uniform over the workgroup
  const double* Ab = g.A + item * g.sA;
  const double* Bb = g.B + item * g.sB;
  double* Cb = g.C + item * g.sC;
  const int M = g.M, N = g.N, K = g.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
  const int li = lane & 15, gq = lane >> 4;
  // staging: A rows (and op(B) rows when TRANSB) as thread t -> row t / 4,
  // k 8 (t % 4) .. + 7; op(B) when B is [K][N]: k t / 8, columns 8 (t % 8) .. + 7
  const int ar = tid >> 2, ak = 8 * (tid & 3);
  const int bk = tid >> 3, bn = 8 * (tid & 7);
  auto cnt4 = [](int left) { return left < 0 ? 0 : (left > 4 ? 4 : left); };
  auto fetch = [&](int kc, double (&va)[8], double (&vb)[8]) {
    const int m = m0 + ar;
    const double* pa = Ab + static_cast<int64_t>(m < M ? m : 0) * g.lda + kc + ak;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      load4(pa + 4 * h, 1, m < M ? cnt4(K - kc - ak - 4 * h) : 0,
            *reinterpret_cast<double(*)[4]>(&va[4 * h]));
    if (TRANSB) {
      const int n = n0 + ar;
      const double* pb = Bb + static_cast<int64_t>(n < N ? n : 0) * g.ldb + kc + ak;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        load4(pb + 4 * h, 1, n < N ? cnt4(K - kc - ak - 4 * h) : 0,
              *reinterpret_cast<double(*)[4]>(&vb[4 * h]));
    } else {
      const int k = kc + bk, n = n0 + bn;
      const double* pb = Bb + static_cast<int64_t>(k < K ? k : 0) * g.ldb + n;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        load4(pb + 4 * h, 1, k < K ? cnt4(N - n - 4 * h) : 0,
              *reinterpret_cast<double(*)[4]>(&vb[4 * h]));
    }
  };
  auto stage = [&](int buf, const double (&va)[8], const double (&vb)[8]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f64x2_t*>(&s.a[buf][ar][ak + 2 * q]) = f64x2_t{va[2 * q], va[2 * q + 1]};
    if (TRANSB) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f64x2_t*>(&s.b[buf][ar][ak + 2 * q]) = f64x2_t{vb[2 * q], vb[2 * q + 1]};
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) s.b[buf][bn + t][bk] = vb[t];
    }
  };
  f64x4_t acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f64x4_t{0.0, 0.0, 0.0, 0.0};
  const int nch = (K + kBk - 1) / kBk;
  double va[8], vb[8];
  fetch(0, va, vb);
  stage(0, va, vb);
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < nch;
    if (more) fetch((c + 1) * kBk, va, vb);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      double a[2][4], b[2][4];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const f64x2_t* pa =
            reinterpret_cast<const f64x2_t*>(&s.a[buf][wr + 16 * x + li][16 * h + 4 * gq]);
        const f64x2_t lo = pa[0], hi = pa[1];
        a[x][0] = lo.x, a[x][1] = lo.y, a[x][2] = hi.x, a[x][3] = hi.y;
        const f64x2_t* pb =
            reinterpret_cast<const f64x2_t*>(&s.b[buf][wc + 16 * x + li][16 * h + 4 * gq]);
        const f64x2_t blo = pb[0], bhi = pb[1];
        b[x][0] = blo.x, b[x][1] = blo.y, b[x][2] = bhi.x, b[x][3] = bhi.y;
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[x][t], b[y][t], acc[x][y], 0, 0, 0);
    }
    if (more) stage(buf ^ 1, va, vb);
    __syncthreads();
  }
  // result register r of lane l of block (x, y) = D[l/16 + 4r][l%16]
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int n = n0 + wc + 16 * y + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wr + 16 * x + gq + 4 * r;
        if (m < M && n < N) {
          double* p = Cb + static_cast<int64_t>(m) * g.ldc + n;
          *p = g.beta == 0.0 ? g.alpha * acc[x][y][r] : g.alpha * acc[x][y][r] + g.beta * *p;
        }
      }
    }
}

template <bool TRANSB, bool UPPER>
__global__ void __launch_bounds__(256)
    dgemm64_kernel(GemmArgs g, const uint8_t* __restrict__ active,
                   const uint8_t* __restrict__ failed) {
  const int64_t item = blockIdx.z;
  if (!active[item] || failed[item]) return;
  __shared__ __attribute__((aligned(16))) Big64Lds s;
  dgemm64_tile<TRANSB, UPPER>(g, static_cast<int>(blockIdx.y) * kBt,
                              static_cast<int>(blockIdx.x) * kBt, item, s);
}

__global__ void __launch_bounds__(256)
    dgemm64_pair_kernel(GemmArgs g0, int nt0, int tiles0, GemmArgs g1, int nt1,
                        const uint8_t* __restrict__ active, const uint8_t* __restrict__ failed) {
  const int64_t item = blockIdx.z;
  if (!active[item] || failed[item]) return;
  __shared__ __attribute__((aligned(16))) Big64Lds s;
  const int t = static_cast<int>(blockIdx.x);
  if (t < tiles0)
    dgemm64_tile<true, true>(g0, (t / nt0) * kBt, (t % nt0) * kBt, item, s);
  else
    dgemm64_tile<false, false>(g1, ((t - tiles0) / nt1) * kBt, ((t - tiles0) % nt1) * kBt,
                               item, s);
}

// U = fp32(W) (upper), zero below the diagonal, for items that succeeded.
__global__ void emit_u_kernel(const double* __restrict__ W, int64_t C,
                              const uint8_t* __restrict__ active,
                              const uint8_t* __restrict__ failed, float* __restrict__ U) {
  const int64_t b = blockIdx.y;
  if (!active[b] || failed[b]) return;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < C * C;
       e += (int64_t)gridDim.x * blockDim.x) {
    U[b * C * C + e] = (e / C <= e % C) ? static_cast<float>(W[b * C * C + e]) : 0.0f;
  }
}

// Workspace plan: A, W (B x C x C fp64 each), lam (B floats), P (largest
// top x bottom block product) and one Q slot per recursion depth.
struct Layout {
  int64_t lam_off, p_off, q_off[32], total;
  int64_t p_elems, q_elems[32];
};

void plan_sizes(int64_t b0, int64_t b1, int64_t C, int depth, Layout* L) {
  if (b1 - b0 <= 1) return;
  const int64_t mid = b0 + (b1 - b0) / 2;
  const int64_t r0 = b0 * kNb, rm = mid * kNb, r1 = std::min(b1 * kNb, C);
  const int64_t hs = (rm - r0) * (r1 - rm);
  L->p_elems = std::max(L->p_elems, hs);
  L->q_elems[depth] = std::max(L->q_elems[depth], hs);
  plan_sizes(mid, b1, C, depth + 1, L);
  plan_sizes(b0, mid, C, depth + 1, L);
}

Layout make_layout(int64_t B, int64_t C) {
  Layout L{};
  const int64_t nblk = ceil_div(C, kNb);
  plan_sizes(0, nblk, C, 0, &L);
  int64_t off = 2 * B * C * C * 8;
  L.lam_off = off;
  off += ceil_div(B * 4, 256) * 256;
  L.p_off = off;
  off += B * L.p_elems * 8;
  for (int d = 0; d < 32; ++d) {
    L.q_off[d] = off;
    off += B * L.q_elems[d] * 8;
  }
  L.total = off + 256;
  return L;
}

struct Ctx {
  double* A;
  double* W;
  double* P;
  double* Q[32];
  int64_t B, C;
  const uint8_t* active;
  uint8_t* failed;
  hipStream_t s;
};

GemmArgs gemm_args(const double* A, int64_t lda, int64_t sA, const double* Bm, int64_t ldb,
                   int64_t sB, double* Cm, int64_t ldc, int64_t sC, int64_t M, int64_t N,
                   int64_t K, double alpha, double beta) {
  return GemmArgs{A,  lda, sA, Bm, ldb, sB, Cm, ldc, sC, static_cast<int>(M), static_cast<int>(N),
                  static_cast<int>(K), alpha, beta};
}

bool big(const GemmArgs& g) { return g.M >= kBigEdge && g.N >= kBigEdge; }

template <bool TRANSB, bool UPPER = false>
int gemm(const Ctx& x, const GemmArgs& g) {
  if (big(g)) {
    dim3 grid(static_cast<unsigned>(ceil_div(g.N, kBt)), static_cast<unsigned>(ceil_div(g.M, kBt)),
              static_cast<unsigned>(x.B));
    dgemm64_kernel<TRANSB, UPPER><<<grid, 256, 0, x.s>>>(g, x.active, x.failed);
  } else {
    dim3 grid(static_cast<unsigned>(ceil_div(g.N, kMt)), static_cast<unsigned>(ceil_div(g.M, kMt)),
              static_cast<unsigned>(x.B));
    dgemm_kernel<TRANSB, UPPER><<<grid, 256, 0, x.s>>>(g, x.active, x.failed);
  }
  return check_launch("hinv gemm");
}

// g0 with TRANSB and UPPER, g1 plain, in one launch
int gemm_pair(const Ctx& x, const GemmArgs& g0, const GemmArgs& g1) {
  const bool b64 = big(g0) && big(g1);
  const int64_t t = b64 ? kBt : kMt;
  const int nt0 = static_cast<int>(ceil_div(g0.N, t));
  const int tiles0 = nt0 * static_cast<int>(ceil_div(g0.M, t));
  const int nt1 = static_cast<int>(ceil_div(g1.N, t));
  const int tiles1 = nt1 * static_cast<int>(ceil_div(g1.M, t));
  dim3 grid(static_cast<unsigned>(tiles0 + tiles1), 1, static_cast<unsigned>(x.B));
  if (b64)
    dgemm64_pair_kernel<<<grid, 256, 0, x.s>>>(g0, nt0, tiles0, g1, nt1, x.active, x.failed);
  else
    dgemm_pair_kernel<<<grid, 256, 0, x.s>>>(g0, nt0, tiles0, g1, nt1, x.active, x.failed);
  return check_launch("hinv gemm pair");
}

int factor_rec(const Ctx& x, int64_t b0, int64_t b1, int depth) {
  const int64_t C = x.C, CC = C * C;
  const int64_t r0 = b0 * kNb, r1 = std::min(b1 * kNb, C);
  if (b1 - b0 == 1) {
    leaf_kernel<<<static_cast<unsigned>(x.B), 256, 0, x.s>>>(x.A, x.W, C, r0,
                                                            static_cast<int>(r1 - r0), x.active,
                                                            x.failed);
    return check_launch("hinv leaf");
  }
  const int64_t mid = b0 + (b1 - b0) / 2;
  const int64_t rm = mid * kNb, h = rm - r0, s2 = r1 - rm;
  if (int rc = factor_rec(x, mid, b1, depth + 1)) return rc;
  const double* Wss = x.W + rm * C + rm;
  // P = A_TS W_SS^T
  if (int rc = gemm<true>(x, gemm_args(x.A + r0 * C + rm, C, CC, Wss, C, CC, x.P, s2, h * s2, h,
                                       s2, s2, 1.0, 0.0)))
    return rc;
  // A_TT -= P P^T (upper tiles) and Q = P W_SS
  double* Q = x.Q[depth];
  if (int rc = gemm_pair(x,
                         gemm_args(x.P, s2, h * s2, x.P, s2, h * s2, x.A + r0 * C + r0, C, CC, h,
                                   h, s2, -1.0, 1.0),
                         gemm_args(x.P, s2, h * s2, Wss, C, CC, Q, s2, h * s2, h, s2, s2, 1.0,
                                   0.0)))
    return rc;
  if (int rc = factor_rec(x, b0, mid, depth + 1)) return rc;
  // W_TS = -W_TT Q
  return gemm<false>(x, gemm_args(x.W + r0 * C + r0, C, CC, Q, s2, h * s2, x.W + r0 * C + rm, C,
                                  CC, h, s2, h, -1.0, 0.0));
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int64_t mgq_hinv_full_workspace_size(int64_t B, int64_t C) {
  if (B < 0 || C < 1) return 0;
  return make_layout(B, C).total;
}

// One factorisation pass for the items with active[b] != 0, using per-item
// damp[b]; failed[b] (device, cleared by the caller) reports pivot failure.
extern "C" int mgq_hinv_full_pass(const float* H, int64_t B, int64_t C, const float* damp,
                                  const uint8_t* active, uint8_t* failed, float* U,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  MGQ_REQUIRE(B >= 0 && C >= 1, MGQ_ERR_SHAPE, "bad shape");
  const Layout L = make_layout(B, C);
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, MGQ_ERR_WORKSPACE,
              "hinv workspace too small");
  if (B == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  Ctx x;
  x.A = reinterpret_cast<double*>(ws);
  x.W = x.A + B * C * C;
  x.P = reinterpret_cast<double*>(ws + L.p_off);
  for (int d = 0; d < 32; ++d) x.Q[d] = reinterpret_cast<double*>(ws + L.q_off[d]);
  x.B = B;
  x.C = C;
  x.active = active;
  x.failed = failed;
  x.s = s;
  float* lam = reinterpret_cast<float*>(ws + L.lam_off);
  const unsigned gb = static_cast<unsigned>(B);
  lam_kernel<<<gb, 256, 0, s>>>(H, C, damp, active, lam);
  if (int rc = check_launch("hinv lam")) return rc;
  build_kernel<<<dim3(std::min<unsigned>(elementwise_blocks(C * C, 256), 1024u), gb), 256, 0, s>>>(
      H, C, lam, active, x.A, x.W);
  if (int rc = check_launch("hinv build")) return rc;
  if (int rc = factor_rec(x, 0, ceil_div(C, kNb), 0)) return rc;
  emit_u_kernel<<<dim3(std::min<unsigned>(elementwise_blocks(C * C, 256), 1024u), gb), 256, 0, s>>>(
      x.W, C, active, failed, U);
  return check_launch("hinv emit");
}
