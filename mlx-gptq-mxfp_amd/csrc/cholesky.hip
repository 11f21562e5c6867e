// Damped Cholesky-inverse upper factors (gptq.py:27-66, _prepare_hinv).
//
// For every square diagonal block Hb of size n (n = 32: the per-group blocks
// of the MXFP solver, gptq.py:99-100) compute the upper-triangular U with
//     U^T U = (Hb + lam I)^-1,   lam = damp * max(mean(diag Hb), 1e-8),
// escalating damp *= 10 (fp32, per block) until the factorisation succeeds,
// at most max_attempts times, exactly as the reference escalates failed batch
// items. Hd = Hb + lam I is formed in fp32 as the reference does; the
// factorisation and inverse run in fp64 and are rounded to fp32 once, so U
// is the correctly rounded factor up to fp64 error.
//
// Method (one wavefront per block, fp64 in LDS): factor Hd = V V^T with V
// upper triangular (Cholesky in reverse index order); then
// (Hd)^-1 = V^-T V^-1 = W^T W with W = V^-1 upper, and by uniqueness of the
// Cholesky factor U = W. This needs one factorisation and one triangular
// inverse instead of the reference's factor / invert / re-factor sequence.
// A pivot <= 0 or NaN fails the attempt (LAPACK potrf semantics).
#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

constexpr int kN = 32;

// attempts[g*B + b]: 1..max_attempts on success, 0 if every attempt failed.
// sym[b*G + g] (optional): 1 when the undamped block is exactly symmetric.
// Hc (optional): compact [B*G][32][32] copy of each undamped block.
__global__ void __launch_bounds__(64)
    hinv32_kernel(const float* __restrict__ H, int64_t B, int64_t C, float damp,
                  int max_attempts, float* __restrict__ U, int32_t* __restrict__ attempts,
                  uint8_t* __restrict__ sym, float* __restrict__ Hc) {
  __shared__ double A[kN][kN + 1];
  __shared__ double Wm[kN][kN + 1];
  const int64_t G = C / kN;
  const int64_t b = blockIdx.x / G;
  const int64_t g = blockIdx.x % G;
  const int lane = threadIdx.x;
  const float* Hb = H + b * C * C + (g * kN) * C + g * kN;

  // diag mean (fp64 sum, rounded once) clamped like torch .clamp(min=1e-8)
  double dsum = 0.0;
  for (int i = 0; i < kN; ++i) dsum += static_cast<double>(Hb[static_cast<int64_t>(i) * C + i]);
  float dmean = static_cast<float>(dsum / kN);
  dmean = (dmean < 1e-8f) ? 1e-8f : dmean;  // NaN stays NaN

  if (Hc) {
    float* dst = Hc + (b * G + g) * kN * kN;
    for (int e = lane; e < kN * kN; e += 64) dst[e] = Hb[static_cast<int64_t>(e / kN) * C + e % kN];
  }
  if (sym) {
    bool same = true;
    for (int e = lane; e < kN * kN; e += 64) {
      const int i = e / kN, j = e % kN;
      same = same && (__float_as_uint(Hb[static_cast<int64_t>(i) * C + j]) ==
                      __float_as_uint(Hb[static_cast<int64_t>(j) * C + i]));
    }
    const bool all_same = __all(same);
    if (lane == 0) sym[b * G + g] = all_same ? 1 : 0;
  }

  float cur = damp;
  int used = 0;
  for (int att = 1; att <= max_attempts; ++att) {
    const float lam = dmean * cur;
    // Hd in fp32 (diag += lam), widened to fp64
    for (int e = lane; e < kN * kN; e += 64) {
      const int i = e / kN, j = e % kN;
      float v = Hb[static_cast<int64_t>(i) * C + j];
      if (i == j) v = v + lam;
      A[i][j] = static_cast<double>(v);
    }
    __syncthreads();
    bool ok = true;
    for (int j = kN - 1; j >= 0; --j) {
      const double d = A[j][j];
      if (!(d > 0.0)) {  // uniform: every lane reads the same pivot
        ok = false;
        break;
      }
      const double s = sqrt(d);
      __syncthreads();
      if (lane < j) A[lane][j] = A[lane][j] / s;
      if (lane == 0) A[j][j] = s;
      __syncthreads();
      // trailing update of the leading j x j block, upper part:
      // A[i][k] -= V[i][j] * V[k][j] for i <= k < j
      const int i = lane & 31;
      if (i < j) {
        const double vi = A[i][j];
        for (int k = i + (lane >> 5); k < j; k += 2) A[i][k] = A[i][k] - vi * A[k][j];
      }
      __syncthreads();
    }
    if (ok) {
      used = att;
      break;
    }
    cur = cur * 10.0f;
    __syncthreads();
  }
  float* Ub = U + (b * G + g) * kN * kN;
  if (used == 0) {
    for (int e = lane; e < kN * kN; e += 64) Ub[e] = 0.0f;
    if (lane == 0) attempts[g * B + b] = 0;
    return;
  }
  // W = V^-1 (upper): lane j back-substitutes column j.
  if (lane < kN) {
    const int j = lane;
    Wm[j][j] = 1.0 / A[j][j];
    for (int i = j - 1; i >= 0; --i) {
      double s = 0.0;
      for (int k = i + 1; k <= j; ++k) s += A[i][k] * Wm[k][j];
      Wm[i][j] = -s / A[i][i];
    }
  }
  __syncthreads();
  for (int e = lane; e < kN * kN; e += 64) {
    const int i = e / kN, j = e % kN;
    Ub[e] = (i <= j) ? static_cast<float>(Wm[i][j]) : 0.0f;
  }
  if (lane == 0) attempts[g * B + b] = used;
}

}  // namespace

// Launch helper shared with the MXFP solver.
int launch_hinv32(const float* H, int64_t B, int64_t C, float damp, int max_attempts, float* U,
                  int32_t* attempts, uint8_t* sym, float* Hc, hipStream_t s) {
  const int64_t G = C / kN;
  if (B * G == 0) return MGQ_OK;
  hinv32_kernel<<<static_cast<unsigned>(B * G), 64, 0, s>>>(H, B, C, damp, max_attempts, U,
                                                          attempts, sym, Hc);
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
  return launch_hinv32(H, B, C, damp, max_attempts, U, attempts, nullptr, nullptr,
                       as_stream(stream));
}
