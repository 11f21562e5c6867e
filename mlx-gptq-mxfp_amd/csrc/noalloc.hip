// Allocation-free MXFP GPTQ solve: mgq_gptq_mxfp with its workspace taken
// from a fixed device array instead of a caller-provided buffer, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).
//
// The array `scratch` is a file-scope __device__ object: every GPU the
// library runs on holds its own copy (kNoAllocScratchBytes) from the moment
// this code object is loaded on it until the process ends. Its host-side
// name is only a stand-in for the symbol, so host code never passes it to a
// kernel: the device address comes from hipGetSymbolAddress, looked up once
// per device (with that device current) and cached. All calls on one GPU
// share that GPU's array, so calls that overlap on one GPU (two streams, two
// threads) race; serialise them. Nothing in the array needs clearing: the
// solver writes every region (dead-column flags, U and H blocks, rel_err
// partials) before it reads it.
#include <mutex>

#include "mgq_capi.h"

namespace mgq {
namespace {

constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;  // 32 MiB per GPU
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's `scratch` (the current device's), looked up
// on the first call on that device.
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  MGQ_REQUIRE(dev >= 0 && dev < kMaxDevices, MGQ_ERR_VALUE, "device %d outside [0, %d)", dev,
              kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "hipGetSymbolAddress(scratch)"))
      return rc;
    MGQ_REQUIRE(p != nullptr, MGQ_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MGQ_OK;
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int64_t mgq_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int mgq_gptq_mxfp_noalloc(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C,
                                     float* H, int mode, int algorithm, float damp,
                                     int max_attempts, const int32_t* offsets, int n_offsets,
                                     uint8_t* q_out, uint8_t* scales_out, float* W_dq,
                                     float* rel_err, int32_t* attempts, void* stream) {
  clear_error();
  MGQ_REQUIRE(B >= 0 && R >= 0 && C >= 0, MGQ_ERR_SHAPE, "bad shape");
  const int64_t need = mgq_gptq_mxfp_workspace_size(B, R, C);
  MGQ_REQUIRE(need <= kNoAllocScratchBytes, MGQ_ERR_WORKSPACE,
              "mgq_gptq_mxfp_noalloc: [B=%lld, R=%lld, C=%lld] needs %lld bytes of scratch, more "
              "than the %lld-byte per-GPU array; split the batch or use mgq_gptq_mxfp",
              (long long)B, (long long)R, (long long)C, (long long)need,
              (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return mgq_gptq_mxfp(W, w_dtype, B, R, C, H, mode, algorithm, damp, max_attempts, offsets,
                       n_offsets, q_out, scales_out, W_dq, rel_err, attempts, ws,
                       kNoAllocScratchBytes, stream);
}
