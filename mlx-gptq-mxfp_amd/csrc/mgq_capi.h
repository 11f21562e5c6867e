// Host-side plumbing for the C-ABI entry points: status codes, a per-thread
// last-error message, and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/mlx_gptq_amd.h"

namespace mgq {

void set_error(const char* fmt, ...);
void clear_error();

// Map the error of the last kernel launch (or any HIP call) to a status.
int check_launch(const char* what);
int check_hip(hipError_t e, const char* what);

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Grid size for a grid-stride elementwise kernel of `n` items.
inline unsigned elementwise_blocks(int64_t n, int threads) {
  int64_t b = (n + threads - 1) / threads;
  if (b < 1) b = 1;
  if (b > 65536 * 4) b = 65536 * 4;
  return static_cast<unsigned>(b);
}

}  // namespace mgq

#define MGQ_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      ::mgq::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)
