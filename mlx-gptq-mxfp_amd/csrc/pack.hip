// Code packing into the MLX layouts: uint32 words, LSB-first, 32/bits codes
// per word (packing.py:15-39) and nibble bytes, low nibble first
// (artifacts.py:30-39). Pure HBM streaming: each thread moves 16 output
// bytes with vector loads/stores when the buffers are 16-byte aligned.
#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

constexpr int kThreads = 256;

// word = OR_i (uint32)q[per*w + i] << (bits*i), uint32 arithmetic (no mask),
// exactly the numpy loop of packing.py:22-25.
template <int BITS>
__device__ inline uint32_t pack_word(const uint8_t* p) {
  constexpr int per = 32 / BITS;
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < per; ++i) w |= static_cast<uint32_t>(p[i]) << (BITS * i);
  return w;
}

template <int BITS>
__device__ inline uint32_t pack_word_from_u32(const uint32_t* v) {
  // v holds 32/BITS bytes as little-endian uint32 chunks.
  constexpr int per = 32 / BITS;
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < per; ++i) {
    const uint32_t byte = (v[i >> 2] >> (8 * (i & 3))) & 0xffu;
    w |= byte << (BITS * i);
  }
  return w;
}

// Vector path: each thread emits 4 consecutive words (16 bytes) from
// 4*per consecutive codes (4*per bytes = 64 / 32 / 16 bytes).
template <int BITS>
__global__ void pack_q_vec_kernel(const uint8_t* __restrict__ q, int64_t n_quads,
                                  uint32_t* __restrict__ words) {
  constexpr int per = 32 / BITS;
  constexpr int in_u4 = per / 4;  // uint4 loads per thread (4 words * per bytes / 16)
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n_quads;
       t += (int64_t)gridDim.x * blockDim.x) {
    const uint4* src = reinterpret_cast<const uint4*>(q + t * 4 * per);
    uint32_t v[4 * per / 4];
#pragma unroll
    for (int k = 0; k < in_u4; ++k) {
      const uint4 x = src[k];
      v[4 * k + 0] = x.x;
      v[4 * k + 1] = x.y;
      v[4 * k + 2] = x.z;
      v[4 * k + 3] = x.w;
    }
    uint4 out;
    out.x = pack_word_from_u32<BITS>(v + 0 * (per / 4));
    out.y = pack_word_from_u32<BITS>(v + 1 * (per / 4));
    out.z = pack_word_from_u32<BITS>(v + 2 * (per / 4));
    out.w = pack_word_from_u32<BITS>(v + 3 * (per / 4));
    reinterpret_cast<uint4*>(words)[t] = out;
  }
}

template <int BITS>
__global__ void pack_q_kernel(const uint8_t* __restrict__ q, int64_t n_words, int64_t first,
                              uint32_t* __restrict__ words) {
  constexpr int per = 32 / BITS;
  for (int64_t w = first + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < n_words;
       w += (int64_t)gridDim.x * blockDim.x) {
    words[w] = pack_word<BITS>(q + w * per);
  }
}

__global__ void unpack_q_kernel(const uint32_t* __restrict__ words, int64_t rows,
                                int64_t n_words, int bits, int64_t out_cols,
                                uint8_t* __restrict__ q) {
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t n = rows * out_cols;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / out_cols, c = i - r * out_cols;
    const uint32_t w = words[r * n_words + c / per];
    q[i] = static_cast<uint8_t>((w >> (bits * (c % per))) & mask);
  }
}

// 16 codes -> 8 bytes per step; lo | (hi << 4) in uint8 arithmetic.
__global__ void pack_nibbles_vec_kernel(const uint8_t* __restrict__ q, int64_t n_chunks,
                                        uint8_t* __restrict__ out) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < n_chunks;
       t += (int64_t)gridDim.x * blockDim.x) {
    const uint4 x = reinterpret_cast<const uint4*>(q)[t];
    const uint32_t in[4] = {x.x, x.y, x.z, x.w};
    uint32_t o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t acc = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t src = in[2 * h + (k >> 1)];
        const uint32_t lo = (src >> (16 * (k & 1))) & 0xffu;
        const uint32_t hi = (src >> (16 * (k & 1) + 8)) & 0xffu;
        acc |= ((lo | (hi << 4)) & 0xffu) << (8 * k);
      }
      o[h] = acc;
    }
    reinterpret_cast<uint2*>(out)[t] = make_uint2(o[0], o[1]);
  }
}

__global__ void pack_nibbles_kernel(const uint8_t* __restrict__ q, int64_t n_out, int64_t first,
                                    uint8_t* __restrict__ out) {
  for (int64_t i = first + blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_out;
       i += (int64_t)gridDim.x * blockDim.x) {
    out[i] = static_cast<uint8_t>(q[2 * i] | (q[2 * i + 1] << 4));
  }
}

__global__ void unpack_nibbles_kernel(const uint8_t* __restrict__ p, int64_t n_in,
                                      uint8_t* __restrict__ q) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_in;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t b = p[i];
    q[2 * i] = static_cast<uint8_t>(b & 0xfu);
    q[2 * i + 1] = static_cast<uint8_t>(b >> 4);
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int BITS>
int launch_pack(const uint8_t* q, int64_t n_words, uint32_t* words, hipStream_t s) {
  constexpr int per = 32 / BITS;
  int64_t done = 0;
  if (aligned16(q) && aligned16(words)) {
    const int64_t quads = n_words / 4;
    if (quads > 0) {
      pack_q_vec_kernel<BITS><<<elementwise_blocks(quads, kThreads), kThreads, 0, s>>>(
          q, quads, words);
      done = quads * 4;
    }
  }
  if (done < n_words) {
    pack_q_kernel<BITS><<<elementwise_blocks(n_words - done, kThreads), kThreads, 0, s>>>(
        q, n_words, done, words);
  }
  (void)per;
  return check_launch("pack_q");
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int mgq_pack_q(const uint8_t* q, int64_t rows, int64_t cols, int bits,
                          uint32_t* words, void* stream) {
  clear_error();
  MGQ_REQUIRE(bits == 2 || bits == 4 || bits == 8, MGQ_ERR_VALUE,
              "cannot pack %d-bit for MLX (supported: (2, 4, 8))", bits);
  const int per = 32 / bits;
  MGQ_REQUIRE(rows >= 0 && cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(cols % per == 0, MGQ_ERR_SHAPE, "last dim %lld not divisible by %d",
              (long long)cols, per);
  const int64_t n_words = rows * (cols / per);
  if (n_words == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  if (bits == 2) return launch_pack<2>(q, n_words, words, s);
  if (bits == 4) return launch_pack<4>(q, n_words, words, s);
  return launch_pack<8>(q, n_words, words, s);
}

extern "C" int mgq_unpack_q(const uint32_t* words, int64_t rows, int64_t n_words, int bits,
                            int64_t out_cols, uint8_t* q, void* stream) {
  clear_error();
  MGQ_REQUIRE(bits == 1 || bits == 2 || bits == 4 || bits == 8 || bits == 16, MGQ_ERR_VALUE,
              "cannot unpack %d-bit", bits);
  MGQ_REQUIRE(rows >= 0 && n_words >= 0 && out_cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(out_cols <= n_words * (32 / bits), MGQ_ERR_SHAPE,
              "out_cols %lld exceeds %lld packed values", (long long)out_cols,
              (long long)(n_words * (32 / bits)));
  const int64_t n = rows * out_cols;
  if (n == 0) return MGQ_OK;
  unpack_q_kernel<<<elementwise_blocks(n, kThreads), kThreads, 0, as_stream(stream)>>>(
      words, rows, n_words, bits, out_cols, q);
  return check_launch("unpack_q");
}

extern "C" int mgq_pack_nibbles(const uint8_t* q, int64_t rows, int64_t cols, uint8_t* packed,
                                void* stream) {
  clear_error();
  MGQ_REQUIRE(rows >= 0 && cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  MGQ_REQUIRE(cols % 2 == 0, MGQ_ERR_SHAPE, "last dim %lld is odd", (long long)cols);
  const int64_t n_out = rows * (cols / 2);
  if (n_out == 0) return MGQ_OK;
  hipStream_t s = as_stream(stream);
  int64_t done = 0;
  if (aligned16(q) && (reinterpret_cast<uintptr_t>(packed) & 7u) == 0) {
    const int64_t chunks = n_out / 8;
    if (chunks > 0) {
      pack_nibbles_vec_kernel<<<elementwise_blocks(chunks, kThreads), kThreads, 0, s>>>(
          q, chunks, packed);
      done = chunks * 8;
    }
  }
  if (done < n_out) {
    pack_nibbles_kernel<<<elementwise_blocks(n_out - done, kThreads), kThreads, 0, s>>>(
        q, n_out, done, packed);
  }
  return check_launch("pack_nibbles");
}

extern "C" int mgq_unpack_nibbles(const uint8_t* packed, int64_t rows, int64_t packed_cols,
                                  uint8_t* q, void* stream) {
  clear_error();
  MGQ_REQUIRE(rows >= 0 && packed_cols >= 0, MGQ_ERR_SHAPE, "bad shape");
  const int64_t n_in = rows * packed_cols;
  if (n_in == 0) return MGQ_OK;
  unpack_nibbles_kernel<<<elementwise_blocks(n_in, kThreads), kThreads, 0, as_stream(stream)>>>(
      packed, n_in, q);
  return check_launch("unpack_nibbles");
}
