// Hessian accumulation H_g = X_g^T X_g (capture.py:68-76) as a grouped bf16
// MFMA SYRK with fp32 accumulation.
//
// One launch covers any number of groups (one dense linear, or every routed
// expert of a layer). Group g owns tokens [k_begin, k_end) of a token list;
// token t reads row `row_index ? row_index[t] : t` of X, so the routed-expert
// gather is fused into the tile loads. Only the lower triangle of 256x256
// output tiles is computed; each tile is mirrored on store, so H is exactly
// symmetric.
//
// Tile kernel (256 threads = 4 waves, 1 workgroup per CU):
//   - output tile 256x256, each wave 128x128 = 4x4 blocks of
//     v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane, in AGPRs);
//   - token rows are copied HBM -> LDS by global_load_lds_dwordx4 with a
//     scalar (SGPR) row address per token, so the gather costs no vector
//     work; MFMA operands are read with ds_read_b64_tr_b16 transposing loads
//     from the token-major LDS rows (see syrk_dma_kernel);
//   - one work item accumulates at most 262144 tokens in the MFMA fp32
//     accumulators (longer token ranges are split into partial tiles), which
//     bounds the accumulation chain well inside the 1e-5 Frobenius budget.
// Work items are planned on the host (mgq_hessian_plan): groups are spread
// over the 8 XCDs by token load (LPT) and all tiles of a group stay on one
// XCD so its token rows are shared through that XCD's L2. Heavy groups are
// split along K into partial tiles summed in a fixed order by a second
// kernel, keeping H deterministic.
#include <string.h>

#include <algorithm>
#include <numeric>
#include <vector>

#include "mgq_capi.h"
#include "mgq_common.h"

namespace mgq {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTile = 256;
constexpr int kKs = 64;          // token granularity of work-item ranges
constexpr int kThreads = 256;
constexpr int64_t kMaxItemTokens = 262144;  // longest fp32 accumulation chain per item
constexpr int kXcds = 8;

struct HessItem {
  int32_t g;     // group, -1 = no-op padding
  int32_t ti;    // output tile row (>= tj)
  int32_t tj;
  int32_t slot;  // -1: write H directly; >= 0: partial tile slot
  int64_t k0;    // token range [k0, k1)
  int64_t k1;
};

struct SplitTile {
  int32_t g, ti, tj, slot0, nslots, pad;
};

struct PlanHeader {
  int64_t n_items;
  int64_t n_split;
  int64_t n_slots;
  int64_t C;
  int64_t n_groups;
  int64_t items_off;   // byte offsets inside the plan
  int64_t split_off;
  int64_t plan_bytes;
  int64_t k_end_max;  // offsets[n_groups]: token list length the plan reads
};

constexpr int64_t kAlign = 256;
inline int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
// A row of C bf16 zeros that tail tokens (past a work item's range) load.
inline int64_t zero_row_bytes(int64_t C) { return align_up(2 * C); }

// Flush the wave's 128x128 accumulators into `out` (row stride ld). Direct
// tiles (H_g, global coordinates) keep the lower triangle and
// mirror it; partial tiles (local 256x256 slot) are stored whole. Offsets are
// 32-bit (C*C < 2^31 is checked on the host) and the stride is kept in a
// VGPR so the 64 row offsets are formed per element instead of occupying
// scalar registers.
__device__ inline void flush(f32x16_t (&acc)[4][4], float* __restrict__ out, uint32_t ld_s,
                             bool direct, bool add, uint32_t C, uint32_t gi0, uint32_t gj0,
                             int lane, bool interior) {
  uint32_t ld;
  asm volatile("v_mov_b32 %0, %1" : "=v"(ld) : "s"(ld_s));
  const uint32_t gj_l = gj0 + (lane & 31);
  const uint32_t gi_l = gi0 + 4 * (lane >> 5);
  if (interior) {
    // Strictly-lower tile inside H: no masking. Registers 4q..4q+3 of a
    // block hold rows gi..gi+3 of one column gj, so the mirrored values are
    // 4 consecutive floats of row gj: one 16-byte store.
#pragma unroll
    for (int ma = 0; ma < 4; ++ma) {
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        const uint32_t gi = gi_l + ma * 32 + 8 * rq;
#pragma unroll
        for (int na = 0; na < 4; ++na) {
          const uint32_t gj = gj_l + na * 32;
          float nv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float* p = out + ((gi + e) * ld + gj);
            const float v = acc[ma][na][4 * rq + e];
            nv[e] = add ? (*p + v) : v;
            *p = nv[e];
          }
          const float4 m = {nv[0], nv[1], nv[2], nv[3]};
          *reinterpret_cast<float4*>(out + (gj * ld + gi)) = m;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int ma = 0; ma < 4; ++ma) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t gi = gi_l + ma * 32 + 8 * (r >> 2) + (r & 3);
      const uint32_t row_off = gi * ld;
#pragma unroll
      for (int na = 0; na < 4; ++na) {
        const uint32_t gj = gj_l + na * 32;
        const float v = acc[ma][na][r];
        if (direct) {
          if (gi < C && gj < C && gi >= gj) {
            float* p = out + (row_off + gj);
            const float nv = add ? (*p + v) : v;
            *p = nv;
            if (gi != gj) out[gj * ld + gi] = nv;
          }
        } else {
          float* p = out + (row_off + gj);
          *p = add ? (*p + v) : v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS SYRK (production kernel).
//
// Token rows go from HBM straight into LDS with global_load_lds_dwordx4 (no
// VGPR staging, no register transpose): one instruction moves one token's
// 256 A channels (lanes 0-31) and 256 B channels (lanes 32-63), 1 KB, with
// a 64-bit SGPR row address, so the routed gather costs scalar work only.
// LDS keeps token-major rows (as in HBM); MFMA operands (one channel x 8
// consecutive tokens per lane) come out of ds_read_b64_tr_b16, which hands
// lane i of each 16-lane group element i%4 of source lanes 4j + i/4, j=0..3:
// pointing source lane 4j+q at token j, channels 4q..4q+3 gives lane i
// channel i of tokens 0..3. Four 32-token stages are in flight; each wave
// waits for its own DMA of a stage (vmcnt) before the stage barrier. The
// 16-byte chunk index of LDS token row t is XORed with 4*(t & 3), so the 64
// bytes a transposed read takes from each of its 8 token rows land on four
// distinct 64-byte bank groups (two LDS cycles per read, no conflicts).
constexpr int kTokB = 1024;  // LDS bytes per token: A row | B row
#ifndef MGQ_SYRK_KB
#define MGQ_SYRK_KB 64  // tokens per LDS stage (one barrier each)
#endif
#ifndef MGQ_SYRK_NB
#define MGQ_SYRK_NB 2   // stage buffers (NB - 1 stages of DMA in flight)
#endif
constexpr int kDK = MGQ_SYRK_KB;
constexpr int kDBuf = MGQ_SYRK_NB;
constexpr int kStageB = kDK * kTokB;
constexpr int kDmaWave = kDK / 4;  // tokens (= DMA instructions) per wave and stage
static_assert(kDBuf * kStageB <= 160 * 1024, "LDS budget");
static_assert((kDBuf - 2) * kDmaWave <= 63, "vmcnt range");

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;
typedef __attribute__((address_space(3))) char lds_char_t;

__device__ inline void dma_row(uint32_t lds_dst, uint32_t voff, const void* saddr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_dst), "v"(voff), "s"(saddr)
               : "memory");
}

// Wait until at most N of this wave's DMA loads are outstanding and its LDS
// reads / scalar loads are done, then barrier.
template <int N>
__device__ inline void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "i"(N) : "memory");
}

// `ahead` stages of DMA (kDmaWave loads each) were issued after the stage
// being waited for; the count is an immediate, so dispatch on it.
__device__ inline void stage_barrier_ahead(int ahead) {
  if constexpr (kDBuf - 2 >= 3) {
    if (ahead >= 3) {
      stage_barrier<3 * kDmaWave>();
      return;
    }
  }
  if constexpr (kDBuf - 2 >= 2) {
    if (ahead >= 2) {
      stage_barrier<2 * kDmaWave>();
      return;
    }
  }
  if constexpr (kDBuf - 2 >= 1) {
    if (ahead >= 1) {
      stage_barrier<kDmaWave>();
      return;
    }
  }
  stage_barrier<0>();
}

__device__ inline bf16x8_t tr_frag(const lds_char_t* p) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 4 * kTokB));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

template <bool GATHER>
__device__ inline void stage_rows(const char* __restrict__ Xb, uint32_t ldx2, uint32_t n_rows,
                                  const int32_t* __restrict__ row_index, int64_t t0, int64_t k1,
                                  const char* zero_row, const char* (&src)[kDmaWave]) {
#pragma unroll
  for (int i = 0; i < kDmaWave; ++i) {
    const int64_t t = t0 + i;
    uint32_t row;
    if (GATHER) {
      const uint32_t r = static_cast<uint32_t>(row_index[t < k1 ? t : k1 - 1]);
      row = r < n_rows ? r : n_rows - 1;
    } else {
      row = static_cast<uint32_t>(t < k1 ? t : k1 - 1);
    }
    src[i] = t < k1 ? Xb + static_cast<uint64_t>(row) * ldx2 : zero_row;
  }
}

__device__ inline void issue_stage(uint32_t dst, const uint32_t (&voff)[4],
                                   const char* const (&src)[kDmaWave]) {
#pragma unroll
  for (int i = 0; i < kDmaWave; ++i) dma_row(dst + i * kTokB, voff[i & 3], src[i]);
}

template <bool GATHER>
__global__ void __launch_bounds__(kThreads, 1)
    syrk_dma_kernel(const uint16_t* __restrict__ X, int64_t n_rows, int64_t ldx, int64_t C,
                    const int32_t* __restrict__ row_index, const HessItem* __restrict__ items,
                    float* __restrict__ H, float* __restrict__ partials, int accumulate,
                    const uint16_t* __restrict__ zero_row) {
  __shared__ __attribute__((aligned(1024))) char lds[kDBuf * kStageB];

  const HessItem it = items[blockIdx.x];
  if (it.g < 0) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 1, wc = wave & 1;
  const bool diag = it.ti == it.tj;
  const bool direct = it.slot < 0;
  float* out = direct ? H + static_cast<int64_t>(it.g) * C * C
                      : partials + static_cast<int64_t>(it.slot) * kTile * kTile;
  const uint32_t ld = direct ? static_cast<uint32_t>(C) : kTile;
  const uint32_t gi0 = (direct ? static_cast<uint32_t>(it.ti) * kTile : 0u) + wr * 128;
  const uint32_t gj0 = (direct ? static_cast<uint32_t>(it.tj) * kTile : 0u) + wc * 128;

  // DMA lane role: slot (lane & 31) of the A (lane < 32) or B half of LDS
  // token row t holds chunk slot ^ 4*(t & 3); channels past C are clamped (they
  // only feed output rows / columns >= C, which are never stored). Diagonal
  // tiles load the A channels into both halves.
  const int half = lane >> 5;
  const int64_t tile_ch = static_cast<int64_t>(half && !diag ? it.tj : it.ti) * kTile;
  uint32_t voff[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int64_t ch = tile_ch + 8 * ((lane & 31) ^ (4 * f));
    voff[f] = static_cast<uint32_t>(2 * (ch < C - 8 ? ch : C - 8));
  }
  // Transposed-read lane role: group g = lane/16, source j = (lane/4)%4, q = lane%4.
  // Source j reads LDS token row 4r + j (+ 8, 16 multiples), so its swizzle is j.
  const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
  const uint32_t rd_lo = static_cast<uint32_t>((8 * (g >> 1) + j) * kTokB + (g & 1) * 32 +
                                               (q >> 1) * 16 + (q & 1) * 8);
  uint32_t offA[4], offB[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    offA[m] = rd_lo + wr * 256 + (m ^ j) * 64;
    offB[m] = rd_lo + 512 + wc * 256 + (m ^ j) * 64;
  }
  const lds_char_t* lds3 = (const lds_char_t*)lds;
  const uint32_t lds_u32 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds3));
  const uint32_t wave_dst = wave * kDmaWave * kTokB;

  f32x16_t acc[4][4];
#pragma unroll
  for (int ma = 0; ma < 4; ++ma)
#pragma unroll
    for (int na = 0; na < 4; ++na)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[ma][na][r] = 0.0f;

  const char* Xb = reinterpret_cast<const char*>(X);
  const char* zr = reinterpret_cast<const char*>(zero_row);
  const uint32_t ldx2 = static_cast<uint32_t>(2 * ldx);
  const uint32_t nr = static_cast<uint32_t>(n_rows);
  const int64_t k0 = it.k0, k1 = it.k1;
  const int n_stages = static_cast<int>((k1 - k0 + kDK - 1) / kDK);
  const int64_t twave = k0 + wave * kDmaWave;  // this wave's first token of stage 0

  const char* src[kDmaWave];
  // prologue: stages 0 .. kDBuf-2 in flight
#pragma unroll
  for (int p = 0; p < kDBuf - 1; ++p) {
    if (p < n_stages) {
      stage_rows<GATHER>(Xb, ldx2, nr, row_index, twave + p * kDK, k1, zr, src);
      issue_stage(lds_u32 + p * kStageB + wave_dst, voff, src);
    }
  }
  if (kDBuf - 1 < n_stages)
    stage_rows<GATHER>(Xb, ldx2, nr, row_index, twave + (kDBuf - 1) * kDK, k1, zr, src);

  int rbuf = 0, wbuf = kDBuf - 1;  // buffer of stage s, buffer of stage s + kDBuf - 1
  for (int s = 0; s < n_stages; ++s) {
    stage_barrier_ahead(n_stages - 1 - s);
    const uint32_t rd = static_cast<uint32_t>(rbuf * kStageB);
    bf16x8_t fa[2][4], fb[2][4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      fa[0][m] = tr_frag(lds3 + rd + offA[m]);
      fb[0][m] = tr_frag(lds3 + rd + offB[m]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < kDK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < kDK / 16) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          fa[cur ^ 1][m] = tr_frag(lds3 + rd + offA[m] + (ks + 1) * 16 * kTokB);
          fb[cur ^ 1][m] = tr_frag(lds3 + rd + offB[m] + (ks + 1) * 16 * kTokB);
        }
      }
      if (ks == 0 && s + kDBuf - 1 < n_stages) {
        // the buffer of stage s-1: every wave finished it before the barrier
        issue_stage(lds_u32 + wbuf * kStageB + wave_dst, voff, src);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ma = 0; ma < 4; ++ma)
#pragma unroll
        for (int na = 0; na < 4; ++na)
          acc[ma][na] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][ma], fb[cur][na],
                                                                acc[ma][na], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s + kDBuf < n_stages)
      stage_rows<GATHER>(Xb, ldx2, nr, row_index, twave + static_cast<int64_t>(s + kDBuf) * kDK,
                         k1, zr, src);
    rbuf = rbuf + 1 == kDBuf ? 0 : rbuf + 1;
    wbuf = wbuf + 1 == kDBuf ? 0 : wbuf + 1;
  }
  // Empty ranges (n_stages == 0) still flush, so an unrouted group gets H = 0.
  const bool interior =
      direct && it.ti > it.tj && (static_cast<int64_t>(it.ti) + 1) * kTile <= C;
  flush(acc, out, ld, direct, direct && accumulate, static_cast<uint32_t>(C), gi0, gj0, lane,
        interior);
}

__global__ void zero_fill_kernel(uint32_t* __restrict__ p, int64_t n_words) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_words;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Sum the K-split partial tiles of one output tile in slot order and write
// the lower triangle (+ mirror) of H.
__global__ void reduce_split_kernel(const SplitTile* __restrict__ tiles,
                                    const float* __restrict__ partials, float* __restrict__ H,
                                    int64_t C, int accumulate) {
  const SplitTile st = tiles[blockIdx.y];
  float* Hg = H + static_cast<int64_t>(st.g) * C * C;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < kTile * kTile;
       e += gridDim.x * blockDim.x) {
    const int li = e / kTile, lj = e % kTile;
    const int64_t gi = static_cast<int64_t>(st.ti) * kTile + li;
    const int64_t gj = static_cast<int64_t>(st.tj) * kTile + lj;
    if (gi >= C || gj >= C || gi < gj) continue;
    float v = partials[static_cast<int64_t>(st.slot0) * kTile * kTile + e];
    for (int s = 1; s < st.nslots; ++s)
      v += partials[static_cast<int64_t>(st.slot0 + s) * kTile * kTile + e];
    float* p = Hg + gi * C + gj;
    const float nv = accumulate ? (*p + v) : v;
    *p = nv;
    if (gi != gj) Hg[gj * C + gi] = nv;
  }
}

// ---------------------------------------------------------------------------
// Host planning.
// ---------------------------------------------------------------------------
struct Plan {
  PlanHeader hdr;
  std::vector<HessItem> items;
  std::vector<SplitTile> split;
};

int build_plan(int64_t C, int64_t n_groups, const int64_t* offsets, int64_t target_items,
               Plan* plan) {
  const int64_t nt = ceil_div(C, kTile);
  const int64_t T = nt * (nt + 1) / 2;
  std::vector<std::pair<int32_t, int32_t>> tiles;
  tiles.reserve(T);
  for (int32_t i = 0; i < nt; ++i)
    for (int32_t j = 0; j <= i; ++j) tiles.emplace_back(i, j);

  int64_t total_tokens = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t n = offsets[g + 1] - offsets[g];
    MGQ_REQUIRE(n >= 0, MGQ_ERR_SHAPE, "offsets must be non-decreasing (group %lld)",
                (long long)g);
    total_tokens += n;
  }
  if (target_items <= 0) target_items = 4 * 256;
  // K chunk per work item: balance the grid, never below 2048 tokens.
  const int64_t work = std::max<int64_t>(total_tokens, 1) * T;
  int64_t chunk = std::max<int64_t>(2048, ceil_div(work, target_items));
  chunk = std::min<int64_t>(chunk, kMaxItemTokens);
  chunk = ceil_div(chunk, kKs) * kKs;

  // Work units: a group's items (tiles x K splits) in tile order, cut into at
  // most 8 contiguous chunks of >= 32 items (one XCD has 32 CUs). Small groups
  // (one expert) stay whole on one XCD so their token rows are reused from
  // that XCD's L2; big dense groups spread over all XCDs. Chunks go to the
  // least-loaded XCD, heaviest first (LPT).
  struct Chunk {
    int64_t work;
    std::vector<HessItem> items;
  };
  std::vector<Chunk> chunks;
  int64_t n_slots = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t k0 = offsets[g], k1 = offsets[g + 1];
    const int64_t n = k1 - k0;
    const int64_t S = std::max<int64_t>(1, ceil_div(n, chunk));
    const int64_t per = ceil_div(ceil_div(std::max<int64_t>(n, 1), S), kKs) * kKs;
    std::vector<HessItem> gi;
    for (const auto& t : tiles) {
      if (S == 1) {
        gi.push_back(HessItem{static_cast<int32_t>(g), t.first, t.second, -1, k0, k1});
      } else {
        const int32_t slot0 = static_cast<int32_t>(n_slots);
        int32_t ns = 0;
        for (int64_t a = k0; a < k1; a += per, ++ns) {
          gi.push_back(HessItem{static_cast<int32_t>(g), t.first, t.second,
                                static_cast<int32_t>(n_slots++), a, std::min(a + per, k1)});
        }
        plan->split.push_back(SplitTile{static_cast<int32_t>(g), t.first, t.second, slot0, ns, 0});
      }
    }
    const int64_t n_items = static_cast<int64_t>(gi.size());
    const int64_t parts = std::min<int64_t>(kXcds, std::max<int64_t>(1, n_items / 32));
    const int64_t step = ceil_div(n_items, parts);
    for (int64_t a = 0; a < n_items; a += step) {
      Chunk c;
      c.items.assign(gi.begin() + a, gi.begin() + std::min(a + step, n_items));
      c.work = 0;
      for (const auto& it : c.items) c.work += std::max<int64_t>(it.k1 - it.k0, 1);
      chunks.push_back(std::move(c));
    }
  }
  std::stable_sort(chunks.begin(), chunks.end(),
                   [](const Chunk& a, const Chunk& b) { return a.work > b.work; });
  std::vector<std::vector<HessItem>> bins(kXcds);
  std::vector<int64_t> load(kXcds, 0);
  for (auto& c : chunks) {
    const int x = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += c.work;
    bins[x].insert(bins[x].end(), c.items.begin(), c.items.end());
  }
  size_t longest = 0;
  for (auto& b : bins) longest = std::max(longest, b.size());
  plan->items.clear();
  plan->items.reserve(longest * kXcds);
  for (size_t j = 0; j < longest; ++j)
    for (int x = 0; x < kXcds; ++x)
      plan->items.push_back(j < bins[x].size() ? bins[x][j] : HessItem{-1, 0, 0, -1, 0, 0});
  // trailing all-padding rows are dropped by construction (longest bin)

  PlanHeader& h = plan->hdr;
  h.n_items = static_cast<int64_t>(plan->items.size());
  h.n_split = static_cast<int64_t>(plan->split.size());
  h.n_slots = n_slots;
  h.C = C;
  h.n_groups = n_groups;
  h.items_off = align_up(sizeof(PlanHeader));
  h.split_off = align_up(h.items_off + h.n_items * static_cast<int64_t>(sizeof(HessItem)));
  h.plan_bytes = align_up(h.split_off + h.n_split * static_cast<int64_t>(sizeof(SplitTile)));
  h.k_end_max = offsets[n_groups];
  return MGQ_OK;
}

}  // namespace
}  // namespace mgq

using namespace mgq;

extern "C" int mgq_hessian_plan(int64_t C, int64_t n_groups, const int64_t* offsets,
                                int64_t target_items, void* plan, int64_t plan_capacity,
                                int64_t* plan_bytes, int64_t* workspace_bytes) {
  clear_error();
  MGQ_REQUIRE(C >= 1 && n_groups >= 1, MGQ_ERR_SHAPE, "bad Hessian shape C=%lld groups=%lld",
              (long long)C, (long long)n_groups);
  MGQ_REQUIRE(offsets != nullptr, MGQ_ERR_VALUE, "offsets required");
  Plan p;
  if (int rc = build_plan(C, n_groups, offsets, target_items, &p)) return rc;
  const int64_t need = p.hdr.plan_bytes;
  if (plan_bytes) *plan_bytes = need;
  if (workspace_bytes)
    *workspace_bytes = need + zero_row_bytes(C) + p.hdr.n_slots * static_cast<int64_t>(kTile) * kTile * 4;
  if (plan == nullptr) return MGQ_OK;  // size query
  MGQ_REQUIRE(plan_capacity >= need, MGQ_ERR_WORKSPACE, "plan buffer %lld < %lld bytes",
              (long long)plan_capacity, (long long)need);
  char* base = static_cast<char*>(plan);
  ::memset(base, 0, need);
  ::memcpy(base, &p.hdr, sizeof(PlanHeader));
  ::memcpy(base + p.hdr.items_off, p.items.data(), p.items.size() * sizeof(HessItem));
  ::memcpy(base + p.hdr.split_off, p.split.data(), p.split.size() * sizeof(SplitTile));
  return MGQ_OK;
}

extern "C" int mgq_hessian(const void* X, int64_t n_rows, int64_t ldx, int64_t C,
                           const int32_t* row_index, const void* plan_host, float* H, int accumulate, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  clear_error();
  MGQ_REQUIRE(plan_host != nullptr, MGQ_ERR_VALUE, "plan required (mgq_hessian_plan)");
  PlanHeader h;
  ::memcpy(&h, plan_host, sizeof(PlanHeader));
  MGQ_REQUIRE(h.C == C, MGQ_ERR_VALUE, "plan was built for C=%lld, got %lld", (long long)h.C,
              (long long)C);
  MGQ_REQUIRE(C % 8 == 0 && ldx % 8 == 0 && ldx >= C, MGQ_ERR_SHAPE,
              "hessian: C (%lld) and the row stride (%lld) must be multiples of 8",
              (long long)C, (long long)ldx);
  MGQ_REQUIRE((reinterpret_cast<uintptr_t>(X) & 15u) == 0, MGQ_ERR_SHAPE,
              "hessian: X must be 16-byte aligned");
  MGQ_REQUIRE(n_rows >= 1 || h.k_end_max == 0, MGQ_ERR_SHAPE, "hessian: X has no rows");
  MGQ_REQUIRE(row_index != nullptr || h.k_end_max <= n_rows, MGQ_ERR_SHAPE,
              "hessian: offsets reach token %lld but X has %lld rows", (long long)h.k_end_max,
              (long long)n_rows);
  MGQ_REQUIRE(C <= 46340, MGQ_ERR_SHAPE, "hessian: C=%lld exceeds 46340 (C*C >= 2^31)",
              (long long)C);
  const int64_t zbytes = zero_row_bytes(C);
  const int64_t need = h.plan_bytes + zbytes + h.n_slots * static_cast<int64_t>(kTile) * kTile * 4;
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= need, MGQ_ERR_WORKSPACE,
              "hessian workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)need);
  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  const HessItem* items = reinterpret_cast<const HessItem*>(ws + h.items_off);
  const SplitTile* split = reinterpret_cast<const SplitTile*>(ws + h.split_off);
  uint16_t* zero_row = reinterpret_cast<uint16_t*>(ws + h.plan_bytes);
  float* partials = reinterpret_cast<float*>(ws + h.plan_bytes + zbytes);
  if (h.n_items > 0) {
    zero_fill_kernel<<<1, 256, 0, s>>>(reinterpret_cast<uint32_t*>(zero_row), zbytes / 4);
    if (int rc = check_launch("hessian zero row")) return rc;
    if (row_index) {
      syrk_dma_kernel<true><<<static_cast<unsigned>(h.n_items), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(X), n_rows, ldx, C, row_index, items, H, partials,
          accumulate, zero_row);
    } else {
      syrk_dma_kernel<false><<<static_cast<unsigned>(h.n_items), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(X), n_rows, ldx, C, nullptr, items, H, partials,
          accumulate, zero_row);
    }
    if (int rc = check_launch("hessian syrk")) return rc;
  }
  if (h.n_split > 0) {
    dim3 grid(64, static_cast<unsigned>(h.n_split));
    reduce_split_kernel<<<grid, 256, 0, s>>>(split, partials, H, C, accumulate);
    if (int rc = check_launch("hessian split reduce")) return rc;
  }
  return MGQ_OK;
}
