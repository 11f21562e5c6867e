// Hessian accumulation H_g = X_g^T X_g (capture.py:68-76) as a grouped bf16
// MFMA SYRK with fp32 accumulation.
//
// One launch covers any number of groups (one dense linear, or every routed
// expert of a layer). Group g owns tokens [k_begin, k_end) of a token list;
// token t reads row `row_index ? row_index[t] : t` of X, so the routed-expert
// gather is fused into the tile loads. Only the lower triangle of 256x256
// output tiles is computed; each tile is mirrored on store, so H is exactly
// symmetric. Diagonal tiles go in pairs: one workgroup computes the lower
// triangles of two of them, which costs it about what one off-diagonal tile
// costs (the same bytes per token, 18 MFMAs per K-step against 16).
//
// Tile kernel (512 threads = 8 waves, two per SIMD, 1 workgroup per CU):
//   - output tile 256x256, each wave 128x64 = 4x2 blocks of
//     v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators per lane);
//   - token rows are copied HBM -> LDS by global_load_lds_dwordx4 (no VGPR
//     staging); MFMA operands are read with ds_read_b64_tr_b16 transposing
//     loads from the token-major LDS rows (see syrk_kernel);
//   - one MFMA at a time is interleaved with the other work of its K-step
//     (one LDS fragment read, the next stage's DMA, address arithmetic), so
//     the matrix pipe never waits for a burst of non-MFMA instructions;
//   - one work item accumulates at most 262144 tokens in the MFMA fp32
//     accumulators (longer token ranges are split into partial tiles), which
//     bounds the accumulation chain well inside the 1e-5 Frobenius budget.
// Work items are planned on the host (mgq_hessian_plan), see build_plan.
#include <stdlib.h>
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
constexpr int kThreads = 512;  // SYRK workgroup: 8 waves
constexpr int64_t kMaxItemTokens = 262144;  // longest fp32 accumulation chain per item
constexpr int kXcds = 8;
constexpr int kCUs = 256;

struct HessItem {
  int32_t g;     // group, -1 = no-op padding
  int32_t ti;    // output tile row (>= tj)
  int32_t tj;
  int32_t slot;  // -1: write H directly; >= 0: partial tile slot
  int64_t k0;    // token range [k0, k1)
  int64_t k1;
};

struct SplitTile {
  int32_t g, ti, tj, slot0, nslots, stride;  // slots slot0 + stride * i, i < nslots
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

// MFMA j of a K-step and the fragments it takes, numbered in the order the
// K-step reads them:
//   - 8 MFMAs (a 128x64 part, 4x2 blocks): reads a0 b0 b1 a1 a2 a3, MFMA j is
//     block (j / 2, j % 2);
//   - 10 MFMAs (the lower triangle of a 128x128 diagonal part): reads F0..F3,
//     the four 32-channel blocks, each of them both an A and a B operand;
//     MFMA j is block (r, c), c <= r, row by row.
constexpr int tri_row(int j) { return j < 1 ? 0 : j < 3 ? 1 : j < 6 ? 2 : 3; }
constexpr int tri_col(int j) { return j - tri_row(j) * (tri_row(j) + 1) / 2; }
template <int NM>
constexpr int op_a(int j) {
  return NM == 8 ? ((j >> 1) == 0 ? 0 : (j >> 1) + 2) : tri_row(j);
}
template <int NM>
constexpr int op_b(int j) {
  return NM == 8 ? 1 + (j & 1) : tri_col(j);
}

// The stride is kept in a VGPR so the row offsets are formed per element
// instead of occupying scalar registers.
__device__ inline uint32_t ld_vgpr(uint32_t ld_s) {
  uint32_t ld;
  asm volatile("v_mov_b32 %0, %1" : "=v"(ld) : "s"(ld_s));
  return ld;
}

// One 32x32 block at rows gi_l + 32 ma, columns gj (this lane's column). A
// strictly-lower block inside H (whole) needs no masking: registers
// 4q..4q+3 hold rows gi..gi+3 of column gj, so the mirrored values are 4
// consecutive floats of row gj, one 16-byte store. Otherwise each entry is
// kept if it lies in H's lower triangle (direct) and mirrored, or stored as
// it is (a partial tile's slot).
__device__ inline void flush_block(const f32x16_t& a, float* __restrict__ out, uint32_t ld,
                                   bool whole, bool direct, bool add, uint32_t C, uint32_t gi_b,
                                   uint32_t gj) {
  if (whole) {
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const uint32_t gi = gi_b + 8 * rq;
      float nv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float* p = out + ((gi + e) * ld + gj);
        nv[e] = add ? (*p + a[4 * rq + e]) : a[4 * rq + e];
        *p = nv[e];
      }
      *reinterpret_cast<float4*>(out + (gj * ld + gi)) = float4{nv[0], nv[1], nv[2], nv[3]};
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t gi = gi_b + 8 * (r >> 2) + (r & 3);
    const float v = a[r];
    float* p = out + (gi * ld + gj);
    if (direct) {
      if (gi < C && gj < C && gi >= gj) {
        const float nv = add ? (*p + v) : v;
        *p = nv;
        if (gi != gj) out[gj * ld + gi] = nv;
      }
    } else {
      *p = add ? (*p + v) : v;
    }
  }
}

// Flush a wave's 128x64 part (4x2 blocks) at rows gi0.., columns gj0.. of
// `out` (row stride ld): direct parts (H_g, global coordinates) keep the lower
// triangle and mirror it; partial tiles (local 256x256 slot) are stored whole.
// interior: the part lies strictly below H's diagonal and inside H. Offsets
// are 32-bit (C*C < 2^31 is checked on the host).
__device__ inline void flush_part(f32x16_t (&acc)[8], float* __restrict__ out, uint32_t ld_s,
                                  bool direct, bool add, uint32_t C, uint32_t gi0, uint32_t gj0,
                                  int lane, bool interior) {
  const uint32_t ld = ld_vgpr(ld_s);
  const uint32_t gj_l = gj0 + (lane & 31);
  const uint32_t gi_l = gi0 + 4 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    flush_block(acc[j], out, ld, interior, direct, add, C, gi_l + 32 * (j >> 1),
                gj_l + 32 * (j & 1));
}

// Flush the lower triangle of a 128x128 diagonal part at rows and columns
// base.. of `out`: into H (direct), its strictly-lower blocks inside H
// stored whole and mirrored, its diagonal blocks (and blocks crossing C)
// masked; into a partial tile's slot, every block as it is (the blocks above
// the diagonal are never written, and the reduction reads only the lower
// triangle of a diagonal tile).
__device__ inline void flush_tri(f32x16_t (&acc)[10], float* __restrict__ out, uint32_t ld_s,
                                 bool direct, bool add, uint32_t C, uint32_t base, int lane) {
  const uint32_t ld = ld_vgpr(ld_s);
  const uint32_t gj_l = base + (lane & 31);
  const uint32_t gi_l = base + 4 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < 10; ++j) {
    const int r = tri_row(j), c = tri_col(j);
    const bool whole = direct && c < r && base + 32 * r + 32 <= C;
    flush_block(acc[j], out, ld, whole, direct, add, C, gi_l + 32 * r, gj_l + 32 * c);
  }
}

// ---------------------------------------------------------------------------
// SYRK tile kernel.
//
// LDS holds NB stages of KB tokens; token row t of a stage is 1 KB: the 256
// A channels, then the 256 B channels of the tile (diagonal tiles load the A
// channels into both halves). One global_load_lds_dwordx4 moves one token
// row (lanes 0-31 the A half, 32-63 the B half) straight from HBM into LDS.
// Its address is saddr (SGPR pair) + a 32-bit VGPR offset:
//   - dense: saddr = the stage's first row of this wave, offset = lane chunk
//     + i * row pitch (fixed per lane);
//   - gathered, X < 4 GB: saddr = X, offset = row_index[t] * pitch + lane
//     chunk (one v_readlane + multiply-add per token; the wave's KB / 8
//     indices of a stage arrive in one vector load a stage ahead);
//   - gathered, X >= 4 GB (BIG): saddr = X + row * pitch per token.
// Tokens past the item's range read a zero row.
//
// MFMA operands (one channel x 8 consecutive tokens per lane) come from
// ds_read_b64_tr_b16, which hands lane i of each 16-lane group element i%4
// of source lanes 4j + i/4, j=0..3: pointing source lane 4j+q at token j,
// channels 4q..4q+3 gives lane i channel i of tokens 0..3. The 16-byte chunk
// index of LDS token row t is XORed with 4*(t & 3), so the 64 bytes a
// transposed read takes from each of its 8 token rows land on four distinct
// 64-byte bank groups (no conflicts).
//
// Schedule of one stage s (nks = KB/16 K-steps of 8 MFMAs for the 4x2
// blocks of a 128x64 part, 10 for a triangle): segment k (k = 1..nks-1) runs
// the MFMAs of K-step k-1, the first ones each followed by one of the
// fragment reads of K-step k (six for a 4x2 part, a0 b0 b1 a1 a2 a3; four
// for a triangle). Then the stage barrier (this wave's DMA
// of stage s+1 done: vmcnt; every wave done reading stage s: lgkmcnt(0)
// before s_barrier), after which segment 0 of stage s+1 runs the last
// K-step's MFMAs of stage s together with the first fragment reads of stage
// s+1 and the DMA of stage s+NB into the buffer stage s just released.
// Fragments are double-buffered in VGPRs (fr[2][6] or fr[2][4]); each MFMA
// is fenced by sched_barrier so this order is kept.
__device__ inline void dma_tok(uint32_t lds_dst, uint32_t voffset, const char* saddr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_dst), "v"(voffset), "s"(saddr)
               : "memory");
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;
typedef __attribute__((address_space(3))) char lds_char_t;
constexpr int kTokB = 1024;  // LDS bytes per token: A row | B row
constexpr int kRingWave = 512;  // a wave's index ring: 2 blocks of 64 int32

__device__ inline bf16x8_t tr_frag(const lds_char_t* p) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 4 * kTokB));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

// Waves: eight per workgroup, two per SIMD. Wave (wr, wc) = (w / 4, w % 4)
// owns rows 128 wr .. +128 and columns 64 wc .. +64 of the tile (4 x 2
// blocks, 128 fp32 accumulators per lane) and issues KB / 8 of a stage's
// DMAs. With two waves on a SIMD, the issue stall of one wave's DMA (the TA
// accepts a 1 KB request per ~16 cycles) leaves the matrix pipe to the other
// wave's MFMAs; with one wave per SIMD (a 128x128 quarter each) the same
// stall idled the pipe (measured 3-6 % slower, same results bit for bit).
//
// Diagonal tiles. An item with ti <= tj is diagonal:
// ti == tj one tile, ti < tj the pair of tiles (ti, ti) and (tj, tj), whose
// channels the A and B halves of the LDS rows hold (a pair moves the same
// 1 KB per token as an off-diagonal tile). Each diagonal tile is cut into
// rows 128..255 x columns 0..127 (two 4x2 parts, as in an off-diagonal
// tile) and the lower triangles of its two 128x128 diagonal blocks (10
// blocks each, the four 32-channel fragments of a K-step serving as both
// operands). Waves 0-3 take the parts of tile ti and waves 4-7 those of tj,
// arranged so that each SIMD runs one 4x2 part and one triangle: 18 MFMAs per
// K-step against 16 for an off-diagonal tile, for two tiles. A single
// diagonal tile leaves waves 4-7 with their DMAs only (10 MFMAs per K-step on
// the busiest SIMD). A pair's partial tiles (split items) go to slots slot
// and slot + 1.
#define SYRK_MFMA(P, j)                                                                   \
  acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[P][op_a<NM>(j)], fr[P][op_b<NM>(j)], \
                                                   acc[j], 0, 0, 0)
#define SYRK_READ(P, qq, b) fr[P][qq] = tr_frag(lds3 + (b) + off[qq])

template <bool GATHER, bool BIG, int KB, int NB>
__global__ void __launch_bounds__(kThreads, 1)
    syrk_kernel(const uint16_t* __restrict__ X, int64_t n_rows, int64_t ldx, int64_t C,
                 const int32_t* __restrict__ row_index, const HessItem* __restrict__ items,
                 float* __restrict__ H, float* __restrict__ partials, int accumulate,
                 const uint16_t* __restrict__ zero_row) {
  constexpr int kDmaWave = KB / 8;  // tokens (= DMA instructions) per wave and stage
  constexpr int kStageB = KB * kTokB;
  constexpr int nks = KB / 16;
  constexpr int L = (nks - 1) & 1;  // fragment buffer of a stage's last K-step
  constexpr int kDmaEvery = 8 / kDmaWave;  // one DMA every kDmaEvery MFMAs of segment 0
  static_assert(KB % 32 == 0 && kDmaWave <= 8 && (kDmaWave & (kDmaWave - 1)) == 0, "stage shape");
  // Gathered launches with more than two stages take their row indices from
  // an LDS ring (kRing, see idx_ring below); with two they load them one
  // stage ahead into VGPRs.
  constexpr bool kRing = GATHER && NB > 2;
  static_assert(!kRing || kDmaWave == 4, "index ring blocks are 16 stages of 4 tokens");
  static_assert(NB * kStageB + (kRing ? 8 * kRingWave : 0) <= 160 * 1024, "LDS budget");
  constexpr int kVm = (NB - 2) * kDmaWave;
  static_assert(kVm <= 63, "vmcnt range");
  constexpr int kWait = (kVm & 15) | ((kVm >> 4) << 14) | (7 << 4);
  __shared__ __attribute__((aligned(1024))) char lds[NB * kStageB + (kRing ? 8 * kRingWave : 0)];

  const HessItem it = items[blockIdx.x];
  if (it.g < 0) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool diag = it.ti == it.tj;
  const bool direct = it.slot < 0;
  const bool dtile = it.ti <= it.tj;  // one diagonal tile or a pair
  float* out = direct ? H + static_cast<int64_t>(it.g) * C * C
                      : partials + static_cast<int64_t>(it.slot) * kTile * kTile;
  const uint32_t ld = direct ? static_cast<uint32_t>(C) : kTile;

  const int half = lane >> 5;
  const int64_t tile_ch = static_cast<int64_t>(half && !diag ? it.tj : it.ti) * kTile;
  uint32_t voff[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int64_t ch = tile_ch + 8 * ((lane & 31) ^ (4 * f));
    voff[f] = static_cast<uint32_t>(2 * (ch < C - 8 ? ch : C - 8));
  }
  const int g = lane >> 4, j4 = (lane >> 2) & 3, q = lane & 3;
  const uint32_t rd_lo = static_cast<uint32_t>((8 * (g >> 1) + j4) * kTokB + (g & 1) * 32 +
                                               (q >> 1) * 16 + (q & 1) * 8);
  // fragment of 32-channel block m (0..7) of LDS half h
  auto frag_off = [&](int h, int m) -> uint32_t {
    return rd_lo + static_cast<uint32_t>(h * 512 + (m ^ j4) * 64);
  };
  const lds_char_t* lds3 = (const lds_char_t*)lds;
  const uint32_t lds_u32 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds3));
  const uint32_t wave_dst = wave * kDmaWave * kTokB;

  const char* Xb = reinterpret_cast<const char*>(X);
  const char* zr = reinterpret_cast<const char*>(zero_row);
  const uint32_t ldx2 = static_cast<uint32_t>(2 * ldx);
  const uint32_t nr1 = static_cast<uint32_t>(n_rows - 1);
  const int64_t k0 = it.k0, k1 = it.k1;
  const int n_stages = static_cast<int>((k1 - k0 + KB - 1) / KB);
  const int64_t twave = k0 + wave * kDmaWave;
  uint32_t vofs[kDmaWave];
#pragma unroll
  for (int i = 0; i < kDmaWave; ++i) vofs[i] = voff[i & 3] + i * ldx2;

  // L2 prefetch (gathered launches, X < 4 GB): while the DMAs of stage s + NB
  // are issued, one 2-byte load per 128-byte line brings the rows of stage
  // s + NB + 1 into the XCD's L2, so that those DMAs find their lines there
  // instead of missing. The items of one token chunk of a group run
  // together on one XCD and read the same rows; the lines of each 256-column
  // block of a stage (KB tokens x 4 lines) are cut into nt slices, and item
  // (ti, tj) takes slice tj of block ti and slice ti of block tj (a diagonal
  // item slice d of its block d), so every line is requested once per
  // token chunk. The loaded values are dead; they are kept live until the
  // stage barrier's vmcnt(0) so that their registers are not reused while a
  // load is in flight.
  constexpr bool kPf = GATHER && !BIG && !kRing;
  constexpr int kPfAhead = 1;
  const int nt = static_cast<int>((C + kTile - 1) / kTile);
  const int pf_parts = it.ti == it.tj ? 1 : 2;
  const int pf_S = (4 * KB + nt - 1) / nt;
  const bool pf_wave = kPf && wave * 64 < pf_parts * pf_S;
  int pf_tok = 0;
  uint32_t pf_col = 0;
  bool pf_ok = false;
  if (kPf) {
    const int pi = wave * 64 + lane;
    const int part = pi / pf_S, r = pi % pf_S;
    const int b = part == 0 ? it.ti : it.tj;
    const int o = it.ti > it.tj ? (part == 0 ? it.tj : it.ti) : b;
    const int Lx = o * pf_S + r;
    const int col = b * kTile + (Lx & 3) * 64;
    pf_ok = part < pf_parts && Lx < 4 * KB && col < C;
    pf_tok = Lx >> 2;
    pf_col = static_cast<uint32_t>(2 * col);
  }
  auto pf_index = [&](int s) -> int32_t {
    const int64_t t = k0 + static_cast<int64_t>(s + NB + kPfAhead) * KB + pf_tok;
    return row_index[t < k1 ? t : k1 - 1];
  };
  auto pf_load = [&](int s, int32_t pidx) -> uint32_t {
    const int64_t t = k0 + static_cast<int64_t>(s + NB + kPfAhead) * KB + pf_tok;
    uint32_t r = static_cast<uint32_t>(pidx);
    r = r < nr1 ? r : nr1;
    const uint32_t o = (pf_ok && t < k1) ? r * ldx2 + pf_col : 0u;
    return X[o >> 1];
  };

  auto load_idx = [&](int64_t t0) -> int32_t {
    if constexpr (GATHER) {
      const int64_t t = t0 + (lane & (kDmaWave - 1));
      return row_index[t < k1 ? t : k1 - 1];
    } else {
      return 0;
    }
  };
  auto dma_i = [&](int i, uint32_t dst, int rem, int32_t idxv, const char* base, int lbase = 0) {
    const char* sa;
    uint32_t vo;
    if constexpr (GATHER) {
      uint32_t r = static_cast<uint32_t>(__builtin_amdgcn_readlane(idxv, lbase + i));
      r = r < nr1 ? r : nr1;
      if constexpr (BIG) {
        sa = Xb + static_cast<uint64_t>(r) * ldx2;
        vo = voff[i & 3];
      } else {
        sa = Xb;
        vo = r * ldx2 + voff[i & 3];
      }
    } else {
      sa = base;
      vo = vofs[i];
    }
    const bool ok = i < rem;
    dma_tok(dst + i * kTokB, ok ? vo : voff[i & 3], ok ? sa : zr);
  };
  auto stage_rem = [&](int64_t t0) -> int {
    const int64_t r = k1 - t0;
    return static_cast<int>(r < 0 ? 0 : (r > kDmaWave ? kDmaWave : r));
  };
  auto stage_base = [&](int64_t t0) -> const char* {
    return Xb + static_cast<uint64_t>(t0 < k1 ? t0 : k0) * ldx2;
  };
  // this wave's DMAs of stage p (p < NB) before the loop; idxv lanes
  // lbase.. hold the stage's row indices (gathered launches)
  auto first_dmas = [&](int p, int32_t idxv, int lbase = 0) {
    const int64_t t0 = twave + p * KB;
    const int rem = stage_rem(t0);
    const char* base = stage_base(t0);
#pragma unroll
    for (int i = 0; i < kDmaWave; ++i)
      dma_i(i, lds_u32 + p * kStageB + wave_dst, rem, idxv, base, lbase);
  };

  // Index ring (kRing). A wave's row indices come into LDS 64 at a time (16
  // stages of 4 tokens) by one global_load_lds_dword, 15 iterations before
  // their first use, into a ring of two blocks: block c holds the indices
  // of stages NB + 16c .. NB + 16c + 15 and sits in slot c % 2; block c + 1 is
  // fetched at iteration 16c, after the barrier that follows the last read
  // of the block it replaces. Each iteration reads the next stage's 4
  // indices from the ring with one ds_read_b32, a whole stage before its
  // DMAs take them by v_readlane. Indices loaded into VGPRs would be vector
  // loads, which complete in order: waiting for one would also wait for
  // every row DMA issued before it, and the pipeline would drain.
  const uint32_t ring = lds_u32 + NB * kStageB + wave * kRingWave;
  auto ring_pos = [&](int st0) -> uint32_t {  // lane l: stage st0 + l / 4, token l % 4
    const int64_t t = twave + static_cast<int64_t>(st0 + (lane >> 2)) * KB + (lane & 3);
    return static_cast<uint32_t>(t < k1 ? t : k1 - 1);
  };
  auto ring_fetch = [&](int c) {  // block c into slot c % 2
    const uint64_t a = reinterpret_cast<uint64_t>(row_index);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
    const int32_t* sa = reinterpret_cast<const int32_t*>((static_cast<uint64_t>(hi) << 32) | lo);
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
                 :
                 : "s"(ring + (c & 1) * 256), "v"(4 * ring_pos(NB + 16 * c)), "s"(sa)
                 : "memory");
  };
  auto ring_read = [&](int st) -> int32_t {  // stage st's 4 indices in lanes 0..3 (and repeats)
    const int c = (st - NB) >> 4;
    const uint32_t a = ring - lds_u32 + (c & 1) * 256 + ((st - NB) & 15) * 16 + 4 * (lane & 3);
    return *reinterpret_cast<const __attribute__((address_space(3))) int32_t*>(lds3 + a);
  };
  // Prologue DMAs of stages 0 .. NB - 2; returns the indices of stage NB - 1
  // (in lanes 4 (NB - 1)..) for its DMAs after the first barrier. The ring's
  // first block is fetched before them, so the barrier's wait covers it.
  auto prologue_dmas = [&](int32_t& idx_last, int& lb_last) {
    if constexpr (kRing) {
      const int32_t idx_pre = row_index[ring_pos(0)];  // stages 0 .. NB-1, lanes 0 .. 4 NB - 1
      ring_fetch(0);
#pragma unroll
      for (int p = 0; p < NB - 1; ++p) first_dmas(p, idx_pre, 4 * p);
      idx_last = idx_pre;
      lb_last = 4 * (NB - 1);
    } else {
#pragma unroll
      for (int p = 0; p < NB - 1; ++p) first_dmas(p, load_idx(twave + p * KB));
      idx_last = load_idx(twave + (NB - 1) * KB);
      lb_last = 0;
    }
  };

  // The K loop of one wave: NM MFMAs per K-step into acc[NM], fragments at
  // the NR LDS offsets off[] (read order).
  auto run = [&](auto& acc, const auto& off) __attribute__((always_inline)) {
    constexpr int NM = static_cast<int>(sizeof(acc) / sizeof(acc[0]));
    constexpr int NR = static_cast<int>(sizeof(off) / sizeof(off[0]));
#pragma unroll
    for (int j = 0; j < NM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    if (n_stages <= 0) return;
    bf16x8_t fr[2][NR];
    int32_t idx_n;
    int lb_n;
    prologue_dmas(idx_n, lb_n);
    __builtin_amdgcn_s_waitcnt(GATHER && !kRing ? 0 : kWait);
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int qq = 0; qq < NR; ++qq) SYRK_READ(0, qq, 0u);
    first_dmas(NB - 1, idx_n, lb_n);
    if constexpr (kRing) idx_n = ring_read(NB);  // for iteration 0's DMAs (stage NB)
    __builtin_amdgcn_sched_barrier(0);
    int rbuf = 0;
    uint32_t pf_v = 0, pf_sink = 0;
    int32_t pf_idx = 0;
    for (int s = 0; s < n_stages - 1; ++s) {
      const uint32_t rd = static_cast<uint32_t>(rbuf * kStageB);
#pragma unroll
      for (int ks = 1; ks < nks; ++ks) {
        const int P = (ks - 1) & 1;
#pragma unroll
        for (int j = 0; j < NM; ++j) {
          SYRK_MFMA(P, j);
          if (j < NR) SYRK_READ(P ^ 1, j, rd + ks * 16 * kTokB);
          if (GATHER && !kRing && ks == 1 && j == 1)
            idx_n = load_idx(twave + static_cast<int64_t>(s + NB) * KB);
          if (kPf && ks == 1 && j == 2 && pf_wave) pf_idx = pf_index(s);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      const uint32_t wbuf = static_cast<uint32_t>(rbuf);
      rbuf = rbuf + 1 == NB ? 0 : rbuf + 1;
      __builtin_amdgcn_s_waitcnt(GATHER && !kRing ? 0 : kWait);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      int32_t idx_next = 0;
      if constexpr (kRing) {
        if ((s & 15) == 0) ring_fetch((s >> 4) + 1);
        idx_next = ring_read(s + NB + 1);
      }
      const uint32_t nrd = static_cast<uint32_t>(rbuf * kStageB);
      const uint32_t dst = lds_u32 + wbuf * kStageB + wave_dst;
      const int64_t t0 = twave + static_cast<int64_t>(s + NB) * KB;
      const int rem = stage_rem(t0);
      const char* base = stage_base(t0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        SYRK_MFMA(L, j);
        if (j < NR) SYRK_READ(L ^ 1, j, nrd);
        if (j < 8 && j % kDmaEvery == kDmaEvery - 1) dma_i(j / kDmaEvery, dst, rem, idx_n, base);
        if (kPf && j == NM - 1 && pf_wave) {
          pf_sink ^= pf_v;
          pf_v = pf_load(s, pf_idx);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kRing) idx_n = idx_next;
    }
    {
      const uint32_t rd = static_cast<uint32_t>(rbuf * kStageB);
#pragma unroll
      for (int ks = 1; ks < nks; ++ks) {
        const int P = (ks - 1) & 1;
#pragma unroll
        for (int j = 0; j < NM; ++j) {
          SYRK_MFMA(P, j);
          if (j < NR) SYRK_READ(P ^ 1, j, rd + ks * 16 * kTokB);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int j = 0; j < NM; ++j) SYRK_MFMA(L, j);
    }
    __builtin_amdgcn_s_waitcnt(0);
    if constexpr (kPf) asm volatile("" ::"v"(pf_sink), "v"(pf_v));
  };

  if (dtile) {
    const int h = wave >> 2;
    const int rho = ((wave & 3) + 2 * h) & 3;  // 0, 1: a 4x2 part; 2, 3: a triangle
    const uint32_t tile = direct ? static_cast<uint32_t>(h ? it.tj : it.ti) * kTile : 0u;
    float* out_h = out + (!direct && h ? kTile * kTile : 0);
    if (h == 1 && diag) {
      // a single diagonal tile: the B half repeats the A half; DMAs only
      if (n_stages > 0) {
        int32_t idx_n;
        int lb_n;
        prologue_dmas(idx_n, lb_n);
        __builtin_amdgcn_s_waitcnt(GATHER && !kRing ? 0 : kWait);
        __builtin_amdgcn_s_barrier();
        first_dmas(NB - 1, idx_n, lb_n);
        if constexpr (kRing) idx_n = ring_read(NB);
        int rbuf = 0;
        for (int s = 0; s < n_stages - 1; ++s) {
          if constexpr (!kRing) idx_n = load_idx(twave + static_cast<int64_t>(s + NB) * KB);
          const uint32_t wbuf = static_cast<uint32_t>(rbuf);
          rbuf = rbuf + 1 == NB ? 0 : rbuf + 1;
          __builtin_amdgcn_s_waitcnt(GATHER && !kRing ? 0 : kWait);
          __builtin_amdgcn_s_barrier();
          int32_t idx_next = 0;
          if constexpr (kRing) {
            if ((s & 15) == 0) ring_fetch((s >> 4) + 1);
            idx_next = ring_read(s + NB + 1);
          }
          const int64_t t0 = twave + static_cast<int64_t>(s + NB) * KB;
          const int rem = stage_rem(t0);
          const char* base = stage_base(t0);
#pragma unroll
          for (int i = 0; i < kDmaWave; ++i)
            dma_i(i, lds_u32 + wbuf * kStageB + wave_dst, rem, idx_n, base);
          if constexpr (kRing) idx_n = idx_next;
        }
        __builtin_amdgcn_s_waitcnt(0);
      }
      return;
    }
    if (rho >= 2) {
      const int m0 = 4 * (rho - 2);
      const uint32_t off[4] = {frag_off(h, m0), frag_off(h, m0 + 1), frag_off(h, m0 + 2),
                               frag_off(h, m0 + 3)};
      f32x16_t acc[10];
      run(acc, off);
      flush_tri(acc, out_h, ld, direct, direct && accumulate, static_cast<uint32_t>(C),
                tile + 128 * static_cast<uint32_t>(rho - 2), lane);
      return;
    }
  }
  // a 4x2 part: rows 128 wr.., columns 64 wc.. of an off-diagonal tile (into
  // H, or its partial slot), or rows 128.., columns 64 rho.. of a diagonal
  // tile
  uint32_t off[6], gi0, gj0;
  bool interior;
  float* out_p = out;
  if (dtile) {
    const int h = wave >> 2;
    const int rho = ((wave & 3) + 2 * h) & 3;
    const uint32_t tile = direct ? static_cast<uint32_t>(h ? it.tj : it.ti) * kTile : 0u;
    out_p = out + (!direct && h ? kTile * kTile : 0);
    off[0] = frag_off(h, 4);
    off[1] = frag_off(h, 2 * rho);
    off[2] = frag_off(h, 2 * rho + 1);
    off[3] = frag_off(h, 5);
    off[4] = frag_off(h, 6);
    off[5] = frag_off(h, 7);
    gi0 = tile + 128;
    gj0 = tile + 64 * static_cast<uint32_t>(rho);
    interior = direct && static_cast<int64_t>(tile) + kTile <= C;
  } else {
    const int wr = wave >> 2, wc = wave & 3;
    off[0] = frag_off(0, 4 * wr);
    off[1] = frag_off(1, 2 * wc);
    off[2] = frag_off(1, 2 * wc + 1);
    off[3] = frag_off(0, 4 * wr + 1);
    off[4] = frag_off(0, 4 * wr + 2);
    off[5] = frag_off(0, 4 * wr + 3);
    gi0 = (direct ? static_cast<uint32_t>(it.ti) * kTile : 0u) + wr * 128;
    gj0 = (direct ? static_cast<uint32_t>(it.tj) * kTile : 0u) + wc * 64;
    interior = direct && it.ti > it.tj && (static_cast<int64_t>(it.ti) + 1) * kTile <= C;
  }
  f32x16_t acc[8];
  run(acc, off);
  flush_part(acc, out_p, ld, direct, direct && accumulate, static_cast<uint32_t>(C), gi0, gj0,
             lane, interior);
}
#undef SYRK_MFMA
#undef SYRK_READ

__global__ void zero_fill_kernel(uint32_t* __restrict__ p, int64_t n_words) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n_words;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Sum the K-split partial tiles of one output tile in slot order and write
// the lower triangle (+ mirror) of H. One block per 64x64 sub-tile: thread
// (rr = tid / 16, c4 = 4 (tid % 16)) takes columns c4..c4+3 of rows rr,
// rr+16, rr+32, rr+48 with 16-byte loads, the slots of a row loaded eight
// at a time before they are added (in slot order, so H is deterministic);
// the mirrored values go out through an LDS transpose, so both stores are
// coalesced.
constexpr int kRedSub = 64;
constexpr int kRedSlots = 8;
__global__ void __launch_bounds__(256) reduce_split_kernel(const SplitTile* __restrict__ tiles,
                                                           const float* __restrict__ partials,
                                                           float* __restrict__ H, int64_t C,
                                                           int accumulate) {
  __shared__ float tr[kRedSub][kRedSub + 1];
  const SplitTile st = tiles[blockIdx.y];
  float* Hg = H + static_cast<int64_t>(st.g) * C * C;
  const int sr = blockIdx.x / (kTile / kRedSub), sc = blockIdx.x % (kTile / kRedSub);
  const int64_t bi = static_cast<int64_t>(st.ti) * kTile + sr * kRedSub;  // global row base
  const int64_t bj = static_cast<int64_t>(st.tj) * kTile + sc * kRedSub;  // global column base
  const int c4 = (threadIdx.x & 15) * 4, rr = threadIdx.x >> 4;
  const float* p0 = partials + static_cast<int64_t>(st.slot0) * kTile * kTile;
  constexpr int64_t kSlot = static_cast<int64_t>(kTile) * kTile;
#pragma unroll
  for (int qr = 0; qr < kRedSub / 16; ++qr) {
    const int r = rr + 16 * qr;
    const int e = (sr * kRedSub + r) * kTile + sc * kRedSub + c4;
    float4 v = *reinterpret_cast<const float4*>(p0 + e);
    for (int s0 = 1; s0 < st.nslots; s0 += kRedSlots) {
      float4 t[kRedSlots];
#pragma unroll
      for (int i = 0; i < kRedSlots; ++i)
        if (s0 + i < st.nslots)
          t[i] = *reinterpret_cast<const float4*>(p0 + static_cast<int64_t>(s0 + i) * st.stride * kSlot + e);
#pragma unroll
      for (int i = 0; i < kRedSlots; ++i)
        if (s0 + i < st.nslots) {
          v.x += t[i].x;
          v.y += t[i].y;
          v.z += t[i].z;
          v.w += t[i].w;
        }
    }
    const int64_t gi = bi + r, gj = bj + c4;
    float nv[4] = {v.x, v.y, v.z, v.w};
    float* p = Hg + gi * C + gj;
    if (gi < C && gj + 3 < C && gi >= gj + 3) {  // four lower-triangle entries
      if (accumulate) {
        const float4 h = *reinterpret_cast<const float4*>(p);
        nv[0] += h.x, nv[1] += h.y, nv[2] += h.z, nv[3] += h.w;
      }
      *reinterpret_cast<float4*>(p) = float4{nv[0], nv[1], nv[2], nv[3]};
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (gi < C && gj + k < C && gi >= gj + k) {
          nv[k] = accumulate ? p[k] + nv[k] : nv[k];
          p[k] = nv[k];
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) tr[c4 + k][r] = nv[k];
  }
  __syncthreads();
  // mirror: H[bj + r][bi + c] = value of (bi + c, bj + r), strictly below the diagonal
  const int c = threadIdx.x & (kRedSub - 1), r0 = threadIdx.x / kRedSub;
#pragma unroll 4
  for (int r = r0; r < kRedSub; r += 256 / kRedSub) {
    const int64_t gi = bi + c, gj = bj + r;
    if (gi < C && gj < C && gi > gj) Hg[gj * C + gi] = tr[r][c];
  }
}

// ---------------------------------------------------------------------------
// Host planning.
//
// The hardware hands workgroup i to XCD i mod 8, and each XCD (32 CUs) has
// its own L2; token rows fetched by one tile are reused from that L2 by the
// other tiles that read the same channel blocks at about the same time. So:
//   - tiles are enumerated in 4x4 super-block order of the lower triangle,
//     and the work items of a group are laid out split-major (all tiles of
//     token chunk 0, then chunk 1, ...): the ~32 items an XCD runs together
//     share one token range and touch few channel blocks;
//   - a group's item list is cut into at most 8 contiguous runs (>= 32 items)
//     that go to the least-loaded XCD, heaviest first (LPT), and the XCD
//     queues are interleaved into the grid;
//   - K splits: every item covers at most kMaxItemTokens tokens; when a
//     one-group launch has few tile items (one dense layer), the token range
//     is split further to fill the 256 CUs, choosing the split count by a
//     cost model (rounds of 256 items x tokens per item, plus the
//     partial-tile traffic). In a launch of several groups, a group longer
//     than the average per-CU load is split instead. Partial tiles are summed in a fixed order by
//     reduce_split_kernel, so H is deterministic. target_items > 0 instead
//     sets the split directly (chunk = max(2048, tokens*tiles/target_items));
//   - items pair a group's diagonal tiles (a split pair's two partial tiles
//     take interleaved slots).
// ---------------------------------------------------------------------------
struct Plan {
  PlanHeader hdr;
  std::vector<HessItem> items;
  std::vector<SplitTile> split;
};

std::vector<std::pair<int32_t, int32_t>> blocked_tiles(int64_t nt) {
  constexpr int64_t SB = 4;
  std::vector<std::pair<int32_t, int32_t>> t;
  const int64_t nsb = ceil_div(nt, SB);
  for (int64_t I = 0; I < nsb; ++I)
    for (int64_t J = 0; J <= I; ++J)
      for (int64_t i = SB * I; i < std::min(nt, SB * I + SB); ++i)
        for (int64_t j = SB * J; j < std::min(nt, SB * J + SB); ++j)
          if (j <= i) t.emplace_back(static_cast<int32_t>(i), static_cast<int32_t>(j));
  return t;
}

// Items pair a group's diagonal tiles in the order above: (d, d')
// with d < d' stands for tiles (d, d) and (d', d') (see syrk_kernel); an odd
// one out stays (d, d).
std::vector<std::pair<int32_t, int32_t>> pair_diagonals(
    const std::vector<std::pair<int32_t, int32_t>>& tiles) {
  std::vector<std::pair<int32_t, int32_t>> out;
  int64_t open = -1;  // index in out of an unpaired diagonal tile
  for (const auto& t : tiles) {
    if (t.first != t.second) {
      out.push_back(t);
    } else if (open >= 0) {
      out[open].second = t.first;
      open = -1;
    } else {
      open = static_cast<int64_t>(out.size());
      out.push_back(t);
    }
  }
  return out;
}

int build_plan(int64_t C, int64_t n_groups, const int64_t* offsets, int64_t target_items,
               Plan* plan) {
  const int64_t nt = ceil_div(C, kTile);
  auto tiles = pair_diagonals(blocked_tiles(nt));
  const int64_t T = static_cast<int64_t>(tiles.size());
  // A group whose items fit one round of an XCD (32 CUs) runs them side by
  // side, so their order only decides which CUs free up first: the costlier
  // items go first (a diagonal pair, 18 MFMAs per K-step on its busiest
  // SIMD, then the off-diagonal tiles, 16, then a lone diagonal tile, 10),
  // so that the next group's items fill the CUs that finish early. Larger
  // groups keep the super-block order, which their rounds' L2 reuse needs.
  if (T <= kCUs / kXcds) {
    auto cost = [](const std::pair<int32_t, int32_t>& t) {
      return t.first < t.second ? 18 : (t.first > t.second ? 16 : 10);
    };
    std::stable_sort(tiles.begin(), tiles.end(),
                     [&](const auto& a, const auto& b) { return cost(a) > cost(b); });
  }
  int64_t active = 0, n_max = 0, total_tokens = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t n = offsets[g + 1] - offsets[g];
    MGQ_REQUIRE(n >= 0, MGQ_ERR_SHAPE, "offsets must be non-decreasing (group %lld)",
                (long long)g);
    if (n > 0) ++active;
    n_max = std::max(n_max, n);
    total_tokens += n;
  }
  // tokens per item: explicit (target_items > 0) or from the cost model
  int64_t s_bal = 1, chunk_explicit = 0;
  if (target_items > 0) {
    const int64_t work = std::max<int64_t>(total_tokens, 1) * T;
    chunk_explicit = std::max<int64_t>(2048, ceil_div(work, target_items));
  } else if (active == 1) {
    // one group (a dense layer): split to fill the CUs. Launches of several
    // groups split only their heavy groups (below): this model prices every
    // item at the longest group's tokens, which misjudges skewed groups.
    const int64_t base = active * T;
    if (base > 0 && base < 8 * kCUs) {
      double best = 1e300;
      for (int64_t sv = 1; sv <= 16; ++sv) {
        const int64_t per = ceil_div(ceil_div(n_max, sv), kKs) * kKs;
        if (sv > 1 && per < 512) break;
        // 40 ns per token per 256x256 tile item, 100 ns per partial tile
        const double cost = static_cast<double>(ceil_div(base * sv, kCUs)) * per * 40e-9 +
                            (sv > 1 ? static_cast<double>(base * sv) * 100e-9 : 0.0);
        if (cost < best * 0.98) {
          best = cost;
          s_bal = sv;
        }
      }
    }
  }

  // Multi-group launches: a group whose items would each run longer than the
  // average per-CU load (tokens x items / CUs) is split along K, so that its
  // few long items do not keep one XCD busy after the others finish (a routed
  // down projection with C = 768 has 5 items per expert, and its heaviest
  // expert can hold 1.4x the average CU load).
  int64_t heavy_cap = 0;
  if (chunk_explicit == 0 && n_groups > 1) {
    const int64_t avg = total_tokens * T / kCUs;
    heavy_cap = std::max<int64_t>(avg, 4096);
  }

  struct Chunk {
    int64_t work;
    std::vector<HessItem> items;
  };
  std::vector<Chunk> chunks;
  int64_t n_slots = 0;
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t k0 = offsets[g], k1 = offsets[g + 1];
    const int64_t n = k1 - k0;
    int64_t per;
    if (n == 0) {
      per = 1;
    } else if (chunk_explicit > 0) {
      per = std::min<int64_t>(chunk_explicit, kMaxItemTokens);
    } else {
      int64_t S = std::max<int64_t>(ceil_div(n, kMaxItemTokens), s_bal);
      if (heavy_cap > 0 && n > heavy_cap) S = std::max<int64_t>(S, ceil_div(n, heavy_cap));
      per = ceil_div(n, S);
    }
    per = ceil_div(per, kKs) * kKs;
    const int64_t S = n == 0 ? 1 : ceil_div(n, per);  // chunks actually used
    std::vector<HessItem> gi;
    gi.reserve(T * S);
    if (S == 1) {
      for (const auto& t : tiles)
        gi.push_back(HessItem{static_cast<int32_t>(g), t.first, t.second, -1, k0, k1});
    } else {
      // a tile's partials take S slots; a pair's two tiles take 2S, chunk c's
      // at 2c (tile (ti, ti)) and 2c + 1 (tile (tj, tj))
      std::vector<int64_t> first(T);
      for (int64_t e = 0; e < T; ++e) {
        first[e] = n_slots;
        n_slots += (tiles[e].first < tiles[e].second ? 2 : 1) * S;
      }
      for (int64_t c = 0; c < S; ++c) {
        const int64_t a = k0 + c * per;
        for (int64_t e = 0; e < T; ++e) {
          const bool pair = tiles[e].first < tiles[e].second;
          gi.push_back(HessItem{static_cast<int32_t>(g), tiles[e].first, tiles[e].second,
                                static_cast<int32_t>(first[e] + (pair ? 2 * c : c)), a,
                                std::min(a + per, k1)});
        }
      }
      for (int64_t e = 0; e < T; ++e) {
        const int32_t ti = tiles[e].first, tj = tiles[e].second;
        const int32_t f = static_cast<int32_t>(first[e]), ns = static_cast<int32_t>(S);
        if (ti < tj) {
          plan->split.push_back(SplitTile{static_cast<int32_t>(g), ti, ti, f, ns, 2});
          plan->split.push_back(SplitTile{static_cast<int32_t>(g), tj, tj, f + 1, ns, 2});
        } else {
          plan->split.push_back(SplitTile{static_cast<int32_t>(g), ti, tj, f, ns, 1});
        }
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
  MGQ_REQUIRE(n_slots < (int64_t(1) << 31), MGQ_ERR_SHAPE, "hessian plan: too many partial tiles");
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

// Gathered launches use the 32-bit row-offset form when every row of X is
// addressable with a 32-bit offset from X; MGQ_HESSIAN_WIDE_ADDR=1 forces the
// 64-bit per-token form (used to test it on small inputs).
bool wide_gather_addr(int64_t n_rows, int64_t ldx) {
  const char* e = getenv("MGQ_HESSIAN_WIDE_ADDR");
  return (e != nullptr && e[0] == '1') || n_rows * ldx * 2 + 16 > (int64_t(1) << 32);
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
  // A caller asks for the size first and then for the plan itself with the
  // same arguments: the plan built for the size query is kept (per thread)
  // and handed out by the second call instead of being built again.
  thread_local Plan last;
  thread_local std::vector<int64_t> last_key;
  std::vector<int64_t> key(offsets, offsets + n_groups + 1);
  key.push_back(C);
  key.push_back(target_items);
  if (key != last_key) {
    last_key.clear();
    Plan built;
    if (int rc = build_plan(C, n_groups, offsets, target_items, &built)) return rc;
    last = std::move(built);
    last_key = std::move(key);
  }
  const Plan& p = last;
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
    const dim3 grid(static_cast<unsigned>(h.n_items));
    const uint16_t* Xh = static_cast<const uint16_t*>(X);
    const char* gs = getenv("MGQ_HESSIAN_GATHER_STAGES");
    const bool two_stage = gs != nullptr && strcmp(gs, "2") == 0;
    if (row_index && wide_gather_addr(n_rows, ldx)) {
      if (two_stage)
        syrk_kernel<true, true, 64, 2><<<grid, kThreads, 0, s>>>(
            Xh, n_rows, ldx, C, row_index, items, H, partials, accumulate, zero_row);
      else
        syrk_kernel<true, true, 32, 4><<<grid, kThreads, 0, s>>>(
            Xh, n_rows, ldx, C, row_index, items, H, partials, accumulate, zero_row);
    } else if (row_index) {
      if (two_stage)
        syrk_kernel<true, false, 64, 2><<<grid, kThreads, 0, s>>>(
            Xh, n_rows, ldx, C, row_index, items, H, partials, accumulate, zero_row);
      else
        syrk_kernel<true, false, 32, 4><<<grid, kThreads, 0, s>>>(
            Xh, n_rows, ldx, C, row_index, items, H, partials, accumulate, zero_row);
    } else {
      syrk_kernel<false, false, 32, 4><<<grid, kThreads, 0, s>>>(
          Xh, n_rows, ldx, C, nullptr, items, H, partials, accumulate, zero_row);
    }
    if (int rc = check_launch("hessian syrk")) return rc;
  }
  if (h.n_split > 0) {
    dim3 grid((kTile / kRedSub) * (kTile / kRedSub), static_cast<unsigned>(h.n_split));
    reduce_split_kernel<<<grid, 256, 0, s>>>(split, partials, H, C, accumulate);
    if (int rc = check_launch("hessian split reduce")) return rc;
  }
  return MGQ_OK;
}
