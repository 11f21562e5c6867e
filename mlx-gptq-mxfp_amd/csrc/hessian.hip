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
//     v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane);
//   - K stages of 64 tokens, double-buffered in LDS (2 x 64 KB); a thread
//     loads an 8-token x 8-channel block with 16-byte global loads
//     (coalesced along channels), transposes it in registers with v_perm so
//     channel rows become token-contiguous, and stores 16-byte rows into an
//     XOR-swizzled LDS layout that keeps both the stores and the MFMA operand
//     reads (ds_read_b128) free of bank conflicts;
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
// Native clang vectors (not HIP's u32x4 struct) so register arrays of them
// are promoted to VGPRs instead of private memory.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 256;
constexpr int kKs = 64;          // tokens per LDS stage
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

// LDS: [buf][operand][256 rows][8 chunks of 16 B], chunk index XOR-swizzled.
__device__ inline int swz(int row, int chunk) {
  return row * 8 + (chunk ^ ((row ^ (row >> 3)) & 7));
}

__device__ inline uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// Per-stage global traffic of a loader thread: its 8 tokens' rows (one
// 16-byte load per token and operand). The three steps are kept apart so the
// loop can software-pipeline them: gather indices for stage s+2 and row
// loads for stage s+1 are in flight while stage s runs on the MFMAs; the
// zero-masking of out-of-range tokens happens only when the rows are stored
// to LDS. Everything is branch-free (a branch around a load makes the
// compiler wait for it at the join). Out-of-range tokens read a clamped
// valid row; gathered indices are clamped into X so a bad index cannot
// fault.
template <bool GATHER>
__device__ inline void load_index(const int32_t* __restrict__ row_index, int64_t tok0,
                                  int64_t t_end, int32_t (&idx)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t t = tok0 + r;
    idx[r] = GATHER ? row_index[t < t_end ? t : t_end - 1] : 0;
  }
}

template <bool GATHER>
__device__ inline void load_rows(const uint16_t* __restrict__ X, int64_t ldx, int64_t n_rows,
                                 const int32_t (&idx)[8], int64_t tok0, int64_t t_end,
                                 int64_t chanA, int64_t chanB, u32x4 (&ra)[8], u32x4 (&rb)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int64_t t = tok0 + r;
    const int64_t row = GATHER ? min(max(static_cast<int64_t>(idx[r]), int64_t(0)), n_rows - 1)
                               : (t < t_end ? t : t_end - 1);
    const uint16_t* p = X + row * ldx;
    ra[r] = *reinterpret_cast<const u32x4*>(p + chanA);
    rb[r] = *reinterpret_cast<const u32x4*>(p + chanB);
  }
}

__device__ inline void mask_rows(int64_t tok0, int64_t t_end, bool ok, u32x4 (&rr)[8]) {
  const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int r = 0; r < 8; ++r) rr[r] = (ok && tok0 + r < t_end) ? rr[r] : z;
}

// Transpose an 8x8 bf16 block in registers (v_perm) so each channel's 8
// tokens are contiguous, and store the 8 channel rows into the swizzled LDS
// tile. Row cb*8+c, chunk kb lands at (cb*8+c)*8 + (kb ^ f(row)) with
// f(row) = (c ^ cb) & 7, i.e. chunk (u ^ c) for u = (kb ^ cb) & 7.
__device__ inline uint32_t dword(const u32x4& v, int d) { return v[d]; }

__device__ inline void store_block(u32x4* __restrict__ lds, int cb, int u, const u32x4 (&in)[8]) {
  u32x4* base = lds + cb * 64;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    const int d = c >> 1;  // dword holding channel c of each token
    u32x4 o;
    o.x = perm(dword(in[1], d), dword(in[0], d), sel);
    o.y = perm(dword(in[3], d), dword(in[2], d), sel);
    o.z = perm(dword(in[5], d), dword(in[4], d), sel);
    o.w = perm(dword(in[7], d), dword(in[6], d), sel);
    base[c * 8 + (u ^ c)] = o;
  }
}

// Flush the wave's 128x128 accumulators into `out` (row stride ld). Direct
// tiles (H_g, global coordinates) keep the lower triangle and
// mirror it; partial tiles (local 256x256 slot) are stored whole. Offsets are
// 32-bit (C*C < 2^31 is checked on the host) and the stride is kept in a
// VGPR so the 64 row offsets are formed per element instead of occupying
// scalar registers.
__device__ inline void flush(f32x16_t (&acc)[4][4], float* __restrict__ out, uint32_t ld_s,
                             bool direct, bool add, uint32_t C, uint32_t gi0, uint32_t gj0,
                             int lane) {
  uint32_t ld;
  asm volatile("v_mov_b32 %0, %1" : "=v"(ld) : "s"(ld_s));
  const uint32_t gj_l = gj0 + (lane & 31);
  const uint32_t gi_l = gi0 + 4 * (lane >> 5);
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

template <bool GATHER>
__global__ void __launch_bounds__(kThreads, 1)
    syrk_tile_kernel(const uint16_t* __restrict__ X, int64_t n_rows, int64_t ldx, int64_t C,
                     const int32_t* __restrict__ row_index, const HessItem* __restrict__ items,
                     float* __restrict__ H, float* __restrict__ partials, int accumulate) {
  __shared__ u32x4 lds[2][2][kTile * 8];  // 2 bufs x (A, B) x 256 rows x 128 B = 128 KB

  const HessItem it = items[blockIdx.x];
  if (it.g < 0) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const bool diag = it.ti == it.tj;
  const bool direct = it.slot < 0;
  float* out = direct ? H + static_cast<int64_t>(it.g) * C * C
                      : partials + static_cast<int64_t>(it.slot) * kTile * kTile;
  const uint32_t ld = direct ? static_cast<uint32_t>(C) : kTile;
  const uint32_t gi0 = (direct ? static_cast<uint32_t>(it.ti) * kTile : 0u) + wr * 128;
  const uint32_t gj0 = (direct ? static_cast<uint32_t>(it.tj) * kTile : 0u) + wc * 128;

  // loader role: 8-token block kb, 8-channel block cb, for A and (off-diagonal) B
  const int kb = tid & 7, cb = tid >> 3;
  const int u = (kb ^ cb) & 7;
  const int64_t cA = static_cast<int64_t>(it.ti) * kTile + cb * 8;
  const int64_t cB = static_cast<int64_t>(it.tj) * kTile + cb * 8;
  const bool okA = cA < C, okB = cB < C;
  const int64_t chanA = okA ? cA : 0;
  const int64_t chanB = diag ? chanA : (okB ? cB : 0);

  // MFMA operand offsets (u32x4 units) within a 256-row LDS tile: row
  // base + 32m + l, chunk 2ks + h lands at row*8 + ((2ks + h) ^ f(row)) with
  // f(row) = (l ^ (l >> 3) ^ 4(m & 1)) & 7, so only xo[ks ^ 2(m & 1)] varies.
  const int l = lane & 31, h = lane >> 5;
  const int v = h ^ ((l ^ (l >> 3)) & 7);
  int xo[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) xo[c] = l * 8 + (v ^ (2 * c));
  const int a_base = wr * 128 * 8, b_base = wc * 128 * 8;

  f32x16_t acc[4][4];
#pragma unroll
  for (int ma = 0; ma < 4; ++ma)
#pragma unroll
    for (int na = 0; na < 4; ++na)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[ma][na][r] = 0.0f;

  u32x4 ra[8], rb[8];
  int32_t idx[8];
  const int64_t k0 = it.k0, k1 = it.k1;
  const int n_stages = static_cast<int>((k1 - k0 + kKs - 1) / kKs);
  const int64_t tk = k0 + kb * 8;  // this thread's first token of stage 0
  if (n_stages > 0) {
    load_index<GATHER>(row_index, tk, k1, idx);
    load_rows<GATHER>(X, ldx, n_rows, idx, tk, k1, chanA, chanB, ra, rb);
    if (n_stages > 1) load_index<GATHER>(row_index, tk + kKs, k1, idx);
    mask_rows(tk, k1, okA, ra);
    mask_rows(tk, k1, okB, rb);
    store_block(lds[0][0], cb, u, ra);
    if (!diag) store_block(lds[0][1], cb, u, rb);
  }
  __syncthreads();
  for (int s = 0; s < n_stages; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < n_stages;
    const int64_t t1 = tk + static_cast<int64_t>(s + 1) * kKs;  // stage s+1
    if (more) {
      load_rows<GATHER>(X, ldx, n_rows, idx, t1, k1, chanA, chanB, ra, rb);
      if (s + 2 < n_stages) load_index<GATHER>(row_index, t1 + kKs, k1, idx);
    }
    const u32x4* A = lds[buf][0] + a_base;
    const u32x4* B = (diag ? lds[buf][0] : lds[buf][1]) + b_base;
#pragma unroll
    for (int ks = 0; ks < kKs / 16; ++ks) {
      bf16x8_t af[4], bfv[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int off = m * 256 + xo[ks ^ (2 * (m & 1))];
        af[m] = __builtin_bit_cast(bf16x8_t, A[off]);
        bfv[m] = __builtin_bit_cast(bf16x8_t, B[off]);
      }
#pragma unroll
      for (int ma = 0; ma < 4; ++ma)
#pragma unroll
        for (int na = 0; na < 4; ++na)
          acc[ma][na] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ma], bfv[na], acc[ma][na], 0, 0, 0);
    }
    if (more) {
      mask_rows(t1, k1, okA, ra);
      mask_rows(t1, k1, okB, rb);
      store_block(lds[buf ^ 1][0], cb, u, ra);
      if (!diag) store_block(lds[buf ^ 1][1], cb, u, rb);
    }
    __syncthreads();
  }
  // Empty ranges (n_stages == 0) still flush, so an unrouted group gets H = 0.
  flush(acc, out, ld, direct, direct && accumulate, static_cast<uint32_t>(C), gi0, gj0, lane);
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
    *workspace_bytes = need + p.hdr.n_slots * static_cast<int64_t>(kTile) * kTile * 4;
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
  const int64_t need = h.plan_bytes + h.n_slots * static_cast<int64_t>(kTile) * kTile * 4;
  MGQ_REQUIRE(workspace != nullptr && workspace_bytes >= need, MGQ_ERR_WORKSPACE,
              "hessian workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)need);
  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  const HessItem* items = reinterpret_cast<const HessItem*>(ws + h.items_off);
  const SplitTile* split = reinterpret_cast<const SplitTile*>(ws + h.split_off);
  float* partials = reinterpret_cast<float*>(ws + h.plan_bytes);
  if (h.n_items > 0) {
    if (row_index) {
      syrk_tile_kernel<true><<<static_cast<unsigned>(h.n_items), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(X), n_rows, ldx, C, row_index, items, H, partials,
          accumulate);
    } else {
      syrk_tile_kernel<false><<<static_cast<unsigned>(h.n_items), kThreads, 0, s>>>(
          static_cast<const uint16_t*>(X), n_rows, ldx, C, nullptr, items, H, partials,
          accumulate);
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
