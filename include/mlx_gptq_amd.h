/*
 * mlx_gptq_amd.h -- C ABI of the MI355X-native GPTQ calibration solver.
 *
 * One shared library (libmlxgptq_hip.so, gfx950 code objects) replaces the
 * torch/numpy arithmetic behind the reference's Python solver API
 * (mlx_gptq/gptq.py, grid.py, packing.py, artifacts.py:30-39,
 * capture.py:68-76). Each entry point below names the reference function it
 * replaces as file:line, relative to the reference repository root.
 *
 * Conventions
 *   - Plain C types only: device pointers, sizes, dtype/mode codes and a
 *     hipStream_t passed as `void* stream` (0 = legacy default stream). All
 *     work is enqueued on that stream; no call synchronises the device unless
 *     its comment says so.
 *   - Tensors are dense and row-major ("contiguous"); a [..., k] tensor is
 *     passed as (pointer, n_groups = prod(leading dims), k).
 *   - Return value: MGQ_OK (0) or a negative status. mgq_last_error() returns
 *     the message of the calling thread's most recent failure. The Python
 *     layer maps MGQ_ERR_VALUE -> ValueError, MGQ_ERR_SHAPE -> AssertionError,
 *     MGQ_ERR_NOT_PD -> RuntimeError, as the reference raises them.
 *   - Entry points are reentrant: they keep no mutable global state, so one
 *     host thread per device may call them concurrently (the reference's
 *     thread-per-device solve, sequential.py:610-626). The one exception is
 *     mgq_gptq_mxfp_noalloc, whose calls on one GPU share its scratch array
 *     (see there).
 *   - Nothing here allocates device memory. Entry points that need scratch
 *     take a caller-owned `workspace` of at least the size reported by the
 *     matching *_workspace_size query.
 */
#ifndef MLX_GPTQ_AMD_H
#define MLX_GPTQ_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define MGQ_OK 0
#define MGQ_ERR_VALUE (-1)     /* unsupported mode / bits / algorithm          */
#define MGQ_ERR_SHAPE (-2)     /* shape or divisibility violation              */
#define MGQ_ERR_NOT_PD (-3)    /* Hessian not PD after damping escalation      */
#define MGQ_ERR_HIP (-4)       /* HIP runtime / launch failure                 */
#define MGQ_ERR_WORKSPACE (-5) /* workspace missing or too small               */

/* ---- dtype / mode / method codes --------------------------------------- */
#define MGQ_DTYPE_F32 0
#define MGQ_DTYPE_BF16 1
#define MGQ_DTYPE_F16 2

#define MGQ_MODE_AFFINE 0
#define MGQ_MODE_MXFP4 1
#define MGQ_MODE_MXFP8 2

#define MGQ_CLIP_MINMAX 0
#define MGQ_CLIP_MSE 1

/* Library version (major*10000 + minor*100 + patch). */
int mgq_version(void);

/* Message of this thread's last failed call ("" if none). */
const char* mgq_last_error(void);

/* ======================================================================== *
 * Quantization grids -- mlx_gptq/grid.py                                    *
 * ======================================================================== */

/* grid.py:61-79 choose_mxfp_scale(w, mode).
 * w: f32 [n_groups, group_len] -> scale_bytes u8 [n_groups] (E8M0, e+127),
 * scales f32 [n_groups] (= 2^e). mode: MGQ_MODE_MXFP4 (fmax 6) or _MXFP8
 * (fmax 448). */
int mgq_choose_mxfp_scale(const float* w, int64_t n_groups, int64_t group_len, int mode,
                          uint8_t* scale_bytes, float* scales, void* stream);

/* grid.py:108-124 quantize_mxfp_with_scale(w, scales, mode).
 * w: f32 [n_groups, group_len], scales: f32 [n_groups] ->
 * q u8 and dq f32, both [n_groups, group_len]. */
int mgq_quantize_mxfp_with_scale(const float* w, const float* scales, int64_t n_groups,
                                 int64_t group_len, int mode, uint8_t* q, float* dq,
                                 void* stream);

/* grid.py:127-139 dequantize_mxfp(q, scale_bytes, mode).
 * q: u8 [n_groups, 32], scale_bytes: u8 [n_groups] -> out f32 [n_groups, 32]. */
int mgq_dequantize_mxfp(const uint8_t* q, const uint8_t* scale_bytes, int64_t n_groups,
                        int mode, float* out, void* stream);

/* grid.py:142-151 rtn_quantize_mxfp(W, mode).
 * W: [rows, cols] of w_dtype (f32/bf16/f16, read as f32), cols % 32 == 0 ->
 * q u8 [rows, cols], scale_bytes u8 [rows, cols/32], dq f32 [rows, cols]. */
int mgq_rtn_quantize_mxfp(const void* W, int w_dtype, int64_t rows, int64_t cols, int mode,
                          uint8_t* q, uint8_t* scale_bytes, float* dq, void* stream);

/* grid.py:154-164 dequantize_artifact, affine branch: q*scale + bias.
 * q: u8 [n_groups, group_size]; scales, biases: storage_dtype [n_groups]. */
int mgq_dequantize_affine(const uint8_t* q, const void* scales, const void* biases,
                          int storage_dtype, int64_t n_groups, int64_t group_size, float* out,
                          void* stream);

/* validate_artifacts.py:15-68 range audit of one artifact, fused: dequantize
 * (grid.py:154-164) and, per 32-column group, compare max|deq| with
 * max(32 * max|source|, 2^-126), in one pass.
 * source: [rows, cols] of source_dtype; q: u8 [rows, cols]; scales: u8 E8M0
 * [rows, cols/32] (mxfp) or storage_dtype [rows, cols/group_size] with
 * biases alike (affine). stats: u64[5] on the device, zeroed by the caller:
 * [0] non-finite dequantized values, [1] groups over the limit, [2] max
 * ratio (fp64 bits), [3] max |source| (fp32 bits), [4] max |deq| (fp32 bits). */
int mgq_range_audit(const void* source, int source_dtype, const uint8_t* q, const void* scales,
                    const void* biases, int storage_dtype, int mode, int64_t rows, int64_t cols,
                    int64_t group_size, unsigned long long* stats, void* stream);

/* grid.py:167-212 choose_qparams(w, bits, method, storage_dtype, grid_steps,
 * max_shrink). w: f32 [n_groups, group_len] -> s_store, b_store in
 * storage_dtype and s32, b32 f32, all [n_groups]. method: MGQ_CLIP_*. */
int mgq_choose_qparams(const float* w, int64_t n_groups, int64_t group_len, int bits,
                       int method, int storage_dtype, int grid_steps, double max_shrink,
                       void* s_store, void* b_store, float* s32, float* b32, void* stream);

/* grid.py:215-221 quantize_with_params(w, s32, b32, bits).
 * w: f32 [n_groups, group_len]; s32, b32: f32 [n_groups] -> q f32, dq f32. */
int mgq_quantize_with_params(const float* w, const float* s32, const float* b32,
                             int64_t n_groups, int64_t group_len, int bits, float* q, float* dq,
                             void* stream);

/* grid.py:224-246 rtn_quantize(W, bits, group_size, method, storage_dtype).
 * W: [rows, cols] of w_dtype -> q u8 [rows, cols], s_store/b_store
 * storage_dtype [rows, cols/group_size], dq f32 [rows, cols]. Uses the
 * reference's default grid (20 steps, max_shrink 0.2). */
int mgq_rtn_quantize_affine(const void* W, int w_dtype, int64_t rows, int64_t cols, int bits,
                            int group_size, int method, int storage_dtype, uint8_t* q,
                            void* s_store, void* b_store, float* dq, void* stream);

/* ======================================================================== *
 * Packing -- mlx_gptq/packing.py, mlx_gptq/artifacts.py                     *
 * ======================================================================== */

/* packing.py:15-26 pack_q(q, bits): u8 [rows, cols] -> u32 [rows, cols*bits/32],
 * LSB-first, codes not masked (as the numpy original). bits in {2, 4, 8};
 * cols % (32/bits) == 0. pack_mxfp4 (packing.py:29-31) is bits = 4. */
int mgq_pack_q(const uint8_t* q, int64_t rows, int64_t cols, int bits, uint32_t* words,
               void* stream);

/* packing.py:34-39 unpack_q(words, bits, out_cols): u32 [rows, n_words] ->
 * u8 [rows, out_cols], out_cols <= n_words*32/bits. */
int mgq_unpack_q(const uint32_t* words, int64_t rows, int64_t n_words, int bits,
                 int64_t out_cols, uint8_t* q, void* stream);

/* artifacts.py:30-32 pack_nibbles(q): u8 [rows, cols] -> u8 [rows, cols/2],
 * byte = q[2k] | (q[2k+1] << 4) in uint8 arithmetic; cols even. */
int mgq_pack_nibbles(const uint8_t* q, int64_t rows, int64_t cols, uint8_t* packed,
                     void* stream);

/* artifacts.py:35-39 unpack_nibbles(p): u8 [rows, packed_cols] ->
 * u8 [rows, 2*packed_cols] (low nibble first). */
int mgq_unpack_nibbles(const uint8_t* packed, int64_t rows, int64_t packed_cols, uint8_t* q,
                       void* stream);

/* ======================================================================== *
 * Hessian accumulation -- mlx_gptq/capture.py:68-76 (Stash.hessian)        *
 * ======================================================================== */

/* Plan a grouped Hessian launch (host only, no device work).
 * Group g owns entries [offsets[g], offsets[g+1]) of the token list
 * (offsets: host int64 [n_groups+1], non-decreasing). target_items <= 0
 * picks a default grid size. With plan == NULL only the sizes are returned:
 * plan_bytes (host plan size) and workspace_bytes (device workspace size,
 * which includes the plan). Otherwise the plan is written to `plan`
 * (plan_capacity bytes available). */
int mgq_hessian_plan(int64_t C, int64_t n_groups, const int64_t* offsets, int64_t target_items,
                     void* plan, int64_t plan_capacity, int64_t* plan_bytes,
                     int64_t* workspace_bytes);

/* capture.py:68-76 Stash.hessian for every group at once:
 *   H[g] (+)= X_g^T X_g,  X_g = rows row_index[offsets[g] .. offsets[g+1])
 * of X (row_index == NULL: rows offsets[g] .. offsets[g+1] themselves).
 * X: bf16 [n_rows, ldx] (device, 16-byte aligned; C and ldx multiples of 8;
 * C <= 46340), row_index entries must lie in [0, n_rows) (out-of-range
 * entries are clamped, never dereferenced) and the list must hold at least
 * offsets[n_groups] entries,
 * row_index: int32 device array or NULL, H: f32 [n_groups, C, C] device.
 * accumulate = 0 overwrites H, 1 adds into it. H comes out exactly
 * symmetric. plan_host: the plan from mgq_hessian_plan; the caller must have
 * copied it (plan_bytes) to the start of `workspace` before this call, in
 * stream order. bf16 x bf16 products are exact in fp32 and accumulated by
 * v_mfma_f32_32x32x16_bf16. */
int mgq_hessian(const void* X, int64_t n_rows, int64_t ldx, int64_t C,
                const int32_t* row_index, const void* plan_host, float* H, int accumulate, void* workspace,
                int64_t workspace_bytes, void* stream);

/* ======================================================================== *
 * Solver -- mlx_gptq/gptq.py                                                *
 * ======================================================================== */

/* gptq.py:27-66 _prepare_hinv for every 32x32 diagonal block:
 * U[b, g] (upper, f32 [B, C/32, 32, 32]) with U^T U = (Hb + lam I)^-1,
 * lam = damp * max(mean(diag Hb), 1e-8), damp escalated x10 per block up to
 * max_attempts times. attempts[g*B + b] = attempts used (1..max_attempts),
 * or 0 when every attempt failed (the reference's RuntimeError case; U is
 * zero there). H: f32 [B, C, C], C % 32 == 0; block must be 32. */
int mgq_prepare_hinv_blocks(const float* H, int64_t B, int64_t C, int64_t block, float damp,
                            int max_attempts, float* U, int32_t* attempts, void* stream);

/* Workspace bytes needed by mgq_gptq_mxfp for W [B, R, C]. */
int64_t mgq_gptq_mxfp_workspace_size(int64_t B, int64_t R, int64_t C);

/* gptq.py:183-272 gptq_quantize / 275-302 solve_gptq for mode mxfp4 / mxfp8
 * (gptq.py:69-180 _gptq_quantize_mxfp_groupwise), one launch sequence:
 *   dead-column fix (gptq.py:216-222: diag(H) <= 0 -> diagonal set to 1 in
 *   place in H, weights of that column treated as 0), per-group damped
 *   Cholesky-inverse (mgq_prepare_hinv_blocks), fused group solver.
 * W: [B, R, C] of w_dtype (f32 / bf16 / f16), H: f32 [B, C, C] (modified in
 * place as the reference does), C % 32 == 0. W, H, W_dq and q_out must be
 * 16-byte aligned (the kernels move 16-byte pieces; MGQ_ERR_SHAPE otherwise).
 * mode: MGQ_MODE_MXFP4 / MGQ_MODE_MXFP8. algorithm: 0 = groupwise,
 * 1 = safe-scale-search with exponent `offsets[n_offsets]` tried in order
 * (reference: {0,-1,-2,-3,-4,1,2} for mxfp4, {0,-1,1} for mxfp8; <= 8).
 * Outputs: q_out u8 [B, R, C], scales_out u8 [B, R, C/32] (E8M0),
 * W_dq f32 [B, R, C] (may alias W when w_dtype is f32), rel_err f32 [B]
 * (||W_dq - W||_F / max(||W||_F, 1e-12), NULL to skip), attempts i32
 * [C/32, B] (see mgq_prepare_hinv_blocks; any 0 means the reference would
 * raise its "not positive definite" RuntimeError -- outputs are then
 * unspecified). workspace: mgq_gptq_mxfp_workspace_size bytes. */
int mgq_gptq_mxfp(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C, float* H,
                  int mode, int algorithm, float damp, int max_attempts, const int32_t* offsets,
                  int n_offsets, uint8_t* q_out, uint8_t* scales_out, float* W_dq,
                  float* rel_err, int32_t* attempts, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* The two halves of mgq_gptq_mxfp, for a caller that wants the attempts
 * before the solve finishes. The reference computes _prepare_hinv
 * (gptq.py:27-66, after the dead-column fix of gptq.py:216-222) to
 * completion -- warnings and RuntimeError included -- before its group loop
 * (gptq.py:99-180); reading `attempts` after mgq_gptq_mxfp_prepare and before
 * the solve's outputs gives that order without waiting for the solve.
 * prepare: the dead-column fix (H in place) and the per-group damped
 * Cholesky-inverse into `workspace`, attempts as in mgq_gptq_mxfp.
 * solve: the fused group solver on a workspace prepared for the same
 * B, R, C (the same argument meanings as mgq_gptq_mxfp). */
int mgq_gptq_mxfp_prepare(float* H, int64_t B, int64_t R, int64_t C, float damp, int max_attempts,
                          int32_t* attempts, void* workspace, int64_t workspace_bytes, void* stream);
int mgq_gptq_mxfp_solve(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C, int mode,
                        int algorithm, const int32_t* offsets, int n_offsets, uint8_t* q_out,
                        uint8_t* scales_out, float* W_dq, float* rel_err, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* mgq_gptq_mxfp_solve followed by packing.py:15-26 pack_q of its codes
 * (what sequential.py / pack.py do with a solved projection's q), in the
 * solver's own launch: packed_out (u32 [B, R, C / 8] for mxfp4, [B, R, C / 4]
 * for mxfp8, 16-byte aligned) receives exactly mgq_pack_q(q_out, bits), and
 * the codes are not read back from HBM by a separate packing pass. Every
 * other argument and result as mgq_gptq_mxfp_solve. */
int mgq_gptq_mxfp_solve_packed(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C,
                               int mode, int algorithm, const int32_t* offsets, int n_offsets,
                               uint8_t* q_out, uint32_t* packed_out, uint8_t* scales_out,
                               float* W_dq, float* rel_err, void* workspace,
                               int64_t workspace_bytes, void* stream);

/* gptq.py:300-302 rel_err of an affine (or any) solve: rel[b] =
 * ||W_dq[b] - W[b]||_F / max(||W[b]||_F, 1e-12), W_dq f32 [B, n], W [B, n] of
 * w_dtype (f32 / bf16 / f16, read as it is), both contiguous. partials:
 * double [B, n_partials, 2] scratch (1 <= n_partials <= 65535; each partial
 * sums about n / n_partials elements in double, in a fixed order, so rel is
 * deterministic); B <= 65535. */
int mgq_rel_err(const float* W_dq, const void* W, int w_dtype, int64_t B, int64_t n,
                double* partials, int64_t n_partials, float* rel, void* stream);

/* Allocation-free variant of mgq_gptq_mxfp. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and results as mgq_gptq_mxfp without the
 * workspace: the solver's scratch is a fixed per-GPU device array of
 * mgq_noalloc_scratch_bytes() bytes (32 MiB) that the library holds on every
 * GPU it runs on until the process ends. Calls needing more than that
 * (mgq_gptq_mxfp_workspace_size(B, R, C)) fail with MGQ_ERR_WORKSPACE before
 * anything is launched; split the batch. The stream must belong to the
 * current device. All calls on one GPU share its array: calls that overlap
 * on one GPU race and must be serialised by the caller. Allocates nothing. */
int64_t mgq_noalloc_scratch_bytes(void);
int mgq_gptq_mxfp_noalloc(const void* W, int w_dtype, int64_t B, int64_t R, int64_t C, float* H,
                          int mode, int algorithm, float damp, int max_attempts,
                          const int32_t* offsets, int n_offsets, uint8_t* q_out,
                          uint8_t* scales_out, float* W_dq, float* rel_err, int32_t* attempts,
                          void* stream);

/* Workspace bytes needed by mgq_hinv_full_pass for H [B, C, C] (two fp64
 * [B, C, C] arrays). */
int64_t mgq_hinv_full_workspace_size(int64_t B, int64_t C);

/* One damping attempt of gptq.py:27-66 _prepare_hinv on full [C, C]
 * matrices (the affine solver's factor, gptq.py:229): for every item with
 * active[b] != 0, U[b] (f32 upper, zero below the diagonal) with
 *   U^T U = (H[b] + lam_b I)^-1,  lam_b = damp[b] * max(mean(diag H[b]), 1e-8).
 * Factorisation and inverse run in fp64 (blocked UL Cholesky, nb = 64) and
 * are rounded to f32 once. failed[b] is set to 1 (and U[b] left unwritten)
 * when a pivot is <= 0 or NaN; the caller clears failed[] before the call.
 * The reference's escalation (damp x10 for the failed items only, up to 6
 * attempts) is the caller's loop over this pass with active = failed.
 * damp: f32 [B], active/failed: u8 [B], all device. */
int mgq_hinv_full_pass(const float* H, int64_t B, int64_t C, const float* damp,
                       const uint8_t* active, uint8_t* failed, float* U, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* gptq.py:216-222: dead columns (diag(H) <= 0) are zeroed in W f32
 * [B, R, C] (W may be NULL) and their H diagonal set to 1, in place. */
int mgq_dead_fix(float* W, int64_t B, int64_t R, int64_t C, float* H, void* stream);

/* One lazy block [i1, i1 + n) of the affine column loop, gptq.py:241-270:
 * every G-column group starts with grid.py:167-212 choose_qparams on the
 * block-updated weights (scales/biases stored in storage_dtype at group
 * index col / G), then each column is quantized (grid.py:215-221), its
 * error e = (w - dq) / U[c, c] is propagated to the block's later columns
 * and stored in Err; afterwards W[:, :, i1+n:] -= Err @ U[i1:i1+n, i1+n:]
 * (gptq.py:269-270). W f32 [B, R, C] (columns of the block become dq),
 * U f32 [B, C, C] from mgq_hinv_full_pass, q_out u8 [B, R, C],
 * s_store / b_store [B, R, C/G] of storage_dtype, Err f32 [B, R, n].
 * G <= 128, C, i1 and n multiples of G, n <= 2048. */
int mgq_gptq_affine_block(float* W, const float* U, int64_t B, int64_t R, int64_t C, int64_t i1,
                          int64_t n, int group_size, int bits, int method, int storage_dtype,
                          int grid_steps, double max_shrink, uint8_t* q_out, void* s_store,
                          void* b_store, float* Err, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLX_GPTQ_AMD_H */
