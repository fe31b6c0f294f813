/*
 * hi2x — MI355X (gfx950) encode path of the hi2 / rdna_hint_flex quantizer.
 *
 * C ABI of libhi2x.so.  Every buffer argument is a raw device pointer (the library
 * borrows it for the duration of the call and never frees it); sizes are int64;
 * `stream` is a hipStream_t passed as void*.  Calls are asynchronous on `stream`
 * unless stated otherwise.  Every entry returns an int status:
 *
 *   HI2X_OK (0), HI2X_EINVAL (bad argument), HI2X_ENOTPD (matrix not positive
 *   definite), HI2X_ELAUNCH (a HIP call failed), HI2X_ERANGE (a code outside the
 *   ladder).  hi2x_last_error() returns the calling thread's last message.
 *
 * The last-error text is thread-local, so one host thread per device may call the
 * library concurrently.  Process-wide mutable state, each piece guarded by its own lock:
 *   - the opt-in launch-timing record of the measurement section at the end
 *     (hi2x_timing_*), which the encode path never reads;
 *   - the set of streams marked background (hi2x_stream_background), read by every
 *     GPTQ cross-block update launch to size its LDS reservation (a scheduling hint:
 *     results are unchanged); callers clear their marks when their chains end;
 *   - the per-device address of the 64 MiB error array of hi2x_gptq_run_noalloc,
 *     looked up once per device.  The array itself is part of the library's code
 *     object, so it is resident on every GPU the library's GPTQ kernels are loaded on,
 *     whether or not that entry point is called.
 * No kernel of the library uses a private (scratch) segment, so no launch makes the HIP
 * runtime allocate device memory.
 *
 * Reference interfaces are cited as path:line of BlivionIaG/hi2.
 */
#ifndef HI2X_H
#define HI2X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HI2X_OK 0
#define HI2X_EINVAL (-1)
#define HI2X_ENOTPD (-2)
#define HI2X_ELAUNCH (-3)
#define HI2X_ERANGE (-4)

#define HI2X_BLOCK_COLUMNS 128 /* GPTQ lazy block (hi2/hessian.py:20) */

/* Library version (major*10000 + minor*100 + patch). */
int hi2x_version(void);

/* Last error message of the calling thread ("" if none). */
const char* hi2x_last_error(void);

/* ---- GPTQ ------------------------------------------------------------------------ */

/* One lazy block of the GPTQ column loop for every row of a batch.
 * Replaces the fused kernel launched by hi2/gptq_kernel.py:103-127 (`gptq_block`,
 * Python entry hi2/gptq_kernel.py:187-196), same arguments and meaning:
 *   wc [n, k] f32 (read only; columns in rounding order), err1 [n, len] f32 out,
 *   codes [n, k] u8 out (rounding-order positions i1..i1+len), lo/st [n, ldp] f32
 *   decoded block params, row_grp [n] i32 (sorted ascending), u_ptrs [G] i64 device
 *   addresses of contiguous [k, k] f32 factors, blk [G, k] i32 block of each column,
 *   nmax [G] f32 (codes - 1), comp [n, k] f32 out or NULL.  Consecutive groups with
 *   the same u_ptrs address form one run: their rows share one pass (each row with its
 *   own group's blk and nmax), so they need no padding between them; a workgroup of 16
 *   rows holding rows of two factors runs once per factor (same results, slower).
 * Bit-exact to the reference column loop (hi2/hessian.py:248-261). */
int hi2x_gptq_block(const float* wc, int64_t n, int64_t k, int64_t i1, int64_t len,
                    float* err1, uint8_t* codes, const float* lo, const float* st,
                    int64_t ldp, const int32_t* row_grp, const int64_t* u_ptrs,
                    const int32_t* blk, const float* nmax, float* comp, void* stream);

/* Cross-block update of hi2/hessian.py:310-312 for every row r (group g):
 *   wc[r, c] -= err1[r, :len] @ U_g[i1:i1+len, c]   for c in [c0, c1)
 * err1 [n, lde] f32.  Each product is a sequential fp32 FMA chain over the rank in
 * order, then one subtraction: the rounding of the reference's BLAS call.  A tile whose
 * rows all have one factor address (any number of groups) is one pass; a tile of several
 * factors runs one masked pass per run of equal addresses. */
int hi2x_gptq_trailing(float* wc, int64_t n, int64_t k, int64_t i1, int64_t len,
                       const float* err1, int64_t lde, int64_t c0, int64_t c1,
                       const int32_t* row_grp, const int64_t* u_ptrs, void* stream);

/* The whole column loop of _round_kernel (hi2/hessian.py:267-315): for every
 * 128-column block, hi2x_gptq_block then the cross-block update, with the updates
 * of `super_blocks` consecutive blocks applied to the far columns in one pass
 * (each block's product still subtracted separately, in block order, so the result
 * is bit-identical to the per-block schedule).  wc is modified in place.
 * err_ws: device workspace of n * 128 * super_blocks floats. */
int hi2x_gptq_run(float* wc, int64_t n, int64_t k, uint8_t* codes, const float* lo,
                  const float* st, int64_t ldp, const int32_t* row_grp,
                  const int64_t* u_ptrs, const int32_t* blk, const float* nmax,
                  float* comp, float* err_ws, int64_t super_blocks, void* stream);

/* hi2x_gptq_run without allocation: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same computation and results as hi2x_gptq_run,
 * with its error workspace taken from a 64 MiB array the library holds on each GPU it
 * runs on until the process ends (n * 128 * super_blocks * 4 bytes must fit: HI2X_EINVAL
 * otherwise, before anything is launched).  Calls no allocating routine; call it with the
 * stream's device current.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (concurrent streams or host threads) race and must be serialised
 * by the caller. */
int hi2x_gptq_run_noalloc(float* wc, int64_t n, int64_t k, uint8_t* codes, const float* lo,
                          const float* st, int64_t ldp, const int32_t* row_grp,
                          const int64_t* u_ptrs, const int32_t* blk, const float* nmax,
                          float* comp, int64_t super_blocks, void* stream);

/* ---- ladder fit and block parameters ---------------------------------------------- */

/* fit_ladder (hi2/encode.py:53-92; grid part = ladder_grid_k, hi2/ladder_kernel.py:44-86):
 * w [rows, k] f32 (stored basis, rows contiguous), d [k] f32 = diag(Hs), block B in
 * {16,32,64}, nlev = 2^nbits, grid [g] f32, ls refits.  Outputs lo, step [rows, k/B].
 * err (optional, [rows, k/B]) receives the best weighted error.  Sums follow the
 * reference's torch CPU order, so results are bit-identical to hi2.encode.fit_ladder. */
int hi2x_ladder_fit(const float* w, const float* d, int64_t rows, int64_t k, int64_t block,
                    int nlev, const float* grid, int g, int ls, float* lo, float* step,
                    float* err, void* stream);

/* hi2x_ladder_fit for rows of several jobs at once (the per-chunk fits of _prepare,
 * hi2/hessian.py:208-232, each chunk with its own job's d): row r is fitted with the
 * weights d + d_row[r] * k (d is [G, k] f32, d_row [rows] i32 device arrays).  Results
 * equal hi2x_ladder_fit on each row with its own d. */
int hi2x_ladder_fit_rows(const float* w, const float* d, const int32_t* d_row, int64_t rows,
                         int64_t k, int64_t block, int nlev, const float* grid, int g,
                         int ls, float* lo, float* step, float* err, void* stream);

/* quantize_params + decode_params (hi2/encode.py:95-119, hi2/format.py:45-60):
 * lo, step [rows, nb] -> lo_u8, step_u8 [rows, nb], consts [rows, 3] fp16 bits
 * (lo_min, lo_scale, step_scale), lo_d, step_d [rows, ldd] f32 decoded values
 * (ldd >= nb; padding untouched).  lo_d/step_d may be NULL. */
int hi2x_params(const float* lo, const float* step, int64_t rows, int64_t nb,
                uint8_t* lo_u8, uint8_t* step_u8, uint16_t* consts, float* lo_d,
                float* step_d, int64_t ldd, void* stream);

/* decode_params alone (hi2/format.py:45-60) on [rows, nb] bytes with per-row constants
 * consts [rows, 3] fp16 bits; outputs fp16 bits lo_h, step_h [rows, nb]. */
int hi2x_decode_params(const uint8_t* lo_u8, const uint8_t* step_u8, const uint16_t* consts,
                       int64_t rows, int64_t nb, uint16_t* lo_h, uint16_t* step_h,
                       void* stream);

/* _finish (hi2/hessian.py:318-345): codes_ro/comp_ro [n, k] in rounding order ->
 * codes/comp in column order (perm [k] i64 or NULL), sse [n] = sum_c d_c (rec - w)^2
 * with rec = fp16(lo + code*step) in f32 and the sum in torch's CPU order.
 * lo_d/step_d [n, ldd] f32, w [n, k] f32 original rows, d [k] f32.  With perm NULL,
 * codes == codes_ro and comp == comp_ro (aliases) are allowed: then only sse is written. */
int hi2x_finish(const uint8_t* codes_ro, const float* comp_ro, const int64_t* perm,
                int64_t n, int64_t k, int64_t block, const float* lo_d, const float* step_d,
                int64_t ldd, const float* w, const float* d, uint8_t* codes, float* comp,
                float* sse, void* stream);

/* One group of rows of a batch for hi2x_finish_rows: rows [row0, row0 + rows) of the
 * batch are the uncompensated rows w [rows, k] f32 (stored basis, rounding order =
 * storage order), weighted by d [k] f32, on ladders of `block` columns. */
typedef struct hi2x_rows_group {
  const float* w;
  const float* d;
  int64_t row0;
  int64_t rows;
  int64_t block;
} hi2x_rows_group;

/* The sse of _finish (hi2/hessian.py:318-345, without a column permutation) for every
 * row of a batch of several jobs at once: row r belongs to groups[row_grp[r]] (a device
 * array of G groups; row_grp [n] i32 on the device); codes [n, k] u8, lo_d/step_d
 * [n, ldd] f32 (ldd >= k / 16) in batch layout.  sse [n] f32 equals hi2x_finish's on each
 * group; rows outside their group's range (padding) are left unwritten. */
int hi2x_finish_rows(const uint8_t* codes, int64_t n, int64_t k, const float* lo_d,
                     const float* step_d, int64_t ldd, const int32_t* row_grp,
                     const hi2x_rows_group* groups, float* sse, void* stream);

/* The codes of encode_rows (hi2/encode.py:151-155), nearest rounding onto the fitted
 * ladders: codes [rows, k] u8 = clamp(st == 0 ? 0 : rint((w - lo) / st), 0, 2^nbits - 1)
 * with w [rows, k] f32 (16-byte aligned), lo_d/st_d [rows, ldd] f32 the decoded ladder of
 * each block of `block` columns.  With hi2x_ladder_fit, hi2x_params and hi2x_finish (the
 * sse) it is the whole of encode_rows: no factor, no error propagation. */
int hi2x_nearest_codes(const float* w, int64_t rows, int64_t k, int64_t block,
                       const float* lo_d, const float* st_d, int64_t ldd, int nbits,
                       uint8_t* codes, void* stream);

/* ladder_dequantize (hi2/format.py:63-69): out_h [rows, nb*B] fp16 bits of
 * lo + code*step evaluated in f32 (f64 when exact != 0), one rounding to fp16.
 * lo/step [rows, nb] f32. */
int hi2x_ladder_dequantize(const uint8_t* codes, const float* lo, const float* step,
                           int64_t rows, int64_t nb, int64_t block, int exact,
                           uint16_t* out_h, void* stream);

/* ---- format ------------------------------------------------------------------------ */

/* fwht_groups (hi2/format.py:30-41): flagged 16-column groups of x [rows, k] times
 * the normalised order-16 Hadamard (an involution).  dtype: 0 = f32, 1 = f64 (in and
 * out share the dtype; sums in the reference matmul's sequential order). */
int hi2x_fwht16(const void* x, void* y, int dtype, int64_t rows, int64_t k,
                const uint8_t* flags, void* stream);

/* fwht_groups(w.float() * col_scale, flags)[rows] in one pass: the reference's smoothing
 * (hi2/calibrate.py:106-111), staging to fp32 and rotation (hi2/calibrate.py:329-330,
 * fwht_groups hi2/format.py:30-41) and row selection per candidate
 * (hi2/calibrate.py:353-357): w [nw, ldw] f32 (dtype 0) or bf16 (dtype 2), rows [n]
 * i64 device indices (null: rows 0..n-1; an index outside [0, nw) yields a row of NaN),
 * col_scale [k] f32 (null: none), flags [k/16] u8 (null: no group transformed); out
 * [n, ldo] f32.  Rows 16-byte aligned.  Bit-identical to the cast, the product and
 * hi2x_fwht16 in turn. */
int hi2x_rotate_rows(const void* w, int dtype, int64_t ldw, int64_t nw, const int64_t* rows,
                     int64_t n, int64_t k, const float* col_scale, const uint8_t* flags,
                     float* out, int64_t ldo, void* stream);

/* pack_codes (hi2/format.py:73-85): codes [rows, k] u8 -> words [rows, k*nbits/32]
 * i32, LSB first.  bad: device i32 counter incremented per code >= 2^nbits (the
 * caller raises ValueError when nonzero). */
int hi2x_pack_codes(const uint8_t* codes, int64_t rows, int64_t k, int nbits,
                    int32_t* words, int32_t* bad, void* stream);

/* One piece of assemble (hi2/format.py:155-171): rows [r] i64 tensor-row indices,
 * codes [r, k] u8, params [r, k/block, 2] u8, consts [r, 3] fp16 bits scattered into
 * the flat buffers out_codes (i32 words at code_off[row]), out_params (2 bytes per
 * block at param_off[row]), out_consts [R, 3].  code_off/param_off are i64 device
 * arrays.  bad as in hi2x_pack_codes. */
int hi2x_assemble_piece(const int64_t* rows, int64_t r, const uint8_t* codes,
                        const uint8_t* params, const uint16_t* consts, int64_t k, int nbits,
                        int64_t block, const int64_t* code_off, const int64_t* param_off,
                        int32_t* out_codes, uint8_t* out_params, uint16_t* out_consts,
                        int32_t* bad, void* stream);

/* One piece of hi2x_assemble_batch: the arguments of hi2x_assemble_piece. */
typedef struct hi2x_piece {
  const int64_t* rows;
  int64_t r;
  const uint8_t* codes;
  const uint8_t* params;
  const uint16_t* consts;
  int64_t k;
  int32_t nbits;
  int32_t pad_;
  int64_t block;
  const int64_t* code_off;
  const int64_t* param_off;
  int32_t* out_codes;
  uint8_t* out_params;
  uint16_t* out_consts;
} hi2x_piece;

/* hi2x_assemble_piece for n_pieces pieces (pieces: a host array) in one call, in order,
 * sharing the range counter bad: the packing of many tensors (every expert of an MoE
 * layer) without a call per piece.  The reference assembles one tensor at a time
 * (hi2/format.py:127-184); the result is the same. */
int hi2x_assemble_batch(const hi2x_piece* pieces, int64_t n_pieces, int32_t* bad, void* stream);

/* ---- Hessian ------------------------------------------------------------------------ */

/* Workspaces.  Entry points that need device scratch take (ws, ws_bytes): a 256-byte
 * aligned device buffer of at least the size the matching *_workspace_bytes query
 * returns (-1 for bad arguments).  ws = NULL makes the library allocate it stream-ordered
 * (hipMallocAsync) and release it after the call's work; callers that run several
 * streams at once should pass their own, since a block the allocator hands from one
 * stream to another orders the two streams. */

/* Workspace of hi2x_hessian_syrk for t rows of width k (0 for f32 input). */
int64_t hi2x_hessian_workspace_bytes(int dtype, int64_t t, int64_t k);

/* HessianStats.update (hi2/hessian.py:35-40): s [k, k] f32 += x^T x over t rows of
 * x [t, k] (dtype 0 = f32, 2 = bf16).  bf16 runs on bf16 MFMA with f32 accumulation
 * (products exact); f32 on f32 MFMA.  The result is exactly symmetric. */
int hi2x_hessian_syrk(const void* x, int dtype, int64_t t, int64_t k, float* s, void* ws,
                      int64_t ws_bytes, void* stream);

/* As hi2x_hessian_syrk, but only the upper triangle (i <= j) of s is brought up to date
 * (bf16; f32 input still writes both): for callers that read the sum through
 * hi2x_sigma_transform_upper, or mirror it later with hi2x_hessian_mirror.  The split of
 * HessianStats.update's symmetric result into these two steps has no counterpart in the
 * reference (hi2/hessian.py:35-40 keeps the full matrix). */
int hi2x_hessian_syrk_upper(const void* x, int dtype, int64_t t, int64_t k, float* s,
                            void* ws, int64_t ws_bytes, void* stream);

/* s[j][i] = s[i][j] for i < j: the lower triangle from the upper. */
int hi2x_hessian_mirror(float* s, int64_t k, void* stream);

/* Workspace of hi2x_hessian_syrk_grouped (-1 for bad arguments). */
int64_t hi2x_hessian_grouped_workspace_bytes(int64_t t_total, int64_t n_groups, int64_t k);

/* HessianStats.update of every expert of an MoE layer from one routed token batch, in one
 * launch sequence (the per-expert calls of hi2/moe.py:83-100 -> hi2/hessian.py:35-40):
 * group e accumulates the tokens j in [offs[e], offs[e+1]) into s + e * s_stride
 * ([k, k] f32, s_stride >= k * k), token j being row rows[j] of x [x_rows, k] bf16
 * (dtype 2), or row j when rows is NULL (a batch already sorted by expert).  offs
 * (n_groups + 1 entries, ascending within [0, t_total]) and rows (t_total entries) are
 * device arrays: the token counts never travel to the host.  A group outside that
 * range counts as empty, a row outside [0, x_rows) as zeros.  The groups run largest
 * first over one transposed, gathered copy of the tokens; upper_only != 0 leaves the
 * lower triangles stale (as hi2x_hessian_syrk_upper).  At most 4M tokens per call. */
int hi2x_hessian_syrk_grouped(const void* x, int64_t x_rows, int dtype, const int64_t* rows,
                              const int64_t* offs, int64_t n_groups, int64_t t_total,
                              int64_t k, float* s, int64_t s_stride, int upper_only, void* ws,
                              int64_t ws_bytes, void* stream);

/* transform_sigma (hi2/hessian.py:50-68): hs [k, k] f32 = sym(M diag(1/s) sigma
 * diag(1/s) M^T) with M block-diagonal (H16/4 on flagged groups, I elsewhere).
 * col_scale: fp16 bits [k] or NULL; had [k/16] u8.  Bit-identical to the reference's
 * fp32 einsum order. */
int hi2x_sigma_transform(const float* sigma, const uint16_t* col_scale, const uint8_t* had,
                         int64_t k, float* hs, void* stream);

/* transform_sigma(HessianStats.mean()) (hi2/hessian.py:46-47 then 50-68) in one pass from
 * the upper triangle of the running sum s [k, k] over n rows: sigma = s / max(n, 1) by
 * IEEE division (the reference's CPU mean), then exactly the ops of
 * hi2x_sigma_transform.  The lower triangle of s is not read. */
int hi2x_sigma_transform_upper(const float* s, int64_t n, const uint16_t* col_scale,
                               const uint8_t* had, int64_t k, float* hs, void* stream);

/* hi2x_sigma_transform_upper for `batch` running sums of one size at once (the experts of
 * an MoE projection, each factored on its own input by hi2/calibrate.py:332-348): matrix z
 * at s + z * s_stride over n[z] tokens (device int64 [batch]) into hs + z * hs_stride
 * (strides in floats, >= k * k), every matrix with the same col_scale and had. */
int hi2x_sigma_transform_upper_batched(const float* s, int64_t s_stride, const int64_t* n,
                                       int64_t batch, const uint16_t* col_scale,
                                       const uint8_t* had, int64_t k, float* hs,
                                       int64_t hs_stride, void* stream);

/* The MoE token floor on the experts' Hessians (hi2/layerwise.py:245-257 through
 * hi2/moe.py:152-156 blend): with tot = the fp32 sum of the n_groups sums s + e * s_stride
 * in expert order (taken before any changes), every expert with mask[e] != 0 (device u8)
 * becomes s_e + fill[e] * tot (fill: device f32, the fp32 value of (need - n_e) / n_total),
 * elementwise in fp32 as the reference's torch ops; the upper triangle only when
 * upper_only != 0.  The caller sets the topped-up experts' counts to `need`. */
int hi2x_hessian_blend(float* s, int64_t s_stride, int64_t n_groups, int64_t k,
                       const float* fill, const uint8_t* mask, int upper_only, void* stream);

/* ---- Cholesky chain ------------------------------------------------------------------ */

/* The damping term of attempt `attempt` (hi2/hessian.py:75-79): *lam (device) =
 * damp * max(mean(diag hs), 1e-12) * 10^attempt in fp32, the mean reduced in the order
 * of torch's CPU sum of a strided vector.  The entry points below compute it the same
 * way. */
int hi2x_chol_lambda(const float* hs, int64_t k, float damp, int attempt, float* lam,
                     void* stream);

/* Workspace of the two entry points below for a k x k matrix. */
int64_t hi2x_chol_workspace_bytes(int64_t k);

/* One attempt of inverse_factor (hi2/hessian.py:71-86): with lam = damp * mean(diag hs)
 * (clamped at 1e-12) * 10^attempt, writes u [k, k] f32 = the upper Cholesky factor of
 * (hs + lam I)^-1 (lower triangle zero).  Computed as U = (J chol(J (hs + lam I) J) J)^-1
 * (J = reversal), the same matrix as the reference's chol -> cholesky_inverse ->
 * chol(upper) chain.  k is a multiple of 4 (the leaves move 16-byte vectors; the
 * reference's widths are multiples of 16, its golden factors multiples of 8).
 * Synchronises `stream`; returns
 * HI2X_ENOTPD when the damped matrix is not numerically positive definite (the caller
 * retries with attempt + 1). */
int hi2x_chol_inv_upper(const float* hs, int64_t k, float damp, int attempt, float* u,
                        void* ws, int64_t ws_bytes, void* stream);

/* Asynchronous form of hi2x_chol_inv_upper (same computation, same reference
 * interface hi2/hessian.py:71-86): nothing is synchronised; `status` (device i32)
 * receives 0x7fffffff when the factorisation succeeded, else 1 + the first row of the
 * failing 128-block, once `stream` reaches it.  Lets independent factors (one per
 * calibration input) run concurrently on separate streams. */
int hi2x_chol_inv_upper_async(const float* hs, int64_t k, float damp, int attempt, float* u,
                              int32_t* status, void* ws, int64_t ws_bytes, void* stream);

/* Workspace of hi2x_chol_inv_upper_batched_async for `batch` k x k matrices. */
int64_t hi2x_chol_batched_workspace_bytes(int64_t k, int64_t batch);

/* The first attempt of inverse_factor (hi2/hessian.py:71-86) for `batch` Hessians of one
 * size at once: the per-expert factors of an MoE projection (hi2/calibrate.py:332-348
 * factors each expert's input separately; the experts of hi2/moe.py share the size).
 * Matrix z: hs + z * hs_stride -> u + z * u_stride (strides in floats, >= k * k), status
 * word status[z] as in hi2x_chol_inv_upper_async.  Every kernel of the chain covers the
 * whole batch (grid z), so small factors fill the chip.  Nothing is synchronised; the
 * caller retries a failed z with hi2x_chol_inv_upper at attempt 1.. as the reference. */
int hi2x_chol_inv_upper_batched_async(const float* hs, int64_t hs_stride, int64_t k,
                                      int64_t batch, float damp, int attempt, float* u,
                                      int64_t u_stride, int32_t* status, void* ws,
                                      int64_t ws_bytes, void* stream);

/* ---- calibration statistics ------------------------------------------------------------ */

/* Workspace of hi2x_colstats_update for t tokens of width k (-1 for bad arguments). */
int64_t hi2x_colstats_workspace_bytes(int64_t t, int64_t k);

/* ColumnStats.update (hi2/stats.py:26-33): s [k/16, 16, 16] f64 += the 16 x 16 second
 * moments x_g^T x_g of every column group of x [t, k] (dtype 0 = f32, 2 = bf16), chunk by
 * chunk of 4096 tokens: each chunk's moments in fp32 (sub-chunks of 256 tokens, each a
 * sequential FMA chain, summed in order), then added to s in f64, chunks in order. */
int hi2x_colstats_update(const void* x, int dtype, int64_t t, int64_t k, double* s, void* ws,
                         int64_t ws_bytes, void* stream);

/* ColumnStats.diag (hi2/stats.py:39-55): out [k] f32 = E[x_j^2] of the activation
 * x * inv_scale (inv_scale f32 [k] or NULL), in the rotated basis where flags [k/16] u8
 * (or NULL: none) is set; s as above over n tokens. */
int hi2x_colstats_diag(const double* s, int64_t k, int64_t n, const uint8_t* flags,
                       const float* inv_scale, float* out, void* stream);

/* The cached-Sigma payload's triangle (hi2/cache.py:266-277, sigma_payload): tri =
 * sigma [k, k]'s upper triangle row-major (row i: columns i..k-1; k(k+1)/2 elements),
 * f32 or, with fp16 != 0, fp16 bits; *asym (device i32, zeroed by the caller) += the
 * number of pairs with sigma[i][j] != sigma[j][i] (zero: the matrix is exactly
 * symmetric and the triangle is the payload). */
int hi2x_sigma_pack_upper(const float* sigma, int64_t k, int fp16, void* tri, int32_t* asym,
                          void* stream);

/* ---- local code refinement ------------------------------------------------------------ */

/* Workspace of hi2x_refine_run for n rows of width k and `passes` sweeps. */
int64_t hi2x_refine_workspace_bytes(int64_t n, int64_t k, int64_t passes);

/* Local code refinement after GPTQ (hi2/refine.py:43-106 refine_expanded, called through
 * refine_groups hi2/refine.py:125-144 from calibrate.encode_many hi2/calibrate.py:374-391):
 *   w [n, k] f32 rows in the stored basis, codes [n, k] u8 refined in place,
 *   lo/st [n, ldp] f32 decoded ladders, row r's column j using entry j / block[r]
 *   (block [n] i32: the row's ladder block, 1 for per-column ladders), top [n] f32 the
 *   row's highest code, hs [k, k] f32 the Hessian in the stored basis, `passes` sweeps.
 * The reference stops after a sweep that moves no code; here that check runs on the
 * device (no host synchronisation).  moved: device u64 [passes] or NULL, receives the
 * codes moved by each sweep (0 for sweeps that did not run).  Codes are bit-identical
 * to the reference loop given its products' rounding (each product a sequential fp32
 * FMA chain, as the reference's CPU BLAS evaluates them at its tests' shapes). */
int hi2x_refine_run(const float* w, uint8_t* codes, int64_t n, int64_t k, const float* lo,
                    const float* st, int64_t ldp, const int32_t* block, const float* top,
                    const float* hs, int64_t passes, unsigned long long* moved, void* ws,
                    int64_t ws_bytes, void* stream);

/* The start of refine_expanded (hi2/refine.py:72-74) and of objective (hi2/refine.py:33-36):
 * e [n, k] f32 = fp16(lo + code * st) - w, then (g not NULL) g [n, k] f32 = e @ hs with
 * each element a sequential fp32 FMA chain over k.  Arguments as hi2x_refine_run. */
int hi2x_refine_gradient(const float* w, const uint8_t* codes, int64_t n, int64_t k,
                         const float* lo, const float* st, int64_t ldp, const int32_t* block,
                         const float* hs, float* e, float* g, void* stream);

/* One block of the sweep (the fused kernel of hi2/refine_kernel.py:52-91, Python entry
 * hi2/refine_kernel.py:171-176): columns [b0, b0 + len) (len <= 128) of every row, with
 * g [n, ldg] f32 the block's slice of g = e hs (read only: g + r * ldg + i is column
 * b0 + i of row r), codes/lo/st/block/top/hs as hi2x_refine_run; dw [n, ldw] f32 out
 * receives the change of each decoded value (0 where the code did not move); moved
 * (device u64 or NULL) is incremented by the number of moves. */
int hi2x_refine_block(const float* g, int64_t ldg, int64_t n, int64_t k, int64_t b0,
                      int64_t len, uint8_t* codes, const float* lo, const float* st,
                      int64_t ldp, const int32_t* block, const float* top, const float* hs,
                      float* dw, int64_t ldw, unsigned long long* moved, void* stream);

/* ---- QAD decode (the fake-quantised Linears of quantisation-aware distillation) --------- */

/* decode_fwd (hi2/qad_kernel.py:88-108, Python side hi2/qad_kernel.py:276-293): for the
 * n_rows rows of one (nbits, block) group, out[rows[r], :] = fp16(lo + q * step) as f32,
 * with v = latent[rows[r], :] (times unit[rows[r], :] when unit is not NULL), the block's
 * lo/step decoded from the continuous bytes lo_u/st_u [n_rows, k / block] f32
 * (clamp(rint(u), 0, 255)) and the row constants consts [n_rows, 3] fp16 bits (lo_min,
 * lo_scale, step_scale), q = clamp(rint((v - lo) / step), 0, nmax) (0 for a zero step).
 * latent/unit/out are [r_total, k] f32 row-major, 16-byte aligned; block 16, 32 or 64;
 * rows int64 on the device: a row outside [0, r_total) is skipped (nothing read or
 * written for it; the reference does not check). */
int hi2x_qad_decode_fwd(const float* latent, const float* unit, const float* lo_u,
                        const float* st_u, const uint16_t* consts, const int64_t* rows,
                        int64_t n_rows, int64_t r_total, int64_t k, int block, float nmax,
                        float* out, void* stream);

/* decode_bwd (hi2/qad_kernel.py:110-159, Python side hi2/qad_kernel.py:295-318): the
 * gradients of the straight-through graph of decode_fwd given grad [R, k] f32 of its
 * output: g_latent [r_total, k] (rows of the group written), g_lo / g_st
 * [n_rows, k / block] (the per-block sums as a pairwise tree over the block, times
 * lo_scale / step_scale; 0 for a skipped row).  Other arguments as hi2x_qad_decode_fwd. */
int hi2x_qad_decode_bwd(const float* grad, const float* latent, const float* unit,
                        const float* lo_u, const float* st_u, const uint16_t* consts,
                        const int64_t* rows, int64_t n_rows, int64_t r_total, int64_t k,
                        int block, float nmax, float* g_latent, float* g_lo, float* g_st,
                        void* stream);

/* wht_scale (hi2/qad_kernel.py:165-189, Python side hi2/qad_kernel.py:321-336): out =
 * H16(x) / scale over the flagged 16-column groups (x / scale elsewhere), or with pre_div
 * H16(x / scale); H16 the normalised order-16 Walsh-Hadamard butterfly.  x/out [n_rows, k]
 * f32 row-major, 16-byte aligned; flags [k / 16] u8; scale [k] fp16 bits or NULL. */
int hi2x_qad_wht_scale(const float* x, int64_t n_rows, int64_t k, const uint8_t* flags,
                       const uint16_t* scale, int pre_div, float* out, void* stream);

/* ---- streams ---------------------------------------------------------------------------- */

/* Background hint for a stream.  No counterpart in the reference (its encode runs one
 * input at a time on the CPU); it is for callers that run independent encodes on several
 * streams of one GPU, where one of them is the critical path.  With background != 0 the
 * GPTQ cross-block updates (hi2x_gptq_run, hi2x_gptq_trailing) launched on `stream`
 * reserve more LDS per workgroup than they use, so fewer of their workgroups share a CU
 * and the latency-bound kernels of the other streams (the factor's small products and
 * leaves) find room; background 0 clears the mark.  Results are unchanged.
 * Process-wide; marks streams by handle (a destroyed stream's handle may be reused:
 * clear the mark first). */
int hi2x_stream_background(void* stream, int background);

/* ---- measurement ------------------------------------------------------------------------ */

/* Launch-timing hook.  No counterpart in the reference (whose profiling is host-side
 * timers, hi2/hessian.py stage clocks); it exists so a benchmark can time the dominant
 * kernels with HIP events on the streams they are launched on.  While bit `kind` of
 * `mask` is set, every launch of that kernel family is bracketed by two events on its
 * stream and its algorithmic work recorded.  hi2x_timing_enable clears earlier records
 * (waiting for their events); mask 0 stops recording.  Process-wide, not meant to be
 * switched while other threads launch. */
#define HI2X_TIME_GPTQ_TRAILING 0 /* work = 2 * rows * rank * columns (flops) */
#define HI2X_TIME_HESSIAN_SYRK 1  /* work = tokens * k * (k + 1) (flops, upper triangle) */
#define HI2X_TIME_CHOL_GEMM 2     /* work = flops of the triangular product (fp32 MFMA) */
#define HI2X_TIME_CHOL_LEAF 3     /* work = 2 * n^3 / 3 (factor + inverse of the leaf) */
#define HI2X_TIME_GPTQ_BLOCK 4    /* work = rows * len * (len - 1) (intra-block flops) */
#define HI2X_TIME_REFINE_GEMM 5   /* work = 2 * rows * rank * columns (flops) */
#define HI2X_TIME_REFINE_BLOCK 6  /* work = rows * len (column decisions) */
#define HI2X_TIME_FWHT 7          /* work = bytes read + written (rows * k * 2 * size) */
#define HI2X_TIME_LADDER_FIT 8    /* work = bytes of w read (rows * k * 4) */
#define HI2X_TIME_PACK 9          /* work = bytes: codes read, words, params and consts moved */
#define HI2X_TIME_FINISH 10       /* work = bytes: codes and w read (sse; + the unpermute) */
#define HI2X_TIME_CHOL_SPLIT 11   /* work = fp16 MFMA flops executed by the factor's split-plane
                                     products: 3 products per fp32-equivalent product of the
                                     triangular shape (M * N * rank each) */
int hi2x_timing_enable(unsigned mask);

/* Sum over the recorded launches of `kind`: count, event-timed milliseconds, work. */
int hi2x_timing_query(int kind, int64_t* launches, double* ms, double* work);

#ifdef __cplusplus
}
#endif

#endif /* HI2X_H */
