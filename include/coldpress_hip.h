/* coldpress_hip.h -- C ABI of libcoldpress_hip.so, the MI355X (gfx950) encoder
 * hot path of coldpress: GGUF container codec, Hessian X^T X, damped
 * inverse-Hessian factor, GPTQ-style error feedback (EF) into committed k-quant
 * grids, and the PERM channel moves and container objective.
 *
 * Conventions
 *  - Every pointer argument named x, qw, raw, out, y, H, U, W, order, X ... is a
 *    DEVICE pointer owned by the caller (e.g. a torch tensor's data_ptr()).
 *    Row-major, densely packed. Float inputs 16-byte aligned, byte outputs
 *    4-byte aligned (CP_ERR_ALIGN otherwise).
 *  - ``stream`` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    on it in order; functions that must read a device result back (the
 *    factorization's positive-definiteness check) synchronize that stream.
 *  - Return 0 (CP_OK) or a negative cp_status. cp_last_error() gives a
 *    thread-local message for the last failure on the calling thread.
 *  - Type codes are ggml's: Q8_0 = 8, Q2_K = 10, Q3_K = 11, Q4_K = 12, Q5_K = 13,
 *    Q6_K = 14.
 */
#ifndef COLDPRESS_HIP_H
#define COLDPRESS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum cp_status {
  CP_OK = 0,
  CP_ERR_SHAPE = -1,     /* n % 256 != 0, non-positive sizes, mismatched dims   */
  CP_ERR_TTYPE = -2,     /* container type not supported                         */
  CP_ERR_NOT_PD = -3,    /* factorization failed after every damping escalation  */
  CP_ERR_HIP = -4,       /* a HIP runtime call failed                            */
  CP_ERR_ARG = -5,       /* null pointer / invalid argument                      */
  CP_ERR_ALIGN = -6,     /* pointer alignment requirement violated               */
  CP_ERR_WORKSPACE = -7, /* workspace too small                                  */
  CP_ERR_INDEX = -8,     /* an index argument out of range / not a permutation    */
  CP_ERR_TIMEOUT = -9    /* a device-side bounded wait gave up (results invalid)  */
};

enum cp_ttype { CP_Q8_0 = 8, CP_Q2_K = 10, CP_Q3_K = 11, CP_Q4_K = 12, CP_Q5_K = 13, CP_Q6_K = 14 };

/* Message for the last failure on this thread ("" if none). */
const char* cp_last_error(void);

/* Bytes per block of a container type (a 256-weight superblock for the k-quants,
 * a 32-weight block for Q8_0), or a negative status. */
int cp_kq_block_bytes(int ttype);

/* Container encode of x [nrow, n] into out [nrow, n/block_weights*block_bytes]
 * (n % 256 == 0 for the k-quants, n % 32 == 0 for Q8_0). qw [n] is the importance
 * vector (imatrix means) or NULL for the unweighted path; Q8_0 ignores it, as the
 * reference does. Replaces kquant.QUANTIZE[tt](x, qw) -- coldpress/kquant.py:732
 * (encoders quantize_q2_K :347, quantize_q3_K :432, quantize_q4_K :588,
 * quantize_q5_K :592, quantize_q6_K :632, quantize_q8_0 :706). Bit-exact with the
 * reference encoder. nrow == 0 is a no-op. */
int cp_kq_quantize(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                   uint8_t* out, void* stream);

/* Container decode of raw [nrow, n/block_weights*block_bytes] into y [nrow, n]
 * float32. Replaces kquant.DEQUANTIZE[tt](raw, n) -- coldpress/kquant.py:734
 * (decoders :416, :489, :596, :610, :681, :721). Bit-exact. nrow == 0 is a no-op
 * (an empty container decodes to an empty tensor, as the reference's does). */
int cp_kq_dequantize(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* y,
                     void* stream);

/* ---- damped inverse-Hessian factor (coldpress/ef.py:46-84, 187-189) ---- */

/* order[z][jj] = column visited jj-th: stable argsort of -diag(H_z) for each of
 * ``batch`` [n, n] matrices (h_dtype 0 = float32, 1 = float64). Replaces
 * ef.py:187 ``np.argsort(-np.diag(H))`` (ties broken by index; NaN entries last,
 * by index, as numpy sorts them). Always a permutation. */
int cp_act_order(const void* H, int h_dtype, int64_t n, int batch, int32_t* order, void* stream);

/* Workspace bytes cp_chol_inv_upper needs for ``batch`` matrices of size n. */
size_t cp_chol_ws_bytes(int64_t n, int batch);

/* U_z = chol(inv(Hp_z + lambda I))^T, upper triangular [n, n] with
 * U^T U = inv(Hp + lambda I), where Hp = H[order][:, order] (identity order when
 * order is NULL), lambda = damp * mean(diag Hp) + 1e-8 (mean replaced by 1 when
 * not positive). Computed in float64; stored as float32 (u_dtype 0, what the EF
 * sweep consumes) or float64 (u_dtype 1). A matrix whose factorization fails is
 * retried with damp x 10, up to max_tries attempts; damp_used (host array of
 * ``batch`` doubles, may be NULL) receives the damp that succeeded.
 * Returns CP_ERR_NOT_PD when a matrix fails every attempt, CP_ERR_INDEX when an
 * order is not a permutation of n (no read ever leaves H: its entries are clamped
 * before use), CP_ERR_TIMEOUT when a chain step of a call of at most four matrices
 * (one launch per 64 columns) gave up its bounded wait for its diagonal block
 * (cp_chol_wait_limit; the result is then invalid). A NaN pivot counts as a failed
 * attempt, as LAPACK's does.
 * Replaces ef.cholesky_inv_upper(Hp, damp, _max_tries) -- coldpress/ef.py:46-84
 * -- together with the gather and float32 cast of ef.py:188-189.
 * Synchronizes ``stream`` (it reads the per-matrix failure flags). */
int cp_chol_inv_upper(const void* H, int h_dtype, int64_t n, int batch, const int32_t* order,
                      double damp, int max_tries, void* U, int u_dtype, double* damp_used,
                      void* ws, size_t ws_bytes, void* stream);

/* One attempt of cp_chol_inv_upper at ``damp`` for every matrix, without waiting
 * on the stream: flags[z] (device int32 array of ``batch``) has bit 0 set where
 * matrix z met a non-positive or NaN pivot, bit 1 where its order is not a
 * permutation and bit 2 where a chain step gave up its bounded wait; that U_z is
 * then meaningless. Work
 * that consumes U can be queued behind it; a caller that later finds a set flag
 * re-runs cp_chol_inv_upper, whose escalation reproduces the reference's
 * (coldpress/ef.py:60-84). Same workspace as cp_chol_inv_upper. */
int cp_chol_inv_upper_async(const void* H, int h_dtype, int64_t n, int batch,
                            const int32_t* order, double damp, void* U, int u_dtype,
                            int32_t* flags, void* ws, size_t ws_bytes, void* stream);

/* Per-thread GEMM tile policy of the factorizations this thread queues: 0 (the default)
 * picks the fastest tiles for a GPU the factorization has to itself; 1 keeps every fp64
 * GEMM at 64 x 64 tiles, which fit on a CU beside the EF sweep's workgroups, for a
 * factorization queued to run concurrently with EF work (perm_amd.ef.encode_size_classes).
 * Results are the same bit for bit either way: every output element sums its K range in
 * the same order for either tile. No counterpart in the reference, which factorizes with
 * LAPACK. */
void cp_chol_compact_tiles(int on);

/* Per-thread bound of the fused chain step's wait (a panel tile waiting for its diagonal
 * block) in this thread's later factorizations: ``sleeps`` sleeps of about 512 clocks;
 * negative restores the default 65536 (about 14 ms at 2.4 GHz, against a diagonal block
 * of about 30 us). A small bound makes the waits give up early (a test of the timeout
 * path); every kernel still ends. No counterpart in the reference. */
void cp_chol_wait_limit(int sleeps);

/* ---- EF encode (coldpress/ef.py:179-218) ---- */

enum cp_ef_mode {
  CP_EF_EXACT = 0,      /* error propagation in the reference's sequential float32 order
                           (products on MFMA, ordered subtraction on VALU): bit-exact          */
  CP_EF_MFMA = 1,       /* cross-block propagation as float32-accumulated MFMA GEMMs (lazy
                           batch of 32 columns); in-block propagation exact; not bit-exact   */
  CP_EF_EXACT_VALU = 2  /* as CP_EF_EXACT with products and subtractions on VALU only        */
};

typedef struct cp_ef_tensor {
  int ttype;             /* CP_Q2_K, CP_Q3_K, CP_Q4_K, CP_Q5_K or CP_Q6_K              */
  int64_t nrow, n;       /* weight shape, n % 256 == 0                                  */
  const float* x;        /* [nrow, n] weights                                           */
  const float* qw;       /* [n] importance (imatrix means) or NULL                      */
  const float* U;        /* [n, n] float32 upper factor in visiting order (cp_chol_inv_upper) */
  const int32_t* order;  /* [n] visiting order (cp_act_order)                           */
  uint8_t* raw;          /* out: [nrow, n/256*block_bytes] container bytes              */
  float* recon;          /* out: [nrow, n] decoded weights, or NULL                     */
} cp_ef_tensor;

/* Workspace bytes cp_ef_encode_batch needs for these tensors. The first 4 bytes of the
 * workspace are the call's status word (int32, cleared by the call before its sweep):
 * bit 0 set means a sweep wave gave up a bounded wait and the call's bytes are not
 * valid. cp_ef_read_status reads it. */
size_t cp_ef_ws_bytes(const cp_ef_tensor* tensors, int count);

/* GPTQ error feedback into committed k-quant grids for ``count`` independent
 * tensors in one pass. Each order must be a permutation of its n (as cp_act_order
 * gives); one that is not never makes a read or write leave the tensor's buffers,
 * but its bytes are meaningless (the host wrappers check caller-supplied orders
 * before the call). Per iteration, commit the container with the stock
 * encoder (cp_kq_quantize) on the current targets, sweep the columns in
 * visiting order quantizing onto the committed grid and propagating the
 * error through U, re-pack the codes; after n_iter iterations decode into
 * recon. Replaces ef.ef_encode(x, tt, qw, H, n_iter, damp, act_order=True)
 * (coldpress/ef.py:179-218) once U and order are computed. */
int cp_ef_encode_batch(const cp_ef_tensor* tensors, int count, int n_iter, int mode, void* ws,
                       size_t ws_bytes, void* stream);

/* Single-tensor form of cp_ef_encode_batch (CP_EF_EXACT). */
int cp_ef_encode(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                 const float* U, const int32_t* order, int n_iter, uint8_t* raw, float* recon,
                 void* ws, size_t ws_bytes, void* stream);

/* cp_ef_encode without a caller workspace and without any device allocation. No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The EF workspace is a static device array of cp_ef_noalloc_max_ws_bytes() bytes
 * (64 MiB: any tensor up to about 3.8 M weights, e.g. every Qwen3-0.6B linear) that
 * each GPU the library runs on holds until the process ends; a larger tensor returns
 * CP_ERR_WORKSPACE before anything is launched. The array is looked up once per device
 * (hipGetSymbolAddress) on that device's first call. Every call on one GPU shares it,
 * so calls that overlap on one GPU (other streams, other host threads) race: order
 * them. Same results as cp_ef_encode, byte for byte; phase timing is off inside it. */
int cp_ef_encode_noalloc(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                         const float* U, const int32_t* order, int n_iter, uint8_t* raw,
                         float* recon, void* stream);

/* Bytes of the static workspace behind cp_ef_encode_noalloc. */
size_t cp_ef_noalloc_max_ws_bytes(void);

/* Status of the EF call that last used workspace ``ws`` (NULL: the static workspace of
 * cp_ef_encode_noalloc on the current device), after the work queued on ``stream``:
 * CP_OK, or CP_ERR_TIMEOUT when one of the call's multi-wave sweep waves waited for an
 * earlier block of its stripe past the spin bound (cp_ef_wait_limit) and went on without
 * it, so the call's raw and recon are not valid. Synchronizes ``stream``. No counterpart
 * in the reference, whose sweep is one sequential loop. */
int cp_ef_read_status(const void* ws, void* stream);

/* Per-thread spin bound of the multi-wave sweep's waits for this thread's later EF calls:
 * ``spins`` sleeps of about 512 clocks each; negative restores the default 65536 (about
 * 14 ms at 2.4 GHz, far above a block's sweep time). A small bound makes waves give up
 * early (a test of the status path); every kernel still ends. */
void cp_ef_wait_limit(int spins);

/* Per-thread switch for phase timing of EF calls (hipEvents recorded on the
 * call's stream; no synchronization inside the call). No counterpart in the
 * reference, which times whole tensors with time.time() (coldpress/ef.py:277, 304). */
void cp_ef_profile(int enable);

/* Milliseconds spent by the calling thread's last profiled EF call in each
 * phase: out[0] setup (index, gather), out[1] commit (encode + grid decode),
 * out[2] sweep, out[3] repack (+ target scatter), out[4] final decode.
 * Waits for the call's last event. Returns the number of phases written. */
int cp_ef_phase_ms(float* out, int nphase);

/* Shape of the calling thread's last EF sweep launch: rows per stripe (16 or 32) and
 * waves per stripe (1: ef_sweep_rows_kernel; 2, 4 or 8: ef_sweep_pipe_kernel). Returns
 * that call's mode, or -1 when the thread has run no EF call. A profiling aid with no
 * counterpart in the reference, like cp_ef_profile. */
int cp_ef_last_sweep(int* rows_per_stripe, int* waves);

/* ---- encode statistics (coldpress/ef.py:298-304) ---- */

/* Workspace bytes of cp_sq_err_sum for [nrow, n] arrays (4 bytes per 8192 terms). */
size_t cp_sq_err_ws_bytes(int64_t nrow, int64_t n);

/* out[0] (device float32) = (((a - b) ** 2) * w).sum() for float32 a, b [nrow, n] and
 * w [n] broadcast over rows (NULL: ones), with numpy's rounding of every term and its
 * summation order for the full reduction of a contiguous array: 8192-term chunks of
 * the flattened terms, each summed pairwise, the chunk sums added left to right from
 * 0.0. Replaces e_base / e_ours of encode_gguf's err-vs-stock statistic
 * (coldpress/ef.py:298-304). Bit-identical. n % 4 == 0; 16-byte aligned a, b, w. */
int cp_sq_err_sum(const float* a, const float* b, const float* w, int64_t nrow, int64_t n,
                  float* out, void* ws, size_t ws_bytes, void* stream);

/* ---- Hessian accumulation (coldpress/hessians.py:137-154) ---- */

/* H [d, d] float32 += X^T X for X [N, d] row-major (x_dtype 0 = float32,
 * 1 = bfloat16 with d % 8 == 0). Float32 accumulation on MFMA. Replaces the
 * forward hook's ``acc += (x.float().T @ x)`` (coldpress/hessians.py:142-152),
 * with the accumulator kept on the device. Reproducible: the summation order
 * over rows is fixed by the shapes alone (row splits are summed in split order,
 * then added to H), so the same X and H give the same result bit for bit. For
 * bf16 X the result is symmetric and H's upper triangle is not read (the lower
 * triangle is mirrored into it). The workspace the row splits need is taken
 * stream-ordered (hipMallocAsync / hipFreeAsync on ``stream``); use
 * cp_hess_accum_batch_ws to pass one instead. */
int cp_hess_accum(const void* X, int x_dtype, int64_t N, int64_t d, float* H, void* stream);

/* H[z] += X[z]^T X[z] for ``count`` jobs of one shape (host arrays of device pointers),
 * bf16 jobs in as few launches as fit (224 per launch): many Hessians share one grid, so
 * small d needs fewer row splits. The batched form of cp_hess_accum (the hook of
 * coldpress/hessians.py:137-154 for every hooked module of a forward pass); the same
 * summation order per job as cp_hess_accum with count = 1 only when the launch plans
 * agree, so compare a job with itself, not across batch sizes. */
int cp_hess_accum_batch(const void* const* X, float* const* H, int count, int x_dtype,
                        int64_t N, int64_t d, void* stream);

/* Workspace bytes cp_hess_accum_batch_ws needs for these jobs (0 when every launch
 * runs as one row split). */
size_t cp_hess_ws_bytes(int count, int x_dtype, int64_t N, int64_t d);

/* cp_hess_accum_batch with a caller workspace (device, 16-byte aligned, at least
 * cp_hess_ws_bytes bytes; CP_ERR_WORKSPACE otherwise): the row splits' partial tiles.
 * Its contents need no clearing. Same results as cp_hess_accum_batch, bit for bit. */
int cp_hess_accum_batch_ws(const void* const* X, float* const* H, int count, int x_dtype,
                           int64_t N, int64_t d, void* ws, size_t ws_bytes, void* stream);

/* ---- Hessian storage (coldpress/hessians.py:163-243) ---- */

/* Pack a float32 [n, n] Hessian for storage: diag32 = diag(H) (float32, exact);
 * hscale[0] = max|H| / 32768 when max|H| > 32768, else 1; H16 = float16(H / hscale)
 * rounded to nearest even. Output pointers are device pointers; ws holds 4 bytes.
 * Replaces the arithmetic of hessians.save_hessians (coldpress/hessians.py:180-194);
 * the npz write stays with the caller. Bit-exact. */
int cp_h2_pack(const float* H, int64_t n, uint16_t* H16, float* diag32, float* hscale,
               void* ws, size_t ws_bytes, void* stream);

/* Expand a stored Hessian to float64: H = double(Hs) * hscale, then the diagonal
 * overwritten with diag32 when given. Hs is float16 (in_dtype 1) or float32 (0, the
 * older format). Replaces the arithmetic of hessians.load_hessian
 * (coldpress/hessians.py:225-243). Bit-exact. */
int cp_h2_expand(const void* Hs, int in_dtype, int64_t n, double hscale, const float* diag32,
                 double* H, void* stream);

/* ---- linear form of a k-quant tensor (coldpress/scale_tune.py) ---- */

/* W = d (x) A - dmin (x) B with the codes fixed: d, dmin [nrow, n/256] float32 (the fp16
 * fields), A, B [nrow, n] integer products as int16 (ab_dtype 0) or float32 (1). dmin and
 * B are written for Q2_K / Q4_K / Q5_K only (may be NULL otherwise). Replaces
 * scale_tune.extract_linear -- coldpress/scale_tune.py:67-159. Bit-exact. */
int cp_lin_extract(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* d, float* dmin,
                   void* A, void* B, int ab_dtype, void* stream);

/* W[r][c] = d[r][c/256] * A[r][c] - dmin[r][c/256] * B[r][c] in float32 (dmin and B NULL
 * for the types without a min). Equal to the container's decode bit for bit. Replaces
 * scale_tune.reconstruct / reconstruct_np -- coldpress/scale_tune.py:162-173, 245-269. */
int cp_lin_reconstruct(int64_t nrow, int64_t n, const float* d, const float* dmin,
                       const int16_t* A, const int16_t* B, float* W, void* stream);

/* The gradient of that form: gd[r][s] = sum over the superblock of gW * A, gdmin = -sum
 * of gW * B (float32, summed in a fixed order). The backward of scale_tune.reconstruct. */
int cp_lin_reconstruct_grad(int64_t nrow, int64_t n, const float* gW, const int16_t* A,
                            const int16_t* B, float* gd, float* gdmin, void* stream);

/* out = raw with only the fp16 d / dmin fields replaced by float16(d), float16(dmin)
 * (round to nearest even); in place when out == raw. Replaces scale_tune.write_back --
 * coldpress/scale_tune.py:176-203. */
int cp_lin_write_back(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, const float* d,
                      const float* dmin, uint8_t* out, void* stream);

/* ---- PERM channel permutations (coldpress/perm/spacemaps/qwen3.py, ef.py:289-290) ---- */

/* dst[r][c] = src[row_perm[r]][col_perm[c]] for a row-major [rows, cols] matrix of
 * elem_bytes-byte elements (1, 2, 4 or 8); a NULL permutation is the identity.
 * An index outside [0, rows) / [0, cols) is clamped into it, so no read leaves src
 * (the host wrapper rejects such indices with IndexError before the call).
 * Replaces the index_select / fancy-index moves of qwen3.apply_perms
 * (coldpress/perm/spacemaps/qwen3.py:141-188) and H[np.ix_(p, p)] (ef.py:289-290).
 * Not in place. */
int cp_permute_gather(const void* src, void* dst, const int32_t* row_perm,
                      const int32_t* col_perm, int64_t rows, int64_t cols, int elem_bytes,
                      void* stream);

/* ---- PERM container objective (coldpress/perm/objective.py) ---- */

typedef struct cp_err_tensor {
  int ttype;             /* any cp_ttype                                                */
  int x_dtype;           /* 0 = float32, 1 = float16 (GGUF F16 weights)                 */
  int64_t nrow, n;       /* x is [nrow, n] row-major, n a multiple of the block width   */
  const void* x;
  const float* qw;       /* [n] importance (imatrix means) or NULL                      */
  const int32_t* perm;   /* [n] column permutation, or NULL for the identity            */
  const double* wvec;    /* [n] error weights (indexed through perm) or NULL            */
  const int32_t* rows;   /* [rows_used] sorted row sample, or NULL for every row        */
  int64_t rows_used;
} cp_err_tensor;

/* Workspace bytes cp_tensor_err_batch needs (0 for an invalid type). */
size_t cp_tensor_err_ws_bytes(const cp_err_tensor* tensors, int count);

/* out[i] (device float64) = the quantization error of tensor i, for ``count``
 * tensors in one pass. Replaces objective.tensor_err(x, ttype, qw, perm, wvec,
 * rows_sample, seed) -- coldpress/perm/objective.py:17-39 -- once the caller has
 * drawn the row sample (objective.py:21-24) and dropped the F16/F32/BF16 types
 * (error 0). Bit-identical to the reference: the column sums run row after row
 * and the weighted total is numpy's pairwise float64 sum. An index outside its
 * range is never dereferenced; that tensor's result is NaN. */
int cp_tensor_err_batch(const cp_err_tensor* tensors, int count, void* ws, size_t ws_bytes,
                        double* out, void* stream);

/* Per-thread switch for phase timing of cp_tensor_err_batch calls (hipEvents on
 * the call's stream). No counterpart in the reference. */
void cp_err_profile(int enable);

/* Milliseconds of the calling thread's last profiled cp_tensor_err_batch call per
 * phase: out[0] gather, out[1] encode, out[2] decode, out[3] column sums, out[4]
 * weighted total. Waits for the call's last event. Returns the phases written. */
int cp_err_phase_ms(float* out, int nphase);

typedef struct cp_col_tensor {
  const void* x;         /* [nrow, n] row-major                                         */
  int x_dtype;           /* 0 = float32, 1 = float16                                    */
  int64_t nrow, n;
  double* out;           /* [n] device float64 result                                   */
} cp_col_tensor;

/* Workspace bytes of cp_col_sq_sums / cp_col_log_rms. */
size_t cp_col_sums_ws_bytes(int64_t nrow, int64_t n, int64_t row_step);

/* Workspace bytes of cp_col_sq_sums_batch. */
size_t cp_col_sums_batch_ws_bytes(const cp_col_tensor* tensors, int count, int64_t row_step);

/* cp_col_sq_sums (log_rms = 0) or cp_col_log_rms (log_rms = 1) for ``count``
 * tensors in one pass (the profiles a space-map search sorts by). */
int cp_col_sq_sums_batch(const cp_col_tensor* tensors, int count, int64_t row_step, int log_rms,
                         void* ws, size_t ws_bytes, void* stream);

/* acc[c] (device float64) = sum over rows of x[r][c]^2 in float64, summed in chunks
 * of row_step rows with the chunk sums added in order (objective.py:44-48).
 * Bit-identical. */
int cp_col_sq_sums(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* acc, void* ws, size_t ws_bytes, void* stream);

/* out[c] = log(sqrt(acc[c] / nrow) + 1e-12) -- objective.col_log_rms(x, row_step),
 * coldpress/perm/objective.py:42-49. The sums are bit-identical; log is the
 * device libm's (within 2 ulp of the host's). */
int cp_col_log_rms(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* out, void* ws, size_t ws_bytes, void* stream);

/* Self-check of the device division shortcut the k-quant affine fits use for
 * divisions that share a divisor (a refined reciprocal formed once per divisor):
 * n pseudo-random float32 pairs (seeded) inside its operand range, zero numerators
 * and the range's end values, each compared bit for bit with the compiler's IEEE
 * division. *mismatches receives the count (0 expected). Synchronizes the stream.
 * No counterpart in the reference: it checks an implementation choice of this library. */
int cp_check_division(int64_t n, uint64_t seed, int64_t* mismatches, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* COLDPRESS_HIP_H */
