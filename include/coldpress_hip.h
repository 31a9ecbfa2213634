/* coldpress_hip.h -- C ABI of libcoldpress_hip.so, the MI355X (gfx950) encoder
 * hot path of coldpress: k-quant codec, Hessian X^T X, damped inverse-Hessian
 * factor, and GPTQ-style error feedback (EF) into committed k-quant grids.
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
 *  - Type codes are ggml's: Q2_K = 10, Q3_K = 11, Q4_K = 12, Q6_K = 14.
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
  CP_ERR_WORKSPACE = -7  /* workspace too small                                  */
};

enum cp_ttype { CP_Q2_K = 10, CP_Q3_K = 11, CP_Q4_K = 12, CP_Q6_K = 14 };

/* Message for the last failure on this thread ("" if none). */
const char* cp_last_error(void);

/* Bytes per 256-weight superblock of a container type, or a negative status. */
int cp_kq_block_bytes(int ttype);

/* k-quant encode of x [nrow, n] (n % 256 == 0) into out [nrow, n/256*block_bytes].
 * qw [n] is the importance vector (imatrix means) or NULL for the unweighted path.
 * Replaces kquant.QUANTIZE[tt](x, qw) -- coldpress/kquant.py:732 (encoders
 * quantize_q2_K :347, quantize_q3_K :432, quantize_q4_K :588, quantize_q6_K :632).
 * Bit-exact with the reference encoder. */
int cp_kq_quantize(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                   uint8_t* out, void* stream);

/* k-quant decode of raw [nrow, n/256*block_bytes] into y [nrow, n] float32.
 * Replaces kquant.DEQUANTIZE[tt](raw, n) -- coldpress/kquant.py:734 (decoders
 * :416, :489, :596, :681). Bit-exact. */
int cp_kq_dequantize(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* y,
                     void* stream);

#ifdef __cplusplus
}
#endif
#endif /* COLDPRESS_HIP_H */
