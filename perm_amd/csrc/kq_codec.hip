// GGUF container codec on gfx950: encoders and decoders for Q2_K, Q3_K, Q4_K,
// Q5_K, Q6_K and Q8_0, bit-exact with coldpress/kquant.py (k-quant block
// bodies in kq_blocks.h).
//
// The k-quant encoders are VALU-bound (the candidate sweeps of make_qkx cost
// ~700 f32 ops per weight on the weighted path), not HBM-bound: 4.33-4.69
// B/weight of traffic. Q8_0 is a max, a divide and a rounding per weight and
// runs at HBM speed: 4 B read + 34/32 B written per weight.
#include <hip/hip_runtime.h>

#include "kq_blocks.h"

namespace cp {

__global__ __launch_bounds__(256) void q8_encode_kernel(const float* __restrict__ x, int64_t nblk,
                                                        uint8_t* __restrict__ out) {
  q8_encode_block(x, nblk, out, blockIdx.x);
}

__global__ __launch_bounds__(256) void q8_decode_kernel(const uint8_t* __restrict__ raw,
                                                        int64_t nblk, float* __restrict__ y) {
  q8_decode_thread(raw, nblk, y, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
}

template <int TT, bool IMAT>
__global__ __launch_bounds__(256) void kq_encode_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ qw,
                                                        int64_t NB, int64_t nsb,
                                                        uint8_t* __restrict__ out) {
  kq_encode_block<TT, IMAT>(x, qw, NB, nsb, out, blockIdx.x);
}

// 16 superblocks per workgroup (4 waves x kDecSb): grid ceil(NB / 16).
template <int TT>
__global__ __launch_bounds__(256) void kq_decode_kernel(const uint8_t* __restrict__ raw,
                                                        int64_t NB, float* __restrict__ y) {
  __shared__ __align__(16) KqDecodeLds<TT> lds;
  kq_decode_block<TT>(raw, NB, y, blockIdx.x, lds);
}

// ---------------------------------------------------------------- launchers

template <int TT>
static void launch_encode(const float* x, const float* qw, int64_t NB, int64_t nsb, uint8_t* out,
                          hipStream_t st) {
  constexpr int S = 64 / Kq<TT>::G;
  const int64_t waves = (NB + S - 1) / S;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (qw)
    kq_encode_kernel<TT, true><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, qw, NB, nsb, out);
  else
    kq_encode_kernel<TT, false><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, qw, NB, nsb, out);
}

int kq_quantize(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                uint8_t* out, hipStream_t st) {
  KqGeom geo;
  if (!kq_geom(ttype, &geo)) return set_error(CP_ERR_TTYPE, "unsupported container type %d", ttype);
  if (nrow < 0 || n <= 0 || n % geo.block_weights)
    return set_error(CP_ERR_SHAPE, "x is [%lld, %lld]; rows must be positive multiples of %d",
                     (long long)nrow, (long long)n, geo.block_weights);
  if (nrow == 0) return CP_OK;  // an empty tensor: nothing to encode
  if (!x || !out) return set_error(CP_ERR_ARG, "null x/out");
  if (!aligned(x, 16) || (qw && !aligned(qw, 16)) || !aligned(out, 4))
    return set_error(CP_ERR_ALIGN, "x/qw need 16-byte and out 4-byte alignment");
  if (ttype == CP_Q8_0) {
    const int64_t nblk = nrow * (n / 32);
    const int64_t blocks = (nblk + 8 * kWavesPerBlock - 1) / (8 * kWavesPerBlock);
    if (blocks > 0x7FFFFFFF) return set_error(CP_ERR_SHAPE, "tensor too large");
    q8_encode_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(x, nblk, out);
    CP_LAUNCHED("Q8_0 encode launch");
    return CP_OK;
  }
  const int64_t nsb = n / 256, NB = nrow * nsb;
  if ((NB + 3) / 4 > (int64_t)0x7FFFFFFF * 4) return set_error(CP_ERR_SHAPE, "tensor too large");
  switch (ttype) {
    case CP_Q2_K: launch_encode<CP_Q2_K>(x, qw, NB, nsb, out, st); break;
    case CP_Q3_K: launch_encode<CP_Q3_K>(x, qw, NB, nsb, out, st); break;
    case CP_Q4_K: launch_encode<CP_Q4_K>(x, qw, NB, nsb, out, st); break;
    case CP_Q5_K: launch_encode<CP_Q5_K>(x, qw, NB, nsb, out, st); break;
    case CP_Q6_K: launch_encode<CP_Q6_K>(x, qw, NB, nsb, out, st); break;
  }
  CP_LAUNCHED("k-quant encode launch");
  return CP_OK;
}

int kq_dequantize(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* y,
                  hipStream_t st) {
  KqGeom geo;
  if (!kq_geom(ttype, &geo)) return set_error(CP_ERR_TTYPE, "unsupported container type %d", ttype);
  if (nrow < 0 || n <= 0 || n % geo.block_weights)
    return set_error(CP_ERR_SHAPE, "y is [%lld, %lld]; rows must be positive multiples of %d",
                     (long long)nrow, (long long)n, geo.block_weights);
  if (nrow == 0) return CP_OK;  // an empty container: nothing to decode
  if (!raw || !y) return set_error(CP_ERR_ARG, "null raw/y");
  if (!aligned(y, 16) || !aligned(raw, 2))
    return set_error(CP_ERR_ALIGN, "y needs 16-byte and raw 2-byte alignment");
  if (ttype == CP_Q8_0) {
    const int64_t nblk = nrow * (n / 32);
    const int64_t blocks = (nblk * 8 + 255) / 256;
    if (blocks > 0x7FFFFFFF) return set_error(CP_ERR_SHAPE, "tensor too large");
    q8_decode_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, nblk, y);
    CP_LAUNCHED("Q8_0 decode launch");
    return CP_OK;
  }
  const int64_t NB = nrow * (n / 256);
  const int64_t blocks = (NB + 4 * kDecSb - 1) / (4 * kDecSb);
  switch (ttype) {
    case CP_Q2_K: kq_decode_kernel<CP_Q2_K><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, NB, y); break;
    case CP_Q3_K: kq_decode_kernel<CP_Q3_K><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, NB, y); break;
    case CP_Q4_K: kq_decode_kernel<CP_Q4_K><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, NB, y); break;
    case CP_Q5_K: kq_decode_kernel<CP_Q5_K><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, NB, y); break;
    case CP_Q6_K: kq_decode_kernel<CP_Q6_K><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(raw, NB, y); break;
  }
  CP_LAUNCHED("k-quant decode launch");
  return CP_OK;
}

}  // namespace cp

extern "C" {

int cp_kq_block_bytes(int ttype) {
  cp::KqGeom g;
  if (!cp::kq_geom(ttype, &g)) return cp::set_error(CP_ERR_TTYPE, "unsupported container type %d", ttype);
  return g.block_bytes;
}

int cp_kq_quantize(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                   uint8_t* out, void* stream) {
  cp::clear_error();
  return cp::kq_quantize(ttype, x, nrow, n, qw, out, (hipStream_t)stream);
}

int cp_kq_dequantize(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* y,
                     void* stream) {
  cp::clear_error();
  return cp::kq_dequantize(ttype, raw, nrow, n, y, (hipStream_t)stream);
}

}  // extern "C"
