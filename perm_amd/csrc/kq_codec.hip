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

// ---------------------------------------------------------------- Q8_0
// Blocks of 32 weights: d = max|x|/127 (fp16), codes int8 = round-half-away(x/d)
// (kquant.py:706-727). A wave covers 256 consecutive weights (8 blocks) with one
// float4 per lane; the 8 lanes of a block reduce max|x| with xor shuffles (max is
// exact in any order). The wave's 8*34 = 272 output bytes are assembled in LDS
// and leave as 68 dword stores.
constexpr int kQ8Bytes = 34;

// numpy's float32 -> int8 cast of sign(v)*floor(|v|+0.5) on x86: truncation to
// int32 (0x80000000 for NaN, inf and |v| >= 2^31), then the low byte. Finite
// scales keep |v| <= 127; a scale whose reciprocal overflows (max|x| < 3.7e-37)
// sends v to +-inf or NaN, and the reference then stores code 0.
__device__ __forceinline__ uint32_t q8_code(float x, float inv) {
  const float v = x * inv;
  const float a = floorf(fabsf(v) + 0.5f);
  int q = a < 2147483648.0f ? (int)a : 0;
  q = v < 0.0f ? -q : q;
  return (uint32_t)q & 0xFFu;
}

__global__ __launch_bounds__(256) void q8_encode_kernel(const float* __restrict__ x, int64_t nblk,
                                                        uint8_t* __restrict__ out) {
  __shared__ uint32_t s_out[kWavesPerBlock][68];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t chunk = (int64_t)blockIdx.x * kWavesPerBlock + wv;  // 8 blocks per chunk
  const int64_t blk = chunk * 8 + (lane >> 3);
  const bool valid = blk < nblk;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (valid) v = reinterpret_cast<const float4*>(x)[chunk * 64 + lane];
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  amax = fmaxf(amax, __shfl_xor(amax, 4));
  const float d = amax / 127.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  const uint32_t codes = q8_code(v.x, inv) | q8_code(v.y, inv) << 8 | q8_code(v.z, inv) << 16 |
                         q8_code(v.w, inv) << 24;
  uint16_t* so = reinterpret_cast<uint16_t*>(s_out[wv]);
  const int h = (lane >> 3) * (kQ8Bytes / 2) + 1 + 2 * (lane & 7);  // in halfwords
  so[h] = (uint16_t)codes;
  so[h + 1] = (uint16_t)(codes >> 16);
  if ((lane & 7) == 0) so[h - 1] = half_bits(d);
  __syncthreads();
  if (chunk * 8 >= nblk) return;
  const int64_t nvalid = nblk - chunk * 8 < 8 ? nblk - chunk * 8 : 8;
  const int bytes = (int)nvalid * kQ8Bytes;
  uint8_t* dst = out + chunk * 8 * kQ8Bytes;
  for (int dw = lane; dw < bytes / 4; dw += 64) reinterpret_cast<uint32_t*>(dst)[dw] = s_out[wv][dw];
  if ((bytes & 3) && lane == 0)
    reinterpret_cast<uint16_t*>(dst)[bytes / 2 - 1] = so[bytes / 2 - 1];
}

// One thread per 4 consecutive weights: y = d * code in float32.
__global__ __launch_bounds__(256) void q8_decode_kernel(const uint8_t* __restrict__ raw,
                                                        int64_t nblk, float* __restrict__ y) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk = t >> 3;
  if (blk >= nblk) return;
  const uint16_t* b = reinterpret_cast<const uint16_t*>(raw + blk * kQ8Bytes);
  const int j = (int)(t & 7);
  const float d = half_value(b[0]);
  const uint32_t c = (uint32_t)b[1 + 2 * j] | (uint32_t)b[2 + 2 * j] << 16;
  reinterpret_cast<float4*>(y)[t] =
      make_float4(d * (float)(int8_t)(c & 0xFF), d * (float)(int8_t)((c >> 8) & 0xFF),
                  d * (float)(int8_t)((c >> 16) & 0xFF), d * (float)(int8_t)(c >> 24));
}

template <int TT, bool IMAT>
__global__ __launch_bounds__(256) void kq_encode_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ qw,
                                                        int64_t NB, int64_t nsb,
                                                        uint8_t* __restrict__ out) {
  kq_encode_block<TT, IMAT>(x, qw, NB, nsb, out, blockIdx.x);
}

template <int TT>
__global__ __launch_bounds__(256) void kq_decode_kernel(const uint8_t* __restrict__ raw,
                                                        int64_t NB, float* __restrict__ y) {
  kq_decode_thread<TT>(raw, NB, y, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
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
  if (nrow <= 0 || n <= 0 || n % geo.block_weights)
    return set_error(CP_ERR_SHAPE, "x is [%lld, %lld]; rows must be positive multiples of %d",
                     (long long)nrow, (long long)n, geo.block_weights);
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
  if (nrow <= 0 || n <= 0 || n % geo.block_weights)
    return set_error(CP_ERR_SHAPE, "y is [%lld, %lld]; rows must be positive multiples of %d",
                     (long long)nrow, (long long)n, geo.block_weights);
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
  const int64_t blocks = (NB * 16 + 255) / 256;
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
