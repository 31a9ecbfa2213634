// Linear form of a k-quant tensor on gfx950 (coldpress/scale_tune.py:1-269): with the
// integer codes fixed, dequantization is linear in the per-superblock fp16 scales,
//
//     W[r, c] = d[r, c/256] * A[r, c] - dmin[r, c/256] * B[r, c]
//
// A = integer sub-block scale x signed code, B = integer sub-block min (Q2_K, Q4_K,
// Q5_K; Q3_K and Q6_K have no min side). Every |A| <= 4096 and |B| <= 63, so A and B are
// exact in int16; d * A needs at most 11 + 13 significant bits, so the float32 form
// fl(fl(d*A) - fl(dmin*B)) equals the decoders' float32 result bit for bit.
//
//   extract       container bytes -> d, dmin (float32 of the fp16 fields), A, B
//   reconstruct   W from (d, dmin, A, B), float32, the distill stage's forward
//   grad          dL/dd[r, s] = sum_c dL/dW * A, dL/ddmin = -sum_c dL/dW * B over the
//                 superblock's 256 entries (one wave per superblock)
//   write_back    the container bytes with only the fp16 d / dmin fields replaced
// All HBM-bound.
#include <hip/hip_runtime.h>

#include "cp_device.h"
#include "cp_host.h"

namespace cp {

struct LinLayout {
  int bp, d_off, dmin_off;  // dmin_off < 0: no min side
};

__host__ __device__ inline bool lin_layout(int ttype, LinLayout* L) {
  switch (ttype) {
    case CP_Q2_K: *L = {84, 80, 82}; return true;
    case CP_Q3_K: *L = {110, 108, -1}; return true;
    case CP_Q4_K: *L = {144, 0, 2}; return true;
    case CP_Q5_K: *L = {176, 0, 2}; return true;
    case CP_Q6_K: *L = {210, 208, -1}; return true;
    default: return false;
  }
}

// One thread per 16 consecutive weights of a superblock: the sub-block's integer scale
// and min, and the signed codes (the field layouts of the k-quant decoders).
template <int TT, class T>
__global__ __launch_bounds__(256) void lin_extract_kernel(const uint8_t* __restrict__ raw,
                                                          int64_t NB, float* __restrict__ d,
                                                          float* __restrict__ dmin,
                                                          T* __restrict__ A, T* __restrict__ B) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t sb = t >> 4;
  if (sb >= NB) return;
  const int k = (int)(t & 15);
  LinLayout L;
  lin_layout(TT, &L);
  const uint8_t* b = raw + sb * L.bp;
  if (k == 0) {
    d[sb] = half_value(b[L.d_off] | b[L.d_off + 1] << 8);
    if (L.dmin_off >= 0) dmin[sb] = half_value(b[L.dmin_off] | b[L.dmin_off + 1] << 8);
  }
  int sc, mn = 0, q[16];
  if constexpr (TT == CP_Q2_K) {
    sc = b[k] & 0xF;
    mn = b[k] >> 4;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      q[i] = (b[16 + h * 32 + l] >> (2 * gq)) & 3;
    }
  } else if constexpr (TT == CP_Q3_K) {
    const uint8_t* s = b + 96;
    const int lo = (k < 8) ? (s[k] & 0xF) : (s[k - 8] >> 4);
    const int hi = (s[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    sc = (lo | hi << 4) - 32;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      const int lo2 = (b[32 + h * 32 + l] >> (2 * gq)) & 3;
      const int hb = (b[e & 31] >> (e >> 5)) & 1;
      q[i] = lo2 - (hb ? 0 : 4);
    }
  } else if constexpr (TT == CP_Q4_K || TT == CP_Q5_K) {
    constexpr int body = TT == CP_Q5_K ? 48 : 16;
    const uint8_t* s = b + 4;
    const int j = k >> 1;
    if (j < 4) {
      sc = s[j] & 63;
      mn = s[j + 4] & 63;
    } else {
      sc = (s[j + 4] & 0xF) | (s[j - 4] >> 6) << 4;
      mn = (s[j + 4] >> 4) | (s[j] >> 6) << 4;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * k + i, c = e >> 6, r = e & 63;
      int v = (r < 32) ? (b[body + c * 32 + r] & 0xF) : (b[body + c * 32 + r - 32] >> 4);
      if constexpr (TT == CP_Q5_K) v |= ((b[16 + (r & 31)] >> (2 * c + (r >> 5))) & 1) << 4;
      q[i] = v;
    }
  } else {  // Q6_K
    sc = (int8_t)b[192 + k];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = 16 * k + i, h = e >> 7, gq = (e >> 5) & 3, l = e & 31;
      const int qlb = b[h * 64 + (gq & 1) * 32 + l];
      const int low = (gq < 2) ? (qlb & 0xF) : (qlb >> 4);
      const int high = (b[128 + h * 32 + l] >> (2 * gq)) & 3;
      q[i] = (low | high << 4) - 32;
    }
  }
  T* a = A + sb * 256 + 16 * k;
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = (T)(sc * q[i]);
  if (L.dmin_off >= 0) {
    T* m = B + sb * 256 + 16 * k;
#pragma unroll
    for (int i = 0; i < 16; ++i) m[i] = (T)mn;
  }
}

// Four consecutive weights per thread.
__global__ __launch_bounds__(256) void lin_reconstruct_kernel(int64_t count,
                                                              const float* __restrict__ d,
                                                              const float* __restrict__ dmin,
                                                              const int16_t* __restrict__ A,
                                                              const int16_t* __restrict__ B,
                                                              float* __restrict__ W) {
  const int64_t i4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 >= count) return;
  const int64_t sb = i4 >> 8;
  const float ds = d[sb];
  const short4 a = *reinterpret_cast<const short4*>(A + i4);
  float4 w = make_float4(ds * (float)a.x, ds * (float)a.y, ds * (float)a.z, ds * (float)a.w);
  if (dmin) {
    const float ms = dmin[sb];
    const short4 m = *reinterpret_cast<const short4*>(B + i4);
    w.x = w.x - ms * (float)m.x;
    w.y = w.y - ms * (float)m.y;
    w.z = w.z - ms * (float)m.z;
    w.w = w.w - ms * (float)m.w;
  }
  *reinterpret_cast<float4*>(W + i4) = w;
}

// One wave per superblock: each lane takes 4 of the 256 entries, then an xor butterfly.
__global__ __launch_bounds__(256) void lin_grad_kernel(int64_t NB, const float* __restrict__ gW,
                                                       const int16_t* __restrict__ A,
                                                       const int16_t* __restrict__ B,
                                                       float* __restrict__ gd,
                                                       float* __restrict__ gdmin) {
  const int64_t sb = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (sb >= NB) return;
  const int lane = threadIdx.x & 63;
  const int64_t o = sb * 256 + 4 * lane;
  const float4 g = *reinterpret_cast<const float4*>(gW + o);
  const short4 a = *reinterpret_cast<const short4*>(A + o);
  float sa = (g.x * (float)a.x + g.y * (float)a.y) + (g.z * (float)a.z + g.w * (float)a.w);
  float sm = 0.0f;
  if (gdmin) {
    const short4 m = *reinterpret_cast<const short4*>(B + o);
    sm = (g.x * (float)m.x + g.y * (float)m.y) + (g.z * (float)m.z + g.w * (float)m.w);
  }
  for (int s = 32; s >= 1; s >>= 1) {
    sa += __shfl_xor(sa, s);
    sm += __shfl_xor(sm, s);
  }
  if (lane == 0) {
    gd[sb] = sa;
    if (gdmin) gdmin[sb] = -sm;
  }
}

// One thread per byte: the field bytes of d / dmin from the new values, the rest copied.
// raw and out may be the same buffer (each thread reads and writes one byte of its own).
__global__ __launch_bounds__(256) void lin_write_back_kernel(const uint8_t* raw, int64_t nbytes,
                                                             LinLayout L,
                                                             const float* __restrict__ d,
                                                             const float* __restrict__ dmin,
                                                             uint8_t* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nbytes) return;
  const int64_t sb = i / L.bp;
  const int off = (int)(i - sb * L.bp);
  uint8_t v = raw[i];
  if (off == L.d_off || off == L.d_off + 1)
    v = (uint8_t)(half_bits(d[sb]) >> (8 * (off - L.d_off)));
  else if (L.dmin_off >= 0 && (off == L.dmin_off || off == L.dmin_off + 1))
    v = (uint8_t)(half_bits(dmin[sb]) >> (8 * (off - L.dmin_off)));
  out[i] = v;
}

static int lin_check(int ttype, int64_t nrow, int64_t n, LinLayout* L) {
  if (!lin_layout(ttype, L)) return set_error(CP_ERR_TTYPE, "no linear form for container type %d", ttype);
  if (nrow < 0 || n <= 0 || n % 256 || nrow * (n / 256) > ((int64_t)1 << 31))
    return set_error(CP_ERR_SHAPE, "[%lld, %lld]: rows must be positive multiples of 256",
                     (long long)nrow, (long long)n);
  return CP_OK;
}

}  // namespace cp

extern "C" {

int cp_lin_extract(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, float* d, float* dmin,
                   void* A, void* B, int ab_dtype, void* stream) {
  cp::clear_error();
  cp::LinLayout L;
  if (int s = cp::lin_check(ttype, nrow, n, &L)) return s;
  if (nrow == 0) return CP_OK;  // an empty tensor
  const bool has_min = L.dmin_off >= 0;
  if (!raw || !d || !A || (has_min && (!dmin || !B)))
    return cp::set_error(CP_ERR_ARG, "null pointer (dmin and B are required for this type)");
  if (ab_dtype != 0 && ab_dtype != 1) return cp::set_error(CP_ERR_ARG, "ab_dtype must be 0 or 1");
  const int64_t NB = nrow * (n / 256);
  const unsigned blocks = (unsigned)((NB * 16 + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
#define CP_LIN_EXTRACT(TT)                                                                      \
  if (ab_dtype)                                                                                 \
    cp::lin_extract_kernel<TT, float><<<blocks, 256, 0, st>>>(raw, NB, d, dmin, (float*)A,      \
                                                              (float*)B);                       \
  else                                                                                          \
    cp::lin_extract_kernel<TT, int16_t><<<blocks, 256, 0, st>>>(raw, NB, d, dmin, (int16_t*)A,  \
                                                                (int16_t*)B);
  switch (ttype) {
    case CP_Q2_K: CP_LIN_EXTRACT(CP_Q2_K) break;
    case CP_Q3_K: CP_LIN_EXTRACT(CP_Q3_K) break;
    case CP_Q4_K: CP_LIN_EXTRACT(CP_Q4_K) break;
    case CP_Q5_K: CP_LIN_EXTRACT(CP_Q5_K) break;
    default: CP_LIN_EXTRACT(CP_Q6_K) break;
  }
#undef CP_LIN_EXTRACT
  CP_LAUNCHED("linear-form extract");
  return CP_OK;
}

int cp_lin_reconstruct(int64_t nrow, int64_t n, const float* d, const float* dmin,
                       const int16_t* A, const int16_t* B, float* W, void* stream) {
  cp::clear_error();
  if (nrow < 0 || n <= 0 || n % 256) return cp::set_error(CP_ERR_SHAPE, "rows must be multiples of 256");
  if (nrow == 0) return CP_OK;  // an empty tensor
  if (!d || !A || !W || (!dmin != !B)) return cp::set_error(CP_ERR_ARG, "null pointer (dmin and B go together)");
  if (!cp::aligned(A, 8) || (B && !cp::aligned(B, 8)) || !cp::aligned(W, 16))
    return cp::set_error(CP_ERR_ALIGN, "A/B need 8-byte and W 16-byte alignment");
  const int64_t count = nrow * n;
  cp::lin_reconstruct_kernel<<<(unsigned)((count / 4 + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      count, d, dmin, A, B, W);
  CP_LAUNCHED("linear-form reconstruct");
  return CP_OK;
}

int cp_lin_reconstruct_grad(int64_t nrow, int64_t n, const float* gW, const int16_t* A,
                            const int16_t* B, float* gd, float* gdmin, void* stream) {
  cp::clear_error();
  if (nrow < 0 || n <= 0 || n % 256) return cp::set_error(CP_ERR_SHAPE, "rows must be multiples of 256");
  if (nrow == 0) return CP_OK;  // an empty tensor
  if (!gW || !A || !gd || (!gdmin != !B)) return cp::set_error(CP_ERR_ARG, "null pointer (gdmin and B go together)");
  if (!cp::aligned(A, 8) || (B && !cp::aligned(B, 8)) || !cp::aligned(gW, 16))
    return cp::set_error(CP_ERR_ALIGN, "A/B need 8-byte and gW 16-byte alignment");
  const int64_t NB = nrow * (n / 256);
  cp::lin_grad_kernel<<<(unsigned)((NB + 3) / 4), 256, 0, (hipStream_t)stream>>>(NB, gW, A, B, gd,
                                                                                  gdmin);
  CP_LAUNCHED("linear-form gradient");
  return CP_OK;
}

int cp_lin_write_back(int ttype, const uint8_t* raw, int64_t nrow, int64_t n, const float* d,
                      const float* dmin, uint8_t* out, void* stream) {
  cp::clear_error();
  cp::LinLayout L;
  if (int s = cp::lin_check(ttype, nrow, n, &L)) return s;
  if (nrow == 0) return CP_OK;  // an empty tensor
  if (!raw || !d || !out || (L.dmin_off >= 0 && !dmin))
    return cp::set_error(CP_ERR_ARG, "null pointer (dmin is required for this type)");
  const int64_t nbytes = nrow * (n / 256) * L.bp;
  cp::lin_write_back_kernel<<<(unsigned)((nbytes + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      raw, nbytes, L, d, dmin, out);
  CP_LAUNCHED("linear-form write-back");
  return CP_OK;
}

}  // extern "C"
