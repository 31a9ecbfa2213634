// Hessian storage format on gfx950 (coldpress/hessians.py:163-243): H is kept as
// float16 off-diagonal values over a per-matrix scale, with the diagonal exact in
// float32.
//
// pack    amax = max |H| (order-free, exact); hscale = amax / 32768 when amax > 32768,
//         else 1 -- 32768 is a power of two, so amax * 2^-15 is exact in float32;
//         H16 = f16(H / hscale) with a correctly rounded float32 division and
//         round-to-nearest-even to f16 (numpy's astype); diag32 = diag(H).
// expand  H = double(H16) * double(hscale) (exact: 11 + 24 significant bits), then the
//         float32 diagonal written over it; a float32 H (the older format) is widened.
// Both are HBM-bound elementwise passes (pack: 4 B in, 2 B out per entry after the
// absmax pass's 4 B; expand: 2 or 4 B in, 8 B out).
#include <hip/hip_runtime.h>

#include "cp_device.h"
#include "cp_host.h"

namespace cp {

constexpr float kFp16SafeMax = 32768.0f;

// max |x| over the matrix: non-negative floats order like their bit patterns, so an
// unsigned atomic max on the bits is exact and order-free. amax_bits starts at 0.
// One atomic per block (the waves' maxima meet in LDS first): atomics on one address
// serialize, so their count, not the reads, would otherwise set the time.
constexpr int kAbsmaxBlocks = 512;

__global__ __launch_bounds__(256) void h2_absmax_kernel(const float* __restrict__ H, int64_t count,
                                                        unsigned* __restrict__ amax_bits) {
  __shared__ unsigned wmax[4];
  unsigned m = 0;
  // 16-byte loads when H is 16-byte aligned (the usual case), 4-byte ones otherwise
  const int64_t n4 = ((uintptr_t)H & 15) == 0 ? count / 4 : 0;
  const uint4* H4 = reinterpret_cast<const uint4*>(H);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const uint4 v = H4[i];
    const unsigned a = max(v.x & 0x7FFFFFFFu, v.y & 0x7FFFFFFFu);
    const unsigned b = max(v.z & 0x7FFFFFFFu, v.w & 0x7FFFFFFFu);
    m = max(m, max(a, b));
  }
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * 256)
    m = max(m, __float_as_uint(H[i]) & 0x7FFFFFFFu);
  for (int o = 32; o >= 1; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) atomicMax(amax_bits, max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3])));
}

__global__ void h2_clear_kernel(unsigned* __restrict__ p) { *p = 0u; }

// The elementwise passes take rows r = blockIdx.y, blockIdx.y + gridDim.y, ... and give
// each thread four consecutive columns of them; VEC (n a multiple of 4, the buffers
// aligned for it): 16-byte loads and 8- or 16-byte stores. The row and column come from
// the grid, so the diagonal is found without dividing the flat index by n.
constexpr int kH2Cols = 4 * 256;  // columns per block
constexpr int kH2MaxRowBlocks = 65535;

template <bool VEC>
__global__ __launch_bounds__(256) void h2_pack_kernel(const float* __restrict__ H, int64_t n,
                                                      const unsigned* __restrict__ amax_bits,
                                                      uint16_t* __restrict__ H16,
                                                      float* __restrict__ diag32,
                                                      float* __restrict__ hscale_out) {
  const float amax = __uint_as_float(*amax_bits);
  const float hs = amax > kFp16SafeMax ? amax * (1.0f / kFp16SafeMax) : 1.0f;
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *hscale_out = hs;
  const int64_t c = (int64_t)blockIdx.x * kH2Cols + 4 * (int64_t)threadIdx.x;
  if (c >= n) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) {
    const float* h = H + r * n + c;
    uint16_t* o = H16 + r * n + c;
    float v[4];
    if constexpr (VEC) {
      const float4 q = *reinterpret_cast<const float4*>(h);
      v[0] = q.x;
      v[1] = q.y;
      v[2] = q.z;
      v[3] = q.w;
      ushort4 b;
      b.x = half_bits(v[0] / hs);
      b.y = half_bits(v[1] / hs);
      b.z = half_bits(v[2] / hs);
      b.w = half_bits(v[3] / hs);
      *reinterpret_cast<ushort4*>(o) = b;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = c + j < n ? h[j] : 0.0f;
        if (c + j < n) o[j] = half_bits(v[j] / hs);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c + j == r) diag32[r] = v[j];
  }
}

template <bool F16, bool VEC>
__global__ __launch_bounds__(256) void h2_expand_kernel(const void* __restrict__ Hs, int64_t n,
                                                        double hscale,
                                                        const float* __restrict__ diag32,
                                                        double* __restrict__ H) {
  const int64_t c = (int64_t)blockIdx.x * kH2Cols + 4 * (int64_t)threadIdx.x;
  if (c >= n) return;
  for (int64_t r = blockIdx.y; r < n; r += gridDim.y) {
    const int64_t base = r * n + c;
    double v[4];
    if constexpr (VEC) {
      if constexpr (F16) {
        const ushort4 q = *reinterpret_cast<const ushort4*>(reinterpret_cast<const uint16_t*>(Hs) + base);
        v[0] = (double)half_value(q.x);
        v[1] = (double)half_value(q.y);
        v[2] = (double)half_value(q.z);
        v[3] = (double)half_value(q.w);
      } else {
        const float4 q = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(Hs) + base);
        v[0] = (double)q.x;
        v[1] = (double)q.y;
        v[2] = (double)q.z;
        v[3] = (double)q.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[j] = c + j >= n ? 0.0
               : F16      ? (double)half_value(reinterpret_cast<const uint16_t*>(Hs)[base + j])
                          : (double)reinterpret_cast<const float*>(Hs)[base + j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = v[j] * hscale;
      if (diag32 && c + j == r) v[j] = (double)diag32[r];
    }
    double* o = H + base;
    if constexpr (VEC) {
      *reinterpret_cast<double2*>(o) = make_double2(v[0], v[1]);
      *reinterpret_cast<double2*>(o + 2) = make_double2(v[2], v[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c + j < n) o[j] = v[j];
    }
  }
}

static dim3 h2_grid(int64_t n) {
  return dim3((unsigned)((n + kH2Cols - 1) / kH2Cols), (unsigned)(n < kH2MaxRowBlocks ? n : kH2MaxRowBlocks));
}

}  // namespace cp

extern "C" {

int cp_h2_pack(const float* H, int64_t n, uint16_t* H16, float* diag32, float* hscale,
               void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  if (!H || !H16 || !diag32 || !hscale) return cp::set_error(CP_ERR_ARG, "null pointer");
  if (n <= 0 || n > (1 << 19)) return cp::set_error(CP_ERR_SHAPE, "bad size %lld", (long long)n);
  if (!ws || ws_bytes < 4) return cp::set_error(CP_ERR_WORKSPACE, "workspace %zu < 4 bytes", ws_bytes);
  if (!cp::aligned(H, 4) || !cp::aligned(H16, 2) || !cp::aligned(diag32, 4) ||
      !cp::aligned(hscale, 4) || !cp::aligned(ws, 4))
    return cp::set_error(CP_ERR_ALIGN, "misaligned buffer");
  hipStream_t st = (hipStream_t)stream;
  unsigned* amax = (unsigned*)ws;
  const int64_t count = n * n;
  cp::h2_clear_kernel<<<1, 1, 0, st>>>(amax);
  const int64_t ablocks = (count + 1023) / 1024;
  cp::h2_absmax_kernel<<<(unsigned)(ablocks < 1 ? 1 : (ablocks < cp::kAbsmaxBlocks ? ablocks : cp::kAbsmaxBlocks)),
                         256, 0, st>>>(H, count, amax);
  if (!(n & 3) && cp::aligned(H, 16) && cp::aligned(H16, 8))
    cp::h2_pack_kernel<true><<<cp::h2_grid(n), 256, 0, st>>>(H, n, amax, H16, diag32, hscale);
  else
    cp::h2_pack_kernel<false><<<cp::h2_grid(n), 256, 0, st>>>(H, n, amax, H16, diag32, hscale);
  CP_LAUNCHED("Hessian pack");
  return CP_OK;
}

int cp_h2_expand(const void* Hs, int in_dtype, int64_t n, double hscale, const float* diag32,
                 double* H, void* stream) {
  cp::clear_error();
  if (!Hs || !H) return cp::set_error(CP_ERR_ARG, "null pointer");
  if (in_dtype != 0 && in_dtype != 1) return cp::set_error(CP_ERR_ARG, "in_dtype must be 0 or 1");
  if (n <= 0 || n > (1 << 19)) return cp::set_error(CP_ERR_SHAPE, "bad size %lld", (long long)n);
  if (!cp::aligned(Hs, in_dtype ? 2 : 4) || !cp::aligned(H, 8) || (diag32 && !cp::aligned(diag32, 4)))
    return cp::set_error(CP_ERR_ALIGN, "misaligned buffer");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = cp::h2_grid(n);
  const bool vec = !(n & 3) && cp::aligned(Hs, in_dtype ? 8 : 16) && cp::aligned(H, 16);
  if (in_dtype) {
    if (vec)
      cp::h2_expand_kernel<true, true><<<grid, 256, 0, st>>>(Hs, n, hscale, diag32, H);
    else
      cp::h2_expand_kernel<true, false><<<grid, 256, 0, st>>>(Hs, n, hscale, diag32, H);
  } else {
    if (vec)
      cp::h2_expand_kernel<false, true><<<grid, 256, 0, st>>>(Hs, n, hscale, diag32, H);
    else
      cp::h2_expand_kernel<false, false><<<grid, 256, 0, st>>>(Hs, n, hscale, diag32, H);
  }
  CP_LAUNCHED("Hessian expand");
  return CP_OK;
}

}  // extern "C"
