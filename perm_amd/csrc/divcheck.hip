// Device self-check of the shared-divisor division (cp_device.h: div_recip / div_by)
// against the compiler's IEEE float32 division, on pseudo-random operands inside
// div_box (random sign, exponent and mantissa), zero numerators, and the box's end
// values. No counterpart in the reference.
#include "cp_device.h"
#include "cp_host.h"

namespace cp {
namespace {

__device__ __forceinline__ uint32_t mix32(uint64_t x) {
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdULL;
  x ^= x >> 33;
  x *= 0xc4ceb9fe1a85ec53ULL;
  x ^= x >> 33;
  return (uint32_t)x;
}

// A float in div_box from 32 random bits: sign, exponent in [-40, 39], mantissa.
// Every 64th value is an end of the box (2^-40 or the largest float below 2^40, or
// 2^40 itself), with a random sign.
__device__ __forceinline__ float box_value(uint32_t r, uint32_t r2) {
  const uint32_t sign = r & 0x80000000u;
  if ((r2 & 63) == 0) {
    const uint32_t e = (r2 >> 6) % 3;
    const uint32_t bits = e == 0 ? 0x2B800000u : e == 1 ? 0x537FFFFFu : 0x53800000u;
    return __uint_as_float(sign | bits);
  }
  const uint32_t exp = 127 - 40 + (r >> 23 & 0xFF) % 80;
  return __uint_as_float(sign | exp << 23 | (r & 0x7FFFFF));
}

__global__ void div_check_kernel(int64_t n, uint64_t seed, unsigned long long* bad) {
  unsigned long long local = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t k = seed + 4 * (uint64_t)i;
    const float b = box_value(mix32(k), mix32(k + 1));
    const uint32_t ra = mix32(k + 2);
    const float a = (ra & 255) == 0 ? __uint_as_float(ra & 0x80000000u) : box_value(ra, mix32(k + 3));
    const float ref = a / b;
    const float got = div_by(a, b, div_recip(b));
    local += __float_as_uint(ref) != __float_as_uint(got);
  }
  if (local) atomicAdd(bad, local);
}

}  // namespace
}  // namespace cp

extern "C" int cp_check_division(int64_t n, uint64_t seed, int64_t* mismatches, void* stream) {
  cp::clear_error();
  if (n < 0 || !mismatches) return cp::set_error(CP_ERR_ARG, "cp_check_division: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  unsigned long long* d_bad = nullptr;
  CP_HIP(hipMallocAsync((void**)&d_bad, sizeof(unsigned long long), st));
  CP_HIP(hipMemsetAsync(d_bad, 0, sizeof(unsigned long long), st));
  cp::div_check_kernel<<<2048, 256, 0, st>>>(n, seed, d_bad);
  unsigned long long h = 0;
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(&h, d_bad, sizeof(h), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFreeAsync(d_bad, st);
  if (e != hipSuccess) return cp::hip_fail(e, "cp_check_division");
  *mismatches = (int64_t)h;
  return CP_OK;
}
