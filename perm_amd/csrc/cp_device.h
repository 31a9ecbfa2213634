// Device-side numerics shared by the k-quant and EF kernels (gfx950).
//
// Every routine here reproduces a float32 operation sequence of the numpy
// encoder in coldpress/kquant.py bit for bit. The library is compiled with
// -ffp-contract=off (no fused multiply-add), IEEE division and sqrt, and f32
// denormals preserved, so each C++ expression below rounds exactly where the
// numpy expression it restates rounds.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cp {

// ggml nearest_int: round half to even via the 1.5*2^23 magic add
// (kquant.py:25-28). Outside |v| < 2^22 this returns the same deterministic
// bit pattern as the reference, which callers clip.
__device__ __forceinline__ int rint_magic(float v) {
  float s = v + 12582912.0f;
  return (__float_as_int(s) & 0x7FFFFF) - 0x400000;
}

// IEEE float32 division with a shared divisor. The correctly rounded quotient the
// compiler emits for a / b is: y = rcp(b') refined once, y1 = fma(fma(-b', y, 1), y, y);
// q0 = a' * y1; two corrections q = fma(fma(-b', q, a'), y1, q); then v_div_fixup.
// a' and b' are a and b after v_div_scale, which rescales only operands near the
// ends of the exponent range, and v_div_fixup changes only special results. For a
// and b inside div_box both are identities, so div_by(a, b, div_recip(b)) runs the
// same operations on the same values and returns the same bits, while the refined
// reciprocal y1 is formed once per divisor instead of once per quotient. A zero a
// keeps its sign (a * y1). cp_check_division compares the two on the device.
__device__ __forceinline__ bool div_box(float v) {
  const float m = fabsf(v);
  return m >= 0x1p-40f && m <= 0x1p40f;
}

__device__ __forceinline__ float div_recip(float b) {
  const float y = __builtin_amdgcn_rcpf(b);
  return __fmaf_rn(__fmaf_rn(-b, y, 1.0f), y, y);
}

// a / b for b in div_box and a == 0 or in div_box; y1 = div_recip(b).
__device__ __forceinline__ float div_by(float a, float b, float y1) {
  const float q0 = a * y1;
  const float q1 = __fmaf_rn(__fmaf_rn(-b, q0, a), y1, q0);
  const float q2 = __fmaf_rn(__fmaf_rn(-b, q1, a), y1, q1);
  return a == 0.0f ? q0 : q2;
}

// Whether div_by gives a / b for this numerator (the divisor checked separately).
__device__ __forceinline__ bool div_num_ok(float a) { return a == 0.0f || div_box(a); }

__device__ __forceinline__ uint16_t half_bits(float v) {
  _Float16 h = (_Float16)v;  // v_cvt_f16_f32, round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float half_value(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// The last step of psum: the eight strided partial sums added as a fixed tree (and
// + 0.0f, so a -0 total becomes +0 as numpy's reduction from its +0 identity gives).
__device__ __forceinline__ float psum_tree(const float (&r)[8]) {
  const float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  return 0.0f + s;
}

// numpy's float32 pairwise sum of N contiguous values (8 <= N <= 128, N % 8 == 0):
// eight interleaved accumulators r[j] = a[j] + a[j+8] + ..., then
// ((r0+r1)+(r2+r3)) + ((r4+r5)+(r6+r7)); the reduction starts from +0.0.
template <int N>
__device__ __forceinline__ float psum(const float (&a)[N]) {
  static_assert(N % 8 == 0 && N >= 8 && N <= 128, "pairwise block");
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = a[j];
#pragma unroll
  for (int i = 8; i < N; i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = r[j] + a[i + j];
  }
  return psum_tree(r);
}

// The same sum over G lanes (one value per lane, G = 8 or 16) as an xor
// butterfly: xor 8 forms r[j] = a[j] + a[j+8], then xor 1, 2, 4 build the tree.
// IEEE addition is commutative, so every lane of the group ends with the
// identical, numpy-ordered result.
template <int G>
__device__ __forceinline__ float gsum(float v) {
  static_assert(G == 8 || G == 16, "group width");
  if (G == 16) v = v + __shfl_xor(v, 8);
  v = v + __shfl_xor(v, 1);
  v = v + __shfl_xor(v, 2);
  v = v + __shfl_xor(v, 4);
  return 0.0f + v;
}

template <int G>
__device__ __forceinline__ float gmax(float v) {
#pragma unroll
  for (int k = G / 2; k >= 1; k >>= 1) v = fmaxf(v, __shfl_xor(v, k));
  return v;
}

// First (lowest lane) value of largest |v| over the group: returns the signed
// value; |value| in *amax (numpy argmax tie rule).
template <int G>
__device__ __forceinline__ float gfirst_absmax(float v, int g, float* amax) {
  float a = fabsf(v);
  int idx = g;
#pragma unroll
  for (int k = G / 2; k >= 1; k >>= 1) {
    float ao = __shfl_xor(a, k);
    float vo = __shfl_xor(v, k);
    int io = __shfl_xor(idx, k);
    bool take = (ao > a) || (ao == a && io < idx);
    a = take ? ao : a;
    v = take ? vo : v;
    idx = take ? io : idx;
  }
  *amax = a;
  return v;
}

template <int G>
__device__ __forceinline__ float gbcast(float v, int src) {
  return __shfl(v, src, G);
}

}  // namespace cp
