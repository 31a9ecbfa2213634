// The encode driver's err-vs-stock statistic (coldpress/ef.py:298-304):
//   S = float((((a - b) ** 2) * w).sum())
// over float32 [nrow, n] arrays, w [n] broadcast over rows (ones when absent), every
// term rounded as numpy rounds it (difference, square, product) and summed in numpy's
// order for a full reduction of a contiguous array: the flattened terms in chunks of
// 8192, each chunk summed pairwise, the chunk sums added left to right from 0.0.
//
// numpy's pairwise sum of n values: under 8 values left to right from -0.0; up to 128
// values eight interleaved accumulators r[j] = a[j] + a[j + 8] + ..., then
// ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7)) and the remainder left to right;
// above 128 a split at n2 = n / 2 - (n / 2) % 8 and the two halves' sums added. A full
// chunk of 8192 therefore is a balanced tree over 64 leaves of 128, which one wave
// evaluates with lane j on leaf j and an xor butterfly over the lanes (IEEE addition is
// commutative, so every level adds the same pairs). The last, partial chunk takes the
// general recursion on one thread.
#include <hip/hip_runtime.h>

#include "cp_host.h"

namespace cp {

constexpr int kNpChunk = 8192;  // elements per inner-loop call of numpy's reduction
constexpr int kLeaf = 128;

struct SqErrTerms {
  const float* a;
  const float* b;
  const float* w;  // [n] or null
  int64_t n;
  __device__ __forceinline__ float at(int64_t e) const {
    const float d = a[e] - b[e];
    const float t = d * d;
    return w ? t * w[e % n] : t;
  }
};

// numpy's pairwise sum of a leaf (len <= 128 terms from s).
__device__ __forceinline__ float pw_leaf(const SqErrTerms& f, int64_t s, int len) {
  if (len < 8) {
    float r = -0.0f;
    for (int i = 0; i < len; ++i) r = r + f.at(s + i);
    return r;
  }
  float r[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) r[q] = f.at(s + q);
  const int m = len - len % 8;
  for (int i = 8; i < m; i += 8) {
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = r[q] + f.at(s + i + q);
  }
  float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (int i = m; i < len; ++i) res = res + f.at(s + i);
  return res;
}

// One wave per full chunk c: lane j sums terms c * 8192 + 128 j .. + 127 with eight
// accumulators (float4 loads; n % 4 == 0, so a 4-term group never crosses a row), then
// the butterfly. part[c] receives the chunk's sum.
__global__ __launch_bounds__(256) void sqerr_chunk_kernel(SqErrTerms f, int64_t nfull,
                                                          float* __restrict__ part) {
  const int64_t c = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;  // uniform per wave
  if (c >= nfull) return;
  const int j = threadIdx.x & 63;
  const int64_t e0 = c * kNpChunk + (int64_t)j * kLeaf;
  const float4* a4 = reinterpret_cast<const float4*>(f.a + e0);
  const float4* b4 = reinterpret_cast<const float4*>(f.b + e0);
  int64_t col = e0 % f.n;
  float r[8];
#pragma unroll
  for (int k = 0; k < kLeaf / 4; ++k) {
    const float4 av = a4[k], bv = b4[k];
    float d0 = av.x - bv.x, d1 = av.y - bv.y, d2 = av.z - bv.z, d3 = av.w - bv.w;
    float t0 = d0 * d0, t1 = d1 * d1, t2 = d2 * d2, t3 = d3 * d3;
    if (f.w) {
      const float4 wv = *reinterpret_cast<const float4*>(f.w + col);
      t0 = t0 * wv.x;
      t1 = t1 * wv.y;
      t2 = t2 * wv.z;
      t3 = t3 * wv.w;
    }
    col += 4;
    if (col >= f.n) col -= f.n;
    const int q = 4 * (k & 1);  // terms 4k .. 4k + 3 feed accumulators q .. q + 3
    if (k < 2) {
      r[q] = t0;
      r[q + 1] = t1;
      r[q + 2] = t2;
      r[q + 3] = t3;
    } else {
      r[q] = r[q] + t0;
      r[q + 1] = r[q + 1] + t1;
      r[q + 2] = r[q + 2] + t2;
      r[q + 3] = r[q + 3] + t3;
    }
  }
  float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s = s + __shfl_xor(s, m);
  if (j == 0) part[c] = s;
}

// One thread: the chunk sums left to right from 0.0, then the partial chunk by numpy's
// recursion, unrolled onto an explicit stack in LDS (a frame per pending right half; a
// chunk under 8192 terms splits at most 7 times before its leaves).
__global__ __launch_bounds__(64) void sqerr_finish_kernel(SqErrTerms f, int64_t N,
                                                          const float* __restrict__ part,
                                                          float* __restrict__ out) {
  __shared__ int64_t st_s[8];
  __shared__ int st_n[8], st_state[8];
  __shared__ float st_left[8];
  if (threadIdx.x != 0) return;
  const int64_t nfull = N / kNpChunk;
  float total = 0.0f;
  for (int64_t c = 0; c < nfull; ++c) total = total + part[c];
  int64_t s = nfull * kNpChunk;
  int n = (int)(N - s);
  if (n > 0) {
    int top = 0;
    float v = 0.0f;
    for (;;) {
      while (n > kLeaf) {  // split: the right half waits on the stack
        int n2 = n / 2;
        n2 -= n2 % 8;
        st_s[top] = s + n2;
        st_n[top] = n - n2;
        st_state[top] = 0;
        ++top;
        n = n2;
      }
      v = pw_leaf(f, s, n);
      while (top > 0 && st_state[top - 1] == 1) {  // both halves known: combine
        v = st_left[top - 1] + v;
        --top;
      }
      if (top == 0) break;
      st_left[top - 1] = v;  // a left half done: sum the right half next
      st_state[top - 1] = 1;
      s = st_s[top - 1];
      n = st_n[top - 1];
    }
    total = total + v;
  }
  *out = total;
}

}  // namespace cp

extern "C" size_t cp_sq_err_ws_bytes(int64_t nrow, int64_t n) {
  if (nrow <= 0 || n <= 0) return 0;
  return (size_t)((nrow * n) / cp::kNpChunk) * sizeof(float);
}

extern "C" int cp_sq_err_sum(const float* a, const float* b, const float* w, int64_t nrow, int64_t n,
                             float* out, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  if (nrow < 0 || n <= 0 || n % 4) return cp::set_error(CP_ERR_SHAPE, "bad shape [%lld, %lld] (n %% 4 == 0)",
                                                        (long long)nrow, (long long)n);
  if (!out || (nrow && (!a || !b))) return cp::set_error(CP_ERR_ARG, "null pointer");
  if (!cp::aligned(a, 16) || !cp::aligned(b, 16) || (w && !cp::aligned(w, 16)) || !cp::aligned(out, 4))
    return cp::set_error(CP_ERR_ALIGN, "a, b, w need 16-byte alignment");
  const int64_t N = nrow * n, nfull = N / cp::kNpChunk;
  if (nfull && (!ws || ws_bytes < (size_t)nfull * sizeof(float)))
    return cp::set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes,
                         (size_t)nfull * sizeof(float));
  hipStream_t st = (hipStream_t)stream;
  const cp::SqErrTerms f{a, b, w, n};
  float* part = (float*)ws;
  if (nfull) {
    cp::sqerr_chunk_kernel<<<dim3((unsigned)((nfull + 3) / 4)), 256, 0, st>>>(f, nfull, part);
    CP_LAUNCHED("sq err chunks");
  }
  cp::sqerr_finish_kernel<<<1, 64, 0, st>>>(f, N, part, out);
  CP_LAUNCHED("sq err finish");
  return CP_OK;
}
