// Input-Hessian accumulation H += X^T X on gfx950 MFMA (coldpress/hessians.py:137-154).
//
// X is [N, d] row-major activations (bf16 or f32), H is [d, d] float32 and is
// accumulated in place (beta = 1), so hook batches can stream in.
//
// Tiling: a workgroup (4 waves) owns a 128x128 tile of H and a contiguous range
// of rows of X (split-K over rows: N is 65536-131072 while d is 1024-14336, so
// the row dimension is what fills 256 CUs). Each wave computes a 64x64 quadrant
// with 2x2 MFMA 32x32 tiles. Per 32-row step the workgroup stages the two
// 32x128 X panels (rows t, columns i-tile and j-tile) in LDS, double buffered.
//
//  bf16: v_mfma_f32_32x32x16_bf16 needs 8 consecutive rows t per lane for both
//        operands, while X is channel-contiguous; each thread loads a 4(t) x
//        8(i) block with 16-byte loads, transposes it in registers
//        (v_perm_b32) and writes t-contiguous 8-byte runs into [i][t] LDS.
//  f32:  v_mfma_f32_32x32x2f32 takes one t per lane, so the [t][i] panel is
//        used as loaded.
// The finished tile is added into H with float32 atomics (one per element per
// workgroup): the sum over row splits is exact up to float32 rounding order.
#include <hip/hip_runtime.h>

#include "cp_host.h"

namespace cp {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int HT = 128;  // H tile edge
constexpr int KT = 32;   // rows of X per step

// Row of the 32x32 MFMA result held by register v of lane l (column = l % 32).
__device__ __forceinline__ int mfma32_row(int v, int l) { return 8 * (v >> 2) + 4 * (l >> 5) + (v & 3); }

// ---------------------------------------------------------------- bf16 input
// LDS panel for bf16: [HT][KT + 8] (padding breaks the 64-byte row stride)
constexpr int KP = KT + 8;

__device__ __forceinline__ void load_block_bf16(const uint16_t* __restrict__ X, int64_t N, int d,
                                                int64_t t0, int c0, uint4 (&v)[4]) {
  // rows t0..t0+3, channels c0..c0+7
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int64_t t = t0 + q;
    if (t < N && c0 + 7 < d) {
      v[q] = *reinterpret_cast<const uint4*>(X + t * d + c0);
    } else {
      uint32_t w[4] = {0, 0, 0, 0};
      if (t < N)
        for (int c = 0; c < 8; ++c)
          if (c0 + c < d) w[c >> 1] |= (uint32_t)X[t * d + c0 + c] << (16 * (c & 1));
      v[q] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

__device__ __forceinline__ void store_block_bf16(uint16_t* panel, int i0, int tl, const uint4 (&v)[4]) {
  // transpose 4(t) x 8(i) -> for each i, 4 consecutive t (8 bytes)
  const uint32_t w[4][4] = {{v[0].x, v[0].y, v[0].z, v[0].w},
                            {v[1].x, v[1].y, v[1].z, v[1].w},
                            {v[2].x, v[2].y, v[2].z, v[2].w},
                            {v[3].x, v[3].y, v[3].z, v[3].w}};
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    uint32_t lo = __builtin_amdgcn_perm(w[1][c >> 1], w[0][c >> 1], sel);
    uint32_t hi = __builtin_amdgcn_perm(w[3][c >> 1], w[2][c >> 1], sel);
    *reinterpret_cast<uint2*>(panel + (i0 + c) * KP + tl) = make_uint2(lo, hi);
  }
}

__global__ __launch_bounds__(256) void hess_bf16_kernel(const uint16_t* __restrict__ X, int64_t N,
                                                        int d, int64_t rows_per_split,
                                                        float* __restrict__ H) {
  __shared__ uint16_t sA[2][HT * KP];
  __shared__ uint16_t sB[2][HT * KP];
  const int ti = blockIdx.y, tj = blockIdx.x;
  const int i0 = ti * HT, j0 = tj * HT;
  const int64_t r0 = (int64_t)blockIdx.z * rows_per_split;
  const int64_t r1 = min(N, r0 + rows_per_split);
  if (r0 >= r1) return;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = (w >> 1) * 64, wn = (w & 1) * 64;
  // loader role: 128 threads per panel, each a 4(t) x 8(i) block
  const bool loadsA = tid < 128;
  const int lb = tid & 127;
  const int lt = (lb >> 4) * 4;    // 0..28
  const int lc = (lb & 15) * 8;    // 0..120
  const int cbase = loadsA ? i0 : j0;

  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  uint4 blk[4];
  load_block_bf16(X, r1, d, r0 + lt, cbase + lc, blk);
  store_block_bf16(loadsA ? sA[0] : sB[0], lc, lt, blk);
  __syncthreads();
  int buf = 0;
  for (int64_t t0 = r0; t0 < r1; t0 += KT) {
    const bool more = t0 + KT < r1;
    if (more) load_block_bf16(X, r1, d, t0 + KT + lt, cbase + lc, blk);
#pragma unroll
    for (int kk = 0; kk < KT / 16; ++kk) {
      const int koff = kk * 16 + 8 * (l >> 5);
      bf16x8 a[2], b[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        a[x] = *reinterpret_cast<const bf16x8*>(&sA[buf][(wm + x * 32 + (l & 31)) * KP + koff]);
        b[x] = *reinterpret_cast<const bf16x8*>(&sB[buf][(wn + x * 32 + (l & 31)) * KP + koff]);
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[x], b[y], acc[x][y], 0, 0, 0);
    }
    if (more) store_block_bf16(loadsA ? sA[buf ^ 1] : sB[buf ^ 1], lc, lt, blk);
    __syncthreads();
    buf ^= 1;
  }
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int i = i0 + wm + x * 32 + mfma32_row(v, l);
        int j = j0 + wn + y * 32 + (l & 31);
        if (i < d && j < d) atomicAdd(H + (int64_t)i * d + j, acc[x][y][v]);
      }
}

// ---------------------------------------------------------------- f32 input
__global__ __launch_bounds__(256) void hess_f32_kernel(const float* __restrict__ X, int64_t N, int d,
                                                       int64_t rows_per_split, float* __restrict__ H) {
  __shared__ float sA[KT][HT + 4];
  __shared__ float sB[KT][HT + 4];
  const int i0 = blockIdx.y * HT, j0 = blockIdx.x * HT;
  const int64_t r0 = (int64_t)blockIdx.z * rows_per_split;
  const int64_t r1 = min(N, r0 + rows_per_split);
  if (r0 >= r1) return;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = (w >> 1) * 64, wn = (w & 1) * 64;
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  for (int64_t t0 = r0; t0 < r1; t0 += KT) {
    for (int idx = tid; idx < KT * HT; idx += 256) {
      int tt = idx / HT, c = idx % HT;
      int64_t t = t0 + tt;
      sA[tt][c] = (t < r1 && i0 + c < d) ? X[t * d + i0 + c] : 0.0f;
      sB[tt][c] = (t < r1 && j0 + c < d) ? X[t * d + j0 + c] : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < KT; k += 2) {
      float a[2], b[2];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        a[x] = sA[k + (l >> 5)][wm + x * 32 + (l & 31)];
        b[x] = sB[k + (l >> 5)][wn + x * 32 + (l & 31)];
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[x], b[y], acc[x][y], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int i = i0 + wm + x * 32 + mfma32_row(v, l);
        int j = j0 + wn + y * 32 + (l & 31);
        if (i < d && j < d) atomicAdd(H + (int64_t)i * d + j, acc[x][y][v]);
      }
}

}  // namespace cp

extern "C" int cp_hess_accum(const void* X, int x_dtype, int64_t N, int64_t d, float* H, void* stream) {
  cp::clear_error();
  if (!X || !H) return cp::set_error(CP_ERR_ARG, "null X/H");
  if (N <= 0 || d <= 0 || d > (1 << 20)) return cp::set_error(CP_ERR_SHAPE, "bad X shape [%lld, %lld]", (long long)N, (long long)d);
  if (x_dtype != 0 && x_dtype != 1) return cp::set_error(CP_ERR_ARG, "x_dtype must be 0 (f32) or 1 (bf16)");
  if (!cp::aligned(X, 16) || !cp::aligned(H, 4)) return cp::set_error(CP_ERR_ALIGN, "X needs 16-byte alignment");
  if (x_dtype == 1 && d % 8) return cp::set_error(CP_ERR_SHAPE, "bf16 X needs d %% 8 == 0 (got %lld)", (long long)d);
  hipStream_t st = (hipStream_t)stream;
  const int tiles = (int)((d + cp::HT - 1) / cp::HT);
  // enough row splits for ~4 workgroups per CU, each at least 512 rows
  int64_t want = (1024 + (int64_t)tiles * tiles - 1) / ((int64_t)tiles * tiles);
  int64_t splits = want < 1 ? 1 : want;
  int64_t rps = (N + splits - 1) / splits;
  if (rps < 512) rps = 512;
  rps = (rps + cp::KT - 1) / cp::KT * cp::KT;
  splits = (N + rps - 1) / rps;
  dim3 grid(tiles, tiles, (unsigned)splits);
  if (x_dtype == 1)
    cp::hess_bf16_kernel<<<grid, 256, 0, st>>>((const uint16_t*)X, N, (int)d, rps, H);
  else
    cp::hess_f32_kernel<<<grid, 256, 0, st>>>((const float*)X, N, (int)d, rps, H);
  CP_LAUNCHED("hessian launch");
  return CP_OK;
}
