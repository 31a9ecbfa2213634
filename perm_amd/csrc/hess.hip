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
  // rows t0..t0+3, channels c0..c0+7; d % 8 == 0 and c0 % 8 == 0, so the 8
  // channels are either all inside the matrix or all outside. Out-of-range
  // blocks load a clamped in-range address and are zeroed without branching.
  const bool cin = c0 < d;
  const int cc = cin ? c0 : 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t t = t0 + q;
    const bool ok = cin && t < N;
    const int64_t tc = t < N ? t : N - 1;
    uint4 x = *reinterpret_cast<const uint4*>(X + tc * d + cc);
    v[q] = ok ? x : make_uint4(0, 0, 0, 0);
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

// ---------------------------------------------------------------- bf16, large tiles
// Lower-triangle tiles of 256 x 256 (H is symmetric; hess_mirror_kernel copies
// the lower triangle into the upper one afterwards). Each of the 8 waves owns
// a 128 x 64 block as 4 x 2 MFMA 32x32 tiles (128 float32 accumulators), so a
// 16-byte LDS fragment feeds 2 to 4 MFMAs; two waves share each SIMD. Work items
// (row split, tile) are ordered split-major and handed out XCD-contiguously:
// the hardware places workgroup w on XCD w % 8, so item = (w % 8) * per + w / 8
// keeps the workgroups of one XCD on the same rows of X (shared in its L2).
constexpr int BT = 256;

__global__ __launch_bounds__(512) void hess_bf16_tri_kernel(const uint16_t* __restrict__ X, int64_t N,
                                                            int d, int ntiles, int splits,
                                                            int64_t rows_per_split,
                                                            float* __restrict__ H) {
  __shared__ uint16_t sA[2][BT * KP];
  __shared__ uint16_t sB[2][BT * KP];
  const int total = ntiles * splits;
  const int per = (total + 7) / 8;
  const int item = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (item >= total) return;
  const int split = item / ntiles, tile = item - split * ntiles;
  int ti = (int)((sqrtf(8.0f * (float)tile + 1.0f) - 1.0f) * 0.5f);
  while (ti * (ti + 1) / 2 > tile) --ti;
  while ((ti + 1) * (ti + 2) / 2 <= tile) ++ti;
  const int tj = tile - ti * (ti + 1) / 2;
  const int i0 = ti * BT, j0 = tj * BT;
  const int64_t r0 = (int64_t)split * rows_per_split;
  const int64_t r1 = min(N, r0 + rows_per_split);
  if (r0 >= r1) return;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = (w >> 2) * 128, wn = (w & 3) * 64;  // 8 waves: 2 x 4 quadrants of 128 x 64
  // loader: threads 0..255 stage the i-panel, 256..511 the j-panel, a 4(t) x 8 block each
  // Lanes 8k..8k+7 take rows 0, 4, .., 28 of one 8-channel block, so each
  // transposed 8-byte LDS store of a 16-lane phase covers two 64-byte row runs
  // on disjoint banks; a wave's 16-byte global loads read 8 rows x 128 bytes.
  const bool loadsA = tid < 256;
  const int lt = (tid & 7) * 4;            // 0..28
  const int lc = ((tid & 255) >> 3) * 8;   // 0..248
  const int cbase = (loadsA ? i0 : j0) + lc;

  f32x16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

  uint4 blk[4];
  load_block_bf16(X, r1, d, r0 + lt, cbase, blk);
  store_block_bf16(loadsA ? sA[0] : sB[0], lc, lt, blk);
  __syncthreads();
  int buf = 0;
  for (int64_t t0 = r0; t0 < r1; t0 += KT) {
    // the next step's rows (clamped loads past the end are discarded)
    load_block_bf16(X, r1, d, t0 + KT + lt, cbase, blk);
#pragma unroll
    for (int kk = 0; kk < KT / 16; ++kk) {
      const int koff = kk * 16 + 8 * (l >> 5);
      bf16x8 a[4], b[2];
#pragma unroll
      for (int x = 0; x < 4; ++x)
        a[x] = *reinterpret_cast<const bf16x8*>(&sA[buf][(wm + x * 32 + (l & 31)) * KP + koff]);
#pragma unroll
      for (int y = 0; y < 2; ++y)
        b[y] = *reinterpret_cast<const bf16x8*>(&sB[buf][(wn + y * 32 + (l & 31)) * KP + koff]);
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[x], b[y], acc[x][y], 0, 0, 0);
    }
    store_block_bf16(loadsA ? sA[buf ^ 1] : sB[buf ^ 1], lc, lt, blk);
    __syncthreads();
    buf ^= 1;
  }
  // lane l holds, for register v of tile (x, y), row wm + 32x + mfma32_row(v, l)
  // and column wn + 32y + l % 32 of the workgroup tile
  float* Hb = H + (int64_t)(i0 + wm + 4 * (l >> 5)) * d + (j0 + wn + (l & 31));
  if (ti != tj && i0 + BT <= d) {
    // interior tile strictly below the diagonal: every element is stored
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          atomicAdd(Hb + (int64_t)(x * 32 + 8 * (v >> 2) + (v & 3)) * d + y * 32, acc[x][y][v]);
  } else {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int i = i0 + wm + x * 32 + mfma32_row(v, l);
          const int j = j0 + wn + y * 32 + (l & 31);
          if (i < d && j <= i)
            atomicAdd(Hb + (int64_t)(x * 32 + 8 * (v >> 2) + (v & 3)) * d + y * 32, acc[x][y][v]);
        }
  }
}

// H[i][j] = H[j][i] for i < j, through 64 x 64 LDS tiles.
__global__ __launch_bounds__(256) void hess_mirror_kernel(float* __restrict__ H, int d) {
  __shared__ float tl[64][65];
  const int bi = blockIdx.y, bj = blockIdx.x;  // target tile (upper): rows bi, cols bj
  if (bj < bi) return;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // source: lower tile rows bj, cols bi
  for (int r = ty; r < 64; r += 4) {
    int i = bj * 64 + r, j = bi * 64 + tx;
    if (i < d && j < d) tl[r][tx] = H[(int64_t)i * d + j];
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    int i = bi * 64 + r, j = bj * 64 + tx;
    if (i < d && j < d && j > i) H[(int64_t)i * d + j] = tl[tx][r];
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

// Row splits for the triangle kernel: as many workgroups as fill whole rounds
// of the 256 CUs (one 80 KB-LDS workgroup per CU), each split >= 1024 rows.
static int pick_splits(int ntiles, int64_t N) {
  int best_s = 1;
  double best_eff = -1.0;
  for (int s = 1; s <= 256; ++s) {
    if (s > 1 && N / s < 1024) break;
    const int64_t wg = (int64_t)ntiles * s;
    const int64_t rounds = (wg + 255) / 256;
    const double eff = (double)wg / (double)(rounds * 256);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best_s = s;
    }
  }
  return best_s;
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
  if (x_dtype == 1) {
    const int T = (int)((d + cp::BT - 1) / cp::BT);
    const int ntiles = T * (T + 1) / 2;
    const int splits = cp::pick_splits(ntiles, N);
    int64_t rps = (N + splits - 1) / splits;
    rps = (rps + cp::KT - 1) / cp::KT * cp::KT;
    const int total = ntiles * splits;
    const int per = (total + 7) / 8;
    cp::hess_bf16_tri_kernel<<<dim3(8 * per), 512, 0, st>>>((const uint16_t*)X, N, (int)d, ntiles,
                                                            splits, rps, H);
    CP_LAUNCHED("hessian launch");
    const int tb = (int)((d + 63) / 64);
    cp::hess_mirror_kernel<<<dim3(tb, tb), 256, 0, st>>>(H, (int)d);
    CP_LAUNCHED("hessian mirror");
    return CP_OK;
  }
  const int tiles = (int)((d + cp::HT - 1) / cp::HT);
  // enough row splits for ~4 workgroups per CU, each at least 512 rows
  int64_t want = (1024 + (int64_t)tiles * tiles - 1) / ((int64_t)tiles * tiles);
  int64_t splits = want < 1 ? 1 : want;
  int64_t rps = (N + splits - 1) / splits;
  if (rps < 512) rps = 512;
  rps = (rps + cp::KT - 1) / cp::KT * cp::KT;
  splits = (N + rps - 1) / rps;
  dim3 grid(tiles, tiles, (unsigned)splits);
  cp::hess_f32_kernel<<<grid, 256, 0, st>>>((const float*)X, N, (int)d, rps, H);
  CP_LAUNCHED("hessian launch");
  return CP_OK;
}
