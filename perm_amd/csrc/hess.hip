// Input-Hessian accumulation H += X^T X on gfx950 MFMA (coldpress/hessians.py:137-154).
//
// X is [N, d] row-major activations (bf16 or f32), H is [d, d] float32 and is
// accumulated in place (beta = 1), so hook batches can stream in. Split-K over
// rows of X: N is 65536-131072 while d is 1024-14336, so the row dimension is
// what fills 256 CUs. Each workgroup adds its finished tile into H with
// float32 atomics (one per element per workgroup): the sum over row splits is
// exact up to float32 rounding order.
//
//  bf16: lower-triangle 256 x 256 tiles on v_mfma_f32_32x32x16_bf16, operands
//        read transposed from LDS (hess_bf16_tri_kernel), then a mirror pass;
//  f32:  128 x 128 tiles on v_mfma_f32_32x32x2f32, which takes one row t per
//        lane, so the [t][i] panel is used as loaded.
#include <hip/hip_runtime.h>

#include "cp_host.h"

namespace cp {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int HT = 128;  // f32 kernel: H tile edge
constexpr int KT = 32;   // f32 kernel: rows of X per step

// Row of the 32x32 MFMA result held by register v of lane l (column = l % 32).
__device__ __forceinline__ int mfma32_row(int v, int l) { return 8 * (v >> 2) + 4 * (l >> 5) + (v & 3); }

// ---------------------------------------------------------------- bf16 input
// Lower-triangle tiles of 256 x 256 (H is symmetric; hess_mirror_kernel copies
// the lower triangle into the upper one afterwards), split-K over rows of X.
// A workgroup is 4 waves, each owning a 128 x 128 block as 4 x 4 MFMA 32x32
// tiles (256 float32 accumulators): the largest block a wave can hold, because
// the LDS reads per MFMA, not the MFMAs, bound this kernel.
//
// Rows of X are staged 32 at a time: both 32 x 256 panels (columns of the i-
// and j-tile; one panel on a diagonal tile) are fetched into registers two
// stages ahead of use, stored into a 3-slot LDS ring in X's own [t][c] layout,
// and read as MFMA operands with ds_read_b64_tr_b16, which returns 4
// consecutive rows t of one column per lane: v_mfma_f32_32x32x16_bf16 takes 8
// consecutive t per lane for both operands. Panel rows are 512 bytes, so the
// four rows of one transposed read would share banks; 64-byte chunks are
// XOR-swizzled by t & 3 to spread them over all banks.
//
// Work items (row split, tile) are ordered split-major and handed out
// XCD-contiguously: the hardware places workgroup w on XCD w % 8, so
// item = (w % 8) * per + w / 8 keeps the workgroups of one XCD on the same
// rows of X (shared in its L2).
constexpr int BT = 256;             // H tile edge
constexpr int KS = 32;              // rows of X per stage
constexpr int PROW = BT * 2;        // bytes per panel row
constexpr int PANEL = KS * PROW;    // 16 KB
constexpr int HNT = 256;            // threads per workgroup
constexpr int NSLOT = 3;            // LDS ring
constexpr int CPT = 2048 / HNT;     // 16-byte chunks per thread per stage (two panels)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4i16* lds_v4p;

__device__ __forceinline__ int pofs(int t, int c) {  // byte offset of (row t, bf16 column c)
  const int b = 2 * c;
  return t * PROW + ((((b >> 6) ^ (t & 3)) << 6) | (b & 63));
}

// chunk ch of a stage: panel ch / 1024, row (ch % 1024) / 32, 16-byte column chunk ch % 32
template <bool DIAG>
__device__ __forceinline__ void stage_load(const uint16_t* X, int64_t N, int d, int64_t t0, int i0,
                                           int j0, int tid, uint4 (&g)[CPT]) {
#pragma unroll
  for (int q = 0; q < (DIAG ? CPT / 2 : CPT); ++q) {
    const int ch = tid + HNT * q, panel = ch >> 10, row = (ch & 1023) >> 5, c16 = ch & 31;
    const int64_t t = t0 + row;
    const int c = (panel ? j0 : i0) + 8 * c16;  // d % 8 == 0: 8 columns all in or all out
    uint4 z = make_uint4(0, 0, 0, 0);
    if (t < N && c < d) z = *reinterpret_cast<const uint4*>(X + t * d + c);
    g[q] = z;
  }
}

template <bool DIAG>
__device__ __forceinline__ void stage_store(char* slot, int tid, const uint4 (&g)[CPT]) {
#pragma unroll
  for (int q = 0; q < (DIAG ? CPT / 2 : CPT); ++q) {
    const int ch = tid + HNT * q, panel = ch >> 10, row = (ch & 1023) >> 5, c16 = ch & 31;
    *reinterpret_cast<uint4*>(slot + panel * PANEL + pofs(row, 8 * c16)) = g[q];
  }
}

// MFMA operand for columns col..col+31 and rows krow..krow+15 of a panel:
// lane l gets column col + l % 32, rows krow + 8 * (l / 32) + 0..7
__device__ __forceinline__ bf16x8 operand(const char* panel, int krow, int col, int l) {
  const int g = l >> 4, c = l & 15;
  const int row = krow + 8 * (g >> 1) + (c >> 2);
  const int cc = col + 16 * (g & 1) + 4 * (c & 3);
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4p)(panel + pofs(row, cc)));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4p)(panel + pofs(row + 4, cc)));
  const v8i16 r = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, r);
}

struct Operands {
  bf16x8 a[4], b[4];
};

__device__ __forceinline__ void read_operands(const char* pa, const char* pb, int half, int wm,
                                              int wn, int l, Operands& f) {
#pragma unroll
  for (int x = 0; x < 4; ++x) f.a[x] = operand(pa, 16 * half, wm + 32 * x, l);
#pragma unroll
  for (int y = 0; y < 4; ++y) f.b[y] = operand(pb, 16 * half, wn + 32 * y, l);
}

__device__ __forceinline__ void multiply(const Operands& f, f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y)
      acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[x], f.b[y], acc[x][y], 0, 0, 0);
}

template <bool DIAG>
__device__ __forceinline__ void tile_rows(const uint16_t* X, int64_t r0, int64_t r1, int d, int i0,
                                          int j0, char* lds, f32x16 (&acc)[4][4]) {
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = (w >> 1) * 128, wn = (w & 1) * 128;
  const int ns = (int)((r1 - r0 + KS - 1) / KS);
  constexpr int SLOT = DIAG ? PANEL : 2 * PANEL;
  auto pa = [&](int s) -> const char* { return lds + (s % NSLOT) * SLOT; };
  auto pb = [&](int s) -> const char* { return DIAG ? pa(s) : pa(s) + PANEL; };
  // rows past r1 load as zeros, so a short split needs no special case
  uint4 g0[CPT], g1[CPT];
  stage_load<DIAG>(X, r1, d, r0, i0, j0, tid, g0);
  stage_load<DIAG>(X, r1, d, r0 + KS, i0, j0, tid, g1);
  stage_store<DIAG>(lds, tid, g0);
  stage_store<DIAG>(lds + SLOT, tid, g1);
  stage_load<DIAG>(X, r1, d, r0 + 2 * KS, i0, j0, tid, g0);
  stage_load<DIAG>(X, r1, d, r0 + 3 * KS, i0, j0, tid, g1);
  __syncthreads();
  Operands f0, f1;
  read_operands(pa(0), pb(0), 0, wm, wn, l, f0);
  // stage s: store stage s + 2 (fetched two stages ago) into the slot stage
  // s - 1 used, fetch stage s + 4 into the same registers, and multiply stage
  // s while reading the next operands (its second half, then the first half of
  // stage s + 1)
  auto step = [&](int s, uint4 (&g)[CPT]) {
    __syncthreads();
    if (s + 2 < ns) stage_store<DIAG>(lds + ((s + 2) % NSLOT) * SLOT, tid, g);
    if (s + 4 < ns) stage_load<DIAG>(X, r1, d, r0 + (int64_t)(s + 4) * KS, i0, j0, tid, g);
    read_operands(pa(s), pb(s), 1, wm, wn, l, f1);
    multiply(f0, acc);
    if (s + 1 < ns) read_operands(pa(s + 1), pb(s + 1), 0, wm, wn, l, f0);
    multiply(f1, acc);
  };
  for (int s = 0; s < ns; s += 2) {
    step(s, g0);
    if (s + 1 < ns) step(s + 1, g1);
  }
}

__global__ __launch_bounds__(HNT) void hess_bf16_tri_kernel(const uint16_t* __restrict__ X, int64_t N,
                                                            int d, int ntiles, int splits,
                                                            int64_t rows_per_split,
                                                            float* __restrict__ H) {
  __shared__ __align__(16) char lds[NSLOT * 2 * PANEL];
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
  const int wm = (w >> 1) * 128, wn = (w & 1) * 128;
  f32x16 acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  if (ti == tj)
    tile_rows<true>(X, r0, r1, d, i0, j0, lds, acc);
  else
    tile_rows<false>(X, r0, r1, d, i0, j0, lds, acc);
  // lane l holds, for register v of tile (x, y), row wm + 32x + mfma32_row(v, l)
  // and column wn + 32y + l % 32 of the workgroup tile
  float* Hb = H + (int64_t)(i0 + wm + 4 * (l >> 5)) * d + (j0 + wn + (l & 31));
  const bool full = ti != tj && i0 + BT <= d;  // interior tile strictly below the diagonal
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = i0 + wm + x * 32 + mfma32_row(v, l);
        const int j = j0 + wn + y * 32 + (l & 31);
        if (full || (i < d && j <= i))
          atomicAdd(Hb + (int64_t)(x * 32 + 8 * (v >> 2) + (v & 3)) * d + y * 32, acc[x][y][v]);
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

// Row splits for the triangle kernel: one 96 KB-LDS workgroup per CU, so the
// time is about rounds x (stages per split + epilogue); the epilogue's
// atomics cost about 16 stages.
static int pick_splits(int ntiles, int64_t N) {
  int best_s = 1;
  double best = 1e30;
  for (int s = 1; s <= 512; ++s) {
    const int64_t rows = (N + s - 1) / s;
    if (s > 1 && rows < 256) break;
    const double stages = (double)((rows + KS - 1) / KS);
    const double rounds = (double)(((int64_t)ntiles * s + 255) / 256);
    const double cost = rounds * (stages + 16.0);
    if (cost < best - 1e-9) {
      best = cost;
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
    rps = (rps + cp::KS - 1) / cp::KS * cp::KS;
    const int total = ntiles * splits;
    const int per = (total + 7) / 8;
    cp::hess_bf16_tri_kernel<<<dim3(8 * per), cp::HNT, 0, st>>>((const uint16_t*)X, N, (int)d,
                                                                ntiles, splits, rps, H);
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
