// GPTQ-style error feedback (EF) into committed k-quant grids on gfx950
// (coldpress/ef.py:179-218, with _grid_params :87-127 and _repack :130-176).
//
// Data layout in HBM, per tensor (nrow x n weights, columns visited in act order):
//   WpT    [n][nrow] f32  original weights, visiting order, column-major (one
//                         visiting column is one coalesced 4*nrow-byte row)
//   E      [n][nrow] f32  scaled errors e_j of every visited column
//   WcurT  [n][nrow] f32  error-compensated targets at quantization time
//   LT     [n][nrow] u8   stored codes (q - lo) per visited column
//   dlT/mlT [n/sub][nrow] f32  committed grid step / offset per storage sub-block
//
// Sweep (exact mode): one wavefront owns a stripe of 32 rows and walks the
// visiting order in 64-column blocks. Left-looking: before a block is swept,
// each of its elements receives the updates of all earlier columns,
//     t -= e_jj * U[jj][k]   (float32 multiply, then subtract, jj ascending),
// which is exactly the order in which ef.py:213 applies them, so the sweep is
// bit-identical to the reference. The products come from the matrix cores
// (one rounding each), the subtractions from the VALU. E is re-read from L2 /
// HBM by the wave that wrote it, so stripes never synchronize with each other.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

#include "cp_device.h"
#include "cp_host.h"
#include "kq_blocks.h"
#include "phase_clock.h"

namespace cp {


constexpr int BLK = 32;  // columns per sweep block

struct SweepTask {
  const float* WpT;
  const float* U;
  const float* dlT;
  const float* mlT;  // null for the symmetric containers
  const int* sbidx;  // storage sub-block of each visiting column
  float* E;
  float* WcurT;
  uint8_t* LT;
  int nrow, n, lo, hi;
  int first;  // index of the task's first stripe in the row-stripe sweep's item list
};

// Up to kTasksPerLaunch tensors travel by value in the kernel arguments.
constexpr int kTasksPerLaunch = 44;
struct SweepBatch {
  SweepTask t[kTasksPerLaunch];
};
static_assert(sizeof(SweepBatch) <= 4000, "kernel argument block");

// The task table reaches device memory through the kernel arguments of a
// one-block copy kernel (no host staging buffer whose lifetime would have to
// outlast an asynchronous copy).
// status (when not null): the call's status word, cleared before any sweep can set it
__global__ void ef_tasks_store_kernel(const SweepBatch batch, int count, SweepTask* dst, int* status) {
  if ((int)threadIdx.x < count) dst[threadIdx.x] = batch.t[threadIdx.x];
  if (status && threadIdx.x == 0) *status = 0;
}

// Address-space views. U is read-only for the whole sweep and its row
// segments are wave-uniform, so the exact kernel reads it through the constant
// address space (scalar loads into SGPRs); per-lane traffic goes through
// global loads/stores.
typedef const float __attribute__((address_space(4)))* ConstF;
typedef const float __attribute__((address_space(1)))* GlobF;
typedef float __attribute__((address_space(1)))* GlobFw;
typedef uint8_t __attribute__((address_space(1)))* GlobBw;

__device__ __forceinline__ float ld_uniform(const float* p, int64_t i) { return ((ConstF)p)[i]; }
__device__ __forceinline__ float ld_lane(const float* p, int64_t i) { return ((GlobF)p)[i]; }

constexpr int SUBP = 16;  // sub-panel width inside a block

// The block's diagonal U tile, U[i1 + a][i1 + b], staged in LDS.
template <int B>
struct LdsTile {
  const float (*su)[B];
  __device__ __forceinline__ float operator()(int a, int b) const { return su[a][b]; }
};

// In-block part of the sweep for one lane (= one row), shared by the kernels.
// On entry trow[k] (k < B, LDS, stride 1) holds the block's targets after all
// earlier blocks' updates; su(a, b) reads the block's diagonal U tile.
// The block is walked in sub-panels of SUBP columns, left-looking: a
// sub-panel's columns first receive the updates of the block's earlier
// columns (jj ascending), then are quantized and propagated among themselves.
// Every element therefore still sees its updates one at a time in ascending
// jj, as in ef.py:199-213. A consumed target slot trow[c] is reused for e_c.
template <int B, typename Tile>
__device__ __forceinline__ void sweep_block(const SweepTask& tk, int i1, int r, int rr, bool valid,
                                            float* trow, const Tile su) {
  const int nrow = tk.nrow;
#pragma unroll
  for (int s0 = 0; s0 < B; s0 += SUBP) {
    float ts[SUBP];
#pragma unroll
    for (int c = 0; c < SUBP; ++c) ts[c] = trow[s0 + c];
#pragma unroll 1
    for (int jj = 0; jj < s0; ++jj) {
      const float e = trow[jj];
#pragma unroll
      for (int c = 0; c < SUBP; ++c) ts[c] = ts[c] - e * su(jj, s0 + c);
    }
#pragma unroll
    for (int j = 0; j < SUBP; ++j) {
      const int cb = s0 + j, c = i1 + cb;
      const int sb = tk.sbidx[c];
      const float dl = ld_lane(tk.dlT, (int64_t)sb * nrow + rr);
      const float ml = tk.mlT ? ld_lane(tk.mlT, (int64_t)sb * nrow + rr) : 0.0f;
      const bool nz = dl != 0.0f;
      const int q = nz ? clampi(rint_magic((ts[j] + ml) / dl), tk.lo, tk.hi) : 0;
      const float recon = dl * (float)q - ml;
      const float e = nz ? (ts[j] - recon) / su(cb, cb) : 0.0f;
      if (valid) {
        ((GlobFw)tk.E)[(int64_t)c * nrow + r] = e;
        ((GlobFw)tk.WcurT)[(int64_t)c * nrow + r] = ts[j];
        ((GlobBw)tk.LT)[(int64_t)c * nrow + r] = (uint8_t)(q - tk.lo);
      }
      trow[cb] = e;
#pragma unroll
      for (int k = j + 1; k < SUBP; ++k) ts[k] = ts[k] - e * su(cb, s0 + k);
    }
  }
}

// The block's diagonal U tile is kept compact in LDS: a tile row is read only
// by the columns of its 16-column piece onwards, so row cb (piece p = cb / 16)
// holds block columns 16 p .. 63 from tile_base(p) + (cb % 16) * (64 - 16 p):
// 10 KB instead of 16. Within a row the columns are ordered by lane group of
// the row-split sweep (tile_pos), so a group's entries are contiguous.
// sg[k][rl] / sm[k][rl] hold the committed grid step and offset of column k of
// the current quarter block (kGridCols columns) for the stripe's row rl, staged
// in LDS so no global load sits on the column-to-column chain.
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int TILE_FLOATS = 16 * (64 + 48 + 32 + 16);
constexpr int kGridCols = 16;  // block columns per staged part of the grid

__device__ __forceinline__ constexpr int tile_base(int piece) {
  return piece == 0 ? 0 : piece == 1 ? 16 * 64 : piece == 2 ? 16 * (64 + 48) : 16 * (64 + 48 + 32);
}

// Position of block column c (16 p <= c < 64) in a tile row of piece p. In the
// row-split sweep lane group g (of P = 64 / RS) holds columns g, g + P, g + 2P, ...,
// register k holding column P k + g; a row of piece p stores, group after group,
// the registers k >= kp = RS p / 4 (the columns c >= 16 p), so group g's entry
// for register k sits at g (RS - kp) + k - kp.
template <int RS>
__device__ __forceinline__ constexpr int tile_pos(int c, int p) {
  constexpr int P = 64 / RS;
  const int kp = RS * p / 4;
  return (c % P) * (RS - kp) + c / P - kp;
}

// Quantization of one column for one row (ef.py:199-208): code q on the
// committed grid (step dl, offset ml; a zero step gives code 0 and e = 0) and
// the scaled error e = (t - recon) / U[j][j], in the reference's float32 order.
// The divisions run on a safe divisor and are selected away, so there is no
// branch.
__device__ __forceinline__ void quantize_col(const SweepTask& tk, float t, float dl, float ml,
                                             float diag, float& e, int& q) {
  const bool nz = dl != 0.0f;
  const int qv = clampi(rint_magic((t + ml) / (nz ? dl : 1.0f)), tk.lo, tk.hi);
  q = nz ? qv : 0;
  const float recon = dl * (float)q - ml;
  const float ev = (t - recon) / diag;
  e = nz ? ev : 0.0f;
}

// In-block sweep with each row split over the wave: RS rows, P = 64 / RS lanes
// per row, lane l of group g = l / RS holding elements g, g + P, g + 2P, ... of
// row l % RS of the block in registers 0 .. RS - 1 (all 64 lanes work, where
// the one-lane-per-row queue above keeps 64 - RS of them idle). Column cb's
// target is register cb / P of group cb % P; it is broadcast to the row's other
// lanes with v_permlane16/32_swap, every lane quantizes it (the same value, the
// same code and error), and every lane applies the column's update to its
// registers from (cb + 1) / P on, the first register that holds a later column
// in some group. Interleaving the columns over the groups keeps every group's
// remaining columns in the same registers, so a column updates about
// (63 - cb) / P registers per lane, where contiguous column ranges per group
// left the whole register set of the later groups to update. An element
// already quantized that shares a register index with a later one receives
// updates too and is never read again. Each element still receives its
// updates one at a time in ascending column order (ef.py:199-213).
template <int RS>
__device__ __forceinline__ float bcast_group(float x, int own) {
  const unsigned v = __float_as_uint(x);
  if constexpr (RS == 32) {
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(own == 0 ? s[0] : s[1]);
  } else {
    const auto h = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    const unsigned y = (own & 1) ? h[1] : h[0];
    const auto s = __builtin_amdgcn_permlane32_swap(y, y, false, false);
    return __uint_as_float(own < 2 ? s[0] : s[1]);
  }
}

// Columns HB .. HB + kGridCols - 1 (one quarter block; sg / sm hold its grid). tile is
// the compact diagonal tile; row cb holds columns 16 * (cb / 16) .. 63. HB is a
// template argument so every column's lane group and register are compile-time.
template <int RS, int HB>
__device__ __forceinline__ void sweep_part_split(const SweepTask& tk, int i1, int rr, int rl, int g,
                                                 float (&tl)[RS], const float* tile,
                                                 const float (*sg)[RS], const float (*sm)[RS]) {
  constexpr int hb = HB;
  const int nrow = tk.nrow;
  // Running output pointers (row rr, column i1 + hb + a), opaque to the
  // compiler so the unrolled columns do not each keep a precomputed address.
  // Every lane stores: the lanes of a row hold the same values, and a lane past
  // the last row (rr = nrow - 1) computed exactly that row's values from that
  // row's data, so duplicate stores write identical bytes; a branch around the
  // stores would split the unrolled columns into blocks the per-column
  // scheduling fences cannot hold together.
  const int64_t o0 = (int64_t)(i1 + hb) * nrow + rr;
  float* pe = tk.E + o0;
  float* pw = tk.WcurT + o0;
  uint8_t* pl = tk.LT + o0;
  // Column cb's LDS operands (grid step and offset of the row, the diagonal entry and
  // the lane's part of tile row cb) do not depend on the column chain. They are read
  // one column ahead, so no LDS round trip sits between one column's error and the
  // next column's quantization.
  struct ColOps {
    float dl, ml, diag;
    f32x4 u[RS / 4];
  };
  // Column cb updates registers jlo_of(cb) .. RS - 1: from (cb + 1) / P, the first
  // register holding a later column in some group, rounded down to a float4 of the
  // tile row (never below kp, the row's first stored register).
  constexpr int P = 64 / RS;
  const auto jlo_of = [](int cb) { return ((cb + 1) / P) & ~3; };
  const auto read_ops = [&](int a, ColOps& c) {
    const int cb = hb + a, p = cb / 16, kp = RS * p / 4;
    const float* row = tile + tile_base(p) + (cb % 16) * (64 - 16 * p);
    c.dl = sg[a][rl];
    c.ml = sm[a][rl];
    c.diag = row[tile_pos<RS>(cb, p)];
    // the group's entry of register k is ul[k / 4] component k % 4 (k >= kp). The
    // address is formed in 4-float units (the row start, kp and RS - kp are multiples
    // of 4 floats) and read as a native 4-vector (HIP's float4 struct is copied element
    // by element, which left two-dword reads and an address add per pair), so each read
    // is one 16-byte LDS load with an immediate offset.
    const f32x4* ul = reinterpret_cast<const f32x4*>(__builtin_assume_aligned(tile, 16)) +
                      (tile_base(p) + (cb % 16) * (64 - 16 * p) - kp) / 4 + g * ((RS - kp) / 4);
    const int jlo = jlo_of(cb);
#pragma unroll
    for (int j4 = 0; j4 < RS / 4; ++j4)
      if (4 * j4 >= jlo) c.u[j4] = ul[j4];  // constant once the column loop is unrolled
  };
  // Column cb's update of register k of every lane group, t = fl(t - fl(e * u)).
  const auto apply = [&](float e, const ColOps& c, int k) {
    const f32x4 u = c.u[k / 4];
    const float uk = (k % 4 == 0) ? u.x : (k % 4 == 1) ? u.y : (k % 4 == 2) ? u.z : u.w;
    tl[k] = tl[k] - e * uk;
  };
  // The updates of a column are split in two. The register holding the next column's
  // target (index (cb + 1) / P in every lane group) takes column cb's update at once,
  // so the next quantization can start; the other registers take it in the next
  // column's scheduling region, where those independent subtractions fill the latency
  // of that column's divisions. Each register still receives the columns' updates in
  // ascending order, each exactly once; registers of finished columns take updates
  // that are never read.
  ColOps ops[3];
  read_ops(0, ops[0]);
  float e_prev = 0.0f;
#pragma unroll
  for (int a = 0; a < kGridCols; ++a) {
    const int cb = hb + a;
    const int own = cb % P, i = cb / P;
    ColOps& cur = ops[a % 3];
    if (a + 1 < kGridCols) read_ops(a + 1, ops[(a + 1) % 3]);
    if (a > 0) {  // column cb - 1's remaining updates; register i took it already
      const ColOps& prev = ops[(a + 2) % 3];
      const int jlo = jlo_of(cb - 1);
#pragma unroll
      for (int k = 0; k < RS; ++k)
        if (k >= jlo && k != i) apply(e_prev, prev, k);  // constant once unrolled
    }
    const float tb = bcast_group<RS>(tl[i], own);
    float e;
    int q;
    quantize_col(tk, tb, cur.dl, cur.ml, cur.diag, e, q);
    *(GlobFw)pe = e;
    *(GlobFw)pw = tb;
    *(GlobBw)pl = (uint8_t)(q - tk.lo);
    pe += nrow;
    pw += nrow;
    pl += nrow;
    asm volatile("" : "+v"(pe), "+v"(pw), "+v"(pl));
    if (cb + 1 < 64) apply(e, cur, (cb + 1) / P);  // the next column's target first
    e_prev = e;
    // one column's region at a time; the next column's operands are already in flight
    __builtin_amdgcn_sched_barrier(0);
  }
  {  // the part's last column: its remaining updates before the next part's grid
    const int cb = hb + kGridCols - 1;
    const ColOps& last = ops[(kGridCols - 1) % 3];
    const int jlo = jlo_of(cb), nx = (cb + 1) / P;
#pragma unroll
    for (int k = 0; k < RS; ++k)
      if (k >= jlo && (cb + 1 >= 64 || k != nx)) apply(e_prev, last, k);
  }
}

// The committed grid step / offset of block columns hb .. hb + kGridCols - 1 for
// the stripe's rows: lane l covers row l % RS and every (64 / RS)-th column.
// load_grid issues the loads into registers, store_grid writes them to sg /
// sm. sbo[k] = (storage sub-block of block column k) * nrow.
template <int RS>
struct GridPart {
  static constexpr int P = 64 / RS, NC = kGridCols / P;
  float d[NC], m[NC];
};

template <int RS>
__device__ __forceinline__ void load_grid(const SweepTask& tk, const int* sbo, int hb, int l, int rr,
                                          GridPart<RS>& g) {
  constexpr int P = GridPart<RS>::P, NC = GridPart<RS>::NC;
  const int part = l / RS;
#pragma unroll
  for (int k = 0; k < NC; ++k) g.d[k] = ld_lane(tk.dlT, (int64_t)sbo[hb + part + P * k] + rr);
  if (tk.mlT) {
#pragma unroll
    for (int k = 0; k < NC; ++k) g.m[k] = ld_lane(tk.mlT, (int64_t)sbo[hb + part + P * k] + rr);
  } else {
#pragma unroll
    for (int k = 0; k < NC; ++k) g.m[k] = 0.0f;
  }
}

template <int RS>
__device__ __forceinline__ void store_grid(const GridPart<RS>& g, int l, float (*sg)[RS], float (*sm)[RS]) {
  constexpr int P = GridPart<RS>::P, NC = GridPart<RS>::NC;
  const int rl = l % RS, part = l / RS;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    sg[part + P * k][rl] = g.d[k];
    sm[part + P * k][rl] = g.m[k];
  }
}

// The block's four quarter blocks in order: each stages its grid in LDS, then sweeps
// its 16 columns. sync orders the LDS writes against the reads (a wave barrier when
// the LDS is the wave's own, a workgroup barrier otherwise).
template <int RS, class Sync>
__device__ __forceinline__ void sweep_quarters(const SweepTask& tk, int i1, int rr, int l,
                                               float (&tl)[RS], const float* tile,
                                               const GridPart<RS> (&gp)[64 / kGridCols],
                                               float (*sg)[RS], float (*sm)[RS], Sync sync) {
  static_assert(64 / kGridCols == 4, "four quarter blocks");
  const int rl = l % RS, part = l / RS;
  store_grid<RS>(gp[0], l, sg, sm);
  sync();
  sweep_part_split<RS, 0>(tk, i1, rr, rl, part, tl, tile, sg, sm);
  sync();
  store_grid<RS>(gp[1], l, sg, sm);
  sync();
  sweep_part_split<RS, kGridCols>(tk, i1, rr, rl, part, tl, tile, sg, sm);
  sync();
  store_grid<RS>(gp[2], l, sg, sm);
  sync();
  sweep_part_split<RS, 2 * kGridCols>(tk, i1, rr, rl, part, tl, tile, sg, sm);
  sync();
  store_grid<RS>(gp[3], l, sg, sm);
  sync();
  sweep_part_split<RS, 3 * kGridCols>(tk, i1, rr, rl, part, tl, tile, sg, sm);
  sync();
}

template <int B>
__device__ __forceinline__ void load_diag_tile(const SweepTask& tk, int i1, int lane, int nthreads,
                                               float (*su)[B]) {
  for (int idx = lane; idx < B * B; idx += nthreads)
    su[idx / B][idx % B] = ld_lane(tk.U, (int64_t)(i1 + idx / B) * tk.n + i1 + idx % B);
}

// Exact mode on the VALU only (cross-check of the MFMA-product kernel).
// Grid: x = groups of 4 stripes (256 rows), y = task. Cross-block
// updates in the reference's order: t -= e_jj * U[jj][k], jj ascending, one
// float32 multiply and one subtract each, U row segments via scalar loads.
template <int B>
__global__ __launch_bounds__(256, 2) void ef_sweep_exact_kernel(const SweepTask* __restrict__ tasks) {
  const SweepTask tk = tasks[blockIdx.y];
  if ((int)(blockIdx.x * 256) >= tk.nrow) return;
  const int r = blockIdx.x * 256 + threadIdx.x;
  const int nrow = tk.nrow, n = tk.n;
  const bool valid = r < nrow;
  const int rr = valid ? r : nrow - 1;
  __shared__ float su[B][B];
  __shared__ float st[256][B + 1];
  float* trow = st[threadIdx.x];
  for (int i1 = 0; i1 < n; i1 += B) {
    float t[B];
#pragma unroll
    for (int k = 0; k < B; ++k) t[k] = ld_lane(tk.WpT, (int64_t)(i1 + k) * nrow + rr);
    for (int jj = 0; jj < i1; ++jj) {
      const float e = ld_lane(tk.E, (int64_t)jj * nrow + rr);
      const int64_t ub = (int64_t)jj * n + i1;
#pragma unroll
      for (int k = 0; k < B; ++k) t[k] = t[k] - e * ld_uniform(tk.U, ub + k);
    }
#pragma unroll
    for (int k = 0; k < B; ++k) trow[k] = t[k];
    __syncthreads();
    load_diag_tile<B>(tk, i1, threadIdx.x, 256, su);
    __syncthreads();
    sweep_block<B>(tk, i1, r, rr, valid, trow, LdsTile<B>{su});
  }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

// Row of the 32x32 MFMA result held by register v of lane l (column = l % 32).
__device__ __forceinline__ int mfma32_row(int v, int l) { return 8 * (v >> 2) + 4 * (l >> 5) + (v & 3); }

// Exact mode on the matrix cores: one wave per stripe of RS rows (32 or 16),
// 64-column blocks. A stripe's cross-block work is a sequential chain (every
// column of a row depends on all earlier ones), so the stripe height sets the
// chain each wave carries; 16-row stripes halve it for calls whose 32-row
// stripes would not give every SIMD two waves. For every earlier column jj one
// MFMA with k = 1 forms the RS x 64 products e_jj (x) U[jj][block]:
// v_mfma_f32_32x32x1_2b_f32 (blocks = column halves) for RS = 32,
// v_mfma_f32_16x16x1_4b_f32 (blocks = column quarters) for RS = 16, both with
// the inline-zero accumulator, so each product is rounded once to float32; the
// VALU subtracts them in jj order. The products for jj + 1 are formed while
// those for jj are subtracted; E and U for the next 8 columns are loaded while
// the current 8 are applied. The in-block sweep runs on lanes 0..RS-1 (lane =
// row) with the block's diagonal U tile in LDS.
template <int RS>
struct StripeLayout;
template <>
struct StripeLayout<32> {  // register v of lane l -> (row, column) of the stripe's block
  static constexpr int NV = 32;
  __device__ static int row(int v, int l) { return mfma32_row(v & 15, l); }
  __device__ static int col(int v, int l) { return 32 * (v >> 4) + (l & 31); }
};
template <>
struct StripeLayout<16> {
  static constexpr int NV = 16;
  __device__ static int row(int v, int l) { return 4 * (l >> 4) + (v & 3); }
  __device__ static int col(int v, int l) { return 16 * (v >> 2) + (l & 15); }
};

// Items are the stripes of every task, task by task (tasks[k].first is the
// first item of task k). With xcd_runs set (every task of the call has the same
// n, so items are equally long), each XCD takes one contiguous run of items:
// workgroup w runs on XCD w % 8, so item = (w % 8) * per + w / 8. The stripes
// resident on an XCD then belong to a few tensors -- tensors sharing one H share
// one U -- and read the same strips of U through that XCD's L2 instead of every
// XCD's L2 holding strips of every tensor. Otherwise item = w, in the table's
// longest-first order.
__device__ __forceinline__ int sweep_item(const SweepTask* tasks, int count, int total, bool xcd_runs,
                                          int* task) {
  const int w = (int)blockIdx.x;
  int item = w;
  if (xcd_runs) {
    const int per = (total + 7) / 8;
    item = (w % 8) * per + w / 8;
  }
  if (item >= total) return -1;
  int lo = 0, hi = count - 1;  // last task with first <= item
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (tasks[mid].first <= item)
      lo = mid;
    else
      hi = mid - 1;
  }
  *task = lo;
  return item - tasks[lo].first;
}

// Per-wave LDS of the row-stripe sweep, about 14.6 KB: one buffer for the RS x 64
// target transpose and then the compact diagonal U tile, the storage sub-block offsets
// of the block's columns, and the grid steps / offsets of a quarter block.
struct StripeLds {
  float tile[TILE_FLOATS];
  int sbo[64];
  float sg[kGridCols][32], sm[kGridCols][32];
};

// LDS ordering between the lanes of one wave (each wave has its own StripeLds).
struct WaveSync {
  __device__ __forceinline__ void operator()() const {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }
};

template <int RS>
using StripeVec = float __attribute__((ext_vector_type(StripeLayout<RS>::NV)));

// One k = 1 outer product e (x) u on the matrix cores with the inline-zero accumulator:
// every product rounded once to float32, as np.outer forms it.
template <int RS>
__device__ __forceinline__ StripeVec<RS> stripe_product(float a, float b) {
  const StripeVec<RS> z = {};
  if constexpr (RS == 32)
    return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, z, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, z, 0, 0, 0);
}

// The block's original targets (visiting order) in the MFMA layout, and the storage
// sub-block offsets of its columns: lane l stages row rl, columns part * CPP .. + CPP - 1.
template <int RS>
__device__ __forceinline__ StripeVec<RS> stage_block(const SweepTask& tk, int i1, int rr, int l,
                                                     StripeLds& s) {
  constexpr int B = 64, NV = StripeLayout<RS>::NV, CPP = B * RS / 64;
  const int rl = l % RS, part = l / RS, nrow = tk.nrow;
  float (*st)[B + 1] = reinterpret_cast<float (*)[B + 1]>(s.tile);
  s.sbo[l] = tk.sbidx[i1 + l] * nrow;
#pragma unroll
  for (int k = 0; k < CPP; ++k)
    st[rl][part * CPP + k] = ld_lane(tk.WpT, (int64_t)(i1 + part * CPP + k) * nrow + rr);
  WaveSync()();
  StripeVec<RS> t;
#pragma unroll
  for (int v = 0; v < NV; ++v) t[v] = st[StripeLayout<RS>::row(v, l)][StripeLayout<RS>::col(v, l)];
  return t;
}

// Cross-block updates of the block at i1 from visiting columns j0 .. j1 - 1 (multiples of
// 64), in ascending column order: t = fl(t - fl(e_jj * U[jj][c])). E and U come in
// groups of G columns through a ring of 16 / G static register buffers, each group
// loaded 16 / G - 1 groups ahead (16 - G columns before its first use; the ring holds 16
// columns of E and U whatever G); per column, the MFMA for the next column is issued
// before the subtractions that consume the current one, fenced by scheduling barriers so
// the two products stay in separate registers and each MFMA runs under the VALU work of
// the column before it.
constexpr int kSweepGroup = 8;  // cross-block columns per E / U load group

template <int RS, int G = kSweepGroup>
__device__ __forceinline__ void cross_range(const SweepTask& tk, int i1, int rr, int l,
                                            StripeVec<RS>& t, int j0, int j1) {
  constexpr int NB = 16 / G, NV = StripeLayout<RS>::NV;
  static_assert(G * NB == 16 && G % 2 == 0, "16 columns in flight, columns in pairs");
  const int nrow = tk.nrow, n = tk.n;
  float e[NB][G], u[NB][G];
  // buffer loads rebased per group: the lane's byte offset stays in a VGPR and the
  // column's offset is scalar, so no per-lane address arithmetic runs per column
  const int eoff = 4 * rr, uoff = 4 * l;
  auto load = [&](int g, float (&eg)[G], float (&ug)[G]) {
    const int jg = j0 + g * G;
    const auto re = __builtin_amdgcn_make_buffer_rsrc((void*)(tk.E + (int64_t)jg * nrow), 0,
                                                      0x7fffffff, 0x00020000);
    const auto ru = __builtin_amdgcn_make_buffer_rsrc((void*)(tk.U + (int64_t)jg * n + i1), 0,
                                                      0x7fffffff, 0x00020000);
#pragma unroll
    for (int q = 0; q < G; ++q) {
      eg[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(re, eoff, 4 * q * nrow, 0));
      ug[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ru, uoff, 4 * q * n, 0));
    }
  };
  StripeVec<RS> P0, P1;
  auto group = [&](const float (&eg)[G], const float (&ug)[G], const float (&en)[G],
                   const float (&un)[G]) {
#pragma unroll
    for (int q = 0; q < G; q += 2) {
      // P0 holds column q of the group on entry; the last group's final product is unused
      P1 = stripe_product<RS>(eg[q + 1], ug[q + 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < NV; ++v) t[v] = t[v] - P0[v];
      __builtin_amdgcn_sched_barrier(0);
      P0 = stripe_product<RS>(q + 2 < G ? eg[q + 2] : en[0], q + 2 < G ? ug[q + 2] : un[0]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < NV; ++v) t[v] = t[v] - P1[v];
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const int groups = (j1 - j0) / G;  // a multiple of NB: j1 - j0 is a multiple of 64
  // past the end: a valid group, loaded and unused
  const auto clampg = [groups](int h) { return h < groups ? h : groups - 1; };
#pragma unroll
  for (int b = 0; b + 1 < NB; ++b) load(clampg(b), e[b], u[b]);
  P0 = stripe_product<RS>(e[0][0], u[0][0]);
  for (int g = 0; g < groups; g += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      // the buffer group b - 1 has just consumed takes group g + b + NB - 1 (for b = 0 the
      // last group of this window, always valid: groups is a multiple of NB)
      const int h = g + b + NB - 1;
      load(b == 0 ? h : clampg(h), e[(b + NB - 1) % NB], u[(b + NB - 1) % NB]);
      group(e[b], u[b], e[(b + 1) % NB], u[(b + 1) % NB]);
    }
  }
}

// The block's own 64 columns for the stripe's rows, after every earlier column's
// updates: the targets move to the row-split layout (lane l: elements l / RS,
// l / RS + P, ... of row l % RS, P = 64 / RS), the compact diagonal tile and the block's committed grid
// come in through one round trip, and the four quarter blocks are swept in order.
template <int RS>
__device__ __forceinline__ void sweep_block_rows(const SweepTask& tk, int i1, int rr, int l,
                                                 const StripeVec<RS>& t, StripeLds& s) {
  constexpr int B = 64, NV = StripeLayout<RS>::NV;
  static_assert(RS * (B + 1) <= TILE_FLOATS, "target transpose fits the tile buffer");
  const int rl = l % RS, part = l / RS, n = tk.n;
  float (*st)[B + 1] = reinterpret_cast<float (*)[B + 1]>(s.tile);
  float (*sg)[RS] = reinterpret_cast<float (*)[RS]>(&s.sg[0][0]);
  float (*sm)[RS] = reinterpret_cast<float (*)[RS]>(&s.sm[0][0]);
  WaveSync()();
#pragma unroll
  for (int v = 0; v < NV; ++v) st[StripeLayout<RS>::row(v, l)][StripeLayout<RS>::col(v, l)] = t[v];
  WaveSync()();
  float tl[RS];
#pragma unroll
  for (int k = 0; k < RS; ++k) tl[k] = st[rl][(64 / RS) * k + part];
  WaveSync()();
  // the block's grid steps / offsets (both halves into registers) and the compact
  // diagonal tile share one round trip to memory; lane l fills column 16 p + l of the
  // tile rows of piece p
  GridPart<RS> gp[64 / kGridCols];
#pragma unroll
  for (int q = 0; q < 64 / kGridCols; ++q) load_grid<RS>(tk, s.sbo, q * kGridCols, l, rr, gp[q]);
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float u[16];
    const bool in = l < 64 - 16 * p;
#pragma unroll
    for (int a = 0; a < 16; ++a)
      u[a] = in ? ld_lane(tk.U, (int64_t)(i1 + 16 * p + a) * n + i1 + 16 * p + l) : 0.0f;
    if (in) {
#pragma unroll
      for (int a = 0; a < 16; ++a) s.tile[tile_base(p) + a * (64 - 16 * p) + tile_pos<RS>(16 * p + l, p)] = u[a];
    }
  }
  sweep_quarters<RS>(tk, i1, rr, l, tl, s.tile, gp, sg, sm, WaveSync());
}

template <int RS>
__global__ __launch_bounds__(64, 2) void ef_sweep_rows_kernel(const SweepTask* __restrict__ tasks, int count,
                                                            int total, int xcd_runs) {
  constexpr int B = 64, NV = StripeLayout<RS>::NV, CPP = B * RS / 64;
  int ti;
  const int stripe = sweep_item(tasks, count, total, xcd_runs != 0, &ti);
  if (stripe < 0) return;
  const SweepTask tk = tasks[ti];
  const int row0 = stripe * RS;
  if (row0 >= tk.nrow) return;
  const int l = threadIdx.x, rl = l % RS, part = l / RS;
  const int nrow = tk.nrow, n = tk.n;
  // lanes past the last row work on the last row (and store its values again)
  const int rr = row0 + rl < nrow ? row0 + rl : nrow - 1;
  // one LDS buffer: the RS x 64 target transpose, then the compact diagonal
  // U tile; the grid steps / offsets of a quarter block. About 14.5 KB in all,
  // so eight of these one-wave workgroups leave 44 KB of a CU's LDS free for a
  // concurrent stream's workgroups (the factorization's GEMM and diagonal-block
  // kernels need 34-37 KB), instead of the 10 KB a half-block staging left.
  // Occupancy: the RS = 32 variant holds two waves per SIMD (228 registers, v175
  // reserved as it always was); the RS = 16 variant (141) runs up to ten waves per CU,
  // the LDS limit, so a call with a few more 16-row stripes than two per SIMD (the
  // Llama-3-8B layer's 2432) still runs them in one round.
  if constexpr (RS == 32) asm volatile("" ::: "v175");
  static_assert(RS * (B + 1) <= TILE_FLOATS, "target transpose fits the tile buffer");
  __shared__ __align__(16) float lds[TILE_FLOATS];
  __shared__ int sbo[B];
  __shared__ float sg_[kGridCols][32], sm_[kGridCols][32];
  float (*sg)[RS] = reinterpret_cast<float (*)[RS]>(&sg_[0][0]);
  float (*sm)[RS] = reinterpret_cast<float (*)[RS]>(&sm_[0][0]);
  float (*st)[B + 1] = reinterpret_cast<float (*)[B + 1]>(lds);
  float* trow = st[rl];
  for (int i1 = 0; i1 < n; i1 += B) {
    // targets: lane l stages row rl, columns part * CPP .. + CPP - 1, then
    // moves to the MFMA layout
    sbo[l] = tk.sbidx[i1 + l] * nrow;
#pragma unroll
    for (int k = 0; k < CPP; ++k)
      trow[part * CPP + k] = ld_lane(tk.WpT, (int64_t)(i1 + part * CPP + k) * nrow + rr);
    __syncthreads();
    StripeVec<RS> t;
#pragma unroll
    for (int v = 0; v < NV; ++v) t[v] = st[StripeLayout<RS>::row(v, l)][StripeLayout<RS>::col(v, l)];
    if (i1 > 0) cross_range<RS>(tk, i1, rr, l, t, 0, i1);
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NV; ++v) st[StripeLayout<RS>::row(v, l)][StripeLayout<RS>::col(v, l)] = t[v];
    __syncthreads();
    // lane l: elements l / RS, l / RS + P, ... of row l % RS (P = 64 / RS)
    float tl[RS];
#pragma unroll
    for (int k = 0; k < RS; ++k) tl[k] = trow[(64 / RS) * k + part];
    __syncthreads();
    // the block's grid steps / offsets (both halves into registers) and the
    // compact diagonal tile share one round trip to memory; lane l fills
    // column 16 p + l of the tile rows of piece p
    GridPart<RS> gp[64 / kGridCols];
#pragma unroll
    for (int q = 0; q < 64 / kGridCols; ++q) load_grid<RS>(tk, sbo, q * kGridCols, l, rr, gp[q]);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float u[16];
      const bool in = l < 64 - 16 * p;
#pragma unroll
      for (int a = 0; a < 16; ++a)
        u[a] = in ? ld_lane(tk.U, (int64_t)(i1 + 16 * p + a) * n + i1 + 16 * p + l) : 0.0f;
      if (in) {
#pragma unroll
        for (int a = 0; a < 16; ++a) lds[tile_base(p) + a * (64 - 16 * p) + tile_pos<RS>(16 * p + l, p)] = u[a];
      }
    }
    sweep_quarters<RS>(tk, i1, rr, l, tl, lds, gp, sg, sm, [] { __syncthreads(); });
  }
}

// Wait (bounded) until *done > c, the count of the stripe's blocks complete so far, and
// return that count. The producing wave releases the count at workgroup scope after
// its error stores, so the acquire here orders this wave's later reads of those errors.
// The bound is ``limit`` sleeps of s_sleep 8 (about 512 clocks each): the default
// 2^16 is about 14 ms at 2.4 GHz, far above any wait the schedule makes (one block's
// sweep). Past it the wave sets bit 0 of the call's status word (read by the host,
// which then rejects the call's bytes) and goes on with one more block rather than
// spin for ever, so every wave still ends.
__device__ __forceinline__ int wait_blocks(int* done, int c, int limit, int* status, int lane) {
  int v = __hip_atomic_load(done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
  for (int spins = 0; v <= c && spins < limit; ++spins) {
    __builtin_amdgcn_s_sleep(8);
    v = __hip_atomic_load(done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  v = __builtin_amdgcn_readfirstlane(v);
  if (v <= c) {
    if (lane == 0) __hip_atomic_fetch_or(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return c + 1;
  }
  return v;
}

// W waves per stripe, for calls whose stripes alone would leave most SIMDs idle (few
// rows, long rows). Wave w owns blocks w, w + W, w + 2W, ... For each of its blocks a
// wave applies the updates of every earlier block's columns in ascending order, taking
// at each step all the leading blocks that are complete, and waits only when the next
// block it needs is still being swept; then it sweeps its own block and publishes the
// new count of complete blocks. Blocks complete in order (block b is swept only after
// blocks 0 .. b - 1 are applied to it), so one counter in LDS describes them, and every
// wait ends: block c depends only on blocks below c. Every element still receives its
// updates one at a time in ascending column order, as in the one-wave kernel. The
// errors a wave writes reach the others through global memory, ordered by the
// counter's release and acquire.
template <int RS, int W>
__global__ __launch_bounds__(64 * W, 2) void ef_sweep_pipe_kernel(const SweepTask* __restrict__ tasks,
                                                                  int count, int total, int xcd_runs,
                                                                  int wait_limit, int* status) {
  int ti;
  const int stripe = sweep_item(tasks, count, total, xcd_runs != 0, &ti);
  if (stripe < 0) return;  // uniform over the workgroup
  const SweepTask tk = tasks[ti];
  const int row0 = stripe * RS;
  if (row0 >= tk.nrow) return;
  const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x / 64);
  const int l = threadIdx.x % 64, rl = l % RS;
  const int rr = row0 + rl < tk.nrow ? row0 + rl : tk.nrow - 1;
  __shared__ __align__(16) StripeLds s_all[W];
  __shared__ int done;  // the stripe's blocks complete so far
  StripeLds& s = s_all[wv];
  if (threadIdx.x == 0) done = 0;
  __syncthreads();
  const int nblocks = tk.n / 64;
  for (int b = wv; b < nblocks; b += W) {
    const int i1 = b * 64;
    StripeVec<RS> t = stage_block<RS>(tk, i1, rr, l, s);
    for (int c = 0; c < b;) {
      const int avail = min(wait_blocks(&done, c, wait_limit, status, l), b);
      cross_range<RS>(tk, i1, rr, l, t, c * 64, avail * 64);
      c = avail;
    }
    sweep_block_rows<RS>(tk, i1, rr, l, t, s);
    // a maximum, not a store: after a wait gave up, a late wave must not move the count back
    __hip_atomic_fetch_max(&done, b + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// MFMA mode. One wave per 64-row stripe (grid: x = stripe, y = task).
// Cross-block updates of a block are one GEMM, acc[64 x B] = E[64 x i1] *
// U[i1 x B], on v_mfma_f32_32x32x2f32 (A = E from the column-major error
// buffer, B = U rows, both coalesced, prefetched one 8-column group ahead);
// the targets are then x - acc (one float32 subtraction of the float32-
// accumulated sum), and the block itself is swept exactly as in exact mode.
template <int B>
__global__ __launch_bounds__(64, 2) void ef_sweep_mfma_kernel(const SweepTask* __restrict__ tasks) {
  static_assert(B == 32, "one 32-wide MFMA column tile per block");
  const SweepTask tk = tasks[blockIdx.y];
  const int row0 = blockIdx.x * 64;
  if (row0 >= tk.nrow) return;
  const int l = threadIdx.x;
  const int nrow = tk.nrow, n = tk.n;
  const int r = row0 + l;
  const bool valid = r < nrow;
  const int rr = valid ? r : nrow - 1;
  __shared__ float su[B][B];
  __shared__ float st[64][B + 1];
  float* trow = st[l];
  const int kl = l >> 5, cl = l & 31;
  const int ra0 = min(row0 + cl, nrow - 1), ra1 = min(row0 + 32 + cl, nrow - 1);
  for (int i1 = 0; i1 < n; i1 += B) {
    f32x16 acc0, acc1;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc0[v] = 0.0f;
      acc1[v] = 0.0f;
    }
    // jj in groups of 8 (4 MFMA k-steps), next group's operands loaded ahead
    float a0[4], a1[4], b[4], na0[4], na1[4], nb[4];
    const int groups = i1 / 8;
    auto load = [&](int g, float (&x0)[4], float (&x1)[4], float (&y)[4]) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int64_t jj = (int64_t)g * 8 + 2 * s + kl;
        x0[s] = ld_lane(tk.E, jj * nrow + ra0);
        x1[s] = ld_lane(tk.E, jj * nrow + ra1);
        y[s] = ld_lane(tk.U, jj * n + i1 + cl);
      }
    };
    if (groups > 0) load(0, a0, a1, b);
    for (int g = 0; g < groups; ++g) {
      if (g + 1 < groups) load(g + 1, na0, na1, nb);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[s], b[s], acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[s], b[s], acc1, 0, 0, 0);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        a0[s] = na0[s];
        a1[s] = na1[s];
        b[s] = nb[s];
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      st[mfma32_row(v, l)][cl] = acc0[v];
      st[32 + mfma32_row(v, l)][cl] = acc1[v];
    }
    load_diag_tile<B>(tk, i1, l, 64, su);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < B; ++k) trow[k] = ld_lane(tk.WpT, (int64_t)(i1 + k) * nrow + rr) - trow[k];
    sweep_block<B>(tk, i1, r, rr, valid, trow, LdsTile<B>{su});
    __syncthreads();
  }
}

// ---------------------------------------------------------------- many-tensor kernels
// Every step outside the sweep runs as one launch over all tensors of a call
// (blockIdx.y or .z = row of the tensor table; blocks past a tensor's extent
// exit), so a call costs a few dozen launches instead of a dozen per tensor.

// Per-tensor device descriptor (the workspace views plus the caller's buffers).
struct EfDev {
  const float* x;
  const float* qw;
  const int* order;
  uint8_t* raw;
  float* recon;
  float* WpT;
  float* WcurT;
  float* Wcur;
  uint8_t* LT;
  float* dlT;
  float* mlT;
  int* inv;
  int* sbidx;
  int nrow, n, ttype, sub;
};

constexpr int kDevPerStore = 24;
struct EfDevBatch {
  EfDev t[kDevPerStore];
};
static_assert(sizeof(EfDevBatch) <= 4000, "kernel argument block");

__global__ void ef_dev_store_kernel(const EfDevBatch batch, int count, EfDev* dst) {
  if ((int)threadIdx.x < count) dst[threadIdx.x] = batch.t[threadIdx.x];
}

// inv[order[jj]] = jj and sbidx[jj] = order[jj] / sub. An order that is not a
// permutation writes no entry out of range (sbidx of an out-of-range entry is 0), and
// the readers of inv take its entries into [0, n), so unwritten ones stay harmless.
__global__ void ef_index_kernel(const EfDev* __restrict__ tab) {
  const EfDev& t = tab[blockIdx.y];
  const int jj = blockIdx.x * blockDim.x + threadIdx.x;
  if (jj >= t.n) return;
  const int c = t.order[jj];
  if ((unsigned)c >= (unsigned)t.n) {
    t.sbidx[jj] = 0;
    return;
  }
  t.inv[c] = jj;
  t.sbidx[jj] = c / t.sub;
}

// dst[inv[c]][r] = src[r][c] (row-major storage order -> column-major visiting
// order) or its inverse, through a 64x64 LDS tile (coalesced on both sides).
// WHICH: 0 = x -> WpT, 2 = WcurT -> Wcur.
template <int WHICH>
__global__ __launch_bounds__(256) void ef_transpose_kernel(const EfDev* __restrict__ tab) {
  static_assert(WHICH == 0 || WHICH == 2, "float transposes only");
  typedef float T;
  const EfDev& t = tab[blockIdx.z];
  const int nrow = t.nrow, n = t.n;
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  if (c0 >= n || r0 >= nrow) return;
  __shared__ T tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int* __restrict__ inv = t.inv;
  const T* vsrc = WHICH == 0 ? (const T*)t.x : (const T*)t.WcurT;
  const T* vdst = WHICH == 0 ? (const T*)t.WpT : (const T*)t.Wcur;
  const bool vec = (nrow % 4) == 0 && (n % 4) == 0 &&
                   ((reinterpret_cast<uintptr_t>(vsrc) | reinterpret_cast<uintptr_t>(vdst)) & 15) == 0;
  if (vec) {
    // 16-byte accesses on both sides: lane l holds 4 consecutive entries of one tile
    // row (storage side: 4 columns of row r; visiting side: 4 rows of column v).
    // Rows and columns are multiples of 4, so a quad is wholly inside or outside.
    const int q = threadIdx.x & 15, g = threadIdx.x >> 4;  // quad within a line, line
    if (WHICH == 0) {  // storage [nrow][n] -> visiting [n][nrow]
      const float4* src = reinterpret_cast<const float4*>(t.x);
      float4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = r0 + g + 16 * k, c = c0 + 4 * q;
        v[k] = (r < nrow && c < n) ? src[((int64_t)r * n + c) / 4] : make_float4(0, 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = g + 16 * k;
        tile[i][4 * q] = v[k].x;
        tile[i][4 * q + 1] = v[k].y;
        tile[i][4 * q + 2] = v[k].z;
        tile[i][4 * q + 3] = v[k].w;
      }
      __syncthreads();
      float4* dst = reinterpret_cast<float4*>(t.WpT);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = g + 16 * k, c = c0 + j, r = r0 + 4 * q;
        const int vv = c < n ? inv[c] : -1;
        if (r < nrow && (unsigned)vv < (unsigned)n)
          dst[((int64_t)vv * nrow + r) / 4] =
              make_float4(tile[4 * q][j], tile[4 * q + 1][j], tile[4 * q + 2][j], tile[4 * q + 3][j]);
      }
    } else {  // visiting [n][nrow] -> storage [nrow][n]
      const float4* src = reinterpret_cast<const float4*>(t.WcurT);
      float4 v[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = g + 16 * k, c = c0 + j, r = r0 + 4 * q;
        const int vv = c < n ? inv[c] : -1;
        v[k] = (r < nrow && (unsigned)vv < (unsigned)n) ? src[((int64_t)vv * nrow + r) / 4]
                                                         : make_float4(0, 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = g + 16 * k;
        tile[4 * q][j] = v[k].x;
        tile[4 * q + 1][j] = v[k].y;
        tile[4 * q + 2][j] = v[k].z;
        tile[4 * q + 3][j] = v[k].w;
      }
      __syncthreads();
      float4* dst = reinterpret_cast<float4*>(t.Wcur);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = r0 + g + 16 * k, c = c0 + 4 * q;
        const int i = g + 16 * k;
        if (r < nrow && c < n)
          dst[((int64_t)r * n + c) / 4] =
              make_float4(tile[i][4 * q], tile[i][4 * q + 1], tile[i][4 * q + 2], tile[i][4 * q + 3]);
      }
    }
    return;
  }
  if (WHICH == 0) {  // storage -> visiting
    const float* src = t.x;
    float* dst = t.WpT;
    for (int i = ty; i < 64; i += 4) {
      const int r = r0 + i, c = c0 + tx;
      if (r < nrow && c < n) tile[i][tx] = src[(int64_t)r * n + c];
    }
    __syncthreads();
    for (int j = ty; j < 64; j += 4) {
      const int c = c0 + j, r = r0 + tx;
      const int v = c < n ? inv[c] : -1;
      if (r < nrow && (unsigned)v < (unsigned)n) dst[(int64_t)v * nrow + r] = tile[tx][j];
    }
  } else {  // visiting -> storage
    const T* src = (const T*)t.WcurT;
    T* dst = (T*)t.Wcur;
    for (int j = ty; j < 64; j += 4) {
      const int c = c0 + j, r = r0 + tx;
      const int v = c < n ? inv[c] : -1;
      if (r < nrow && (unsigned)v < (unsigned)n) tile[tx][j] = src[(int64_t)v * nrow + r];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
      const int r = r0 + i, c = c0 + tx;
      if (r < nrow && c < n) dst[(int64_t)r * n + c] = tile[i][tx];
    }
  }
}

// Commit: the k-quant encode of every tensor of a (type, importance) group,
// from the original weights (first iteration) or the compensated targets.
// At most 168 VGPRs, three waves per SIMD: the 32-value sub-block searches of Q4_K and
// Q5_K (146-152 registers since their pairwise sums accumulate as the terms are formed)
// held 171-179 before, two waves per SIMD.
template <int TT, bool IMAT>
__global__ __launch_bounds__(256, 3) void ef_commit_kernel(const EfDev* __restrict__ tab, int from_wcur) {
  const EfDev& t = tab[blockIdx.y];
  constexpr int S = 64 / Kq<TT>::G;
  const int64_t nsb = t.n / 256, NB = (int64_t)t.nrow * nsb;
  const int64_t blocks = ((NB + S - 1) / S + kWavesPerBlock - 1) / kWavesPerBlock;
  if ((int64_t)blockIdx.x >= blocks) return;
  kq_encode_block<TT, IMAT>(from_wcur ? t.Wcur : t.x, t.qw, NB, nsb, t.raw, blockIdx.x);
}

// 16 superblocks per workgroup (kq_decode_block); a tensor without a reconstruction
// output skips the whole workgroup.
template <int TT>
__global__ __launch_bounds__(256) void ef_decode_kernel(const EfDev* __restrict__ tab) {
  __shared__ __align__(16) KqDecodeLds<TT> lds;
  const EfDev& t = tab[blockIdx.y];
  if (!t.recon) return;
  kq_decode_block<TT>(t.raw, (int64_t)t.nrow * (t.n / 256), t.recon, blockIdx.x, lds);
}

// ---------------------------------------------------------------- committed grid
// Per (row, storage sub-block): step dl and offset ml of the committed bytes,
// written transposed [sub][row] (ef.py:87-127). One thread per (row, 16 weights).
__global__ void ef_grid_kernel(const EfDev* __restrict__ tab) {
  const EfDev& T = tab[blockIdx.y];
  const int ttype = T.ttype, nrow = T.nrow, n = T.n;
  const uint8_t* __restrict__ raw = T.raw;
  float* __restrict__ dlT = T.dlT;
  float* __restrict__ mlT = T.mlT;
  const int nsub16 = n / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int r = (int)(t % nrow);
  const int s16 = (int)(t / nrow);  // sub-block index in units of 16 weights
  if (s16 >= nsub16) return;
  const int sb = s16 >> 4, k = s16 & 15;
  float dl, ml = 0.0f;
  if (ttype == CP_Q2_K) {
    const uint8_t* b = raw + ((int64_t)r * (n / 256) + sb) * 84;
    float d = half_value(b[80] | b[81] << 8), dm = half_value(b[82] | b[83] << 8);
    dl = d * (float)(b[k] & 0xF);
    ml = dm * (float)(b[k] >> 4);
  } else if (ttype == CP_Q3_K) {
    const uint8_t* b = raw + ((int64_t)r * (n / 256) + sb) * 110;
    float d = half_value(b[108] | b[109] << 8);
    const uint8_t* sc = b + 96;
    int lo = (k < 8) ? (sc[k] & 0xF) : (sc[k - 8] >> 4);
    int hi = (sc[8 + (k & 3)] >> (2 * (k >> 2))) & 3;
    dl = d * (float)((lo | hi << 4) - 32);
  } else if (ttype == CP_Q4_K || ttype == CP_Q5_K) {
    if (k & 1) return;  // 32-wide sub-blocks: one thread per pair of 16s
    const int bp = ttype == CP_Q5_K ? 176 : 144;
    const uint8_t* b = raw + ((int64_t)r * (n / 256) + sb) * bp;
    float d = half_value(b[0] | b[1] << 8), dm = half_value(b[2] | b[3] << 8);
    const uint8_t* sc = b + 4;
    int j = k >> 1, s, m;
    if (j < 4) {
      s = sc[j] & 63;
      m = sc[j + 4] & 63;
    } else {
      s = (sc[j + 4] & 0xF) | (sc[j - 4] >> 6) << 4;
      m = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4;
    }
    dl = d * (float)s;
    ml = dm * (float)m;
    const int64_t o = (int64_t)(s16 >> 1) * nrow + r;
    dlT[o] = dl;
    mlT[o] = ml;
    return;
  } else {  // Q6_K
    const uint8_t* b = raw + ((int64_t)r * (n / 256) + sb) * 210;
    float d = half_value(b[208] | b[209] << 8);
    dl = d * (float)(int8_t)b[192 + k];
  }
  const int64_t o = (int64_t)s16 * nrow + r;
  dlT[o] = dl;
  if (mlT) mlT[o] = ml;
}

// ---------------------------------------------------------------- repack
// Rewrite the code bytes of committed superblocks from the sweep's codes, keeping
// the scale bytes (ef.py:130-176). The codes come straight from the visiting-order
// store LT[inv[c]][r]: a workgroup takes 128 rows x one superblock column, stages
// the 128 x 256 codes in LDS column by column (128 contiguous bytes of LT each), then
// writes the superblocks' code bytes, two per thread.

// Code byte b of one superblock from its codes c(k) (code of element k).
template <class C>
__device__ __forceinline__ uint32_t pack_code_byte(int ttype, const C& c, int b) {
  if (ttype == CP_Q2_K) {
    const int k = b - 16, base = (k >> 5) * 128 + (k & 31);
    return c(base) | c(base + 32) << 2 | c(base + 64) << 4 | c(base + 96) << 6;
  }
  if (ttype == CP_Q3_K) {
    if (b < 32) {
      uint32_t v = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) v |= ((c(32 * j + b) >> 2) & 1u) << j;
      return v;
    }
    const int k = b - 32, base = (k >> 5) * 128 + (k & 31);
    return (c(base) & 3) | (c(base + 32) & 3) << 2 | (c(base + 64) & 3) << 4 | (c(base + 96) & 3) << 6;
  }
  if (ttype == CP_Q4_K) {
    const int k = b - 16, base = (k >> 5) * 64 + (k & 31);
    return (c(base) & 0xF) | (c(base + 32) & 0xF) << 4;
  }
  if (ttype == CP_Q5_K) {
    if (b < 48) {  // qh: bit q of byte j is code (32q + j) >= 16
      uint32_t v = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q) v |= (uint32_t)(c(32 * q + b - 16) >> 4) << q;
      return v;
    }
    const int k = b - 48, base = (k >> 5) * 64 + (k & 31);
    return (c(base) & 0xF) | (c(base + 32) & 0xF) << 4;
  }
  if (b < 128) {  // Q6_K
    const int h = b >> 6, k = b & 63;
    const int base = h * 128 + (k & 31) + (k >= 32 ? 32 : 0);
    return (c(base) & 0xF) | (c(base + 64) & 0xF) << 4;
  }
  const int k = b - 128, base = (k >> 5) * 128 + (k & 31);
  return (c(base) >> 4) | (c(base + 32) >> 4) << 2 | (c(base + 64) >> 4) << 4 | (c(base + 96) >> 4) << 6;
}

__device__ __forceinline__ void code_span(int ttype, int* lo_b, int* hi_b, int* bp) {
  switch (ttype) {
    case CP_Q2_K: *lo_b = 16; *hi_b = 80; *bp = 84; break;
    case CP_Q3_K: *lo_b = 0; *hi_b = 96; *bp = 110; break;
    case CP_Q4_K: *lo_b = 16; *hi_b = 144; *bp = 144; break;
    case CP_Q5_K: *lo_b = 16; *hi_b = 176; *bp = 176; break;
    default: *lo_b = 0; *hi_b = 192; *bp = 210; break;
  }
}

constexpr int kPackRows = 128;   // rows per workgroup: one 128-byte line of each LT column
constexpr int kPackPitch = 132;  // LDS bytes per staged column: 33 words, so a wave's columns hit distinct banks

__global__ __launch_bounds__(256) void ef_pack_kernel(const EfDev* __restrict__ tab) {
  const EfDev& T = tab[blockIdx.y];
  const int nrow = T.nrow, n = T.n, nsb = n / 256;
  const int row_tiles = (nrow + kPackRows - 1) / kPackRows;
  if ((int)blockIdx.x >= row_tiles * nsb) return;
  const int rt = blockIdx.x / nsb, sb = blockIdx.x - rt * nsb;
  const int r0 = rt * kPackRows, rows = nrow - r0 < kPackRows ? nrow - r0 : kPackRows;
  __shared__ __align__(16) uint8_t codes[256 * kPackPitch];  // [column][row]
  const int t = threadIdx.x;
  {
    const int v = T.inv[sb * 256 + t];
    const uint8_t* src = T.LT + (int64_t)((unsigned)v < (unsigned)n ? v : 0) * nrow + r0;
    uint8_t* dst = codes + t * kPackPitch;
    if ((nrow & 15) == 0) {  // 16-byte aligned runs; rows is a multiple of 16
      for (int q = 0; q < rows / 16; ++q) {
        const uint4 v = reinterpret_cast<const uint4*>(src)[q];
        uint32_t* d = reinterpret_cast<uint32_t*>(dst + 16 * q);
        d[0] = v.x;
        d[1] = v.y;
        d[2] = v.z;
        d[3] = v.w;
      }
    } else {
      for (int i = 0; i < rows; ++i) dst[i] = src[i];
    }
  }
  __syncthreads();
  int lo_b, hi_b, bp;
  code_span(T.ttype, &lo_b, &hi_b, &bp);
  const int half = (hi_b - lo_b) / 2;  // byte pairs per superblock
  for (int p = t; p < rows * half; p += 256) {
    const int row = p / half, b = lo_b + 2 * (p - row * half);
    auto c = [&](int k) -> uint32_t { return codes[k * kPackPitch + row]; };
    const uint32_t v = pack_code_byte(T.ttype, c, b) | pack_code_byte(T.ttype, c, b + 1) << 8;
    *reinterpret_cast<uint16_t*>(T.raw + ((int64_t)(r0 + row) * nsb + sb) * bp + b) = (uint16_t)v;
  }
}

// ---------------------------------------------------------------- host driver

static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

struct EfLayout {
  size_t WpT, E, WcurT, Wcur, LT, dlT, mlT, inv, sbidx, end;
};

static EfLayout ef_layout(int64_t nrow, int64_t n, size_t base) {
  EfLayout L;
  const size_t w = (size_t)nrow * n;
  size_t o = base;
  L.WpT = o; o += a256(w * 4);
  L.E = o; o += a256(w * 4);
  L.WcurT = o; o += a256(w * 4);
  L.Wcur = o; o += a256(w * 4);
  L.LT = o; o += a256(w);
  L.dlT = o; o += a256((size_t)nrow * (n / 16) * 4);
  L.mlT = o; o += a256((size_t)nrow * (n / 16) * 4);
  L.inv = o; o += a256((size_t)n * 4);
  L.sbidx = o; o += a256((size_t)n * 4);
  L.end = o;
  return L;
}

// workspace: [status word (256 bytes)][sweep task table][tensor table][per-tensor buffers]
constexpr size_t kStatusBytes = 256;
static size_t ef_tables_bytes(int count) {
  return kStatusBytes + a256((size_t)count * sizeof(SweepTask)) + a256((size_t)count * sizeof(EfDev));
}

size_t ef_ws_bytes(const cp_ef_tensor* t, int count) {
  size_t o = ef_tables_bytes(count);
  for (int i = 0; i < count; ++i) o = ef_layout(t[i].nrow, t[i].n, o).end;
  return o;
}

static void grid_range(int ttype, int* lo, int* hi, int* sub) {
  switch (ttype) {
    case CP_Q2_K: *lo = 0; *hi = 3; *sub = 16; break;
    case CP_Q3_K: *lo = -4; *hi = 3; *sub = 16; break;
    case CP_Q4_K: *lo = 0; *hi = 15; *sub = 32; break;
    case CP_Q5_K: *lo = 0; *hi = 31; *sub = 32; break;
    default: *lo = -32; *hi = 31; *sub = 16; break;
  }
}

// Optional per-phase timing of an EF call (cp_ef_profile / cp_ef_phase_ms):
// setup, commit, sweep, repack, decode.
static thread_local PhaseClock g_clock;
#define CP_PHASE(p)                                                                \
  do {                                                                             \
    if (timed && g_clock.on) CP_HIP((p) < 0 ? g_clock.start(st) : g_clock.mark((p), st)); \
  } while (0)

// Spin bound of the pipe sweep's waits for the calling thread's EF calls (cp_ef_wait_limit).
constexpr int kDefaultWaitLimit = 1 << 16;
static thread_local int g_wait_limit = kDefaultWaitLimit;

// The calling thread's last sweep launch (cp_ef_last_sweep): rows per stripe, waves per
// stripe, mode (-1: none yet).
static thread_local int g_sweep_shape[3] = {0, 0, -1};

// A run of table rows sharing (type, importance) for the templated codec launches.
struct EfGroup {
  int first, count, ttype;
  bool imat;
  int64_t max_nb;  // superblocks of the largest tensor
};

template <int TT>
static void launch_commit(const EfDev* tab, const EfGroup& g, int from_wcur, hipStream_t st) {
  constexpr int S = 64 / Kq<TT>::G;
  const int64_t blocks = ((g.max_nb + S - 1) / S + kWavesPerBlock - 1) / kWavesPerBlock;
  const dim3 grid((unsigned)blocks, (unsigned)g.count);
  if (g.imat)
    ef_commit_kernel<TT, true><<<grid, 256, 0, st>>>(tab + g.first, from_wcur);
  else
    ef_commit_kernel<TT, false><<<grid, 256, 0, st>>>(tab + g.first, from_wcur);
}

template <int TT>
static void launch_decode(const EfDev* tab, const EfGroup& g, hipStream_t st) {
  const dim3 grid((unsigned)((g.max_nb + 4 * kDecSb - 1) / (4 * kDecSb)), (unsigned)g.count);
  ef_decode_kernel<TT><<<grid, 256, 0, st>>>(tab + g.first);
}

// timed: phases are recorded when the calling thread has timing on (cp_ef_profile)
int ef_encode_batch(const cp_ef_tensor* ts, int count, int n_iter, int mode, void* ws,
                    size_t ws_bytes, hipStream_t st, bool timed = true) {
  if (!ts || count <= 0) return set_error(CP_ERR_ARG, "no tensors");
  if (count > 65535) return set_error(CP_ERR_ARG, "at most 65535 tensors per call (got %d)", count);
  if (n_iter < 1) return set_error(CP_ERR_ARG, "n_iter must be >= 1");
  if (mode != CP_EF_EXACT && mode != CP_EF_MFMA && mode != CP_EF_EXACT_VALU)
    return set_error(CP_ERR_ARG, "unknown EF mode %d", mode);
  for (int i = 0; i < count; ++i) {
    const cp_ef_tensor& t = ts[i];
    KqGeom g;
    if (!kq_geom(t.ttype, &g) || g.block_weights != 256)
      return set_error(CP_ERR_TTYPE, "tensor %d: unsupported type %d", i, t.ttype);
    if (t.nrow <= 0 || t.n <= 0 || t.n % 256 || t.nrow > 65535 * 64 || t.n > (1 << 20) ||
        (t.n / 16) * t.nrow >= ((int64_t)1 << 31))
      return set_error(CP_ERR_SHAPE, "tensor %d: bad shape [%lld, %lld]", i, (long long)t.nrow, (long long)t.n);
    if (!t.x || !t.U || !t.order || !t.raw) return set_error(CP_ERR_ARG, "tensor %d: null pointer", i);
    if (!aligned(t.x, 16) || !aligned(t.raw, 4) || (t.qw && !aligned(t.qw, 16)) ||
        (t.recon && !aligned(t.recon, 16)))
      return set_error(CP_ERR_ALIGN, "tensor %d: misaligned buffer", i);
  }
  if (!ws || ws_bytes < ef_ws_bytes(ts, count))
    return set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, ef_ws_bytes(ts, count));
  if (!aligned(ws, 256)) return set_error(CP_ERR_ALIGN, "workspace needs 256-byte alignment");
  CP_PHASE(-1);
  char* base = (char*)ws;
  int* dstatus = (int*)base;
  SweepTask* dtasks = (SweepTask*)(base + kStatusBytes);
  EfDev* dtab = (EfDev*)(base + kStatusBytes + a256((size_t)count * sizeof(SweepTask)));
  std::vector<SweepTask> tasks(count);
  std::vector<EfDev> devs(count);
  int max_n = 0, max_rows = 0;
  size_t o = ef_tables_bytes(count);
  for (int i = 0; i < count; ++i) {
    const cp_ef_tensor& t = ts[i];
    const EfLayout L = ef_layout(t.nrow, t.n, o);
    o = L.end;
    int lo, hi, sub;
    grid_range(t.ttype, &lo, &hi, &sub);
    const bool affine = t.ttype == CP_Q2_K || t.ttype == CP_Q4_K || t.ttype == CP_Q5_K;
    float* mlT = affine ? (float*)(base + L.mlT) : nullptr;
    tasks[i] = SweepTask{(const float*)(base + L.WpT), t.U, (const float*)(base + L.dlT), mlT,
                         (const int*)(base + L.sbidx), (float*)(base + L.E),
                         (float*)(base + L.WcurT), (uint8_t*)(base + L.LT),
                         (int)t.nrow, (int)t.n, lo, hi};
    devs[i] = EfDev{t.x, t.qw, t.order, t.raw, t.recon, (float*)(base + L.WpT),
                    (float*)(base + L.WcurT), (float*)(base + L.Wcur), (uint8_t*)(base + L.LT),
                    (float*)(base + L.dlT), mlT, (int*)(base + L.inv),
                    (int*)(base + L.sbidx), (int)t.nrow, (int)t.n, t.ttype, sub};
    max_n = (int)t.n > max_n ? (int)t.n : max_n;
    max_rows = (int)t.nrow > max_rows ? (int)t.nrow : max_rows;
  }
  // tensor table ordered by (type, importance) so each codec group is one run
  // of rows; the sweep table longest stripes (largest n) first, so they do not
  // start last and set the tail
  std::vector<int> by_kind(count), by_len(count);
  for (int i = 0; i < count; ++i) by_kind[i] = by_len[i] = i;
  std::stable_sort(by_kind.begin(), by_kind.end(), [&](int a, int b) {
    if (ts[a].ttype != ts[b].ttype) return ts[a].ttype < ts[b].ttype;
    return (ts[a].qw != nullptr) < (ts[b].qw != nullptr);
  });
  std::stable_sort(by_len.begin(), by_len.end(),
                   [&](int a, int b) { return tasks[a].n > tasks[b].n; });
  std::vector<EfGroup> groups;
  for (int k = 0; k < count; ++k) {
    const cp_ef_tensor& t = ts[by_kind[k]];
    const int64_t nb = t.nrow * (t.n / 256);
    if (groups.empty() || groups.back().ttype != t.ttype || groups.back().imat != (t.qw != nullptr))
      groups.push_back(EfGroup{k, 0, t.ttype, t.qw != nullptr, 0});
    EfGroup& g = groups.back();
    ++g.count;
    g.max_nb = nb > g.max_nb ? nb : g.max_nb;
  }
  // Row stripes and waves per stripe (exact mode). A stripe of RS rows is one wave, or W
  // waves (blocks in rounds): W doubles while the call's waves still fit the GPU's 2048
  // two-per-SIMD slots and every tensor has a 64-column block per wave. 32-row stripes
  // halve the in-block quantization chain per row, so they are taken whenever some W
  // fills at least 1536 of those slots; otherwise 16-row stripes, which double the waves.
  int64_t stripes32 = 0, stripes16 = 0;
  int min_blocks = 1 << 30;
  for (int i = 0; i < count; ++i) {
    stripes32 += (ts[i].nrow + 31) / 32;
    stripes16 += (ts[i].nrow + 15) / 16;
    min_blocks = std::min(min_blocks, (int)(ts[i].n / 64));
  }
  const auto fill = [&](int64_t stripes) {
    int w = 1;
    while (w < 8 && stripes * 2 * w <= 2048 && 2 * w <= min_blocks) w *= 2;
    return w;
  };
  int RS, waves = 1;
  {
    const int w32 = fill(stripes32);
    if (stripes32 * w32 >= 1536) {
      RS = 32;
      waves = w32;
    } else {
      RS = 16;
      waves = fill(stripes16);
    }
  }
  if (mode == CP_EF_EXACT) {
    if (const char* e = getenv("CP_EF_SWEEP_ROWS")) {  // tuning override: 16 or 32
      const int r = atoi(e);
      if (r == 16 || r == 32) {
        RS = r;
        waves = fill(r == 32 ? stripes32 : stripes16);
      }
    }
    if (const char* e = getenv("CP_EF_SWEEP_WAVES")) {  // tuning override: 1, 2, 4 or 8
      const int w = atoi(e);
      if (w == 1 || w == 2 || w == 4 || w == 8) {
        waves = w;  // the largest of 1, 2, 4, 8 within the request and every tensor's blocks
        while (waves > 1 && waves > min_blocks) waves /= 2;
      }
    }
  } else {
    waves = 1;
  }
  int64_t total_stripes = 0;
  bool same_n = true;
  for (int k = 0; k < count; ++k) {
    SweepTask& tk = tasks[by_len[k]];
    tk.first = (int)total_stripes;
    total_stripes += (tk.nrow + RS - 1) / RS;
    same_n = same_n && tk.n == tasks[by_len[0]].n;
  }
  if (total_stripes > ((int64_t)1 << 30)) return set_error(CP_ERR_SHAPE, "too many row stripes");
  for (int c0 = 0; c0 < count; c0 += kTasksPerLaunch) {
    const int cn = count - c0 < kTasksPerLaunch ? count - c0 : kTasksPerLaunch;
    SweepBatch b;
    for (int i = 0; i < cn; ++i) b.t[i] = tasks[by_len[c0 + i]];
    ef_tasks_store_kernel<<<1, 64, 0, st>>>(b, cn, dtasks + c0, c0 == 0 ? dstatus : nullptr);
  }
  for (int c0 = 0; c0 < count; c0 += kDevPerStore) {
    const int cn = count - c0 < kDevPerStore ? count - c0 : kDevPerStore;
    EfDevBatch b;
    for (int i = 0; i < cn; ++i) b.t[i] = devs[by_kind[c0 + i]];
    ef_dev_store_kernel<<<1, 64, 0, st>>>(b, cn, dtab + c0);
  }
  const unsigned col_tiles = (unsigned)((max_n + 63) / 64), row_tiles = (unsigned)((max_rows + 63) / 64);
  ef_index_kernel<<<dim3((unsigned)((max_n + 255) / 256), (unsigned)count), 256, 0, st>>>(dtab);
  ef_transpose_kernel<0><<<dim3(col_tiles, row_tiles, (unsigned)count), 256, 0, st>>>(dtab);
  CP_LAUNCHED("EF setup");
  CP_PHASE(0);

  for (int it = 0; it < n_iter; ++it) {
    for (const EfGroup& g : groups) {
      switch (g.ttype) {
        case CP_Q2_K: launch_commit<CP_Q2_K>(dtab, g, it > 0, st); break;
        case CP_Q3_K: launch_commit<CP_Q3_K>(dtab, g, it > 0, st); break;
        case CP_Q4_K: launch_commit<CP_Q4_K>(dtab, g, it > 0, st); break;
        case CP_Q5_K: launch_commit<CP_Q5_K>(dtab, g, it > 0, st); break;
        default: launch_commit<CP_Q6_K>(dtab, g, it > 0, st); break;
      }
    }
    const int64_t grid_threads = (int64_t)max_rows * (max_n / 16);
    ef_grid_kernel<<<dim3((unsigned)((grid_threads + 255) / 256), (unsigned)count), 256, 0, st>>>(dtab);
    CP_LAUNCHED("EF commit");
    CP_PHASE(1);
    g_sweep_shape[0] = RS;
    g_sweep_shape[1] = mode == CP_EF_EXACT ? waves : 1;
    g_sweep_shape[2] = mode;
    if (mode == CP_EF_EXACT_VALU)
      ef_sweep_exact_kernel<BLK><<<dim3((unsigned)((max_rows + 255) / 256), (unsigned)count), 256, 0, st>>>(dtasks);
    else if (mode == CP_EF_EXACT && waves == 1 && RS == 32)
      ef_sweep_rows_kernel<32><<<(unsigned)(8 * ((total_stripes + 7) / 8)), 64, 0, st>>>(
          dtasks, count, (int)total_stripes, same_n ? 1 : 0);
    else if (mode == CP_EF_EXACT && waves == 1)
      ef_sweep_rows_kernel<16><<<(unsigned)(8 * ((total_stripes + 7) / 8)), 64, 0, st>>>(
          dtasks, count, (int)total_stripes, same_n ? 1 : 0);
    else if (mode == CP_EF_EXACT) {
      const unsigned g = (unsigned)(8 * ((total_stripes + 7) / 8));
      const int xr = same_n ? 1 : 0, ns = (int)total_stripes, wl = g_wait_limit;
      if (RS == 32) {
        switch (waves) {
          case 2: ef_sweep_pipe_kernel<32, 2><<<g, 128, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
          case 4: ef_sweep_pipe_kernel<32, 4><<<g, 256, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
          default: ef_sweep_pipe_kernel<32, 8><<<g, 512, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
        }
      } else {
        switch (waves) {
          case 2: ef_sweep_pipe_kernel<16, 2><<<g, 128, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
          case 4: ef_sweep_pipe_kernel<16, 4><<<g, 256, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
          default: ef_sweep_pipe_kernel<16, 8><<<g, 512, 0, st>>>(dtasks, count, ns, xr, wl, dstatus); break;
        }
      }
    }
    else
      ef_sweep_mfma_kernel<BLK><<<dim3((unsigned)((max_rows + 63) / 64), (unsigned)count), 64, 0, st>>>(dtasks);
    CP_LAUNCHED("EF sweep");
    CP_PHASE(2);
    const int64_t pack_units = (int64_t)((max_rows + kPackRows - 1) / kPackRows) * (max_n / 256);
    ef_pack_kernel<<<dim3((unsigned)pack_units, (unsigned)count), 256, 0, st>>>(dtab);
    if (it + 1 < n_iter)
      ef_transpose_kernel<2><<<dim3(col_tiles, row_tiles, (unsigned)count), 256, 0, st>>>(dtab);
    CP_LAUNCHED("EF repack");
    CP_PHASE(3);
  }
  for (const EfGroup& g : groups) {
    switch (g.ttype) {
      case CP_Q2_K: launch_decode<CP_Q2_K>(dtab, g, st); break;
      case CP_Q3_K: launch_decode<CP_Q3_K>(dtab, g, st); break;
      case CP_Q4_K: launch_decode<CP_Q4_K>(dtab, g, st); break;
      case CP_Q5_K: launch_decode<CP_Q5_K>(dtab, g, st); break;
      default: launch_decode<CP_Q6_K>(dtab, g, st); break;
    }
  }
  CP_LAUNCHED("EF decode");
  CP_PHASE(4);
  return CP_OK;
}

int ef_phase_ms(float* out, int nphase) {
  CP_HIP(g_clock.read(out, nphase));
  return nphase < 5 ? nphase : 5;
}

// ---------------------------------------------------------------- allocation-free entry
// The EF workspace of cp_ef_encode_noalloc: a static device array that every GPU the
// library runs on holds until the process ends. Its name is a host-side stand-in,
// never a device address: host code only uses the address hipGetSymbolAddress gives
// for the current device, looked up once per device on that device's first call.
// Nothing in the EF workspace has to start at zero (every buffer is written before
// it is read), so a call may find the previous call's contents there.
constexpr size_t kNoAllocWsBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kNoAllocWsBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_ptr(void** out) {
  int dev = -1;
  CP_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(CP_ERR_ARG, "device %d out of range", dev);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(CP_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CP_OK;
}

int ef_encode_noalloc(const cp_ef_tensor& t, int n_iter, hipStream_t st) {
  const size_t need = t.nrow > 0 && t.n > 0 ? ef_ws_bytes(&t, 1) : 0;  // bad shapes: ef_encode_batch's error
  if (need > kNoAllocWsBytes)
    return set_error(CP_ERR_WORKSPACE,
                     "tensor [%lld, %lld] needs %zu bytes of EF workspace; the allocation-free "
                     "entry point holds %zu (use cp_ef_encode with a caller workspace)",
                     (long long)t.nrow, (long long)t.n, need, kNoAllocWsBytes);
  void* ws = nullptr;
  if (int e = scratch_ptr(&ws)) return e;
  // untimed: phase timing would create events on first use
  return ef_encode_batch(&t, 1, n_iter, CP_EF_EXACT, ws, kNoAllocWsBytes, st, false);
}

// CP_OK, or CP_ERR_TIMEOUT when the status word of the EF call that used workspace ws
// (the static one of cp_ef_encode_noalloc on the current device when ws is null) says
// a sweep wave gave up waiting. Synchronizes st.
int ef_read_status(const void* ws, hipStream_t st) {
  const void* src = ws;
  if (!src) {
    void* p = nullptr;
    if (int e = scratch_ptr(&p)) return e;
    src = p;
  }
  int status = 0;
  CP_HIP(hipMemcpyAsync(&status, src, sizeof(int), hipMemcpyDeviceToHost, st));
  CP_HIP(hipStreamSynchronize(st));
  if (status & 1)
    return set_error(CP_ERR_TIMEOUT,
                     "EF sweep: a wave gave up waiting for an earlier block of its stripe (spin "
                     "bound exhausted); the call's bytes are not valid");
  return CP_OK;
}

}  // namespace cp

extern "C" {

void cp_ef_profile(int enable) { cp::g_clock.on = enable != 0; }

void cp_ef_wait_limit(int spins) { cp::g_wait_limit = spins < 0 ? cp::kDefaultWaitLimit : spins; }

int cp_ef_read_status(const void* ws, void* stream) {
  cp::clear_error();
  return cp::ef_read_status(ws, (hipStream_t)stream);
}

int cp_ef_phase_ms(float* out, int nphase) {
  cp::clear_error();
  if (!out || nphase <= 0) return cp::set_error(CP_ERR_ARG, "bad phase buffer");
  return cp::ef_phase_ms(out, nphase);
}

int cp_ef_last_sweep(int* rows_per_stripe, int* waves) {
  cp::clear_error();
  if (!rows_per_stripe || !waves) return cp::set_error(CP_ERR_ARG, "null output");
  *rows_per_stripe = cp::g_sweep_shape[0];
  *waves = cp::g_sweep_shape[1];
  return cp::g_sweep_shape[2];
}

size_t cp_ef_ws_bytes(const cp_ef_tensor* tensors, int count) {
  if (!tensors || count <= 0) return 0;
  return cp::ef_ws_bytes(tensors, count);
}

int cp_ef_encode_batch(const cp_ef_tensor* tensors, int count, int n_iter, int mode, void* ws,
                       size_t ws_bytes, void* stream) {
  cp::clear_error();
  return cp::ef_encode_batch(tensors, count, n_iter, mode, ws, ws_bytes, (hipStream_t)stream);
}

int cp_ef_encode(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                 const float* U, const int32_t* order, int n_iter, uint8_t* raw, float* recon,
                 void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  cp_ef_tensor t{ttype, nrow, n, x, qw, U, order, raw, recon};
  return cp::ef_encode_batch(&t, 1, n_iter, CP_EF_EXACT, ws, ws_bytes, (hipStream_t)stream);
}

size_t cp_ef_noalloc_max_ws_bytes(void) { return cp::kNoAllocWsBytes; }

int cp_ef_encode_noalloc(int ttype, const float* x, int64_t nrow, int64_t n, const float* qw,
                         const float* U, const int32_t* order, int n_iter, uint8_t* raw,
                         float* recon, void* stream) {
  cp::clear_error();
  cp_ef_tensor t{ttype, nrow, n, x, qw, U, order, raw, recon};
  return cp::ef_encode_noalloc(t, n_iter, (hipStream_t)stream);
}

}  // extern "C"
