// Input-Hessian accumulation H += X^T X on gfx950 MFMA (coldpress/hessians.py:137-154).
//
// X is [N, d] row-major activations (bf16 or f32), H is [d, d] float32 and is
// accumulated in place (beta = 1), so hook batches can stream in. Split-K over
// rows of X: N is 65536-131072 while d is 1024-14336, so the row dimension is
// what fills 256 CUs. The result does not depend on scheduling: with one row
// split a workgroup adds its finished tile into H itself (one writer per
// element); with several, each split stores its tile into a workspace slot of
// its own and one reduction pass adds the splits' tiles to H in split order
// (H + ((p0 + p1) + p2 ...)). The same X therefore gives the same H bit for
// bit, run after run.
//
//  bf16: lower-triangle 256 x 256 tiles on v_mfma_f32_32x32x16_bf16, operands
//        read transposed from LDS (hess_bf16_tri_kernel), then a pass that
//        reduces the splits and mirrors the lower triangle into the upper one;
//  f32:  128 x 128 tiles on v_mfma_f32_32x32x2f32, which takes one row t per
//        lane, so the [t][i] panel is used as loaded.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <type_traits>

#include "cp_host.h"

namespace cp {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int HT = 128;  // f32 kernel: H tile edge
constexpr int KT = 32;   // f32 kernel: rows of X per step

// Row of the 32x32 MFMA result held by register v of lane l (column = l % 32).
__device__ __forceinline__ int mfma32_row(int v, int l) { return 8 * (v >> 2) + 4 * (l >> 5) + (v & 3); }

// ---------------------------------------------------------------- bf16 input
// Lower-triangle tiles of 256 x 256 (H is symmetric; hess_tri_reduce_kernel copies
// the lower triangle into the upper one afterwards), split-K over rows of X.
// A workgroup is 4 waves, each owning a 128 x 128 block as 4 x 4 MFMA 32x32
// tiles (256 float32 accumulators): the largest block a wave can hold, because
// the LDS traffic per MFMA, not the MFMAs, bounds this kernel.
//
// Rows of X are staged 32 at a time: both 32 x 256 panels (columns of the i-
// and j-tile; one panel on a diagonal tile) are fetched into registers two
// stages ahead of use, stored into a 4-slot LDS ring in X's own [t][c] layout,
// and read as MFMA operands with ds_read_b64_tr_b16, which returns 4
// consecutive rows t of one column per lane: v_mfma_f32_32x32x16_bf16 takes 8
// consecutive t per lane for both operands. Panel rows are padded from 512 to
// 576 bytes so the four rows of one transposed read fall 64 bytes apart in
// bank space (conflict-free), and every LDS address in the loop is a per-lane
// base plus an immediate: with one wave per SIMD, address arithmetic between
// the MFMAs is not hidden by anything.
//
// Work items (row split, tile) are ordered split-major and handed out
// XCD-contiguously: the hardware places workgroup w on XCD w % 8, so
// item = (w % 8) * per + w / 8 keeps the workgroups of one XCD on the same
// rows of X (shared in its L2).
constexpr int BT = 256;             // H tile edge
constexpr int KS = 32;              // rows of X per stage
constexpr int PROW = BT * 2 + 64;   // bytes per padded panel row
constexpr int PANEL = KS * PROW;    // 18 KB
constexpr int HNT = 256;            // threads per workgroup
constexpr int NSLOT = 4;            // LDS ring (stage s in slot s % 4)
constexpr int CPT = 2048 / HNT;     // 16-byte chunks per thread per stage (two panels)

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4i16* lds_v4p;

// Global side of the staging: raw buffer loads over the workgroup's row split
// (base X + r0 * d, num_records = its byte length). A load whose offset is at or
// past num_records returns zeros, so rows past the split's end and 8-column
// chunks past d (given an offset past the end) need no branch, and the loop
// has no control flow between loads: the compiler then waits only for the
// load a store needs, not for every load in flight.
//
// Chunk q of a stage (16 bytes per thread, q < 4 on the i-panel, q >= 4 on the
// j-panel): row (tid / 32) + 8 (q % 4), column chunk tid % 32.
constexpr uint32_t kOob = 0x80000000u;  // past any num_records the host allows

template <int NQ>
struct Stager {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t off[NQ];  // chunk q's byte offset at stage 0 (kOob when outside d)
  uint32_t sbytes;   // bytes per stage (KS rows)
};

template <int NQ>
__device__ __forceinline__ Stager<NQ> make_stager(const uint16_t* X, int64_t r0, int64_t nrows,
                                                  int d, int i0, int j0, int tid) {
  Stager<NQ> s;
  const uint32_t rowb = 2u * (uint32_t)d;
  s.rs = __builtin_amdgcn_make_buffer_rsrc((void*)(X + r0 * d), 0, (int)(nrows * rowb), 0x00020000);
  const int c8 = 8 * (tid & 31);
  const uint32_t row0 = (uint32_t)(tid >> 5) * rowb;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int c = (q >= 4 ? j0 : i0) + c8;  // d % 8 == 0: the 8 columns are all in or all out
    s.off[q] = c < d ? row0 + (uint32_t)(8 * (q & 3)) * rowb + 2u * (uint32_t)c : kOob;
  }
  s.sbytes = (uint32_t)KS * rowb;
  return s;
}

template <int NQ>
__device__ __forceinline__ void stage_load_one(const Stager<NQ>& st, int s, uint4 (&g)[CPT], int q) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(st.rs, (int)(st.off[q] + (uint32_t)s * st.sbytes),
                                                       0, 0);
  g[q] = make_uint4(v[0], v[1], v[2], v[3]);
}

// LDS byte offset of chunk q within a slot, relative to the thread's store base
// (tid / 32) * PROW + 16 * (tid % 32)
__device__ __forceinline__ constexpr int chunk_ofs(int q) { return (q >> 2) * PANEL + 8 * (q & 3) * PROW; }

struct Operands {
  bf16x8 a[4], b[4];
};

// Piece i (0..15) of one half of a stage's operands: the lo or hi four rows of
// one operand, in the order a0, b0, b1, b2, b3, a1, a2, a3 -- the order the
// MFMAs (x, y) = (i / 4, i % 4) first use them. ra / rb: this lane's read base
// in the A / B panel of the slot; the rest of the address is an immediate.
// Lane l gets column col + l % 32, rows 8 * (l / 32) + 0..7 of the half.
__device__ __forceinline__ void read_piece(const char* ra, const char* rb, int half, int i,
                                           Operands& f) {
  const int op = i >> 1, hi = i & 1;
  const bool isb = op >= 1 && op <= 4;
  const int idx = isb ? op - 1 : (op == 0 ? 0 : op - 4);
  const char* p = (isb ? rb : ra) + (16 * half + 4 * hi) * PROW + 64 * idx;
  const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4p)p);
  const v8i16 w = __builtin_shufflevector(v, v, 0, 1, 2, 3, 0, 1, 2, 3);
  v8i16 cur = __builtin_bit_cast(v8i16, isb ? f.b[idx] : f.a[idx]);
  if (hi)
    cur = __builtin_shufflevector(cur, w, 0, 1, 2, 3, 12, 13, 14, 15);
  else
    cur = __builtin_shufflevector(w, cur, 0, 1, 2, 3, 12, 13, 14, 15);
  if (isb)
    f.b[idx] = __builtin_bit_cast(bf16x8, cur);
  else
    f.a[idx] = __builtin_bit_cast(bf16x8, cur);
}

// STAGE_ONLY: the wave stages its share of the panels and meets every barrier but
// reads no operands and issues no MFMAs -- the wave of a diagonal tile whose 128 x 128
// block lies wholly above the diagonal, whose sums would be discarded.
template <bool DIAG, bool STAGE_ONLY = false>
__device__ __forceinline__ void tile_rows(const uint16_t* X, int64_t r0, int64_t r1, int d, int i0,
                                          int j0, char* lds, f32x16 (&acc)[4][4]) {
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = (w >> 1) * 128, wn = (w & 1) * 128;
  constexpr int NQ = DIAG ? CPT / 2 : CPT;  // 16-byte chunks per thread per stage
  constexpr int SLOT = DIAG ? PANEL : 2 * PANEL;
  // stages rounded up to a multiple of 4 (the unrolled loop body): stages past
  // the split's end load as zeros and add nothing
  const int ns = (int)((r1 - r0 + 4 * KS - 1) / (4 * KS)) * 4;
  const Stager<NQ> st = make_stager<NQ>(X, r0, r1 - r0, d, i0, j0, tid);
  // per-lane LDS bases: transposed reads (row 8 * (g / 2) + c / 4, column
  // 16 * (g % 2) + 4 * (c % 4) of the wave's block, g = l / 16, c = l % 16) and
  // stores (row tid / 32, 16-byte chunk tid % 32)
  const int g4 = l >> 4, c4 = l & 15;
  const int rlane = (8 * (g4 >> 1) + (c4 >> 2)) * PROW + 2 * (16 * (g4 & 1) + 4 * (c4 & 3));
  char* const ra0 = lds + rlane + 2 * wm;
  char* const rb0 = lds + rlane + 2 * wn + (DIAG ? 0 : PANEL);
  char* const wr0 = lds + (tid >> 5) * PROW + 16 * (tid & 31);
  uint4 g0[CPT], g1[CPT];
#pragma unroll
  for (int q = 0; q < NQ; ++q) stage_load_one(st, 0, g0, q);
#pragma unroll
  for (int q = 0; q < NQ; ++q) stage_load_one(st, 1, g1, q);
#pragma unroll
  for (int q = 0; q < NQ; ++q) *reinterpret_cast<uint4*>(wr0 + chunk_ofs(q)) = g0[q];
#pragma unroll
  for (int q = 0; q < NQ; ++q) *reinterpret_cast<uint4*>(wr0 + SLOT + chunk_ofs(q)) = g1[q];
#pragma unroll
  for (int q = 0; q < NQ; ++q) stage_load_one(st, 2, g0, q);
#pragma unroll
  for (int q = 0; q < NQ; ++q) stage_load_one(st, 3, g1, q);
  __syncthreads();
  Operands f0, f1;
  if constexpr (!STAGE_ONLY) {
#pragma unroll
    for (int i = 0; i < 16; ++i) read_piece(ra0, rb0, 0, i, f0);
  }
  // Stage s (K = s % 4): store stage s + 2 (fetched two stages ago) into slot
  // K + 2, fetch stage s + 4 into the same registers, and multiply stage s
  // while reading the next operands (its second half, then the first half of
  // stage s + 1). Past the end the same steps run on zero stages and slots no
  // stage reads, so the body has no branches.
  //
  // With one wave per SIMD nothing hides a wave's own LDS waits, so the step
  // is issued as one interleaved stream, pinned in place by scheduling
  // barriers: each of the 32 MFMAs is followed by one of the 32 transposed
  // reads of the next operands, and the stores are spread over the step, each
  // chunk's store followed by the load of the same chunk four stages ahead
  // (so every store waits only for the oldest load in flight), keeping the
  // LDS busy while the MFMAs run instead of the two taking turns.
  auto step = [&](auto kc, int s, uint4 (&g)[CPT]) {
    constexpr int K = decltype(kc)::value;
    __syncthreads();
    const char* ra = ra0 + K * SLOT;
    const char* rb = rb0 + K * SLOT;
    const char* na = ra0 + ((K + 1) % NSLOT) * SLOT;
    const char* nb = rb0 + ((K + 1) % NSLOT) * SLOT;
    char* dst = wr0 + ((K + 2) % NSLOT) * SLOT;
    constexpr int SE = 32 / NQ;  // MFMAs per store
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (!STAGE_ONLY) {
        acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f0.a[i >> 2], f0.b[i & 3],
                                                                     acc[i >> 2][i & 3], 0, 0, 0);
        read_piece(ra, rb, 1, i, f1);
      }
      if (i % SE == 0) {
        *reinterpret_cast<uint4*>(dst + chunk_ofs(i / SE)) = g[i / SE];
        stage_load_one(st, s + 4, g, i / SE);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (!STAGE_ONLY) {
        acc[i >> 2][i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f1.a[i >> 2], f1.b[i & 3],
                                                                     acc[i >> 2][i & 3], 0, 0, 0);
        read_piece(na, nb, 0, i, f0);
      }
      if (i % SE == 0) {
        *reinterpret_cast<uint4*>(dst + chunk_ofs(NQ / 2 + i / SE)) = g[NQ / 2 + i / SE];
        stage_load_one(st, s + 4, g, NQ / 2 + i / SE);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int s = 0; s < ns; s += 4) {
    step(std::integral_constant<int, 0>(), s, g0);
    step(std::integral_constant<int, 1>(), s + 1, g1);
    step(std::integral_constant<int, 2>(), s + 2, g0);
    step(std::integral_constant<int, 3>(), s + 3, g1);
  }
}

// Up to kHessJobs Hessians of one shape per launch, by value in the kernel arguments.
constexpr int kHessJobs = 224;
struct HessJobs {
  const uint16_t* X[kHessJobs];
  float* H[kHessJobs];
};
static_assert(sizeof(HessJobs) <= 4000, "kernel argument block");

// part == nullptr (one row split): the workgroup adds its tile into H's lower
// triangle. Otherwise it stores the whole 256 x 256 tile, row-major, into slot
// (job, split, tile) of part, for hess_tri_reduce_kernel.
__global__ __launch_bounds__(HNT) void hess_bf16_tri_kernel(const HessJobs jobs, int njobs,
                                                            int64_t N, int d, int ntiles, int splits,
                                                            int64_t rows_per_split,
                                                            float* __restrict__ part) {
  __shared__ __align__(16) char lds[NSLOT * 2 * PANEL];
  // items run job by job, then split by split: the XCD-contiguous hand-out keeps one
  // XCD on the same rows of one X
  const int per_job = ntiles * splits;
  const int total = per_job * njobs;
  const int per = (total + 7) / 8;
  const int item = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (item >= total) return;
  const int job = item / per_job, rem = item - job * per_job;
  const int split = rem / ntiles, tile = rem - split * ntiles;
  const uint16_t* __restrict__ X = jobs.X[job];
  float* __restrict__ H = jobs.H[job];
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
  if (ti != tj)
    tile_rows<false>(X, r0, r1, d, i0, j0, lds, acc);
  else if (wn > wm)  // wave 1: its block is above the diagonal
    tile_rows<true, true>(X, r0, r1, d, i0, j0, lds, acc);
  else
    tile_rows<true>(X, r0, r1, d, i0, j0, lds, acc);
  // lane l holds, for register v of tile (x, y), row wm + 32x + mfma32_row(v, l)
  // and column wn + 32y + l % 32 of the workgroup tile
  if (part) {
    // every register stored (zeros where the wave skipped its block; rows and
    // columns past d hold sums of zero-filled loads): the reduction reads only
    // the lower-triangle entries inside d
    float* Pb = part + ((int64_t)(job * splits + split) * ntiles + tile) * (BT * BT) +
                (wm + 4 * (l >> 5)) * BT + wn + (l & 31);
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int v = 0; v < 16; ++v) Pb[(x * 32 + 8 * (v >> 2) + (v & 3)) * BT + y * 32] = acc[x][y][v];
    return;
  }
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
        float* p = Hb + (int64_t)(x * 32 + 8 * (v >> 2) + (v & 3)) * d + y * 32;
        if (full || (i < d && j <= i)) *p = *p + acc[x][y][v];
      }
}

// Finishes a bf16 accumulation over the 64 x 64 blocks (bi, bj), bj <= bi, of the lower
// triangle, one workgroup each (blockIdx.x: the job's lower blocks in row order,
// blockIdx.y: the job). With part, each entry (i, j) becomes H + (p_0 + p_1 + ... +
// p_{splits-1}), the row splits' tiles summed in split order; then the block is written
// to the mirror position (j, i) as well, through LDS, so H leaves symmetric. Thread t
// covers 4 consecutive columns (16-byte accesses; d % 4 == 0, so a 4-column group is
// wholly inside or outside d) of rows t / 16 + 16 q. A diagonal block's entries above
// the diagonal are first written with the sums of their own (meaningless) positions and
// then overwritten by the mirror after the barrier, so its float4 stores need no mask;
// the mirror stores mask the entries on and below the diagonal. H's upper triangle is
// never used.
__global__ __launch_bounds__(256) void hess_tri_reduce_kernel(const HessJobs jobs, int d, int ntiles,
                                                              int splits,
                                                              const float* __restrict__ part) {
  float* __restrict__ H = jobs.H[blockIdx.y];
  __shared__ float tl[64][65];
  int bi = (int)((sqrtf(8.0f * (float)blockIdx.x + 1.0f) - 1.0f) * 0.5f);
  while (bi * (bi + 1) / 2 > (int)blockIdx.x) --bi;
  while ((bi + 1) * (bi + 2) / 2 <= (int)blockIdx.x) ++bi;
  const int bj = (int)blockIdx.x - bi * (bi + 1) / 2;
  const int cg = threadIdx.x & 15, rt = threadIdx.x >> 4;
  const int j = bj * 64 + 4 * cg;
  const int tj = j / BT;
  const int64_t slot = (int64_t)ntiles * (BT * BT);  // floats between one split's tiles
  const float* pj = part ? part + (int64_t)blockIdx.y * splits * slot : nullptr;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = rt + 16 * q, i = bi * 64 + r;
    if (i >= d || j >= d) continue;
    float4 h = *reinterpret_cast<const float4*>(H + (int64_t)i * d + j);
    if (pj) {
      const int ti = i / BT;
      const float* p = pj + (int64_t)(ti * (ti + 1) / 2 + tj) * (BT * BT) + (i % BT) * BT + (j % BT);
      float4 s = *reinterpret_cast<const float4*>(p);
      for (int k = 1; k < splits; ++k) {
        const float4 v = *reinterpret_cast<const float4*>(p + k * slot);
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
      }
      h.x += s.x;
      h.y += s.y;
      h.z += s.z;
      h.w += s.w;
      *reinterpret_cast<float4*>(H + (int64_t)i * d + j) = h;
    }
    tl[r][4 * cg] = h.x;
    tl[r][4 * cg + 1] = h.y;
    tl[r][4 * cg + 2] = h.z;
    tl[r][4 * cg + 3] = h.w;
  }
  __syncthreads();
  // upper block: rows bj, columns bi; entry (bj*64 + r, bi*64 + c) = lower (bi*64 + c, bj*64 + r)
  const int jj = bi * 64 + 4 * cg;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = rt + 16 * q, i = bj * 64 + r;
    if (i >= d || jj >= d) continue;
    float* dst = H + (int64_t)i * d + jj;
    const float4 v = make_float4(tl[4 * cg][r], tl[4 * cg + 1][r], tl[4 * cg + 2][r], tl[4 * cg + 3][r]);
    if (bi != bj || jj > i) {
      *reinterpret_cast<float4*>(dst) = v;
    } else {
      if (jj + 1 > i) dst[1] = v.y;
      if (jj + 2 > i) dst[2] = v.z;
      if (jj + 3 > i) dst[3] = v.w;
    }
  }
}

// ---------------------------------------------------------------- f32 input
// part == nullptr (one row split): the workgroup adds its tile into H. Otherwise
// it stores the tile into split blockIdx.z's full [d, d] partial in part, for
// hess_f32_reduce_kernel.
__global__ __launch_bounds__(256) void hess_f32_kernel(const float* __restrict__ X, int64_t N, int d,
                                                       int64_t rows_per_split, float* __restrict__ H,
                                                       float* __restrict__ part) {
  __shared__ float sA[KT][HT + 4];
  __shared__ float sB[KT][HT + 4];
  const int i0 = blockIdx.y * HT, j0 = blockIdx.x * HT;
  const int64_t r0 = (int64_t)blockIdx.z * rows_per_split;
  const int64_t r1 = min(N, r0 + rows_per_split);
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
  float* const dst = part ? part + (int64_t)blockIdx.z * d * d : H;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int i = i0 + wm + x * 32 + mfma32_row(v, l);
        int j = j0 + wn + y * 32 + (l & 31);
        if (i < d && j < d) {
          float* p = dst + (int64_t)i * d + j;
          *p = part ? acc[x][y][v] : *p + acc[x][y][v];
        }
      }
}

// H[e] = H[e] + (p_0[e] + p_1[e] + ... + p_{splits-1}[e]): the f32 path's row
// splits summed in split order.
__global__ __launch_bounds__(256) void hess_f32_reduce_kernel(float* __restrict__ H, int64_t dd,
                                                              int splits,
                                                              const float* __restrict__ part) {
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < dd; e += (int64_t)gridDim.x * 256) {
    float s = part[e];
    for (int k = 1; k < splits; ++k) s += part[k * dd + e];
    H[e] = H[e] + s;
  }
}

// Row splits for the triangle kernel: one 144 KB-LDS workgroup per CU, so the
// main pass takes about rounds x (stages per split + epilogue), the epilogue (a
// 256 KB tile store) about 6 stages; with more than one split the reduction then
// reads every split's tile once, about 0.05 of a stage per tile and split
// spread over the GPU. A split spans at most 2^30 bytes of X, so the buffer
// offsets of its loads (up to eight stages past its end) stay below 2^31.
// Returns the split count (0 if none fits); *rows_per_split is a multiple of KS
// and every split has rows.
static int pick_splits(int ntiles, int64_t N, int64_t d, int64_t* rows_per_split) {
  int best_s = 0;
  double best = 1e30;
  for (int s = 1; s <= 4096; ++s) {
    const int64_t rows = (N + s - 1) / s;
    if ((rows + KS - 1) / KS * KS * 2 * d > (int64_t(1) << 30)) continue;
    if (best_s && rows < 256) break;
    const double stages = (double)((rows + KS - 1) / KS);
    const double rounds = (double)(((int64_t)ntiles * s + 255) / 256);
    const double cost = rounds * (stages + 6.0) + (s > 1 ? 0.05 * s * ntiles : 0.0);
    if (cost < best - 1e-9) {
      best = cost;
      best_s = s;
    }
  }
  if (const char* e = getenv("CP_HESS_SPLITS")) {  // tuning override (measurement only)
    const int s = atoi(e);
    if (s >= 1 && s <= 4096 && ((N + s - 1) / s + KS - 1) / KS * KS * 2 * d <= (int64_t(1) << 30)) best_s = s;
  }
  if (best_s == 0) return 0;
  int64_t rps = (N + best_s - 1) / best_s;
  rps = (rps + KS - 1) / KS * KS;
  *rows_per_split = rps;
  return (int)((N + rps - 1) / rps);  // rounding rps up may leave fewer splits with rows
}

// Row splits of the f32 kernel: about 4 workgroups per CU, each at least 512 rows.
static int f32_splits(int64_t N, int64_t d, int64_t* rows_per_split) {
  const int tiles = (int)((d + HT - 1) / HT);
  const int64_t want = (1024 + (int64_t)tiles * tiles - 1) / ((int64_t)tiles * tiles);
  const int64_t splits = want < 1 ? 1 : want;
  int64_t rps = (N + splits - 1) / splits;
  if (rps < 512) rps = 512;
  rps = (rps + KT - 1) / KT * KT;
  *rows_per_split = rps;
  return (int)((N + rps - 1) / rps);
}

constexpr size_t kTileBytes = (size_t)BT * BT * sizeof(float);

// Workspace of one bf16 launch of cn jobs (0 when it runs as one split).
static size_t bf16_ws(int cn, int64_t N, int64_t d) {
  const int T = (int)((d + BT - 1) / BT);
  const int ntiles = T * (T + 1) / 2;
  int64_t rps = 0;
  const int s = pick_splits(ntiles * cn, N, d, &rps);
  return s > 1 ? (size_t)cn * s * ntiles * kTileBytes : 0;
}

static size_t hess_ws_need(int count, int x_dtype, int64_t N, int64_t d) {
  if (N <= 0 || d <= 0 || count <= 0) return 0;
  if (x_dtype == 0) {
    int64_t rps = 0;
    const int s = f32_splits(N, d, &rps);
    return s > 1 ? (size_t)s * d * d * sizeof(float) : 0;  // jobs run one after another
  }
  size_t need = bf16_ws(count < kHessJobs ? count : kHessJobs, N, d);
  if (count > kHessJobs && count % kHessJobs) {
    const size_t tail = bf16_ws(count % kHessJobs, N, d);
    if (tail > need) need = tail;
  }
  return need;
}

}  // namespace cp

namespace cp {

// H_z += X_z^T X_z for count jobs of one shape, bf16 X.
static int hess_bf16_batch(const void* const* X, float* const* H, int count, int64_t N, int64_t d,
                           void* ws, size_t ws_bytes, hipStream_t st) {
  const int T = (int)((d + BT - 1) / BT);
  const int ntiles = T * (T + 1) / 2;
  for (int c0 = 0; c0 < count; c0 += kHessJobs) {
    const int cn = count - c0 < kHessJobs ? count - c0 : kHessJobs;
    HessJobs jobs;
    for (int i = 0; i < cn; ++i) {
      if (!X[c0 + i] || !H[c0 + i]) return set_error(CP_ERR_ARG, "job %d: null X/H", c0 + i);
      if (!aligned(X[c0 + i], 16) || !aligned(H[c0 + i], 4))
        return set_error(CP_ERR_ALIGN, "job %d: X needs 16-byte alignment", c0 + i);
      jobs.X[i] = (const uint16_t*)X[c0 + i];
      jobs.H[i] = H[c0 + i];
    }
    int64_t rps = 0;
    const int splits = pick_splits(ntiles * cn, N, d, &rps);
    if (splits == 0 || (int64_t)ntiles * cn * splits * 8 > INT32_MAX)
      return set_error(CP_ERR_SHAPE, "X [%lld, %lld] too large for one accumulation; pass fewer rows",
                       (long long)N, (long long)d);
    float* part = nullptr;
    if (splits > 1) {
      const size_t need = (size_t)cn * splits * ntiles * kTileBytes;
      if (!ws || ws_bytes < need)
        return set_error(CP_ERR_WORKSPACE, "Hessian workspace: need %zu bytes, have %zu", need, ws_bytes);
      if (!aligned(ws, 16)) return set_error(CP_ERR_ALIGN, "Hessian workspace needs 16-byte alignment");
      part = (float*)ws;
    }
    const int total = ntiles * splits * cn;
    const int per = (total + 7) / 8;
    hess_bf16_tri_kernel<<<dim3(8 * per), HNT, 0, st>>>(jobs, cn, N, (int)d, ntiles, splits, rps, part);
    CP_LAUNCHED("hessian launch");
    const int tb = (int)((d + 63) / 64);
    hess_tri_reduce_kernel<<<dim3(tb * (tb + 1) / 2, cn), 256, 0, st>>>(jobs, (int)d, ntiles, splits, part);
    CP_LAUNCHED("hessian reduce");
  }
  return CP_OK;
}

static int hess_f32(const float* X, int64_t N, int64_t d, float* H, void* ws, size_t ws_bytes,
                    hipStream_t st) {
  const int tiles = (int)((d + HT - 1) / HT);
  int64_t rps = 0;
  const int splits = f32_splits(N, d, &rps);
  float* part = nullptr;
  if (splits > 1) {
    const size_t need = (size_t)splits * d * d * sizeof(float);
    if (!ws || ws_bytes < need)
      return set_error(CP_ERR_WORKSPACE, "Hessian workspace: need %zu bytes, have %zu", need, ws_bytes);
    part = (float*)ws;
  }
  dim3 grid(tiles, tiles, (unsigned)splits);
  hess_f32_kernel<<<grid, 256, 0, st>>>(X, N, (int)d, rps, H, part);
  CP_LAUNCHED("hessian launch");
  if (part) {
    const int64_t dd = d * d;
    const int64_t blocks = (dd + 255) / 256 < 4096 ? (dd + 255) / 256 : 4096;
    hess_f32_reduce_kernel<<<dim3((unsigned)blocks), 256, 0, st>>>(H, dd, splits, part);
    CP_LAUNCHED("hessian reduce");
  }
  return CP_OK;
}

static int hess_check(int x_dtype, int64_t N, int64_t d) {
  if (N < 0 || d <= 0 || d > (1 << 20)) return set_error(CP_ERR_SHAPE, "bad X shape [%lld, %lld]", (long long)N, (long long)d);
  if (x_dtype != 0 && x_dtype != 1) return set_error(CP_ERR_ARG, "x_dtype must be 0 (f32) or 1 (bf16)");
  if (x_dtype == 1 && d % 8) return set_error(CP_ERR_SHAPE, "bf16 X needs d %% 8 == 0 (got %lld)", (long long)d);
  return CP_OK;
}

static int hess_run(const void* const* X, float* const* H, int count, int x_dtype, int64_t N,
                    int64_t d, void* ws, size_t ws_bytes, hipStream_t st) {
  if (x_dtype == 1) return hess_bf16_batch(X, H, count, N, d, ws, ws_bytes, st);
  for (int i = 0; i < count; ++i) {
    if (!X[i] || !H[i]) return set_error(CP_ERR_ARG, "job %d: null X/H", i);
    if (!aligned(X[i], 16) || !aligned(H[i], 4)) return set_error(CP_ERR_ALIGN, "job %d: misaligned", i);
    if (int s = hess_f32((const float*)X[i], N, d, H[i], ws, ws_bytes, st)) return s;
  }
  return CP_OK;
}

// hess_run with a stream-ordered workspace of its own, freed on the stream after
// the last launch that reads it.
static int hess_run_alloc(const void* const* X, float* const* H, int count, int x_dtype, int64_t N,
                          int64_t d, hipStream_t st) {
  const size_t need = hess_ws_need(count, x_dtype, N, d);
  void* ws = nullptr;
  if (need) CP_HIP(hipMallocAsync(&ws, need, st));
  const int s = hess_run(X, H, count, x_dtype, N, d, ws, need, st);
  if (ws) {
    const hipError_t e = hipFreeAsync(ws, st);
    if (s == CP_OK && e != hipSuccess) return hip_fail(e, "hipFreeAsync");
  }
  return s;
}

}  // namespace cp

extern "C" size_t cp_hess_ws_bytes(int count, int x_dtype, int64_t N, int64_t d) {
  return cp::hess_ws_need(count, x_dtype, N, d);
}

extern "C" int cp_hess_accum(const void* X, int x_dtype, int64_t N, int64_t d, float* H, void* stream) {
  cp::clear_error();
  if (int s = cp::hess_check(x_dtype, N, d)) return s;
  if (!H) return cp::set_error(CP_ERR_ARG, "null H");
  if (N == 0) return CP_OK;  // no rows: H += 0
  if (!X) return cp::set_error(CP_ERR_ARG, "null X");
  return cp::hess_run_alloc(&X, &H, 1, x_dtype, N, d, (hipStream_t)stream);
}

extern "C" int cp_hess_accum_batch(const void* const* X, float* const* H, int count, int x_dtype,
                                   int64_t N, int64_t d, void* stream) {
  cp::clear_error();
  if (!X || !H || count <= 0) return cp::set_error(CP_ERR_ARG, "no jobs");
  if (int s = cp::hess_check(x_dtype, N, d)) return s;
  if (N == 0) return CP_OK;  // no rows: every H += 0
  return cp::hess_run_alloc(X, H, count, x_dtype, N, d, (hipStream_t)stream);
}

extern "C" int cp_hess_accum_batch_ws(const void* const* X, float* const* H, int count, int x_dtype,
                                      int64_t N, int64_t d, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  if (!X || !H || count <= 0) return cp::set_error(CP_ERR_ARG, "no jobs");
  if (int s = cp::hess_check(x_dtype, N, d)) return s;
  if (N == 0) return CP_OK;  // no rows: every H += 0
  return cp::hess_run(X, H, count, x_dtype, N, d, ws, ws_bytes, (hipStream_t)stream);
}
