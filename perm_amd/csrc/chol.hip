// Damped inverse-Hessian upper factor in fp64 on gfx950 (coldpress/ef.py:46-84,
// with the act_order permutation of ef.py:187-189 applied first).
//
// The reference computes U = chol(inv(H + lambda I))^T with LAPACK (dgesv, then
// dpotrf). The same U -- the unique upper-triangular factor with positive
// diagonal and U^T U = inv(Hd) -- is reached here without forming inv(Hd):
// with J the index reversal, J Hd J = L L^T (lower Cholesky) gives
// Hd = (J L J)(J L J)^T, so U = (J L J)^{-1} = J L^{-1} J. Work: n^3/3 for the
// Cholesky plus n^3/3 for the triangular inverse.
//
//  * the act_order gather, the reversal and the damping shift fuse into one
//    pass over H (fact_prepare);
//  * Cholesky is left-looking in two levels: a 256-wide block column first
//    receives the updates of everything to its left in two large-K fp64 MFMA
//    GEMMs (wide enough in N to fill the GPU): the columns up to its left
//    neighbour, queued one block column ahead (on a second stream for small
//    batches), then the neighbour's 256. Inside it each 64-wide column takes
//    its left neighbours' updates, then its diagonal block is factored by
//    four waves in registers and inverted by blocked doubling, and the panel
//    below it is a GEMM with that inverse;
//  * L^{-1} is assembled by recursive doubling: diagonal 64-blocks come from
//    the panel step, then at block size s, X21 = -X22 (L21 X11) for every pair
//    of neighbouring s-blocks -- two batched fp64 MFMA GEMMs per level that
//    skip the all-zero K blocks of their triangular operand;
//  * a non-positive (or NaN) pivot raises a per-matrix flag; the host reads
//    the flags and re-runs failed matrices with damp x 10, up to max_tries
//    attempts, as the reference does.
//
// All matrices of a call share one size n and are batched over blockIdx.z.
#include <hip/hip_runtime.h>

#include <cmath>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "cp_host.h"

namespace cp {

typedef double dbl4 __attribute__((ext_vector_type(4)));

constexpr int NB = 64;   // diagonal block and panel width
constexpr int NW = 256;  // outer block-column width of the left-looking sweep
constexpr int CHUNK_N = 8192;  // n from which outer updates sum K in chunks of KC
constexpr int KC = 1024;

// ---------------------------------------------------------------- fp64 MFMA GEMM
// C[M,N] = alpha * A[M,K] * op(B) + beta * C, row-major with leading dims.
// op(B) = B [K,N] or, with BT, B^T for B stored [N,K]. Batched over blockIdx.z
// as z = z1 * nz2 + z2 with separate strides per level.
//
// Block tile 64 x 64 or 128 x 128, K tile 16, 4 waves each building a 64-column
// slab from v_mfma_f64_16x16x4f64: stacked along M for 64 x 64 (16 x 64 each), a
// 2 x 2 grid for 128 x 128 (64 x 64 each, half the LDS fragment reads per MFMA of
// the stacked form). The next K tile is fetched into
// registers while the current one is multiplied, then stored into the other half
// of a double-buffered LDS, so one barrier separates K tiles. The operands of one
// MFMA step s are read from LDS just before its MFMAs, which keeps the 128 x 128
// tile at two waves per SIMD (its 64 accumulator doubles per lane take half the
// register file). Within a K tile, lane group g = lane/16 supplies k = 4g + s to
// MFMA step s (the MFMA sums over g, and any fixed assignment of the 16 k values
// to (g, s) gives the same sum of products).
//
// tri: bit 0 -- A is lower triangular (A[r][k] = 0 for k > r), so row tile bm
// only needs k < bm + BM; bit 1 -- B ([K,N], not transposed) is lower
// triangular (B[k][c] = 0 for k < c), so column tile bn needs k >= bn; bit 2 --
// C above the diagonal is not wanted, so tiles entirely above it are skipped.
// The skipped K ranges are multiplied in at K-tile granularity, so the zeros of
// a triangular operand must be stored.
struct GemmArgs {
  const double* A;
  const double* B;
  double* C;
  int M, N, K, lda, ldb, ldc;
  double alpha, beta;
  int64_t sA1, sB1, sC1, sA2, sB2, sC2;
  int nz2;
  int tri;
  int kc;              // > 0: batch index z2 picks the K range [z2 * kc, z2 * kc + kc)
  int ntx, nty, nzt;  // block grid: column tiles, row tiles, batch entries (set by dgemm())
  int fold;           // 1: grid row by also takes row tile rt - 1 - by; 2: the same for columns
  int rt, ct;         // row and column tiles of the product (set by dgemm())
};

// Block -> tile: items run matrix by matrix, then by groups of 8 row tiles,
// column by column, row by row within a group. The hardware places block w on
// XCD w % 8, so item = (w % 8) * per + w / 8 gives every XCD a contiguous run
// of items, and the ~64 blocks resident on an XCD share 8 row tiles of A and
// 8 column tiles of B through its L2 instead of each fetching its own.
__device__ __forceinline__ bool gemm_tile(const GemmArgs& g, int& bx, int& by, int& bz) {
  const int total = g.ntx * g.nty * g.nzt;
  const int per = (total + 7) / 8;
  const int t = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (t >= total) return false;
  const int T = g.ntx * g.nty;
  bz = t / T;
  const int r = t - bz * T;
  const int rg = r / (8 * g.ntx);
  const int gy = min(8, g.nty - rg * 8);
  const int rem = r - rg * 8 * g.ntx;
  bx = rem / gy;
  by = rg * 8 + rem % gy;
  return true;
}

constexpr int GBK = 16;       // K tile
constexpr int GLD = GBK + 2;  // LDS row of a [rows][K] tile: 144 B, fragment reads conflict-free

// p[0], p[1] at column indices c, c + 1, zero where the row is out of range
// (!ok) or the column reaches lim. VEC: p is 16-byte aligned.
template <bool VEC>
__device__ inline double2 ld_pair(const double* p, bool ok, int c, int lim) {
  double2 v;
  if (VEC && ok && c + 1 < lim) {
    v = *reinterpret_cast<const double2*>(p);
  } else {
    v.x = (ok && c < lim) ? p[0] : 0.0;
    v.y = (ok && c + 1 < lim) ? p[1] : 0.0;
  }
  return v;
}

// The block's LDS: double-buffered A and B K tiles.
template <bool BT, int BM, int BN>
struct GemmLds {
  static constexpr int BROWS = BT ? BN : GBK;
  static constexpr int BLD = BT ? GLD : BN + 4;
  double As[2][BM][GLD];
  double Bs[2][BROWS][BLD];
};

// One block's tile (bx, by) of matrix bz (and its mirror when the grid folds).
template <bool BT, int BM, int BN, bool VEC>
__device__ __forceinline__ void dgemm_block(const GemmArgs& g, int bx, int by, int bz,
                                            GemmLds<BT, BM, BN>& lds) {
  // waves: stacked along M for BN = 64 (each BM/4 x 64), a 2 x 2 grid for BN = 128
  // (each BM/2 x 64); fragments of one MFMA step s are read from LDS at a time
  constexpr int WN = BN / 64;
  constexpr int WM = 4 / WN;
  constexpr int TI = BM / WM / 16;  // 16-row MFMA tiles per wave
  constexpr int TJ = 4;             // 16-column MFMA tiles per wave (64 columns)
  constexpr int AQ = BM / 32;  // A-tile pairs fetched per thread
  constexpr int BQ = BN / 32;  // B-tile pairs fetched per thread
  auto& As = lds.As;
  auto& Bs = lds.Bs;
  const int z1 = bz / g.nz2, z2 = bz % g.nz2;
  const double* A = g.A + z1 * g.sA1 + z2 * g.sA2;
  const double* B = g.B + z1 * g.sB1 + z2 * g.sB2;
  double* C = g.C + z1 * g.sC1 + z2 * g.sC2;
  const int t = threadIdx.x, l = t & 63, w = t >> 6;
  const int wm = (w % WM) * (BM / WM), wn = (w / WM) * 64;
  const int lr = l & 15, lg = l >> 4;
  const int tr = t >> 3, tk = (t & 7) * 2;
  const int nr = t / (BN / 2), nc = (t % (BN / 2)) * 2;
  // A triangular operand makes a tile's K range grow with its row (tri & 1) or shrink
  // with its column (tri & 2). The block then takes a tile and its mirror, whose ranges
  // add up to the same length for every block, so no long tile is left running alone
  // at the end of the grid.
  const int mir = g.fold == 1 ? g.rt - 1 - by : (g.fold == 2 ? g.ct - 1 - bx : -1);
  const int np = mir >= 0 && mir != (g.fold == 1 ? by : bx) ? 2 : 1;
#pragma unroll 1
  for (int p = 0; p < np; ++p) {
    const int bm = (p && g.fold == 1 ? mir : by) * BM;
    const int bn = (p && g.fold == 2 ? mir : bx) * BN;
    if ((g.tri & 4) && bn >= bm + BM) continue;

    dbl4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j) acc[i][j] = dbl4{0.0, 0.0, 0.0, 0.0};

    int kbeg = (g.tri & 2) ? (bn & ~(GBK - 1)) : 0;
    int kend = (g.tri & 1) ? min(g.K, bm + BM) : g.K;
    if (g.kc > 0) {
      kbeg = max(kbeg, z2 * g.kc);
      kend = min(kend, z2 * g.kc + g.kc);
    }
    // columns at or past klim load as zero: K's end, or the end of this block's chunk
    const int klim = g.kc > 0 ? kend : g.K;
    const int nt = kend > kbeg ? (kend - kbeg + GBK - 1) / GBK : 0;

    double2 ra[AQ], rb[BQ];
    auto fetch = [&](int k0) {
#pragma unroll
      for (int q = 0; q < AQ; ++q) {
        const int r = bm + tr + 32 * q;
        ra[q] = ld_pair<VEC>(A + (int64_t)r * g.lda + k0 + tk, r < g.M, k0 + tk, klim);
      }
#pragma unroll
      for (int q = 0; q < BQ; ++q) {
        if (BT) {
          const int r = bn + tr + 32 * q;
          rb[q] = ld_pair<VEC>(B + (int64_t)r * g.ldb + k0 + tk, r < g.N, k0 + tk, klim);
        } else {
          const int k = k0 + nr + (512 / BN) * q;
          rb[q] = ld_pair<VEC>(B + (int64_t)k * g.ldb + bn + nc, k < klim, bn + nc, g.N);
        }
      }
    };
    auto stash = [&](int b) {
#pragma unroll
      for (int q = 0; q < AQ; ++q) *reinterpret_cast<double2*>(&As[b][tr + 32 * q][tk]) = ra[q];
#pragma unroll
      for (int q = 0; q < BQ; ++q) {
        if (BT)
          *reinterpret_cast<double2*>(&Bs[b][tr + 32 * q][tk]) = rb[q];
        else
          *reinterpret_cast<double2*>(&Bs[b][nr + (512 / BN) * q][nc]) = rb[q];
      }
    };

    // the previous tile's last K step ended with a barrier, so its LDS reads are done
    if (nt > 0) {
      fetch(kbeg);
      stash(0);
    }
    __syncthreads();
    for (int it = 0; it < nt; ++it) {
      const int b = it & 1;
      if (it + 1 < nt) fetch(kbeg + (it + 1) * GBK);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        double af[TI], bf[TJ];
#pragma unroll
        for (int ti = 0; ti < TI; ++ti) af[ti] = As[b][wm + 16 * ti + lr][4 * lg + s];
#pragma unroll
        for (int tj = 0; tj < TJ; ++tj)
          bf[tj] = BT ? Bs[b][wn + 16 * tj + lr][4 * lg + s] : Bs[b][4 * lg + s][wn + 16 * tj + lr];
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
          for (int tj = 0; tj < TJ; ++tj)
            acc[ti][tj] = __builtin_amdgcn_mfma_f64_16x16x4f64(af[ti], bf[tj], acc[ti][tj], 0, 0, 0);
      }
      if (it + 1 < nt) stash(b ^ 1);
      __syncthreads();
    }
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
      for (int tj = 0; tj < TJ; ++tj)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          // v_mfma_f64_16x16x4f64 result: register r of lane l holds row 4r + l/16, column l%16
          const int i = bm + wm + 16 * ti + 4 * r + lg;
          const int j = bn + wn + 16 * tj + lr;
          if (i < g.M && j < g.N) {
            double* q = C + (int64_t)i * g.ldc + j;
            const double v = g.alpha * acc[ti][tj][r];
            *q = g.beta == 0.0 ? v : v + g.beta * *q;
          }
        }
  }
}

template <bool BT, int BM, int BN, bool VEC>
__global__ __launch_bounds__(256, 2) void dgemm_kernel(GemmArgs g) {
  __shared__ __align__(16) GemmLds<BT, BM, BN> lds;
  int bx, by, bz;
  if (!gemm_tile(g, bx, by, bz)) return;
  dgemm_block<BT, BM, BN, VEC>(g, bx, by, bz, lds);
}

template <bool BT, int BM, int BN>
static void launch_gemm(const GemmArgs& a, dim3 grid, bool vec, hipStream_t st) {
  if (vec)
    dgemm_kernel<BT, BM, BN, true><<<grid, 256, 0, st>>>(a);
  else
    dgemm_kernel<BT, BM, BN, false><<<grid, 256, 0, st>>>(a);
}

// every (z1, z2) base of the operand is 16-byte aligned and so are its rows
static bool pairs_aligned(const double* p, int ld, int64_t s1, int64_t s2) {
  return aligned(p, 16) && !(ld & 1) && !(s1 & 1) && !(s2 & 1);
}

// The calling thread's GEMM tile policy (cp_chol_compact_tiles): 0 picks the fastest tile
// for a GPU the factorization has to itself; 1 keeps every GEMM at 64 x 64, whose blocks
// (112 VGPRs, 36 KB of LDS) fit on a CU beside two EF sweep waves per SIMD, where the
// 128 x 128 tile (234-256 VGPRs, 69-72 KB) waits for whole CUs to drain.
static thread_local int g_compact_tiles = 0;

// Fused chain steps for calls of at most this many matrices, and the bounded wait of a
// panel item for its diagonal block (sleeps of about 512 clocks; cp_chol_wait_limit).
constexpr int kFusedBatch = 4;
constexpr int kDefaultCholWait = 1 << 16;
static thread_local int g_chol_wait_limit = kDefaultCholWait;

static int dgemm(const GemmArgs& a0, int nz1, bool bt, hipStream_t st) {
  if (a0.M <= 0 || a0.N <= 0 || nz1 <= 0) return CP_OK;
  const bool vec = pairs_aligned(a0.A, a0.lda, a0.sA1, a0.sA2) &&
                   pairs_aligned(a0.B, a0.ldb, a0.sB1, a0.sB2);
  // 64 x 64 tiles: 112 VGPRs and 36 KB of LDS let four blocks (16 waves) share a CU,
  // which hides the loads and barriers of short K loops better than two 128 x 128
  // blocks do. 128 x 128 tiles only for K >= 4096 with at least 512 of them (two per
  // CU): there the larger tile's lower L2 traffic per MFMA wins.
  // A triangular operand folds the grid: a block takes a tile and its mirror.
  const int64_t z = (int64_t)nz1 * a0.nz2;
  const int fold = (a0.tri & 1) ? 1 : ((a0.tri & 2) ? 2 : 0);
  auto blocks = [&](int tm, int tn) {
    const int64_t r = (a0.M + tm - 1) / tm, c = (a0.N + tn - 1) / tn;
    return (fold == 1 ? (r + 1) / 2 : r) * (fold == 2 ? (c + 1) / 2 : c) * z;
  };
  const int kblock = a0.kc > 0 ? min(a0.kc, a0.K) : a0.K;  // K of one block's loop
  const bool wide = !g_compact_tiles && a0.M >= 128 && a0.N >= 128 && kblock >= 4096 &&
                    blocks(128, 128) >= 512;
  const int bm = wide ? 128 : 64, bn = bm;
  GemmArgs a = a0;
  a.fold = fold;
  a.ct = (a.N + bn - 1) / bn;
  a.rt = (a.M + bm - 1) / bm;
  a.ntx = fold == 2 ? (a.ct + 1) / 2 : a.ct;
  a.nty = fold == 1 ? (a.rt + 1) / 2 : a.rt;
  a.nzt = (int)z;
  const int64_t total = (int64_t)a.ntx * a.nty * a.nzt;
  if (total > (int64_t)1 << 30) return set_error(CP_ERR_SHAPE, "fp64 GEMM grid too large");
  const dim3 grid((unsigned)(8 * ((total + 7) / 8)));
  if (bt)
    wide ? launch_gemm<true, 128, 128>(a, grid, vec, st) : launch_gemm<true, 64, 64>(a, grid, vec, st);
  else
    wide ? launch_gemm<false, 128, 128>(a, grid, vec, st) : launch_gemm<false, 64, 64>(a, grid, vec, st);
  CP_LAUNCHED("fp64 GEMM launch");
  return CP_OK;
}

// ---------------------------------------------------------------- prepare
// An order entry taken into [0, n): a caller's order that is not a permutation is
// flagged by fact_shift_kernel and must never address memory outside H.
__device__ inline int clamp_index(int p, int n) { return p < 0 ? 0 : (p >= n ? n - 1 : p); }

// numpy's pairwise float64 sum of a strided vector (same recursion as the
// float32 one: 8 accumulators up to 128 elements, halving split above).
__device__ double pw_sum_f64(const double* a, int n, int stride) {
  if (n < 8) {
    double s = 0.0;
    for (int i = 0; i < n; ++i) s = s + a[(int64_t)i * stride];
    return s;
  }
  if (n <= 128) {
    double r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[(int64_t)j * stride];
    int i = 8;
    for (; i < n - (n % 8); i += 8)
      for (int j = 0; j < 8; ++j) r[j] = r[j] + a[(int64_t)(i + j) * stride];
    double s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) s = s + a[(int64_t)i * stride];
    return s;
  }
  int n2 = n / 2;
  n2 -= n2 % 8;
  return pw_sum_f64(a, n2, stride) + pw_sum_f64(a + (int64_t)n2 * stride, n - n2, stride);
}

// numpy reduces a float64 vector in chunks of 8192 values (its ufunc buffer
// size): the pairwise recursion runs inside each chunk, and the chunk sums are
// added left to right onto +0.0. This holds for contiguous and strided inputs
// alike (np.diag(H) is a strided view).
constexpr int kNpChunk = 8192;

// Leaves of numpy's pairwise sum over n values, chunk by chunk and in order:
// inside a chunk the recursion above splits until a piece has at most 128
// values. Returns the leaf count (at most max_leaves written).
__device__ int pw_leaves(int n, int max_leaves, int* off, int* len) {
  int k = 0;
  for (int c0 = 0; c0 < n; c0 += kNpChunk) {
    int stack_off[32], stack_len[32], sp = 0;
    stack_off[sp] = c0;
    stack_len[sp++] = min(kNpChunk, n - c0);
    while (sp > 0) {
      --sp;
      const int o = stack_off[sp], m = stack_len[sp];
      if (m <= 128) {
        if (k < max_leaves) {
          off[k] = o;
          len[k] = m;
        }
        ++k;
        continue;
      }
      int m2 = m / 2;
      m2 -= m2 % 8;
      stack_off[sp] = o + m2;  // right piece below the left one: leaves come out in order
      stack_len[sp++] = m - m2;
      stack_off[sp] = o;
      stack_len[sp++] = m2;
    }
  }
  return k;
}

// One chunk's pairwise tree combined from its leaf sums, in the recursion's order.
__device__ double pw_combine(int n, const double* leaf, int& k) {
  if (n <= 128) return leaf[k++];
  int n2 = n / 2;
  n2 -= n2 % 8;
  const double a = pw_combine(n2, leaf, k);
  return a + pw_combine(n - n2, leaf, k);
}

// np.add.reduce of n float64 values from their leaf sums: chunk trees added in order.
__device__ double np_sum_from_leaves(int n, const double* leaf) {
  double total = 0.0;
  int k = 0;
  for (int c0 = 0; c0 < n; c0 += kNpChunk) total = total + pw_combine(min(kNpChunk, n - c0), leaf, k);
  return total;
}

// np.add.reduce of n float64 values, serially.
__device__ double np_sum_f64(const double* a, int n) {
  double total = 0.0;
  for (int c0 = 0; c0 < n; c0 += kNpChunk) total = total + pw_sum_f64(a + c0, min(kNpChunk, n - c0), 1);
  return total;
}

constexpr int kShiftLeaves = 1024;  // pairwise leaves summed in parallel (n <= 131072)

// Diagonal of the act-ordered H in visiting order, then the damping shift
// damp * mean + 1e-8 (mean replaced by 1 when not positive), as ef.py:64-69
// computes it from np.mean(np.diag(Hp)). One block per matrix: the leaves of
// the chunked pairwise sum run on separate threads, then one thread combines
// them in numpy's order (same additions, same order as the serial sum).
//
// The order is checked here as well: an entry outside [0, n) or a repeated one sets
// bit 2 of fail[z] (marks: n ints of scratch per matrix, cleared here). Every
// kernel of the factorization clamps the order's entries, so a bad order never
// reads outside H.
template <typename T>
__global__ __launch_bounds__(256) void fact_shift_kernel(const T* H, int n, int64_t sH,
                                                         const int* order, int64_t sO,
                                                         const double* damp, double* diag_tmp,
                                                         double* shift, const int* active,
                                                         int* marks, int64_t sM, int* fail) {
  __shared__ int loff[kShiftLeaves], llen[kShiftLeaves];
  __shared__ double lsum[kShiftLeaves];
  __shared__ int nleaves, bad_order;
  const int z = blockIdx.x;
  if (active && !active[z]) return;
  const T* h = H + z * sH;
  const int* o = order ? order + z * sO : nullptr;
  double* dg = diag_tmp + (int64_t)z * n;
  if (threadIdx.x == 0) bad_order = 0;
  if (o) {
    int* mk = marks + z * sM;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mk[i] = 0;
    __syncthreads();
    int bad = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int p = o[i];
      if ((unsigned)p >= (unsigned)n) bad = 1;
      else if (atomicExch(&mk[p], 1)) bad = 1;
    }
    if (bad) atomicOr(&bad_order, 1);
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int p = o ? clamp_index(o[i], n) : i;
    dg[i] = (double)h[(int64_t)p * n + p];
  }
  if (threadIdx.x == 0) nleaves = pw_leaves(n, kShiftLeaves, loff, llen);
  __syncthreads();
  if (threadIdx.x == 0 && bad_order) fail[z] |= 2;
  const int nl = nleaves;
  if (nl <= kShiftLeaves) {
    for (int k = threadIdx.x; k < nl; k += blockDim.x) lsum[k] = pw_sum_f64(dg + loff[k], llen[k], 1);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    double total;
    if (nl <= kShiftLeaves)
      total = np_sum_from_leaves(n, lsum);
    else
      total = np_sum_f64(dg, n);
    const double mean = total / (double)n;
    const double base = mean > 0.0 ? mean : 1.0;
    shift[z] = damp[z] * base + 1e-8;
  }
}

// A[i][j] = H[q_i][q_j] (+ shift on the diagonal) for i >= j, with
// q_i = order[n-1-i]: the act_order gather and the index reversal in one pass.
// Entries above the diagonal are not written: every reader of A takes the lower
// triangle only (the Cholesky GEMMs' operands lie strictly below the diagonal,
// the diagonal-block kernel loads i <= r and stores its own zeros, and the outer
// updates already change the upper part of the tiles they straddle).
// Element-wise form, for rows too long to stage.
template <typename T>
__global__ void fact_prepare_gather_kernel(const T* H, int n, int64_t sH, const int* order,
                                           int64_t sO, const double* shift, double* A, int64_t sA,
                                           const int* active) {
  const int z = blockIdx.z;
  if (active && !active[z]) return;
  const int j = blockIdx.x * 64 + (threadIdx.x & 63);
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= n || j >= n) return;
  if (j > i) return;
  double* a = A + z * sA;
  const int* o = order ? order + z * sO : nullptr;
  int qi = o ? clamp_index(o[n - 1 - i], n) : n - 1 - i;
  int qj = o ? clamp_index(o[n - 1 - j], n) : n - 1 - j;
  double v = (double)H[z * sH + (int64_t)qi * n + qj];
  if (i == j) v = v + shift[z];
  a[(int64_t)i * n + j] = v;
}

// The same with rows staged: a block copies rows q_i of R consecutive rows i into LDS
// (read whole, coalesced), then writes the R rows of A from there.
template <typename T>
__global__ __launch_bounds__(256) void fact_prepare_kernel(const T* H, int n, int64_t sH,
                                                           const int* order, int64_t sO,
                                                           const double* shift, double* A,
                                                           int64_t sA, const int* active, int R) {
  extern __shared__ __align__(16) char prep_lds[];
  T* rows = reinterpret_cast<T*>(prep_lds);
  const int z = blockIdx.y;
  if (active && !active[z]) return;
  const int i0 = blockIdx.x * R;
  const int* o = order ? order + z * sO : nullptr;
  const T* h = H + z * sH;
  const int rows_here = min(R, n - i0);
  // stage the block's source rows: every load of a batch is issued before the LDS
  // stores that consume it (16-byte loads when rows are 16-byte aligned)
  constexpr int V = 16 / sizeof(T), B = 4;
  const bool vec = (n % V) == 0 && (reinterpret_cast<uintptr_t>(h) % 16) == 0;
  for (int r = 0; r < rows_here; ++r) {
    const int qi = o ? clamp_index(o[n - 1 - (i0 + r)], n) : n - 1 - (i0 + r);
    const T* src = h + (int64_t)qi * n;
    T* dst = rows + (int64_t)r * n;
    if (vec) {
      const uint4* s4 = reinterpret_cast<const uint4*>(src);
      uint4* d4 = reinterpret_cast<uint4*>(dst);
      const int nv = n / V;
      for (int c0 = threadIdx.x; c0 < nv; c0 += B * blockDim.x) {
        uint4 t[B];
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const int c = c0 + b * blockDim.x;
          if (c < nv) t[b] = s4[c];
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
          const int c = c0 + b * blockDim.x;
          if (c < nv) d4[c] = t[b];
        }
      }
    } else {
      for (int c = threadIdx.x; c < n; c += blockDim.x) dst[c] = src[c];
    }
  }
  __syncthreads();
  double* a = A + z * sA;
  const int jend = min(n, i0 + R);  // columns up to the block's last row
  for (int j0 = threadIdx.x; j0 < jend; j0 += B * blockDim.x) {
    int qj[B];  // the batch's column indices, loaded before any of them is used
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int j = j0 + b * blockDim.x;
      qj[b] = j < jend ? (o ? clamp_index(o[n - 1 - j], n) : n - 1 - j) : 0;
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int j = j0 + b * blockDim.x;
      if (j >= jend) continue;
      for (int r = 0; r < rows_here; ++r) {
        const int i = i0 + r;
        if (j <= i) {
          double v = (double)rows[(int64_t)r * n + qj[b]];
          if (j == i) v = v + shift[z];
          a[(int64_t)i * n + j] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- diagonal block
// Factor the nb x nb diagonal block at (k, k) (nb = min(64, n - k)), write L_kk
// back to A and inv(L_kk) into the matching diagonal block of X; flag a bad
// pivot. A partial last block is padded with identity rows.
//
// Four waves per matrix, the block in LDS. Cholesky is blocked by 16-column panels:
// each panel is factored by one wave without barriers and its outer product leaves the
// trailing tiles on the matrix cores (diag_block). Entries above the diagonal collect
// finite garbage on the way and are never stored. The inverse is blocked doubling:
// each wave inverts one 16 x 16 diagonal block by forward substitution (lane c solves
// column c, no exchange between lanes), then two levels of X21 = -X22 (L21 X11) on
// v_mfma_f64_16x16x4f64 join them into 32 x 32 and 64 x 64: three barriers where a
// column-by-column inverse needs 64.
__device__ inline double readlane_f64(double v, int lane) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, lane);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), lane);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}

struct DiagLds {
  double L[NB][NB + 1];
};

__device__ __forceinline__ void diag_block(double* A, int64_t sA, double* X, int64_t sX, int n, int k,
                                           int* fail, int z, DiagLds& lds) {
  auto& L = lds.L;
  const int nb = min(NB, n - k);
  double* Ak = A + z * sA + (int64_t)k * n + k;
  double* Xk = X + z * sX + (int64_t)k * n + k;
  const int t = threadIdx.x, i = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  {
    double v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int r = 4 * q + w;
      v[q] = r == i ? 1.0 : 0.0;
      if (r < nb && i < nb && i <= r) v[q] = Ak[(int64_t)r * n + i];
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) L[4 * q + w][i] = v[q];
  }
  __syncthreads();

  // Blocked Cholesky over four 16-column panels. Panel q is factored by wave q alone (lane
  // i = row i, the panel's columns in registers, right-looking inside the panel, no
  // barrier between its pivots); then the four waves subtract the panel's outer product
  // from the 16 x 16 tiles of the lower triangle to its right on the matrix cores (four
  // v_mfma_f64_16x16x4f64 per tile). Each finished column goes to L at once: the next
  // column takes its multiplier L[c + 1][c] by readlane (the pivot chain), the later
  // columns read theirs from LDS as broadcasts, off the chain. A pivot's chain is its
  // reciprocal square root (v_rsq_f64 and one Newton step) and the column scale; the
  // diagonal itself is the IEEE square root of the pivot, taken once per panel for all
  // its rows, so a diagonal H still gives U = 1 / sqrt(h + shift) with correctly rounded
  // operations (the inverse divides by it).
  int bad = 0;
  const int lr = i & 15, lg = i >> 4;
#pragma unroll 1
  for (int q = 0; q < 4; ++q) {
    if (w == q) {
      double a[16];
#pragma unroll
      for (int m = 0; m < 16; ++m) a[m] = L[i][16 * q + m];
      double pv = 1.0;  // this lane's pivot, for the rows of the panel
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        const int c = 16 * q + m;
        const double piv = readlane_f64(a[m], c);
        bad |= !(piv > 0.0);
        const double p = piv > 0.0 ? piv : 1.0;
        const double r0 = __builtin_amdgcn_rsq(p);
        const double r = __builtin_fma(r0, __builtin_fma(-0.5 * p * r0, r0, 0.5), r0);
        pv = i == c ? p : pv;
        a[m] = i > c ? a[m] * r : 0.0;
        L[i][c] = a[m];
        if (m + 1 < 16) a[m + 1] = __builtin_fma(-a[m], readlane_f64(a[m], c + 1), a[m + 1]);
#pragma unroll
        for (int m2 = m + 2; m2 < 16; ++m2) a[m2] = __builtin_fma(-a[m], L[16 * q + m2][c], a[m2]);
      }
      const int mi = i - 16 * q;  // the panel's diagonal: the square root of each row's pivot
      if (mi >= 0 && mi < 16) L[i][i] = sqrt(pv);
    }
    __syncthreads();
    // the tiles (I, J), q < J <= I < 4, of the trailing lower triangle, round robin over the
    // waves: C -= P_I P_J^T with P the panel's rows. In v_mfma_f64_16x16x4f64 lane l gives
    // A[l % 16][l / 16] and B[l / 16][l % 16]; result register e holds row 4 e + l / 16,
    // column l % 16.
    const int T = 3 - q;
    for (int tile = w; tile < T * (T + 1) / 2; tile += 4) {
      int I = q + 1, J = q + 1, left = tile;
      while (left > I - q - 1) {  // row I holds I - q tiles
        left -= I - q;
        ++I;
      }
      J += left;
      dbl4 acc;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = L[16 * I + 4 * e + lg][16 * J + lr];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int kc = 16 * q + 4 * kk + lg;
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(-L[16 * I + lr][kc], L[16 * J + lr][kc], acc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) L[16 * I + 4 * e + lg][16 * J + lr] = acc[e];
    }
    __syncthreads();
  }

  // inv(L_kk) by blocked doubling. X = inv(L_kk) shares the LDS array with L: X[r][c]
  // (c <= r) sits at L[c][r + 1], in the strict upper triangle and the padding column,
  // which L does not use.
  auto xget = [&](int r, int c) -> double { return c <= r ? L[c][r + 1] : 0.0; };
  // 1) the four 16 x 16 diagonal blocks, one per wave: lane c < 16 solves column c by
  //    forward substitution, x_r = (e_c[r] - sum_{m<r} L[r][m] x_m) / L[r][r] (the other
  //    lanes compute zeros and store nothing)
  {
    const int o = 16 * w;
    double x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      double v = r == i ? 1.0 : 0.0;
#pragma unroll
      for (int m = 0; m < r; ++m) v = __builtin_fma(-L[o + r][o + m], x[m], v);
      x[r] = v / L[o + r][o + r];
      asm volatile("" :: "v"(x[r]) : "memory");  // x_r before row r + 1's reads
    }
    if (i < 16) {
#pragma unroll
      for (int m = 0; m < 16; ++m)
        if (m >= i) L[o + i][o + m + 1] = x[m];
    }
  }
  __syncthreads();
  // 2) 16 -> 32: for the block pairs at 0 and 32, X21 = -X22 (L21 X11), waves 0 and 2.
  //    In v_mfma_f64_16x16x4f64, lane l gives A[l % 16][k] and B[k][l % 16] with
  //    k = 4 s + l / 16 at step s, and result register q holds row 4 q + l / 16, column
  //    l % 16: so T's register s is the B operand of step s of the second product.
  if (w == 0 || w == 2) {
    const int o0 = 16 * w, o1 = o0 + 16;
    dbl4 tacc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int k = 4 * s4 + lg;
      tacc = __builtin_amdgcn_mfma_f64_16x16x4f64(L[o1 + lr][o0 + k], xget(o0 + k, o0 + lr), tacc,
                                                  0, 0, 0);
    }
    dbl4 xacc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      const int k = 4 * s4 + lg;
      xacc = __builtin_amdgcn_mfma_f64_16x16x4f64(xget(o1 + lr, o1 + k), tacc[s4], xacc, 0, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) L[o0 + lr][o1 + 4 * q + lg + 1] = -xacc[q];
  }
  __syncthreads();
  // 3) 32 -> 64: X21 = -X22 (L21 X11) with 32 x 32 blocks; wave w owns 16 x 16 block
  //    (bi, bj) of each product. T goes where X21 will be stored.
  {
    const int bi = w >> 1, bj = w & 1;
    dbl4 tacc = {0.0, 0.0, 0.0, 0.0};
    for (int bk = bj; bk < 2; ++bk) {  // X11[bk][bj] = 0 for bk < bj
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int k = 16 * bk + 4 * s4 + lg;
        tacc = __builtin_amdgcn_mfma_f64_16x16x4f64(L[32 + 16 * bi + lr][k], xget(k, 16 * bj + lr),
                                                    tacc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) L[16 * bj + lr][33 + 16 * bi + 4 * q + lg] = tacc[q];
    __syncthreads();
    dbl4 xacc = {0.0, 0.0, 0.0, 0.0};
    for (int bk = 0; bk <= bi; ++bk) {  // X22[bi][bk] = 0 for bk > bi
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const int k = 16 * bk + 4 * s4 + lg;
        xacc = __builtin_amdgcn_mfma_f64_16x16x4f64(xget(32 + 16 * bi + lr, 32 + k),
                                                    L[16 * bj + lr][33 + k], xacc, 0, 0, 0);
      }
    }
    __syncthreads();  // every wave has read T
#pragma unroll
    for (int q = 0; q < 4; ++q) L[16 * bj + lr][33 + 16 * bi + 4 * q + lg] = -xacc[q];
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    const int r = 4 * m + w;
    if (r < nb && i < nb) {
      Xk[(int64_t)r * n + i] = i <= r ? L[i][r + 1] : 0.0;
      Ak[(int64_t)r * n + i] = i <= r ? L[r][i] : 0.0;
    }
  }
  if (i == 0 && bad) atomicOr(&fail[z], 1);
}

__global__ __launch_bounds__(256) void fact_diag_kernel(double* A, int64_t sA, double* X,
                                                        int64_t sX, int n, int k, int* fail,
                                                        const int* active) {
  __shared__ DiagLds lds;
  const int z = blockIdx.x;
  if (active && !active[z]) return;
  diag_block(A, sA, X, sX, n, k, fail, z, lds);
}

// ---------------------------------------------------------------- fused chain step
// One 64-column step of the chain in one launch, for calls with few matrices (where the
// chain's short launches leave the GPU idle): the inner update of every 64-row tile of
// the column, the diagonal block, and the panel below it. Work items are handed out by
// a ticket counter, matrix by matrix with the diagonal item first, so an item's diagonal
// block always belongs to a workgroup that has already started. The diagonal item
// updates its tile, factors and inverts it, and publishes the step in done[z] (each
// thread's stores released at agent scope first); a panel item updates its tile, waits
// for that flag (bounded: past wait_limit sleeps it sets bit 2 of fail[z] and goes on,
// so every workgroup ends, and the host reports a timeout), then multiplies by the
// inverse. The tile updates and products are the same block code, with the same
// arguments, as the separate inner-update, diagonal and panel launches, so U does not
// depend on which form ran.
struct FactStep {
  double *A, *X;
  int64_t sA;
  int n, k, k0, step, items;  // items per matrix: the diagonal block and the panel tiles
  int *fail, *done, *tickets;
  const int* active;
  int wait_limit;
};

template <bool VEC>
__global__ __launch_bounds__(256, 2) void fact_step_kernel(FactStep f) {
  __shared__ __align__(16) union {
    GemmLds<true, 64, 64> g;
    DiagLds d;
  } lds;
  __shared__ int s_item;
  if (threadIdx.x == 0) s_item = atomicAdd(&f.tickets[f.step], 1);
  __syncthreads();
  const int item = s_item, z = item / f.items, t = item % f.items;
  if (f.active && !f.active[z]) return;
  const int n = f.n, k = f.k, wk = n - k < NB ? n - k : NB;
  // A[k:, k:k+wk] -= L[k:, k0:k] L[k:k+wk, k0:k]^T, tile t of 64 rows
  const GemmArgs inner{f.A + (int64_t)k * n + f.k0, f.A + (int64_t)k * n + f.k0, f.A + (int64_t)k * n + k,
                       n - k, wk, k - f.k0, n, n, n, -1.0, 1.0, f.sA, f.sA, f.sA, 0, 0, 0, 1, 0};
  if (k > f.k0) {
    dgemm_block<true, 64, 64, VEC>(inner, 0, t, z, lds.g);
    __syncthreads();  // the tile's stores before this workgroup reads it back
  }
  if (t == 0) {
    diag_block(f.A, f.sA, f.X, f.sA, n, k, f.fail, z, lds.d);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(&f.done[z], f.step + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (threadIdx.x == 0) {
    int v = __hip_atomic_load(&f.done[z], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int spins = 0; v <= f.step && spins < f.wait_limit; ++spins) {
      __builtin_amdgcn_s_sleep(8);
      v = __hip_atomic_load(&f.done[z], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (v <= f.step) atomicOr(&f.fail[z], 4);
  }
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // panel: A[k+64:, k:k+64] <- A[k+64:, k:k+64] * inv(L_kk)^T, row tile t - 1
  const int m = n - k - NB;
  const GemmArgs panel{f.A + (int64_t)(k + NB) * n + k, f.X + (int64_t)k * n + k, f.A + (int64_t)(k + NB) * n + k,
                       m, NB, NB, n, n, n, 1.0, 0.0, f.sA, f.sA, f.sA, 0, 0, 0, 1, 0};
  dgemm_block<true, 64, 64, VEC>(panel, 0, t - 1, z, lds.g);
}

// U[i][j] = X[n-1-i][n-1-j] for i <= j, 0 below the diagonal (OutT = float:
// the float32 cast of ef.py:189; OutT = double: cholesky_inv_upper's result).
// A thread takes four consecutive columns of one row. VEC (n a multiple of 4, X, U and
// their strides 16-byte aligned for four elements): the four X values are two 16-byte
// loads (columns n-4-j .. n-1-j of X's row, read in reverse) and the four U values one
// or two 16-byte stores; elements below the diagonal are zeros that read nothing
// (28 x n = 3072: 0.63 -> 0.38 ms against one element per thread).
template <typename OutT, bool VEC>
__global__ __launch_bounds__(256) void fact_output_kernel(const double* X, int64_t sX, int n, OutT* U,
                                                          int64_t sU, const int* active) {
  const int z = blockIdx.z;
  if (active && !active[z]) return;
  const int j = (blockIdx.x * 64 + (threadIdx.x & 63)) * 4;
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= n || j >= n) return;
  const double* x = X + z * sX + (int64_t)(n - 1 - i) * n + (n - 1 - j);  // x[-c]: column j + c
  OutT* u = U + z * sU + (int64_t)i * n + j;
  OutT v[4];
  if (VEC && j >= i) {
    const double2 hi = *reinterpret_cast<const double2*>(x - 1);  // columns j + 1, j
    const double2 lo = *reinterpret_cast<const double2*>(x - 3);  // columns j + 3, j + 2
    v[0] = (OutT)hi.y;
    v[1] = (OutT)hi.x;
    v[2] = (OutT)lo.y;
    v[3] = (OutT)lo.x;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = (i <= j + c && j + c < n) ? (OutT)x[-c] : (OutT)0;
  }
  if (VEC) {
    if constexpr (sizeof(OutT) == 4) {
      *reinterpret_cast<float4*>(u) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      *reinterpret_cast<double2*>(u) = make_double2(v[0], v[1]);
      *reinterpret_cast<double2*>(u + 2) = make_double2(v[2], v[3]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (j + c < n) u[c] = v[c];
  }
}

// C[i][j] -= P[0][i][j], then P[1][i][j], ... P[S-1][i][j], for i >= j (the lower part
// an outer update keeps): the chunk partials of a split outer update, subtracted in the
// order a chunk-by-chunk GEMM would subtract them.
__global__ void fact_chunk_sub_kernel(const double* P, int64_t sP, int64_t sPc, int S, double* C,
                                      int ldc, int64_t sC, int M, int N, const int* active) {
  const int z = blockIdx.z;
  if (active && !active[z]) return;
  const int j = blockIdx.x * 64 + (threadIdx.x & 63);
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= M || j >= N || i < j) return;
  const double* p = P + z * sP + (int64_t)i * N + j;
  double* c = C + z * sC + (int64_t)i * ldc + j;
  double v = *c;
  for (int s = 0; s < S; ++s) v = v - p[s * sPc];
  *c = v;
}

__global__ void fill_kernel(double* p, int64_t count, double v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i < count; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

__global__ void fill_i32_kernel(int* p, int64_t count, int v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = v;
}

// ---------------------------------------------------------------- act order
// order = stable argsort of -diag(H): rank of i = #{j: d_j > d_i} + #{j < i: d_j == d_i}
// among the non-NaN entries; NaN entries come after all of them, by index, where
// numpy's sort places NaN. The ranks are then a permutation for any input.
// STAGE: the block first copies the diagonal into LDS (n * sizeof(T) bytes, dynamic),
// so each diagonal entry leaves HBM once per block instead of once per thread.
template <typename T, bool STAGE>
__global__ __launch_bounds__(256) void act_order_kernel(const T* H, int n, int64_t sH, int* order,
                                                        int64_t sO) {
  extern __shared__ __align__(16) char act_lds[];
  T* dg = reinterpret_cast<T*>(act_lds);
  const int z = blockIdx.y;
  const T* h = H + z * sH;
  if (STAGE) {
    for (int j = threadIdx.x; j < n; j += blockDim.x) dg[j] = h[(int64_t)j * n + j];
    __syncthreads();
  }
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // compared in T: widening to double is monotonic, so the order is the same
  const T di = STAGE ? dg[i] : h[(int64_t)i * n + i];
  const bool nan_i = di != di;
  int rank = 0;
#pragma unroll 8
  for (int j = 0; j < n; ++j) {
    const T dj = STAGE ? dg[j] : h[(int64_t)j * n + j];
    const bool nan_j = dj != dj;
    rank += nan_i ? (!nan_j || j < i) : (dj > di || (dj == di && j < i));
  }
  order[z * sO + rank] = i;
}

// The same order by sorting: one workgroup per matrix sorts the pairs (key, i) of its
// diagonal with a bitonic network in LDS, where key is an unsigned image of d_i that
// decreases as d_i increases (-0 taken as +0, so equal values tie and fall back to the
// index) and NaN maps to the largest key; pairs compare key first, then index, so the
// sorted indices are the stable descending order with NaN last, by index: the ranks
// above. npad (a power of two >= n, at most NPAD) entries are sorted, the padding
// after every real pair. O(n log^2 n) work where the rank count is O(n^2).
template <typename T>
struct SortKey;
template <>
struct SortKey<float> {
  typedef uint32_t K;
  __device__ static K of(float d) {
    if (d != d) return 0xffffffffu;
    const uint32_t u = __float_as_uint(d == 0.0f ? 0.0f : d);
    const uint32_t asc = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // increases with d
    return ~asc;
  }
};
template <>
struct SortKey<double> {
  typedef unsigned long long K;
  __device__ static K of(double d) {
    if (d != d) return ~0ull;
    const unsigned long long u = __double_as_longlong(d == 0.0 ? 0.0 : d);
    const unsigned long long asc = (u >> 63) ? ~u : (u | (1ull << 63));
    return ~asc;
  }
};

template <typename T, int NPAD>
__global__ __launch_bounds__(1024) void act_order_sort_kernel(const T* H, int n, int64_t sH, int* order,
                                                              int64_t sO, int npad) {
  typedef typename SortKey<T>::K K;
  __shared__ K key[NPAD];
  __shared__ uint32_t idx[NPAD];
  const int z = blockIdx.x, tid = threadIdx.x;
  const T* h = H + z * sH;
  for (int i = tid; i < npad; i += 1024) {
    key[i] = i < n ? SortKey<T>::of(h[(int64_t)i * n + i]) : (K)~(K)0;
    idx[i] = (uint32_t)i;
  }
  __syncthreads();
  for (int k = 2; k <= npad; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = tid; t < npad / 2; t += 1024) {
        const int a = ((t & ~(j - 1)) << 1) | (t & (j - 1)), b = a | j;
        const K ka = key[a], kb = key[b];
        const uint32_t ia = idx[a], ib = idx[b];
        const bool gt = ka > kb || (ka == kb && ia > ib);
        if (gt == ((a & k) == 0)) {
          key[a] = kb;
          key[b] = ka;
          idx[a] = ib;
          idx[b] = ia;
        }
      }
      __syncthreads();
    }
  }
  for (int r = tid; r < n; r += 1024) order[z * sO + r] = (int)idx[r];
}

// ---------------------------------------------------------------- driver

static size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// the fused chain step's ticket counters (one per 64-column step) and per-matrix flags
static size_t fact_step_ints(int64_t n, int batch) { return (size_t)((n + NB - 1) / NB) + (size_t)batch; }

size_t fact_ws_bytes(int64_t n, int batch) {
  size_t nn = (size_t)n * n * batch * sizeof(double);
  return align_up(nn) * 3 + align_up((size_t)n * batch * sizeof(double)) +
         4 * align_up((size_t)batch * 8) + align_up(fact_step_ints(n, batch) * sizeof(int));
}

// Pinned host staging for the per-matrix damping, activity and failure flags.
// Copies from pageable memory go through the runtime's staging path, and a
// device-to-host one waits there for the whole factorization, holding up
// other host threads' launches; pinned buffers are plain DMA. Buffers are
// pooled process-wide (hipHostMalloc is slow) and handed to one call at a time.
struct PinnedPool {
  std::mutex mu;
  std::vector<std::pair<void*, size_t>> free_list;
  void* take(size_t bytes) {
    {
      std::lock_guard<std::mutex> g(mu);
      for (size_t i = 0; i < free_list.size(); ++i)
        if (free_list[i].second >= bytes) {
          void* p = free_list[i].first;
          free_list.erase(free_list.begin() + i);
          return p;
        }
    }
    void* p = nullptr;
    const size_t cap = bytes < 4096 ? 4096 : bytes;
    if (hipHostMalloc(&p, cap, hipHostMallocDefault) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> g(mu);
    sizes[p] = cap;
    return p;
  }
  void give(void* p) {
    std::lock_guard<std::mutex> g(mu);
    free_list.emplace_back(p, sizes[p]);
  }
  std::map<void*, size_t> sizes;
};
static PinnedPool g_pinned;

struct PinnedLease {
  void* p;
  explicit PinnedLease(size_t bytes) : p(g_pinned.take(bytes)) {}
  ~PinnedLease() {
    if (p) g_pinned.give(p);
  }
};

// Workspace views shared by the attempt and the driver.
struct FactWs {
  double *A, *X, *Tm, *diag_tmp, *shift, *damp_d;
  int *fail, *active;
  int *tickets, *done;  // fused chain step: ticket counter per step, last step done per matrix
};

static FactWs fact_ws(char* ws, int n, int batch) {
  const size_t nn = (size_t)n * n;
  FactWs w;
  w.A = reinterpret_cast<double*>(ws);
  w.X = reinterpret_cast<double*>(ws + align_up(nn * batch * 8));
  w.Tm = reinterpret_cast<double*>(ws + 2 * align_up(nn * batch * 8));
  char* p = ws + 3 * align_up(nn * batch * 8);
  w.diag_tmp = reinterpret_cast<double*>(p);
  p += align_up((size_t)n * batch * 8);
  w.shift = reinterpret_cast<double*>(p);
  p += align_up((size_t)batch * 8);
  w.damp_d = reinterpret_cast<double*>(p);
  p += align_up((size_t)batch * 8);
  w.fail = reinterpret_cast<int*>(p);
  p += align_up((size_t)batch * 8);
  w.tickets = reinterpret_cast<int*>(p);  // cleared with fail (fact_clear_ints)
  w.done = w.tickets + (n + NB - 1) / NB;
  p += align_up(fact_step_ints(n, batch) * sizeof(int));
  w.active = reinterpret_cast<int*>(p);
  return w;
}

// fail, then the fused step's tickets and flags: one contiguous run of ints
static int64_t fact_clear_ints(int n, int batch) {
  return (int64_t)(align_up((size_t)batch * 8) / sizeof(int) + fact_step_ints(n, batch));
}

// A second stream per calling stream for the look-ahead outer updates, created on first
// use and kept for the process, with its events: chain (the calling stream reached the end
// of a block column), far[2] (a look-ahead update done, by block-column parity) and join.
// Calls that share a calling stream must not run from two host threads at once. At most
// kMaxAhead calling streams get one; calls on further streams queue the look-ahead
// updates in place on the calling stream (same result).
struct AheadStreams {
  hipStream_t aux;
  hipEvent_t chain, far[2], join;
};
constexpr size_t kMaxAhead = 64;
static std::mutex g_ahead_mu;
static std::map<std::pair<int, hipStream_t>, AheadStreams> g_ahead;
static const AheadStreams* ahead_streams(hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> g(g_ahead_mu);
  const auto key = std::make_pair(dev, st);
  auto it = g_ahead.find(key);
  if (it != g_ahead.end()) return &it->second;
  if (g_ahead.size() >= kMaxAhead) return nullptr;
  // on any failure: release what was made, clear HIP's last error, and let the call queue
  // its look-ahead updates on the calling stream
  AheadStreams a{};
  if (hipStreamCreateWithFlags(&a.aux, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipEvent_t* evs[4] = {&a.chain, &a.far[0], &a.far[1], &a.join};
  for (int e = 0; e < 4; ++e) {
    if (hipEventCreateWithFlags(evs[e], hipEventDisableTiming) != hipSuccess) {
      for (int f = 0; f < e; ++f) (void)hipEventDestroy(*evs[f]);
      (void)hipStreamDestroy(a.aux);
      (void)hipGetLastError();
      return nullptr;
    }
  }
  return &(g_ahead[key] = a);
}

// One factorization attempt of every active matrix at its damp (w.damp_d),
// raising w.fail[z] on a bad pivot. Stream-ordered, nothing read back.
template <typename T>
static int fact_attempt(const T* H, int64_t sH, int n, int batch, const int* order, int64_t sO,
                        void* U, int u_dtype, int64_t sU, const FactWs& w, hipStream_t st) {
  const size_t nn = (size_t)n * n;
  const int64_t sA = (int64_t)nn;
  double *A = w.A, *X = w.X, *Tm = w.Tm;
  {
    const int64_t c = fact_clear_ints(n, batch);
    fill_i32_kernel<<<(unsigned)((c + 255) / 256), 256, 0, st>>>(w.fail, c, 0);
  }
  // Every entry of X that is read is written first: the diagonal-block kernel stores
  // whole 64 x 64 blocks (zeros above their diagonal), each doubling level stores its
  // X21 blocks with beta = 0, and the output reads the lower triangle only. The one
  // exception is a 128 x 128 GEMM tile, whose K range starts at its first row or
  // column and so covers the zero 64-block above a diagonal pair. Those tiles need a
  // K loop of at least 4096, i.e. a doubling level with s >= 4096, i.e. n > 4096; only
  // there is X cleared first.
  if (n > 4096) fill_kernel<<<1024, 256, 0, st>>>(X, (int64_t)nn * batch, 0.0);
  // the order check's marks live in the GEMM scratch Tm, which the split outer updates
  // and the doubling GEMMs later overwrite before reading
  fact_shift_kernel<T><<<batch, 256, 0, st>>>(H, n, sH, order, sO, w.damp_d, w.diag_tmp, w.shift,
                                                w.active, reinterpret_cast<int*>(Tm),
                                                (int64_t)(2 * nn), w.fail);
  // rows of H staged per block: as many as fit in 16 KB (at least one), up to 8; rows
  // longer than 64 KB take the element-wise gather. More blocks of fewer rows per CU keep
  // more loads in flight than a few 48 KB blocks did (28 x n = 3072: 0.70 -> 0.56 ms,
  // 28 x n = 2048: 0.29 -> 0.21 ms).
  const int64_t row_bytes = (int64_t)n * sizeof(T);
  if (row_bytes <= 64 * 1024) {
    int R = (int)((16 * 1024) / row_bytes);
    R = R < 1 ? 1 : (R > 8 ? 8 : R);
    fact_prepare_kernel<T><<<dim3((n + R - 1) / R, batch), 256, (size_t)R * row_bytes, st>>>(
        H, n, sH, order, sO, w.shift, A, sA, w.active, R);
  } else {
    fact_prepare_gather_kernel<T><<<dim3((n + 63) / 64, (n + 3) / 4, batch), 256, 0, st>>>(
        H, n, sH, order, sO, w.shift, A, sA, w.active);
  }
  CP_LAUNCHED("factor prepare");
  // left-looking in two levels: an NW-wide block column first receives all
  // earlier columns' updates in one large-K GEMM; inside it, each NB-wide
  // column receives its left neighbours' updates, then its diagonal block is
  // factored and the panel below it solved
  // Block column J (columns [k0, k0 + w0), k0 = J * NW) takes the outer updates of the
  // columns left of it in two GEMMs: the far part, columns [0, k0 - NW), and then the near
  // part, the 256 columns of block column J - 1. The far part of J + 2 only needs block
  // columns up to J, so with a look-ahead stream it runs there while J + 1's near part and
  // 64-column chain (inner updates, diagonal blocks, panels: short launches that leave most
  // of the GPU idle) run on the calling stream. Without one it is queued in the same place
  // on the calling stream; either way every element takes the same two subtractions.
  // Batches of up to four matrices take the look-ahead stream, and so does a larger batch
  // on a GPU the factorization has to itself (its 64-column chain still leaves CUs idle:
  // 28 matrices of n = 3072 15.4 -> 15.1 ms, n = 2048 5.7 -> 5.6 ms). Beside other size
  // classes' work (compact tiles) a second stream per class only took hardware queues and
  // CUs from a large batch.
  const AheadStreams* ah = (batch <= 4 || !g_compact_tiles) ? ahead_streams(st) : nullptr;
  hipStream_t aux = ah ? ah->aux : st;
  bool aux_used = false;
  auto join = [&]() -> int {
    if (!aux_used) return CP_OK;
    aux_used = false;
    CP_HIP(hipEventRecord(ah->join, aux));
    CP_HIP(hipStreamWaitEvent(st, ah->join, 0));
    return CP_OK;
  };
  // A[kt:, kt:kt+w] -= L[kt:, kb:ke] * L[kt:kt+w, kb:ke]^T, lower part. For n >= CHUNK_N
  // the K range is summed in chunks of KC columns from kb, each chunk's product subtracted
  // in turn: by one GEMM per chunk when the GEMM has blocks enough to fill the GPU, else
  // (few row tiles left, long K) by one GEMM whose blocks each take one chunk, writing
  // the chunk products into Tm (free during the Cholesky), and fact_chunk_sub_kernel.
  // Both give every element the same subtractions, so U does not depend on the choice.
  auto outer = [&](int kt, int kb, int ke, hipStream_t s) -> int {
    const int nw = n - kt < NW ? n - kt : NW;
    const int M = n - kt, K = ke - kb;
    const int S = n >= CHUNK_N ? (K + KC - 1) / KC : 1;
    auto part = [&](int c0, int c1) -> int {
      GemmArgs g{A + (int64_t)kt * n + c0, A + (int64_t)kt * n + c0, A + (int64_t)kt * n + kt, M,
                 nw, c1 - c0, n, n, n, -1.0, 1.0, sA, sA, sA, 0, 0, 0, 1, 4};
      return dgemm(g, batch, true, s);
    };
    if (S == 1) return part(kb, ke);
    const int64_t blocks = (int64_t)((M + 63) / 64) * ((nw + 63) / 64) * batch;
    if (blocks < 512) {
      // chunk products P[z][c][i][j] = sum over chunk c of L[kt+i][k] L[kt+j][k]
      GemmArgs g{A + (int64_t)kt * n + kb, A + (int64_t)kt * n + kb, Tm, M, nw, K, n, n, nw,
                 1.0, 0.0, sA, sA, (int64_t)nn, 0, 0, (int64_t)M * nw, S, 4};
      g.kc = KC;
      if (int e = dgemm(g, batch, true, s)) return e;
      fact_chunk_sub_kernel<<<dim3((nw + 63) / 64, (M + 3) / 4, batch), 256, 0, s>>>(
          Tm, (int64_t)nn, (int64_t)M * nw, S, A + (int64_t)kt * n + kt, n, sA, M, nw, w.active);
      CP_LAUNCHED("factor chunk subtraction");
      return CP_OK;
    }
    for (int c = 0; c < S; ++c)
      if (int e = part(kb + c * KC, kb + (c + 1) * KC < ke ? kb + (c + 1) * KC : ke)) return e;
    return CP_OK;
  };
  // Few matrices on a GPU the factorization has to itself: each 64-column step of the
  // chain as one fused launch, whose tiles take the same block code as the separate
  // launches (vec only picks the load width). Beside EF work (compact tiles) the separate
  // launches stay: the fused step's panel items hold CU slots while they wait, which
  // measured slower there (Llama-3-8B layer step 124.4 / 125.6 -> 127.3 / 127.2 ms).
  const bool fused = batch <= kFusedBatch && !g_compact_tiles;
  const bool fused_vec = !(n & 1) && aligned(A, 16) && aligned(X, 16);
  auto chol_loop = [&]() -> int {
    const int nJ = (n + NW - 1) / NW;
    for (int J = 0; J < nJ; ++J) {
      const int k0 = J * NW;
      const int w0 = n - k0 < NW ? n - k0 : NW;
      if (J >= 2 && ah) CP_HIP(hipStreamWaitEvent(st, ah->far[J & 1], 0));
      if (J >= 1)
        if (int s = outer(k0, k0 - NW, k0, st)) return s;
      for (int k = k0; k < k0 + w0; k += NB) {
        const int wk = n - k < NB ? n - k : NB;
        if (fused) {
          const int m = n - k - NB;
          FactStep fs{A, X, sA, n, k, k0, k / NB, 1 + (m > 0 ? (m + NB - 1) / NB : 0),
                      w.fail, w.done, w.tickets, w.active, g_chol_wait_limit};
          const unsigned grid = (unsigned)(fs.items * batch);
          if (fused_vec)
            fact_step_kernel<true><<<grid, 256, 0, st>>>(fs);
          else
            fact_step_kernel<false><<<grid, 256, 0, st>>>(fs);
          CP_LAUNCHED("factor chain step");
          if (m <= 0) break;
          continue;
        }
        if (k > k0) {
          // A[k:, k:k+wk] -= L[k:, k0:k] * L[k:k+wk, k0:k]^T
          GemmArgs gb{A + (int64_t)k * n + k0, A + (int64_t)k * n + k0, A + (int64_t)k * n + k,
                      n - k, wk, k - k0, n, n, n, -1.0, 1.0, sA, sA, sA, 0, 0, 0, 1, 0};
          if (int s = dgemm(gb, batch, true, st)) return s;
        }
        fact_diag_kernel<<<batch, 256, 0, st>>>(A, sA, X, sA, n, k, w.fail, w.active);
        CP_LAUNCHED("factor diagonal block");
        const int m = n - k - NB;
        if (m <= 0) break;
        // panel: A[k+NB:, k:k+NB] <- A[k+NB:, k:k+NB] * inv(L_kk)^T  (in place, row tiles)
        GemmArgs pa{A + (int64_t)(k + NB) * n + k, X + (int64_t)k * n + k,
                    A + (int64_t)(k + NB) * n + k, m, NB, NB, n, n, n, 1.0, 0.0, sA, sA, sA,
                    0, 0, 0, 1, 0};
        if (int s = dgemm(pa, batch, true, st)) return s;
      }
      if (J + 2 < nJ) {
        if (ah) {
          CP_HIP(hipEventRecord(ah->chain, st));
          CP_HIP(hipStreamWaitEvent(aux, ah->chain, 0));
          aux_used = true;
        }
        if (int s = outer(k0 + 2 * NW, 0, k0 + NW, aux)) return s;
        if (ah) CP_HIP(hipEventRecord(ah->far[J & 1], aux));
      }
    }
    return CP_OK;
  };
  {
    const int s = chol_loop();
    const int j = join();  // nothing of this call is left on the look-ahead stream
    if (s) return s;
    if (j) return j;
  }
  // L^{-1} by recursive doubling over neighbouring s-blocks
  for (int s = NB; s < n; s *= 2) {
    const int full = n / (2 * s);          // pairs with a full second block
    const int rem = n - full * 2 * s - s;  // size of a trailing partial second block
    for (int part = 0; part < 2; ++part) {
      const int pairs = part == 0 ? full : (rem > 0 ? 1 : 0);
      if (pairs == 0) continue;
      const int s2 = part == 0 ? s : rem;
      const int b0 = part == 0 ? 0 : full * 2 * s;
      const int64_t step = (int64_t)2 * s * (n + 1);
      // T_p = L21 X11
      GemmArgs g1{A + (int64_t)(b0 + s) * n + b0, X + (int64_t)b0 * n + b0, Tm, s2, s, s, n, n, s,
                  1.0, 0.0, sA, sA, (int64_t)nn, step, step, (int64_t)s * s, pairs, 2};
      if (int e = dgemm(g1, batch, false, st)) return e;
      // X21 = -X22 T_p
      GemmArgs g2{X + (int64_t)(b0 + s) * n + b0 + s, Tm, X + (int64_t)(b0 + s) * n + b0, s2, s, s2,
                  n, s, n, -1.0, 0.0, sA, (int64_t)nn, sA, step, (int64_t)s * s, step, pairs, 1};
      if (int e = dgemm(g2, batch, false, st)) return e;
    }
  }
  const dim3 og((n + 255) / 256, (n + 3) / 4, batch);
  const bool ovec = !(n & 3) && !(sU & 3) && aligned(U, 16) && aligned(X, 16);
  if (u_dtype == 1) {
    if (ovec)
      fact_output_kernel<double, true><<<og, 256, 0, st>>>(X, sA, n, (double*)U, sU, w.active);
    else
      fact_output_kernel<double, false><<<og, 256, 0, st>>>(X, sA, n, (double*)U, sU, w.active);
  } else {
    if (ovec)
      fact_output_kernel<float, true><<<og, 256, 0, st>>>(X, sA, n, (float*)U, sU, w.active);
    else
      fact_output_kernel<float, false><<<og, 256, 0, st>>>(X, sA, n, (float*)U, sU, w.active);
  }
  CP_LAUNCHED("factor output");
  return CP_OK;
}

// flags_out == nullptr: the reference's escalation loop, reading the failure
// flags back after each attempt. Otherwise one attempt at damp0 whose flags are
// copied to flags_out (device) and nothing is read back.
template <typename T>
static int fact_run(const T* H, int64_t sH, int n, int batch, const int* order, int64_t sO,
                    double damp0, int max_tries, void* U, int u_dtype, int64_t sU,
                    double* damp_used, char* ws, hipStream_t st, int32_t* flags_out = nullptr) {
  const FactWs w = fact_ws(ws, n, batch);
  if (flags_out) {
    fill_kernel<<<(batch + 255) / 256, 256, 0, st>>>(w.damp_d, batch, damp0);
    fill_i32_kernel<<<(batch + 255) / 256, 256, 0, st>>>(w.active, batch, 1);
    if (int e = fact_attempt<T>(H, sH, n, batch, order, sO, U, u_dtype, sU, w, st)) return e;
    CP_HIP(hipMemcpyAsync(flags_out, w.fail, batch * sizeof(int), hipMemcpyDeviceToDevice, st));
    return CP_OK;
  }
  std::vector<double> damp(batch, damp0);
  std::vector<int> act(batch, 1), done(batch, 0);
  // pinned: [damp f64 x batch][active i32 x batch][fail i32 x batch]
  PinnedLease lease((size_t)batch * 16);
  if (!lease.p) return set_error(CP_ERR_HIP, "hipHostMalloc of %zu bytes failed", (size_t)batch * 16);
  double* damp_h = static_cast<double*>(lease.p);
  int* act_h = reinterpret_cast<int*>(damp_h + batch);
  int* fail_h = act_h + batch;
  for (int attempt = 0; attempt < max_tries; ++attempt) {
    // the previous attempt ended with a stream synchronize, so the pinned
    // buffers are free to rewrite
    for (int z = 0; z < batch; ++z) {
      damp_h[z] = damp[z];
      act_h[z] = act[z];
    }
    CP_HIP(hipMemcpyAsync(w.damp_d, damp_h, batch * sizeof(double), hipMemcpyHostToDevice, st));
    CP_HIP(hipMemcpyAsync(w.active, act_h, batch * sizeof(int), hipMemcpyHostToDevice, st));
    if (int e = fact_attempt<T>(H, sH, n, batch, order, sO, U, u_dtype, sU, w, st)) return e;
    CP_HIP(hipMemcpyAsync(fail_h, w.fail, batch * sizeof(int), hipMemcpyDeviceToHost, st));
    CP_HIP(hipStreamSynchronize(st));
    for (int z = 0; z < batch; ++z)
      if (act[z] && (fail_h[z] & 2))
        return set_error(CP_ERR_INDEX, "order of matrix %d is not a permutation of %d", z, n);
    for (int z = 0; z < batch; ++z)
      if (act[z] && (fail_h[z] & 4))
        return set_error(CP_ERR_TIMEOUT,
                         "factorization of matrix %d (n=%d): a chain step gave up waiting for its "
                         "diagonal block; the result is invalid", z, n);
    int pending = 0;
    for (int z = 0; z < batch; ++z) {
      if (!act[z]) continue;
      if (fail_h[z]) {
        damp[z] *= 10.0;
        ++pending;
      } else {
        act[z] = 0;
        done[z] = 1;
        if (damp_used) damp_used[z] = damp[z];
        if (attempt)
          fprintf(stderr, "[ef] cholesky_inv_upper: damp escalated %g -> %g in %d step(s) for a "
                          "borderline Hessian (n=%d)\n", damp0, damp[z], attempt, n);
      }
    }
    if (!pending) return CP_OK;
  }
  for (int z = 0; z < batch; ++z)
    if (!done[z])
      return set_error(CP_ERR_NOT_PD,
                       "cholesky_inv_upper: inv(H) not positive definite even after escalating "
                       "damp to %g (n=%d); Hessian appears degenerate",
                       damp[z] / 10.0, n);
  return CP_OK;
}

}  // namespace cp

extern "C" {

size_t cp_chol_ws_bytes(int64_t n, int batch) { return cp::fact_ws_bytes(n, batch); }

void cp_chol_compact_tiles(int on) { cp::g_compact_tiles = on != 0; }

void cp_chol_wait_limit(int sleeps) { cp::g_chol_wait_limit = sleeps < 0 ? cp::kDefaultCholWait : sleeps; }

int cp_act_order(const void* H, int h_dtype, int64_t n, int batch, int32_t* order, void* stream) {
  cp::clear_error();
  if (!H || !order || n <= 0 || batch <= 0) return cp::set_error(CP_ERR_ARG, "bad act_order arguments");
  hipStream_t st = (hipStream_t)stream;
  // the sort in LDS where its arrays fit (float: n <= 16384, double: n <= 8192)
  int npad = 1;
  while (npad < n) npad <<= 1;
  if (h_dtype != 1 && npad <= 16384) {
    const float* Hf = (const float*)H;
    if (npad <= 4096)
      cp::act_order_sort_kernel<float, 4096><<<batch, 1024, 0, st>>>(Hf, (int)n, n * n, order, n, npad);
    else
      cp::act_order_sort_kernel<float, 16384><<<batch, 1024, 0, st>>>(Hf, (int)n, n * n, order, n, npad);
    CP_LAUNCHED("act_order sort");
    return CP_OK;
  }
  if (h_dtype == 1 && npad <= 8192) {
    const double* Hd = (const double*)H;
    if (npad <= 4096)
      cp::act_order_sort_kernel<double, 4096><<<batch, 1024, 0, st>>>(Hd, (int)n, n * n, order, n, npad);
    else
      cp::act_order_sort_kernel<double, 8192><<<batch, 1024, 0, st>>>(Hd, (int)n, n * n, order, n, npad);
    CP_LAUNCHED("act_order sort");
    return CP_OK;
  }
  dim3 grid((unsigned)((n + 255) / 256), batch);
  const size_t lds = (size_t)n * (h_dtype == 1 ? 8 : 4);
  const bool stage = lds <= 64 * 1024;
  if (h_dtype == 1) {
    if (stage)
      cp::act_order_kernel<double, true><<<grid, 256, lds, st>>>((const double*)H, (int)n, n * n, order, n);
    else
      cp::act_order_kernel<double, false><<<grid, 256, 0, st>>>((const double*)H, (int)n, n * n, order, n);
  } else {
    if (stage)
      cp::act_order_kernel<float, true><<<grid, 256, lds, st>>>((const float*)H, (int)n, n * n, order, n);
    else
      cp::act_order_kernel<float, false><<<grid, 256, 0, st>>>((const float*)H, (int)n, n * n, order, n);
  }
  CP_LAUNCHED("act_order launch");
  return CP_OK;
}

int cp_chol_inv_upper_async(const void* H, int h_dtype, int64_t n, int batch,
                            const int32_t* order, double damp, void* U, int u_dtype,
                            int32_t* flags, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  if (!H || !U || !ws || !flags) return cp::set_error(CP_ERR_ARG, "null H/U/flags/ws");
  if (u_dtype != 0 && u_dtype != 1) return cp::set_error(CP_ERR_ARG, "u_dtype must be 0 (f32) or 1 (f64)");
  if (n <= 0 || batch <= 0 || n > 65536) return cp::set_error(CP_ERR_SHAPE, "bad n=%lld / batch=%d", (long long)n, batch);
  if (ws_bytes < cp::fact_ws_bytes(n, batch))
    return cp::set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, cp::fact_ws_bytes(n, batch));
  if (!cp::aligned(ws, 256)) return cp::set_error(CP_ERR_ALIGN, "workspace needs 256-byte alignment");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nn = n * n;
  if (h_dtype == 1)
    return cp::fact_run<double>((const double*)H, nn, (int)n, batch, order, n, damp, 1, U, u_dtype,
                                nn, nullptr, (char*)ws, st, flags);
  if (h_dtype == 0)
    return cp::fact_run<float>((const float*)H, nn, (int)n, batch, order, n, damp, 1, U, u_dtype,
                               nn, nullptr, (char*)ws, st, flags);
  return cp::set_error(CP_ERR_ARG, "h_dtype must be 0 (f32) or 1 (f64)");
}

int cp_chol_inv_upper(const void* H, int h_dtype, int64_t n, int batch, const int32_t* order,
                      double damp, int max_tries, void* U, int u_dtype, double* damp_used,
                      void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  if (!H || !U || !ws) return cp::set_error(CP_ERR_ARG, "null H/U/ws");
  if (u_dtype != 0 && u_dtype != 1) return cp::set_error(CP_ERR_ARG, "u_dtype must be 0 (f32) or 1 (f64)");
  if (n <= 0 || batch <= 0 || n > 65536) return cp::set_error(CP_ERR_SHAPE, "bad n=%lld / batch=%d", (long long)n, batch);
  if (max_tries <= 0) return cp::set_error(CP_ERR_ARG, "max_tries must be positive");
  if (ws_bytes < cp::fact_ws_bytes(n, batch))
    return cp::set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, cp::fact_ws_bytes(n, batch));
  if (!cp::aligned(ws, 256)) return cp::set_error(CP_ERR_ALIGN, "workspace needs 256-byte alignment");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nn = n * n;
  if (h_dtype == 1)
    return cp::fact_run<double>((const double*)H, nn, (int)n, batch, order, n, damp, max_tries, U, u_dtype,
                                nn, damp_used, (char*)ws, st);
  if (h_dtype == 0)
    return cp::fact_run<float>((const float*)H, nn, (int)n, batch, order, n, damp, max_tries, U, u_dtype,
                               nn, damp_used, (char*)ws, st);
  return cp::set_error(CP_ERR_ARG, "h_dtype must be 0 (f32) or 1 (f64)");
}

}  // extern "C"
