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
//  * Cholesky is left-looking with 64-wide block columns: a block column first
//    receives the updates of everything to its left in one large-K fp64 MFMA
//    GEMM, then its diagonal block is factored and inverted in LDS and the
//    panel below it is a GEMM with that inverse;
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
#include <vector>

#include "cp_host.h"

namespace cp {

typedef double dbl4 __attribute__((ext_vector_type(4)));

constexpr int NB = 64;  // panel width

// ---------------------------------------------------------------- fp64 MFMA GEMM
// C[M,N] = alpha * A[M,K] * op(B) + beta * C, row-major with leading dims.
// op(B) = B [K,N] or, with BT, B^T for B stored [N,K]. Batched over blockIdx.z
// as z = z1 * nz2 + z2 with separate strides per level. LOWER skips tiles
// strictly above the diagonal of C and writes only C[i][j] with i >= j.
// Tile 64x64x16, 4 waves of 32x32 each built from v_mfma_f64_16x16x4f64.
// tri: bit 0 -- A is lower triangular (A[r][k] = 0 for k > r), so output row
// tile bm only needs k < bm + 64; bit 1 -- B ([K,N], not transposed) is lower
// triangular (B[k][c] = 0 for k < c), so output column tile bn needs k >= bn.
struct GemmArgs {
  const double* A;
  const double* B;
  double* C;
  int M, N, K, lda, ldb, ldc;
  double alpha, beta;
  int64_t sA1, sB1, sC1, sA2, sB2, sC2;
  int nz2;
  int tri;
};

template <bool BT, bool LOWER>
__global__ __launch_bounds__(256) void dgemm_kernel(GemmArgs g) {
  __shared__ double As[16][64 + 1];
  __shared__ double Bs[16][64 + 1];
  const int z1 = blockIdx.z / g.nz2, z2 = blockIdx.z % g.nz2;
  const double* A = g.A + z1 * g.sA1 + z2 * g.sA2;
  const double* B = g.B + z1 * g.sB1 + z2 * g.sB2;
  double* C = g.C + z1 * g.sC1 + z2 * g.sC2;
  const int bm = blockIdx.y * 64, bn = blockIdx.x * 64;
  if (LOWER && bn > bm + 63) return;
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
  dbl4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = dbl4{0.0, 0.0, 0.0, 0.0};

  const int kbeg = (g.tri & 2) ? (bn & ~15) : 0;
  const int kend = (g.tri & 1) ? min(g.K, bm + 64) : g.K;
  for (int k0 = kbeg; k0 < kend; k0 += 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      int idx = t + 256 * q;
      int r = idx >> 4, c = idx & 15;
      int gr = bm + r, gc = k0 + c;
      As[c][r] = (gr < g.M && gc < g.K) ? A[(int64_t)gr * g.lda + gc] : 0.0;
      if (BT) {
        int gn = bn + r;
        Bs[c][r] = (gn < g.N && gc < g.K) ? B[(int64_t)gn * g.ldb + gc] : 0.0;
      } else {
        int c2 = idx >> 6, r2 = idx & 63;
        int gk = k0 + c2, gn = bn + r2;
        Bs[c2][r2] = (gk < g.K && gn < g.N) ? B[(int64_t)gk * g.ldb + gn] : 0.0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int kr = kk * 4 + (l >> 4);
      double a0 = As[kr][wm + (l & 15)], a1 = As[kr][wm + 16 + (l & 15)];
      double b0 = Bs[kr][wn + (l & 15)], b1 = Bs[kr][wn + 16 + (l & 15)];
      acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // v_mfma_f64_16x16x4f64 result: register r of lane l holds row 4r + l/16, column l%16
        int i = bm + wm + ti * 16 + 4 * r + (l >> 4);
        int j = bn + wn + tj * 16 + (l & 15);
        if (i < g.M && j < g.N && (!LOWER || i >= j)) {
          double* p = C + (int64_t)i * g.ldc + j;
          double v = g.alpha * acc[ti][tj][r];
          *p = g.beta == 0.0 ? v : v + g.beta * *p;
        }
      }
}

static int dgemm(const GemmArgs& a, int nz1, bool bt, bool lower, hipStream_t st) {
  if (a.M <= 0 || a.N <= 0) return CP_OK;
  dim3 grid((a.N + 63) / 64, (a.M + 63) / 64, nz1 * a.nz2);
  if (bt) {
    if (lower) dgemm_kernel<true, true><<<grid, 256, 0, st>>>(a);
    else dgemm_kernel<true, false><<<grid, 256, 0, st>>>(a);
  } else {
    if (lower) dgemm_kernel<false, true><<<grid, 256, 0, st>>>(a);
    else dgemm_kernel<false, false><<<grid, 256, 0, st>>>(a);
  }
  CP_LAUNCHED("fp64 GEMM launch");
  return CP_OK;
}

// ---------------------------------------------------------------- prepare
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

// Diagonal of the act-ordered H in visiting order, then the damping shift
// damp * mean + 1e-8 (mean replaced by 1 when not positive), as ef.py:64-69
// computes it from np.mean(np.diag(Hp)). One thread per matrix.
template <typename T>
__global__ void fact_shift_kernel(const T* H, int n, int64_t sH, const int* order, int64_t sO,
                                  const double* damp, double* diag_tmp, double* shift,
                                  const int* active) {
  const int z = blockIdx.x;
  if (active && !active[z]) return;
  const T* h = H + z * sH;
  const int* o = order ? order + z * sO : nullptr;
  double* dg = diag_tmp + (int64_t)z * n;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    int p = o ? o[i] : i;
    dg[i] = (double)h[(int64_t)p * n + p];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double mean = pw_sum_f64(dg, n, 1) / (double)n;
    double base = mean > 0.0 ? mean : 1.0;
    shift[z] = damp[z] * base + 1e-8;
  }
}

// A[i][j] = H[q_i][q_j] (+ shift on the diagonal) for i >= j, with
// q_i = order[n-1-i]: the act_order gather and the index reversal in one pass.
template <typename T>
__global__ void fact_prepare_kernel(const T* H, int n, int64_t sH, const int* order, int64_t sO,
                                    const double* shift, double* A, int64_t sA,
                                    const int* active) {
  const int z = blockIdx.z;
  if (active && !active[z]) return;
  const int j = blockIdx.x * 64 + (threadIdx.x & 63);
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= n || j >= n) return;
  double* a = A + z * sA;
  if (j > i) {
    a[(int64_t)i * n + j] = 0.0;
    return;
  }
  const int* o = order ? order + z * sO : nullptr;
  int qi = o ? o[n - 1 - i] : n - 1 - i;
  int qj = o ? o[n - 1 - j] : n - 1 - j;
  double v = (double)H[z * sH + (int64_t)qi * n + qj];
  if (i == j) v = v + shift[z];
  a[(int64_t)i * n + j] = v;
}

// ---------------------------------------------------------------- diagonal block
// Factor the nb x nb diagonal block at (k, k) in LDS, write L_kk back to A and
// inv(L_kk) into the matching diagonal block of X; flag a bad pivot.
__global__ __launch_bounds__(256) void fact_diag_kernel(double* A, int64_t sA, double* X,
                                                        int64_t sX, int n, int k, int* fail,
                                                        const int* active) {
  __shared__ double a[NB][NB + 1];
  __shared__ double x[NB][NB + 1];
  const int z = blockIdx.x;
  if (active && !active[z]) return;
  const int nb = min(NB, n - k);
  double* Ak = A + z * sA + (int64_t)k * n + k;
  double* Xk = X + z * sX + (int64_t)k * n + k;
  const int t = threadIdx.x;
  for (int idx = t; idx < NB * NB; idx += 256) {
    int i = idx / NB, j = idx % NB;
    a[i][j] = (i < nb && j <= i) ? Ak[(int64_t)i * n + j] : 0.0;
  }
  __syncthreads();
  __shared__ int bad;
  if (t == 0) bad = 0;
  __syncthreads();
  for (int j = 0; j < nb; ++j) {
    if (t == 0) {
      double v = a[j][j];
      if (!(v > 0.0)) bad = 1;
      a[j][j] = sqrt(v > 0.0 ? v : 1.0);
    }
    __syncthreads();
    const double piv = a[j][j];
    for (int i = j + 1 + t; i < nb; i += 256) a[i][j] = a[i][j] / piv;
    __syncthreads();
    const int m = nb - j - 1;
    for (int idx = t; idx < m * m; idx += 256) {
      int i = j + 1 + idx / m, c = j + 1 + idx % m;
      if (c <= i) a[i][c] = a[i][c] - a[i][j] * a[c][j];
    }
    __syncthreads();
  }
  // inverse of the lower-triangular block, one column per thread
  if (t < nb) {
    const int c = t;
    for (int i = 0; i < c; ++i) x[i][c] = 0.0;
    x[c][c] = 1.0 / a[c][c];
    for (int i = c + 1; i < nb; ++i) {
      double s = 0.0;
      for (int kk = c; kk < i; ++kk) s = s + a[i][kk] * x[kk][c];
      x[i][c] = -s / a[i][i];
    }
  }
  __syncthreads();
  for (int idx = t; idx < nb * nb; idx += 256) {
    int i = idx / nb, j = idx % nb;
    Ak[(int64_t)i * n + j] = j <= i ? a[i][j] : 0.0;
    Xk[(int64_t)i * n + j] = x[i][j];
  }
  if (t == 0 && bad) fail[z] = 1;
}

// U[i][j] = X[n-1-i][n-1-j] for i <= j, 0 below the diagonal (OutT = float:
// the float32 cast of ef.py:189; OutT = double: cholesky_inv_upper's result).
template <typename OutT>
__global__ void fact_output_kernel(const double* X, int64_t sX, int n, OutT* U, int64_t sU,
                                   const int* active) {
  const int z = blockIdx.z;
  if (active && !active[z]) return;
  const int j = blockIdx.x * 64 + (threadIdx.x & 63);
  const int i = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (i >= n || j >= n) return;
  OutT v = 0;
  if (i <= j) v = (OutT)X[z * sX + (int64_t)(n - 1 - i) * n + (n - 1 - j)];
  U[z * sU + (int64_t)i * n + j] = v;
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
// order = stable argsort of -diag(H): rank of i = #{j: d_j > d_i} + #{j < i: d_j == d_i}.
template <typename T>
__global__ void act_order_kernel(const T* H, int n, int64_t sH, int* order, int64_t sO) {
  const int z = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const T* h = H + z * sH;
  const double di = (double)h[(int64_t)i * n + i];
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    double dj = (double)h[(int64_t)j * n + j];
    rank += (dj > di) || (dj == di && j < i);
  }
  order[z * sO + rank] = i;
}

// ---------------------------------------------------------------- driver

static size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

size_t fact_ws_bytes(int64_t n, int batch) {
  size_t nn = (size_t)n * n * batch * sizeof(double);
  return align_up(nn) * 3 + align_up((size_t)n * batch * sizeof(double)) +
         4 * align_up((size_t)batch * 8);
}

template <typename T>
static int fact_run(const T* H, int64_t sH, int n, int batch, const int* order, int64_t sO,
                    double damp0, int max_tries, void* U, int u_dtype, int64_t sU,
                    double* damp_used, char* ws, hipStream_t st) {
  const size_t nn = (size_t)n * n;
  double* A = reinterpret_cast<double*>(ws);
  double* X = reinterpret_cast<double*>(ws + align_up(nn * batch * 8));
  double* Tm = reinterpret_cast<double*>(ws + 2 * align_up(nn * batch * 8));
  char* p = ws + 3 * align_up(nn * batch * 8);
  double* diag_tmp = reinterpret_cast<double*>(p);
  p += align_up((size_t)n * batch * 8);
  double* shift = reinterpret_cast<double*>(p);
  p += align_up((size_t)batch * 8);
  double* damp_d = reinterpret_cast<double*>(p);
  p += align_up((size_t)batch * 8);
  int* fail = reinterpret_cast<int*>(p);
  p += align_up((size_t)batch * 8);
  int* active = reinterpret_cast<int*>(p);

  std::vector<double> damp(batch, damp0);
  std::vector<int> act(batch, 1), failed(batch, 0), done(batch, 0);
  const int64_t sA = (int64_t)nn;
  for (int attempt = 0; attempt < max_tries; ++attempt) {
    CP_HIP(hipMemcpyAsync(damp_d, damp.data(), batch * sizeof(double), hipMemcpyHostToDevice, st));
    CP_HIP(hipMemcpyAsync(active, act.data(), batch * sizeof(int), hipMemcpyHostToDevice, st));
    fill_i32_kernel<<<(batch + 255) / 256, 256, 0, st>>>(fail, batch, 0);
    fill_kernel<<<1024, 256, 0, st>>>(X, (int64_t)nn * batch, 0.0);
    fact_shift_kernel<T><<<batch, 256, 0, st>>>(H, n, sH, order, sO, damp_d, diag_tmp, shift, active);
    fact_prepare_kernel<T><<<dim3((n + 63) / 64, (n + 3) / 4, batch), 256, 0, st>>>(
        H, n, sH, order, sO, shift, A, sA, active);
    CP_LAUNCHED("factor prepare");
    // left-looking: block column k first receives all earlier columns' updates
    // in one large-K GEMM, then its diagonal block is factored and the panel
    // below it solved
    for (int k = 0; k < n; k += NB) {
      const int w = n - k < NB ? n - k : NB;
      if (k > 0) {
        // A[k:, k:k+w] -= L[k:, 0:k] * L[k:k+w, 0:k]^T
        GemmArgs ga{A + (int64_t)k * n, A + (int64_t)k * n, A + (int64_t)k * n + k, n - k, w, k,
                    n, n, n, -1.0, 1.0, sA, sA, sA, 0, 0, 0, 1, 0};
        if (int s = dgemm(ga, batch, true, false, st)) return s;
      }
      fact_diag_kernel<<<batch, 256, 0, st>>>(A, sA, X, sA, n, k, fail, active);
      CP_LAUNCHED("factor diagonal block");
      const int m = n - k - NB;
      if (m <= 0) break;
      // panel: A[k+NB:, k:k+NB] <- A[k+NB:, k:k+NB] * inv(L_kk)^T  (in place, row tiles)
      GemmArgs pa{A + (int64_t)(k + NB) * n + k, X + (int64_t)k * n + k, A + (int64_t)(k + NB) * n + k,
                  m, NB, NB, n, n, n, 1.0, 0.0, sA, sA, sA, 0, 0, 0, 1, 0};
      if (int s = dgemm(pa, batch, true, false, st)) return s;
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
        if (int e = dgemm(g1, batch, false, false, st)) return e;
        // X21 = -X22 T_p
        GemmArgs g2{X + (int64_t)(b0 + s) * n + b0 + s, Tm, X + (int64_t)(b0 + s) * n + b0, s2, s, s2,
                    n, s, n, -1.0, 0.0, sA, (int64_t)nn, sA, step, (int64_t)s * s, step, pairs, 1};
        if (int e = dgemm(g2, batch, false, false, st)) return e;
      }
    }
    const dim3 og((n + 63) / 64, (n + 3) / 4, batch);
    if (u_dtype == 1)
      fact_output_kernel<double><<<og, 256, 0, st>>>(X, sA, n, (double*)U, sU, active);
    else
      fact_output_kernel<float><<<og, 256, 0, st>>>(X, sA, n, (float*)U, sU, active);
    CP_LAUNCHED("factor output");
    CP_HIP(hipMemcpyAsync(failed.data(), fail, batch * sizeof(int), hipMemcpyDeviceToHost, st));
    CP_HIP(hipStreamSynchronize(st));
    int pending = 0;
    for (int z = 0; z < batch; ++z) {
      if (!act[z]) continue;
      if (failed[z]) {
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

int cp_act_order(const void* H, int h_dtype, int64_t n, int batch, int32_t* order, void* stream) {
  cp::clear_error();
  if (!H || !order || n <= 0 || batch <= 0) return cp::set_error(CP_ERR_ARG, "bad act_order arguments");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((n + 255) / 256), batch);
  if (h_dtype == 1)
    cp::act_order_kernel<double><<<grid, 256, 0, st>>>((const double*)H, (int)n, n * n, order, n);
  else
    cp::act_order_kernel<float><<<grid, 256, 0, st>>>((const float*)H, (int)n, n * n, order, n);
  CP_LAUNCHED("act_order launch");
  return CP_OK;
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
