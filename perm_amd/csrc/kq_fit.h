// Sub-block grid fits of the k-quant encoders, on the device.
//
// In-lane fits (one lane owns one sub-block of N values in registers):
//   fit_affine<N, NUMS> make_qkx2 / make_qkx3 search      coldpress/kquant.py:42-94
//   fit_signed<N>       make_qx_quants, rmse_type 1        coldpress/kquant.py:97-133
//   fit_signed_descent  make_q3_quants                     coldpress/kquant.py:136-179
// Cross-lane fits (one lane owns one element of a G-wide vector of super-block
// scales; G = 16 for Q2_K/Q3_K, 8 for Q4_K):
//   gfit_nonneg<G>      make_qp_quants                     coldpress/kquant.py:182-235
//   gfit_signed<G>      make_qx_quants on super-scales     coldpress/kquant.py:460
//
// Each function evaluates the same float32 expressions, in the same order, as
// the numpy routine it restates; reductions go through psum / gsum, which
// reproduce numpy's pairwise summation order.
#pragma once
#include "cp_device.h"

namespace cp {

// The terms are summed as they are formed, into psum's eight strided accumulators
// (element i goes to accumulator i % 8, in ascending i), so no N-term array is live:
// the same additions in the same order as psum over the stored terms.
template <int N>
__device__ __forceinline__ float affine_err(const float (&x)[N], const float (&w)[N],
                                            const float (&lf)[N], float scale, float off,
                                            bool mad) {
  static_assert(N % 8 == 0 && N >= 8 && N <= 128, "pairwise block");
  float r8[8];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float r = (scale * lf[i] + off) - x[i];
    r = mad ? fabsf(r) : r * r;
    const float t = w[i] * r;
    r8[i % 8] = i < 8 ? t : r8[i % 8] + t;
  }
  return psum_tree(r8);
}

// Codes of one candidate, clip(nearest_int(inv * (x - lo)), 0, nmax), as floats.
// fast: the same codes as rint(med3(v, 0, nmax)) (v_med3_f32, v_rndne_f32), valid when
// every v = inv * (x - lo) is finite and inside (-2^22, 2^22 - 1/2). There the magic add
// rounds to the nearest integer, ties to even, as v_rndne_f32 does, and clipping to the
// integer bounds first changes no result: v below 0 gives +0 either way, v above nmax
// gives nmax either way (outside the range the integer form returns a bit pattern the
// float form does not).
template <int N, bool FAST>
__device__ __forceinline__ void affine_codes(const float (&x)[N], float inv, float lo, int nmax,
                                             float (&lf)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float v = inv * (x[i] - lo);
    if constexpr (FAST)
      lf[i] = __builtin_rintf(__builtin_amdgcn_fmed3f(v, 0.0f, (float)nmax));
    else
      lf[i] = (float)clampi(rint_magic(v), 0, nmax);
  }
}

// The candidate numerators (rmin + rdelta * step) + nmax, step = 0 .. NSTEP, of a
// make_qkx search, evaluated at compile time in float32 with every operation rounded
// once, as the device would evaluate them (rmin = RMIN100 / 100, rdelta = RDELTA100 /
// 100, each the float nearest the decimal, as the reference's np.float32 constants).
// The search reads them from constant memory with scalar loads.
template <int NMAX, int RMIN100, int RDELTA100, int NSTEP>
struct QkxNums {
  static constexpr int kNmax = NMAX, kSteps = NSTEP;
  float v[NSTEP + 1];
  constexpr QkxNums() : v() {
    const float rmin = (float)RMIN100 / 100.0f, rdelta = (float)RDELTA100 / 100.0f;
    for (int s = 0; s <= NSTEP; ++s) v[s] = (rmin + rdelta * (float)s) + (float)NMAX;
  }
};
// the five searches of the encoders (kquant.py:359-360, :385-386, :518-520, :541-542, :593)
static __constant__ const QkxNums<3, -90, 5, 36> kQkxQ2Imat = QkxNums<3, -90, 5, 36>();
static __constant__ const QkxNums<3, -50, 10, 15> kQkxQ2Ref = QkxNums<3, -50, 10, 15>();
static __constant__ const QkxNums<15, -90, 5, 36> kQkxQ4Imat = QkxNums<15, -90, 5, 36>();
static __constant__ const QkxNums<15, -100, 10, 20> kQkxQ4Ref = QkxNums<15, -100, 10, 20>();
static __constant__ const QkxNums<31, -90, 5, 36> kQkxQ5Imat = QkxNums<31, -90, 5, 36>();
static __constant__ const QkxNums<31, -50, 10, 15> kQkxQ5Ref = QkxNums<31, -50, 10, 15>();

// Result of fit_affine: the scale, -lo (the "min" the containers store), and the
// inverse scale and offset whose codes are the best (affine_final_codes forms them).
struct AffineFit {
  float scale, min;
  float inv, lo;
  bool dead;
};

// clip(nearest_int(inv * (x - lo)), 0, nmax) of the best candidate (0 for a dead block).
template <int N>
__device__ __forceinline__ void affine_final_codes(const float (&x)[N], const AffineFit& f,
                                                   int nmax, int (&L)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) L[i] = f.dead ? 0 : clampi(rint_magic(f.inv * (x[i] - f.lo)), 0, nmax);
}

// Weighted affine fit x ~ scale * L + lo, L in [0, NUMS::kNmax], over the candidates of
// the table NUMS (its numerators, step = 0 .. kSteps). Returns scale, -lo and the best
// candidate's (inverse scale, offset), whose codes depend on that pair alone: the search
// keeps the pair and the caller forms the codes with affine_final_codes only where it
// needs them (the encoders requantize every sub-block whose grid step is non-zero).
//
// A candidate takes the float form of the codes when, on every lane of the wave, x is
// finite, inv is finite and inv * (min(x) - lo) > -2^22: inv > 0 and rounding is
// monotonic, so every inv * (x_i - lo) then lies between that bound and
// inv * (hi - lo), which is at most about nmax + 1.
template <int N, class NUMS>
__device__ __forceinline__ AffineFit fit_affine(const float (&x)[N], const float (&w)[N],
                                                const NUMS& nums, bool mad, bool strict_dead) {
  constexpr int nmax = NUMS::kNmax;
  float hi = x[0], lo = x[0];
  bool fin = isfinite(x[0]);
#pragma unroll
  for (int i = 1; i < N; ++i) {
    hi = fmaxf(hi, x[i]);
    lo = fminf(lo, x[i]);
    fin = fin && isfinite(x[i]);
  }
  const float xmin = lo;
  lo = fminf(lo, 0.0f);
  float t[N];
  float sw = psum<N>(w);
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = w[i] * x[i];
  float swx = psum<N>(t);
  const bool dead = strict_dead ? (hi <= lo) : (hi == lo);

  float inv = (float)nmax / (dead ? 1.0f : hi - lo);
  float scale = 1.0f / inv;
  float lf[N];
  affine_codes<N, false>(x, inv, lo, nmax, lf);
  float best = affine_err<N>(x, w, lf, scale, lo, mad);
  float best_inv = inv, best_lo = lo;  // the pair whose codes are the best so far

  for (int step = 0; step <= NUMS::kSteps; ++step) {
    float span = hi - lo;
    span = span > 0.0f ? span : 1.0f;
    const float num = nums.v[step];  // in div_box
    float inv_c;
    if (__all(div_box(span)))
      inv_c = div_by(num, span, div_recip(span));
    else
      inv_c = num / span;
    const bool fast = fin && inv_c <= 3.40282347e38f && inv_c * (xmin - lo) > -4194304.0f;
    if (__all(fast))
      affine_codes<N, true>(x, inv_c, lo, nmax, lf);
    else
      affine_codes<N, false>(x, inv_c, lo, nmax, lf);
    // sum_l, sum_l2, sum_xl as psum forms them, accumulated as the products are formed
    float a8[8], b8[8], c8[8];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const float wl = w[i] * lf[i];
      const float bl = wl * lf[i], cl = wl * x[i];
      a8[i % 8] = i < 8 ? wl : a8[i % 8] + wl;
      b8[i % 8] = i < 8 ? bl : b8[i % 8] + bl;
      c8[i % 8] = i < 8 ? cl : c8[i % 8] + cl;
    }
    float sl = psum_tree(a8);
    float sl2 = psum_tree(b8);
    float sxl = psum_tree(c8);
    float det = sw * sl2 - sl * sl;
    const float ns = sw * sxl - swx * sl, nm = sl2 * swx - sl * sxl;
    float s_c, m_c;
    // both quotients share det; lanes that reject the candidate whatever its fit
    // (det <= 0 or a dead block) do not hold the wave to the general division
    if (__all(!(det > 0.0f) || dead || (div_box(det) && div_num_ok(ns) && div_num_ok(nm)))) {
      const float y = div_recip(det);
      s_c = div_by(ns, det, y);
      m_c = div_by(nm, det, y);
    } else {
      s_c = ns / det;
      m_c = nm / det;
    }
    // the scale without an offset is needed only where the fitted offset is positive;
    // its division (about as costly as 18 subtractions) runs only when some lane needs it
    if (__any(m_c > 0.0f)) {
      float s_alt = sxl / sl2;
      if (m_c > 0.0f) {
        m_c = 0.0f;
        s_c = s_alt;
      }
    }
    float e_c = affine_err<N>(x, w, lf, s_c, m_c, mad);
    if (det > 0.0f && e_c < best && !dead) {
      best_inv = inv_c;
      best_lo = lo;
      best = e_c;
      scale = s_c;
      lo = m_c;
    }
  }
  return AffineFit{dead ? 0.0f : scale, -lo, best_inv, best_lo, dead};
}

// Symmetric signed fit x ~ scale * L, L in [-nmax, nmax-1]; weights w (pass
// x*x for the unweighted path). L receives codes + nmax.
template <int N>
__device__ __forceinline__ float fit_signed(const float (&x)[N], const float (&w)[N], int nmax,
                                            int (&L)[N]) {
  float amax = fabsf(x[0]), sext = x[0];
#pragma unroll
  for (int i = 1; i < N; ++i) {
    float a = fabsf(x[i]);
    if (a > amax) {
      amax = a;
      sext = x[i];
    }
  }
  const bool dead = amax < 1e-15f;
  sext = dead ? 1.0f : sext;
  float wx[N];
#pragma unroll
  for (int i = 0; i < N; ++i) wx[i] = w[i] * x[i];

  float inv = -(float)nmax / sext;
  float p[N], q[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    L[i] = clampi(rint_magic(inv * x[i]), -nmax, nmax - 1);
    float lf = (float)L[i];
    p[i] = wx[i] * lf;
    q[i] = (w[i] * lf) * lf;
  }
  float slx = psum<N>(p), sl2 = psum<N>(q);
  float scale = sl2 != 0.0f ? slx / sl2 : 0.0f;
  float best = scale * slx;
  for (int s = -9; s <= 9; ++s) {
    if (s == 0) continue;
    float inv_c = -((float)nmax + 0.1f * (float)s) / sext;
    int Lc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      Lc[i] = clampi(rint_magic(inv_c * x[i]), -nmax, nmax - 1);
      float lf = (float)Lc[i];
      p[i] = wx[i] * lf;
      q[i] = (w[i] * lf) * lf;
    }
    float slx_c = psum<N>(p), sl2_c = psum<N>(q);
    if (sl2_c > 0.0f && slx_c * slx_c > best * sl2_c && !dead) {
      float s_c = slx_c / sl2_c;
#pragma unroll
      for (int i = 0; i < N; ++i) L[i] = Lc[i];
      scale = s_c;
      best = s_c * slx_c;
    }
  }
  if (dead) {
    scale = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) L[i] = 0;
  }
#pragma unroll
  for (int i = 0; i < N; ++i) L[i] += nmax;
  return scale;
}

// Coordinate descent on fixed-grid codes, elements visited in order, at most 5
// sweeps, stopping after a sweep without a move (kquant.py:152-174, :208-230).
// SIGNED selects the make_q3_quants rules (codes clipped to [lo, hi], the new
// suml2 must stay positive) versus make_qp_quants (codes capped at hi, both
// partial sums must be positive).
template <int N, bool SIGNED>
__device__ __forceinline__ void descend(const float (&x)[N], const float (&w)[N], float (&Lf)[N],
                                        float* slx_io, float* sl2_io, int lo, int hi,
                                        bool active) {
  float slx = *slx_io, sl2 = *sl2_io;
  for (int sweep = 0; sweep < 5 && active; ++sweep) {
    bool moved = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      float wxi = w[i] * x[i];
      float slx_o = slx - wxi * Lf[i];
      float sl2_o = sl2 - (w[i] * Lf[i]) * Lf[i];
      bool ok = SIGNED ? (slx_o > 0.0f) : (slx_o > 0.0f && sl2_o > 0.0f);
      int qi = rint_magic((x[i] * sl2_o) / (slx_o == 0.0f ? 1.0f : slx_o));
      qi = SIGNED ? clampi(qi, lo, hi) : (qi < hi ? qi : hi);
      float qf = (float)qi;
      float slx_n = slx_o + wxi * qf;
      float sl2_n = sl2_o + (w[i] * qf) * qf;
      bool take = ok && qf != Lf[i] && (slx_n * slx_n) * sl2 > (slx * slx) * sl2_n;
      if (SIGNED) take = take && sl2_n > 0.0f;
      if (take) {
        Lf[i] = qf;
        slx = slx_n;
        sl2 = sl2_n;
        moved = true;
      }
    }
    active = moved;
  }
  *slx_io = slx;
  *sl2_io = sl2;
}

// make_q3_quants on one 16-value sub-block: returns scale, L receives codes + nmax.
__device__ __forceinline__ float fit_signed_descent16(const float (&x)[16], int nmax,
                                                      int (&L)[16]) {
  float amax = fabsf(x[0]), sext = x[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    float a = fabsf(x[i]);
    if (a > amax) {
      amax = a;
      sext = x[i];
    }
  }
  const bool dead = amax < 1e-15f;
  sext = dead ? 1.0f : sext;
  float inv = -(float)nmax / sext;
  float w[16], Lf[16], p[16], q[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    w[i] = x[i] * x[i];
    Lf[i] = (float)clampi(rint_magic(inv * x[i]), -nmax, nmax - 1);
    p[i] = (w[i] * x[i]) * Lf[i];
    q[i] = (w[i] * Lf[i]) * Lf[i];
  }
  float slx = psum<16>(p), sl2 = psum<16>(q);
  descend<16, true>(x, w, Lf, &slx, &sl2, -nmax, nmax - 1, !dead);
  float scale = sl2 > 0.0f ? slx / sl2 : 0.0f;
  if (dead) scale = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) L[i] = (dead ? 0 : (int)Lf[i]) + nmax;
  return scale;
}

// make_qp_quants over a G-lane vector (lane g holds x[g], w[g]). The candidate
// search runs lane-parallel with butterfly sums. The descent is sequential, so
// every lane replays it on gathered copies. Returns d; *Lout receives this
// lane's code. Lanes with ``run_descent`` false skip the descent (they must
// not use *Lout).
template <int G>
__device__ __forceinline__ float gfit_nonneg_search(float x, float w, int nmax, float* inv_out,
                                                    bool* dead_out) {
  float top = gmax<G>(x);
  const bool dead = top < 1e-15f;
  top = dead ? 1.0f : top;
  float inv = (float)nmax / top;
  float L0 = (float)rint_magic(inv * x);
  float r = x - (1.0f / inv) * L0;
  float best = gsum<G>((w * r) * r);
  for (int s = -4; s <= 4; ++s) {
    if (s == 0) continue;
    float inv_c = (0.1f * (float)s + (float)nmax) / top;
    int li = rint_magic(inv_c * x);
    float lc = (float)(li < nmax ? li : nmax);
    float rc = x - (1.0f / inv_c) * lc;
    float e_c = gsum<G>((w * rc) * rc);
    if (e_c < best && !dead) {
      best = e_c;
      inv = inv_c;
    }
  }
  *inv_out = inv;
  *dead_out = dead;
  return top;
}

// Descent half of make_qp_quants on gathered copies; returns d and fills Lf.
template <int G>
__device__ __forceinline__ float nonneg_descent(const float (&xs)[G], const float (&ws)[G],
                                                float inv, bool dead, int nmax,
                                                float (&Lf)[G]) {
  float p[G], q[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    int li = rint_magic(inv * xs[i]);
    Lf[i] = (float)(li < nmax ? li : nmax);
    p[i] = (ws[i] * xs[i]) * Lf[i];
    q[i] = (ws[i] * Lf[i]) * Lf[i];
  }
  float slx = psum<G>(p), sl2 = psum<G>(q);
  descend<G, false>(xs, ws, Lf, &slx, &sl2, 0, nmax, !dead);
  float d = sl2 > 0.0f ? slx / sl2 : 0.0f;
  if (dead) {
    d = 0.0f;
#pragma unroll
    for (int i = 0; i < G; ++i) Lf[i] = 0.0f;
  }
  return d;
}

// The make_qp_quants problems of one workgroup, staged in LDS: P vectors of G values
// (two per superblock, its scales then its mins, sharing one weight vector), the
// candidate search's inverse scale and dead flag of each, and the descent's results.
// Rows are padded to G + 1 floats, so the lanes of the descent, one row each, read
// distinct banks.
template <int G, int P>
struct QpStage {
  float x[P][G + 1];
  float w[P / 2][G + 1];
  float inv[P];
  int dead[P];
  float d[P];
  uint8_t L[P][G];
};

// make_qp_quants for the two G-vectors of every superblock of the workgroup (the
// super-block scales and mins; group ``grp`` of the workgroup's P / 2 superblocks, this
// lane holding element g of a, b and their weights w). The candidate search runs
// lane-parallel with butterfly sums in each lane group. The coordinate descent is
// sequential along a vector, so one lane per vector runs it: lanes 0 .. P - 1 of the
// workgroup's first wave (P <= 64), instead of every lane of a group replaying its
// group's descent. Every wave of the workgroup must call this (two barriers).
// Returns this lane's (d_a, La) and (d_b, Lb).
template <int G, int P>
__device__ __forceinline__ void gfit_nonneg_pair(float a, float b, float w, int nmax, int g,
                                                 int grp, QpStage<G, P>& st, float* da, int* La,
                                                 float* db, int* Lb) {
  static_assert(P <= 64, "one lane per vector in the first wave");
  float inv_a, inv_b;
  bool dead_a, dead_b;
  gfit_nonneg_search<G>(a, w, nmax, &inv_a, &dead_a);
  gfit_nonneg_search<G>(b, w, nmax, &inv_b, &dead_b);
  st.x[2 * grp][g] = a;
  st.x[2 * grp + 1][g] = b;
  st.w[grp][g] = w;
  if (g == 0) {
    st.inv[2 * grp] = inv_a;
    st.inv[2 * grp + 1] = inv_b;
    st.dead[2 * grp] = dead_a;
    st.dead[2 * grp + 1] = dead_b;
  }
  __syncthreads();
  const int p = (int)threadIdx.x;
  if (p < P) {
    float xs[G], ws[G], Lf[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      xs[i] = st.x[p][i];
      ws[i] = st.w[p >> 1][i];
    }
    st.d[p] = nonneg_descent<G>(xs, ws, st.inv[p], st.dead[p] != 0, nmax, Lf);
#pragma unroll
    for (int i = 0; i < G; ++i) st.L[p][i] = (uint8_t)(int)Lf[i];
  }
  __syncthreads();
  *da = st.d[2 * grp];
  *db = st.d[2 * grp + 1];
  *La = st.L[2 * grp][g];
  *Lb = st.L[2 * grp + 1][g];
}

// make_qx_quants (rmse_type 1) over a G-lane vector with weights w: returns the
// scale; *L receives this lane's code + nmax.
template <int G>
__device__ __forceinline__ float gfit_signed(float x, float w, int nmax, int g, int* Lout) {
  float amax;
  float sext = gfirst_absmax<G>(x, g, &amax);
  const bool dead = amax < 1e-15f;
  sext = dead ? 1.0f : sext;
  float wx = w * x;
  float inv = -(float)nmax / sext;
  int L = clampi(rint_magic(inv * x), -nmax, nmax - 1);
  float lf = (float)L;
  float slx = gsum<G>(wx * lf), sl2 = gsum<G>((w * lf) * lf);
  float scale = sl2 != 0.0f ? slx / sl2 : 0.0f;
  float best = scale * slx;
  for (int s = -9; s <= 9; ++s) {
    if (s == 0) continue;
    float inv_c = -((float)nmax + 0.1f * (float)s) / sext;
    int Lc = clampi(rint_magic(inv_c * x), -nmax, nmax - 1);
    float lc = (float)Lc;
    float slx_c = gsum<G>(wx * lc), sl2_c = gsum<G>((w * lc) * lc);
    if (sl2_c > 0.0f && slx_c * slx_c > best * sl2_c && !dead) {
      float s_c = slx_c / sl2_c;
      L = Lc;
      scale = s_c;
      best = s_c * slx_c;
    }
  }
  if (dead) {
    scale = 0.0f;
    L = 0;
  }
  *Lout = L + nmax;
  return scale;
}

}  // namespace cp
