// PERM container objective on gfx950 (coldpress/perm/objective.py:17-49).
//
// tensor_err(x, ttype, qw, perm, wvec, rows) =
//     sum_c w[c] * sum_r (roundtrip(x[rows][:, perm])[r, c] - x[rows][r, perm[c]])^2
// with w = wvec[perm], qw[perm] or 1, evaluated for many tensors in one pass:
//   gather   x rows (a sorted sample) and permuted columns, f16 or f32 -> f32
//   encode   the container codec bodies of kq_blocks.h, one launch per type group
//   decode   the same decoders as cp_kq_dequantize
//   colsum   per column, the float64 squared errors added row after row -- the
//            order of numpy's d2.sum(0) over a C-contiguous array, so the result is
//            bit-identical
//   final    +0.0 plus numpy's pairwise sum of colerr * w (the order of a
//            contiguous float64 .sum()), one lane per tensor
// col_log_rms(x, row_step) is the per-column float64 sum of squares in row chunks
// (a sequential chain per chunk, the chunk sums added in order), then
// log(sqrt(acc / nrow) + 1e-12).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "kq_blocks.h"

namespace cp {

struct ErrDev {
  const void* x;
  const int32_t* rows;
  const int32_t* perm;
  const float* qw;
  const double* wvec;
  float* xs;       // [R, n] gathered targets
  float* qwp;      // [n] qw[perm] (or null)
  uint8_t* raw;    // [R, n / block_weights * block_bytes]
  float* recon;    // [R, n]
  double* colerr;  // [n]
  int* bad;        // set when an index is out of range
  int64_t nrow_src;
  int R, n, ttype, x_f16;
  int slot;  // the caller's index of this tensor (its result slot)
};

// --------------------------------------------------------------- gather
// Four consecutive columns of one gathered row per thread (n % 32 == 0, so the
// four never straddle rows). Out-of-range indices read element 0 and flag the
// tensor; its result becomes NaN.
__global__ __launch_bounds__(256) void err_gather_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int n = T.n;
  if (blockIdx.x == 0 && T.qwp) {
    for (int j = threadIdx.x; j < n; j += 256) {
      int c = T.perm ? T.perm[j] : j;
      if (c < 0 || c >= n) {
        *T.bad = 1;
        c = 0;
      }
      T.qwp[j] = T.qw[c];
    }
  }
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= (int64_t)T.R * n) return;
  const int i = (int)(e / n), j = (int)(e - (int64_t)i * n);
  int64_t src = T.rows ? T.rows[i] : i;
  bool bad = src < 0 || src >= T.nrow_src;
  src = bad ? 0 : src;
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int c = T.perm ? T.perm[j + k] : j + k;
    if (c < 0 || c >= n) {
      bad = true;
      c = 0;
    }
    const int64_t o = src * n + c;
    v[k] = T.x_f16 ? half_value(reinterpret_cast<const uint16_t*>(T.x)[o])
                   : reinterpret_cast<const float*>(T.x)[o];
  }
  if (bad) *T.bad = 1;
  reinterpret_cast<float4*>(T.xs)[e >> 2] = make_float4(v[0], v[1], v[2], v[3]);
}

// --------------------------------------------------------------- codec
template <int TT, bool IMAT>
__global__ __launch_bounds__(256) void err_encode_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int64_t w = (int64_t)T.R * T.n;
  if constexpr (TT == CP_Q8_0) {
    const int64_t nblk = w / 32;
    if ((int64_t)blockIdx.x * 8 * kWavesPerBlock >= nblk) return;
    q8_encode_block(T.xs, nblk, T.raw, blockIdx.x);
  } else {
    constexpr int S = 64 / Kq<TT>::G;
    const int64_t NB = w / 256;
    const int64_t blocks = ((NB + S - 1) / S + kWavesPerBlock - 1) / kWavesPerBlock;
    if ((int64_t)blockIdx.x >= blocks) return;
    kq_encode_block<TT, IMAT>(T.xs, T.qwp, NB, T.n / 256, T.raw, blockIdx.x);
  }
}

template <int TT>
__global__ __launch_bounds__(256) void err_decode_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t w = (int64_t)T.R * T.n;
  if constexpr (TT == CP_Q8_0)
    q8_decode_thread(T.raw, w / 32, T.recon, t);
  else
    kq_decode_thread<TT>(T.raw, w / 256, T.recon, t);
}

// --------------------------------------------------------------- column sums
// One lane per column: colerr[c] = (((0 + d2[0,c]) + d2[1,c]) + ...), d2 the
// float64 square of the float64 difference. Eight rows of loads are issued
// before their adds.
__global__ __launch_bounds__(64) void err_colsum_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int n = T.n, R = T.R;
  if (c >= n) return;
  const float* xs = T.xs + c;
  const float* rc = T.recon + c;
  double acc = 0.0;
  int r = 0;
  for (; r + 8 <= R; r += 8) {
    float a[8], b[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      a[k] = xs[(int64_t)(r + k) * n];
      b[k] = rc[(int64_t)(r + k) * n];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const double d = (double)b[k] - (double)a[k];
      acc = acc + d * d;
    }
  }
  for (; r < R; ++r) {
    const double d = (double)rc[(int64_t)r * n] - (double)xs[(int64_t)r * n];
    acc = acc + d * d;
  }
  T.colerr[c] = acc;
}

// --------------------------------------------------------------- pairwise sum
// numpy's pairwise summation of a contiguous float64 array of n values v(i):
// fewer than 8 sequentially from 0.0; up to 128 with eight strided accumulators,
// ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the remainder; longer runs split at
// n/2 rounded down to a multiple of 8, the two halves summed recursively. The
// recursion runs on an explicit stack (depth <= 32 for n < 2^36).
template <class V>
__device__ double pw_leaf(const V& v, int64_t lo, int64_t n) {
  if (n < 8) {
    double r = 0.0;
    for (int64_t i = 0; i < n; ++i) r = r + v(lo + i);
    return r;
  }
  double r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = v(lo + j);
  int64_t i = 8;
  for (; i < n - (n % 8); i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) r[j] = r[j] + v(lo + i + j);
  }
  double s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) s = s + v(lo + i);
  return s;
}

template <class V>
__device__ double pw_sum(const V& v, int64_t n) {
  struct Frame {
    int64_t lo, n;
    double left;
    int right;
  };
  Frame st[32];
  int sp = 0;
  st[0] = Frame{0, n, 0.0, 0};
  for (;;) {
    Frame& f = st[sp];
    if (f.n <= 128) {
      double val = pw_leaf(v, f.lo, f.n);
      for (;;) {  // hand the value to the parents
        if (--sp < 0) return val;
        Frame& p = st[sp];
        if (!p.right) {
          p.left = val;
          p.right = 1;
          int64_t n2 = p.n / 2;
          n2 -= n2 % 8;
          st[sp + 1] = Frame{p.lo + n2, p.n - n2, 0.0, 0};
          ++sp;
          break;
        }
        val = p.left + val;
      }
    } else {
      int64_t n2 = f.n / 2;
      n2 -= n2 % 8;
      f.right = 0;
      st[sp + 1] = Frame{f.lo, n2, 0.0, 0};
      ++sp;
    }
  }
}

__global__ __launch_bounds__(64) void err_final_kernel(const ErrDev* __restrict__ tab,
                                                       double* __restrict__ out) {
  if (threadIdx.x != 0) return;
  const ErrDev& T = tab[blockIdx.x];
  if (*T.bad) {
    out[T.slot] = __builtin_nan("");
    return;
  }
  const double* ce = T.colerr;
  double s;
  if (T.wvec) {
    const int32_t* perm = T.perm;
    const double* wv = T.wvec;
    s = pw_sum([=](int64_t i) { return ce[i] * wv[perm ? perm[i] : i]; }, T.n);
  } else if (T.qwp) {
    const float* q = T.qwp;
    s = pw_sum([=](int64_t i) { return ce[i] * (double)q[i]; }, T.n);
  } else {
    s = pw_sum([=](int64_t i) { return ce[i]; }, T.n);
  }
  out[T.slot] = 0.0 + s;
}

__global__ void err_clear_kernel(int* __restrict__ bad, int count) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < count) bad[t] = 0;
}

// --------------------------------------------------------------- col_log_rms
// One lane per (column, chunk of row_step rows): the chunk's float64 sum of
// squares row after row. A second pass adds the chunk sums in order.
template <bool F16>
__global__ __launch_bounds__(64) void col_chunk_kernel(const void* __restrict__ x, int64_t nrow,
                                                       int n, int64_t row_step,
                                                       double* __restrict__ part) {
  const int c = blockIdx.x * 64 + threadIdx.x;
  if (c >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * row_step;
  const int64_t r1 = r0 + row_step < nrow ? r0 + row_step : nrow;
  auto ld = [&](int64_t r) -> double {
    const int64_t o = r * n + c;
    return F16 ? (double)half_value(reinterpret_cast<const uint16_t*>(x)[o])
               : (double)reinterpret_cast<const float*>(x)[o];
  };
  double acc = 0.0;
  int64_t r = r0;
  for (; r + 8 <= r1; r += 8) {
    double v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = ld(r + k);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc = acc + v[k] * v[k];
  }
  for (; r < r1; ++r) {
    const double v = ld(r);
    acc = acc + v * v;
  }
  part[(int64_t)blockIdx.y * n + c] = acc;
}

__global__ void col_combine_kernel(const double* __restrict__ part, int64_t nchunk, int n,
                                   int64_t nrow, int log_rms, double* __restrict__ out) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n) return;
  double acc = 0.0;
  for (int64_t k = 0; k < nchunk; ++k) acc = acc + part[k * n + c];
  out[c] = log_rms ? log(sqrt(acc / (double)nrow) + 1e-12) : acc;
}

// --------------------------------------------------------------- host side

static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

struct ErrLayout {
  size_t xs, qwp, raw, recon, colerr, end;
};

static ErrLayout err_layout(const cp_err_tensor& t, size_t o) {
  KqGeom g;
  kq_geom(t.ttype, &g);
  const int64_t R = t.rows ? t.rows_used : t.nrow;
  ErrLayout L;
  L.xs = o; o += a256((size_t)R * t.n * 4);
  L.qwp = o; o += a256((size_t)t.n * 4);
  L.raw = o; o += a256((size_t)R * (t.n / g.block_weights) * g.block_bytes);
  L.recon = o; o += a256((size_t)R * t.n * 4);
  L.colerr = o; o += a256((size_t)t.n * 8);
  L.end = o;
  return L;
}

static size_t err_tables_bytes(int count) {
  return a256((size_t)count * sizeof(ErrDev)) + a256((size_t)count * sizeof(int));
}

size_t err_ws_bytes(const cp_err_tensor* ts, int count) {
  size_t o = err_tables_bytes(count);
  for (int i = 0; i < count; ++i) o = err_layout(ts[i], o).end;
  return o;
}

constexpr int kErrPerStore = 32;
struct ErrBatch {
  ErrDev t[kErrPerStore];
};
static_assert(sizeof(ErrBatch) <= 4000, "kernel argument block");
__global__ void err_store_kernel(ErrBatch b, int cn, ErrDev* __restrict__ dst) {
  // the table leaves through vector stores, one 8-byte word per lane
  const int words = cn * (int)(sizeof(ErrDev) / 8);
  const uint64_t* s = reinterpret_cast<const uint64_t*>(b.t);
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  for (int w = threadIdx.x; w < words; w += blockDim.x) d[w] = s[w];
}
static_assert(sizeof(ErrDev) % 8 == 0, "table rows are whole 8-byte words");

struct ErrGroup {
  int first, count, ttype;
  bool imat;
  int64_t max_w;  // weights of the largest gathered tensor
};

template <int TT>
static void launch_err_codec(const ErrDev* tab, const ErrGroup& g, hipStream_t st) {
  const dim3 grid_dec((unsigned)((g.max_w / 4 + 255) / 256), (unsigned)g.count);
  int64_t blocks;
  if constexpr (TT == CP_Q8_0) {
    blocks = (g.max_w / 32 + 8 * kWavesPerBlock - 1) / (8 * kWavesPerBlock);
  } else {
    constexpr int S = 64 / Kq<TT>::G;
    blocks = ((g.max_w / 256 + S - 1) / S + kWavesPerBlock - 1) / kWavesPerBlock;
  }
  const dim3 grid_enc((unsigned)blocks, (unsigned)g.count);
  if constexpr (TT == CP_Q8_0)  // no weighted path
    err_encode_kernel<TT, false><<<grid_enc, 256, 0, st>>>(tab + g.first);
  else if (g.imat)
    err_encode_kernel<TT, true><<<grid_enc, 256, 0, st>>>(tab + g.first);
  else
    err_encode_kernel<TT, false><<<grid_enc, 256, 0, st>>>(tab + g.first);
  if constexpr (TT == CP_Q8_0)
    err_decode_kernel<TT><<<grid_dec, 256, 0, st>>>(tab + g.first);
  else
    err_decode_kernel<TT><<<dim3((unsigned)((g.max_w / 256 * 16 + 255) / 256), (unsigned)g.count),
                            256, 0, st>>>(tab + g.first);
}

int err_batch(const cp_err_tensor* ts, int count, void* ws, size_t ws_bytes, double* out,
              hipStream_t st) {
  if (!ts || count <= 0) return set_error(CP_ERR_ARG, "no tensors");
  if (count > 65535) return set_error(CP_ERR_ARG, "at most 65535 tensors per call (got %d)", count);
  if (!out) return set_error(CP_ERR_ARG, "null out");
  for (int i = 0; i < count; ++i) {
    const cp_err_tensor& t = ts[i];
    KqGeom g;
    if (!kq_geom(t.ttype, &g)) return set_error(CP_ERR_TTYPE, "tensor %d: unsupported type %d", i, t.ttype);
    const int64_t R = t.rows ? t.rows_used : t.nrow;
    if (t.nrow <= 0 || t.n <= 0 || t.n % g.block_weights || t.n > (1 << 24) || R <= 0 ||
        R > 0x7FFFFFFF || R * t.n / 4 > (int64_t)0x7FFFFFFF * 256)
      return set_error(CP_ERR_SHAPE, "tensor %d: bad shape [%lld, %lld] (rows used %lld)", i,
                       (long long)t.nrow, (long long)t.n, (long long)R);
    if (t.x_dtype != 0 && t.x_dtype != 1) return set_error(CP_ERR_ARG, "tensor %d: x_dtype must be 0 or 1", i);
    if (!t.x) return set_error(CP_ERR_ARG, "tensor %d: null x", i);
    if (!aligned(t.x, t.x_dtype ? 2 : 4) || (t.qw && !aligned(t.qw, 4)) ||
        (t.wvec && !aligned(t.wvec, 8)))
      return set_error(CP_ERR_ALIGN, "tensor %d: misaligned buffer", i);
  }
  if (!ws || ws_bytes < err_ws_bytes(ts, count))
    return set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, err_ws_bytes(ts, count));
  if (!aligned(ws, 256)) return set_error(CP_ERR_ALIGN, "workspace needs 256-byte alignment");

  char* base = (char*)ws;
  ErrDev* dtab = (ErrDev*)base;
  int* bad = (int*)(base + a256((size_t)count * sizeof(ErrDev)));
  std::vector<ErrDev> devs(count);
  size_t o = err_tables_bytes(count);
  int max_n = 0;
  int64_t max_w = 0;
  for (int i = 0; i < count; ++i) {
    const cp_err_tensor& t = ts[i];
    const ErrLayout L = err_layout(t, o);
    o = L.end;
    const int R = (int)(t.rows ? t.rows_used : t.nrow);
    devs[i] = ErrDev{t.x, t.rows, t.perm, t.qw, t.wvec,
                     (float*)(base + L.xs), t.qw ? (float*)(base + L.qwp) : nullptr,
                     (uint8_t*)(base + L.raw), (float*)(base + L.recon), (double*)(base + L.colerr),
                     bad + i, t.nrow, R, (int)t.n, t.ttype, t.x_dtype, i};
    max_n = (int)t.n > max_n ? (int)t.n : max_n;
    max_w = (int64_t)R * t.n > max_w ? (int64_t)R * t.n : max_w;
  }
  // table ordered by (type, importance) so each codec group is one run of rows
  std::vector<int> order(count);
  for (int i = 0; i < count; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    if (ts[a].ttype != ts[b].ttype) return ts[a].ttype < ts[b].ttype;
    return (ts[a].qw != nullptr) < (ts[b].qw != nullptr);
  });
  std::vector<ErrDev> sorted(count);
  for (int k = 0; k < count; ++k) sorted[k] = devs[order[k]];
  std::vector<ErrGroup> groups;
  for (int k = 0; k < count; ++k) {
    const ErrDev& d = sorted[k];
    const bool imat = d.qw != nullptr;
    const int64_t w = (int64_t)d.R * d.n;
    if (groups.empty() || groups.back().ttype != d.ttype || groups.back().imat != imat)
      groups.push_back(ErrGroup{k, 0, d.ttype, imat, 0});
    ErrGroup& g = groups.back();
    ++g.count;
    g.max_w = w > g.max_w ? w : g.max_w;
  }
  for (int c0 = 0; c0 < count; c0 += kErrPerStore) {
    const int cn = count - c0 < kErrPerStore ? count - c0 : kErrPerStore;
    ErrBatch b;
    for (int i = 0; i < cn; ++i) b.t[i] = sorted[c0 + i];
    err_store_kernel<<<1, 256, 0, st>>>(b, cn, dtab + c0);
  }
  err_clear_kernel<<<(count + 255) / 256, 256, 0, st>>>(bad, count);
  err_gather_kernel<<<dim3((unsigned)((max_w / 4 + 255) / 256), (unsigned)count), 256, 0, st>>>(dtab);
  CP_LAUNCHED("objective gather");
  for (const ErrGroup& g : groups) {
    switch (g.ttype) {
      case CP_Q8_0: launch_err_codec<CP_Q8_0>(dtab, g, st); break;
      case CP_Q2_K: launch_err_codec<CP_Q2_K>(dtab, g, st); break;
      case CP_Q3_K: launch_err_codec<CP_Q3_K>(dtab, g, st); break;
      case CP_Q4_K: launch_err_codec<CP_Q4_K>(dtab, g, st); break;
      case CP_Q5_K: launch_err_codec<CP_Q5_K>(dtab, g, st); break;
      default: launch_err_codec<CP_Q6_K>(dtab, g, st); break;
    }
  }
  CP_LAUNCHED("objective codec");
  err_colsum_kernel<<<dim3((unsigned)((max_n + 63) / 64), (unsigned)count), 64, 0, st>>>(dtab);
  err_final_kernel<<<count, 64, 0, st>>>(dtab, out);
  CP_LAUNCHED("objective reduce");
  return CP_OK;
}

int col_sums(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step, int log_rms,
             double* out, void* ws, size_t ws_bytes, hipStream_t st) {
  if (!x || !out) return set_error(CP_ERR_ARG, "null x/out");
  if (x_dtype != 0 && x_dtype != 1) return set_error(CP_ERR_ARG, "x_dtype must be 0 or 1");
  if (nrow <= 0 || n <= 0 || n > (1 << 24) || row_step <= 0)
    return set_error(CP_ERR_SHAPE, "x is [%lld, %lld], row_step %lld", (long long)nrow,
                     (long long)n, (long long)row_step);
  const int64_t nchunk = (nrow + row_step - 1) / row_step;
  if (nchunk > 65535) return set_error(CP_ERR_SHAPE, "more than 65535 row chunks");
  if (!ws || ws_bytes < (size_t)nchunk * n * 8)
    return set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, (size_t)nchunk * n * 8);
  if (!aligned(x, x_dtype ? 2 : 4) || !aligned(ws, 8) || !aligned(out, 8))
    return set_error(CP_ERR_ALIGN, "misaligned buffer");
  double* part = (double*)ws;
  const dim3 grid((unsigned)((n + 63) / 64), (unsigned)nchunk);
  if (x_dtype)
    col_chunk_kernel<true><<<grid, 64, 0, st>>>(x, nrow, (int)n, row_step, part);
  else
    col_chunk_kernel<false><<<grid, 64, 0, st>>>(x, nrow, (int)n, row_step, part);
  col_combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(part, nchunk, (int)n, nrow,
                                                                   log_rms, out);
  CP_LAUNCHED("column sums");
  return CP_OK;
}

}  // namespace cp

extern "C" {

size_t cp_tensor_err_ws_bytes(const cp_err_tensor* tensors, int count) {
  if (!tensors || count <= 0) return 0;
  for (int i = 0; i < count; ++i) {
    cp::KqGeom g;
    if (!cp::kq_geom(tensors[i].ttype, &g)) return 0;
  }
  return cp::err_ws_bytes(tensors, count);
}

int cp_tensor_err_batch(const cp_err_tensor* tensors, int count, void* ws, size_t ws_bytes,
                        double* out, void* stream) {
  cp::clear_error();
  return cp::err_batch(tensors, count, ws, ws_bytes, out, (hipStream_t)stream);
}

size_t cp_col_sums_ws_bytes(int64_t nrow, int64_t n, int64_t row_step) {
  if (nrow <= 0 || n <= 0 || row_step <= 0) return 0;
  return (size_t)((nrow + row_step - 1) / row_step) * (size_t)n * 8;
}

int cp_col_sq_sums(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* acc, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  return cp::col_sums(x, x_dtype, nrow, n, row_step, 0, acc, ws, ws_bytes, (hipStream_t)stream);
}

int cp_col_log_rms(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* out, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  return cp::col_sums(x, x_dtype, nrow, n, row_step, 1, out, ws, ws_bytes, (hipStream_t)stream);
}

}  // extern "C"
