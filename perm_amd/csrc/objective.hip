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
#include "phase_clock.h"

namespace cp {

// Table-held pointers are generic to the compiler; reads through these global
// address-space types become global loads (a flat load also waits on LDS traffic
// and forces the loads ahead of it to drain).
typedef const float __attribute__((address_space(1)))* GF32;
typedef const uint16_t __attribute__((address_space(1)))* GU16;

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
// four never straddle rows). Negative indices count from the end, as numpy's do;
// indices still out of range read element 0 and flag the tensor, whose result
// becomes NaN.
__global__ __launch_bounds__(256) void err_gather_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int n = T.n;
  if (blockIdx.x == 0 && T.qwp) {
    for (int j = threadIdx.x; j < n; j += 256) {
      int c = T.perm ? T.perm[j] : j;
      c = c < 0 ? c + n : c;  // numpy's negative indices
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
  src = src < 0 ? src + T.nrow_src : src;
  bool bad = src < 0 || src >= T.nrow_src;
  src = bad ? 0 : src;
  float v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int c = T.perm ? T.perm[j + k] : j + k;
    c = c < 0 ? c + n : c;
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

// Q8_0: one thread per 4 weights; k-quants: 16 superblocks per workgroup
// (kq_decode_block).
template <int TT>
__global__ __launch_bounds__(256) void err_decode_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int64_t w = (int64_t)T.R * T.n;
  if constexpr (TT == CP_Q8_0) {
    q8_decode_thread(T.raw, w / 32, T.recon, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  } else {
    __shared__ __align__(16) KqDecodeLds<TT> lds;
    kq_decode_block<TT>(T.raw, w / 256, T.recon, blockIdx.x, lds);
  }
}

// --------------------------------------------------------------- column sums
// One lane per column: colerr[c] = (((0 + d2[0,c]) + d2[1,c]) + ...), d2 the
// float64 square of the float64 difference, loads pipelined by chain_rows.
// The sequential chain of one column over rows [r0, r1), loads running one block
// of B rows ahead of the adds. The block after next is always loaded (clamped to
// the last full block), so no branch sits between a load and its use and the
// loads never have to drain early.
template <int B, class T, class Ld, class Use>
__device__ __forceinline__ void chain_rows(int64_t r0, int64_t r1, const Ld& ld, const Use& use) {
  const int64_t nfull = (r1 - r0) / B;
  T a[B], b[B];
  auto fill = [&](T (&v)[B], int64_t r) {
#pragma unroll
    for (int i = 0; i < B; ++i) v[i] = ld(r + i);
  };
  auto drain = [&](const T (&v)[B]) {
#pragma unroll
    for (int i = 0; i < B; ++i) use(v[i]);
  };
  if (nfull > 0) fill(a, r0);
  int64_t k = 0;
  for (; k + 1 < nfull; k += 2) {
    fill(b, r0 + (k + 1) * B);
    drain(a);
    const int64_t ra = r0 + (k + 2) * B;
    fill(a, ra < r1 - B ? ra : r1 - B);  // past the end: a valid block, never used
    drain(b);
  }
  if (k < nfull) drain(a);
  for (int64_t r = r0 + nfull * B; r < r1; ++r) {
    T v = ld(r);
    use(v);
  }
}

__global__ __launch_bounds__(64) void err_colsum_kernel(const ErrDev* __restrict__ tab) {
  const ErrDev& T = tab[blockIdx.y];
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int64_t n = T.n;
  if (c >= n) return;
  const GF32 xs = (GF32)T.xs;
  const GF32 rc = (GF32)T.recon;
  double acc = 0.0;
  chain_rows<16, float2>(
      0, T.R, [&](int64_t r) { return make_float2((xs + r * n)[c], (rc + r * n)[c]); },
      [&](float2 v) {
        const double d = (double)v.y - (double)v.x;
        acc = acc + d * d;
      });
  T.colerr[c] = acc;
}

// --------------------------------------------------------------- pairwise sum
// numpy's summation of a float64 array of n values v(i). It reduces in chunks
// of 8192 values (its ufunc buffer size), adding the chunk sums left to right
// onto +0.0. Inside a chunk the sum is pairwise: fewer than 8 values
// sequentially from 0.0; up to 128 with eight strided accumulators,
// ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), then the remainder; longer runs split at
// n/2 rounded down to a multiple of 8, the two halves summed recursively. The
// recursion runs on an explicit stack (depth <= 32).
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
__device__ double pw_tree(const V& v, int64_t lo0, int64_t n) {
  struct Frame {
    int64_t lo, n;
    double left;
    int right;
  };
  Frame st[32];
  int sp = 0;
  st[0] = Frame{lo0, n, 0.0, 0};
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

constexpr int64_t kNpChunk = 8192;

template <class V>
__device__ double pw_sum(const V& v, int64_t n) {
  double s = 0.0;
  for (int64_t c0 = 0; c0 < n; c0 += kNpChunk) s = s + pw_tree(v, c0, n - c0 < kNpChunk ? n - c0 : kNpChunk);
  return s;
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
    const int64_t n = T.n;
    s = pw_sum([=](int64_t i) {
      const int64_t c = perm ? perm[i] : i;
      return ce[i] * wv[c < 0 ? c + n : c];
    }, T.n);
  } else if (T.qwp) {
    const float* q = T.qwp;
    s = pw_sum([=](int64_t i) { return ce[i] * (double)q[i]; }, T.n);
  } else {
    s = pw_sum([=](int64_t i) { return ce[i]; }, T.n);
  }
  out[T.slot] = s;
}

__global__ void err_clear_kernel(int* __restrict__ bad, int count) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t < count) bad[t] = 0;
}

// --------------------------------------------------------------- col_log_rms
// One lane per (column, chunk of row_step rows): the chunk's float64 sum of
// squares row after row, for many tensors in one launch. A second pass adds the
// chunk sums in order (and takes log(sqrt(acc / nrow) + 1e-12) when asked).
struct ColDev {
  const void* x;
  double* part;  // [nchunk, n] chunk sums
  double* out;   // [n]
  int64_t nrow;
  int n, x_f16, nchunk, col_groups;
};

template <bool F16>
__global__ __launch_bounds__(64) void col_chunk_kernel(const ColDev* __restrict__ tab,
                                                       int64_t row_step) {
  const ColDev& T = tab[blockIdx.y];
  const int chunk = (int)(blockIdx.x / T.col_groups);
  if (chunk >= T.nchunk) return;
  const int c = (int)(blockIdx.x - chunk * T.col_groups) * 64 + threadIdx.x;
  if (c >= T.n) return;
  const int64_t n = T.n;
  const int64_t r0 = (int64_t)chunk * row_step;
  const int64_t r1 = r0 + row_step < T.nrow ? r0 + row_step : T.nrow;
  double acc = 0.0;
  if constexpr (F16) {
    const GU16 x = (GU16)T.x;
    chain_rows<32, uint16_t>(r0, r1, [&](int64_t r) { return (x + r * n)[c]; },
                             [&](uint16_t h) {
                               const double v = (double)half_value(h);
                               acc = acc + v * v;
                             });
  } else {
    const GF32 x = (GF32)T.x;
    chain_rows<32, float>(r0, r1, [&](int64_t r) { return (x + r * n)[c]; },
                          [&](float f) {
                            const double v = (double)f;
                            acc = acc + v * v;
                          });
  }
  T.part[(int64_t)chunk * n + c] = acc;
}

__global__ void col_combine_kernel(const ColDev* __restrict__ tab, int log_rms) {
  const ColDev& T = tab[blockIdx.y];
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= T.n) return;
  double acc = 0.0;
  for (int k = 0; k < T.nchunk; ++k) acc = acc + T.part[(int64_t)k * T.n + c];
  T.out[c] = log_rms ? log(sqrt(acc / (double)T.nrow) + 1e-12) : acc;
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

// Optional per-phase timing (cp_err_profile / cp_err_phase_ms): gather, encode,
// decode, column sums, total.
static thread_local PhaseClock g_err_clock;

template <int TT>
static void launch_err_encode(const ErrDev* tab, const ErrGroup& g, hipStream_t st) {
  int64_t blocks;
  if constexpr (TT == CP_Q8_0) {
    blocks = (g.max_w / 32 + 8 * kWavesPerBlock - 1) / (8 * kWavesPerBlock);
  } else {
    constexpr int S = 64 / Kq<TT>::G;
    blocks = ((g.max_w / 256 + S - 1) / S + kWavesPerBlock - 1) / kWavesPerBlock;
  }
  const dim3 grid((unsigned)blocks, (unsigned)g.count);
  if constexpr (TT == CP_Q8_0)  // no weighted path
    err_encode_kernel<TT, false><<<grid, 256, 0, st>>>(tab + g.first);
  else if (g.imat)
    err_encode_kernel<TT, true><<<grid, 256, 0, st>>>(tab + g.first);
  else
    err_encode_kernel<TT, false><<<grid, 256, 0, st>>>(tab + g.first);
}

template <int TT>
static void launch_err_decode(const ErrDev* tab, const ErrGroup& g, hipStream_t st) {
  // Q8_0: one thread per 4 weights; k-quants: 16 superblocks per workgroup
  const int64_t blocks = TT == CP_Q8_0 ? (g.max_w / 4 + 255) / 256
                                       : (g.max_w / 256 + 4 * kDecSb - 1) / (4 * kDecSb);
  err_decode_kernel<TT><<<dim3((unsigned)blocks, (unsigned)g.count), 256, 0, st>>>(tab + g.first);
}

template <template <int> class L>
static void for_group_type(const ErrDev* tab, const ErrGroup& g, hipStream_t st) {
  switch (g.ttype) {
    case CP_Q8_0: L<CP_Q8_0>::run(tab, g, st); break;
    case CP_Q2_K: L<CP_Q2_K>::run(tab, g, st); break;
    case CP_Q3_K: L<CP_Q3_K>::run(tab, g, st); break;
    case CP_Q4_K: L<CP_Q4_K>::run(tab, g, st); break;
    case CP_Q5_K: L<CP_Q5_K>::run(tab, g, st); break;
    default: L<CP_Q6_K>::run(tab, g, st); break;
  }
}
template <int TT>
struct EncodeL {
  static void run(const ErrDev* t, const ErrGroup& g, hipStream_t st) { launch_err_encode<TT>(t, g, st); }
};
template <int TT>
struct DecodeL {
  static void run(const ErrDev* t, const ErrGroup& g, hipStream_t st) { launch_err_decode<TT>(t, g, st); }
};

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
  CP_PHASE_MARK(g_err_clock, -1);
  err_clear_kernel<<<(count + 255) / 256, 256, 0, st>>>(bad, count);
  err_gather_kernel<<<dim3((unsigned)((max_w / 4 + 255) / 256), (unsigned)count), 256, 0, st>>>(dtab);
  CP_LAUNCHED("objective gather");
  CP_PHASE_MARK(g_err_clock, 0);
  for (const ErrGroup& g : groups) for_group_type<EncodeL>(dtab, g, st);
  CP_LAUNCHED("objective encode");
  CP_PHASE_MARK(g_err_clock, 1);
  for (const ErrGroup& g : groups) for_group_type<DecodeL>(dtab, g, st);
  CP_LAUNCHED("objective decode");
  CP_PHASE_MARK(g_err_clock, 2);
  err_colsum_kernel<<<dim3((unsigned)((max_n + 63) / 64), (unsigned)count), 64, 0, st>>>(dtab);
  CP_LAUNCHED("objective column sums");
  CP_PHASE_MARK(g_err_clock, 3);
  err_final_kernel<<<count, 64, 0, st>>>(dtab, out);
  CP_LAUNCHED("objective total");
  CP_PHASE_MARK(g_err_clock, 4);
  return CP_OK;
}

constexpr int kColPerStore = 64;
struct ColBatch {
  ColDev t[kColPerStore];
};
static_assert(sizeof(ColBatch) <= 4000, "kernel argument block");
static_assert(sizeof(ColDev) % 8 == 0, "table rows are whole 8-byte words");
__global__ void col_store_kernel(ColBatch b, int cn, ColDev* __restrict__ dst) {
  const int words = cn * (int)(sizeof(ColDev) / 8);
  const uint64_t* s = reinterpret_cast<const uint64_t*>(b.t);
  uint64_t* d = reinterpret_cast<uint64_t*>(dst);
  for (int w = threadIdx.x; w < words; w += blockDim.x) d[w] = s[w];
}

size_t col_ws_bytes(const cp_col_tensor* ts, int count, int64_t row_step) {
  size_t o = a256((size_t)count * sizeof(ColDev));
  for (int i = 0; i < count; ++i)
    o += a256((size_t)((ts[i].nrow + row_step - 1) / row_step) * (size_t)ts[i].n * 8);
  return o;
}

int col_sums_batch(const cp_col_tensor* ts, int count, int64_t row_step, int log_rms, void* ws,
                   size_t ws_bytes, hipStream_t st) {
  if (!ts || count <= 0) return set_error(CP_ERR_ARG, "no tensors");
  if (count > 65535) return set_error(CP_ERR_ARG, "at most 65535 tensors per call (got %d)", count);
  if (row_step <= 0) return set_error(CP_ERR_SHAPE, "row_step %lld", (long long)row_step);
  int64_t max_blocks = 0;
  int max_n = 0;
  for (int i = 0; i < count; ++i) {
    const cp_col_tensor& t = ts[i];
    if (!t.x || !t.out) return set_error(CP_ERR_ARG, "tensor %d: null x/out", i);
    if (t.x_dtype != 0 && t.x_dtype != 1) return set_error(CP_ERR_ARG, "tensor %d: x_dtype must be 0 or 1", i);
    if (t.nrow <= 0 || t.n <= 0 || t.n > (1 << 24))
      return set_error(CP_ERR_SHAPE, "tensor %d: x is [%lld, %lld]", i, (long long)t.nrow, (long long)t.n);
    const int64_t nchunk = (t.nrow + row_step - 1) / row_step;
    const int64_t blocks = nchunk * ((t.n + 63) / 64);
    if (nchunk > 0x7FFFFFFF || blocks > 0x7FFFFFFF) return set_error(CP_ERR_SHAPE, "tensor %d: too many row chunks", i);
    if (!aligned(t.x, t.x_dtype ? 2 : 4) || !aligned(t.out, 8))
      return set_error(CP_ERR_ALIGN, "tensor %d: misaligned buffer", i);
    max_blocks = blocks > max_blocks ? blocks : max_blocks;
    max_n = (int)t.n > max_n ? (int)t.n : max_n;
  }
  if (!ws || ws_bytes < col_ws_bytes(ts, count, row_step))
    return set_error(CP_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, col_ws_bytes(ts, count, row_step));
  if (!aligned(ws, 256)) return set_error(CP_ERR_ALIGN, "workspace needs 256-byte alignment");
  char* base = (char*)ws;
  ColDev* dtab = (ColDev*)base;
  size_t o = a256((size_t)count * sizeof(ColDev));
  std::vector<ColDev> devs(count);
  bool any16 = false, any32 = false;
  for (int i = 0; i < count; ++i) {
    const cp_col_tensor& t = ts[i];
    const int nchunk = (int)((t.nrow + row_step - 1) / row_step);
    devs[i] = ColDev{t.x, (double*)(base + o), t.out, t.nrow, (int)t.n, t.x_dtype, nchunk,
                     (int)((t.n + 63) / 64)};
    o += a256((size_t)nchunk * (size_t)t.n * 8);
    (t.x_dtype ? any16 : any32) = true;
  }
  // one table per input dtype: f16 rows first, then f32
  std::stable_partition(devs.begin(), devs.end(), [](const ColDev& d) { return d.x_f16 != 0; });
  int n16 = 0;
  for (const ColDev& d : devs) n16 += d.x_f16 != 0;
  for (int c0 = 0; c0 < count; c0 += kColPerStore) {
    const int cn = count - c0 < kColPerStore ? count - c0 : kColPerStore;
    ColBatch b;
    for (int i = 0; i < cn; ++i) b.t[i] = devs[c0 + i];
    col_store_kernel<<<1, 256, 0, st>>>(b, cn, dtab + c0);
  }
  if (any16)
    col_chunk_kernel<true><<<dim3((unsigned)max_blocks, (unsigned)n16), 64, 0, st>>>(dtab, row_step);
  if (any32)
    col_chunk_kernel<false><<<dim3((unsigned)max_blocks, (unsigned)(count - n16)), 64, 0, st>>>(
        dtab + n16, row_step);
  col_combine_kernel<<<dim3((unsigned)((max_n + 255) / 256), (unsigned)count), 256, 0, st>>>(dtab, log_rms);
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

void cp_err_profile(int enable) { cp::g_err_clock.on = enable != 0; }

int cp_err_phase_ms(float* out, int nphase) {
  cp::clear_error();
  if (!out || nphase <= 0) return cp::set_error(CP_ERR_ARG, "bad phase buffer");
  hipError_t r = cp::g_err_clock.read(out, nphase);
  if (r != hipSuccess) return cp::hip_fail(r, "phase events");
  return nphase < 5 ? nphase : 5;
}

size_t cp_col_sums_ws_bytes(int64_t nrow, int64_t n, int64_t row_step) {
  if (nrow <= 0 || n <= 0 || row_step <= 0) return 0;
  const cp_col_tensor t{nullptr, 0, nrow, n, nullptr};
  return cp::col_ws_bytes(&t, 1, row_step);
}

int cp_col_sq_sums(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* acc, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  const cp_col_tensor t{x, x_dtype, nrow, n, acc};
  return cp::col_sums_batch(&t, 1, row_step, 0, ws, ws_bytes, (hipStream_t)stream);
}

int cp_col_log_rms(const void* x, int x_dtype, int64_t nrow, int64_t n, int64_t row_step,
                   double* out, void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  const cp_col_tensor t{x, x_dtype, nrow, n, out};
  return cp::col_sums_batch(&t, 1, row_step, 1, ws, ws_bytes, (hipStream_t)stream);
}

size_t cp_col_sums_batch_ws_bytes(const cp_col_tensor* tensors, int count, int64_t row_step) {
  if (!tensors || count <= 0 || row_step <= 0) return 0;
  return cp::col_ws_bytes(tensors, count, row_step);
}

int cp_col_sq_sums_batch(const cp_col_tensor* tensors, int count, int64_t row_step, int log_rms,
                         void* ws, size_t ws_bytes, void* stream) {
  cp::clear_error();
  return cp::col_sums_batch(tensors, count, row_step, log_rms != 0, ws, ws_bytes,
                            (hipStream_t)stream);
}

}  // extern "C"
