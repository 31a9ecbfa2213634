// Row / column gathers for the PERM channel permutations (coldpress/perm/spacemaps/
// qwen3.py:141-188 apply_perms, and ef.py:289-290 H[np.ix_(p, p)]).
//
// dst[r][c] = src[row_perm[r]][col_perm[c]] (identity where a permutation is
// NULL), for 1-, 2-, 4- or 8-byte elements. Pure HBM-bound index work: each
// thread writes one output element of a row, so stores are coalesced and the
// gathered loads stay inside one source row. An index outside the axis is
// clamped into it (the host wrapper rejects such permutations before the call),
// so no read ever leaves src.
#include <hip/hip_runtime.h>

#include "cp_host.h"

namespace cp {

template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                     const int* __restrict__ rp,
                                                     const int* __restrict__ cp_, int64_t rows,
                                                     int64_t cols) {
  const int64_t r = blockIdx.y;
  const int64_t sr = rp ? min(max((int64_t)rp[r], (int64_t)0), rows - 1) : r;
  const T* s = src + sr * cols;
  T* o = dst + r * cols;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < cols;
       c += (int64_t)gridDim.x * blockDim.x)
    o[c] = s[cp_ ? min(max((int64_t)cp_[c], (int64_t)0), cols - 1) : c];
}

}  // namespace cp

extern "C" int cp_permute_gather(const void* src, void* dst, const int32_t* row_perm,
                                 const int32_t* col_perm, int64_t rows, int64_t cols,
                                 int elem_bytes, void* stream) {
  cp::clear_error();
  if (rows < 0 || cols < 0 || rows > 0x7FFFFFFF)
    return cp::set_error(CP_ERR_SHAPE, "bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return CP_OK;  // an empty tensor, as numpy indexing of one
  if (!src || !dst) return cp::set_error(CP_ERR_ARG, "null src/dst");
  if (src == dst) return cp::set_error(CP_ERR_ARG, "gather cannot run in place");
  if (!cp::aligned(src, elem_bytes) || !cp::aligned(dst, elem_bytes))
    return cp::set_error(CP_ERR_ALIGN, "buffers need %d-byte alignment", elem_bytes);
  hipStream_t st = (hipStream_t)stream;
  int64_t bx = (cols + 255) / 256;
  if (bx > 64) bx = 64;
  dim3 grid((unsigned)bx, (unsigned)rows);
  switch (elem_bytes) {
    case 1: cp::gather_kernel<uint8_t><<<grid, 256, 0, st>>>((const uint8_t*)src, (uint8_t*)dst, row_perm, col_perm, rows, cols); break;
    case 2: cp::gather_kernel<uint16_t><<<grid, 256, 0, st>>>((const uint16_t*)src, (uint16_t*)dst, row_perm, col_perm, rows, cols); break;
    case 4: cp::gather_kernel<uint32_t><<<grid, 256, 0, st>>>((const uint32_t*)src, (uint32_t*)dst, row_perm, col_perm, rows, cols); break;
    case 8: cp::gather_kernel<uint64_t><<<grid, 256, 0, st>>>((const uint64_t*)src, (uint64_t*)dst, row_perm, col_perm, rows, cols); break;
    default: return cp::set_error(CP_ERR_ARG, "elem_bytes must be 1, 2, 4 or 8 (got %d)", elem_bytes);
  }
  CP_LAUNCHED("permute gather launch");
  return CP_OK;
}
