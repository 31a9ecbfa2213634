// Host-side plumbing shared by the C-ABI entry points: status codes, the
// thread-local error message, and HIP call checking.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/coldpress_hip.h"

namespace cp {

int set_error(int status, const char* fmt, ...);
void clear_error();

inline int hip_fail(hipError_t e, const char* what) {
  return set_error(CP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Block geometry of the supported containers.
struct KqGeom {
  int block_bytes;    // bytes per block
  int sub;            // sub-block width (the scale granularity)
  int block_weights;  // weights per block: 256 (k-quant superblock) or 32 (Q8_0)
};

inline bool kq_geom(int ttype, KqGeom* g) {
  switch (ttype) {
    case CP_Q8_0: *g = {34, 32, 32}; return true;
    case CP_Q2_K: *g = {84, 16, 256}; return true;
    case CP_Q3_K: *g = {110, 16, 256}; return true;
    case CP_Q4_K: *g = {144, 32, 256}; return true;
    case CP_Q5_K: *g = {176, 32, 256}; return true;
    case CP_Q6_K: *g = {210, 16, 256}; return true;
    default: return false;
  }
}

}  // namespace cp

#define CP_HIP(call)                                   \
  do {                                                 \
    hipError_t e_ = (call);                            \
    if (e_ != hipSuccess) return cp::hip_fail(e_, #call); \
  } while (0)

#define CP_LAUNCHED(what)                                  \
  do {                                                     \
    hipError_t e_ = hipGetLastError();                     \
    if (e_ != hipSuccess) return cp::hip_fail(e_, what);   \
  } while (0)
