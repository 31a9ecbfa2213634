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

// Superblock geometry of the supported containers.
struct KqGeom {
  int block_bytes;  // bytes per 256-weight superblock
  int sub;          // sub-block width
};

inline bool kq_geom(int ttype, KqGeom* g) {
  switch (ttype) {
    case CP_Q2_K: *g = {84, 16}; return true;
    case CP_Q3_K: *g = {110, 16}; return true;
    case CP_Q4_K: *g = {144, 32}; return true;
    case CP_Q6_K: *g = {210, 16}; return true;
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
