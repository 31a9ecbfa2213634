// Optional per-phase timing of a library call with hipEvents recorded on the
// call's own stream (no synchronization inside the call). A call marks the end
// of each phase; the host reads the summed milliseconds per phase afterwards.
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

namespace cp {

struct PhaseClock {
  bool on = false;
  std::vector<hipEvent_t> ev;
  std::vector<int> label;  // label[i]: phase of the interval ending at ev[i]
  int used = 0;
  hipError_t start(hipStream_t st) {
    used = 0;
    label.clear();
    return mark(-1, st);
  }
  hipError_t mark(int phase, hipStream_t st) {
    if (used == (int)ev.size()) {
      hipEvent_t e;
      hipError_t r = hipEventCreate(&e);
      if (r != hipSuccess) return r;
      ev.push_back(e);
    }
    label.push_back(phase);
    return hipEventRecord(ev[used++], st);
  }
  // out[p] = milliseconds of phase p over the last profiled call (waits for its
  // last event); returns min(nphase, phases) or a hipError as a negative value.
  hipError_t read(float* out, int nphase) {
    for (int p = 0; p < nphase; ++p) out[p] = 0.0f;
    if (used < 2) return hipSuccess;
    hipError_t r = hipEventSynchronize(ev[used - 1]);
    if (r != hipSuccess) return r;
    for (int i = 1; i < used; ++i) {
      float ms = 0.0f;
      r = hipEventElapsedTime(&ms, ev[i - 1], ev[i]);
      if (r != hipSuccess) return r;
      const int p = label[i];
      if (p >= 0 && p < nphase) out[p] += ms;
    }
    return hipSuccess;
  }
};

}  // namespace cp

#define CP_PHASE_MARK(clock, p)                                        \
  do {                                                                 \
    if ((clock).on) CP_HIP((p) < 0 ? (clock).start(st) : (clock).mark((p), st)); \
  } while (0)
