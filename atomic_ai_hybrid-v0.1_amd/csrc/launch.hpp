// Kernel launch helper for the C-ABI entry points: checks each launch and,
// when the caller passed an atomic_profile, records its events around it.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/atomic_hybrid.h"

namespace ah {

struct Launch {
  atomic_profile* prof;
  hipStream_t st;
  int k = 0;
  template <class F>
  int operator()(const char* name, F&& launch) {
    const bool rec = prof && k < prof->capacity && k < ATOMIC_PROFILE_MAX;
    if (rec && hipEventRecord(static_cast<hipEvent_t>(prof->start[k]), st) != hipSuccess)
      return ATOMIC_ERR_LAUNCH;
    launch();
    if (hipGetLastError() != hipSuccess) return ATOMIC_ERR_LAUNCH;
    if (rec) {
      if (hipEventRecord(static_cast<hipEvent_t>(prof->stop[k]), st) != hipSuccess) return ATOMIC_ERR_LAUNCH;
      prof->names[k] = name;
    }
    ++k;
    if (prof) prof->count = k;
    return ATOMIC_OK;
  }
};

}  // namespace ah
