// Optional per-kernel timing: when enabled through ssm_profile_begin(), each
// kernel launch of the library is bracketed by a pair of HIP events recorded
// on the launch stream; ssm_profile_end() synchronizes and reports the summed
// durations per kernel.  Disabled, a launch pays one flag test.
#pragma once

#include <hip/hip_runtime.h>

namespace ssm {

// Records the start event when constructed and the stop event when destroyed.
class ProfScope {
 public:
  ProfScope(const char* name, hipStream_t st);
  ~ProfScope();
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;

 private:
  int slot_;
  hipStream_t st_;
};

}  // namespace ssm
