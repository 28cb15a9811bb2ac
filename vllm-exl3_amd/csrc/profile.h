// Optional per-phase timing: a ring of HIP events recorded on the launch
// stream at the phase boundaries of each instrumented call.  Recording is
// stream-ordered and never synchronises; exl3_profile_end() waits for the
// recorded events and sums the elapsed time of each phase.
#pragma once

#include <hip/hip_runtime.h>

namespace exl3 {

constexpr int kProfilePhases = 8;

// Records boundary `b` (0 = before the first phase) of the current call on
// stream `st`; no-op when profiling is off.  begin_call() must precede the
// boundaries of each call.
void profile_begin_call();
void profile_mark(int b, hipStream_t st);

}  // namespace exl3
