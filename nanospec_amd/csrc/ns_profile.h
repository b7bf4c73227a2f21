// Launch bracketing for the opt-in kernel timing (profile.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace ns {

bool profiling();
void* profile_start(const char* name, hipStream_t st);
void profile_stop(void* token, hipStream_t st);

// Brackets one launch with timing events when profiling is enabled.
struct ScopedLaunch {
  void* token;
  hipStream_t st;
  ScopedLaunch(const char* name, hipStream_t s) : token(profiling() ? profile_start(name, s) : nullptr), st(s) {}
  ~ScopedLaunch() {
    if (token) profile_stop(token, st);
  }
};

}  // namespace ns

#define NS_CONCAT_INNER(a, b) a##b
#define NS_CONCAT(a, b) NS_CONCAT_INNER(a, b)
#define NS_TIMED(name, st) ::ns::ScopedLaunch NS_CONCAT(ns_scoped_launch_, __LINE__)(name, st)
