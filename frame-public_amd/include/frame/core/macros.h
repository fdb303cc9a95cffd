#pragma once
// Export macro and fatal-check macro of the Frame host library.
// Interface follows the reference's include/frame/core/macros.h (FRAME_API, FRAME_CHECK, FRAME_CONCAT), so that
// backend plugins written against Frame compile unchanged.

#include <cstdio>
#include <cstdlib>

#if defined(FRAME_BUILD_SHARED)
#define FRAME_API __attribute__((visibility("default")))
#else
#define FRAME_API
#endif

// Violated caller invariant: print and abort (recoverable errors use Status/Result instead).
#define FRAME_CHECK(condition)                                                                   \
  do {                                                                                           \
    if (!(condition)) {                                                                          \
      std::fprintf(stderr, "FRAME_CHECK failed: %s at %s:%d\n", #condition, __FILE__, __LINE__); \
      std::abort();                                                                              \
    }                                                                                            \
  } while (0)

// Two-level token paste so __COUNTER__ expands before concatenation (registration macros).
#define FRAME_CONCAT_IMPL(a, b) a##b
#define FRAME_CONCAT(a, b) FRAME_CONCAT_IMPL(a, b)
