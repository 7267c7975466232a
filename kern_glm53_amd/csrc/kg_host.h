// Host-side validation helpers of the C ABI: every entry point checks its sizes, pointers and alignment
// before launching and returns hipErrorInvalidValue (1) without launching when a check fails.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define KG_CHECK(cond)                              \
  do {                                              \
    if (!(cond)) return (int)hipErrorInvalidValue;  \
  } while (0)

static inline bool kg_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
