// Host-side helpers shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fxpr.h"

namespace fxpr {

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FXPR_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool valid_int_bits(int b) { return b == 16 || b == 32 || b == 64; }

inline int int_dtype_for_bits(int b) {
  return b == 16 ? FXPR_DTYPE_I16 : (b == 32 ? FXPR_DTYPE_I32 : FXPR_DTYPE_I64);
}

// Largest positive value of a signed b-bit integer.
inline uint64_t qmax_for_bits(int b) { return (uint64_t(1) << (b - 1)) - 1; }

// 2^e as fp32 (host), e in [-126, 127].
inline float pow2f(int e) {
  uint32_t u = static_cast<uint32_t>(e + 127) << 23;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

}  // namespace fxpr
