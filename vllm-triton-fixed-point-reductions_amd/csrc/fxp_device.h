// Device-side fixed-point primitives shared by every fxpr kernel (gfx950).
//
// Everything here is bit-for-bit specified: it is restated in numpy by the
// CPU oracle and the two must agree exactly. All fp32 arithmetic is single
// IEEE operations in round-to-nearest-even (the library is compiled with
// -ffp-contract=off so no multiply-add is fused), division and square root
// are the correctly rounded forms.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace fxpr {

// Correctly rounded fp32 square root. HIP's __fsqrt_rn maps to the native
// (approximate) v_sqrt_f32 unless OCML_BASIC_ROUNDED_OPERATIONS is defined;
// the llvm.sqrt builtin gets the corrected IEEE sequence that hipcc emits by
// default (-fhip-fp32-correctly-rounded-divide-sqrt). Plain `/` is likewise
// the correctly rounded division.
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }
// RN(a / b) for many a over one b, from y = RN(1 / b) (div_rn(1, b)):
// q0 = RN(a y) is within a few ulps of a / b, and each correction
// q' = RN(q + RN(a - b q) y) (two FMAs) brings q to RN(a / b) once q is
// within an ulp (Markstein's theorem); two corrections. Exact while a / b
// and the residuals a - b q (about 2^-24 a) stay normal: a = 0 or
// |a| in [2^-63, 2^31] with b in [1e-6, 2^31] (the attention outputs) keeps
// every intermediate above 2^-100.
__device__ __forceinline__ float div_rn_by_recip(float a, float b, float y) {
  float q = __fmul_rn(a, y);
  float r = __builtin_fmaf(-b, q, a);
  q = __builtin_fmaf(r, y, q);
  r = __builtin_fmaf(-b, q, a);
  return __builtin_fmaf(r, y, q);
}

// Buffer resource word 3 for raw (unformatted, unswizzled) buffer access on
// gfx9-family parts.
constexpr int kBufferDword3 = 0x00020000;
// A pointer the caller knows to be wave-uniform, as scalar registers (buffer
// resources must be).
template <typename T> __device__ __forceinline__ void* uniform_ptr(const T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(u)), hi = __builtin_amdgcn_readfirstlane(uint32_t(u >> 32));
  return reinterpret_cast<void*>((uint64_t(hi) << 32) | lo);
}

// ---------------------------------------------------------------------------
// Storage types and conversions to / from fp32.

struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16, round half to even; NaN becomes the canonical 0x7FC0 (the
// same rule torch uses on the CPU). The conversion is gfx950's
// v_cvt_pk_bf16_f32 (round half to even, denormals kept); only the NaN
// payload rule is applied on top.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  return f != f ? static_cast<uint16_t>(0x7fc0u) : h;
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> f16, round half to even, of the fp32 value: through the asm the
// conversion cannot fuse with the multiply or FMA that produced f into one
// v_fma_mix*_f16 (a single rounding of the exact product to f16, which
// differs from rounding the fp32 result when that lands on an f16 midpoint).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// I/O element type tags: load one element as fp32, store an fp32 rounded to
// the type (RNE).
template <int DT> struct Io;
template <> struct Io<0> {  // f16
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return f16_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_f16(f); }
};
template <> struct Io<1> {  // bf16
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_bf16(f); }
};
template <> struct Io<2> {  // f32
  using T = float;
  static __device__ __forceinline__ float load(T v) { return v; }
  static __device__ __forceinline__ T store(float f) { return f; }
};
template <> struct Io<3> {  // f64: loaded by rounding to fp32, stored widened
  using T = double;
  static __device__ __forceinline__ float load(T v) { return static_cast<float>(v); }
  static __device__ __forceinline__ T store(float f) { return static_cast<double>(f); }
};

// ---------------------------------------------------------------------------
// float -> fixed. `s` is the already scaled value fl32(x * 2^f).

// v_cvt_i32_f32 saturates out-of-range inputs to INT32_MIN / INT32_MAX and
// maps NaN to 0; fed an integral value it is an exact saturating convert.
__device__ __forceinline__ int32_t cvt_sat_i32(float integral) {
  int32_t o;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(o) : "v"(integral));
  return o;
}

// RNE then saturate to int32; NaN -> 0.
__device__ __forceinline__ int32_t quant_i32(float s) {
  return cvt_sat_i32(__builtin_rintf(s));
}

// RNE then saturate to int16 (held in an int32); NaN -> 0.
__device__ __forceinline__ int32_t quant_i16(float s) {
  int32_t v = quant_i32(s);
  return v < -32768 ? -32768 : (v > 32767 ? 32767 : v);
}

// RNE then saturate to int64; NaN -> 0.
__device__ __forceinline__ int64_t quant_i64(float s) {
  float r = __builtin_rintf(s);
  if (__builtin_fabsf(r) < 2147483648.0f) return static_cast<int64_t>(cvt_sat_i32(r));
  if (r != r) return 0;
  if (r >= 9223372036854775808.0f) return INT64_MAX;
  if (r <= -9223372036854775808.0f) return INT64_MIN;
  return static_cast<int64_t>(r);  // integral and in range: exact
}

template <int BITS> __device__ __forceinline__ int64_t quant(float s) {
  if constexpr (BITS == 16) return quant_i16(s);
  else if constexpr (BITS == 32) return quant_i32(s);
  else return quant_i64(s);
}

// 2^e as an fp32 constant for e in [-126, 127].
__host__ __device__ __forceinline__ float exp2i(int e) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23);
}

// fixed -> float: fl32(q) * 2^-f (int -> fp32 conversion is RNE).
__device__ __forceinline__ float fixed_to_f32(int64_t q, float inv_scale) {
  return __fmul_rn(static_cast<float>(q), inv_scale);
}
__device__ __forceinline__ float fixed_to_f32(int32_t q, float inv_scale) {
  return __fmul_rn(static_cast<float>(q), inv_scale);
}

// ---------------------------------------------------------------------------
// The library's own exp and log (used where results must be reproducible on
// the CPU bit for bit). Method: Cody-Waite style reduction to a power of two
// plus a Taylor polynomial evaluated by Horner's rule, one rounding per
// operation.

// Taylor coefficients of 2^r = sum (ln 2)^i / i! r^i, rounded to fp32.
#define FXPR_EXP2_C1 0.693147180559945309f
#define FXPR_EXP2_C2 0.240226506959100712f
#define FXPR_EXP2_C3 0.0555041086648215800f
#define FXPR_EXP2_C4 0.00961812910762847717f
#define FXPR_EXP2_C5 0.00133335581464284434f
#define FXPR_EXP2_C6 0.000154035303933816099f
#define FXPR_EXP2_C7 1.52527338040598403e-05f
#define FXPR_LOG2E 1.44269504088896341f
#define FXPR_LN2_HI 0.693145751953125f          // 15 significant bits
#define FXPR_LN2_LO 1.42860682030941723e-06f
#define FXPR_SQRT2 1.41421356237309505f
#define FXPR_EXP_FLOOR (-80.0f)

// 2^r for |r| <= 0.5: Horner's rule with fused multiply-adds (v_fma_f32,
// one rounding per step).
__device__ __forceinline__ float exp2_poly(float r) {
  float p = FXPR_EXP2_C7;
  p = __builtin_fmaf(p, r, FXPR_EXP2_C6);
  p = __builtin_fmaf(p, r, FXPR_EXP2_C5);
  p = __builtin_fmaf(p, r, FXPR_EXP2_C4);
  p = __builtin_fmaf(p, r, FXPR_EXP2_C3);
  p = __builtin_fmaf(p, r, FXPR_EXP2_C2);
  p = __builtin_fmaf(p, r, FXPR_EXP2_C1);
  p = __builtin_fmaf(p, r, 1.0f);
  return p;
}

// e^d * 2^f for d <= 0 (d = x - rowmax), 0 when d < -80 or d is NaN.
// t = fl(d*log2e), k = rint(t), r = t - k (exact), result = 2^r * 2^(k+f).
// The power-of-two scaling is exact (no overflow or subnormal for f <= 63
// and d >= -80), so this equals fl32(exp_own(d) * 2^f).
__device__ __forceinline__ float exp_scaled(float d, int f) {
  if (!(d >= FXPR_EXP_FLOOR)) return 0.0f;
  float t = __fmul_rn(d, FXPR_LOG2E);
  float k = __builtin_rintf(t);
  float r = __fsub_rn(t, k);
  return __builtin_ldexpf(exp2_poly(r), static_cast<int>(k) + f);
}

// exp_scaled for a caller that rounds the result to an integer (f <= 63),
// without a branch: d below the floor, or NaN, is raised to the floor, where
// the result is below 2^-52 and rounds to 0 exactly as exp_scaled's 0 does.
__device__ __forceinline__ float exp_scaled_to_round(float d, int f) {
  d = fmaxf(d, FXPR_EXP_FLOOR);  // maxNum: NaN -> the floor
  const float t = __fmul_rn(d, FXPR_LOG2E);
  const float k = __builtin_rintf(t);
  const float r = __fsub_rn(t, k);
  return __builtin_ldexpf(exp2_poly(r), static_cast<int>(k) + f);
}

// ln(y) for a positive normal y: y = m * 2^e with m in (sqrt(1/2), sqrt(2)],
// s = (m - 1) / (m + 1), ln m = 2s * (1 + z/3 + z^2/5 + z^3/7 + z^4/9) with
// z = s^2, ln y = e*ln2_hi + (e*ln2_lo + ln m).
__device__ __forceinline__ float log_own(float y) {
  uint32_t bits = __float_as_uint(y);
  int e = static_cast<int>(bits >> 23) - 127;
  float m = __uint_as_float((bits & 0x007fffffu) | 0x3f800000u);
  if (m > FXPR_SQRT2) {
    m = __fmul_rn(m, 0.5f);
    e += 1;
  }
  float s = div_rn(__fsub_rn(m, 1.0f), __fadd_rn(m, 1.0f));
  float z = __fmul_rn(s, s);
  float p = 0.111111111111111111f;                       // 1/9
  p = __fadd_rn(__fmul_rn(p, z), 0.142857142857142857f);  // 1/7
  p = __fadd_rn(__fmul_rn(p, z), 0.2f);                   // 1/5
  p = __fadd_rn(__fmul_rn(p, z), 0.333333333333333333f);  // 1/3
  p = __fadd_rn(__fmul_rn(p, z), 1.0f);
  float lnm = __fmul_rn(__fmul_rn(s, 2.0f), p);
  float fe = static_cast<float>(e);
  return __fadd_rn(__fmul_rn(fe, FXPR_LN2_HI), __fadd_rn(__fmul_rn(fe, FXPR_LN2_LO), lnm));
}

// ---------------------------------------------------------------------------
// Wave64 / workgroup reductions.

template <typename T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    T w = __shfl_xor(v, o, 64);
    v = v > w ? v : w;
  }
  return v;
}

template <int N, class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
// f(integral_constant<int, i>) for i = 0..N-1, every index a compile-time constant
template <int N, class F> __device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

}  // namespace fxpr
