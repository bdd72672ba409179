// Row-reduction building blocks shared by the row kernels (rows.hip) and the
// greedy sampler (sampling.hip): 16-byte row vectors, workgroup reductions,
// the non-negative quantiser, and the log-softmax's max / exact-sum / lse
// phase, so that the sampler's log-probabilities are the log-softmax's bits.
#pragma once

#include <cmath>
#include <type_traits>

#include "fxp_device.h"
#include "fxpr_internal.h"

namespace fxpr {
namespace rowk {

// N consecutive elements. For N > 1 a native vector, so arrays of them stay
// in registers (a struct holding a plain array is copied with memcpys that
// keep such arrays in scratch memory).
template <typename T, int N, bool = (N > 1)> struct VecImpl { T v[N]; };
template <typename T, int N> struct alignas(sizeof(T) * N) VecImpl<T, N, true> {
  typedef T VT __attribute__((ext_vector_type(N)));
  VT v;
};
template <typename T, int N> using Vec = VecImpl<T, N>;

constexpr int kMaxThreads = 1024;

__device__ __forceinline__ float max_nan(float a, float b) {
  return (a != a || a > b) ? a : b;  // NaN wins, otherwise the larger value
}

__device__ inline float block_max(float v, float* smem) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max_nan(v, __shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  float r = smem[0];
  for (int w = 1; w < nw; ++w) r = max_nan(r, smem[w]);
  return r;
}

using u128 = unsigned __int128;

__device__ __forceinline__ u128 shfl_xor_u128(u128 v, int o) {
  uint64_t lo = static_cast<uint64_t>(v), hi = static_cast<uint64_t>(v >> 64);
  lo = __shfl_xor(lo, o, 64);
  hi = __shfl_xor(hi, o, 64);
  return (static_cast<u128>(hi) << 64) | lo;
}

// Exact workgroup sum of unsigned 64- or 128-bit lane values.
template <class U> __device__ U block_exact_sum(U v, U* smem) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    if constexpr (sizeof(U) == 16) v += shfl_xor_u128(v, o);
    else v += __shfl_xor(v, o, 64);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  U r = smem[0];
  for (int w = 1; w < nw; ++w) r += smem[w];
  return r;
}

__device__ __forceinline__ uint32_t cvt_sat_u32(float integral) {
  // v_cvt_u32_f32 saturates to [0, 2^32 - 1] and maps NaN to 0
  uint32_t o;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(o) : "v"(integral));
  return o;
}

template <int BITS> __device__ __forceinline__ uint64_t quant_nonneg(float s) {
  // s >= 0 or NaN, so the result is in [0, qmax]
  if constexpr (BITS == 64) {
    // RNE, then split r = h 2^32 + l exactly (r integral, h = floor(r 2^-32));
    // branch-free, so arrays of row values around it stay in registers.
    // NaN -> 0; r >= 2^63 -> qmax.
    const float r = __builtin_rintf(s);
    const float h = __builtin_floorf(__fmul_rn(r, 2.3283064365386963e-10f));
    const float l = __fsub_rn(r, __fmul_rn(h, 4294967296.0f));
    const uint64_t v = (static_cast<uint64_t>(cvt_sat_u32(h)) << 32) | cvt_sat_u32(l);
    return v > 0x7fffffffffffffffull ? 0x7fffffffffffffffull : v;
  } else {
    return static_cast<uint64_t>(quant<BITS>(s));
  }
}

inline int threads_for(int64_t nchunks, int per_thread, int max_threads = kMaxThreads) {
  int64_t t = cdiv(nchunks, per_thread);
  t = cdiv(t, 64) * 64;
  if (t < 64) t = 64;
  if (t > max_threads) t = max_threads;
  return static_cast<int>(t);
}

// Log-softmax workgroups are at most 512 threads (two waves per SIMD), so a
// thread may hold 256 registers: a 128256-wide bf16 row stays in registers
// (32 x 16 bytes per thread) next to the exp / log temporaries, unspilled.
constexpr int kLsmThreads = 512;

// quant_nonneg(exp_scaled_to_round(d, f)) by the rounding constant, for
// 1.4143 * 2^f < 2^22 and <= qmax: the scaled value s = p * 2^(k+f) is exact
// (p = 2^r for |r| <= 1/2 is in [0.7071, 1.4143], and k + f >= -116, so 2^(k+f)
// is a normal fp32), fl(s + 1.5 * 2^23) is RNE(s) + 1.5 * 2^23 (the sum lies in
// [2^23, 2^24), spacing 1; the constant is even), no saturation occurs, and
// NaN d was raised to the floor as in exp_scaled_to_round. Returns the sum's
// bit pattern, i.e. the quantised value + 0x4B400000.
// k = rint(t) is taken by the same constant: fl(t + 1.5 * 2^23) - 1.5 * 2^23
// is t rounded half to even (|t| < 116), and the sum's bit pattern is
// 0x4B400000 + k, from which one add-and-shift forms 2^(k+f).
// The caller guarantees d >= exp_zero_below(f) (> -80) or discards the
// result, so the floor clamp of exp_scaled_to_round is not needed here.
__device__ __forceinline__ uint32_t exp_scaled_rc_bits(float d, int f) {
  const float t = __fmul_rn(d, FXPR_LOG2E);
  const float tk = __fadd_rn(t, 12582912.0f);
  const float k = __fsub_rn(tk, 12582912.0f);
  const float r = __fsub_rn(t, k);
  uint32_t s2bits;
  asm("v_add_lshl_u32 %0, %1, %2, 23" : "=v"(s2bits) : "v"(tk), "s"(uint32_t(f + 127) - 0x4B400000u));
  return __float_as_uint(__builtin_fmaf(exp2_poly(r), __uint_as_float(s2bits), 12582912.0f));
}

// A term whose difference to the row maximum is below this quantises to
// exactly 0, so it may be skipped: for d < -(f + 1) ln 2 - 1/16 the exact
// e^d * 2^f is below 0.5 * e^(-1/16) = 0.4697, and the computed value is
// within 6e-6 of it relatively (t = fl(d * log2 e) is off by at most
// 115 * 2^-24 absolutely, the polynomial and its roundings by about 1e-7), so
// it rounds to 0 (and a NaN difference, which compares false, also gives 0).
__host__ __device__ inline float exp_zero_below(int f) { return -(f + 1) * 0.69314718056f - 0.0625f; }

// fl32(v), round half to even, for an unsigned 64- or 128-bit integer. A
// 128-bit value beyond 64 bits is shifted into 64 bits with the dropped bits
// ORed into bit 0 (they lie far below the 24-bit rounding position, so only a
// tie can depend on them), converted, and scaled back exactly.
__device__ __forceinline__ float uint_to_f32(uint64_t v) { return static_cast<float>(v); }
__device__ __forceinline__ float uint_to_f32(u128 v) {
  const uint64_t hi = static_cast<uint64_t>(v >> 64);
  if (hi == 0) return static_cast<float>(static_cast<uint64_t>(v));
  const int n = 64 - __builtin_clzll(hi);
  const u128 dropped = v & ((static_cast<u128>(1) << n) - 1);
  const uint64_t top = static_cast<uint64_t>(v >> n) | (dropped != 0 ? 1u : 0u);
  return __builtin_ldexpf(static_cast<float>(top), n);
}

template <bool WIDE> using LseSum = typename std::conditional<WIDE, u128, uint64_t>::type;

// Exact path: adds RNE_sat_b(exp_scaled(fl32(x_j) - m, f)) of one vector's
// elements to acc. Branch-free (its thresholds, for large f, skip little).
template <int XDT, int VEC, int BITS, class SumT>
__device__ __forceinline__ void add_terms_exact(const Vec<typename Io<XDT>::T, VEC>& xv, float m, int frac,
                                                SumT& acc) {
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const float d = __fsub_rn(Io<XDT>::load(xv.v[j]), m);
    acc += static_cast<SumT>(quant_nonneg<BITS>(exp_scaled_to_round(d, frac)));
  }
}

// Rounding-constant path (same terms): the wave computes an element slot's
// exp only when some lane's difference reaches exp_zero_below (a uniform
// branch: peaked rows skip most slots); the terms it skips are exactly 0.
// The per-lane sum is a plain 32-bit add: the host enables this path only
// when elements per lane x the largest term stay below 2^32.
template <int XDT, int VEC>
__device__ __forceinline__ void add_terms_rc(const Vec<typename Io<XDT>::T, VEC>& xv, float m, int frac,
                                             float zero_below, uint32_t& acc32) {
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const float d = __fsub_rn(Io<XDT>::load(xv.v[j]), m);
    if (__builtin_amdgcn_ballot_w64(d >= zero_below) != 0) {
      const uint32_t q = exp_scaled_rc_bits(d, frac) - 0x4B400000u;
      acc32 += d >= zero_below ? q : 0u;
    }
  }
}

// lse = m + ln(fl32(S) * 2^-f), -inf for S = 0 (so m + lse is NaN for a NaN m).
template <class SumT> __device__ __forceinline__ float lse_of(float m, SumT total, float inv_scale) {
  const float lnS = total == 0 ? -__builtin_inff() : log_own(__fmul_rn(uint_to_f32(total), inv_scale));
  return __fadd_rn(m, lnS);
}

// The log-softmax reduction of one row, shared by every kernel that needs it.
// m = max_j fl32(x_j) (IEEE maximum, NaN propagates: gfx950's
// v_maximum3_f32; the sign of a zero maximum changes no output, as x - m and
// m + ln S come out the same for either zero), S = exact sum_j
// RNE_sat_b(exp_scaled(fl32(x_j) - m, f)), returns lse = m + ln(fl32(S) *
// 2^-f) (-inf for S = 0). The thread's first NREG chunks (chunk c = tid +
// i * blockDim.x) are left in keep[] in their storage type for the caller's
// output pass; later chunks are re-read. fred / ired: kLsmThreads / 64
// entries of shared memory. fast_sum selects the rounding-constant terms with
// 32-bit lane sums (add_terms_rc). WIDE (64-bit terms only) takes 128-bit
// sums.
template <int XDT, int VEC, int NREG, int BITS, bool WIDE>
__device__ __forceinline__ float row_lse(const Vec<typename Io<XDT>::T, VEC>* __restrict__ xr,
                                         Vec<typename Io<XDT>::T, VEC> (&keep)[NREG], int64_t nchunks,
                                         int frac, float inv_scale, int fast_sum, float* fred,
                                         LseSum<WIDE>* ired) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  using SumT = LseSum<WIDE>;
  const int nthr = blockDim.x;
  const int tid = threadIdx.x;

  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * nthr;
    if (c < nchunks) {
      keep[i] = xr[c];
#pragma unroll
      for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(keep[i].v[j]));
    }
  }
  for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) {
    XV xv = xr[c];
#pragma unroll
    for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(xv.v[j]));
  }
  m = block_max(m, fred);

  SumT acc = 0;
  if (BITS != 64 && fast_sum) {
    const float zero_below = exp_zero_below(frac);
    uint32_t acc32 = 0;
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int64_t c = tid + static_cast<int64_t>(i) * nthr;
      if (c < nchunks) add_terms_rc<XDT, VEC>(keep[i], m, frac, zero_below, acc32);
    }
    for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr)
      add_terms_rc<XDT, VEC>(xr[c], m, frac, zero_below, acc32);
    acc = acc32;
  } else {
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int64_t c = tid + static_cast<int64_t>(i) * nthr;
      if (c < nchunks) add_terms_exact<XDT, VEC, BITS>(keep[i], m, frac, acc);
    }
    for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr)
      add_terms_exact<XDT, VEC, BITS>(xr[c], m, frac, acc);
  }
  // The row stays in registers in its storage type: an empty asm "changing"
  // it keeps the compiler from holding every element's fp32 widening (twice
  // the registers) from the sum until the output pass.
  if constexpr (VEC > 1) {
#pragma unroll
    for (int i = 0; i < NREG; ++i) asm volatile("" : "+v"(keep[i].v));
  }
  return lse_of(m, block_exact_sum(acc, ired), inv_scale);
}

// Host side: workgroup size and sum path of a row_lse launch.
struct LseShape {
  int threads;
  int fast_sum;   // rounding-constant terms with 32-bit lane sums
  bool wide;      // 128-bit sums
};

// Whether lanes of lane_elems elements may take the rounding-constant terms
// with 32-bit lane sums: 1.4143 * 2^f below 2^22 and qmax, and a lane's terms
// summing below 2^32.
inline bool lse_fast_sum(int bits, int frac, double lane_elems) {
  const double qmax = double(qmax_for_bits(bits));
  // the largest term: e^0 * 2^f, with margin for the polynomial, or qmax
  const double term_max = std::fmin(1.4143 * std::ldexp(1.0, frac) + 1.0, qmax);
  return bits != 64 && term_max < 4194304.0 && term_max < qmax && lane_elems * term_max < 4294967296.0;
}

inline LseShape lse_shape(int64_t cols, int vec, int nreg, int bits, int frac) {
  LseShape s;
  const int64_t nchunks = cols / vec;
  s.threads = threads_for(nchunks, nreg, kLsmThreads);
  const double term_max = std::fmin(1.4143 * std::ldexp(1.0, frac) + 1.0, double(qmax_for_bits(bits)));
  s.fast_sum = lse_fast_sum(bits, frac, double(cdiv(nchunks, s.threads)) * vec);
  s.wide = double(cols) * term_max >= 18446744073709551616.0;
  return s;
}

}  // namespace rowk
}  // namespace fxpr
