// Row reductions with integer (fixed-point) accumulation: row sum, RMSNorm
// (+fused residual) and log-softmax.
//
// One workgroup owns one row, so a row never depends on its neighbours
// (batch invariance). Within the row every partial is an integer and the
// cross-lane / cross-wave combine is an exact integer sum (saturated once at
// the end where the op saturates), so the bits do not depend on the
// workgroup size or the reduction tree either. Rows are
// streamed with 16-byte vector loads and, up to NREG vectors per thread, kept
// in registers between the reduction pass and the output pass so x is read
// from HBM once.

#include <atomic>
#include <mutex>

#include "rows_impl.h"

namespace fxpr {
namespace {

using namespace rowk;

// ---------------------------------------------------------------------------
// Exact integer row sum, saturated once to OBITS.

template <int QBITS> struct RowSumTypes;
template <> struct RowSumTypes<16> { using Q = int16_t; using Acc = int64_t; };
template <> struct RowSumTypes<32> { using Q = int32_t; using Acc = int64_t; };
template <> struct RowSumTypes<64> { using Q = int64_t; using Acc = __int128; };

__device__ __forceinline__ int64_t shfl_xor_i64(int64_t v, int o) { return __shfl_xor(v, o, 64); }
__device__ __forceinline__ __int128 shfl_xor_i128(__int128 v, int o) {
  uint64_t lo = static_cast<uint64_t>(v), hi = static_cast<uint64_t>(v >> 64);
  lo = __shfl_xor(lo, o, 64);
  hi = __shfl_xor(hi, o, 64);
  return static_cast<__int128>((static_cast<unsigned __int128>(hi) << 64) | lo);
}

// VEC > 1: rows of 16-byte vectors (cols a multiple of VEC, q 16-byte aligned).
template <int QBITS, int OBITS, int VEC>
__global__ __launch_bounds__(256) void row_sum_kernel(
    const typename RowSumTypes<QBITS>::Q* __restrict__ q, void* __restrict__ out, int64_t cols) {
  using Q = typename RowSumTypes<QBITS>::Q;
  using Acc = typename RowSumTypes<QBITS>::Acc;
  __shared__ Acc smem[4];
  const int64_t row = blockIdx.x;
  const auto* p = q + row * cols;
  Acc acc = 0;
  if constexpr (VEC > 1) {
    using V = Vec<Q, VEC>;
    const V* pv = reinterpret_cast<const V*>(p);
    for (int64_t j = threadIdx.x; j < cols / VEC; j += 256) {
      const V v = pv[j];
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc += static_cast<Acc>(v.v[e]);
    }
  } else {
    for (int64_t j = threadIdx.x; j < cols; j += 256) acc += static_cast<Acc>(p[j]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    if constexpr (QBITS == 64) acc += shfl_xor_i128(acc, o);
    else acc += shfl_xor_i64(acc, o);
  }
  if ((threadIdx.x & 63) == 0) smem[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    Acc t = smem[0] + smem[1] + smem[2] + smem[3];
    const Acc hi = static_cast<Acc>((uint64_t(1) << (OBITS - 1)) - 1);
    const Acc lo = -hi - 1;
    t = t > hi ? hi : (t < lo ? lo : t);
    if constexpr (OBITS == 16) static_cast<int16_t*>(out)[row] = static_cast<int16_t>(t);
    else if constexpr (OBITS == 32) static_cast<int32_t*>(out)[row] = static_cast<int32_t>(t);
    else static_cast<int64_t*>(out)[row] = static_cast<int64_t>(t);
  }
}

template <int QBITS, int VEC>
int launch_row_sum_vec(const void* q, void* out, int obits, int64_t rows, int64_t cols, hipStream_t st) {
  using Q = typename RowSumTypes<QBITS>::Q;
  const Q* qp = static_cast<const Q*>(q);
  dim3 grid(static_cast<unsigned>(rows));
  switch (obits) {
    case 16: row_sum_kernel<QBITS, 16, VEC><<<grid, 256, 0, st>>>(qp, out, cols); break;
    case 32: row_sum_kernel<QBITS, 32, VEC><<<grid, 256, 0, st>>>(qp, out, cols); break;
    default: row_sum_kernel<QBITS, 64, VEC><<<grid, 256, 0, st>>>(qp, out, cols); break;
  }
  return launch_status();
}

// 16-byte loads when every row starts 16-byte aligned.
template <int QBITS>
int launch_row_sum(const void* q, void* out, int obits, int64_t rows, int64_t cols, hipStream_t st) {
  constexpr int VEC = 128 / QBITS;
  if (cols % VEC == 0 && aligned(q, 16)) return launch_row_sum_vec<QBITS, VEC>(q, out, obits, rows, cols, st);
  return launch_row_sum_vec<QBITS, 1>(q, out, obits, rows, cols, st);
}

// ---------------------------------------------------------------------------
// RMSNorm(+residual).
//
// The sum of squares is an integer sum in a per-row block floating-point
// format, so it is independent of the reduction order and cannot overflow:
//   e   = exponent of the row's largest |v| (2^e <= max |v| < 2^(e+1); -126
//         for a zero or subnormal maximum), found as the largest magnitude
//         bit pattern (an exact integer maximum);
//   q_j = RNE(fl32(s_j * s_j) * 2^40) with s_j = ldexp(v_j, -e), |s_j| < 2,
//         so q_j < 2^42 and the 64-bit sum of up to 2^22 terms cannot wrap;
//   mean_sq = ldexp(fl32(T) / H, 2e - 40), one rounding per step;
//   rrms = 1 / sqrt(mean_sq + eps) (IEEE sqrt and division).
// A row whose largest magnitude is inf or NaN takes mean_sq = that value.
// Pass 1 (per element j): v = fl32(x) [+ fl32(r)], kept in registers for the
// register-cached part of the row (the sum needs the unrounded v after the
// row maximum is known); with a residual r <- IO(v).
// Pass 2: u = fl32(IO(v)) (what was stored) or fl32(x); y = IO((u * w) * rrms).

constexpr int kRmsSumFrac = 40;
constexpr int64_t kRmsMaxHidden = int64_t(1) << 22;

// q = RNE(t * 2^40) for 0 <= t < 4: fl64(t * 2^40 + 1.5 * 2^52) holds
// 2^51 + q in its mantissa field (t * 2^40 is exact in fp64 and below 2^42;
// in [2^52, 2^53) the spacing is 1 and the constant is even, so the fma's
// one rounding is RNE with ties to even).
__device__ __forceinline__ uint64_t rms_sq_term(float v, int neg_e) {
  const float s = __builtin_ldexpf(v, neg_e);
  const float t = __fmul_rn(s, s);
  const double d = __builtin_fma(static_cast<double>(t), 1099511627776.0, 6755399441055744.0);
  return static_cast<uint64_t>(__builtin_bit_cast(int64_t, d)) & ((uint64_t(1) << 51) - 1);
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

__device__ uint32_t block_max_u32(uint32_t v, uint32_t* smem) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  uint32_t r = smem[0];
  for (int w = 1; w < nw; ++w) r = r > smem[w] ? r : smem[w];
  return r;
}

// Streamed rows are read and written once: non-temporal 16-byte accesses
// (global_load/store ... nt) keep them from displacing reused lines in the
// caches (RMSNorm [16384, 4096] + residual: 5.80 -> 6.05 TB/s).
typedef unsigned nt_u32x4 __attribute__((ext_vector_type(4)));
template <class V> __device__ __forceinline__ V nt_load(const V* p) {
  if constexpr (sizeof(V) == 16)
    return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p)));
  else
    return *p;
}
template <class V> __device__ __forceinline__ void nt_store(V* p, const V& v) {
  if constexpr (sizeof(V) == 16)
    __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x4, v), reinterpret_cast<nt_u32x4*>(p));
  else
    *p = v;
}

template <int DT, int VEC, int NREG, bool RES>
__global__ __launch_bounds__(kMaxThreads) void rms_norm_kernel(
    const typename Io<DT>::T* __restrict__ x, typename Io<DT>::T* __restrict__ r,
    const typename Io<DT>::T* __restrict__ w, typename Io<DT>::T* __restrict__ y,
    int64_t hidden, float eps) {
  using T = typename Io<DT>::T;
  using V = Vec<T, VEC>;
  __shared__ uint32_t mred[kMaxThreads / 64];
  __shared__ uint64_t sred[kMaxThreads / 64];

  const int64_t row = blockIdx.x;
  const int64_t nchunks = hidden / VEC;
  const int nthr = blockDim.x;
  const int tid = threadIdx.x;
  const V* xr = reinterpret_cast<const V*>(x + row * hidden);
  V* rr = reinterpret_cast<V*>(r + row * hidden);
  const V* wr = reinterpret_cast<const V*>(w);
  V* yr = reinterpret_cast<V*>(y + row * hidden);

  // v = fl32(x) [+ fl32(r)] of one chunk
  auto load_v = [&](int64_t c, float (&v)[VEC]) {
    V xv = nt_load(xr + c);
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = Io<DT>::load(xv.v[j]);
    if constexpr (RES) {
      V rv = nt_load(rr + c);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = __fadd_rn(v[j], Io<DT>::load(rv.v[j]));
    }
  };
  auto store_r = [&](int64_t c, const float (&v)[VEC]) {
    V sv;
#pragma unroll
    for (int j = 0; j < VEC; ++j) sv.v[j] = Io<DT>::store(v[j]);
    nt_store(rr + c, sv);
  };

  float keep[NREG][VEC];
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * nthr;
    if (c < nchunks) {
      load_v(c, keep[i]);
      if constexpr (RES) store_r(c, keep[i]);
#pragma unroll
      for (int j = 0; j < VEC; ++j) mx = max(mx, abs_bits(keep[i][j]));
    }
  }
  // rows longer than the register cache: the residual is written back in the
  // sum pass, after v has been formed from the old residual a second time
  for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) {
    float v[VEC];
    load_v(c, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) mx = max(mx, abs_bits(v[j]));
  }

  const uint32_t mbits = block_max_u32(mx, mred);
  const int biased = static_cast<int>(mbits >> 23);
  const int e = (biased > 1 ? biased : 1) - 127;
  const int neg_e = -e;

  uint64_t acc = 0;
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * nthr;
    if (c < nchunks) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc += rms_sq_term(keep[i][j], neg_e);
    }
  }
  for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) {
    float v[VEC];
    load_v(c, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc += rms_sq_term(v[j], neg_e);
    if constexpr (RES) store_r(c, v);
  }

  const uint64_t total = block_exact_sum(acc, sred);
  float ms = __builtin_ldexpf(div_rn(static_cast<float>(total), static_cast<float>(hidden)),
                              2 * e - kRmsSumFrac);
  if (mbits >= 0x7f800000u) ms = __uint_as_float(mbits);  // inf or NaN
  const float rrms = div_rn(1.0f, sqrt_rn(__fadd_rn(ms, eps)));

  auto pass2 = [&](int64_t c, const float (&u)[VEC]) {
    V wv = wr[c];
    V yv;
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      yv.v[j] = Io<DT>::store(__fmul_rn(__fmul_rn(u[j], Io<DT>::load(wv.v[j])), rrms));
    nt_store(yr + c, yv);
  };

#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * nthr;
    if (c < nchunks) {
      float u[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) u[j] = RES ? Io<DT>::load(Io<DT>::store(keep[i][j])) : keep[i][j];
      pass2(c, u);
    }
  }
  for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) {
    V src = RES ? rr[c] : xr[c];  // residual already holds IO(v)
    float u[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) u[j] = Io<DT>::load(src.v[j]);
    pass2(c, u);
  }
}

template <int DT, int VEC>
int launch_rms_vec(const void* x, void* r, const void* w, void* y, int64_t rows, int64_t hidden,
                   float eps, hipStream_t st) {
  using T = typename Io<DT>::T;
  constexpr int NREG = 4;
  const int64_t nchunks = hidden / VEC;
  const int nthr = threads_for(nchunks, 2);
  dim3 grid(static_cast<unsigned>(rows));
  if (r)
    rms_norm_kernel<DT, VEC, NREG, true><<<grid, nthr, 0, st>>>(
        static_cast<const T*>(x), static_cast<T*>(r), static_cast<const T*>(w), static_cast<T*>(y),
        hidden, eps);
  else
    rms_norm_kernel<DT, VEC, NREG, false><<<grid, nthr, 0, st>>>(
        static_cast<const T*>(x), nullptr, static_cast<const T*>(w), static_cast<T*>(y), hidden, eps);
  return launch_status();
}

template <int DT>
int launch_rms(const void* x, void* r, const void* w, void* y, int64_t rows, int64_t hidden,
               float eps, hipStream_t st) {
  using T = typename Io<DT>::T;
  constexpr int VEC = 16 / sizeof(T);
  const bool vec_ok = hidden % VEC == 0 && aligned(x, 16) && aligned(w, 16) && aligned(y, 16) &&
                      (!r || aligned(r, 16));
  if (vec_ok) return launch_rms_vec<DT, VEC>(x, r, w, y, rows, hidden, eps, st);
  return launch_rms_vec<DT, 1>(x, r, w, y, rows, hidden, eps, st);
}

// ---------------------------------------------------------------------------
// Log-softmax.
//
// Pass 1: m = max_j fl32(x_j) (NaN propagates).
// Pass 2: S = exact sum_j RNE_sat_b(exp_scaled(fl32(x_j) - m, f)). The terms
// saturate at the knob's width, the sum never does: it is a 64-bit integer
// (128-bit when cols * the largest term could reach 2^64), so a near-flat
// full-vocabulary row still normalises.
// lse = m + ln(fl32(S) * 2^-f) (fl32 correctly rounded; ln by log_own; S == 0
// gives -inf).
// Pass 3: y_j = OUT(fl32(x_j) - lse).

// One workgroup per row: row_lse, then y_j = OUT(fl32(x_j) - lse) from the
// chunks kept in registers (later chunks re-read).
template <int XDT, int YDT, int VEC, int NREG, int BITS, bool WIDE>
__global__ __launch_bounds__(kLsmThreads) void log_softmax_kernel(
    const typename Io<XDT>::T* __restrict__ x, typename Io<YDT>::T* __restrict__ y, int64_t cols,
    int frac, float inv_scale, int fast_sum) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  using YV = Vec<typename Io<YDT>::T, VEC>;
  __shared__ float fred[kLsmThreads / 64];
  __shared__ LseSum<WIDE> ired[kLsmThreads / 64];

  const int64_t row = blockIdx.x;
  const int64_t nchunks = cols / VEC;
  const int nthr = blockDim.x;
  const int tid = threadIdx.x;
  const XV* xr = reinterpret_cast<const XV*>(x + row * cols);
  YV* yr = reinterpret_cast<YV*>(y + row * cols);

  XV keep[NREG];
  const float lse = row_lse<XDT, VEC, NREG, BITS, WIDE>(xr, keep, nchunks, frac, inv_scale, fast_sum, fred, ired);

  auto emit = [&](int64_t c, const XV& xv) {
    YV yv;
#pragma unroll
    for (int j = 0; j < VEC; ++j) yv.v[j] = Io<YDT>::store(__fsub_rn(Io<XDT>::load(xv.v[j]), lse));
    yr[c] = yv;
  };
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = tid + static_cast<int64_t>(i) * nthr;
    if (c < nchunks) emit(c, keep[i]);
  }
  for (int64_t c = tid + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) emit(c, xr[c]);
}

// ---------------------------------------------------------------------------
// Split log-softmax, for launches of few long rows. With one workgroup per
// row a CU streams its row in, then computes (the maximum, the exp terms, two
// workgroup reductions) with the memory idle, then streams the output. Here
// 2^split_log2 workgroups (up to kSplitMax) share a row, each holding a
// contiguous span of at most kSplitThreads * kSplitNreg 16-byte vectors in
// registers: a CU runs eight spans at once, and the memory streams one
// span's data while others compute. The workgroups of a row exchange their
// span maxima, then their exact span sums (integers: the row's total, hence
// every output bit, is the one-workgroup kernel's), through a sync region of
// device memory, as tagged words: a 64-bit agent-scope atomic store of
// (tag << 32 | 32-bit value), where the tag is the row's generation, one more
// than the previous launch's. Wave 0 of every workgroup polls the row's words
// (one lane per word, agent-scope atomic loads) until all carry the tag. A
// word is written and read whole, so no ordering between different words is
// needed, hence no fences.
// The host takes this kernel only when the whole grid fits on the GPU at once,
// so normally no poll waits for a workgroup that cannot start. Work of other
// kernels or processes on the CUs can still hold a row's spans back, so the
// poll is bounded (about 2^14 tries of an L2 round trip, milliseconds): a
// workgroup whose poll gives up reads the whole row from HBM and computes
// the row maximum and the exact row sum itself (the same integers, so the
// same bits), still publishing its own words for its siblings.
// Every span reads the generation at its start and counts itself in the
// row's start count later (an atomic add issued with its sum word, whose
// return arrives with the sums poll's first loads); the span that completes
// the count resets it and advances the generation. So the generation moves
// only after every span of the launch has read it: a span that starts late,
// after its siblings gave up waiting and finished, still takes its launch's
// tag, and no word of one launch can carry the next launch's tag. Launches on
// one stream do not overlap, so the next launch finds the count at zero and
// the new generation.

constexpr int kSplitMax = 16;        // workgroups per row, a power of two
constexpr int kSplitRows = 1024;     // rows of one split launch
constexpr int kSplitThreads = 256;
constexpr int kSplitNreg = 8;        // 16-byte vectors per thread
constexpr int kSplitMinVectors = 4096;  // shorter rows take the one-workgroup kernel
constexpr int kSpinLimit = 1 << 14;

struct LsmSync {
  uint32_t generation[kSplitRows];
  uint32_t started[kSplitRows];               // spans of the running launch that have read the generation
  uint64_t maxima[kSplitRows][kSplitMax];     // tag | fp32 bit pattern
  uint64_t sums[kSplitRows][kSplitMax * 4];   // tag | 32 bits of a span sum, low word first
};

// One region per stream that launched a split log-softmax, up to
// kSyncRegions per device (later streams take the one-workgroup kernel).
// Zero-initialised with the code object; calls on one stream are ordered, so
// they never share a region at the same time.
constexpr int kSyncRegions = 16;
__device__ __align__(256) LsmSync lsm_sync[kSyncRegions];

template <class U> __device__ __forceinline__ void store_agent(U* p, U v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class U> __device__ __forceinline__ U load_agent(U* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split launches whose poll gave up at least once per span (read by
// fxpr_debug_lsm_fallbacks; the kernels only add to it).
__device__ unsigned long long lsm_fallbacks;

// Wave 0: lane i < n polls words[i] until all n carry the tag, at most
// `tries` times; the lane's 32-bit value in *val. False if the poll gave up.
__device__ __forceinline__ bool poll_tagged(uint64_t* words, int n, uint32_t tag, uint32_t* val, int tries) {
  const int lane = threadIdx.x & 63;
  uint64_t w = 0;
  bool ok = false;
  for (int it = 0; it < tries; ++it) {
    if (lane < n) w = load_agent(words + lane);
    if (__builtin_amdgcn_ballot_w64(lane < n && uint32_t(w >> 32) != tag) == 0) {
      ok = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  *val = uint32_t(w);
  return ok;
}

// Thread 0, at the end of its span: the span that completed the row's start
// count (`before`, the count it found, is split - 1) resets it and advances
// the generation to the launch's tag.
__device__ __forceinline__ void lsm_advance(LsmSync* sync, int row, int split, uint32_t tag, uint32_t before) {
  if (before == uint32_t(split - 1)) {
    store_agent(&sync->started[row], 0u);
    store_agent(&sync->generation[row], tag);
  }
}

// A span whose poll gave up (workgroup-uniform). It reads the whole row back
// from the input and computes the row's maximum (if that exchange was lost)
// and exact sum itself, publishes its own span sum if it had not yet (late
// siblings may wait for it), writes its span's outputs from the input, and
// arrives. The span's registers are not used: this path never rejoins the
// common one, which keeps its 64 VGPRs without spills.
template <int XDT, int YDT, int VEC, int BITS, int NW>
__device__ __forceinline__ void lsm_span_fallback(
    const Vec<typename Io<XDT>::T, VEC>* xrow, Vec<typename Io<YDT>::T, VEC>* yrow, int64_t nchunks, int64_t lo,
    int n, bool need_max, float m, int frac, float inv_scale, float* fred, uint64_t* ired, LsmSync* sync,
    int row, int part, int split, uint32_t tag, uint32_t before) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  using YV = Vec<typename Io<YDT>::T, VEC>;
  const int tid = threadIdx.x;
  if (need_max) {
    float mr = -__builtin_inff();
    for (int64_t c = tid; c < nchunks; c += kSplitThreads) {
      const XV xv = xrow[c];
#pragma unroll
      for (int j = 0; j < VEC; ++j) mr = __builtin_elementwise_maximum(mr, Io<XDT>::load(xv.v[j]));
    }
    m = block_max(mr, fred);
  }
  uint64_t total = 0, mine = 0;
  for (int64_t c = tid; c < nchunks; c += kSplitThreads) {
    uint64_t t = 0;
    add_terms_exact<XDT, VEC, BITS>(xrow[c], m, frac, t);
    total += t;
    if (c >= lo && c < lo + n) mine += t;
  }
  total = block_exact_sum(total, ired);
  if (need_max) {
    mine = block_exact_sum(mine, ired);
    if (tid < NW)
      store_agent(&sync->sums[row][part * NW + tid], (uint64_t(tag) << 32) | uint32_t(mine >> (32 * tid)));
  }
  const float lse = lse_of(m, total, inv_scale);
  for (int c = tid; c < n; c += kSplitThreads) {
    const XV xv = xrow[lo + c];
    YV yv;
#pragma unroll
    for (int j = 0; j < VEC; ++j) yv.v[j] = Io<YDT>::store(__fsub_rn(Io<XDT>::load(xv.v[j]), lse));
    yrow[lo + c] = yv;
  }
  if (tid == 0) {
    __hip_atomic_fetch_add(&lsm_fallbacks, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (need_max)  // gave up before the sums: not counted yet
      before = __hip_atomic_fetch_add(&sync->started[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lsm_advance(sync, row, split, tag, before);
  }
}

// Eight waves per SIMD (at most 64 VGPRs): eight workgroups per CU.
template <int XDT, int YDT, int VEC, int BITS, bool WIDE>
__global__ __launch_bounds__(kSplitThreads, 8) void log_softmax_split_kernel(
    const typename Io<XDT>::T* __restrict__ x, typename Io<YDT>::T* __restrict__ y, int64_t cols,
    int frac, float inv_scale, int fast_sum, int split_log2, LsmSync* __restrict__ sync, int max_tries,
    int sum_tries) {
  static_assert(!WIDE, "span sums are exchanged as 64-bit values");
  using XV = Vec<typename Io<XDT>::T, VEC>;
  using YV = Vec<typename Io<YDT>::T, VEC>;
  using SumT = LseSum<WIDE>;
  constexpr int NREG = kSplitNreg;
  constexpr int NW = 2;  // 32-bit words of a span sum
  __shared__ float fred[kSplitThreads / 64];
  __shared__ SumT ired[kSplitThreads / 64];
  __shared__ float row_max, row_lse_value;
  __shared__ int lost;  // a poll gave up

  const int split = 1 << split_log2;
  const int row = static_cast<int>(blockIdx.x >> split_log2);
  const int part = static_cast<int>(blockIdx.x & (split - 1));
  const int64_t nchunks = cols / VEC;
  const int64_t per = (nchunks + split - 1) >> split_log2;
  const int64_t lo = part * per;
  const int n = static_cast<int>(max<int64_t>(min<int64_t>(lo + per, nchunks) - lo, 0));
  const int tid = threadIdx.x;
  const bool wave0 = tid < 64;
  const XV* xrow = reinterpret_cast<const XV*>(x + int64_t(row) * cols);
  YV* yrow = reinterpret_cast<YV*>(y + int64_t(row) * cols);
  const XV* xr = xrow + lo;
  YV* yr = yrow + lo;

  // the row's tag, read alongside the span (by every thread: one cache line,
  // and no branch whose join would wait for the load before the span's)
  const uint32_t tag = load_agent(&sync->generation[row]) + 1;
  XV keep[NREG];
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int c = tid + i * kSplitThreads;
    if (c < n) keep[i] = nt_load(xr + c);
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    if (tid + i * kSplitThreads < n) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(keep[i].v[j]));
    }
  }
  m = block_max(m, fred);
  if (wave0) {
    if (tid == 0) store_agent(&sync->maxima[row][part], (uint64_t(tag) << 32) | __float_as_uint(m));
    uint32_t v;
    const bool ok = poll_tagged(sync->maxima[row], split, tag, &v, max_tries);
    float mm = tid < split ? __uint_as_float(v) : -__builtin_inff();
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) mm = __builtin_elementwise_maximum(mm, __shfl_xor(mm, o, 64));
    if (tid == 0) {
      row_max = mm;
      lost = ok ? 0 : 1;
    }
  }
  __syncthreads();
  if (lost != 0) {  // workgroup-uniform; the siblings are late: no sum exchange either
    lsm_span_fallback<XDT, YDT, VEC, BITS, NW>(xrow, yrow, nchunks, lo, n, true, 0.f, frac, inv_scale, fred, ired,
                                              sync, row, part, split, tag, 0u);
    return;
  }
  m = row_max;

  SumT acc = 0;
  if (BITS != 64 && fast_sum) {
    const float zero_below = exp_zero_below(frac);
    uint32_t acc32 = 0;
#pragma unroll
    for (int i = 0; i < NREG; ++i)
      if (tid + i * kSplitThreads < n) add_terms_rc<XDT, VEC>(keep[i], m, frac, zero_below, acc32);
    acc = acc32;
  } else {
#pragma unroll
    for (int i = 0; i < NREG; ++i)
      if (tid + i * kSplitThreads < n) add_terms_exact<XDT, VEC, BITS>(keep[i], m, frac, acc);
  }
  if constexpr (VEC > 1) {
#pragma unroll
    for (int i = 0; i < NREG; ++i) asm volatile("" : "+v"(keep[i].v));
  }
  const SumT span_sum = block_exact_sum(acc, ired);
  uint32_t before = 0;
  if (wave0) {
    if (tid < NW)
      store_agent(&sync->sums[row][part * NW + tid], (uint64_t(tag) << 32) | uint32_t(span_sum >> (32 * tid)));
    // count this span in the row's start count (it read the generation long
    // ago); the atomic's return comes with the poll's first loads
    if (tid == 0)
      before = __hip_atomic_fetch_add(&sync->started[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t v;
    const bool ok = poll_tagged(sync->sums[row], split * NW, tag, &v, sum_tries);
    SumT total = tid < split * NW ? static_cast<SumT>(v) << (32 * (tid % NW)) : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) total += __shfl_xor(total, o, 64);
    if (tid == 0) {
      row_lse_value = lse_of(m, total, inv_scale);
      lost = ok ? 0 : 1;
      if (ok) lsm_advance(sync, row, split, tag, before);
    }
  }
  __syncthreads();
  if (lost != 0) {  // workgroup-uniform: the row sum from the input (own sum already published)
    lsm_span_fallback<XDT, YDT, VEC, BITS, NW>(xrow, yrow, nchunks, lo, n, false, m, frac, inv_scale, fred, ired,
                                              sync, row, part, split, tag, before);
    return;
  }
  const float lse = row_lse_value;
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int c = tid + i * kSplitThreads;
    if (c < n) {
      YV yv;
#pragma unroll
      for (int j = 0; j < VEC; ++j) yv.v[j] = Io<YDT>::store(__fsub_rn(Io<XDT>::load(keep[i].v[j]), lse));
      nt_store(yr + c, yv);
    }
  }
}

constexpr int kMaxDevices = 64;

int stream_device(hipStream_t st, int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e == hipSuccess && st != nullptr) e = hipStreamGetDevice(st, dev);
  if (e != hipSuccess) return static_cast<int>(e);
  return (*dev < 0 || *dev >= kMaxDevices) ? FXPR_E_ARG : FXPR_OK;
}

// Poll tries of the split kernel for the maxima and for the sums
// (fxpr_debug_set_lsm_spin_limit lowers them to exercise the give-up paths).
std::atomic<int> lsm_max_tries{kSpinLimit}, lsm_sum_tries{kSpinLimit};

std::mutex sync_mu;
struct DeviceSync {
  LsmSync* base = nullptr;
  hipStream_t owner[kSyncRegions] = {};
  int used = 0;
};
DeviceSync device_sync[kMaxDevices];

// The stream's sync region, or nullptr: then the caller takes the
// one-workgroup kernel. The device address of lsm_sync is looked up with the
// device current, never while the stream is capturing.
LsmSync* sync_region(hipStream_t st, int dev) {
  std::lock_guard<std::mutex> lock(sync_mu);
  DeviceSync& d = device_sync[dev];
  if (d.base == nullptr) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess) return nullptr;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(lsm_sync));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return nullptr;
    d.base = static_cast<LsmSync*>(p);
  }
  for (int i = 0; i < d.used; ++i)
    if (d.owner[i] == st) return d.base + i;
  if (d.used == kSyncRegions) return nullptr;
  d.owner[d.used] = st;
  return d.base + d.used++;
}

// Workgroups of the kernel the device holds at once (cached per device).
template <class K> int64_t resident_workgroups(K kernel, int dev) {
  static std::atomic<int64_t> cache[kMaxDevices];
  int64_t c = cache[dev].load(std::memory_order_relaxed);
  if (c > 0) return c;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kSplitThreads, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  c = int64_t(per_cu) * cus;
  cache[dev].store(c, std::memory_order_relaxed);
  return c;
}

// Launches the split kernel if the shape suits it; false: take the
// one-workgroup kernel (nothing launched).
template <int XDT, int YDT, int VEC, int BITS, bool WIDE>
bool try_lsm_split(const void* x, void* y, int64_t rows, int64_t cols, int frac, hipStream_t st,
                   int* rc) {
  const int64_t nchunks = cols / VEC;
  if (rows > kSplitRows || nchunks < kSplitMinVectors) return false;
  int lg = 1;
  while (lg < 4 && cdiv(nchunks, int64_t(1) << lg) > int64_t(kSplitThreads) * kSplitNreg) ++lg;
  if (cdiv(nchunks, int64_t(1) << lg) > int64_t(kSplitThreads) * kSplitNreg) return false;
  auto kernel = log_softmax_split_kernel<XDT, YDT, VEC, BITS, WIDE>;
  int dev = 0;
  if (stream_device(st, &dev) != FXPR_OK) return false;
  if ((rows << lg) > resident_workgroups(kernel, dev)) return false;
  LsmSync* sync = sync_region(st, dev);
  if (sync == nullptr) return false;
  const int fast = BITS != 64 && lse_fast_sum(BITS, frac, double(kSplitNreg) * VEC);
  kernel<<<dim3(static_cast<unsigned>(rows << lg)), kSplitThreads, 0, st>>>(
      static_cast<const typename Io<XDT>::T*>(x), static_cast<typename Io<YDT>::T*>(y), cols, frac,
      pow2f(-frac), fast, lg, sync, lsm_max_tries.load(std::memory_order_relaxed),
      lsm_sum_tries.load(std::memory_order_relaxed));
  *rc = launch_status();
  return true;
}

template <int XDT, int YDT, int VEC>
int launch_lsm_vec(const void* x, void* y, int64_t rows, int64_t cols, int bits, int frac,
                   hipStream_t st) {
  using XT = typename Io<XDT>::T;
  using YT = typename Io<YDT>::T;
  constexpr int NREG = VEC == 1 ? 8 : 32;
  const LseShape sh = lse_shape(cols, VEC, NREG, bits, frac);
  // (128-bit sums, for near-flat rows at large f, keep the one-workgroup kernel)
  if constexpr (VEC > 1) {
    int rc = FXPR_OK;
    bool done = false;
    if (bits == 16) done = try_lsm_split<XDT, YDT, VEC, 16, false>(x, y, rows, cols, frac, st, &rc);
    else if (bits == 32) done = try_lsm_split<XDT, YDT, VEC, 32, false>(x, y, rows, cols, frac, st, &rc);
    else if (!sh.wide) done = try_lsm_split<XDT, YDT, VEC, 64, false>(x, y, rows, cols, frac, st, &rc);
    if (done) return rc;
  }
  const float inv = pow2f(-frac);
  dim3 grid(static_cast<unsigned>(rows));
  const XT* xp = static_cast<const XT*>(x);
  YT* yp = static_cast<YT*>(y);
  const int n = sh.threads;
  if (bits == 16)
    log_softmax_kernel<XDT, YDT, VEC, NREG, 16, false><<<grid, n, 0, st>>>(xp, yp, cols, frac, inv, sh.fast_sum);
  else if (bits == 32)
    log_softmax_kernel<XDT, YDT, VEC, NREG, 32, false><<<grid, n, 0, st>>>(xp, yp, cols, frac, inv, sh.fast_sum);
  else if (!sh.wide)
    log_softmax_kernel<XDT, YDT, VEC, NREG, 64, false><<<grid, n, 0, st>>>(xp, yp, cols, frac, inv, 0);
  else
    log_softmax_kernel<XDT, YDT, VEC, NREG, 64, true><<<grid, n, 0, st>>>(xp, yp, cols, frac, inv, 0);
  return launch_status();
}

template <int XDT, int YDT>
int launch_lsm(const void* x, void* y, int64_t rows, int64_t cols, int bits, int frac, hipStream_t st) {
  using XT = typename Io<XDT>::T;
  using YT = typename Io<YDT>::T;
  constexpr int VEC = 16 / sizeof(XT);
  if (cols % VEC == 0 && aligned(x, 16) && aligned(y, sizeof(YT) * VEC))
    return launch_lsm_vec<XDT, YDT, VEC>(x, y, rows, cols, bits, frac, st);
  return launch_lsm_vec<XDT, YDT, 1>(x, y, rows, cols, bits, frac, st);
}

// ---------------------------------------------------------------------------
// Vocab-parallel log-softmax: rows whose columns are split over devices (a
// vocab-parallel lm_head's logits). Each shard's row maxima, combined by a
// MAX across shards; each shard's exact integer row sums of the same terms as
// the whole-row kernels, against the combined maxima, combined by an integer
// SUM (order-free); then each shard's outputs from the combined maximum and
// sum. The bits equal fxpr_log_softmax on the whole rows while a row's total
// stays below 2^63 (f <= 32 and rows below 2^29 columns).

constexpr int kShardThreads = 256;

template <int XDT, int VEC>
__global__ __launch_bounds__(kShardThreads) void lsm_shard_max_kernel(const typename Io<XDT>::T* __restrict__ x,
                                                                      float* __restrict__ out, int64_t cols) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  __shared__ float fred[kShardThreads / 64];
  const XV* xr = reinterpret_cast<const XV*>(x + int64_t(blockIdx.x) * cols);
  float m = -__builtin_inff();
  for (int64_t c = threadIdx.x; c < cols / VEC; c += kShardThreads) {
    const XV xv = xr[c];
#pragma unroll
    for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(xv.v[j]));
  }
  m = block_max(m, fred);
  if (threadIdx.x == 0) out[blockIdx.x] = m;
}

template <int XDT, int VEC, int BITS>
__global__ __launch_bounds__(kShardThreads) void lsm_shard_sum_kernel(const typename Io<XDT>::T* __restrict__ x,
                                                                      const float* __restrict__ row_max,
                                                                      int64_t* __restrict__ out, int64_t cols,
                                                                      int frac) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  __shared__ uint64_t ired[kShardThreads / 64];
  const XV* xr = reinterpret_cast<const XV*>(x + int64_t(blockIdx.x) * cols);
  const float m = row_max[blockIdx.x];
  uint64_t acc = 0;
  for (int64_t c = threadIdx.x; c < cols / VEC; c += kShardThreads) add_terms_exact<XDT, VEC, BITS>(xr[c], m, frac, acc);
  acc = block_exact_sum(acc, ired);
  if (threadIdx.x == 0) out[blockIdx.x] = static_cast<int64_t>(acc);
}

template <int XDT, int YDT, int VEC>
__global__ __launch_bounds__(kShardThreads) void lsm_shard_finish_kernel(
    const typename Io<XDT>::T* __restrict__ x, const float* __restrict__ row_max,
    const int64_t* __restrict__ row_sum, typename Io<YDT>::T* __restrict__ y, int64_t cols, float inv_scale) {
  using XV = Vec<typename Io<XDT>::T, VEC>;
  using YV = Vec<typename Io<YDT>::T, VEC>;
  const XV* xr = reinterpret_cast<const XV*>(x + int64_t(blockIdx.x) * cols);
  YV* yr = reinterpret_cast<YV*>(y + int64_t(blockIdx.x) * cols);
  const float lse = lse_of(row_max[blockIdx.x], static_cast<uint64_t>(row_sum[blockIdx.x]), inv_scale);
  for (int64_t c = threadIdx.x; c < cols / VEC; c += kShardThreads) {
    const XV xv = xr[c];
    YV yv;
#pragma unroll
    for (int j = 0; j < VEC; ++j) yv.v[j] = Io<YDT>::store(__fsub_rn(Io<XDT>::load(xv.v[j]), lse));
    yr[c] = yv;
  }
}

// 16-byte vectors when the rows allow them, else element by element.
template <int XDT> bool shard_vec(const void* x, int64_t cols, const void* y = nullptr, int y_bytes = 0) {
  constexpr int VEC = 16 / sizeof(typename Io<XDT>::T);
  return cols % VEC == 0 && aligned(x, 16) && (y == nullptr || aligned(y, uintptr_t(y_bytes) * VEC));
}

template <int XDT> int launch_shard_max(const void* x, float* out, int64_t rows, int64_t cols, hipStream_t st) {
  using T = typename Io<XDT>::T;
  constexpr int VEC = 16 / sizeof(T);
  if (shard_vec<XDT>(x, cols))
    lsm_shard_max_kernel<XDT, VEC><<<unsigned(rows), kShardThreads, 0, st>>>(static_cast<const T*>(x), out, cols);
  else
    lsm_shard_max_kernel<XDT, 1><<<unsigned(rows), kShardThreads, 0, st>>>(static_cast<const T*>(x), out, cols);
  return launch_status();
}

template <int XDT, int BITS>
int launch_shard_sum(const void* x, const float* m, int64_t* out, int64_t rows, int64_t cols, int frac,
                     hipStream_t st) {
  using T = typename Io<XDT>::T;
  constexpr int VEC = 16 / sizeof(T);
  if (shard_vec<XDT>(x, cols))
    lsm_shard_sum_kernel<XDT, VEC, BITS><<<unsigned(rows), kShardThreads, 0, st>>>(static_cast<const T*>(x), m,
                                                                                    out, cols, frac);
  else
    lsm_shard_sum_kernel<XDT, 1, BITS><<<unsigned(rows), kShardThreads, 0, st>>>(static_cast<const T*>(x), m, out,
                                                                                  cols, frac);
  return launch_status();
}

template <int XDT, int YDT>
int launch_shard_finish(const void* x, const float* m, const int64_t* s, void* y, int64_t rows, int64_t cols,
                        int frac, hipStream_t st) {
  using XT = typename Io<XDT>::T;
  using YT = typename Io<YDT>::T;
  constexpr int VEC = 16 / sizeof(XT);
  const float inv = pow2f(-frac);
  if (shard_vec<XDT>(x, cols, y, sizeof(YT)))
    lsm_shard_finish_kernel<XDT, YDT, VEC><<<unsigned(rows), kShardThreads, 0, st>>>(
        static_cast<const XT*>(x), m, s, static_cast<YT*>(y), cols, inv);
  else
    lsm_shard_finish_kernel<XDT, YDT, 1><<<unsigned(rows), kShardThreads, 0, st>>>(
        static_cast<const XT*>(x), m, s, static_cast<YT*>(y), cols, inv);
  return launch_status();
}

}  // namespace
}  // namespace fxpr

using namespace fxpr;

extern "C" int fxpr_fixed_row_sum(const void* q, int q_dtype, void* out, int int_bits,
                                  int64_t rows, int64_t cols, void* stream) {
  if (!valid_int_bits(int_bits)) return FXPR_E_BITS;
  if (rows < 0 || cols < 0 || rows > 0x7fffffff) return FXPR_E_SHAPE;
  if (rows == 0) return FXPR_OK;
  if (!q || !out) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  switch (q_dtype) {
    case FXPR_DTYPE_I16: return launch_row_sum<16>(q, out, int_bits, rows, cols, st);
    case FXPR_DTYPE_I32: return launch_row_sum<32>(q, out, int_bits, rows, cols, st);
    case FXPR_DTYPE_I64: return launch_row_sum<64>(q, out, int_bits, rows, cols, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_rms_norm(const void* x, void* residual, const void* weight, void* y,
                             int io_dtype, int64_t rows, int64_t hidden, float eps, void* stream) {
  if (rows < 0 || hidden < 0 || rows > 0x7fffffff || hidden > kRmsMaxHidden) return FXPR_E_SHAPE;
  if (rows == 0 || hidden == 0) return FXPR_OK;
  if (!x || !weight || !y) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  switch (io_dtype) {
    case FXPR_DTYPE_F16: return launch_rms<FXPR_DTYPE_F16>(x, residual, weight, y, rows, hidden, eps, st);
    case FXPR_DTYPE_BF16: return launch_rms<FXPR_DTYPE_BF16>(x, residual, weight, y, rows, hidden, eps, st);
    case FXPR_DTYPE_F32: return launch_rms<FXPR_DTYPE_F32>(x, residual, weight, y, rows, hidden, eps, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_log_softmax(const void* x, int x_dtype, void* y, int y_dtype, int64_t rows,
                                int64_t cols, int int_bits, int frac_bits, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (rows < 0 || cols < 0 || rows > 0x7fffffff || cols > 0x7fffffff) return FXPR_E_SHAPE;
  if (rows == 0 || cols == 0) return FXPR_OK;
  if (!x || !y) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  const bool f32_out = y_dtype == FXPR_DTYPE_F32;
  if (!f32_out && y_dtype != x_dtype) return FXPR_E_DTYPE;
  switch (x_dtype) {
    case FXPR_DTYPE_F16:
      return f32_out ? launch_lsm<FXPR_DTYPE_F16, FXPR_DTYPE_F32>(x, y, rows, cols, int_bits, frac_bits, st)
                     : launch_lsm<FXPR_DTYPE_F16, FXPR_DTYPE_F16>(x, y, rows, cols, int_bits, frac_bits, st);
    case FXPR_DTYPE_BF16:
      return f32_out ? launch_lsm<FXPR_DTYPE_BF16, FXPR_DTYPE_F32>(x, y, rows, cols, int_bits, frac_bits, st)
                     : launch_lsm<FXPR_DTYPE_BF16, FXPR_DTYPE_BF16>(x, y, rows, cols, int_bits, frac_bits, st);
    case FXPR_DTYPE_F32:
      return launch_lsm<FXPR_DTYPE_F32, FXPR_DTYPE_F32>(x, y, rows, cols, int_bits, frac_bits, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_debug_set_lsm_spin_limit(int max_tries, int sum_tries) {
  if (max_tries < 0 || sum_tries < 0) return FXPR_E_ARG;
  lsm_max_tries.store(max_tries, std::memory_order_relaxed);
  lsm_sum_tries.store(sum_tries, std::memory_order_relaxed);
  return FXPR_OK;
}

extern "C" int fxpr_debug_lsm_default_spin_limit(void) { return kSpinLimit; }

extern "C" int fxpr_debug_lsm_fallbacks(unsigned long long* count) {
  if (!count) return FXPR_E_ARG;
  const hipError_t e = hipMemcpyFromSymbol(count, HIP_SYMBOL(lsm_fallbacks), sizeof(*count), 0,
                                           hipMemcpyDeviceToHost);
  return e == hipSuccess ? FXPR_OK : static_cast<int>(e);
}

extern "C" int fxpr_log_softmax_shard_max(const void* x, int x_dtype, float* row_max, int64_t rows, int64_t cols,
                                          void* stream) {
  if (rows < 0 || cols < 0 || rows > 0x7fffffff || cols > 0x7fffffff) return FXPR_E_SHAPE;
  if (rows == 0) return FXPR_OK;
  if (!row_max || (cols > 0 && !x)) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case FXPR_DTYPE_F16: return launch_shard_max<FXPR_DTYPE_F16>(x, row_max, rows, cols, st);
    case FXPR_DTYPE_BF16: return launch_shard_max<FXPR_DTYPE_BF16>(x, row_max, rows, cols, st);
    case FXPR_DTYPE_F32: return launch_shard_max<FXPR_DTYPE_F32>(x, row_max, rows, cols, st);
    default: return FXPR_E_DTYPE;
  }
}

extern "C" int fxpr_log_softmax_shard_sum(const void* x, int x_dtype, const float* row_max, int64_t* row_sum,
                                          int64_t rows, int64_t cols, int int_bits, int frac_bits, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 32) return FXPR_E_BITS;
  if (rows < 0 || cols < 0 || rows > 0x7fffffff || cols >= (int64_t(1) << 29)) return FXPR_E_SHAPE;
  if (rows == 0) return FXPR_OK;
  if (!row_max || !row_sum || (cols > 0 && !x)) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  auto go = [&](auto bits_tag) -> int {
    constexpr int B = decltype(bits_tag)::value;
    switch (x_dtype) {
      case FXPR_DTYPE_F16: return launch_shard_sum<FXPR_DTYPE_F16, B>(x, row_max, row_sum, rows, cols, frac_bits, st);
      case FXPR_DTYPE_BF16:
        return launch_shard_sum<FXPR_DTYPE_BF16, B>(x, row_max, row_sum, rows, cols, frac_bits, st);
      case FXPR_DTYPE_F32: return launch_shard_sum<FXPR_DTYPE_F32, B>(x, row_max, row_sum, rows, cols, frac_bits, st);
      default: return FXPR_E_DTYPE;
    }
  };
  if (int_bits == 16) return go(std::integral_constant<int, 16>{});
  if (int_bits == 32) return go(std::integral_constant<int, 32>{});
  return go(std::integral_constant<int, 64>{});
}

extern "C" int fxpr_log_softmax_shard_finish(const void* x, int x_dtype, const float* row_max,
                                             const int64_t* row_sum, void* y, int y_dtype, int64_t rows,
                                             int64_t cols, int frac_bits, void* stream) {
  if (frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (rows < 0 || cols < 0 || rows > 0x7fffffff || cols > 0x7fffffff) return FXPR_E_SHAPE;
  if (rows == 0 || cols == 0) return FXPR_OK;
  if (!x || !y || !row_max || !row_sum) return FXPR_E_ARG;
  const bool f32_out = y_dtype == FXPR_DTYPE_F32;
  if (!f32_out && y_dtype != x_dtype) return FXPR_E_DTYPE;
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case FXPR_DTYPE_F16:
      return f32_out ? launch_shard_finish<FXPR_DTYPE_F16, FXPR_DTYPE_F32>(x, row_max, row_sum, y, rows, cols,
                                                                           frac_bits, st)
                     : launch_shard_finish<FXPR_DTYPE_F16, FXPR_DTYPE_F16>(x, row_max, row_sum, y, rows, cols,
                                                                           frac_bits, st);
    case FXPR_DTYPE_BF16:
      return f32_out ? launch_shard_finish<FXPR_DTYPE_BF16, FXPR_DTYPE_F32>(x, row_max, row_sum, y, rows, cols,
                                                                            frac_bits, st)
                     : launch_shard_finish<FXPR_DTYPE_BF16, FXPR_DTYPE_BF16>(x, row_max, row_sum, y, rows, cols,
                                                                             frac_bits, st);
    case FXPR_DTYPE_F32:
      return launch_shard_finish<FXPR_DTYPE_F32, FXPR_DTYPE_F32>(x, row_max, row_sum, y, rows, cols, frac_bits, st);
    default: return FXPR_E_DTYPE;
  }
}
