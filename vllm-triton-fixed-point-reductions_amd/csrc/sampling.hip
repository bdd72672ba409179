// Deterministic greedy sampling with log-probabilities.
//
// Per row of logits: the greedy token is the first element of the row's
// order (largest value first; equal values by ascending index; every NaN
// ranks above +inf; -0 equals +0); the k requested log-probabilities are
// those of the first k elements of the same order. A log-probability is
// fl32(x_j) - lse with lse from row_lse, i.e. exactly the fp32-output
// log_softmax_fxp value of that element.
//
// One workgroup per row (sample_greedy_kernel), the row held in registers as
// in the log-softmax; few rows with a workspace instead spread each row over
// several workgroups (sample_span_kernel, sample_sum_kernel,
// sample_final_kernel below), with the same bits. Selection is by rounds: each round takes the largest 64-bit order key
// below the previous round's, key = order(value) << 32 | (0xfffffffe - j),
// which makes every key of a row distinct, never all ones and never zero.
// One pass keeps each thread's two largest keys (branchless); a round is
// then one workgroup maximum over the threads' heads (one barrier, shared
// slots alternating between rounds), after which only the winning thread
// moves on: its second key becomes its head, and a thread that has given up
// both rescans its elements for the next two below the round's key (rare).
// The first form took every round as a full pass over every element: 5
// rounds over a 128256-wide row cost ~150 us per call.

#include "rows_impl.h"

namespace fxpr {
namespace {

using namespace rowk;

constexpr int kMaxLogprobs = 64;

// Larger value -> larger key; -0 and +0 equal; every NaN above +inf.
__device__ __forceinline__ uint32_t value_order(float v) {
  if (v != v) return 0xffffffffu;
  const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t order_key(float v, int64_t j) {
  return (static_cast<uint64_t>(value_order(v)) << 32) | (0xfffffffeu - static_cast<uint32_t>(j));
}

template <int XDT, int VEC, int NREG, int BITS, bool WIDE>
__global__ __launch_bounds__(kLsmThreads) void sample_greedy_kernel(
    const typename Io<XDT>::T* __restrict__ x, int64_t cols, int rounds, int frac, float inv_scale,
    int fast_sum, int64_t* __restrict__ sampled, float* __restrict__ sampled_logprob,
    int64_t* __restrict__ topk_ids, float* __restrict__ topk_logprobs, int num_logprobs) {
  using XT = typename Io<XDT>::T;
  using XV = Vec<XT, VEC>;
  __shared__ float fred[kLsmThreads / 64];
  __shared__ LseSum<WIDE> ired[kLsmThreads / 64];
  __shared__ uint64_t kred[2][kLsmThreads / 64];

  const int64_t row = blockIdx.x;
  const int64_t nchunks = cols / VEC;
  const int nthr = blockDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
  const XT* xrow = x + row * cols;
  const XV* xr = reinterpret_cast<const XV*>(xrow);

  XV keep[NREG];
  const float lse = row_lse<XDT, VEC, NREG, BITS, WIDE>(xr, keep, nchunks, frac, inv_scale, fast_sum, fred, ired);

  // the thread's two largest keys below `below` (0: none; keys are never 0)
  uint64_t h1 = 0, h2 = 0;
  auto scan = [&](uint64_t below) {
    h1 = 0;
    h2 = 0;
    // keys and indices computed afresh each scan: the empty asm "changing"
    // the row and the thread index keeps the compiler from hoisting every
    // element's 64-bit key out of the rounds (hundreds of live registers)
    int t = tid;
    asm volatile("" : "+v"(t));
    if constexpr (VEC > 1) {
#pragma unroll
      for (int i = 0; i < NREG; ++i) asm volatile("" : "+v"(keep[i].v));
    }
    auto consider = [&](int64_t c, const XV& xv) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        uint64_t key = order_key(Io<XDT>::load(xv.v[j]), c * VEC + j);
        key = key < below ? key : 0;
        const bool gt1 = key > h1, gt2 = key > h2;
        h2 = gt1 ? h1 : (gt2 ? key : h2);
        h1 = gt1 ? key : h1;
      }
    };
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int64_t c = t + static_cast<int64_t>(i) * nthr;
      if (c < nchunks) consider(c, keep[i]);
    }
    for (int64_t c = t + static_cast<int64_t>(NREG) * nthr; c < nchunks; c += nthr) consider(c, xr[c]);
  };
  scan(~uint64_t(0));

  for (int r = 0; r < rounds; ++r) {
    uint64_t best = wave_max(h1);
    if (lane == 0) kred[r & 1][wave] = best;
    __syncthreads();
    best = kred[r & 1][0];
    for (int w = 1; w < nwaves; ++w) best = best > kred[r & 1][w] ? best : kred[r & 1][w];
    if (h1 == best && best != 0) {  // the winner (keys are distinct): its next key below best
      h1 = h2;
      h2 = 0;
      if (h1 == 0 && r + 1 < rounds) scan(best);
    }
    if (tid == 0 && best != 0) {   // k <= cols, so every round finds a key
      const int64_t j = static_cast<int64_t>(0xfffffffeu - static_cast<uint32_t>(best));
      const float lp = __fsub_rn(Io<XDT>::load(xrow[j]), lse);
      if (r == 0) {
        sampled[row] = j;
        sampled_logprob[row] = lp;
      }
      if (r < num_logprobs) {
        topk_ids[row * num_logprobs + r] = j;
        topk_logprobs[row * num_logprobs + r] = lp;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Few rows: the one-workgroup kernel leaves most CUs idle (one row per CU,
// its max, sum and selection passes in sequence). Here S workgroups share a
// row, each over a contiguous span of the row's vectors, in three launches:
//   1. span maximum and the span's first `rounds` order keys (its top keys:
//      keys are distinct, so the row's top keys are among the spans');
//   2. the span's exact integer sum of the row's terms against the row
//      maximum (the maximum of the span maxima);
//   3. per row: the row total (the sum of the span sums: exact integers, any
//      order), lse = lse_of(m, total) as in row_lse, and `rounds` rounds of
//      selection over the spans' keys, with the one-workgroup kernel's outputs.
// The maximum is the IEEE maximum in every kernel (NaN propagates; the sign
// of a zero maximum changes no output), so every output bit equals the
// one-workgroup kernel's. The partials live in a caller's workspace.
constexpr int kSpanThreads = 256;
constexpr int kSpanNreg = 8;
constexpr int kMaxSpans = 16;
constexpr int kMultiMaxRows = 128;   // from here the one-workgroup kernel fills the CUs
constexpr int kFinalThreads = 256;   // kMaxSpans * kMaxLogprobs keys, four per thread
static_assert(kFinalThreads == kSpanThreads, "block_max_key's shared slots are sized for kSpanThreads");
static_assert(kMaxSpans * kMaxLogprobs % kFinalThreads == 0, "whole keys per thread");

__device__ __forceinline__ float block_maximum(float v, float* smem) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = __builtin_elementwise_maximum(v, __shfl_xor(v, o, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if (lane == 0) smem[wave] = v;
  __syncthreads();
  float r = smem[0];
  for (int w = 1; w < nw; ++w) r = __builtin_elementwise_maximum(r, smem[w]);
  return r;
}

// The workgroup's largest key (all threads), shared slots alternating by round.
__device__ __forceinline__ uint64_t block_max_key(uint64_t v, uint64_t (&kred)[2][kSpanThreads / 64], int r) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) kred[r & 1][wave] = v;
  __syncthreads();
  uint64_t best = kred[r & 1][0];
  for (int w = 1; w < nw; ++w) best = best > kred[r & 1][w] ? best : kred[r & 1][w];
  return best;
}

template <int XDT, int VEC>
__global__ __launch_bounds__(kSpanThreads) void sample_span_kernel(
    const typename Io<XDT>::T* __restrict__ x, int64_t cols, int spans, int64_t span_chunks, int rounds,
    float* __restrict__ maxima, uint64_t* __restrict__ cand) {
  using XT = typename Io<XDT>::T;
  using XV = Vec<XT, VEC>;
  constexpr int NREG = kSpanNreg;
  __shared__ float fred[kSpanThreads / 64];
  __shared__ uint64_t kred[2][kSpanThreads / 64];

  const int64_t row = blockIdx.x / spans;
  const int64_t nchunks = cols / VEC;
  const int64_t c0 = (blockIdx.x % spans) * span_chunks;
  const int64_t c1 = min(nchunks, c0 + span_chunks);
  const int nthr = blockDim.x, tid = threadIdx.x;
  const XV* xr = reinterpret_cast<const XV*>(x + row * cols);

  XV keep[NREG];
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < NREG; ++i) {
    const int64_t c = c0 + tid + static_cast<int64_t>(i) * nthr;
    if (c < c1) {
      keep[i] = xr[c];
#pragma unroll
      for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(keep[i].v[j]));
    }
  }
  for (int64_t c = c0 + tid + static_cast<int64_t>(NREG) * nthr; c < c1; c += nthr) {
    const XV xv = xr[c];
#pragma unroll
    for (int j = 0; j < VEC; ++j) m = __builtin_elementwise_maximum(m, Io<XDT>::load(xv.v[j]));
  }
  m = block_maximum(m, fred);
  if (tid == 0) maxima[blockIdx.x] = m;

  // the span's first `rounds` keys, as sample_greedy_kernel selects them
  uint64_t h1 = 0, h2 = 0;
  auto scan = [&](uint64_t below) {
    h1 = 0;
    h2 = 0;
    int t = tid;
    asm volatile("" : "+v"(t));
    if constexpr (VEC > 1) {
#pragma unroll
      for (int i = 0; i < NREG; ++i) asm volatile("" : "+v"(keep[i].v));
    }
    auto consider = [&](int64_t c, const XV& xv) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        uint64_t key = order_key(Io<XDT>::load(xv.v[j]), c * VEC + j);
        key = key < below ? key : 0;
        const bool gt1 = key > h1, gt2 = key > h2;
        h2 = gt1 ? h1 : (gt2 ? key : h2);
        h1 = gt1 ? key : h1;
      }
    };
#pragma unroll
    for (int i = 0; i < NREG; ++i) {
      const int64_t c = c0 + t + static_cast<int64_t>(i) * nthr;
      if (c < c1) consider(c, keep[i]);
    }
    for (int64_t c = c0 + t + static_cast<int64_t>(NREG) * nthr; c < c1; c += nthr) consider(c, xr[c]);
  };
  scan(~uint64_t(0));
  for (int r = 0; r < rounds; ++r) {
    const uint64_t best = block_max_key(h1, kred, r);
    if (h1 == best && best != 0) {
      h1 = h2;
      h2 = 0;
      if (h1 == 0 && r + 1 < rounds) scan(best);
    }
    if (tid == 0) cand[static_cast<int64_t>(blockIdx.x) * rounds + r] = best;  // 0: the span has no more
  }
}

template <int XDT, int VEC, int BITS, bool WIDE>
__global__ __launch_bounds__(kSpanThreads) void sample_sum_kernel(
    const typename Io<XDT>::T* __restrict__ x, int64_t cols, int spans, int64_t span_chunks, int frac,
    int fast_sum, const float* __restrict__ maxima, LseSum<WIDE>* __restrict__ sums) {
  using XT = typename Io<XDT>::T;
  using XV = Vec<XT, VEC>;
  using SumT = LseSum<WIDE>;
  __shared__ SumT ired[kSpanThreads / 64];

  const int64_t row = blockIdx.x / spans;
  const int64_t nchunks = cols / VEC;
  const int64_t c0 = (blockIdx.x % spans) * span_chunks;
  const int64_t c1 = min(nchunks, c0 + span_chunks);
  const XV* xr = reinterpret_cast<const XV*>(x + row * cols);
  float m = -__builtin_inff();
  for (int t = 0; t < spans; ++t) m = __builtin_elementwise_maximum(m, maxima[row * spans + t]);

  SumT acc = 0;
  if (BITS != 64 && fast_sum) {
    const float zero_below = exp_zero_below(frac);
    uint32_t acc32 = 0;
    for (int64_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) add_terms_rc<XDT, VEC>(xr[c], m, frac, zero_below, acc32);
    acc = acc32;
  } else {
    for (int64_t c = c0 + threadIdx.x; c < c1; c += blockDim.x) add_terms_exact<XDT, VEC, BITS>(xr[c], m, frac, acc);
  }
  const SumT total = block_exact_sum(acc, ired);
  if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

template <int XDT, bool WIDE>
__global__ __launch_bounds__(kFinalThreads) void sample_final_kernel(
    const typename Io<XDT>::T* __restrict__ x, int64_t cols, int spans, int rounds, float inv_scale,
    const float* __restrict__ maxima, const LseSum<WIDE>* __restrict__ sums, const uint64_t* __restrict__ cand,
    int64_t* __restrict__ sampled, float* __restrict__ sampled_logprob, int64_t* __restrict__ topk_ids,
    float* __restrict__ topk_logprobs, int num_logprobs) {
  using SumT = LseSum<WIDE>;
  constexpr int KPT = kMaxSpans * kMaxLogprobs / kFinalThreads;  // keys per thread
  __shared__ uint64_t kred[2][kSpanThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  float m = -__builtin_inff();
  SumT total = 0;
  for (int t = 0; t < spans; ++t) {
    m = __builtin_elementwise_maximum(m, maxima[row * spans + t]);
    total += sums[row * spans + t];
  }
  const float lse = lse_of(m, total, inv_scale);

  const int n = spans * rounds;
  const uint64_t* rc = cand + row * n;
  uint64_t key[KPT];
#pragma unroll
  for (int q = 0; q < KPT; ++q) key[q] = tid + q * kFinalThreads < n ? rc[tid + q * kFinalThreads] : 0;
  const auto* xrow = x + row * cols;
  for (int r = 0; r < rounds; ++r) {
    uint64_t mine = 0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) mine = key[q] > mine ? key[q] : mine;
    const uint64_t best = block_max_key(mine, kred, r);
#pragma unroll
    for (int q = 0; q < KPT; ++q) key[q] = key[q] == best ? 0 : key[q];  // keys are distinct
    if (tid == 0 && best != 0) {   // k <= cols, so every round finds a key
      const int64_t j = static_cast<int64_t>(0xfffffffeu - static_cast<uint32_t>(best));
      const float lp = __fsub_rn(Io<XDT>::load(xrow[j]), lse);
      if (r == 0) {
        sampled[row] = j;
        sampled_logprob[row] = lp;
      }
      if (r < num_logprobs) {
        topk_ids[row * num_logprobs + r] = j;
        topk_logprobs[row * num_logprobs + r] = lp;
      }
    }
  }
}

// Workspace bytes of the multi-workgroup form (any span count it picks).
inline int64_t sample_ws_bytes(int64_t rows, int k) {
  const int64_t rounds = k > 1 ? k : 1;
  return rows * kMaxSpans * (4 + 16 + 8 * rounds) + 256;
}

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Launches the multi-workgroup form if the shape suits it and the workspace
// holds its partials; false: take the one-workgroup kernel (nothing launched).
template <int XDT, int VEC>
bool try_sample_multi(const void* x, int64_t rows, int64_t cols, int k, int bits, int frac, int64_t* sampled,
                      float* sampled_lp, int64_t* topk_ids, float* topk_lp, void* ws, int64_t ws_bytes,
                      hipStream_t st, int* rc) {
  const int64_t nchunks = cols / VEC;
  if (!ws || rows > kMultiMaxRows || ws_bytes < sample_ws_bytes(rows, k)) return false;
  int spans = kMaxSpans;
  while (spans > 2 && (rows * spans > 1024 || nchunks / spans < kSpanThreads)) spans /= 2;
  if (nchunks / spans < kSpanThreads) return false;  // short rows: one workgroup is enough
  const int64_t span_chunks = cdiv(nchunks, spans);
  const int rounds = k > 1 ? k : 1;
  const LseShape sh = lse_shape(cols, VEC, kSpanNreg, bits, frac);
  const int fast = bits != 64 && lse_fast_sum(bits, frac, double(cdiv(span_chunks, kSpanThreads)) * VEC);
  const float inv = pow2f(-frac);
  using XT = typename Io<XDT>::T;
  const XT* xp = static_cast<const XT*>(x);
  char* base = static_cast<char*>(ws);
  float* maxima = reinterpret_cast<float*>(base);
  char* sums = base + align_up(rows * spans * 4, 16);
  uint64_t* cand = reinterpret_cast<uint64_t*>(sums + align_up(rows * spans * 16, 16));
  const dim3 sgrid(static_cast<unsigned>(rows * spans));
  sample_span_kernel<XDT, VEC><<<sgrid, kSpanThreads, 0, st>>>(xp, cols, spans, span_chunks, rounds, maxima, cand);
#define FXPR_SAMPLE_MULTI(B, W, FAST)                                                                        \
  do {                                                                                                       \
    sample_sum_kernel<XDT, VEC, B, W><<<sgrid, kSpanThreads, 0, st>>>(xp, cols, spans, span_chunks, frac, FAST, \
                                                                      maxima, reinterpret_cast<LseSum<W>*>(sums)); \
    sample_final_kernel<XDT, W><<<dim3(static_cast<unsigned>(rows)), kFinalThreads, 0, st>>>(                  \
        xp, cols, spans, rounds, inv, maxima, reinterpret_cast<const LseSum<W>*>(sums), cand, sampled,          \
        sampled_lp, topk_ids, topk_lp, k);                                                                   \
  } while (0)
  if (bits == 16) FXPR_SAMPLE_MULTI(16, false, fast);
  else if (bits == 32) FXPR_SAMPLE_MULTI(32, false, fast);
  else if (!sh.wide) FXPR_SAMPLE_MULTI(64, false, 0);
  else FXPR_SAMPLE_MULTI(64, true, 0);
#undef FXPR_SAMPLE_MULTI
  *rc = launch_status();
  return true;
}

template <int XDT, int VEC>
int launch_sample_vec(const void* x, int64_t rows, int64_t cols, int k, int bits, int frac, int64_t* sampled,
                      float* sampled_lp, int64_t* topk_ids, float* topk_lp, void* ws, int64_t ws_bytes,
                      hipStream_t st) {
  int rc = FXPR_OK;
  if (try_sample_multi<XDT, VEC>(x, rows, cols, k, bits, frac, sampled, sampled_lp, topk_ids, topk_lp, ws, ws_bytes,
                                 st, &rc))
    return rc;
  using XT = typename Io<XDT>::T;
  constexpr int NREG = VEC == 1 ? 8 : 32;
  const LseShape sh = lse_shape(cols, VEC, NREG, bits, frac);
  const float inv = pow2f(-frac);
  const int rounds = k > 1 ? k : 1;
  dim3 grid(static_cast<unsigned>(rows));
  const XT* xp = static_cast<const XT*>(x);
  const int n = sh.threads;
#define FXPR_SAMPLE(B, W, FAST) \
  sample_greedy_kernel<XDT, VEC, NREG, B, W><<<grid, n, 0, st>>>(xp, cols, rounds, frac, inv, FAST, sampled, \
                                                                  sampled_lp, topk_ids, topk_lp, k)
  if (bits == 16) FXPR_SAMPLE(16, false, sh.fast_sum);
  else if (bits == 32) FXPR_SAMPLE(32, false, sh.fast_sum);
  else if (!sh.wide) FXPR_SAMPLE(64, false, 0);
  else FXPR_SAMPLE(64, true, 0);
#undef FXPR_SAMPLE
  return launch_status();
}

template <int XDT>
int launch_sample(const void* x, int64_t rows, int64_t cols, int k, int bits, int frac, int64_t* sampled,
                  float* sampled_lp, int64_t* topk_ids, float* topk_lp, void* ws, int64_t ws_bytes,
                  hipStream_t st) {
  constexpr int VEC = 16 / sizeof(typename Io<XDT>::T);
  if (cols % VEC == 0 && aligned(x, 16))
    return launch_sample_vec<XDT, VEC>(x, rows, cols, k, bits, frac, sampled, sampled_lp, topk_ids, topk_lp, ws,
                                       ws_bytes, st);
  return launch_sample_vec<XDT, 1>(x, rows, cols, k, bits, frac, sampled, sampled_lp, topk_ids, topk_lp, ws,
                                   ws_bytes, st);
}

}  // namespace
}  // namespace fxpr

using namespace fxpr;

extern "C" int64_t fxpr_sample_greedy_workspace_bytes(int64_t rows, int num_logprobs) {
  if (rows <= 0 || rows > kMultiMaxRows || num_logprobs < 0 || num_logprobs > kMaxLogprobs) return 0;
  return sample_ws_bytes(rows, num_logprobs);
}

extern "C" int fxpr_sample_greedy(const void* logits, int x_dtype, int64_t rows, int64_t cols,
                                  int num_logprobs, int int_bits, int frac_bits, int64_t* sampled,
                                  float* sampled_logprob, int64_t* topk_ids, float* topk_logprobs,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (rows < 0 || cols < 0 || rows > 0x7fffffff || cols > 0x7fffffff) return FXPR_E_SHAPE;
  if (num_logprobs < 0 || num_logprobs > kMaxLogprobs || num_logprobs > cols) return FXPR_E_SHAPE;
  if (rows == 0) return FXPR_OK;
  if (cols == 0) return FXPR_E_SHAPE;
  if (!logits || !sampled || !sampled_logprob) return FXPR_E_ARG;
  if (num_logprobs > 0 && (!topk_ids || !topk_logprobs)) return FXPR_E_ARG;
  hipStream_t st = as_stream(stream);
  switch (x_dtype) {
    case FXPR_DTYPE_F16:
      return launch_sample<FXPR_DTYPE_F16>(logits, rows, cols, num_logprobs, int_bits, frac_bits, sampled,
                                           sampled_logprob, topk_ids, topk_logprobs, workspace, workspace_bytes, st);
    case FXPR_DTYPE_BF16:
      return launch_sample<FXPR_DTYPE_BF16>(logits, rows, cols, num_logprobs, int_bits, frac_bits, sampled,
                                            sampled_logprob, topk_ids, topk_logprobs, workspace, workspace_bytes, st);
    case FXPR_DTYPE_F32:
      return launch_sample<FXPR_DTYPE_F32>(logits, rows, cols, num_logprobs, int_bits, frac_bits, sampled,
                                           sampled_logprob, topk_ids, topk_logprobs, workspace, workspace_bytes, st);
    default: return FXPR_E_DTYPE;
  }
}
