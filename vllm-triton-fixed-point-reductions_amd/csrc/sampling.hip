// Deterministic greedy sampling with log-probabilities.
//
// Per row of logits: the greedy token is the first element of the row's
// order (largest value first; equal values by ascending index; every NaN
// ranks above +inf; -0 equals +0); the k requested log-probabilities are
// those of the first k elements of the same order. A log-probability is
// fl32(x_j) - lse with lse from row_lse, i.e. exactly the fp32-output
// log_softmax_fxp value of that element.
//
// One workgroup per row, the row held in registers as in the log-softmax.
// Selection is by rounds: each round takes the largest 64-bit order key
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

template <int XDT, int VEC>
int launch_sample_vec(const void* x, int64_t rows, int64_t cols, int k, int bits, int frac, int64_t* sampled,
                      float* sampled_lp, int64_t* topk_ids, float* topk_lp, hipStream_t st) {
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
                  float* sampled_lp, int64_t* topk_ids, float* topk_lp, hipStream_t st) {
  constexpr int VEC = 16 / sizeof(typename Io<XDT>::T);
  if (cols % VEC == 0 && aligned(x, 16))
    return launch_sample_vec<XDT, VEC>(x, rows, cols, k, bits, frac, sampled, sampled_lp, topk_ids, topk_lp, st);
  return launch_sample_vec<XDT, 1>(x, rows, cols, k, bits, frac, sampled, sampled_lp, topk_ids, topk_lp, st);
}

}  // namespace
}  // namespace fxpr

using namespace fxpr;

extern "C" int fxpr_sample_greedy(const void* logits, int x_dtype, int64_t rows, int64_t cols,
                                  int num_logprobs, int int_bits, int frac_bits, int64_t* sampled,
                                  float* sampled_logprob, int64_t* topk_ids, float* topk_logprobs,
                                  void* stream) {
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
                                           sampled_logprob, topk_ids, topk_logprobs, st);
    case FXPR_DTYPE_BF16:
      return launch_sample<FXPR_DTYPE_BF16>(logits, rows, cols, num_logprobs, int_bits, frac_bits, sampled,
                                            sampled_logprob, topk_ids, topk_logprobs, st);
    case FXPR_DTYPE_F32:
      return launch_sample<FXPR_DTYPE_F32>(logits, rows, cols, num_logprobs, int_bits, frac_bits, sampled,
                                           sampled_logprob, topk_ids, topk_logprobs, st);
    default: return FXPR_E_DTYPE;
  }
}
