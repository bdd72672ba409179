// Fixed-point GEMM on MFMA (gfx950).
//
//   C[m, n] = IO( fl32(acc) * 2^-f (+ fl32(bias[n])) ),
//   acc     = sum over K-tiles t (wrapping b-bit) of RNE_sat_b(P_t[m, n] * 2^f),
//   P_t     = fp32 dot of A[m, tile t] and B[tile t, n] (K tail zero-padded).
//
// Replaces _gemm_kernel / _gemm_splitk_kernel (fxpr_vllm/_triton/gemm.py:
// 123-204, 209-325). The K-tile width (128 for bf16/f16, 64 for fp32) is the
// determinism unit of the reference (gemm.py:18-31) and is kept. Every output
// element's P_t is produced by the same fixed chain of MFMA instructions
// (16x16x32 bf16/f16, 16x16x4 f32) in increasing k order, whatever the tile
// configuration, M, N or split count, so results are bitwise invariant to
// all of them. Split-K writes per-split integer partials to a workspace and
// a second kernel sums them; integer addition makes the order irrelevant and
// no atomics or counters are needed (graph-capturable, nothing to re-zero).

#pragma once

#include <type_traits>

#include "fxp_device.h"
#include "fxpr_internal.h"

namespace fxpr {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves per workgroup

// Per-dtype MFMA traits: KI = k per instruction, BKQ = quantisation K-tile,
// BKS = k per LDS stage, CHUNK = elements per 16-byte vector.
template <int DT> struct Mma;
template <> struct Mma<FXPR_DTYPE_BF16> {
  using T = uint16_t;
  using Frag = uint4;
  static constexpr int KI = 32, BKQ = 128, BKS = 64, CHUNK = 8;
  static __device__ __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mma<FXPR_DTYPE_F16> {
  using T = uint16_t;
  using Frag = uint4;
  static constexpr int KI = 32, BKQ = 128, BKS = 64, CHUNK = 8;
  static __device__ __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mma<FXPR_DTYPE_F32> {
  using T = float;
  using Frag = float;
  static constexpr int KI = 4, BKQ = 64, BKS = 32, CHUNK = 4;
  static __device__ __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <int BM_, int BN_, int WM_, int WN_> struct Tile {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int WAVES_N = BN / WN;
  static constexpr int MB = WM / 16, NB = WN / 16;
  static_assert((BM / WM) * (BN / WN) == kThreads / 64, "4 waves per workgroup");
};

struct GemmArgs {
  const void* a;
  const void* b;
  const float* bias;  // fp32 copy of the bias (exact for bf16 / f16 biases) or null
  void* c;
  void* ws;          // split-K partials [splits][M][N] (int32 or int64)
  int64_t M, N, K;
  int64_t lda;       // A row stride (A is K-contiguous)
  int64_t ldb;       // B: stride between n columns (K-contiguous) or k rows (N-contiguous)
  int64_t scm, scn;  // C strides
  float scale, inv_scale;
  // A K-tile whose partials all satisfy |P| < fast_lim (0: never) quantises
  // by the rounding constant (gemm_big_kernel): scale is 2^f with f >= 0 and
  // fast_lim * scale <= 2^22 (32767 for 16-bit accumulators).
  float fast_lim;
  int ktiles, tiles_per_split, tiles_m, tiles_n;
  int c_vec;         // C rows unit-stride, 16-byte aligned (vector row stores)
  // kPartial: write the integer accumulators to ws ([M][N], the split-K
  // layout with one split) instead of C; kFinish: only the epilogue, from the
  // accumulators in ws to C
  int mode;
};

enum GemmMode { kFull = 0, kPartial = 1, kFinish = 2 };

template <int BITS> struct Acc { using T = int32_t; };
template <> struct Acc<64> { using T = int64_t; };

template <int BITS> __device__ __forceinline__ typename Acc<BITS>::T wrap_add(typename Acc<BITS>::T a, int64_t q) {
  if constexpr (BITS == 64) return static_cast<int64_t>(static_cast<uint64_t>(a) + static_cast<uint64_t>(q));
  else return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(q));
}

// fl32 of the b-bit two's-complement value held in the accumulator.
template <int BITS> __device__ __forceinline__ float acc_to_f32(typename Acc<BITS>::T v, float inv) {
  if constexpr (BITS == 16) return fixed_to_f32(static_cast<int32_t>(static_cast<int16_t>(v)), inv);
  else return fixed_to_f32(v, inv);
}

// 16 bytes of CHUNK consecutive elements at p (unit stride), the first
// `valid` of them real and the rest zero.
template <bool VEC, typename T>
__device__ __forceinline__ uint4 load_chunk(const T* p, int valid) {
  constexpr int CH = 16 / sizeof(T);
  if (VEC && valid == CH) return *reinterpret_cast<const uint4*>(p);
  union {
    uint4 v;
    T e[CH];
  } u;
  u.v = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int j = 0; j < CH; ++j)
    if (j < valid) u.e[j] = p[j];
  return u.v;
}

// Workgroup tile -> (tm, tn). Hardware hands consecutive workgroup ids to the
// 8 XCDs round-robin; remap so each XCD gets one contiguous run of logical
// tiles (L2 reuse), then group GROUP_M row tiles per column sweep.
__device__ __forceinline__ void tile_coords(int bid, int nblk, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int q = nblk >> 3, r = nblk & 7, x = bid & 7, i = bid >> 3;
  const int logical = x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
  // GROUP_M row tiles sweep the columns CB at a time; inside a full
  // GROUP_M x CB block each run of four consecutive ids is a 2 x 2 square, so
  // workgroups that start together share both their A rows and B columns
  // (FETCH_SIZE of the M = 8192 lm_head: 29 GB against 35 GB for plain
  // column runs of eight row tiles; the same time)
  constexpr int GROUP_M = 8, CB = 8, MI = 2;
  const int per_group = GROUP_M * tiles_n;
  const int g = logical / per_group;
  const int first_m = g * GROUP_M;
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int idx = logical - g * per_group;
  const int per_cb = gsize * CB;
  const int cb = idx / per_cb;
  const int cw = min(tiles_n - cb * CB, CB);
  const int j = idx - cb * per_cb;
  if (gsize == GROUP_M && cw == CB) {
    constexpr int PER_MI = MI * MI, MROWS = GROUP_M / MI;
    const int mb = j / PER_MI, mi = j % PER_MI;
    tm = first_m + (mb % MROWS) * MI + mi % MI;
    tn = cb * CB + (mb / MROWS) * MI + mi / MI;
  } else {
    tm = first_m + j % gsize;
    tn = cb * CB + j / gsize;
  }
}

template <int DT, int BITS, class TL, bool B_NCONTIG, bool VEC, bool SPLIT>
__global__ __launch_bounds__(kThreads) void gemm_fxp_kernel(GemmArgs args) {
  using M_ = Mma<DT>;
  using T = typename M_::T;
  using Frag = typename M_::Frag;
  using AccT = typename Acc<BITS>::T;
  constexpr int BM = TL::BM, BN = TL::BN, MB = TL::MB, NB = TL::NB;
  constexpr int BKS = M_::BKS, KI = M_::KI, CH = M_::CHUNK;
  constexpr int LDS_K = BKS + CH;     // row pitch in elements (+16 B pad vs bank conflicts)
  constexpr int SPT = M_::BKQ / BKS;  // LDS stages per quantisation tile
  constexpr int CPR = BKS / CH;       // 16-byte chunks per row of a stage
  constexpr int CPRN = BN / CH;       // chunks per k-row of B when N-contiguous
  constexpr int NA = (BM * CPR + kThreads - 1) / kThreads;
  constexpr int NBC = (BN * CPR + kThreads - 1) / kThreads;

  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* As = reinterpret_cast<T*>(smem_raw);  // [2][BM][LDS_K]
  T* Bs = As + 2 * BM * LDS_K;             // [2][BN][LDS_K]

  const T* A = static_cast<const T*>(args.a);
  const T* B = static_cast<const T*>(args.b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / TL::WAVES_N, wn = wave % TL::WAVES_N;
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, tm, tn);
  const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
  const int split = blockIdx.y;
  const int kt_begin = split * args.tiles_per_split;
  const int kt_end = min(args.ktiles, kt_begin + args.tiles_per_split);
  const int ntiles = max(0, kt_end - kt_begin);
  const int nstages = ntiles * SPT;
  const int64_t k_base = int64_t(kt_begin) * M_::BKQ;

  // Per-thread chunk pointers at k = k_base. Rows (columns) past M (N) are
  // clamped to the last valid one: they only feed outputs that are never
  // stored, since an MFMA output row (column) depends on its own A row (B
  // column) only.
  const T* pa[NA];
  const T* pb[NBC];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int c = min(tid + i * kThreads, BM * CPR - 1);
    const int64_t m = min<int64_t>(m0 + c / CPR, args.M - 1);
    pa[i] = A + m * args.lda + k_base + (c % CPR) * CH;
  }
#pragma unroll
  for (int i = 0; i < NBC; ++i) {
    const int c = min(tid + i * kThreads, BN * CPR - 1);
    if constexpr (!B_NCONTIG) {
      const int64_t n = min<int64_t>(n0 + c / CPR, args.N - 1);
      pb[i] = B + n * args.ldb + k_base + (c % CPR) * CH;
    } else {
      const int64_t n = min<int64_t>(n0 + (c % CPRN) * CH, args.N - CH);
      pb[i] = B + (k_base + c / CPRN) * args.ldb + (n < 0 ? 0 : n);
    }
  }

  uint4 ra[NA], rb[NBC];

  // Stage s covers k in [k_base + s*BKS, k_base + (s+1)*BKS).
  auto gload = [&](int s) {
    const int64_t k0 = k_base + int64_t(s) * BKS;
    if (VEC && k0 + BKS <= args.K) {  // full stage: plain 16-byte loads
#pragma unroll
      for (int i = 0; i < NA; ++i) ra[i] = *reinterpret_cast<const uint4*>(pa[i] + int64_t(s) * BKS);
#pragma unroll
      for (int i = 0; i < NBC; ++i) {
        const int64_t off = B_NCONTIG ? int64_t(s) * BKS * args.ldb : int64_t(s) * BKS;
        // Skinny tiles (BM <= 64) are the only M tile, so B streams from HBM
        // exactly once: non-temporal loads (lm_head M = 1: +7 %)
        if constexpr (BM <= 64)
          rb[i] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pb[i] + off)));
        else
          rb[i] = *reinterpret_cast<const uint4*>(pb[i] + off);
      }
      return;
    }
    // K tail (or unaligned operands): masked element loads, zero fill
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = tid + i * kThreads;
      const int row = c / CPR, kc = (c % CPR) * CH;
      const int64_t m = m0 + row, k = k0 + kc;
      const int valid = (c < BM * CPR && m < args.M && k < args.K) ? int(min<int64_t>(CH, args.K - k)) : 0;
      ra[i] = load_chunk<false>(A + (valid ? m * args.lda + k : 0), valid);
    }
#pragma unroll
    for (int i = 0; i < NBC; ++i) {
      const int c = tid + i * kThreads;
      if constexpr (!B_NCONTIG) {
        const int col = c / CPR, kc = (c % CPR) * CH;
        const int64_t n = n0 + col, k = k0 + kc;
        const int valid = (c < BN * CPR && n < args.N && k < args.K) ? int(min<int64_t>(CH, args.K - k)) : 0;
        rb[i] = load_chunk<false>(B + (valid ? n * args.ldb + k : 0), valid);
      } else {
        const int krow = c / CPRN, nc = (c % CPRN) * CH;
        const int64_t k = k0 + krow, n = n0 + nc;
        const int valid = (c < BN * CPR && k < args.K && n < args.N) ? int(min<int64_t>(CH, args.N - n)) : 0;
        rb[i] = load_chunk<false>(B + (valid ? k * args.ldb + n : 0), valid);
      }
    }
  };

  auto lstore = [&](int buf) {
    T* as = As + buf * BM * LDS_K;
    T* bs = Bs + buf * BN * LDS_K;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int c = tid + i * kThreads;
      if (c < BM * CPR) *reinterpret_cast<uint4*>(as + (c / CPR) * LDS_K + (c % CPR) * CH) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NBC; ++i) {
      const int c = tid + i * kThreads;
      if (c < BN * CPR) {
        if constexpr (!B_NCONTIG) {
          *reinterpret_cast<uint4*>(bs + (c / CPR) * LDS_K + (c % CPR) * CH) = rb[i];
        } else {
          const int krow = c / CPRN, nc = (c % CPRN) * CH;
          union {
            uint4 v;
            T e[CH];
          } u;
          u.v = rb[i];
#pragma unroll
          for (int j = 0; j < CH; ++j) bs[(nc + j) * LDS_K + krow] = u.e[j];
        }
      }
    }
  };

  f32x4 P[MB][NB];
  AccT I[MB][NB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) I[i][j][r] = 0;

  const int frag_row = lane & 15, frag_k = (lane >> 4) * (KI / 4);
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  if (nstages > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
#pragma unroll
    for (int st = 0; st < SPT; ++st) {
      const int s = t * SPT + st;
      const int buf = s & 1;
      if (s + 1 < nstages) gload(s + 1);
      const T* as = As + buf * BM * LDS_K + (wm * TL::WM + frag_row) * LDS_K + frag_k;
      const T* bs = Bs + buf * BN * LDS_K + (wn * TL::WN + frag_row) * LDS_K + frag_k;
#pragma unroll
      for (int kk = 0; kk < BKS; kk += KI) {
        Frag fa[MB], fb[NB];
#pragma unroll
        for (int i = 0; i < MB; ++i) fa[i] = *reinterpret_cast<const Frag*>(as + i * 16 * LDS_K + kk);
#pragma unroll
        for (int j = 0; j < NB; ++j) fb[j] = *reinterpret_cast<const Frag*>(bs + j * 16 * LDS_K + kk);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)  // each tile's chain starts from an all-zero C
            P[i][j] = M_::mma(fa[i], fb[j], (st == 0 && kk == 0) ? zero4 : P[i][j]);
      }
      if (st == SPT - 1) {  // quantisation tile complete
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              I[i][j][r] = wrap_add<BITS>(I[i][j][r], quant<BITS>(__fmul_rn(P[i][j][r], args.scale)));
      }
      if (s + 1 < nstages) lstore(buf ^ 1);
      __syncthreads();
    }
  }

  // Epilogue. Lane holds rows 4*(lane/16)+r of each 16x16 block, column lane%16.
  const int64_t row_base = m0 + wm * TL::WM + (lane >> 4) * 4;
  const int64_t col_base = n0 + wn * TL::WN + (lane & 15);
  if constexpr (SPLIT) {
    AccT* ws = static_cast<AccT*>(args.ws) + int64_t(split) * args.M * args.N;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t n = col_base + j * 16;
        if (n >= args.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = row_base + i * 16 + r;
          if (m < args.M) ws[m * args.N + n] = I[i][j][r];
        }
      }
  } else {
    T* C = static_cast<T*>(args.c);
    const float* bias = args.bias;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int64_t n = col_base + j * 16;
      if (n >= args.N) continue;
      const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = row_base + i * 16 + r;
          if (m >= args.M) continue;
          float v = acc_to_f32<BITS>(I[i][j][r], args.inv_scale);
          if (bias) v = __fadd_rn(v, bv);
          C[m * args.scm + n * args.scn] = Io<DT>::store(v);
        }
    }
  }
}

// Sum the per-split integer partials (wrapping b-bit) and apply the epilogue.
// A thread takes kReduceVec consecutive elements of [M][N]: with vec (M * N
// a multiple of kReduceVec and a 16-byte aligned workspace) as 16-byte
// non-temporal loads (two for 64-bit sums), the loads of eight splits in
// flight together; otherwise element by element.
constexpr int kReduceVec = 4;
template <int DT, int BITS>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmArgs args, int splits, int vec) {
  using T = typename Io<DT>::T;
  using AccT = typename Acc<BITS>::T;
  constexpr int V = kReduceVec;
  const int64_t MN = args.M * args.N;
  const int64_t e0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;
  if (e0 >= MN) return;
  const AccT* ws = static_cast<const AccT*>(args.ws);
  AccT acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0;
  if (vec) {
    constexpr int NL = V * int(sizeof(AccT)) / 16;  // 16-byte loads per split
    constexpr int G = 8;                            // splits per batch of loads
    auto add = [&](const u32x4 (&w)[NL]) {
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        if constexpr (BITS == 64) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            acc[2 * l + h] =
                wrap_add<BITS>(acc[2 * l + h], int64_t(uint64_t(w[l][2 * h]) | (uint64_t(w[l][2 * h + 1]) << 32)));
        } else {
#pragma unroll
          for (int h = 0; h < 4; ++h) acc[h] = wrap_add<BITS>(acc[h], int32_t(w[l][h]));
        }
      }
    };
    auto load = [&](int s, u32x4 (&w)[NL]) {
      const u32x4* p = reinterpret_cast<const u32x4*>(ws + int64_t(s) * MN + e0);
#pragma unroll
      for (int l = 0; l < NL; ++l) w[l] = __builtin_nontemporal_load(p + l);
    };
    auto batch = [&](int s, auto n_tag) {
      constexpr int n = decltype(n_tag)::value;
      u32x4 w[n][NL];
#pragma unroll
      for (int g = 0; g < n; ++g) load(s + g, w[g]);
#pragma unroll
      for (int g = 0; g < n; ++g) add(w[g]);
    };
    int s = 0;
    for (; s + G <= splits; s += G) batch(s, std::integral_constant<int, G>{});
    if (s + G / 2 <= splits) {
      batch(s, std::integral_constant<int, G / 2>{});
      s += G / 2;
    }
    for (; s < splits; ++s) {
      u32x4 w[NL];
      load(s, w);
      add(w);
    }
  } else {
    for (int s = 0; s < splits; ++s)
#pragma unroll
      for (int e = 0; e < V; ++e)
        if (e0 + e < MN) acc[e] = wrap_add<BITS>(acc[e], ws[int64_t(s) * MN + e0 + e]);
  }
  int64_t m = e0 / args.N, n = e0 % args.N;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    if (e0 + e >= MN) break;
    float v = acc_to_f32<BITS>(acc[e], args.inv_scale);
    if (args.bias) v = __fadd_rn(v, args.bias[n]);
    static_cast<T*>(args.c)[m * args.scm + n * args.scn] = Io<DT>::store(v);
    if (++n == args.N) {
      n = 0;
      ++m;
    }
  }
}

// ---------------------------------------------------------------------------
// Large-M kernel for 16-bit inputs with K-contiguous A and B (the lm_head /
// linear layout). Same per-output MFMA chain as gemm_fxp_kernel (16x16x32,
// increasing k, zero C at each 128-wide K-tile), so results are bitwise
// identical to every other configuration; only the schedule differs.
//
// Waves of 64 x 64 outputs, two per SIMD: two 4-wave workgroups per CU over
// 128 x 128 tiles, or 64 x 256 ones at M <= 64 (the two waves of a SIMD
// belong to different workgroups and never wait on the same barrier); with
// 64-bit sums one wave per SIMD.
// A and B stages (64 k) go straight from global memory into LDS with
// global_load_lds_dwordx4 (no staging registers).
// Rows are 128 B with the 16-byte chunk c of row r stored at slot
// c ^ ((r >> 1) & 7): each DMA instruction fills 1 KB of LDS contiguously,
// and the 16-row fragment reads hit 16 distinct 16-byte bank groups.
// The compiler would wait for every outstanding DMA before any LDS read it
// can see, so fragment reads are inline asm and the waits are explicit: the
// DMAs of stage s are complete once only the next stage's are outstanding
// (vector memory operations complete in issue order), and a barrier makes
// every wave's part visible. A partial last K-tile is peeled off and done
// first (integer sums do not depend on the order of tiles). The epilogue
// stages each wave's C tile through LDS to write whole 16-byte row pieces.

template <int BM_, int BN_, int WGM_, int WGN_, int NSA_, int NSB_, int WPE_ = 2> struct BigTile {
  static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
  // LDS stages of A and of B: each matrix's DMAs run its ring depth - 1
  // stages ahead (B, the weights streamed from HBM, may get the deeper one)
  static constexpr int NSA = NSA_, NSB = NSB_;
  static constexpr int WPE = WPE_;  // waves per SIMD the register budget is sized for
  static constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int MB = WM / 16, NB = WN / 16;
};
// two 4-wave workgroups per CU (80 KB of LDS each), every M > 16: one 8-wave
// 256 x 128 workgroup per CU measured the same at M = 256 .. 1024 and 1.6-1.8x
// slower at M = 65 .. 128 (half its rows past M)
#ifndef FXPR_TB2_NSB
#define FXPR_TB2_NSB 3
#endif
using TB2 = BigTile<128, 128, 2, 2, 2, FXPR_TB2_NSB>;
// int64 accumulators double the integer state (64 x 64 outputs need 128
// registers of it): one wave per SIMD, one 4-wave workgroup per CU; A two
// stages deep, B three (2 % over three of each)
using TB64 = BigTile<128, 128, 2, 2, 2, 3, 1>;
// M = 17 .. 64 with 16- / 32-bit sums: one row of four 64 x 64 waves over 256
// columns, A and B two stages deep (80 KB: two workgroups per CU). A 128-row
// tile computes 2-4x the MFMAs those rows need and moves 2-4x their A:
// graph-timed at M = 32, K = 4096, N = 28672 / 4096 / 6144 and the lm_head:
// 65.1 / 18.5 / 23.2 / 226.7 -> 53.3 / 17.2 / 21.9 / 181.5 us.
using TS64 = BigTile<64, 256, 1, 4, 2, 2>;
inline bool ts64_rows(int64_t M, int bits) { return M > 16 && M <= 64 && bits != 64; }

template <class BT> constexpr size_t big_lds_bytes() {
  constexpr size_t stages = (size_t(BT::NSA) * BT::BM + size_t(BT::NSB) * BT::BN) * 128;
  constexpr size_t epi = size_t(BT::WAVES) * BT::WM * (BT::WN + 8) * 2;
  return stages > epi ? stages : epi;
}

typedef __attribute__((address_space(3))) void* LdsPtr;
// 16 bytes per lane from a raw buffer into LDS at dst + 16 * lane. (A helper:
// called directly in a kernel template, the builtin makes the host pass drop
// the kernel's launch stub.)
__device__ __forceinline__ void buffer_to_lds(__amdgpu_buffer_rsrc_t r, unsigned dst, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)(uintptr_t)dst, 16, voff, soff, 0, 0);
}
// Wait until at most N LDS operations are outstanding, tied to the registers
// the older reads fill (their uses cannot move above it).
template <int N> __device__ __forceinline__ void lgkm_wait_for(u32x4& a) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "n"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void lgkm_wait_for(u32x4& a, u32x4& b, u32x4& c, u32x4& d, u32x4& e) {
  asm volatile("s_waitcnt lgkmcnt(%5)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e) : "n"(N) : "memory");
}

// WIDEN (BITS = 32, unsplit): the 64-bit accumulator semantics on 32-bit
// sums. When every K-tile of an output tile quantises by the rounding
// constant (|P * 2^f| < 2^22, so |q| < 2^22) and there are fewer than 512
// K-tiles, the 32-bit sum cannot wrap and equals the 64-bit one; the epilogue
// converts it as a 64-bit value. A tile with any K-tile outside that range
// stores nothing but a NaN at C[m0][n0] for the 64-bit kernel's REDO pass,
// which computes exactly those tiles (a NaN there from a NaN bias costs a
// redundant, bit-identical recompute).
template <int DT, int BITS, class BT, bool SPLIT, bool WIDEN = false, bool REDO = false>
__global__ __launch_bounds__(BT::THREADS, BT::WPE) void gemm_big_kernel(GemmArgs args) {
  using M_ = Mma<DT>;
  using T = typename M_::T;
  using AccT = typename Acc<BITS>::T;
  static_assert(DT != FXPR_DTYPE_F32, "16-bit inputs only");
  static_assert(BT::MB == 4 && BT::NB == 4, "fragment asm assumes 64 x 64 wave tiles");
  static_assert(!WIDEN || (BITS == 32 && !SPLIT), "WIDEN: unsplit 32-bit sums");
  constexpr int BM = BT::BM, BN = BT::BN, MB = BT::MB, NB = BT::NB, NW = BT::WAVES;
  constexpr int BKS = 64, CH = 8;
  constexpr int NSA = BT::NSA, NSB = BT::NSB;
  constexpr int A_SLOT = BM * 128, B_SLOT = BN * 128;  // bytes per stage of A, of B
  constexpr int B_RING = NSA * A_SLOT;                 // the B ring follows the A ring
  constexpr int NIA = BM / 8 / NW;        // A DMA instructions per wave per stage (8 rows each)
  constexpr int NIB = BN / 8 / NW;        // B DMA instructions per wave per stage
  constexpr int NDMA = NIA + NIB;         // vector memory instructions per wave per stage
  static_assert(NIA * 8 * NW == BM && NIB * 8 * NW == BN, "tile / wave mismatch");

  extern __shared__ __align__(16) unsigned char smem_raw[];
  const unsigned lds0 = static_cast<unsigned>(reinterpret_cast<uintptr_t>(smem_raw));

  const T* A = static_cast<const T*>(args.a);
  const T* B = static_cast<const T*>(args.b);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS targets in SGPRs
  const int wm = wave / BT::WGN, wn = wave % BT::WGN;
  int tm, tn;
  [[maybe_unused]] uint64_t redo_mask = 0;
  [[maybe_unused]] const int redo_tiles = args.tiles_m * args.tiles_n;
  [[maybe_unused]] const int redo_base = int(blockIdx.x) * 64;
  if constexpr (REDO) {
    // The 64-bit pass over the tiles a WIDEN launch marked (a NaN at the
    // tile's first element): workgroup w checks the marking launch's
    // workgroups 64 w .. 64 w + 63 with one load per lane and runs the tile
    // body for each marked one, in order (the body's end jumps back here).
    // No marks (the common case): 1002 workgroups of one round of loads at
    // M = 8192 instead of 64128 workgroups that each load their mark and exit
    // (0.2 ms).
    bool marked = false;
    if (redo_base + lane < redo_tiles) {
      tile_coords(redo_base + lane, redo_tiles, args.tiles_m, args.tiles_n, tm, tn);
      const float c0 =
          Io<DT>::load(static_cast<const T*>(args.c)[int64_t(tm) * BM * args.scm + int64_t(tn) * BN * args.scn]);
      marked = c0 != c0;
    }
    // every wave loads the same marks: the mask is uniform over the workgroup
    redo_mask = __builtin_amdgcn_ballot_w64(marked);
    if (!redo_mask) return;
  } else {
    tile_coords(blockIdx.x, gridDim.x, args.tiles_m, args.tiles_n, tm, tn);
  }
redo_next:
  if constexpr (REDO) {
    tile_coords(redo_base + __builtin_ctzll(redo_mask), redo_tiles, args.tiles_m, args.tiles_n, tm, tn);
    redo_mask &= redo_mask - 1;
  }
  const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;
  const int split = blockIdx.y;
  const int kt_begin = split * args.tiles_per_split;
  const int kt_end = min(args.ktiles, kt_begin + args.tiles_per_split);
  const bool has_tail = kt_end > kt_begin && int64_t(kt_end) * 128 > args.K;
  const int nfull = max(0, kt_end - kt_begin - (has_tail ? 1 : 0));
  const int64_t kb0 = int64_t(kt_begin) * 128;

  // DMA sources. Instruction q of this wave covers rows 8 i .. 8 i + 7 of
  // the A (B) stage, i = wave + NW q; lane l brings row 8 i + l / 8, chunk
  // (l % 8) ^ ((row >> 1) & 7). Rows past M / N are clamped: they feed only
  // outputs that are never stored. Buffer loads: a resource per matrix based
  // at the tile's first row and k = kb0, a fixed 32-bit lane offset (the host
  // keeps BM * ld * 2 bytes below 2^31; no range limit) and the stage offset in
  // a scalar.
  const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(A + m0 * args.lda + kb0), short(0), -1, kBufferDword3);
  const __amdgpu_buffer_rsrc_t brsrc = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(B + n0 * args.ldb + kb0), short(0), -1, kBufferDword3);
  uint32_t voff[NDMA];
#pragma unroll
  for (int q = 0; q < NDMA; ++q) {
    const bool isa = q < NIA;
    const int i = wave + NW * (isa ? q : q - NIA);
    const int r = 8 * i + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int64_t row = isa ? min<int64_t>(m0 + r, args.M - 1) - m0 : min<int64_t>(n0 + r, args.N - 1) - n0;
    voff[q] = uint32_t((row * (isa ? args.lda : args.ldb) + c * CH) * int64_t(sizeof(T)));
  }
  // stage s (64 k from kb0) of A (isb false) or B into ring slot q % depth
  auto dma = [&](bool isb, int s, int q) {
    const int soff = s * (BKS * int(sizeof(T)));
    const unsigned slot = isb ? B_RING + (q % NSB) * B_SLOT : (q % NSA) * A_SLOT;
#pragma unroll
    for (int q = isb ? NIA : 0; q < (isb ? NDMA : NIA); ++q) {
      const int i = wave + NW * (isb ? q - NIA : q);
      buffer_to_lds(isb ? brsrc : arsrc, lds0 + slot + i * 1024, voff[q], soff);
    }
  };

  f32x4 P[MB][NB];
  AccT I[MB][NB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) I[i][j][r] = 0;
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  // Fragment reads: lane (row lane % 16 of each 16-row block, k slot kg)
  // reads chunk c = 4 h + kg of its row; the row's swizzle (row >> 1) & 7
  // depends on lane % 16 only (blocks start at multiples of 16). Fragment
  // f < 4 is A block f, f >= 4 is B block f - 4 (16 rows = 2048 B apart).
  const int kg = lane >> 4, sw = (lane & 15) >> 1;
  const unsigned arow = (wm * BT::WM + (lane & 15)) * 128;
  const unsigned brow = (wn * BT::WN + (lane & 15)) * 128;
  // fragment address in stage s (ring slot s % NSA of A, s % NSB of B)
  auto frag_addr = [&](int s, int h, bool isb) -> unsigned {
    const unsigned slot = isb ? B_RING + (s % NSB) * B_SLOT : (s % NSA) * A_SLOT;
    return lds0 + slot + ((((h << 2) + kg) ^ sw) << 4) + (isb ? brow : arow);
  };
  auto read_frag = [&](unsigned addr, u32x4& x, auto off_tag) {
    constexpr int OFF = decltype(off_tag)::value;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(x) : "v"(addr), "n"(OFF) : "memory");
  };
  // Issue order A0, B0..B3, A1..A3: the stage loop starts on block row 0 as
  // soon as the first five have landed.
  auto read_frags = [&](int st, int h, u32x4 (&fa)[MB], u32x4 (&fb)[NB]) {
    const unsigned aa = frag_addr(st, h, false), bb = frag_addr(st, h, true);
    read_frag(aa, fa[0], std::integral_constant<int, 0>{});
    read_frag(bb, fb[0], std::integral_constant<int, 0>{});
    read_frag(bb, fb[1], std::integral_constant<int, 2048>{});
    read_frag(bb, fb[2], std::integral_constant<int, 4096>{});
    read_frag(bb, fb[3], std::integral_constant<int, 6144>{});
    read_frag(aa, fa[1], std::integral_constant<int, 2048>{});
    read_frag(aa, fa[2], std::integral_constant<int, 4096>{});
    read_frag(aa, fa[3], std::integral_constant<int, 6144>{});
  };
  auto lds_wait = [&](u32x4 (&fa)[MB], u32x4 (&fb)[NB]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]), "+v"(fb[2]),
                   "+v"(fb[3])
                 :
                 : "memory");
  };
  auto mma = [&](int i, int j, const u32x4& a, const u32x4& b, bool zero_c) {
    P[i][j] = M_::mma(__builtin_bit_cast(uint4, a), __builtin_bit_cast(uint4, b), zero_c ? zero4 : P[i][j]);
  };
  auto quantize_block = [&](int i, int j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (BITS == 64) {
        I[i][j][r] = wrap_add<BITS>(I[i][j][r], quant<BITS>(__fmul_rn(P[i][j][r], args.scale)));
      } else {
        // the accumulator updated in place, as in quantize_block_fast: the
        // two paths then meet without register copies
        const int32_t q = static_cast<int32_t>(quant<BITS>(__fmul_rn(P[i][j][r], args.scale)));
        asm("v_add_u32 %0, %0, %1" : "+v"(I[i][j][r]) : "v"(q));
      }
    }
  };
  // Rounding-constant quantisation, for a K-tile whose partials all satisfy
  // |P| < fast_lim (so |P * 2^f| < 2^22, exact): fl32(x + 1.5 * 2^23) is
  // RNE(x) + 1.5 * 2^23 (the sum lies in [2^23, 2^24), where the spacing is
  // 1, and the constant is even, so a tie goes to the same even integer), and
  // its bit pattern minus the constant's is RNE(x). No saturation can occur
  // (and for 64-bit sums RNE(x) fits 32 bits, sign-extended into the add).
  // Same bits as quantize_block; two instructions per element instead of four
  // (64-bit: five instead of about eight).
  // (The accumulator update is written as an instruction: from C the
  // compiler splits the add off into extra moves and adds.)
  const float magic = 12582912.0f;  // 1.5 * 2^23, bit pattern 0x4B400000
  const uint32_t neg_magic_bits = 0xB4C00000u;  // -0x4B400000 mod 2^32
  auto quantize_block_fast = [&](int i, int j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float y = __builtin_fmaf(P[i][j][r], args.scale, magic);
      if constexpr (BITS == 64) {
        // the 32-bit RNE(x), sign-extended into the 64-bit sum
        const int32_t q = static_cast<int32_t>(__float_as_uint(y) + neg_magic_bits);
        I[i][j][r] = wrap_add<BITS>(I[i][j][r], q);
      } else {
        asm("v_add3_u32 %0, %0, %1, %2" : "+v"(I[i][j][r]) : "v"(y), "v"(neg_magic_bits));
      }
    }
  };
  // The running maximum of |P| over every K-tile quantised by the rounding
  // constant (NaN-propagating): a K-tile is not checked before its
  // quantisation (that would wait for all of the wave's MFMA chains at every
  // K-tile); a tile whose maximum ends at or above fast_lim is recomputed
  // exactly after the loop (or, for WIDEN, marked for the 64-bit kernel).
  float rmax[4] = {0.f, 0.f, 0.f, 0.f};
  auto track_row = [&](int i) {
#pragma unroll
    for (int j = 0; j < NB; j += 2)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        asm("v_maximum3_f32 %0, |%1|, |%2|, %3" : "=v"(rmax[r]) : "v"(P[i][j][r]), "v"(P[i][j + 1][r]), "v"(rmax[r]));
  };
  auto rmax_fast = [&]() -> bool {
    float mm;
    asm("v_maximum3_f32 %0, %1, %2, %3" : "=v"(mm) : "v"(rmax[0]), "v"(rmax[1]), "v"(rmax[2]));
    asm("v_maximum3_f32 %0, %1, %2, %2" : "=v"(mm) : "v"(mm), "v"(rmax[3]));
    return mm < args.fast_lim;
  };
  auto quantize = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) quantize_block(i, j);
  };
  // Plain (unpipelined) stage, used for the peeled tail tile.
  auto compute = [&](int st, bool first) {
    u32x4 fa[MB], fb[NB];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      read_frags(st, h, fa, fb);
      lds_wait(fa, fb);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) mma(i, j, fa[i], fb[j], first && h == 0);
    }
  };

  // P holds the fp32 partial of the K-tile in progress; it is quantised into
  // I when the next K-tile starts (block by block, in the shadow of the new
  // chain's MFMAs) and once more after the last one. Starting from zero,
  // the first such quantisation adds nothing.
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) P[i][j] = zero4;

  // K-tile kt into ring slots 0 and 1 of A and B by masked register loads
  // (zero past K), in the swizzled layout, and its partials into P: the
  // peeled tail tile, and the exact recomputation.
  auto stage_tile = [&](int kt) {
    const int64_t kt0 = int64_t(kt) * 128;
    for (int e = tid; e < 2 * (BM + BN) * 8; e += BT::THREADS) {
      const int st = e / ((BM + BN) * 8), rem = e % ((BM + BN) * 8);
      const int r = rem / 8, c = rem % 8;
      const int64_t k = kt0 + st * BKS + c * CH;
      const bool isa = r < BM;
      const int64_t row = isa ? m0 + r : n0 + (r - BM);
      const bool ok = isa ? row < args.M : row < args.N;
      const int valid = (ok && k < args.K) ? int(min<int64_t>(CH, args.K - k)) : 0;
      const T* base = isa ? A + (valid ? row * args.lda + k : 0) : B + (valid ? row * args.ldb + k : 0);
      const uint4 v = load_chunk<false>(base, valid);
      const int rr = isa ? r : r - BM;
      *reinterpret_cast<uint4*>(smem_raw + (isa ? st * A_SLOT : B_RING + st * B_SLOT) + rr * 128 +
                                ((c ^ ((rr >> 1) & 7)) << 4)) = v;
    }
    __syncthreads();
    compute(0, true);
    compute(1, false);
    __syncthreads();
  };
  // Partial last K-tile first.
  if (has_tail) stage_tile(kt_end - 1);

  // Pipelined full K-tiles: stage s = 64 k of A in its ring slot s % NSA,
  // of B in s % NSB; each matrix's DMAs run its depth - 1 stages ahead.
  // Stages past the end re-load the last one into the free slot (never
  // read), so every iteration issues the same DMAs and the wait count stays
  // exact. Per stage: issue the DMAs (the shallower ring's first); the h = 0
  // MFMAs (with the previous K-tile's quantisation interleaved at a K-tile
  // start, and the h = 1 fragment reads issued between them); the h = 1
  // MFMAs; wait for the next stage's DMAs and barrier; issue the next
  // stage's h = 0 fragment reads, which complete while the MFMAs drain.
  const int nst = 2 * nfull;
  if (nst > 0) {
    u32x4 fa0[MB], fb0[NB], fa1[MB], fb1[NB];
    constexpr bool B_DEEP = NSB > NSA;
    constexpr int NSS = B_DEEP ? NSA : NSB, NSD = B_DEEP ? NSB : NSA;  // shallow, deep depth
    constexpr int NID = B_DEEP ? NIB : NIA;                             // deep ring's DMAs per stage
    // DMAs issued after the later of stage s + 1's: the deep ring's of the
    // same group (if deeper) and NSS - 2 whole groups
    constexpr int WAITN = NSS == NSD ? NDMA * (NSS - 2) : NID + NDMA * (NSS - 2);
    // the DMA group of stage j: shallow stage j + NSS - 1, then deep j + NSD - 1
    // (A counts as the shallow ring when the depths are equal)
    auto dma_group = [&](int j) {
      if (j + NSS - 1 >= 0) dma(/*isb=*/!B_DEEP && NSB < NSA, min(j + NSS - 1, nst - 1), j + NSS - 1);
      if (j + NSD - 1 >= 0) dma(/*isb=*/B_DEEP || NSB == NSA, min(j + NSD - 1, nst - 1), j + NSD - 1);
    };
#pragma unroll
    for (int j = 1 - NSD; j < 0; ++j) dma_group(j);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
    __builtin_amdgcn_s_barrier();
    read_frags(0, 0, fa0, fb0);
    // Landed before the loop: the compiler may move the loop's fragment
    // registers into place here, and an inline-asm read's output looks ready
    // to it at issue.
    lds_wait(fa0, fb0);
    // tile_start: quantise the previous K-tile's partials block by block by
    // the rounding constant, tracking their range (a tile with any K-tile out
    // of range is recomputed after the loop).
    auto stage = [&](int s, auto tile_start_tag) {
      constexpr bool tile_start = decltype(tile_start_tag)::value;
      dma_group(s);
      const unsigned aa1 = frag_addr(s, 1, false), bb1 = frag_addr(s, 1, true);
      __builtin_amdgcn_sched_barrier(0);
      // Block row i: its quantisation (at a K-tile start; registers only, so
      // it runs while the row's fragments land), a wait for them (LDS
      // operations complete in issue order: A(i+1..3) and the h = 1 reads
      // issued so far, two per row, may still be in flight), its MFMAs with
      // the h = 1 reads in between.
      auto row_prologue = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if constexpr (tile_start) {
          track_row(i);
#pragma unroll
          for (int j = 0; j < NB; ++j) quantize_block_fast(i, j);
        }
        if constexpr (BITS == 64) {
          // int64 accumulators spill into AGPRs: the compiler may copy a
          // fragment register it takes for ready, so all of them are bound
          // to one full wait before their first use
          if constexpr (i == 0) lds_wait(fa0, fb0);
        } else if constexpr (i == 0) {
          lgkm_wait_for<3>(fa0[0], fb0[0], fb0[1], fb0[2], fb0[3]);
        } else {
          lgkm_wait_for<3 + i>(fa0[i]);
        }
      };
      // compile-time block index: every read and wait at a fixed place (a
      // runtime switch would put the reads on branches, where the compiler
      // may copy registers whose loads are still in flight)
      static_for<MB * NB>([&](auto bc) {
        constexpr int b = decltype(bc)::value, i = b / NB, j = b % NB;
        if constexpr (j == 0) row_prologue(std::integral_constant<int, i>{});
        mma(i, j, fa0[i], fb0[j], tile_start);
        if constexpr (b % 2 == 0) {
          constexpr int f = b / 2;  // h = 1 fragment f: A 0..3, then B 0..3
          if constexpr (f < MB)
            read_frag(aa1, fa1[f], std::integral_constant<int, 2048 * f>{});
          else
            read_frag(bb1, fb1[f - MB], std::integral_constant<int, 2048 * (f - MB)>{});
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      lds_wait(fa1, fb1);
      // With two 4-wave workgroups per CU, two waves share each SIMD: the
      // one in this MFMA burst takes issue priority, so the other's VALU and
      // LDS instructions go in the gaps between its MFMAs rather than ahead
      // of them (1-4 % at M = 8192).
      if constexpr (NW == 4 && BT::WPE == 2) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) mma(i, j, fa1[i], fb1[j], false);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NW == 4 && BT::WPE == 2) __builtin_amdgcn_s_setprio(0);
      // Own DMAs of stage s + 1 landed (only later stages' may be in
      // flight); the barrier covers everyone's, and everyone's reads of stage
      // s are done (its slots are refilled from the next stage on). A plain
      // s_barrier: __syncthreads() would also fence, i.e. wait for every DMA.
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAITN) : "memory");
      __builtin_amdgcn_s_barrier();
      read_frags(s + 1, 0, fa0, fb0);
    };
    for (int s = 0; s < nst; s += 2) {
      stage(s, std::true_type{});
      stage(s + 1, std::false_type{});
    }
    lds_wait(fa0, fb0);                               // trailing reads (unused)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing DMAs into unused buffers
  }
  if constexpr (WIDEN) {
    // the last K-tile (quantised exactly below) must fit 32-bit sums too
#pragma unroll
    for (int i = 0; i < MB; ++i) track_row(i);
  }
  // a K-tile of the wave outside the rounding-constant range (or NaN / inf)
  const bool out_of_range = __builtin_amdgcn_ballot_w64(!rmax_fast()) != 0;
  quantize();
  __syncthreads();  // LDS is reused by the flags and the epilogue
  {
    // the workgroup's OR of the waves' range flags through the last words of
    // the dynamic LDS (past the epilogue's area; __syncthreads_or would add
    // static LDS, and 80 KB + a few bytes no longer fits two workgroups per
    // CU)
    // (past the recomputation's two stages where they fit there; otherwise
    // right past the epilogue's area: the recomputation starts only after a
    // barrier that follows every wave's read of the flags)
    constexpr size_t EPI = size_t(NW) * BT::WM * (BT::WN + 8) * sizeof(T);
    constexpr size_t LAST = big_lds_bytes<BT>() - 4 * NW;
    constexpr size_t FLAGS = LAST >= size_t(B_RING) + 2 * B_SLOT ? LAST : (EPI + 15) / 16 * 16;
    static_assert(FLAGS >= EPI && FLAGS + 4 * NW <= big_lds_bytes<BT>(), "flags past the epilogue's LDS");
    int* flags = reinterpret_cast<int*>(smem_raw + FLAGS);
    if (lane == 0) flags[wave] = out_of_range ? 1 : 0;
    __syncthreads();
    int any = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) any |= flags[w];
    if (any) {  // rare
      if constexpr (WIDEN) {
        // 64-bit sums needed: the tile stores only its mark
        if (tid == 0) static_cast<T*>(args.c)[m0 * args.scm + n0 * args.scn] = Io<DT>::store(__builtin_nanf(""));
        return;
      } else {
        // recompute the tile's sums exactly, K-tile by K-tile
        __syncthreads();  // every wave has read the flags
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) I[i][j][r] = 0;
        for (int kt = kt_begin; kt < kt_end; ++kt) {
          stage_tile(kt);
          quantize();
        }
      }
    }
  }

  // Epilogue. Lane holds rows 4*(lane/16)+r of each 16x16 block, column lane%16.
  const int64_t row_base = m0 + wm * BT::WM + kg * 4;
  const int64_t col_base = n0 + wn * BT::WN + (lane & 15);
  if constexpr (SPLIT) {
    AccT* ws = static_cast<AccT*>(args.ws) + int64_t(split) * args.M * args.N;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t n = col_base + j * 16;
        if (n >= args.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = row_base + i * 16 + r;
          if (m < args.M) ws[m * args.N + n] = I[i][j][r];
        }
      }
  } else {
    T* C = static_cast<T*>(args.c);
    const float* bias = args.bias;
    float bv[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int64_t n = col_base + j * 16;
      bv[j] = (bias && n < args.N) ? bias[n] : 0.0f;
    }
    auto value = [&](int i, int j, int r) {
      float v = WIDEN ? acc_to_f32<64>(static_cast<int64_t>(I[i][j][r]), args.inv_scale)
                      : acc_to_f32<BITS>(I[i][j][r], args.inv_scale);
      if (bias) v = __fadd_rn(v, bv[j]);
      return Io<DT>::store(v);
    };
    if (args.c_vec) {
      // wave tile -> LDS (wave-private [WM][WN + 8]) -> 16-byte row stores
      constexpr int EP = BT::WN + 8;
      T* ep = reinterpret_cast<T*>(smem_raw) + wave * BT::WM * EP;
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) ep[(i * 16 + kg * 4 + r) * EP + j * 16 + (lane & 15)] = value(i, j, r);
      __builtin_amdgcn_wave_barrier();
      constexpr int CPR = BT::WN / CH;  // 16-byte chunks per row
#pragma unroll
      for (int it = 0; it < BT::WM * CPR / 64; ++it) {
        const int c = it * 64 + lane;
        const int row = c / CPR, col = (c % CPR) * CH;
        const int64_t m = m0 + wm * BT::WM + row, n = n0 + wn * BT::WN + col;
        const u32x4 v = *reinterpret_cast<const u32x4*>(ep + row * EP + col);
        if (m < args.M) {
          if (n + CH <= args.N) {
            // C is written once: non-temporal (0-3 %, most at M = 256)
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(C + m * args.scm + n));
          } else {
            const T* e = reinterpret_cast<const T*>(&v);
            for (int q = 0; q < CH; ++q)
              if (n + q < args.N) C[m * args.scm + n + q] = e[q];
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int64_t n = col_base + j * 16;
        if (n >= args.N) continue;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t m = row_base + i * 16 + r;
            if (m < args.M) C[m * args.scm + n * args.scn] = value(i, j, r);
          }
      }
    }
  }
  if constexpr (REDO) {
    if (redo_mask) {
      __syncthreads();  // the epilogue's LDS before the next tile's DMAs
      goto redo_next;
    }
  }
}

// ---------------------------------------------------------------------------
// Decode-shape kernel: few rows (MB 16-row fragments), 16-bit inputs,
// K-contiguous A and B with 16-byte aligned rows and K a multiple of the
// 128-wide K-tile (the linear layout at decode batch sizes). B streams from
// HBM once and no split-K partials exist. A workgroup owns 16 columns of C
// for every row and all of K; its NW waves split the K-tiles into NW
// contiguous runs of nt = ceil(K-tiles / NW) (the last runs may hold fewer
// real tiles). A wave loads its fragments straight from global memory into
// registers in the MFMA operand layout (lane (r, g) of a 16-row x 32-k
// fragment holds row r, k = 8 g .. 8 g + 7: one 16-byte load; B
// non-temporal, A re-read through L2), DEPTH K-tiles ahead, and runs the
// same per-K-tile MFMA chains as every other kernel (16x16x32 in increasing
// k from a zero accumulator): the bits are theirs. The waves then hand their
// integer sums to wave 0 through LDS (integers: any order), which adds them
// and writes C. Every step issues the same loads (a step past the wave's run
// reads the first 16 bytes of A, never used), so the compiler counts the
// loads in flight exactly.
template <int MB_, int NW_, int DEPTH_> struct StreamTile {
  static constexpr int MB = MB_, NW = NW_, DEPTH = DEPTH_, THREADS = 64 * NW_;
};

template <int DT, int BITS, class ST>
__global__ __launch_bounds__(ST::THREADS) void gemm_stream_kernel(GemmArgs args) {
  using M_ = Mma<DT>;
  using T = typename M_::T;
  using AccT = typename Acc<BITS>::T;
  static_assert(DT != FXPR_DTYPE_F32, "16-bit inputs only");
  constexpr int MB = ST::MB, NW = ST::NW, D = ST::DEPTH;
  constexpr int KS = 4;  // 32-k MFMA steps per 128-k K-tile
  __shared__ AccT red[NW - 1][MB * 4][64];  // waves 1 .. NW - 1 hand their sums to wave 0

  const T* A = static_cast<const T*>(args.a);
  const T* B = static_cast<const T*>(args.b);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n0 = int64_t(blockIdx.x) * 16;
  const int nt = (args.ktiles + NW - 1) / NW;  // steps, every wave
  const int kt0 = wave * nt;                   // this wave's first K-tile
  const int r = lane & 15, g = lane >> 4;
  // rows past M and columns past N are clamped: they feed only outputs that
  // are never stored
  const T* bp = B + min<int64_t>(n0 + r, args.N - 1) * args.ldb + g * 8;
  const T* ap[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) ap[i] = A + min<int64_t>(i * 16 + r, args.M - 1) * args.lda + g * 8;

  struct Frags {
    uint4 b[KS];
    uint4 a[MB][KS];
  };
  Frags f[D];
  // step t: K-tile kt0 + t (a stand-in load past the run)
  auto load = [&](Frags& x, int t) {
    const bool real = kt0 + t < args.ktiles && t < nt;  // uniform
    const int64_t k0 = int64_t(kt0 + t) * 128;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      x.b[s] = __builtin_bit_cast(
          uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(real ? bp + k0 + 32 * s : A)));
#pragma unroll
      for (int i = 0; i < MB; ++i) x.a[i][s] = *reinterpret_cast<const uint4*>(real ? ap[i] + k0 + 32 * s : A);
    }
  };

  AccT I[MB][4];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) I[i][q] = 0;
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Frags& x) {
    f32x4 P[MB];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int i = 0; i < MB; ++i) P[i] = M_::mma(x.a[i][s], x.b[s], s == 0 ? zero4 : P[i]);
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) I[i][q] = wrap_add<BITS>(I[i][q], quant<BITS>(__fmul_rn(P[i][q], args.scale)));
  };

  if (nt > 0) {  // uniform (K > 0)
    static_for<D - 1>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      load(f[j], j);
    });
    for (int t = 0; t < nt; t += D) {
      static_for<D>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        load(f[(j + D - 1) % D], t + j + D - 1);
        if (t + j < nt && kt0 + t + j < args.ktiles) compute(f[j]);  // uniform
      });
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave - 1][i * 4 + q][lane] = I[i][q];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < NW - 1; ++w)
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) I[i][q] = wrap_add<BITS>(I[i][q], red[w][i * 4 + q][lane]);
  // lane (r, g) holds rows 16 i + 4 g + q of column n0 + r
  const int64_t n = n0 + r;
  if (n >= args.N) return;
  const float bv = args.bias ? args.bias[n] : 0.0f;
  T* C = static_cast<T*>(args.c);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t m = i * 16 + 4 * g + q;
      if (m >= args.M) continue;
      float v = acc_to_f32<BITS>(I[i][q], args.inv_scale);
      if (args.bias) v = __fadd_rn(v, bv);
      C[m * args.scm + n * args.scn] = Io<DT>::store(v);
    }
}

// ---------------------------------------------------------------------------
// host side

template <int DT, class TL> constexpr size_t lds_bytes() {
  return size_t(2) * (TL::BM + TL::BN) * (Mma<DT>::BKS + Mma<DT>::CHUNK) * sizeof(typename Mma<DT>::T);
}

template <int DT, int BITS, class TL, bool BN_, bool VEC, bool SPLIT>
int launch_tile(const GemmArgs& a, int splits, hipStream_t st) {
  auto kern = gemm_fxp_kernel<DT, BITS, TL, BN_, VEC, SPLIT>;
  constexpr size_t lds = lds_bytes<DT, TL>();
  static bool attr_done = false;  // benign race: the attribute is idempotent
  if (!attr_done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return int(e);
    attr_done = true;
  }
  dim3 grid(unsigned(a.tiles_m * a.tiles_n), unsigned(splits));
  kern<<<grid, kThreads, lds, st>>>(a);
  return launch_status();
}

template <int DT, int BITS, class BT, bool WIDEN = false, bool REDO = false>
int launch_big(GemmArgs a, int splits, hipStream_t st) {
  a.tiles_m = int(cdiv(a.M, BT::BM));
  a.tiles_n = int(cdiv(a.N, BT::BN));
  constexpr size_t lds = big_lds_bytes<BT>();
  auto go = [&](auto kern) -> int {
    static bool attr_done = false;  // benign race: the attribute is idempotent
    if (!attr_done) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
      if (e != hipSuccess) return int(e);
      attr_done = true;
    }
    const int64_t tiles = int64_t(a.tiles_m) * a.tiles_n;
    kern<<<dim3(unsigned(REDO ? cdiv(tiles, 64) : tiles), unsigned(splits)), BT::THREADS, lds, st>>>(a);
    return launch_status();
  };
  if constexpr (REDO) {
    return go(gemm_big_kernel<DT, BITS, BT, false, false, true>);
  } else if constexpr (WIDEN) {
    return go(gemm_big_kernel<DT, BITS, BT, false, true>);
  } else {
    if (splits > 1 || a.mode == kPartial) return go(gemm_big_kernel<DT, BITS, BT, true>);
    return go(gemm_big_kernel<DT, BITS, BT, false>);
  }
}

template <int DT, int BITS, class TL, bool BNC, bool VEC>
int launch_cfg(GemmArgs a, int splits, hipStream_t st) {
  a.tiles_m = int(cdiv(a.M, TL::BM));
  a.tiles_n = int(cdiv(a.N, TL::BN));
  if (splits > 1 || a.mode == kPartial) return launch_tile<DT, BITS, TL, BNC, VEC, true>(a, splits, st);
  return launch_tile<DT, BITS, TL, BNC, VEC, false>(a, splits, st);
}

// Decode-shape kernel launch: one 16-row fragment (M <= 16), four waves,
// four K-tiles in flight per wave. It is taken where it beats split-K on the
// large tiles (graph-timed, bf16, K = 4096 / 14336): M <= 16 with N <= 8192,
// e.g. N = 4096 at M = 1: 10 against 17 us; N = 6144: 15 against 18 us;
// K = 14336: 28 against 34 us. Wider N streams as fast or faster from the
// long-lived 16 x 256 tiles (N = 28672 / 128256 at M = 1: 43 / 170 us; a
// persistent form of this kernel took 44 / 185), and M = 17 .. 64 from the
// large-M kernel's tiles split over K (32-row fragments here: 16-17 against
// 17-18 us at N = 4096, but 28-31 against 22-23 at N = 6144 and 49-52
// against 33-34 at K = 14336, with two or four K-tiles in flight, two
// workgroups per CU or eight waves; 64-row fragments 50 against 23 at
// N = 4096).
constexpr int64_t kStreamMaxM = 16, kStreamMaxN = 8192;

// Shapes the decode-shape kernel takes (16-bit inputs, unsplit)
inline bool stream_shape(int64_t M, int64_t N) { return M <= kStreamMaxM && N <= kStreamMaxN; }
inline bool stream_ok(const GemmArgs& a, bool vec, bool b_ncontig) {
  return vec && !b_ncontig && stream_shape(a.M, a.N) && a.K % 128 == 0;
}

template <int DT, int BITS, class ST> int launch_stream_tile(const GemmArgs& a, hipStream_t st) {
  gemm_stream_kernel<DT, BITS, ST><<<dim3(unsigned(cdiv(a.N, 16))), ST::THREADS, 0, st>>>(a);
  return launch_status();
}

template <int DT, int BITS> int launch_stream(const GemmArgs& a, hipStream_t st) {
  return launch_stream_tile<DT, BITS, StreamTile<1, 4, 4>>(a, st);
}

// Tile configuration by M. Only speed depends on it: every config issues the
// same MFMA chain per output element.
enum class TileId { M16, M32, M64, Big };
inline TileId pick_tile(int64_t M) {
  if (M <= 16) return TileId::M16;
  if (M <= 32) return TileId::M32;
  if (M <= 64) return TileId::M64;
  return TileId::Big;
}
using T16 = Tile<16, 256, 16, 64>;
using T32 = Tile<32, 256, 32, 64>;
using T64 = Tile<64, 256, 64, 64>;
using TBig = Tile<128, 128, 64, 64>;

// rows for which 16-bit K-contiguous operands take gemm_big_kernel
inline bool big_rows(int64_t M) { return M > 16; }

inline void tile_dims(TileId t, int& bm, int& bn) {
  switch (t) {
    case TileId::M16: bm = T16::BM; bn = T16::BN; break;
    case TileId::M32: bm = T32::BM; bn = T32::BN; break;
    case TileId::M64: bm = T64::BM; bn = T64::BN; break;
    default: bm = TBig::BM; bn = TBig::BN; break;
  }
}

// Instantiation matrix: the vectorised K-contiguous-B path (weights as
// stored by the vLLM glue) gets every tile; the N-contiguous-B path gets a
// skinny and a square tile; misaligned / ragged operands (scalar loads) use
// the square tile only. Tile choice never changes bits.
template <int DT, int BITS>
int dispatch_tile(const GemmArgs& a, bool b_ncontig, bool vec, int splits, hipStream_t st) {
  const TileId t = pick_tile(a.M);
  // gemm_big_kernel's 32-bit lane offsets span up to 256 rows of A or B.
  // From M = 17 its tiles (rows past M clamped, never stored) beat the skinny
  // tiles: 183 / 187 us against 215 / 244 at M = 32 / 64 on the lm_head with
  // 128 x 128 tiles (64-bit sums: 189 / 192 against 245 / 362), and the
  // 64 x 256 ones of M <= 64 more; at M <= 16 the skinny tile streams B
  // faster (153 against 176 us).
  const bool big_ok = vec && !b_ncontig && big_rows(a.M) && a.lda <= (int64_t(1) << 22) &&
                      a.ldb <= (int64_t(1) << 22);
  const bool full = a.mode == kFull;
  if constexpr (DT != FXPR_DTYPE_F32) {
    // decode shapes: stream B once, no split-K partials
    if (full && splits <= 1 && stream_ok(a, vec, b_ncontig)) return launch_stream<DT, BITS>(a, st);
  }
  if constexpr (DT != FXPR_DTYPE_F32 && BITS == 64) {
    if (big_ok) {
      // Unsplit, fewer than 512 K-tiles: 32-bit sums in the two-workgroups-
      // per-CU schedule (the 64-bit state of the exact kernel leaves it one
      // wave per SIMD), then the exact kernel on the tiles that pass marked (a
      // K-tile outside the rounding-constant range). Only for f <= 20 (|P| < 4
      // per K-tile stays in range; at larger f most tiles would be computed
      // twice). 1.4-1.8x faster than the exact kernel alone from M = 65 up.
      if (full && splits <= 1 && a.ktiles < 512 && a.fast_lim >= 4.0f) {
        const int rc = launch_big<DT, 32, TB2, true>(a, 1, st);
        if (rc != FXPR_OK) return rc;
        return launch_big<DT, BITS, TB64, false, true>(a, 1, st);
      }
      return launch_big<DT, BITS, TB64>(a, splits, st);
    }
  }
  if constexpr (DT != FXPR_DTYPE_F32 && BITS != 64) {
    if (big_ok && ts64_rows(a.M, BITS)) return launch_big<DT, BITS, TS64>(a, splits, st);
    if (big_ok) return launch_big<DT, BITS, TB2>(a, splits, st);
  }
  if (vec && !b_ncontig) {
    switch (t) {
      case TileId::M16: return launch_cfg<DT, BITS, T16, false, true>(a, splits, st);
      case TileId::M32: return launch_cfg<DT, BITS, T32, false, true>(a, splits, st);
      case TileId::M64: return launch_cfg<DT, BITS, T64, false, true>(a, splits, st);
      default: return launch_cfg<DT, BITS, TBig, false, true>(a, splits, st);
    }
  }
  if (vec) {
    if (t == TileId::M16) return launch_cfg<DT, BITS, T16, true, true>(a, splits, st);
    return launch_cfg<DT, BITS, TBig, true, true>(a, splits, st);
  }
  if (b_ncontig) return launch_cfg<DT, BITS, TBig, true, false>(a, splits, st);
  return launch_cfg<DT, BITS, TBig, false, false>(a, splits, st);
}

template <int DT, int BITS>
int run_gemm(GemmArgs a, bool b_ncontig, bool vec, int splits, hipStream_t st) {
  if (a.mode != kFinish) {
    const int rc = dispatch_tile<DT, BITS>(a, b_ncontig, vec, splits, st);
    if (rc != FXPR_OK || splits <= 1 || a.mode == kPartial) return rc;
  }
  const int64_t mn = a.M * a.N;
  const int rvec = mn % kReduceVec == 0 && (reinterpret_cast<uintptr_t>(a.ws) & 15) == 0;
  gemm_splitk_reduce_kernel<DT, BITS><<<dim3(unsigned(cdiv(mn, 256 * kReduceVec))), 256, 0, st>>>(a, splits, rvec);
  return launch_status();
}

inline int ktile_for(int io_dtype) { return io_dtype == FXPR_DTYPE_F32 ? 64 : 128; }

// Split count: explicit request wins (clamped to the K-tile count);
// otherwise none for the shapes of the decode-shape kernel (16-bit, M <= 16,
// N <= 8192), and elsewhere a split only when the output tiles (of the
// kernel the shape and accumulator width take) cannot fill the 256 CUs about
// twice: 512 / tiles splits, at most 16.
inline int resolve_splits(int64_t M, int64_t N, int64_t K, int io_dtype, int int_bits, int requested) {
  const int ktiles = int(cdiv(K, ktile_for(io_dtype)));
  if (ktiles <= 1) return 1;
  int s;
  if (requested >= 1) {
    s = requested;
  } else {
    // 16-bit decode shapes take the streaming kernel, which needs no split
    if (io_dtype != FXPR_DTYPE_F32 && stream_shape(M, N)) return 1;
    int bm, bn;
    tile_dims(pick_tile(M), bm, bn);
    if (big_rows(M) && io_dtype != FXPR_DTYPE_F32) {
      const bool s64 = ts64_rows(M, int_bits);
      bm = s64 ? TS64::BM : TB2::BM;  // TB64 has TB2's tile
      bn = s64 ? TS64::BN : TB2::BN;
    }
    const int64_t tiles = cdiv(M, bm) * cdiv(N, bn);
    if (tiles >= 256) return 1;
    s = int(512 / tiles);
    if (s > 16) s = 16;
  }
  if (s > ktiles) s = ktiles;
  return s < 1 ? 1 : s;
}

inline int64_t ws_bytes_for(int64_t M, int64_t N, int int_bits, int splits) {
  return splits > 1 ? int64_t(splits) * M * N * (int_bits == 64 ? 8 : 4) : 0;
}


// Per-dtype entry (one translation unit each, built in parallel).
int run_gemm_bf16(const GemmArgs& a, int bits, bool b_ncontig, bool vec, int splits, hipStream_t st);
int run_gemm_f16(const GemmArgs& a, int bits, bool b_ncontig, bool vec, int splits, hipStream_t st);
int run_gemm_f32(const GemmArgs& a, int bits, bool b_ncontig, bool vec, int splits, hipStream_t st);

}  // namespace gemm
}  // namespace fxpr
