// Paged prefill + decode attention with fixed-point cross-tile reductions
// (gfx950 MFMA). Kernels are instantiated per input type in attn_*.hip.
//
// Per (request r, query row i, head h), keys n of the request's paged KV,
// in absolute chunks C of CT*64 = 512 keys:
//   s_n   = fl32(q . k_n) * scale*log2e  [softcap] [+ alibi*(n - qpos)],
//           -inf where masked (causal n > qpos, window, n >= seq_len)
//   m_C   = max_{n in C} s_n                 (the chunk's own row maximum)
//   w_n   = exp2(s_n - m_C)
//   den_C = sum_{n in C} RNE_sat(w_n * 2^f)                       (integer)
//   wv_C  = sum_{tiles of C} RNE_sat(fl32(sum_{n in tile} IO(w_n) v_n[d]) * 2^f)
//   fold the chunks in ascending order into (M, den, wv):
//     M' = max(M, m_C), den' = rescale(den, 2^(M - M')) + rescale(den_C, 2^(m_C - M')),
//     wv' likewise, rescale(x, f) = RNE_sat(fl64(x) * f)
//   o_d   = IO(fl32(wv_d) 2^-f / max(fl32(den) 2^-f, 1e-6))
// Replaces _attn_fused_kernel / _attn_split_max_kernel / _attn_split_dv_kernel
// (fxpr_vllm/_triton/attention.py:127-301, 306-436, 440-652), which take every
// weight against the row's global maximum and so read K twice (or exchange
// maxima between splits first). Here each key is read once: a chunk's scores
// stay in registers between its K and V halves. A row whose keys fit in one
// chunk gets the reference's formula exactly. Key tiles (64 keys, the
// quantised chains 64 keys for bf16/f16 and 32 for f32, the reference's
// BLOCK_N) and chunks are aligned to absolute key positions, and every score,
// tile partial and fold step comes from the same instruction sequence for a
// given row whatever the workgroup's other rows, the split count or the
// decode / prefill shape, so outputs are bitwise invariant to all of them.
// Splits write per-chunk partials, folded by a combine kernel in the same
// order: no atomics, nothing to pre-zero.
#pragma once

#include <type_traits>
#include <utility>

#include "fxp_device.h"
#include "fxpr_internal.h"

namespace fxpr {
namespace attn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
// 16 bytes as a native vector (HIP's uint4 is a struct whose copies can
// become memcpys that keep arrays of them out of registers)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int TILE = 64;       // keys per iteration (and per split unit)
constexpr int QROWS = 16;      // query rows (query x GQA head) per workgroup

constexpr int CT = 8;          // key tiles per chunk (the unit of the softmax statistics)

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* qsl;
  const int32_t* seq_lens;
  const int32_t* bt;
  const float* alibi;  // per q head, already multiplied by log2(e); or null
  float* pmax;         // [T, Hq, chunk_slots] per-chunk row maxima         (split launches)
  void* den_ws;        // [T, Hq, chunk_slots] denominators, int32 / int64  (split launches)
  void* wv_ws;         // [T, Hq, chunk_slots, D] weighted V, int32 / int64 (split launches)
  int* crange;         // [T, Hq, 2] chunk range [first, end) of the row    (split launches)
  int64_t sq_t, sq_h, sk_b, sk_s, sk_h, sv_b, sv_s, sv_h, so_t, so_h, sbt;
  int num_heads, num_kv_heads, group, head_dim, page_size, num_splits, window, causal;
  int max_blocks;       // block-table row length
  int chunks_per_split;  // > 0: fixed chunks per split (work-balanced); 0: even division
  int chunk_slots;       // chunks per row in the split workspace
  int pq_rows;           // > 0: requests with at least this many rows go to attn_prefill_kernel
  int num_requests;
  int64_t num_blocks;   // physical blocks in the cache
  int64_t num_tokens;   // rows of q / o
  int64_t lmax;         // key capacity of a block-table row (max_blocks * page_size)
  int ps_shift;         // log2(page_size) if a power of two, else -1
  float scale_log2, softcap_log2, fxp_scale, fxp_inv;
};

template <int DT> struct Traits;
template <> struct Traits<FXPR_DTYPE_BF16> {
  using T = uint16_t;
  static constexpr int KI = 32, QUNIT = 64, CH = 8;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Traits<FXPR_DTYPE_F16> {
  using T = uint16_t;
  static constexpr int KI = 32, QUNIT = 64, CH = 8;
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Traits<FXPR_DTYPE_F32> {
  using T = float;
  static constexpr int KI = 4, QUNIT = 32, CH = 4;
  static __device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <int BITS> struct AccOf { using T = int32_t; };
template <> struct AccOf<64> { using T = int64_t; };

template <int BITS> __device__ __forceinline__ typename AccOf<BITS>::T wadd(typename AccOf<BITS>::T a, int64_t b) {
  if constexpr (BITS == 64) return static_cast<int64_t>(static_cast<uint64_t>(a) + static_cast<uint64_t>(b));
  else return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}

template <int BITS> __device__ __forceinline__ float acc_f32(typename AccOf<BITS>::T v, float inv) {
  if constexpr (BITS == 16) return fixed_to_f32(static_cast<int32_t>(static_cast<int16_t>(v)), inv);
  else return fixed_to_f32(v, inv);
}

__device__ __forceinline__ float tanh_approx(float x) {
  // tanh(x) = sign(x) (1 - 2 / (2^(2|x| log2 e) + 1)); tolerance path only
  const float e = __builtin_amdgcn_exp2f(2.0f * 1.44269504088896341f * __builtin_fabsf(x));
  const float t = 1.0f - 2.0f / (e + 1.0f);
  return x < 0.0f ? -t : t;
}

// Query-row bookkeeping for one of the workgroup's 16 rows.
struct RowInfo {
  int64_t token;
  int head;
  int qpos;
  int kstart, kend;  // valid keys [kstart, kend)
  bool valid;
};

__device__ __forceinline__ RowInfo row_info(const AttnArgs& a, int g, int q_start, int q_len, int ctx,
                                            int seq_len, int row) {
  RowInfo ri;
  const int rows_total = q_len * a.group;
  const int rr = row < rows_total ? row : 0;
  const int i = rr / a.group, hh = rr % a.group;
  ri.token = q_start + i;
  // rows past the request, or past q / o (inconsistent metadata), are inert
  ri.valid = row < rows_total && ri.token >= 0 && ri.token < a.num_tokens;
  if (!ri.valid) ri.token = 0;
  ri.head = g * a.group + hh;
  ri.qpos = ctx + i;
  ri.kend = a.causal ? min(seq_len, ri.qpos + 1) : seq_len;
  ri.kstart = a.window > 0 ? max(0, ri.qpos - a.window + 1) : 0;
  return ri;
}

// Per-row statistics of key chunks are folded in fixed point: an accumulator
// (wrapped to BITS) times f <= 1, rounded half-to-even in fp64 and saturated.
// Shared by the kernel's in-register merge and the combine kernel, so both
// produce the same bits.
template <int BITS> __device__ __forceinline__ typename AccOf<BITS>::T rescale(typename AccOf<BITS>::T x, float f) {
  double xv;
  if constexpr (BITS == 16) xv = static_cast<double>(static_cast<int16_t>(x));
  else xv = static_cast<double>(x);
  const double r = __builtin_rint(xv * static_cast<double>(f));
  if constexpr (BITS == 64) {
    // |r| <= |x| <= 2^63; only x near INT64_MAX can round up to 2^63
    if (r >= 9223372036854775808.0) return INT64_MAX;
    return static_cast<int64_t>(r);
  } else {
    return static_cast<int32_t>(r);  // |r| <= 2^31, integral
  }
}

// Running (M, D, W) of a row folded with one chunk's (mc, dc, wc), mc finite:
// M' = max(M, mc), D' = rescale(D, 2^(M - M')) + rescale(dc, 2^(mc - M')).
__device__ __forceinline__ void merge_factors(float M, float mc, float& Mn, float& fa, float& fb) {
  Mn = fmaxf(M, mc);
  fa = __builtin_amdgcn_exp2f(M - Mn);  // M = -inf (empty state): 0
  fb = __builtin_amdgcn_exp2f(mc - Mn);
}

template <int DT, int BITS, int DMAX, bool SPLIT>
__global__ __launch_bounds__(kThreads) void attn_kernel(AttnArgs a) {
  using TR = Traits<DT>;
  using T = typename TR::T;
  using AccT = typename AccOf<BITS>::T;
  using KFrag = typename std::conditional<DT == FXPR_DTYPE_F32, float, u32x4>::type;
  constexpr int KI = TR::KI, CH = TR::CH;
  constexpr int QSTEPS = DMAX / KI;       // MFMAs per 16x16 score block
  constexpr int DBLK = DMAX / 16;         // 16-wide d blocks of the output
  constexpr int DB_PER_WAVE = (DBLK + 3) / 4;
  // LDS pitch of Vt / Ps rows. 16-bit: +8 elements and the key column of Vt
  // XOR-swizzled by d-chunk (keeps 16-byte fragments contiguous, spreads the
  // transposing writes over banks); f32: odd pitch, no swizzle.
  constexpr int VP = DT == FXPR_DTYPE_F32 ? TILE + 1 : TILE + 8;
  constexpr int QUNIT = TR::QUNIT;
  constexpr int VCH = DMAX / CH;                    // 16-byte chunks per key row of a V tile
  constexpr int VITER = TILE * VCH / kThreads;      // V chunks per thread per tile

  // V tile in LDS. f32: transposed [d][key]. 16-bit: natural [key][d] (row
  // pitch VNP), turned into MFMA B operands by ds_read_b64_tr_b16.
  constexpr bool TR16 = DT != FXPR_DTYPE_F32;
  constexpr int VNP = DMAX + 16;
  __shared__ __align__(16) T Vt[TR16 ? TILE * VNP : DMAX * VP];
  __shared__ __align__(16) T Ps[QROWS * VP]; // IO-rounded weights: [row][key]
  __shared__ float red_f[4][QROWS];
  __shared__ AccT red_i[4][QROWS];
  auto vcol = [](int d, int key) -> int {
    if constexpr (DT == FXPR_DTYPE_F32) return key;
    else return key ^ (((d >> 3) & 7) << 3);
  };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The hardware deals consecutive workgroup ids to the 8 XCDs round-robin,
  // so the kv heads of one request (which share every KV page) run at the
  // same time on different XCDs, and the XCDs stay balanced whatever the
  // spread of context lengths.
  const int logical = blockIdx.x;
  const int r = logical / a.num_kv_heads, g = logical % a.num_kv_heads;
  const int qt = blockIdx.y, split = blockIdx.z;
  const int q_start = a.qsl[r];
  const int q_len = a.qsl[r + 1] - q_start;
  const int seq_len = a.seq_lens[r];
  const int ctx = seq_len - q_len;
  const int rows_total = q_len * a.group;
  const int row0 = qt * QROWS;
  if (row0 >= rows_total) return;  // uniform
  if (a.pq_rows > 0 && rows_total >= a.pq_rows) return;  // attn_prefill_kernel's request

  // Key range of the workgroup (union over its rows), in absolute tiles, and
  // the absolute key chunks (CT tiles) it touches. A chunk's statistics are
  // per row, so they do not depend on the workgroup's other rows.
  const int i_min = row0 / a.group;
  const int i_max = min(rows_total - 1, row0 + QROWS - 1) / a.group;
  const int hi = a.causal ? min(seq_len, ctx + i_max + 1) : seq_len;
  const int lo = a.window > 0 ? max(0, ctx + i_min - a.window + 1) : 0;
  const int t_lo = lo / TILE;
  const int t_hi = hi > lo ? (hi + TILE - 1) / TILE : t_lo;
  const int c_lo = t_lo / CT;
  int c_hi = t_hi > t_lo ? (t_hi + CT - 1) / CT : c_lo;
  if constexpr (SPLIT) c_hi = min(c_hi, a.chunk_slots);  // workspace bound (only inconsistent metadata)
  const int nch = max(0, c_hi - c_lo);
  const int per = a.chunks_per_split > 0 ? a.chunks_per_split : (nch + a.num_splits - 1) / a.num_splits;
  const int my_lo = SPLIT ? c_lo + min(nch, split * per) : c_lo;
  const int my_hi = SPLIT ? min(c_lo + nch, my_lo + per) : c_lo + nch;

  const int32_t* bt_row = a.bt + int64_t(r) * a.sbt;
  const T* Kc = static_cast<const T*>(a.k);
  const T* Vc = static_cast<const T*>(a.v);
  const T* Qp = static_cast<const T*>(a.q);
  const int kg = lane >> 4;  // lane group = MFMA k slot

  // Paged addressing. Keys are clamped to [0, seq_len) and block-table /
  // block indices to their ranges, so inconsistent metadata can never address
  // outside the table or the cache (such keys are masked anyway).
  auto clamp_key = [&](int key) { return max(0, min(key, seq_len - 1)); };
  auto bt_entry = [&](int key) -> int {
    const int lb = a.ps_shift >= 0 ? (key >> a.ps_shift) : key / a.page_size;
    return bt_row[min(lb, a.max_blocks - 1)];
  };
  // Element offsets as 32 x 32 -> 64-bit products (the host guarantees
  // cache strides below 2^32): a full 64 x 64 product is expanded with an
  // undefined high half that can land on a register with a load in flight,
  // and reading it would wait for that load.
  const int last_block = int(a.num_blocks - 1 < 0x7fffffff ? a.num_blocks - 1 : 0x7fffffff);
  auto row_addr = [&](int key, int entry, int64_t sb, int64_t ss, int64_t sh) -> uint64_t {
    const uint32_t p = uint32_t(entry < 0 ? 0 : min(entry, last_block));
    const uint32_t slot = uint32_t(a.ps_shift >= 0 ? (key & (a.page_size - 1)) : key % a.page_size);
    return uint64_t(p) * uint32_t(sb) + uint64_t(slot) * uint32_t(ss) + uint64_t(uint32_t(g)) * uint32_t(sh);
  };

  // Q fragments (MFMA A operand): lane holds row lane%16, its k slots.
  KFrag qf[QSTEPS];
  {
    const RowInfo qrow = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + (lane & 15));
    const T* qbase = Qp + qrow.token * a.sq_t + int64_t(qrow.head) * a.sq_h;
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) {
      if constexpr (DT == FXPR_DTYPE_F32) {
        // step j = 4u + e uses d = 16u + 4*kg + e
        const int d = 16 * (j >> 2) + 4 * kg + (j & 3);
        qf[j] = (qrow.valid && d < a.head_dim) ? qbase[d] : 0.0f;
      } else {
        const int d = 32 * j + 8 * kg;
        qf[j] = (qrow.valid && d < a.head_dim) ? *reinterpret_cast<const u32x4*>(qbase + d)
                                                : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }

  // Rows held in the score layout: rows 4*kg + e, key lane%16 of the wave's
  // 16-key block.
  RowInfo srow[4];
  float slope[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    srow[e] = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + 4 * kg + e);
    slope[e] = a.alibi ? a.alibi[srow[e].head] : 0.0f;
  }
  if (SPLIT && split == 0 && tid < QROWS) {
    // the chunk range every split of this workgroup's rows covers together
    const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + tid);
    if (ri.valid) {
      int* cr = a.crange + 2 * (ri.token * a.num_heads + ri.head);
      cr[0] = c_lo;
      cr[1] = c_lo + nch;
    }
  }

  // K fragments of the lane's key of tile t (key clamped, bt entry given).
  // Every load is issued unconditionally: loads under a branch would leave
  // the compiler unable to count outstanding loads, and it would then wait
  // for all of them. Columns past head_dim read column 0 of the same key;
  // their products vanish because the Q fragments there are zero.
  auto k_load = [&](int t, int entry, KFrag (&kf)[QSTEPS]) {
    const int key = clamp_key(t * TILE + wave * 16 + (lane & 15));
    const T* kp = Kc + row_addr(key, entry, a.sk_b, a.sk_s, a.sk_h);
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) {
      if constexpr (DT == FXPR_DTYPE_F32) {
        const int d = 16 * (j >> 2) + 4 * kg + (j & 3);
        kf[j] = kp[d < a.head_dim ? d : 0];
      } else {
        const int d = 32 * j + 8 * kg;
        kf[j] = *reinterpret_cast<const u32x4*>(kp + (d < a.head_dim ? d : 0));
      }
    }
  };
  auto k_entry = [&](int t) { return bt_entry(clamp_key(t * TILE + wave * 16 + (lane & 15))); };

  // Scaled, transformed, masked log2-space scores of tile t.
  auto k_scores = [&](int t, const KFrag (&kf)[QSTEPS], float (&s)[4]) {
    const int key = t * TILE + wave * 16 + (lane & 15);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) acc = TR::mma(qf[j], kf[j], acc);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = __fmul_rn(acc[e], a.scale_log2);
      if (a.softcap_log2 > 0.0f) x = a.softcap_log2 * tanh_approx(x / a.softcap_log2);
      if (a.alibi) x = x + slope[e] * static_cast<float>(key - srow[e].qpos);
      const bool ok = srow[e].valid && key >= srow[e].kstart && key < srow[e].kend;
      s[e] = ok ? x : -__builtin_inff();
    }
  };

  // V chunk c = i*256 + tid of a tile: key c / VCH, d chunk (c % VCH) * CH
  // (each wave instruction reads whole 16-byte-aligned key rows).
  auto v_entries = [&](int t, int (&ve)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i)
      ve[i] = bt_entry(clamp_key(t * TILE + (i * kThreads + tid) / VCH));
  };
  auto v_load = [&](int t, const int (&ve)[VITER], u32x4 (&vr)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i) {
      const int c = i * kThreads + tid;
      const int key = clamp_key(t * TILE + c / VCH), d0 = (c % VCH) * CH;
      // columns past head_dim (read from column 0) only reach output
      // columns that are never stored
      vr[i] = *reinterpret_cast<const u32x4*>(Vc + row_addr(key, ve[i], a.sv_b, a.sv_s, a.sv_h) +
                                              (d0 < a.head_dim ? d0 : 0));
    }
  };

  // Chunk accumulators (lane rows 4*kg + e; PV layout d = db*16 + lane%16)
  // and the row maxima the chunk's weights are taken against.
  float m[4];
  AccT den[4];
  AccT wv[DB_PER_WAVE][4];

  // One key tile: weights from the scores, V tile to LDS, PV partials.
  auto accumulate = [&](int t, const u32x4 (&vr)[VITER], const float (&s)[4]) __attribute__((always_inline)) {
    const int kin = wave * 16 + (lane & 15);  // key within the tile
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float w = __builtin_amdgcn_exp2f(s[e] - m[e]);
      den[e] = wadd<BITS>(den[e], quant<BITS>(__fmul_rn(w, a.fxp_scale)));
      Ps[(4 * kg + e) * VP + kin] = Io<DT>::store(w);
    }
#pragma unroll
    for (int i = 0; i < VITER; ++i) {  // V tile -> LDS
      const int c = i * kThreads + tid;
      const int kk = c / VCH, d0 = (c % VCH) * CH;
      if constexpr (TR16) {
        *reinterpret_cast<u32x4*>(&Vt[kk * VNP + d0]) = vr[i];
      } else {  // transposed to [d][key]
        union {
          u32x4 v;
          T e[CH];
        } u;
        u.v = vr[i];
#pragma unroll
        for (int j = 0; j < CH; ++j) Vt[(d0 + j) * VP + vcol(d0 + j, kk)] = u.e[j];
      }
    }
    __syncthreads();
    // PV: wave handles d blocks wave, wave+4, ...; one quantised chain per
    // QUNIT keys
#pragma unroll
    for (int b = 0; b < DB_PER_WAVE; ++b) {
      const int db = wave + 4 * b;
      if (db < DBLK) {
        const int dv = db * 16 + (lane & 15);
#pragma unroll
        for (int u0 = 0; u0 < TILE; u0 += QUNIT) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int k0 = 0; k0 < QUNIT; k0 += KI) {
            if constexpr (DT == FXPR_DTYPE_F32) {
              const int key = u0 + k0 + kg;
              acc = TR::mma(Ps[(lane & 15) * VP + key], Vt[dv * VP + vcol(dv, key)], acc);
            } else {
              // B operand: lane (kg, i) needs V[keys key..key+7][d = db*16 + i].
              // ds_read_b64_tr_b16 gives lane i of each 16-lane group
              // element (i % 4) of source lane 4c' + i/4, c' = 0..3; source
              // lane j points at V[key0 + j/4][db*16 + 4*(j%4)].
              const int key = u0 + k0 + 8 * kg;
              const int j = lane & 15;
              typedef short v4s __attribute__((ext_vector_type(4)));
              const T* src = &Vt[(key + (j >> 2)) * VNP + db * 16 + 4 * (j & 3)];
              const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(src));
              const v4s hi4 =
                  __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(src + 4 * VNP));
              struct {
                v4s a, b;
              } both = {lo4, hi4};
              acc = TR::mma(*reinterpret_cast<const u32x4*>(&Ps[(lane & 15) * VP + key]),
                            __builtin_bit_cast(u32x4, both), acc);
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) wv[b][e] = wadd<BITS>(wv[b][e], quant<BITS>(__fmul_rn(acc[e], a.fxp_scale)));
        }
      }
    }
    __syncthreads();
  };

  // Running state of the lane's rows (single-pass launches only).
  float Mr[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  AccT Dr[4] = {0, 0, 0, 0};
  AccT Wr[DB_PER_WAVE][4];
#pragma unroll
  for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) Wr[b][e] = 0;

  if (my_lo < my_hi) {
    // One chunk is 2*CT pipeline steps: CT K tiles (scores into registers,
    // then the chunk's row maxima), then the same CT tiles of V (weights
    // against those maxima, integer partials). Loads run R-1 steps ahead of
    // use and page entries R steps ahead of their loads, straight across the
    // K -> V boundary and into the next chunk, so the maxima reduction and
    // the chunk's fold overlap loads in flight. Buffers are indexed by
    // compile-time slots, every load is issued unconditionally (tiles outside
    // the chunk's live range, or past the last chunk, reload a live tile),
    // and only the arithmetic of dead tiles is skipped (uniformly).
    constexpr int R = 2;
    constexpr int NSTEP = 2 * CT;
    static_assert(CT % R == 0, "ring slots must repeat every chunk");
    KFrag kb[R][QSTEPS];
    int eb[R];
    u32x4 vb[R][VITER];
    int veb[R][VITER];
    float sc[CT][4];

    int c = my_lo;
    auto live_lo = [&](int cc) { return max(cc * CT, t_lo); };
    auto live_hi = [&](int cc) { return min(cc * CT + CT, t_hi); };
    int ta = live_lo(c), te = live_hi(c);
    int nc = c + 1 < my_hi ? c + 1 : c;
    int nta = live_lo(nc), nte = live_hi(nc);
    // step j of the current chunk (j < NSTEP) or of the next (j >= NSTEP)
    auto entry_step = [&](auto J) __attribute__((always_inline)) {
      constexpr int j = decltype(J)::value, jj = j % NSTEP, sl = j % R;
      const int base = (j >= NSTEP ? nc : c) * CT, l0 = j >= NSTEP ? nta : ta, l1 = j >= NSTEP ? nte : te;
      const int t = min(max(base + (jj < CT ? jj : jj - CT), l0), l1 - 1);
      if constexpr (jj < CT) eb[sl] = k_entry(t);
      else v_entries(t, veb[sl]);
    };
    auto load_step = [&](auto J) __attribute__((always_inline)) {
      constexpr int j = decltype(J)::value, jj = j % NSTEP, sl = j % R;
      const int base = (j >= NSTEP ? nc : c) * CT, l0 = j >= NSTEP ? nta : ta, l1 = j >= NSTEP ? nte : te;
      const int t = min(max(base + (jj < CT ? jj : jj - CT), l0), l1 - 1);
      if constexpr (jj < CT) k_load(t, eb[sl], kb[sl]);
      else v_load(t, veb[sl], vb[sl]);
    };
    static_for<R>([&](auto I) { entry_step(I); });
    static_for<R - 1>([&](auto I) {
      load_step(I);
      entry_step(std::integral_constant<int, decltype(I)::value + R>{});
    });

    for (;;) {
      float mx[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
      float mc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) den[e] = 0;
#pragma unroll
      for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[b][e] = 0;

      static_for<NSTEP>([&](auto I) __attribute__((always_inline)) {
        constexpr int i = decltype(I)::value, sl = i % R;
        load_step(std::integral_constant<int, i + R - 1>{});
        entry_step(std::integral_constant<int, i + 2 * R - 1>{});
        if constexpr (i < CT) {
          const int t = c * CT + i;
          if (t >= ta && t < te) {
            k_scores(t, kb[sl], sc[i]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[i][e] = -__builtin_inff();
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) mx[e] = fmaxf(mx[e], sc[i][e]);
          if constexpr (i == CT - 1) {
            // the chunk's row maxima: 16 key lanes, then the 4 waves
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
              for (int o = 1; o < 16; o <<= 1) mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], o, 64));
              if ((lane & 15) == 0) red_f[wave][4 * kg + e] = mx[e];
            }
            __syncthreads();
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int row = 4 * kg + e;
              mc[e] = fmaxf(fmaxf(red_f[0][row], red_f[1][row]), fmaxf(red_f[2][row], red_f[3][row]));
              m[e] = (srow[e].valid && mc[e] != -__builtin_inff()) ? mc[e] : 0.0f;  // no key: pin to 0
            }
          }
        } else {
          const int t = c * CT + (i - CT);
          if (t >= ta && t < te) accumulate(t, vb[sl], sc[i - CT]);
        }
      });

      // the chunk's denominators: 16 key lanes, then the 4 waves
      AccT dc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) den[e] = wadd<BITS>(den[e], __shfl_xor(den[e], o, 64));
        if ((lane & 15) == 0) red_i[wave][4 * kg + e] = den[e];
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 4 * kg + e;
        dc[e] = wadd<BITS>(wadd<BITS>(red_i[0][row], red_i[1][row]), wadd<BITS>(red_i[2][row], red_i[3][row]));
      }

      if constexpr (SPLIT) {
        // the chunk's partials, per row: maximum, denominator, weighted V
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (!srow[e].valid) continue;
          const int64_t slot = (srow[e].token * a.num_heads + srow[e].head) * a.chunk_slots + c;
          if ((lane & 15) == 0 && wave == 0) {
            a.pmax[slot] = mc[e];
            static_cast<AccT*>(a.den_ws)[slot] = dc[e];
          }
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b) {
            const int d = (wave + 4 * b) * 16 + (lane & 15);
            if (wave + 4 * b < DBLK && d < a.head_dim) static_cast<AccT*>(a.wv_ws)[slot * a.head_dim + d] = wv[b][e];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (mc[e] == -__builtin_inff()) continue;  // no key of the row in this chunk
          float Mn, fa, fb;
          merge_factors(Mr[e], mc[e], Mn, fa, fb);
          Dr[e] = wadd<BITS>(rescale<BITS>(Dr[e], fa), rescale<BITS>(dc[e], fb));
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b)
            Wr[b][e] = wadd<BITS>(rescale<BITS>(Wr[b][e], fa), rescale<BITS>(wv[b][e], fb));
          Mr[e] = Mn;
        }
      }

      if (++c >= my_hi) break;
      ta = nta;
      te = nte;
      nc = c + 1 < my_hi ? c + 1 : c;
      nta = live_lo(nc);
      nte = live_hi(nc);
    }
  }

  if constexpr (!SPLIT) {
    float den_f[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) den_f[e] = fmaxf(acc_f32<BITS>(Dr[e], a.fxp_inv), 1.0e-6f);
    T* Op = static_cast<T*>(a.o);
#pragma unroll
    for (int b = 0; b < DB_PER_WAVE; ++b) {
      const int d = (wave + 4 * b) * 16 + (lane & 15);
      if (wave + 4 * b >= DBLK || d >= a.head_dim) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (!srow[e].valid) continue;
        const float num = acc_f32<BITS>(Wr[b][e], a.fxp_inv);
        Op[srow[e].token * a.so_t + int64_t(srow[e].head) * a.so_h + d] = Io<DT>::store(div_rn(num, den_f[e]));
      }
    }
  }
}

// Decode-shaped launches through LDS DMA (16-bit inputs, head_dim 64 or 128,
// power-of-two pages of at least 16 keys): attn_kernel's 16-row workgroups,
// chunks and bits, with the K and V tiles brought into an NS-stage LDS ring
// by global_load_lds instead of through registers. Each wave moves 16
// consecutive key rows of a tile, all in one page, so its page entry is one
// scalar load, issued a step before the DMAs that use it (no vector-memory
// traffic besides the DMAs, whose count the explicit waits rely on). LDS rows hold 16-byte chunk c of key row r at
// slot c ^ dswz(r): the K fragment reads (16 consecutive rows, one chunk
// each) and the transposing V reads (4 consecutive rows, 32 bytes each) hit
// distinct banks. Every LDS access in the pipelined loop is inline asm: the
// compiler would otherwise wait for all DMAs in flight before it.
template <int DMAX> struct DmaGeom {
  static constexpr int ROWB = DMAX * 2;          // bytes per key row
  static constexpr int CPR = ROWB / 16;          // 16-byte chunks per row
  static constexpr int KPI = 1024 / ROWB;        // key rows per wave instruction
  static constexpr int TILEB = TILE * ROWB;      // bytes per tile
  static constexpr int NDMA = TILEB / (kThreads * 16);  // DMA instructions per thread per tile
  static constexpr int NS = 4;                   // LDS stages (a power of two: stage index by mask)
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (CPR >= 16) {
      return ((r & 3) << 2) | ((r >> 2) & 3);
    } else {
      const int q = (r >> 1) & 7;  // 128-byte rows: pairs share a 256-byte bank window
      return ((q << 1) | (q >> 2)) & 7;
    }
  }
};

typedef __attribute__((address_space(3))) void* AttnLdsPtr;
typedef const __attribute__((address_space(4))) int32_t* ConstI32Ptr;

__device__ __forceinline__ void lds_read_b128(unsigned addr, u32x4& x) {
  asm volatile("ds_read_b128 %0, %1" : "=v"(x) : "v"(addr) : "memory");
}
__device__ __forceinline__ void lds_read_b64_tr16(unsigned addr, uint64_t& x) {
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(x) : "v"(addr) : "memory");
}
__device__ __forceinline__ void lds_read_b32(unsigned addr, uint32_t& x) {
  asm volatile("ds_read_b32 %0, %1" : "=v"(x) : "v"(addr) : "memory");
}
__device__ __forceinline__ void lds_write_b16(unsigned addr, uint32_t x) {
  asm volatile("ds_write_b16 %0, %1" ::"v"(addr), "v"(x) : "memory");
}
__device__ __forceinline__ void lds_write_b32(unsigned addr, uint32_t x) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(x) : "memory");
}
__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// The wait, tied to the registers the reads filled: their uses cannot move
// above it (the asm reads' outputs are otherwise "ready" at issue).
template <class A> __device__ __forceinline__ void lds_wait_for(A& a) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a) : : "memory");
}
template <class A, class B> __device__ __forceinline__ void lds_wait_for(A& a, B& b) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b) : : "memory");
}
template <class A, class B, class C> __device__ __forceinline__ void lds_wait_for(A& a, B& b, C& c) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c) : : "memory");
}
template <class A, class B, class C, class D>
__device__ __forceinline__ void lds_wait_for(A& a, B& b, C& c, D& d) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : : "memory");
}

// Cache-policy operand of the buffer/global load builtins on gfx950: bit 1
// is nt (non-temporal; glc/sc0 is bit 0, sc1 bit 4).
constexpr int kCpolNT = 2;

// Requests in launch order longest first (by sequence length, ties by index)
// for up to kOrderMax of them: request_by_length(a, k) is the k-th longest,
// so the workgroups of the requests that bound the launch are dispatched
// first, and (with two workgroups per CU placed in dispatch order) a long
// request's workgroup tends to share its CU with a short one's. Only the
// dispatch order depends on it, never a bit of the results; it must be a
// permutation of the requests. Wave-uniform, all lanes active: the lane
// holds the lengths of requests lane + 64 j (negative lengths count as 0),
// a radix select over the length bits finds the (k + 1)-th largest length T
// (31 steps of kOrderMax / 64 ballots), then the requests of length T are
// taken in index order. Launches whose workgroups hold at most one chunk
// each keep the launch order (the order gains nothing there).
constexpr int kOrderMax = 256;
__device__ __forceinline__ int request_by_length(const AttnArgs& a, int k) {
  const int R = a.num_requests;
  const int per_max = a.num_splits <= 1 ? a.chunk_slots + 1
                      : a.chunks_per_split > 0 ? a.chunks_per_split
                                               : (a.chunk_slots + a.num_splits - 1) / a.num_splits;
  if (R <= 1 || R > kOrderMax || k >= R || per_max <= 1) return k;
  constexpr int NB = kOrderMax / 64;
  const int lane = threadIdx.x & 63;
  int len[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) len[j] = a.seq_lens[min(64 * j + lane, R - 1)];
  // (through the asm the loads are unconditional, issued together and waited
  // for once; the compiler would otherwise predicate each behind a wait)
  static_assert(NB == 4, "four length blocks");
  asm volatile("" : "+v"(len[0]), "+v"(len[1]), "+v"(len[2]), "+v"(len[3]));
#pragma unroll
  for (int j = 0; j < NB; ++j) len[j] = 64 * j + lane < R ? max(len[j], 0) : -1;  // -1: no request
  auto count_ge = [&](int v) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < NB; ++j) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(len[j] >= v));
    return c;
  };
  // the largest T >= 0 with more than k lengths >= T
  int T = 0;
  for (int b = 30; b >= 0; --b) {
    const int cand = T | (1 << b);
    if (count_ge(cand) > k) T = cand;
  }
  int greater = 0;
#pragma unroll
  for (int j = 0; j < NB; ++j) greater += __builtin_popcountll(__builtin_amdgcn_ballot_w64(len[j] > T));
  int rr = k - greater;  // rank among the requests of length T, by index
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(len[j] == T);
    const int n = __builtin_popcountll(m);
    if (rr < n) {
      const int below = int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
      const uint64_t hit = __builtin_amdgcn_ballot_w64(len[j] == T && below == rr);
      return 64 * j + __builtin_ctzll(hit);
    }
    rr -= n;
  }
  return k;  // not reached: greater <= k < greater + (count of T)
}

// Wait for the DMAs of a step when `later` steps' DMAs (NDMA instructions
// each) were issued after it, at most K of them; and for every LDS / scalar
// memory operation.
template <int K, int NDMA> __device__ __forceinline__ void dma_wait(int later) {
  if constexpr (K == 0) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  } else {
    if (later >= K) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(K * NDMA) : "memory");
    else dma_wait<K - 1, NDMA>(later);
  }
}

template <int DT, int BITS, int DMAX, bool SPLIT>
__global__ __launch_bounds__(kThreads, 2) void attn_dma_kernel(AttnArgs a) {
  static_assert(DT != FXPR_DTYPE_F32, "16-bit inputs only");
  using TR = Traits<DT>;
  using T = typename TR::T;
  using AccT = typename AccOf<BITS>::T;
  using G = DmaGeom<DMAX>;
  constexpr int KI = TR::KI, QUNIT = TR::QUNIT;
  constexpr int QSTEPS = DMAX / KI;
  constexpr int DBLK = DMAX / 16;
  constexpr int DB_PER_WAVE = (DBLK + 3) / 4;
  constexpr int VP = TILE + 8;             // Ps row pitch (elements)
  constexpr int NS = G::NS;
  // LDS: NS tile stages | weights Ps[2][16][VP] | red_f[4][16] | red_i[4][16]
  constexpr int PS_OFF = NS * G::TILEB;
  constexpr int RF_OFF = PS_OFF + 2 * QROWS * VP * 2;
  constexpr int RI_OFF = RF_OFF + 4 * QROWS * 4;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // The dynamic LDS starts where the static LDS ends, rounded up to its
  // alignment: a constant (the address of smem_raw, cast from a generic
  // pointer, comes back as a null test and a select at every use)
  const unsigned lds0 = (__builtin_amdgcn_groupstaticsize() + 15u) & ~15u;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, kg = lane >> 4;
  const int g = blockIdx.x % a.num_kv_heads;
  // (the request index is wave-uniform: its bounds are scalar loads, issued
  // together and waited for once)
  const int r = __builtin_amdgcn_readfirstlane(request_by_length(a, blockIdx.x / a.num_kv_heads));
  const int qt = blockIdx.y, split = blockIdx.z;
  const ConstI32Ptr bt_row = (ConstI32Ptr)(a.bt + int64_t(r) * a.sbt);
  // Without a window, with a fixed chunk count per split (or one split),
  // the first chunk and so the pages of the first NS steps (its first K
  // tiles) follow from the launch alone: their page entries are loaded with
  // the request's bounds, in the same round trip, and used when the
  // cursor's pages turn out to be these (a short chunk takes the loads
  // again).
  const bool spec = a.window <= 0 && (!SPLIT || a.chunks_per_split > 0);
  const int spec_t0 = (SPLIT ? split * a.chunks_per_split : 0) * CT;
  int spec_lb[NS], spec_pe[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    spec_lb[i] = __builtin_amdgcn_readfirstlane(
        min(max(((spec_t0 + i) * TILE + 16 * wave) >> a.ps_shift, 0), a.max_blocks - 1));
    spec_pe[i] = spec ? bt_row[spec_lb[i]] : 0;
  }
  const int q_start = ((ConstI32Ptr)a.qsl)[r];
  const int q_end = ((ConstI32Ptr)a.qsl)[r + 1];
  const int seq_len = ((ConstI32Ptr)a.seq_lens)[r];
  asm volatile("" ::"s"(q_start), "s"(q_end), "s"(seq_len));
  const int q_len = q_end - q_start;
  const int ctx = seq_len - q_len;
  const int rows_total = q_len * a.group;
  const int row0 = qt * QROWS;
  if (row0 >= rows_total) return;  // uniform
  if (a.pq_rows > 0 && rows_total >= a.pq_rows) return;  // attn_prefill_kernel's request

  const int i_min = row0 / a.group;
  const int i_max = min(rows_total - 1, row0 + QROWS - 1) / a.group;
  const int hi = a.causal ? min(seq_len, ctx + i_max + 1) : seq_len;
  const int lo = a.window > 0 ? max(0, ctx + i_min - a.window + 1) : 0;
  const int t_lo = lo / TILE;
  const int t_hi = hi > lo ? (hi + TILE - 1) / TILE : t_lo;
  const int c_lo = t_lo / CT;
  int c_hi = t_hi > t_lo ? (t_hi + CT - 1) / CT : c_lo;
  if constexpr (SPLIT) c_hi = min(c_hi, a.chunk_slots);
  const int nch = max(0, c_hi - c_lo);
  const int per = a.chunks_per_split > 0 ? a.chunks_per_split : (nch + a.num_splits - 1) / a.num_splits;
  const int my_lo = SPLIT ? c_lo + min(nch, split * per) : c_lo;
  const int my_hi = SPLIT ? min(c_lo + nch, my_lo + per) : c_lo + nch;

  const T* Qp = static_cast<const T*>(a.q);
  const int last_block = int(a.num_blocks - 1 < 0x7fffffff ? a.num_blocks - 1 : 0x7fffffff);

  // DMA of tile t (K or V) into stage buf: the wave moves key rows
  // 16 wave .. 16 wave + 15 (one page), instruction q rows 16 wave + q*KPI
  // .. +KPI-1, lane l row +l/CPR, slot l%CPR, i.e. chunk slot ^ swz(row).
  const T* Kc = static_cast<const T*>(a.k);
  const T* Vc = static_cast<const T*>(a.v);
  auto page_index = [&](int t) -> int {  // the wave's page of tile t (keys clamped)
    const int key0 = min(t * TILE + 16 * wave, seq_len - 1);
    return min(__builtin_amdgcn_readfirstlane(key0 >> a.ps_shift), a.max_blocks - 1);
  };
  auto page_entry = [&](int t) -> int { return bt_row[page_index(t)]; };
  auto dma_tile = [&](bool isv, int t, int ent, int buf) __attribute__((always_inline)) {
    const uint32_t p = uint32_t(ent < 0 ? 0 : min(ent, last_block));
#pragma unroll
    for (int q = 0; q < G::NDMA; ++q) {
      const int row0q = 16 * wave + q * G::KPI;
      const int rr = row0q + lane / G::CPR;
      const int key = min(t * TILE + rr, seq_len - 1);
      const int c = (lane % G::CPR) ^ G::swz(rr);
      const int64_t sb = isv ? a.sv_b : a.sk_b, ss = isv ? a.sv_s : a.sk_s, sh = isv ? a.sv_h : a.sk_h;
      const uint64_t off = uint64_t(p) * uint32_t(sb) + uint64_t(uint32_t(key & (a.page_size - 1))) * uint32_t(ss) +
                           uint64_t(uint32_t(g)) * uint32_t(sh) + uint32_t(c * 8);
      const T* src = (isv ? Vc : Kc) + off;
      const unsigned dst = lds0 + buf * G::TILEB + row0q * G::ROWB;
      // non-temporal (cache-policy bit nt): every K and V row is read once
      // per launch (4.30 -> 4.70 TB/s on the decode batch)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), (AttnLdsPtr)(uintptr_t)dst, 16, 0, kCpolNT);
    }
  };

  // Start-up in three round trips: the request's bounds; then the page
  // entries of the first NS steps (scalar loads issued together) alongside
  // the Q and row-setup loads; then the first NS - 1 steps' DMAs, issued
  // behind the Q loads, so that a wait for all but those DMAs covers Q and
  // the first step waits for its own tile only (one page entry per DMA and a
  // full drain before the first step used to cost two more round trips and
  // the pipeline's depth on every workgroup).
  auto live_lo = [&](int cc) { return max(cc * CT, t_lo); };
  auto live_hi = [&](int cc) { return min(cc * CT + CT, t_hi); };
  // the step after (cc, isv, t)
  auto advance = [&](int& cc, bool& isv, int& t) {
    if (++t < live_hi(cc)) return;
    if (!isv) {
      isv = true;
      t = live_lo(cc);
    } else if (cc + 1 < my_hi) {
      ++cc;
      isv = false;
      t = live_lo(cc);
    } else {
      t = live_hi(cc) - 1;  // past the end (no DMA is issued there)
    }
  };
  int dc_ = my_lo, dt = my_lo < my_hi ? live_lo(my_lo) : 0;  // DMA cursor
  bool dv = false;
  int dent = 0;  // page entry at the cursor
  // steps of this workgroup: per chunk its live K tiles, then the same V tiles
  int total_steps = 0;
  for (int c = my_lo; c < my_hi; ++c) total_steps += 2 * (live_hi(c) - live_lo(c));
  // Cursor states and page entries of steps 0 .. NS - 1. Past the last step
  // the cursor stays on it, so a workgroup with fewer than NS - 1 steps
  // issues its last tile again into stages no step reads: every workgroup
  // issues NS - 1 steps' DMAs before its first wait.
  bool pv[NS];
  int pt[NS], pe[NS];
  if (my_lo < my_hi) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      pv[i] = dv;
      pt[i] = dt;
      const int lb = page_index(dt);
      pe[i] = spec && lb == spec_lb[i] ? spec_pe[i] : bt_row[lb];
      if (i + 1 < NS) advance(dc_, dv, dt);
    }
    dent = pe[NS - 1];
  }

  // Q fragments (MFMA A operand): lane holds row lane%16, its k slots.
  // Inline-asm loads, waited for by an asm wait tied to their registers
  // after the first DMAs: loads the compiler sees before a loop that stores
  // make it drain every vector-memory operation (the DMAs too) ahead of the
  // loop. An invalid row loads token 0 (in bounds) and is zeroed after.
  u32x4 qf[QSTEPS];
  const RowInfo qrow = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + (lane & 15));
  {
    const T* qbase = Qp + qrow.token * a.sq_t + int64_t(qrow.head) * a.sq_h;
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j)
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(qf[j]) : "v"(qbase + 32 * j + 8 * kg) : "memory");
  }
  // Score-layout rows 4*kg + e as valid key ranges (empty outside the request).
  int ks[4], ke[4], qp[4], hd[4];
  float slope[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + 4 * kg + e);
    ks[e] = ri.valid ? ri.kstart : 0x7fffffff;
    ke[e] = ri.valid ? ri.kend : 0;
    qp[e] = ri.qpos;
    hd[e] = ri.head;
  }
  if (a.alibi) {
#pragma unroll
    for (int e = 0; e < 4; ++e) slope[e] = a.alibi[hd[e]];
    // waited for here, before any DMA: a load the loop uses that is still in
    // flight at its entry makes the compiler drain every DMA there
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  }

  if (my_lo < my_hi) {
    __builtin_amdgcn_sched_barrier(0);  // the Q and row-setup loads stay ahead of the DMAs
#pragma unroll
    for (int i = 0; i + 1 < NS; ++i) dma_tile(pv[i], pt[i], pe[i], i);
  }
  // Q landed: at most the NS - 1 steps' DMAs issued behind it are still in
  // flight (loads complete in issue order). A workgroup without chunks
  // issues no DMAs and never reads Q; one wait without a branch keeps the
  // compiler from copying registers of loads in flight into place for a join.
  constexpr int kPro = (NS - 1) * G::NDMA;
  static_assert(kPro < 64, "vmcnt field");
  if constexpr (QSTEPS == 4)
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]) : "n"(kPro) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(%2)" : "+v"(qf[0]), "+v"(qf[1]) : "n"(kPro) : "memory");
  if (!qrow.valid) {
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) qf[j] = u32x4{0u, 0u, 0u, 0u};
  }

  // Per-lane LDS offsets within a stage.
  // K fragment j of the lane's key (row wave*16 + lane%16), chunk 4j + kg.
  unsigned koff[QSTEPS];
  {
    const int rr = wave * 16 + (lane & 15);
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) koff[j] = rr * G::ROWB + ((((4 * j + kg) ^ G::swz(rr))) << 4);
  }
  // V B-operand reads (ds_read_b64_tr_b16): d block db = wave + 4b, keys
  // k0 + 8kg + (j>>2) (+4 for the upper half), columns db*16 + 4*(j&3).
  constexpr int NK0 = QUNIT / KI;  // MFMA k steps per quantised chain (2)
  unsigned voff[DB_PER_WAVE][NK0][2];
#pragma unroll
  for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
    for (int s = 0; s < NK0; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int db = min(wave + 4 * b, DBLK - 1);
        const int j = lane & 15;
        const int rr = s * KI + 8 * kg + (j >> 2) + 4 * h;
        const int c = 2 * db + ((j & 3) >> 1);
        voff[b][s][h] = rr * G::ROWB + ((c ^ G::swz(rr)) << 4) + (j & 1) * 8;
      }

  float Mr[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  AccT Dr[4] = {0, 0, 0, 0};
  AccT Wr[DB_PER_WAVE][4];
#pragma unroll
  for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) Wr[b][e] = 0;

  if (my_lo < my_hi) {
    // Steps: per chunk its live K tiles, then the same V tiles. Step s uses
    // stage s % NS; its DMAs were issued NS - 1 steps earlier, and each step
    // waits for them knowing how many steps' DMAs went out after them (NS - 2,
    // fewer for the last steps: nothing is issued past the last step).

    float sc[CT][4];
    float mx[4];
    AccT den[4];
    AccT wv[DB_PER_WAVE][4];
    int step = 0;
    for (int c = my_lo; c < my_hi; ++c) {
      const int ta = live_lo(c), te = live_hi(c), nt = te - ta;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        mx[e] = -__builtin_inff();
        den[e] = 0;
      }
#pragma unroll
      for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[b][e] = 0;
      auto step_begin = [&]() -> unsigned {
        // own DMAs of this step landed (only later steps' in flight: the
        // last steps have fewer after them, no DMA goes past the end), own
        // LDS writes done; the barrier makes both everyone's
        dma_wait<NS - 2, G::NDMA>(total_steps - 1 - step);
        __builtin_amdgcn_s_barrier();
        if (step + NS - 1 < total_steps) {
          dma_tile(dv, dt, dent, (step + NS - 1) & (NS - 1));
          advance(dc_, dv, dt);
          dent = page_entry(dt);  // for the next step's DMAs
        }
        const unsigned base = lds0 + (step & (NS - 1)) * G::TILEB;
        ++step;
        return base;
      };
      // K half: scores of the live tiles into registers, then the row maxima.
#pragma unroll
      for (int u = 0; u < CT; ++u) {
        if (u < nt) {
          const unsigned base = step_begin();
          u32x4 kf[QSTEPS];
#pragma unroll
          for (int j = 0; j < QSTEPS; ++j) lds_read_b128(base + koff[j], kf[j]);
          if constexpr (QSTEPS == 4) lds_wait_for(kf[0], kf[1], kf[2], kf[3]);
          else lds_wait_for(kf[0], kf[1]);
          const int t = ta + u;
          const int key = t * TILE + wave * 16 + (lane & 15);
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < QSTEPS; ++j) acc = TR::mma(qf[j], kf[j], acc);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float x = __fmul_rn(acc[e], a.scale_log2);
            if (a.softcap_log2 > 0.0f) x = a.softcap_log2 * tanh_approx(x / a.softcap_log2);
            if (a.alibi) x = x + slope[e] * static_cast<float>(key - qp[e]);
            sc[u][e] = (key >= ks[e] && key < ke[e]) ? x : -__builtin_inff();
            mx[e] = fmaxf(mx[e], sc[u][e]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[u][e] = -__builtin_inff();
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], o, 64));
        if ((lane & 15) == 0) lds_write_b32(lds0 + RF_OFF + (wave * QROWS + 4 * kg + e) * 4, __float_as_uint(mx[e]));
      }
      lds_wait();
      __builtin_amdgcn_s_barrier();
      float mc[4], m[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t v[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) lds_read_b32(lds0 + RF_OFF + (w * QROWS + 4 * kg + e) * 4, v[w]);
        lds_wait_for(v[0], v[1], v[2], v[3]);
        mc[e] = fmaxf(fmaxf(__uint_as_float(v[0]), __uint_as_float(v[1])),
                      fmaxf(__uint_as_float(v[2]), __uint_as_float(v[3])));
        m[e] = mc[e] != -__builtin_inff() ? mc[e] : 0.0f;  // no key: pin to 0
      }
      // Weights of live tile u into Ps[u & 1], denominators on the way. Tile
      // 0's go in now, tile u + 1's during V step u; the next step's barrier
      // publishes them (Ps[u & 1] was last read two V steps earlier).
      const int kin = wave * 16 + (lane & 15);
      auto write_p = [&](int u) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float w = __builtin_amdgcn_exp2f(sc[u][e] - m[e]);
          den[e] = wadd<BITS>(den[e], quant<BITS>(__fmul_rn(w, a.fxp_scale)));
          lds_write_b16(lds0 + PS_OFF + (((u & 1) * QROWS + 4 * kg + e) * VP + kin) * 2, Io<DT>::store(w));
        }
      };
      write_p(0);
      // V half: weighted V of the live tiles.
#pragma unroll
      for (int u = 0; u < CT; ++u) {
        if (u < nt) {
          const unsigned base = step_begin();
          static_assert(DB_PER_WAVE * 4 == DBLK && NK0 == 2, "every wave owns whole d blocks");
          // all of the step's LDS reads (the weights once for every d block),
          // one wait, then the MFMA chains
          u32x4 pa[NK0];
          uint64_t vlo[DB_PER_WAVE][NK0], vhi[DB_PER_WAVE][NK0];
#pragma unroll
          for (int s = 0; s < NK0; ++s)
            lds_read_b128(lds0 + PS_OFF + (((u & 1) * QROWS + (lane & 15)) * VP + s * KI + 8 * kg) * 2, pa[s]);
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b)
#pragma unroll
            for (int s = 0; s < NK0; ++s) {
              lds_read_b64_tr16(base + voff[b][s][0], vlo[b][s]);
              lds_read_b64_tr16(base + voff[b][s][1], vhi[b][s]);
            }
          if constexpr (DB_PER_WAVE == 2)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(pa[0]), "+v"(pa[1]), "+v"(vlo[0][0]), "+v"(vlo[0][1]), "+v"(vlo[1][0]),
                           "+v"(vlo[1][1]), "+v"(vhi[0][0]), "+v"(vhi[0][1]), "+v"(vhi[1][0]), "+v"(vhi[1][1])
                         :
                         : "memory");
          else
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(pa[0]), "+v"(pa[1]), "+v"(vlo[0][0]), "+v"(vlo[0][1]), "+v"(vhi[0][0]),
                           "+v"(vhi[0][1])
                         :
                         : "memory");
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NK0; ++s) {
              const u32x4 vb = {uint32_t(vlo[b][s]), uint32_t(vlo[b][s] >> 32), uint32_t(vhi[b][s]),
                                uint32_t(vhi[b][s] >> 32)};
              acc = TR::mma(pa[s], vb, acc);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[b][e] = wadd<BITS>(wv[b][e], quant<BITS>(__fmul_rn(acc[e], a.fxp_scale)));
          }
          if (u + 1 < nt) write_p(u + 1);
        }
      }
      // The chunk's denominators: 16 key lanes, then the 4 waves.
      AccT dc[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) den[e] = wadd<BITS>(den[e], __shfl_xor(den[e], o, 64));
      }
      if ((lane & 15) == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned ad = lds0 + RI_OFF + (wave * QROWS + 4 * kg + e) * 8;
          const uint64_t v = static_cast<uint64_t>(static_cast<int64_t>(den[e]));
          lds_write_b32(ad, uint32_t(v));
          lds_write_b32(ad + 4, uint32_t(v >> 32));
        }
      }
      lds_wait();
      __builtin_amdgcn_s_barrier();
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        AccT sum = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t lo32, hi32;
          const unsigned ad = lds0 + RI_OFF + (w * QROWS + 4 * kg + e) * 8;
          lds_read_b32(ad, lo32);
          lds_read_b32(ad + 4, hi32);
          lds_wait_for(lo32, hi32);
          const int64_t v = static_cast<int64_t>((uint64_t(hi32) << 32) | lo32);
          sum = wadd<BITS>(sum, v);
        }
        dc[e] = sum;
      }

      if constexpr (SPLIT) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + 4 * kg + e);
          if (!ri.valid) continue;
          const int64_t slot = (ri.token * a.num_heads + ri.head) * a.chunk_slots + c;
          if ((lane & 15) == 0 && wave == 0) {
            a.pmax[slot] = mc[e];
            static_cast<AccT*>(a.den_ws)[slot] = dc[e];
          }
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b) {
            const int d = (wave + 4 * b) * 16 + (lane & 15);
            if (wave + 4 * b < DBLK) static_cast<AccT*>(a.wv_ws)[slot * a.head_dim + d] = wv[b][e];
          }
        }
        // No drain here. The stores count in vmcnt and may complete out of
        // order with the loads, but the loads (DMAs included) complete in
        // issue order. While a step's DMA is outstanding, so are the DMAs of
        // every later step, so "at most L outstanding" with L the later
        // steps' DMA count still implies the step's DMA landed; stores in
        // flight only make the wait stricter. A drain here emptied the ring
        // at every chunk boundary.
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (mc[e] == -__builtin_inff()) continue;
          float Mn, fa, fb;
          merge_factors(Mr[e], mc[e], Mn, fa, fb);
          Dr[e] = wadd<BITS>(rescale<BITS>(Dr[e], fa), rescale<BITS>(dc[e], fb));
#pragma unroll
          for (int b = 0; b < DB_PER_WAVE; ++b)
            Wr[b][e] = wadd<BITS>(rescale<BITS>(Wr[b][e], fa), rescale<BITS>(wv[b][e], fb));
          Mr[e] = Mn;
        }
      }
    }
    // No wait here: the last step waited for every DMA (none is issued after
    // it, and a wave's loads complete in issue order), so no DMA can land in
    // the LDS after the workgroup has given it up. Its partial stores need no
    // wait before the wave ends (waiting for them held each workgroup's CU
    // slot for their write latency).
  }

  if (SPLIT && split == 0 && tid < QROWS) {
    const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + tid);
    if (ri.valid) {
      int* cr = a.crange + 2 * (ri.token * a.num_heads + ri.head);
      cr[0] = c_lo;
      cr[1] = c_lo + nch;
    }
  }

  if constexpr (!SPLIT) {
    float den_f[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) den_f[e] = fmaxf(acc_f32<BITS>(Dr[e], a.fxp_inv), 1.0e-6f);
    T* Op = static_cast<T*>(a.o);
#pragma unroll
    for (int b = 0; b < DB_PER_WAVE; ++b) {
      const int d = (wave + 4 * b) * 16 + (lane & 15);
      if (wave + 4 * b >= DBLK) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, row0 + 4 * kg + e);
        if (!ri.valid) continue;
        Op[ri.token * a.so_t + int64_t(ri.head) * a.so_h + d] =
            Io<DT>::store(div_rn(acc_f32<BITS>(Wr[b][e], a.fxp_inv), den_f[e]));
      }
    }
  }
}

template <int DMAX> constexpr size_t dma_lds_bytes() {
  return size_t(DmaGeom<DMAX>::NS) * DmaGeom<DMAX>::TILEB + size_t(2) * QROWS * (TILE + 8) * 2 + 4 * QROWS * 4 +
         4 * QROWS * 8;
}

// Prefill-shaped launches (16-bit inputs, one split): 64 query rows per
// workgroup, each of its four waves owning 16 of them, so a key tile staged
// in LDS serves four times the rows of attn_kernel's 16-row tile. Two
// workgroups share a CU, so the two waves of a SIMD belong to different
// workgroups and do not wait on the same barriers (one 8-wave workgroup of
// 128 rows per CU measured 5 % slower). A chunk's scores are not
// kept: its K tiles are read twice, once for the chunk's row maxima and again
// (with the V tiles) for the weights. Every row gets attn_kernel's bits: the
// same MFMA chains per score and per weighted-V element (rows of one MFMA are
// independent), the same chunk statistics (keys a row cannot see contribute
// exact zeros, so the workgroup's wider key range changes nothing) and the
// same fold.
constexpr int PQ_WAVES = 4;
// Requests with at least this many rows (query tokens x GQA group) use the
// prefill workgroups: from three 16-row tiles on, reading each key tile
// three times (K twice, V once) per 64 rows costs less than twice per 16.
constexpr int kPrefillRows = 48;
constexpr int PQROWS = 16 * PQ_WAVES;
constexpr int kPThreads = 64 * PQ_WAVES;

template <int DT, int BITS, int DMAX>
__global__ __launch_bounds__(kPThreads, 2) void attn_prefill_kernel(AttnArgs a) {
  static_assert(DT != FXPR_DTYPE_F32, "16-bit inputs only");
  using TR = Traits<DT>;
  using T = typename TR::T;
  using AccT = typename AccOf<BITS>::T;
  constexpr int KI = TR::KI, CH = TR::CH, QUNIT = TR::QUNIT;
  constexpr int QSTEPS = DMAX / KI;
  constexpr int DBLK = DMAX / 16;
  constexpr int VP = TILE + 8;
  constexpr int VNP = DMAX + 16;
  constexpr int VCH = DMAX / CH;
  constexpr int VITER = TILE * VCH / kPThreads;
  constexpr int KCPR = DMAX / CH;
  // K tile [key][d], 16-byte chunk c of key row r at slot c ^ kswz(r): a
  // fragment read (16 consecutive rows, one chunk each) hits distinct banks.
  __shared__ __align__(16) T Kt[2][TILE * DMAX];
  __shared__ __align__(16) T Vt[2][TILE * VNP];
  __shared__ __align__(16) T Ps[PQ_WAVES][16 * VP];  // each wave's weights, [row][key]
  auto kswz = [](int r) -> int {
    if constexpr (KCPR >= 16) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (r >> 1) & 7;
  };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, kg = lane >> 4;
  const int r = blockIdx.x / a.num_kv_heads, g = blockIdx.x % a.num_kv_heads;
  const int q_start = a.qsl[r];
  const int q_len = a.qsl[r + 1] - q_start;
  const int seq_len = a.seq_lens[r];
  const int ctx = seq_len - q_len;
  const int rows_total = q_len * a.group;
  const int row0 = int(gridDim.y - 1 - blockIdx.y) * PQROWS;  // last row tiles first
  if (row0 >= rows_total || rows_total < a.pq_rows) return;  // uniform; short requests: attn_kernel
  const int wrow0 = row0 + 16 * wave;

  const int i_min = row0 / a.group;
  const int i_max = min(rows_total - 1, row0 + PQROWS - 1) / a.group;
  const int hi = a.causal ? min(seq_len, ctx + i_max + 1) : seq_len;
  const int lo = a.window > 0 ? max(0, ctx + i_min - a.window + 1) : 0;
  const int t_lo = lo / TILE;
  const int t_hi = hi > lo ? (hi + TILE - 1) / TILE : t_lo;
  const int c_lo = t_lo / CT;
  const int c_hi = t_hi > t_lo ? (t_hi + CT - 1) / CT : c_lo;

  const int32_t* bt_row = a.bt + int64_t(r) * a.sbt;
  const T* Kc = static_cast<const T*>(a.k);
  const T* Vc = static_cast<const T*>(a.v);
  const T* Qp = static_cast<const T*>(a.q);
  auto clamp_key = [&](int key) { return max(0, min(key, seq_len - 1)); };
  auto bt_entry = [&](int key) -> int {
    const int lb = a.ps_shift >= 0 ? (key >> a.ps_shift) : key / a.page_size;
    return bt_row[min(lb, a.max_blocks - 1)];
  };
  const int last_block = int(a.num_blocks - 1 < 0x7fffffff ? a.num_blocks - 1 : 0x7fffffff);
  auto row_addr = [&](int key, int entry, int64_t sb, int64_t ss, int64_t sh) -> uint64_t {
    const uint32_t p = uint32_t(entry < 0 ? 0 : min(entry, last_block));
    const uint32_t slot = uint32_t(a.ps_shift >= 0 ? (key & (a.page_size - 1)) : key % a.page_size);
    return uint64_t(p) * uint32_t(sb) + uint64_t(slot) * uint32_t(ss) + uint64_t(uint32_t(g)) * uint32_t(sh);
  };

  // Q fragments of the wave's rows (MFMA A operand: row lane%16, k slots kg).
  u32x4 qf[QSTEPS];
  {
    const RowInfo qrow = row_info(a, g, q_start, q_len, ctx, seq_len, wrow0 + (lane & 15));
    const T* qbase = Qp + qrow.token * a.sq_t + int64_t(qrow.head) * a.sq_h;
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) {
      const int d = 32 * j + 8 * kg;
      qf[j] = (qrow.valid && d < a.head_dim) ? *reinterpret_cast<const u32x4*>(qbase + d) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  // Rows of the score / PV layout: the wave's rows 4*kg + e, as their valid
  // key ranges (empty for rows outside the request) and query positions.
  int ks[4], ke[4], qp[4];
  float slope[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, wrow0 + 4 * kg + e);
    ks[e] = ri.valid ? ri.kstart : 0x7fffffff;
    ke[e] = ri.valid ? ri.kend : 0;
    qp[e] = ri.qpos;
    slope[e] = a.alibi ? a.alibi[ri.head] : 0.0f;
  }

  // Whole key rows per instruction: chunk c = i*256 + tid of a tile is key
  // c / VCH, d chunk c % VCH. Loads are unconditional (keys clamped).
  // K and V rows of one key share its page entry: entries first, then loads.
  auto tile_entries = [&](int t, int (&ve)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i) ve[i] = bt_entry(clamp_key(t * TILE + (i * kPThreads + tid) / VCH));
  };
  auto tile_load = [&](const T* base, int64_t sb, int64_t ss, int64_t sh, int t, const int (&ve)[VITER],
                       u32x4 (&vr)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i) {
      const int c = i * kPThreads + tid;
      const int key = clamp_key(t * TILE + c / VCH), d0 = (c % VCH) * CH;
      vr[i] = *reinterpret_cast<const u32x4*>(base + row_addr(key, ve[i], sb, ss, sh) + (d0 < a.head_dim ? d0 : 0));
    }
  };
  auto k_store = [&](int buf, const u32x4 (&vr)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i) {
      const int c = i * kPThreads + tid;
      const int rr = c / VCH, cc = c % VCH;
      *reinterpret_cast<u32x4*>(&Kt[buf][rr * DMAX + (cc ^ kswz(rr)) * CH]) = vr[i];
    }
  };
  auto v_store = [&](int buf, const u32x4 (&vr)[VITER]) {
#pragma unroll
    for (int i = 0; i < VITER; ++i) {
      const int c = i * kPThreads + tid;
      *reinterpret_cast<u32x4*>(&Vt[buf][(c / VCH) * VNP + (c % VCH) * CH]) = vr[i];
    }
  };
  // Scores of key block kb (16 keys) of tile t for the lane's rows.
  auto block_scores = [&](int buf, int t, int kb, float (&s)[4]) {
    const int rr = kb * 16 + (lane & 15);
    const T* row = &Kt[buf][rr * DMAX];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j)
      acc = TR::mma(qf[j], *reinterpret_cast<const u32x4*>(row + ((4 * j + kg) ^ kswz(rr)) * CH), acc);
    const int key = t * TILE + rr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = __fmul_rn(acc[e], a.scale_log2);
      if (a.softcap_log2 > 0.0f) x = a.softcap_log2 * tanh_approx(x / a.softcap_log2);
      if (a.alibi) x = x + slope[e] * static_cast<float>(key - qp[e]);
      s[e] = (key >= ks[e] && key < ke[e]) ? x : -__builtin_inff();
    }
  };

  float mx[4], m[4];
  AccT den[4];
  AccT wv[DBLK][4];
  float Mr[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  AccT Dr[4] = {0, 0, 0, 0};
  AccT Wr[DBLK][4];
#pragma unroll
  for (int b = 0; b < DBLK; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) Wr[b][e] = 0;
  auto reset = [&]() {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      mx[e] = -__builtin_inff();
      den[e] = 0;
    }
#pragma unroll
    for (int b = 0; b < DBLK; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) wv[b][e] = 0;
  };

  // Steps: per chunk, phase A over its live tiles (K), then phase B over the
  // same tiles (K and V). Each step's tiles were loaded into registers during
  // the previous step; they are written to an LDS buffer (alternating), then
  // the next step's loads are issued and one barrier separates the writes
  // from the reads (a buffer is rewritten two steps after it was read).
  if (c_lo < c_hi) {
    u32x4 kr[VITER], vr[VITER];
    int c = c_lo, phase = 0, t = max(c * CT, t_lo);
    int ve[VITER];
    auto live_hi = [&](int cc) { return min(cc * CT + CT, t_hi); };
    tile_entries(t, ve);
    tile_load(Kc, a.sk_b, a.sk_s, a.sk_h, t, ve, kr);
    reset();
    int buf = 0;
    for (;;) {
      const int te = live_hi(c);
      k_store(buf, kr);
      if (phase == 1) v_store(buf, vr);
      // the next step
      int nc = c, nphase = phase, nt = t + 1;
      if (nt >= te) {
        if (phase == 0) {
          nphase = 1;
          nt = max(c * CT, t_lo);
        } else {
          nc = c + 1;
          nphase = 0;
          nt = max(nc * CT, t_lo);
        }
      }
      const bool more = nc < c_hi;
      if (more) {
        tile_entries(nt, ve);
        tile_load(Kc, a.sk_b, a.sk_s, a.sk_h, nt, ve, kr);
        if (nphase == 1) tile_load(Vc, a.sv_b, a.sv_s, a.sv_h, nt, ve, vr);
      }
      __syncthreads();

      if (phase == 0) {
#pragma unroll
        for (int kb = 0; kb < TILE / 16; ++kb) {
          float s[4];
          block_scores(buf, t, kb, s);
#pragma unroll
          for (int e = 0; e < 4; ++e) mx[e] = fmaxf(mx[e], s[e]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (nphase == 1 && nc == c) {  // the chunk's row maxima over its 16 key lanes
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) mx[e] = fmaxf(mx[e], __shfl_xor(mx[e], o, 64));
            m[e] = mx[e] != -__builtin_inff() ? mx[e] : 0.0f;  // no key: pin to 0
          }
        }
      } else {
        T* Pw = Ps[wave];
#pragma unroll
        for (int kb = 0; kb < TILE / 16; ++kb) {
          float s[4];
          block_scores(buf, t, kb, s);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float w = __builtin_amdgcn_exp2f(s[e] - m[e]);
            den[e] = wadd<BITS>(den[e], quant<BITS>(__fmul_rn(w, a.fxp_scale)));
            Pw[(4 * kg + e) * VP + kb * 16 + (lane & 15)] = Io<DT>::store(w);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        // Pw is the wave's own: its writes complete before its reads.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const T* Vb = Vt[buf];
#pragma unroll
        for (int db = 0; db < DBLK; ++db) {
#pragma unroll
          for (int u0 = 0; u0 < TILE; u0 += QUNIT) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < QUNIT; k0 += KI) {
              const int key = u0 + k0 + 8 * kg;
              const int j = lane & 15;
              typedef short v4s __attribute__((ext_vector_type(4)));
              const T* src = &Vb[(key + (j >> 2)) * VNP + db * 16 + 4 * (j & 3)];
              const v4s lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(src));
              const v4s hi4 =
                  __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(src + 4 * VNP));
              struct {
                v4s a, b;
              } both = {lo4, hi4};
              acc = TR::mma(*reinterpret_cast<const u32x4*>(&Pw[(lane & 15) * VP + key]),
                            __builtin_bit_cast(u32x4, both), acc);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[db][e] = wadd<BITS>(wv[db][e], quant<BITS>(__fmul_rn(acc[e], a.fxp_scale)));
          }
          // one d block at a time: keeps the scheduler from hoisting every
          // block's LDS reads (and their registers) to the top
          __builtin_amdgcn_sched_barrier(0);
        }
        if (nc != c) {  // end of the chunk: its denominators, then the fold
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) den[e] = wadd<BITS>(den[e], __shfl_xor(den[e], o, 64));
            if (mx[e] == -__builtin_inff()) continue;  // no key of the row in this chunk
            float Mn, fa, fb;
            merge_factors(Mr[e], mx[e], Mn, fa, fb);
            Dr[e] = wadd<BITS>(rescale<BITS>(Dr[e], fa), rescale<BITS>(den[e], fb));
#pragma unroll
            for (int b = 0; b < DBLK; ++b) Wr[b][e] = wadd<BITS>(rescale<BITS>(Wr[b][e], fa), rescale<BITS>(wv[b][e], fb));
            Mr[e] = Mn;
          }
          reset();
        }
      }
      if (!more) break;
      c = nc;
      phase = nphase;
      t = nt;
      buf ^= 1;
    }
  }

  float den_f[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) den_f[e] = fmaxf(acc_f32<BITS>(Dr[e], a.fxp_inv), 1.0e-6f);
  T* Op = static_cast<T*>(a.o);
#pragma unroll
  for (int b = 0; b < DBLK; ++b) {
    const int d = b * 16 + (lane & 15);
    if (d >= a.head_dim) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const RowInfo ri = row_info(a, g, q_start, q_len, ctx, seq_len, wrow0 + 4 * kg + e);
      if (!ri.valid) continue;
      Op[ri.token * a.so_t + int64_t(ri.head) * a.so_h + d] =
          Io<DT>::store(div_rn(acc_f32<BITS>(Wr[b][e], a.fxp_inv), den_f[e]));
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill workgroups fed by LDS DMA (16-bit inputs, rows exactly DMAX wide,
// pages of 16 keys or more): attn_prefill_kernel's rows, chunk statistics and
// bits, with the tiles brought into an NS-stage LDS ring by global_load_lds
// NS - 1 steps ahead (one scalar page-entry load per wave and tile) instead
// of register-staged loads one step ahead. A tile occupies one stage (its
// 64 key rows, 16-byte chunk c of row r at slot c ^ swz(r), as in
// attn_dma_kernel). Steps per chunk: its live K tiles (row maxima), then per
// live tile its K tile (weights, denominators, the wave's P) and its V tile
// (weighted V); one tile and one barrier per step. All LDS accesses of the
// loop are inline asm with explicit waits (the compiler would otherwise wait
// for every DMA in flight before each of them).
template <int DMAX> struct PDmaGeom {
  static constexpr int ROWB = DMAX * 2;              // bytes per key row
  static constexpr int CPR = ROWB / 16;              // 16-byte chunks per row
  static constexpr int KPI = 1024 / ROWB;            // key rows per wave instruction
  static constexpr int TILEB = TILE * ROWB;          // bytes per tile
  static constexpr int RPW = TILE / PQ_WAVES;        // key rows each wave moves per tile
  static constexpr int NDMA = RPW / KPI;             // DMA instructions per wave per tile
  static constexpr int NS = 4;                       // LDS stages (two workgroups per CU)
  static_assert(NDMA >= 1 && NDMA * KPI == RPW, "tile rows per wave");
  static_assert((NS & (NS - 1)) == 0, "stage index by mask");
  // K tiles: the transposed score MFMAs read rows {0-3, 8-11, 16-19, 24-27}
  // (and the same + 4) of a 32-row group in one 16-lane read. Measured with
  // gfx950's LDS conflict counter on that exact pattern: 256-byte rows keep
  // the V swizzle (conflict-free; the alternatives tried were 2-way),
  // 128-byte rows take row bits 1, 3 and 4 (the V swizzle there is 2-way).
  static __device__ __forceinline__ int kswz(int r) {
    if constexpr (CPR >= 16) return DmaGeom<DMAX>::swz(r);
    else return ((r >> 1) & 1) | (((r >> 3) & 3) << 1);
  }
};

template <int DMAX> constexpr size_t prefill_dma_lds_bytes() {
  return size_t(PDmaGeom<DMAX>::NS) * PDmaGeom<DMAX>::TILEB;
}

__device__ __forceinline__ void lds_write_b16_hi(unsigned addr, uint32_t x) {
  asm volatile("ds_write_b16_d16_hi %0, %1" ::"v"(addr), "v"(x) : "memory");
}
// Two weights as 16-bit values (RNE) in one register, low half first; NaN
// payloads as the conversion leaves them.
template <int DT> __device__ __forceinline__ uint32_t p_pack2(float lo, float hi) {
  if constexpr (DT == FXPR_DTYPE_BF16) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Wait until at most N LDS operations are outstanding (they complete in
// issue order, so the older ones, whose registers are bound here, are done).
template <int N, class A, class B> __device__ __forceinline__ void lds_waitn_for(A& a, B& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N) : "memory");
}
template <int N, class A, class B, class C, class D>
__device__ __forceinline__ void lds_waitn_for(A& a, B& b, C& c, D& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "n"(N) : "memory");
}

// max(m, |x0|, |x1|, |x2|, |x3|), NaN-propagating
__device__ __forceinline__ float absmax4(float m, const f32x4& x) {
  return __builtin_elementwise_maximum(
      m, __builtin_elementwise_maximum(__builtin_elementwise_maximum(__builtin_fabsf(x[0]), __builtin_fabsf(x[1])),
                                       __builtin_elementwise_maximum(__builtin_fabsf(x[2]), __builtin_fabsf(x[3]))));
}
// 16 bytes per lane from a raw buffer at voff into LDS at dst + 16 * lane
// (a helper: called directly in a kernel template, the builtin makes the
// host pass drop the kernel's launch stub).
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, unsigned dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (AttnLdsPtr)(uintptr_t)dst, 16, voff, 0, 0, 0);
}
// The same with a scalar offset and an instruction offset OFF, which the
// hardware adds to both the source address (base + voff + soff + OFF) and the
// LDS destination (dst + OFF + 16 * lane): consecutive loads into one stage
// share M0.
template <int OFF>
__device__ __forceinline__ void buffer_to_lds16_off(__amdgpu_buffer_rsrc_t r, unsigned dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (AttnLdsPtr)(uintptr_t)dst, 16, voff, soff, OFF, 0);
}
template <int OFF> __device__ __forceinline__ void lds_read_b64_tr16_off(unsigned addr, uint64_t& x) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(x) : "v"(addr), "n"(OFF) : "memory");
}
template <int OFF> __device__ __forceinline__ void lds_read_b128_off(unsigned addr, u32x4& x) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(x) : "v"(addr), "n"(OFF) : "memory");
}

template <int DT, int BITS, int DMAX>
__global__ __launch_bounds__(kPThreads, 2) void attn_prefill_dma_kernel(AttnArgs a) {
  static_assert(DT != FXPR_DTYPE_F32, "16-bit inputs only");
  using TR = Traits<DT>;
  using T = typename TR::T;
  using AccT = typename AccOf<BITS>::T;
  using G = PDmaGeom<DMAX>;
  using SW = DmaGeom<DMAX>;  // the row swizzle
  constexpr int KI = TR::KI, QUNIT = TR::QUNIT;
  constexpr int QSTEPS = DMAX / KI;
  constexpr int DBLK = DMAX / 16;
  constexpr int NK0 = QUNIT / KI;  // MFMA k steps per quantised chain
  constexpr int NS = G::NS;
  static_assert(TILE == QUNIT, "one quantised chain per tile");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  // The dynamic LDS starts where the static LDS ends, rounded up to its
  // alignment: a constant (the address of smem_raw, cast from a generic
  // pointer, comes back as a null test and a select at every use)
  const unsigned lds0 = (__builtin_amdgcn_groupstaticsize() + 15u) & ~15u;

  const int tid = threadIdx.x, lane = tid & 63, kg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x / a.num_kv_heads, g = blockIdx.x % a.num_kv_heads;
  const int q_start = a.qsl[r];
  const int q_len = a.qsl[r + 1] - q_start;
  const int seq_len = a.seq_lens[r];
  const int ctx = seq_len - q_len;
  const int rows_total = q_len * a.group;
  // Row tiles last to first: under causal masking the later rows attend the
  // most keys, so the longest workgroups start first and the short ones fill
  // the tail (B = 4 x 2048 tokens: -6 %, one 8192-token prompt: -9 %).
  const int row0 = int(gridDim.y - 1 - blockIdx.y) * PQROWS;
  if (row0 >= rows_total || rows_total < a.pq_rows) return;  // uniform; short requests: the 16-row kernels
  const int wrow0 = row0 + 16 * wave;

  const int i_min = row0 / a.group;
  const int i_max = min(rows_total - 1, row0 + PQROWS - 1) / a.group;
  const int hi = a.causal ? min(seq_len, ctx + i_max + 1) : seq_len;
  const int lo = a.window > 0 ? max(0, ctx + i_min - a.window + 1) : 0;
  const int t_lo = lo / TILE;
  const int t_hi = hi > lo ? (hi + TILE - 1) / TILE : t_lo;
  const int c_lo = t_lo / CT;
  const int c_hi = t_hi > t_lo ? (t_hi + CT - 1) / CT : c_lo;

  const ConstI32Ptr bt_row = (ConstI32Ptr)(a.bt + int64_t(r) * a.sbt);
  const int last_block = int(a.num_blocks - 1 < 0x7fffffff ? a.num_blocks - 1 : 0x7fffffff);
  const T* Kc = static_cast<const T*>(a.k);
  const T* Vc = static_cast<const T*>(a.v);
  // The wave moves key rows RPW wave .. RPW wave + RPW - 1 of a tile (within
  // one page: pages hold 16 keys or more); instruction q rows RPW wave +
  // q KPI .., lane l row + l / CPR, chunk slot l % CPR, i.e. chunk
  // (l % CPR) ^ swz(row). Keys past the sequence are clamped (their scores
  // are masked).
  auto page_entry = [&](int t) -> int {
    const int key0 = min(t * TILE + G::RPW * wave, seq_len - 1);
    const int lb = __builtin_amdgcn_readfirstlane(key0 >> a.ps_shift);
    // (an unsigned index: a 32-bit scalar offset of the load, no 64-bit
    // address arithmetic; key0 >= 0, as the kernel visits tiles only when
    // seq_len >= 1)
    return bt_row[uint32_t(min(lb, a.max_blocks - 1))];
  };
  // K and V tiles are separate compile-time instances behind a uniform
  // branch on isv (a select between the two matrices' fields becomes a load
  // through a selected address, which keeps the captured values in scratch
  // memory, reloaded at every DMA; those reloads' vmcnt waits drain the ring).
  // Per-lane byte offsets of the DMA sources, fixed for the kernel: row
  // q KPI + lane / CPR of the wave's 16 key rows of a tile, chunk slot
  // (lane % CPR) ^ the K or V swizzle of its tile row. The wave's 16 rows lie
  // in one page (pages hold 16 keys or more, the rows start 16-aligned), so
  // a whole tile's sources are a uniform base (page, head, the wave's first
  // row) plus these offsets; the last, partial tile of a request clamps its
  // keys per lane instead. (The host keeps 16 key strides below 2^26 bytes.)
  // Instruction q's LDS rows start q KPI ROWB = q KiB past the wave's first
  // row: that goes in the instruction offset, which the source address takes
  // too, so it is taken out of the lane offset here (q KPI key strides are
  // at least q KiB).
  uint32_t dma_ok[G::NDMA], dma_ov[G::NDMA];
#pragma unroll
  for (int q = 0; q < G::NDMA; ++q) {
    const int lr = q * G::KPI + lane / G::CPR, rr = G::RPW * wave + lr;
    dma_ok[q] = (uint32_t(lr) * uint32_t(a.sk_s) + uint32_t(((lane % G::CPR) ^ G::kswz(rr)) * 8)) * uint32_t(sizeof(T)) -
                uint32_t(q * G::KPI * G::ROWB);
    dma_ov[q] = (uint32_t(lr) * uint32_t(a.sv_s) + uint32_t(((lane % G::CPR) ^ SW::swz(rr)) * 8)) * uint32_t(sizeof(T)) -
                uint32_t(q * G::KPI * G::ROWB);
  }
  // the page of a block-table entry (clamped into the cache). (Through the
  // asm, nothing computed from the entry is hoisted to its load a step
  // earlier, which would wait for the load there.)
  auto page_of = [&](int ent) -> uint32_t {
    asm volatile("" : "+s"(ent));
    return uint32_t(ent < 0 ? 0 : min(ent, last_block));
  };
  auto dma_mat = [&](auto isv_tag, int t, uint32_t p, int buf) __attribute__((always_inline)) {
    constexpr bool ISV = decltype(isv_tag)::value;
    const uint32_t ss = uint32_t(ISV ? a.sv_s : a.sk_s);
    // the page's (and head's) first element, uniform
    const T* base = (ISV ? Vc : Kc) + (uint64_t(p) * uint32_t(ISV ? a.sv_b : a.sk_b) +
                                       uint64_t(uint32_t(g)) * uint32_t(ISV ? a.sv_h : a.sk_h));
    const unsigned dst0 = lds0 + buf * G::TILEB + G::RPW * wave * G::ROWB;
    // (temporal: a workgroup reads each K tile twice and neighbouring row
    // blocks share tiles through L2; nt measured 5 % slower)
    if (t * TILE + TILE <= seq_len) {  // uniform: a whole tile  // uniform: a whole tile
      const int key0 = t * TILE + G::RPW * wave;
      // a buffer based at the page's first row, the wave's first row in the
      // scalar offset (the host keeps a page's bytes below 2^31): 32-bit
      // lane offsets, no per-lane address math
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(base), short(0), -1, kBufferDword3);
      const uint32_t soff = uint32_t(key0 & (a.page_size - 1)) * ss * uint32_t(sizeof(T));
      static_for<G::NDMA>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        buffer_to_lds16_off<q * G::KPI * G::ROWB>(rs, dst0, ISV ? dma_ov[q] : dma_ok[q], soff);
      });
    } else {
      // (the lane through an asm: per-lane values derived here stay here, not
      // hoisted out of the loop to hold registers for the whole kernel)
      int ln;
      asm volatile("v_mov_b32 %0, %1" : "=v"(ln) : "v"(lane));
#pragma unroll
      for (int q = 0; q < G::NDMA; ++q) {
        const int rr = G::RPW * wave + q * G::KPI + ln / G::CPR;
        const int key = min(t * TILE + rr, seq_len - 1);
        const uint32_t c = uint32_t(((ln % G::CPR) ^ (ISV ? SW::swz(rr) : G::kswz(rr))) * 8);
        const T* src = base + (uint64_t(uint32_t(key & (a.page_size - 1))) * ss + c);
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src), (AttnLdsPtr)(uintptr_t)(dst0 + q * G::KPI * G::ROWB),
                                         16, 0, 0);
      }
    }
  };
  auto dma_tile = [&](bool isv, int t, int ent, int buf) __attribute__((always_inline)) {
    if (isv)
      dma_mat(std::true_type{}, t, page_of(ent), buf);
    else
      dma_mat(std::false_type{}, t, page_of(ent), buf);
  };

  // The tile stream: per chunk cc, its nt live K tiles (phase 0), then K and
  // V of each live tile in turn (phase 1, 2 nt entries). The DMA cursor runs
  // NS - 1 entries ahead; past the end it re-issues the last entry into the
  // free stage, so every step issues the same DMAs and the wait count stays
  // exact. The first entries go out before the Q and row-setup loads.
  auto live_lo = [&](int cc) { return max(cc * CT, t_lo); };
  auto live_hi = [&](int cc) { return min(cc * CT + CT, t_hi); };
  // DMA cursor: chunk dcc (first live tile dlo), phase dph (0 or 1), entry
  // didx of dlim in the phase; only a phase or chunk change recomputes the
  // bounds (the common advance is an add and a compare)
  int dcc = c_lo, dph = 0, didx = 0;
  int dlo = live_lo(c_lo), dlim = live_hi(c_lo) - dlo;
  auto cur_tile = [&]() { return dlo + (didx >> dph); };
  auto cur_isv = [&]() { return (dph & didx & 1) != 0; };
  auto advance = [&]() {
    if (++didx < dlim) return;
    const int nt = live_hi(dcc) - dlo;
    if (dph == 0) {
      dph = 1;
      didx = 0;
      dlim = 2 * nt;
    } else if (dcc + 1 < c_hi) {
      ++dcc;
      dph = 0;
      didx = 0;
      dlo = live_lo(dcc);
      dlim = live_hi(dcc) - dlo;
    } else {
      didx = 2 * nt - 1;
    }
  };
  // The page entry of the cursor's tile, loaded when the cursor moves to
  // another tile: a tile's V entry follows its K entry in phase 1 and reuses
  // it (a reload there would be waited for by the very next DMA).
  int dent = 0, dent_t = -1;
  auto refresh_entry = [&]() {
    const int t = cur_tile();
    if (t != dent_t) {
      dent = page_entry(t);
      dent_t = t;
    }
  };
  if (c_lo < c_hi) {
    refresh_entry();
#pragma unroll
    for (int i = 0; i + 2 < NS; ++i) {
      dma_tile(cur_isv(), cur_tile(), dent, i);
      advance();
      refresh_entry();
    }
  }

  // The lane's query row. Scores and weighted V are computed transposed:
  // MFMA (s, h) of a tile (s: 32-key step, h: half) takes the key rows
  // pi(i) = 32 s + 8 (i / 4) + 4 h + i % 4 (i = lane % 16) of the K tile as
  // its A operand and the wave's Q rows as its B operand, so lane (kg, row
  // lane % 16) receives the scores of keys 32 s + 8 kg + 4 h + e, e = 0..3;
  // with h = 0, 1 these are the eight consecutive keys 32 s + 8 kg .. + 7 that
  // the weighted-V MFMA (V^T as A operand, P^T as B operand) needs in that
  // lane's B operand, so the weights never leave registers, and every
  // statistic of a row (maximum, denominator, fold) lives in the row's four
  // lanes. The MFMA is bitwise symmetric in its operands and each score and
  // weighted-V element is the same products in the same k order as in the
  // untransposed layout, so every bit is attn_dma_kernel's.
  const RowInfo me = row_info(a, g, q_start, q_len, ctx, seq_len, wrow0 + (lane & 15));
  u32x4 qf[QSTEPS];
  {
    const T* qbase = static_cast<const T*>(a.q) + me.token * a.sq_t + int64_t(me.head) * a.sq_h;
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) {
      const int d = 32 * j + 8 * kg;
      qf[j] = me.valid ? *reinterpret_cast<const u32x4*>(qbase + d) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const int ks = me.valid ? me.kstart : 0x7fffffff;
  const int ke = me.valid ? me.kend : 0;
  const int qp = me.qpos;
  const float slope = a.alibi ? a.alibi[me.head] : 0.0f;
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): Q, row setup and the first DMAs

  // Per-lane LDS offsets within a stage. K A-operand rows pi(i) for h = 0, 1
  // (the step s adds 32 rows, which the K swizzle ignores): chunk 4 j + kg at
  // slot (4 j + kg) ^ kswz(row). V A-operand reads (ds_read_b64_tr_b16) of d
  // block db: keys s*KI + 8kg + (j>>2) (+4 for the upper half), columns
  // db*16 + 4*(j&3), j = lane%16: chunk 2 db + b of row rr sits at slot
  // (2 db + b) ^ swz(rr) = 2 db ^ (b ^ swz(rr)), i.e. at the d block 0 offset
  // XOR db << 5 (bits 5.. of the chunk part; the row and half-chunk parts lie
  // outside them).
  unsigned koff[2][QSTEPS];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int j = 0; j < QSTEPS; ++j) {
      const int i = lane & 15;
      const int rr = 8 * (i >> 2) + 4 * h + (i & 3);
      koff[h][j] = rr * G::ROWB + (((4 * j + kg) ^ G::kswz(rr)) << 4);
    }
  unsigned voff0[NK0][2];
#pragma unroll
  for (int s = 0; s < NK0; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = lane & 15;
      const int rr = s * KI + 8 * kg + (j >> 2) + 4 * h;
      voff0[s][h] = rr * G::ROWB + ((((j & 3) >> 1) ^ SW::swz(rr)) << 4) + (j & 1) * 8;
    }

  float Mr = -__builtin_inff();
  AccT Dr = 0;
  AccT Wr[DBLK][4];
#pragma unroll
  for (int b = 0; b < DBLK; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) Wr[b][e] = 0;

  // Fast variant (same bits): no softcap or ALiBi and a positive scale, so a
  // score is fl(acc * scale) and the chunk maximum is fl(max(acc) * scale)
  // (rounding is monotone); tiles every row of the wave sees whole skip the
  // mask; a weight w in [0, 1] quantises by the rounding constant (2^f within
  // its range, see fast_den); P is packed without the canonical-NaN rule (any
  // NaN weight yields a NaN weighted V either way, which quantises to 0).
  const bool fast_den = BITS != 64 && a.fxp_scale <= (BITS == 16 ? 16384.0f : 4194304.0f);
  const bool fast = fast_den && !(a.softcap_log2 > 0.0f) && !a.alibi && a.scale_log2 > 0.0f;
  const float vlim = (BITS == 16 ? 32767.0f : 4194304.0f) / a.fxp_scale;  // 2^f: exact
  auto run = [&](auto fast_tag) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast_tag)::value;
    // A step consumes C ring entries (1: a K tile of phase 0; 2: a tile's K
    // and V in phase 1) and issues C more: the cursor stays NS - 2 entries
    // ahead, so the two slots a 2-entry step refills are free. Returns the
    // step's first entry (stage entry % NS).
    int step = 0;  // entries consumed
    auto step_begin = [&](auto c_tag) -> int {
      constexpr int C = decltype(c_tag)::value;
      // own DMAs of this step's entries landed (only the NS - 2 - C later
      // entries' in flight), own LDS accesses done; the barrier makes both
      // everyone's
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(G::NDMA * (NS - 2 - C)) : "memory");
      __builtin_amdgcn_s_barrier();
      if constexpr (C == 2) {
        // In phase 1 the cursor usually stands at a tile's K entry with its V
        // entry next (a step consumes a K / V pair and the cursor runs two
        // entries ahead): both from the one page entry, one cursor update
        if (dph != 0 && (didx & 1) == 0 && didx + 1 < dlim) {  // uniform
          const int t = cur_tile();
          const uint32_t p = page_of(dent);
          dma_mat(std::false_type{}, t, p, (step + NS - 2) & (NS - 1));
          dma_mat(std::true_type{}, t, p, (step + NS - 1) & (NS - 1));
          ++didx;  // the first advance(): no phase change by the test above
          advance();
          refresh_entry();
          const int e = step;
          step += C;
          return e;
        }
      }
#pragma unroll
      for (int u = 0; u < C; ++u) {
        dma_tile(cur_isv(), cur_tile(), dent, (step + NS - 2 + u) & (NS - 1));
        advance();
        refresh_entry();
      }
      const int e = step;
      step += C;
      return e;
    };
    auto stage_base = [&](int e) -> unsigned { return lds0 + (e & (NS - 1)) * G::TILEB; };
    // The four transposed score MFMA chains of the tile at base (q = 2 s + h),
    // software-pipelined: chain q + 1's fragment reads are issued before chain
    // q's wait and MFMAs (only the newest chain's QSTEPS reads may remain in
    // flight at the wait). At head_dim 128, fn(q - 1, acc) runs while chain
    // q's MFMAs do (at 64 the extra live registers cost a workgroup per CU).
    auto key_groups = [&](unsigned base, auto&& fn) __attribute__((always_inline)) {
      u32x4 kf[2][QSTEPS];
      f32x4 accs[2];
      auto issue = [&](auto qc) __attribute__((always_inline)) {
        constexpr int q = decltype(qc)::value;
        static_for<QSTEPS>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          lds_read_b128_off<(q >> 1) * 32 * G::ROWB>(base + koff[q & 1][j], kf[q & 1][j]);
        });
      };
      issue(std::integral_constant<int, 0>{});
      static_for<4>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        u32x4(&cur)[QSTEPS] = kf[q & 1];
        if constexpr (q + 1 < 4) {
          issue(std::integral_constant<int, q + 1>{});
          if constexpr (QSTEPS == 4) lds_waitn_for<QSTEPS>(cur[0], cur[1], cur[2], cur[3]);
          else lds_waitn_for<QSTEPS>(cur[0], cur[1]);
        } else {
          if constexpr (QSTEPS == 4) lds_wait_for(cur[0], cur[1], cur[2], cur[3]);
          else lds_wait_for(cur[0], cur[1]);
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < QSTEPS; ++j) acc = TR::mma(cur[j], qf[j], acc);
        if constexpr (QSTEPS == 4) {
          accs[q & 1] = acc;
          if constexpr (q > 0) fn(std::integral_constant<int, q - 1>{}, accs[(q - 1) & 1]);
        } else {
          fn(qc, acc);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      if constexpr (QSTEPS == 4) fn(std::integral_constant<int, 3>{}, accs[1]);
    };
    // Scores of chain q of tile t for the lane's row and keys
    // t * TILE + 32 (q >> 1) + 8 kg + 4 (q & 1) + e; whole: the wave's rows see
    // the whole tile.
    auto chain_scores = [&](const f32x4& acc, int t, int q, bool whole, float (&sc)[4]) __attribute__((always_inline)) {
      const int key0 = t * TILE + 32 * (q >> 1) + 8 * kg + 4 * (q & 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = __fmul_rn(acc[e], a.scale_log2);
        if constexpr (!FAST) {
          if (a.softcap_log2 > 0.0f) x = a.softcap_log2 * tanh_approx(x / a.softcap_log2);
          if (a.alibi) x = x + slope * static_cast<float>(key0 + e - qp);
        }
        sc[e] = (whole || (key0 + e >= ks && key0 + e < ke)) ? x : -__builtin_inff();
      }
    };
    auto tile_whole = [&](int t) -> bool {
      return __builtin_amdgcn_ballot_w64(!(ks <= t * TILE && t * TILE + TILE <= ke)) == 0;
    };

    for (int c = c_lo; c < c_hi; ++c) {
      const int ta = live_lo(c), te = live_hi(c);
      float mx = -__builtin_inff(), mraw = -__builtin_inff();
      // phase 0: the chunk's row maxima
      for (int t = ta; t < te; ++t) {
        const unsigned base = stage_base(step_begin(std::integral_constant<int, 1>{}));
        if (FAST && tile_whole(t)) {
          key_groups(base, [&](auto, const f32x4& acc) __attribute__((always_inline)) {
            mraw = fmaxf(fmaxf(mraw, fmaxf(acc[0], acc[1])), fmaxf(acc[2], acc[3]));
          });
        } else {
          key_groups(base, [&](auto qc, const f32x4& acc) __attribute__((always_inline)) {
            float sc[4];
            chain_scores(acc, t, decltype(qc)::value, false, sc);
            mx = fmaxf(fmaxf(mx, fmaxf(sc[0], sc[1])), fmaxf(sc[2], sc[3]));
          });
        }
      }
      if constexpr (FAST) mx = fmaxf(mx, __fmul_rn(mraw, a.scale_log2));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m = mx != -__builtin_inff() ? mx : 0.0f;  // no key: pin to 0
      // phase 1: weights and weighted V, tile by tile
      AccT den = 0;
      AccT wv[DBLK][4];
#pragma unroll
      for (int b = 0; b < DBLK; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[b][e] = 0;
      for (int t = ta; t < te; ++t) {
        const int e = step_begin(std::integral_constant<int, 2>{});  // K(t), then V(t)
        // P^T B operands of the two 32-key steps: word 2 h + e / 2 of pb[s]
        // holds the weights of keys 32 s + 8 kg + 4 h + e
        u32x4 pb[NK0];
        {
          const unsigned base = stage_base(e);
          // (whole as a type: two calls of one closure type would be merged
          // into one body whose closure references live in scratch memory)
          auto weights = [&](auto whole_tag) __attribute__((always_inline)) {
            constexpr bool WHOLE = decltype(whole_tag)::value;
            key_groups(base, [&](auto qc, const f32x4& acc) __attribute__((always_inline)) {
              constexpr int q = decltype(qc)::value, s = q >> 1, h = q & 1;
              float sc[4];
              chain_scores(acc, t, q, WHOLE, sc);
              float w[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) w[i] = __builtin_amdgcn_exp2f(sc[i] - m);
              if constexpr (FAST) {
                // w * 2^f + 1.5 * 2^23 (exact product, one rounding: RNE) has
                // the bits of RNE(w * 2^f) + 0x4B400000; NaN -> the constant
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const float y = fmaxf(__builtin_fmaf(w[i], a.fxp_scale, 12582912.0f), 12582912.0f);
                  den = static_cast<int32_t>(static_cast<uint32_t>(den) + __float_as_uint(y) - 0x4B400000u);
                }
                pb[s][2 * h] = p_pack2<DT>(w[0], w[1]);
                pb[s][2 * h + 1] = p_pack2<DT>(w[2], w[3]);
              } else {
                uint32_t p16[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  den = wadd<BITS>(den, quant<BITS>(__fmul_rn(w[i], a.fxp_scale)));
                  p16[i] = Io<DT>::store(w[i]);
                }
                pb[s][2 * h] = p16[0] | (p16[1] << 16);
                pb[s][2 * h + 1] = p16[2] | (p16[3] << 16);
              }
            });
          };
          if (FAST && tile_whole(t))
            weights(std::true_type{});
          else
            weights(std::false_type{});
        }
        {
          const unsigned base = stage_base(e + 1);
          // d blocks software-pipelined: block db + 1's V reads go out before
          // block db's wait (only they may remain in flight)
          uint64_t vr[2][NK0][2];
          // (step s reads KI rows further on: voff0[s][h] = voff0[0][h] + s KI
          // ROWB, as the swizzle takes row bits below 4 only; that goes in the
          // read's offset field, one address per (h, d block))
          auto issue_v = [&](auto dbc) __attribute__((always_inline)) {
            constexpr int db = decltype(dbc)::value;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const unsigned va = base + (voff0[0][h] ^ (db << 5));
              static_for<NK0>([&](auto sc) {
                constexpr int s = decltype(sc)::value;
                lds_read_b64_tr16_off<s * KI * G::ROWB>(va, vr[db & 1][s][h]);
              });
            }
          };
          issue_v(std::integral_constant<int, 0>{});
          f32x4 accv[DBLK];  // fast variant: the tile's weighted V, quantised after the range check
          float vmax = 0.0f;
          static_for<DBLK>([&](auto dbc) {
            constexpr int db = decltype(dbc)::value;
            uint64_t(&cur)[NK0][2] = vr[db & 1];
            if constexpr (db + 1 < DBLK) {
              issue_v(std::integral_constant<int, db + 1>{});
              if constexpr (NK0 == 2) lds_waitn_for<4>(cur[0][0], cur[0][1], cur[1][0], cur[1][1]);
              else lds_waitn_for<2>(cur[0][0], cur[0][1]);
            } else {
              if constexpr (NK0 == 2) lds_wait_for(cur[0][0], cur[0][1], cur[1][0], cur[1][1]);
              else lds_wait_for(cur[0][0], cur[0][1]);
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NK0; ++s) {
              const u32x4 vb = {uint32_t(cur[s][0]), uint32_t(cur[s][0] >> 32), uint32_t(cur[s][1]),
                                uint32_t(cur[s][1] >> 32)};
              acc = TR::mma(vb, pb[s], acc);
            }
            // lane: d = 16 db + 4 kg + e of its row
            if constexpr (FAST) {
              // block db - 1's maximum while block db's MFMAs run (reading a
              // result right after its MFMA costs wait states)
              accv[db] = acc;
              if constexpr (db > 0) vmax = absmax4(vmax, accv[db - 1]);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) wv[db][i] = wadd<BITS>(wv[db][i], quant<BITS>(__fmul_rn(acc[i], a.fxp_scale)));
            }
            __builtin_amdgcn_sched_barrier(0);
          });
          if constexpr (FAST) {
            vmax = absmax4(vmax, accv[DBLK - 1]);
            // |acc| * 2^f below 2^22 (and the 16-bit range) for the whole
            // wave: fl(acc * 2^f + 1.5 * 2^23) is RNE(acc * 2^f) + 1.5 * 2^23
            // (exact product, one rounding, spacing 1, even constant), the
            // bits quant gives. The terms go in unconditionally; if a lane is
            // out of range (large values, NaN) the wave takes the same terms
            // out again (sums wrap) and adds the exact ones. (A branch between
            // the two updates left the sums in other registers on one side,
            // and the loop copied all 32 back every tile.)
            auto fast_term = [&](float x) { return __float_as_uint(__builtin_fmaf(x, a.fxp_scale, 12582912.0f)) - 0x4B400000u; };
#pragma unroll
            for (int b = 0; b < DBLK; ++b)
#pragma unroll
              for (int i = 0; i < 4; ++i) wv[b][i] = static_cast<int32_t>(static_cast<uint32_t>(wv[b][i]) + fast_term(accv[b][i]));
            if (__builtin_amdgcn_ballot_w64(!(vmax < vlim)) != 0) {
#pragma unroll
              for (int b = 0; b < DBLK; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  const AccT undone = static_cast<int32_t>(static_cast<uint32_t>(wv[b][i]) - fast_term(accv[b][i]));
                  wv[b][i] = wadd<BITS>(undone, quant<BITS>(__fmul_rn(accv[b][i], a.fxp_scale)));
                }
            }
          }
        }
      }
      // the chunk's denominator over the row's four lanes, then the fold
      den = wadd<BITS>(den, __shfl_xor(den, 16, 64));
      den = wadd<BITS>(den, __shfl_xor(den, 32, 64));
      if (__builtin_amdgcn_ballot_w64(Mr != -__builtin_inff()) == 0) {
        // no row of the wave has folded a chunk yet (W = D = 0, M = -inf):
        // the fold gives the chunk's own sums (rescale(0, 0) + rescale(x, 1));
        // a row without a key here has zero sums (its weights are 0 and a
        // NaN product quantises to 0) and keeps M = -inf
#pragma unroll
        for (int b = 0; b < DBLK; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) Wr[b][i] = wv[b][i];
        Dr = den;
        Mr = mx;
      } else if (mx != -__builtin_inff()) {  // else no key of the row in this chunk
        float Mn, fa, fb;
        merge_factors(Mr, mx, Mn, fa, fb);
        // Mn is M or mc, so fa or fb is 2^0 = 1 unless both maxima are +inf
        // (then inf - inf: NaN). rescale(x, 1) = x for 16- and 32-bit sums
        // (exact in fp64; 16-bit sums are read modulo 2^16 everywhere), so
        // the fold rescales one side only. 64-bit sums round through fp64.
        const bool one_a = fa == 1.0f;
        if (BITS != 64 && __builtin_amdgcn_ballot_w64(!(one_a || fb == 1.0f)) == 0) {
          const float f = one_a ? fb : fa;
          Dr = wadd<BITS>(rescale<BITS>(one_a ? den : Dr, f), one_a ? Dr : den);
#pragma unroll
          for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const AccT x = one_a ? wv[b][i] : Wr[b][i], y = one_a ? Wr[b][i] : wv[b][i];
              Wr[b][i] = wadd<BITS>(rescale<BITS>(x, f), y);
            }
        } else {
          Dr = wadd<BITS>(rescale<BITS>(Dr, fa), rescale<BITS>(den, fb));
#pragma unroll
          for (int b = 0; b < DBLK; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) Wr[b][i] = wadd<BITS>(rescale<BITS>(Wr[b][i], fa), rescale<BITS>(wv[b][i], fb));
        }
        Mr = Mn;
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // DMAs into unused stages
  };
  if (c_lo < c_hi) {
    if constexpr (BITS != 64) {
      if (fast)
        run(std::true_type{});
      else
        run(std::false_type{});
    } else {
      run(std::false_type{});
    }
  }

  if (me.valid) {
    // the row's 32 quotients over one denominator (in [1e-6, 2^31]; the
    // numerators are fixed-point values below 2^31): by its rounded
    // reciprocal, the same bits as div_rn
    const float den_f = fmaxf(acc_f32<BITS>(Dr, a.fxp_inv), 1.0e-6f);
    const float rcp = div_rn(1.0f, den_f);
    T* orow = static_cast<T*>(a.o) + me.token * a.so_t + int64_t(me.head) * a.so_h;
#pragma unroll
    for (int b = 0; b < DBLK; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        orow[b * 16 + 4 * kg + i] = Io<DT>::store(div_rn_by_recip(acc_f32<BITS>(Wr[b][i], a.fxp_inv), den_f, rcp));
  }
}

// Fold the per-chunk partials of each (token, head) in ascending chunk order
// (the kernel's single-pass fold, step for step) and divide.
template <int DT, int BITS>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, int64_t num_tokens) {
  using T = typename Traits<DT>::T;
  using AccT = typename AccOf<BITS>::T;
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  // tokens past query_start_loc[num_requests] belong to no request (e.g. graph
  // padding) and are left untouched, as in the single-pass path
  const int64_t used = min<int64_t>(num_tokens, a.qsl[a.num_requests]);
  const int64_t total = used * a.num_heads * a.head_dim;
  if (idx >= total) return;
  const int d = int(idx % a.head_dim);
  const int64_t th = idx / a.head_dim;  // token * Hq + head
  float M = -__builtin_inff();
  AccT D = 0, W = 0;
  // batches of NB chunks: every load of a batch is issued (clamped to the
  // range) before the sequential fold, so the loads overlap
  constexpr int NB = 16;
  const AccT* den_p = static_cast<const AccT*>(a.den_ws) + th * a.chunk_slots;
  const AccT* wv_p = static_cast<const AccT*>(a.wv_ws) + th * a.chunk_slots * a.head_dim + d;
  const float* pm_p = a.pmax + th * a.chunk_slots;
  float mc[NB];
  AccT dc[NB], wc[NB];
  auto load = [&](int cb, int c_end) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int c = min(cb + k, c_end - 1);
      mc[k] = pm_p[c];
      dc[k] = den_p[c];
      wc[k] = wv_p[int64_t(c) * a.head_dim];
    }
  };
  // Mn is M or mc[k], so fa or fb is 2^0 = 1 (unless both maxima are +inf:
  // inf - inf is NaN), and rescale(x, 1) = x for 16- and 32-bit sums (exact
  // in fp64): those rescale one side only. The side is the same for the
  // whole (token, head), i.e. for every lane of the wave.
  auto fold = [&](int cb, int c_end) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      if (cb + k >= c_end || mc[k] == -__builtin_inff()) continue;
      float Mn, fa, fb;
      merge_factors(M, mc[k], Mn, fa, fb);
      if (BITS != 64 && fa == 1.0f) {
        D = wadd<BITS>(D, rescale<BITS>(dc[k], fb));
        W = wadd<BITS>(W, rescale<BITS>(wc[k], fb));
      } else if (BITS != 64 && fb == 1.0f) {
        D = wadd<BITS>(rescale<BITS>(D, fa), dc[k]);
        W = wadd<BITS>(rescale<BITS>(W, fa), wc[k]);
      } else {
        D = wadd<BITS>(rescale<BITS>(D, fa), rescale<BITS>(dc[k], fb));
        W = wadd<BITS>(rescale<BITS>(W, fa), rescale<BITS>(wc[k], fb));
      }
      M = Mn;
    }
  };
  // The first batch goes out with the range loads (the range of a row
  // usually starts at chunk 0 and fits one batch): one round trip, not two.
  if (a.chunk_slots > 0) load(0, a.chunk_slots);
  const int c0 = max(0, a.crange[2 * th]), c1 = min(a.chunk_slots, a.crange[2 * th + 1]);
  if (c0 == 0 && c1 <= NB) {
    fold(0, c1);
  } else {
    for (int cb = c0; cb < c1; cb += NB) {
      load(cb, c1);
      fold(cb, c1);
    }
  }
  const float den_f = fmaxf(acc_f32<BITS>(D, a.fxp_inv), 1.0e-6f);
  const int64_t token = th / a.num_heads;
  const int head = int(th % a.num_heads);
  static_cast<T*>(a.o)[token * a.so_t + int64_t(head) * a.so_h + d] =
      Io<DT>::store(div_rn(acc_f32<BITS>(W, a.fxp_inv), den_f));
}

// attn_dma_kernel serves a launch when each wave's 16 key rows of a tile lie
// in one page and the rows are exactly DMAX wide.
template <int DT, int DMAX> bool dma_ok(const AttnArgs& a) {
  if constexpr (DT == FXPR_DTYPE_F32 || (DMAX != 64 && DMAX != 128)) {
    return false;
  } else {
    // pages of 16, 32, ... keys; key strides below 2^20 elements (the prefill
    // kernel's 32-bit lane offsets span 16 of them)
    // and a page's K and V rows below 2^31 bytes (the prefill kernel's scalar
    // offset to a wave's first row)
    return a.head_dim == DMAX && a.ps_shift >= 4 && a.sk_s < (int64_t(1) << 20) && a.sv_s < (int64_t(1) << 20) &&
           a.ps_shift < 31 && ((a.sk_s > a.sv_s ? a.sk_s : a.sv_s) << a.ps_shift) < (int64_t(1) << 30);
  }
}

template <int DT, int BITS, int DMAX, bool SPLIT>
int launch_dma(const AttnArgs& a, dim3 grid, hipStream_t st) {
  if constexpr (DT != FXPR_DTYPE_F32 && (DMAX == 64 || DMAX == 128)) {
    auto kern = attn_dma_kernel<DT, BITS, DMAX, SPLIT>;
    constexpr size_t lds = dma_lds_bytes<DMAX>();
    static bool attr_done = false;  // benign race: the attribute is idempotent
    if (!attr_done) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
      if (e != hipSuccess) return int(e);
      attr_done = true;
    }
    kern<<<grid, kThreads, lds, st>>>(a);
  }
  return 0;
}

template <int DT, int BITS, int DMAX>
int launch_prefill_dma(const AttnArgs& a, dim3 grid, hipStream_t st) {
  if constexpr (DT != FXPR_DTYPE_F32 && (DMAX == 64 || DMAX == 128)) {
    auto kern = attn_prefill_dma_kernel<DT, BITS, DMAX>;
    constexpr size_t lds = prefill_dma_lds_bytes<DMAX>();
    static bool attr_done = false;  // benign race: the attribute is idempotent
    if (!attr_done) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
      if (e != hipSuccess) return int(e);
      attr_done = true;
    }
    kern<<<grid, kPThreads, lds, st>>>(a);
  }
  return 0;
}

template <int DT, int BITS, int DMAX>
int launch_attn(const AttnArgs& a, int num_requests, int max_qtiles, int64_t num_tokens, hipStream_t st) {
  dim3 grid(unsigned(num_requests * a.num_kv_heads), unsigned(max_qtiles), unsigned(a.num_splits));
  const bool dma = dma_ok<DT, DMAX>(a);
  if (a.num_splits <= 1) {
    if constexpr (DT != FXPR_DTYPE_F32 && BITS <= 32 && DMAX <= 128) {
      // Requests of at least kPrefillRows rows run in 64-row workgroups,
      // the others (decode steps, short prompts) in attn_kernel's 16-row
      // ones; both kernels see the whole batch and each skips the other's
      // requests. Same bits per row either way.
      if (int64_t(max_qtiles) * QROWS >= kPrefillRows) {
        AttnArgs b = a;
        b.pq_rows = kPrefillRows;
        const int ptiles = int(cdiv(int64_t(max_qtiles) * QROWS, PQROWS));
        const dim3 pgrid(grid.x, unsigned(ptiles), 1);
        if (dma) {
          const int e = launch_prefill_dma<DT, BITS, DMAX>(b, pgrid, st);
          if (e) return e;
        } else {
          attn_prefill_kernel<DT, BITS, DMAX><<<pgrid, kPThreads, 0, st>>>(b);
        }
        // the short requests (fewer than kPrefillRows rows) span at most
        // this many 16-row tiles: a grid over every tile of the longest
        // request would only start workgroups that exit at once
        const int64_t short_tiles = cdiv(kPrefillRows - 1, QROWS);
        const dim3 sgrid(grid.x, unsigned(max_qtiles < short_tiles ? max_qtiles : short_tiles), 1);
        if (dma) {
          const int e = launch_dma<DT, BITS, DMAX, false>(b, sgrid, st);
          if (e) return e;
        } else {
          attn_kernel<DT, BITS, DMAX, false><<<sgrid, kThreads, 0, st>>>(b);
        }
        return launch_status();
      }
    }
    if (dma) {
      const int e = launch_dma<DT, BITS, DMAX, false>(a, grid, st);
      if (e) return e;
    } else {
      attn_kernel<DT, BITS, DMAX, false><<<grid, kThreads, 0, st>>>(a);
    }
    return launch_status();
  }
  if (dma) {
    const int e = launch_dma<DT, BITS, DMAX, true>(a, grid, st);
    if (e) return e;
  } else {
    attn_kernel<DT, BITS, DMAX, true><<<grid, kThreads, 0, st>>>(a);
  }
  const int64_t total = num_tokens * a.num_heads * a.head_dim;
  attn_combine_kernel<DT, BITS><<<dim3(unsigned(cdiv(total, 256))), 256, 0, st>>>(a, num_tokens);
  return launch_status();
}

template <int DT, int BITS>
int dispatch_dmax(const AttnArgs& a, int num_requests, int max_qtiles, int64_t num_tokens, hipStream_t st) {
  if (a.head_dim <= 64) return launch_attn<DT, BITS, 64>(a, num_requests, max_qtiles, num_tokens, st);
  if (a.head_dim <= 128) return launch_attn<DT, BITS, 128>(a, num_requests, max_qtiles, num_tokens, st);
  if constexpr (DT == FXPR_DTYPE_F32) return FXPR_E_SHAPE;  // fp32 tiles beyond 128 exceed LDS
  else return launch_attn<DT, BITS, 256>(a, num_requests, max_qtiles, num_tokens, st);
}

int run_attn_bf16(const AttnArgs& a, int bits, int num_requests, int max_qtiles, int64_t num_tokens, hipStream_t st);
int run_attn_f16(const AttnArgs& a, int bits, int num_requests, int max_qtiles, int64_t num_tokens, hipStream_t st);
int run_attn_f32(const AttnArgs& a, int bits, int num_requests, int max_qtiles, int64_t num_tokens, hipStream_t st);

}  // namespace attn
}  // namespace fxpr
