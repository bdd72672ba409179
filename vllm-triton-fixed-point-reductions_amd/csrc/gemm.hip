// C-ABI entry points of the fixed-point GEMM (kernels: gemm_impl.h,
// instantiated per input type in gemm_{bf16,f16,f32}.hip).
#include "gemm_impl.h"

using namespace fxpr;
using namespace fxpr::gemm;

extern "C" int fxpr_gemm_splits(int64_t m, int64_t n, int64_t k, int io_dtype, int int_bits, int split_k) {
  if (m <= 0 || n <= 0 || k < 0) return 1;
  return resolve_splits(m, n, k, io_dtype, int_bits, split_k);
}

extern "C" int64_t fxpr_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int io_dtype,
                                             int int_bits, int split_k) {
  if (m <= 0 || n <= 0 || k < 0) return 0;
  return ws_bytes_for(m, n, int_bits, resolve_splits(m, n, k, io_dtype, int_bits, split_k));
}

namespace {

// One launch of the GEMM in a mode: kFull (C), kPartial (the integer
// accumulators into `ws` as [M][N]), kFinish (C from the accumulators in `ws`).
int gemm_launch(const void* a, const void* b, const float* bias, void* c, int io_dtype, int64_t m, int64_t n,
                int64_t k, int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                int64_t stride_cm, int64_t stride_cn, int int_bits, int frac_bits, int split_k, void* workspace,
                int64_t workspace_bytes, int mode, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (m < 0 || n < 0 || k < 0 || split_k < 0) return FXPR_E_SHAPE;
  if (m == 0 || n == 0) return FXPR_OK;
  if (mode == kFinish) {
    if (!c || !workspace) return FXPR_E_ARG;
    GemmArgs args{};
    args.bias = bias;
    args.c = c;
    args.ws = workspace;
    args.M = m;
    args.N = n;
    args.scm = stride_cm;
    args.scn = stride_cn;
    args.scale = pow2f(frac_bits);
    args.inv_scale = pow2f(-frac_bits);
    args.mode = kFinish;
    hipStream_t st = as_stream(stream);
    switch (io_dtype) {
      case FXPR_DTYPE_BF16: return run_gemm_bf16(args, int_bits, false, false, 1, st);
      case FXPR_DTYPE_F16: return run_gemm_f16(args, int_bits, false, false, 1, st);
      case FXPR_DTYPE_F32: return run_gemm_f32(args, int_bits, false, false, 1, st);
      default: return FXPR_E_DTYPE;
    }
  }
  if (mode == kPartial ? (!workspace || (k > 0 && (!a || !b))) : (!c || (k > 0 && (!a || !b))))
    return FXPR_E_ARG;  // K = 0: C = bias (or 0); accumulators 0
  if (io_dtype != FXPR_DTYPE_BF16 && io_dtype != FXPR_DTYPE_F16 && io_dtype != FXPR_DTYPE_F32)
    return FXPR_E_DTYPE;
  if (stride_ak != 1 && k > 1) return FXPR_E_ARG;  // A must be K-contiguous
  bool b_ncontig;
  int64_t ldb;
  if (stride_bk == 1 || k <= 1) {
    b_ncontig = false;
    ldb = stride_bn;
  } else if (stride_bn == 1 || n == 1) {
    b_ncontig = true;
    ldb = stride_bk;
  } else {
    return FXPR_E_ARG;  // B needs one unit-stride dimension
  }
  const int splits = mode == kPartial ? 1 : resolve_splits(m, n, k, io_dtype, int_bits, split_k);
  if (splits > 1 && (!workspace || workspace_bytes < ws_bytes_for(m, n, int_bits, splits)))
    return FXPR_E_WORKSPACE;
  if (k > 0 && cdiv(k, ktile_for(io_dtype)) > 0x7fffffff) return FXPR_E_SHAPE;

  const int esz = io_dtype == FXPR_DTYPE_F32 ? 4 : 2;
  const int ch = 16 / esz;
  const bool vec = aligned(a, 16) && aligned(b, 16) && (stride_am % ch == 0 || m == 1) &&
                   (ldb % ch == 0 || (b_ncontig ? k == 1 : n == 1));

  GemmArgs args{};
  args.a = a;
  args.b = b;
  args.bias = bias;
  args.c = c;
  args.ws = workspace;
  args.M = m;
  args.N = n;
  args.K = k;
  args.lda = stride_am;
  args.ldb = ldb;
  args.scm = stride_cm;
  args.scn = stride_cn;
  args.scale = pow2f(frac_bits);
  args.inv_scale = pow2f(-frac_bits);
  // the large-M kernel's rounding-constant bound on a K-tile's partials:
  // |P * 2^f| below 2^22 (and 32767 for 16-bit sums)
  args.fast_lim = frac_bits < 0 ? 0.0f : (int_bits == 16 ? 32767.0f : 4194304.0f) * pow2f(-frac_bits);
  args.ktiles = int(cdiv(k, ktile_for(io_dtype)));
  args.tiles_per_split = int(cdiv(args.ktiles, splits));
  args.c_vec = mode == kFull && (stride_cn == 1 || n == 1) && stride_cm % ch == 0 && aligned(c, 16);
  args.mode = mode;
  hipStream_t st = as_stream(stream);

  switch (io_dtype) {
    case FXPR_DTYPE_BF16: return run_gemm_bf16(args, int_bits, b_ncontig, vec, splits, st);
    case FXPR_DTYPE_F16: return run_gemm_f16(args, int_bits, b_ncontig, vec, splits, st);
    default: return run_gemm_f32(args, int_bits, b_ncontig, vec, splits, st);
  }
}

}  // namespace

extern "C" int fxpr_gemm(const void* a, const void* b, const float* bias, void* c, int io_dtype,
                         int64_t m, int64_t n, int64_t k, int64_t stride_am, int64_t stride_ak,
                         int64_t stride_bk, int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
                         int int_bits, int frac_bits, int split_k, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  return gemm_launch(a, b, bias, c, io_dtype, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, stride_cm,
                     stride_cn, int_bits, frac_bits, split_k, workspace, workspace_bytes, kFull, stream);
}

extern "C" int fxpr_gemm_partial(const void* a, const void* b, void* acc, int io_dtype, int64_t m, int64_t n,
                                 int64_t k, int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                                 int64_t stride_bn, int int_bits, int frac_bits, void* stream) {
  return gemm_launch(a, b, nullptr, nullptr, io_dtype, m, n, k, stride_am, stride_ak, stride_bk, stride_bn, n, 1,
                     int_bits, frac_bits, 1, acc, m * n * (int_bits == 64 ? 8 : 4), kPartial, stream);
}

extern "C" int fxpr_gemm_finish(const void* acc, const float* bias, void* c, int io_dtype, int64_t m, int64_t n,
                                int64_t stride_cm, int64_t stride_cn, int int_bits, int frac_bits, void* stream) {
  return gemm_launch(nullptr, nullptr, bias, c, io_dtype, m, n, 0, 0, 1, 1, 0, stride_cm, stride_cn, int_bits,
                     frac_bits, 1, const_cast<void*>(acc), m * n * (int_bits == 64 ? 8 : 4), kFinish, stream);
}
