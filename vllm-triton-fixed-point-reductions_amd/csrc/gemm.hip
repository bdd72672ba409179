// C-ABI entry points of the fixed-point GEMM (kernels: gemm_impl.h,
// instantiated per input type in gemm_{bf16,f16,f32}.hip).
#include "gemm_impl.h"

using namespace fxpr;
using namespace fxpr::gemm;

extern "C" int fxpr_gemm_splits(int64_t m, int64_t n, int64_t k, int io_dtype, int split_k) {
  if (m <= 0 || n <= 0 || k < 0) return 1;
  return resolve_splits(m, n, k, io_dtype, split_k);
}

extern "C" int64_t fxpr_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int io_dtype,
                                             int int_bits, int split_k) {
  if (m <= 0 || n <= 0 || k < 0) return 0;
  return ws_bytes_for(m, n, int_bits, resolve_splits(m, n, k, io_dtype, split_k));
}

extern "C" int fxpr_gemm(const void* a, const void* b, const float* bias, void* c, int io_dtype,
                         int64_t m, int64_t n, int64_t k, int64_t stride_am, int64_t stride_ak,
                         int64_t stride_bk, int64_t stride_bn, int64_t stride_cm, int64_t stride_cn,
                         int int_bits, int frac_bits, int split_k, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (!valid_int_bits(int_bits) || frac_bits < 0 || frac_bits > 63) return FXPR_E_BITS;
  if (m < 0 || n < 0 || k < 0 || split_k < 0) return FXPR_E_SHAPE;
  if (m == 0 || n == 0) return FXPR_OK;
  if (!c || (k > 0 && (!a || !b))) return FXPR_E_ARG;  // K = 0: C = bias (or 0)
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
  const int splits = resolve_splits(m, n, k, io_dtype, split_k);
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
  args.c_vec = (stride_cn == 1 || n == 1) && stride_cm % ch == 0 && aligned(c, 16);
  hipStream_t st = as_stream(stream);

  switch (io_dtype) {
    case FXPR_DTYPE_BF16: return run_gemm_bf16(args, int_bits, b_ncontig, vec, splits, st);
    case FXPR_DTYPE_F16: return run_gemm_f16(args, int_bits, b_ncontig, vec, splits, st);
    default: return run_gemm_f32(args, int_bits, b_ncontig, vec, splits, st);
  }
}
