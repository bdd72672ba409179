// Fixed-point GEMM kernels instantiated for bf16 inputs (see gemm_impl.h).
#include "gemm_impl.h"

namespace fxpr {
namespace gemm {

int run_gemm_bf16(const GemmArgs& a, int bits, bool b_ncontig, bool vec, int splits, hipStream_t st) {
  switch (bits) {
    case 16: return run_gemm<FXPR_DTYPE_BF16, 16>(a, b_ncontig, vec, splits, st);
    case 32: return run_gemm<FXPR_DTYPE_BF16, 32>(a, b_ncontig, vec, splits, st);
    default: return run_gemm<FXPR_DTYPE_BF16, 64>(a, b_ncontig, vec, splits, st);
  }
}

}  // namespace gemm
}  // namespace fxpr
