// Fixed-point GEMM kernels instantiated for f32 inputs (see gemm_impl.h).
#include "gemm_impl.h"

namespace fxpr {
namespace gemm {

int run_gemm_f32(const GemmArgs& a, int bits, bool b_ncontig, bool vec, int splits, hipStream_t st) {
  switch (bits) {
    case 16: return run_gemm<FXPR_DTYPE_F32, 16>(a, b_ncontig, vec, splits, st);
    case 32: return run_gemm<FXPR_DTYPE_F32, 32>(a, b_ncontig, vec, splits, st);
    default: return run_gemm<FXPR_DTYPE_F32, 64>(a, b_ncontig, vec, splits, st);
  }
}

}  // namespace gemm
}  // namespace fxpr
