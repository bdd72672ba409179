// Paged attention kernels instantiated for f32 inputs (see attn_impl.h).
#include "attn_impl.h"

namespace fxpr {
namespace attn {

int run_attn_f32(const AttnArgs& a, int bits, int num_requests, int max_qtiles, int64_t num_tokens,
                hipStream_t st) {
  switch (bits) {
    case 16: return dispatch_dmax<FXPR_DTYPE_F32, 16>(a, num_requests, max_qtiles, num_tokens, st);
    case 32: return dispatch_dmax<FXPR_DTYPE_F32, 32>(a, num_requests, max_qtiles, num_tokens, st);
    default: return dispatch_dmax<FXPR_DTYPE_F32, 64>(a, num_requests, max_qtiles, num_tokens, st);
  }
}

}  // namespace attn
}  // namespace fxpr
