// Attention forward at cube_m 64 (the kernels are in attn_fwd.h), compiled
// with the default machine-scheduler strategy: with max-ilp, like the
// cube_m 16 and 32 forwards in kernels_attn_fwd.hip, it measured 1 % slower
// (B16 N2048 D2048 H32).
#include "attn_fwd.h"

namespace morpho {

hipError_t launch_attn_fwd_m64(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  if (d.DV == 32) return launch_attn_fwd_t<64, 32>(d, p, out, lse, s);
  if (d.DV == 64) return launch_attn_fwd_t<64, 64>(d, p, out, lse, s);
  if (d.DV == 128) return launch_attn_fwd_t<64, 128>(d, p, out, lse, s);
  return hipErrorInvalidValue;
}

}  // namespace morpho
