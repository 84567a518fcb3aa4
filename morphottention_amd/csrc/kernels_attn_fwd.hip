// Attention forward: scores, softmax and value aggregation.
//
// Reference: packages/morphottention/csrc/cuda/attention/attention.cu:7-189
//   (score s = (2 q.k - qb_i - cb_j) * scale * log2e, causal drop k > q,
//   online softmax in base 2, out = O / l, lse = m + log2 l)
//
// MI355X design:
//  * The exponent is produced by one MFMA accumulator over the code rows
//    [hi | affine(8) | lo] (see ProjBuffers): the chunk products hi.hi, hi.lo
//    and lo.hi of fp16 code pairs make the score exact to ~2^-22, and the
//    8-wide affine block adds the key bias and subtracts the row reference,
//    so exp2 reads the accumulator directly.
//  * The softmax uses a per-row reference R >= (row max - 15) computed by the
//    projection from a closed-form bound on the soft Hamming score, so no
//    running max or rescaling is needed; rows whose bound is loose (gap > 25,
//    only possible with large or negative gates) take an exact two-pass path.
//  * V is carried as fp16 V_hi plus its remainder in e4m3: O^T += V_hi^T P on
//    the fp16 MFMA and the remainder on the scaled fp8 MFMA with P's e5m2
//    bytes; the row normaliser sums exactly the fp16 P values.
//  * V^T fragments are read from a chunk-swizzled LDS tile; the key and value
//    tiles stream through LDS stages by DMA, one barrier per tile.
//  * This file (cube_m 16 and 32) is compiled with the machine scheduler's
//    max-ilp strategy (build.py): those forwards measured 1-4 % faster with
//    it, while the backward and the cube_m 64 forward did not, so cube_m 64
//    is compiled in kernels_attn_fwd_m64.hip with the default strategy.
//    The kernels and their launch helpers are in attn_fwd.h.
#include "attn_fwd.h"

namespace morpho {

hipError_t launch_attn_fwd(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  if (d.M == 64) return launch_attn_fwd_m64(d, p, out, lse, s);
  if (d.M == 16 && d.DV == 32) return launch_attn_fwd_t<16, 32>(d, p, out, lse, s);
  if (d.M == 16 && d.DV == 64) return launch_attn_fwd_t<16, 64>(d, p, out, lse, s);
  if (d.M == 16 && d.DV == 128) return launch_attn_fwd_t<16, 128>(d, p, out, lse, s);
  if (d.M == 32 && d.DV == 32) return launch_attn_fwd_t<32, 32>(d, p, out, lse, s);
  if (d.M == 32 && d.DV == 64) return launch_attn_fwd_t<32, 64>(d, p, out, lse, s);
  if (d.M == 32 && d.DV == 128) return launch_attn_fwd_t<32, 128>(d, p, out, lse, s);
  return hipErrorInvalidValue;
}

}  // namespace morpho
