// Matrix-core instantiations of the paged decode kernels (templates in
// pda_decode.h) at head dim 512: fp16, bf16 and 8-bit K/V (8-bit with fp16
// or bf16 queries and output), GQA groups
// served as units of up to 16 query heads, four-wave workgroups (one wave
// per SIMD). Built without the VGPR-only matrix-core form: the 16 x 512
// output accumulators live in AGPRs.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_mf512(bool q8, bool bf16) {
  if (q8)
    return bf16 ? make_pair<512, 16, true, true, false, true>()
                : make_pair<512, 16, true, false, false, true>();
  if (bf16) return make_pair<512, 16, false, true, false, true>();
  return make_pair<512, 16, false, false, false, true>();
}

}  // namespace pda_decode
