// Matrix-core instantiations of the paged decode kernels (templates in
// pda_decode.h) over 8-bit K/V for bf16 models: bf16 queries and output,
// the fp16 matrix-core step of the 8-bit kernels; a translation unit of its
// own so the build compiles it in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_mf_q8_bf16(int d) {
  switch (d) {
    case 64: return make_pair<64, 16, true, true, false, true>();
    case 128: return make_pair<128, 16, true, true, false, true>();
    case 256: return make_pair<256, 16, true, true, false, true>();
  }
  return {};
}

}  // namespace pda_decode
