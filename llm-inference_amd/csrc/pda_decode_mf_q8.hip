// Matrix-core instantiations of the paged decode kernels (templates in
// pda_decode.h) over 8-bit K/V: int8 rows converted in registers, fp16
// queries, GQA groups served as units of up to 16 query heads; a
// translation unit of its own so the build compiles it in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_mf_q8(int d) {
  switch (d) {
    case 64: return make_pair<64, 16, true, false, false, true>();
    case 128: return make_pair<128, 16, true, false, false, true>();
    case 256: return make_pair<256, 16, true, false, false, true>();
  }
  return {};
}

}  // namespace pda_decode
