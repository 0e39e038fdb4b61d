// Matrix-core instantiations of the paged decode kernels (templates in
// pda_decode.h) for GQA groups of 5 to 16 query heads per unit, in a
// translation unit of their own so the build compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_mf(int d, bool bf16) {
  if (bf16) {
    switch (d) {
      case 64: return make_pair<64, 16, false, true, false, true>();
      case 96: return make_pair<96, 16, false, true, false, true>();
      case 128: return make_pair<128, 16, false, true, false, true>();
      case 256: return make_pair<256, 16, false, true, false, true>();
    }
    return {};
  }
  switch (d) {
    case 64: return make_pair<64, 16, false, false, false, true>();
    case 96: return make_pair<96, 16, false, false, false, true>();
    case 128: return make_pair<128, 16, false, false, false, true>();
    case 256: return make_pair<256, 16, false, false, false, true>();
  }
  return {};
}

}  // namespace pda_decode
