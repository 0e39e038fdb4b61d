// 8-bit K/V instantiations of the paged decode kernels (templates in pda_decode.h), in a
// translation unit of their own so the build compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_q8(int d, int g) {
  switch (d) {
    case 64: return pair_for_g<64, true, false>(g);
    case 128: return pair_for_g<128, true, false>(g);
    case 256: return pair_for_g<256, true, false>(g);
    case 512: return pair_for_g<512, true, false>(g);
  }
  return {};
}

}  // namespace pda_decode
