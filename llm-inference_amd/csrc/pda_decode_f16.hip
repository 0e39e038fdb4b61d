// fp16 instantiations of the paged decode kernels (templates in pda_decode.h), in a
// translation unit of their own so the build compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_f16(int d, int g) {
  switch (d) {
    case 64: return pair_for_g<64, false, false>(g);
    case 80: return pair_for_g<80, false, false>(g);
    case 96: return pair_for_g<96, false, false>(g);
    case 128: return pair_for_g<128, false, false>(g);
    case 256: return pair_for_g<256, false, false>(g);
    case 512: return pair_for_g<512, false, false>(g);
  }
  return {};
}

}  // namespace pda_decode
