// Generic fp16 instantiations of the paged decode kernels (templates in pda_decode.h), in a
// translation unit of their own so the build compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

// Padded head dim dp (a power of two from 8 to 512) for any even head dim.
KernelPair kernels_gen_f16(int dp, int g) {
  switch (dp) {
    case 8: return pair_for_g<8, false, false, true>(g);
    case 16: return pair_for_g<16, false, false, true>(g);
    case 32: return pair_for_g<32, false, false, true>(g);
    case 64: return pair_for_g<64, false, false, true>(g);
    case 128: return pair_for_g<128, false, false, true>(g);
    case 256: return pair_for_g<256, false, false, true>(g);
    case 512: return pair_for_g<512, false, false, true>(g);
  }
  return {};
}

}  // namespace pda_decode
