// Generic 8-bit K/V instantiations of the paged decode kernels (templates in
// pda_decode.h) for bf16 models: bf16 queries and output, any even head dim
// padded to a power of two, in a translation unit of their own so the build
// compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

// Padded head dim dp (a power of two from 8 to 512) for any even head dim.
KernelPair kernels_gen_q8_bf16(int dp, int g) {
  switch (dp) {
    case 8: return pair_for_g<8, true, true, true>(g);
    case 16: return pair_for_g<16, true, true, true>(g);
    case 32: return pair_for_g<32, true, true, true>(g);
    case 64: return pair_for_g<64, true, true, true>(g);
    case 128: return pair_for_g<128, true, true, true>(g);
    case 256: return pair_for_g<256, true, true, true>(g);
    case 512: return pair_for_g<512, true, true, true>(g);
  }
  return {};
}

}  // namespace pda_decode
