// 8-bit K/V instantiations of the paged decode kernels (templates in
// pda_decode.h) for bf16 models: bf16 queries and output over int8 rows, in a
// translation unit of their own so the build compiles them in parallel.
#include "pda_decode.h"

namespace pda_decode {

KernelPair kernels_q8_bf16(int d, int g) {
  switch (d) {
    case 64: return pair_for_g<64, true, true>(g);
    case 128: return pair_for_g<128, true, true>(g);
    case 256: return pair_for_g<256, true, true>(g);
    case 512: return pair_for_g<512, true, true>(g);
  }
  return {};
}

}  // namespace pda_decode
