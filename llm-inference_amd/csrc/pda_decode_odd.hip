// Odd head dim instantiations of the paged decode kernels (templates in pda_decode.h): the
// generic kernels with element-wise loads and stores, one query head per unit, for fp16 and
// bf16 queries over 16-bit or 8-bit K/V, in a translation unit of their own.
#include "pda_decode.h"

namespace pda_decode {

namespace {

template <int D>
KernelPair odd_for(bool q8, bool bf16) {
  if (q8) return bf16 ? make_odd_pair<D, true, true>() : make_odd_pair<D, true, false>();
  return bf16 ? make_odd_pair<D, false, true>() : make_odd_pair<D, false, false>();
}

}  // namespace

// Padded head dim dp (a power of two from 8 to 512) for any odd head dim.
KernelPair kernels_odd(int dp, bool q8, bool bf16) {
  switch (dp) {
    case 8: return odd_for<8>(q8, bf16);
    case 16: return odd_for<16>(q8, bf16);
    case 32: return odd_for<32>(q8, bf16);
    case 64: return odd_for<64>(q8, bf16);
    case 128: return odd_for<128>(q8, bf16);
    case 256: return odd_for<256>(q8, bf16);
    case 512: return odd_for<512>(q8, bf16);
  }
  return {};
}

}  // namespace pda_decode
