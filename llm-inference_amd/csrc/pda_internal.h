// Internal helpers shared by the libpda.so sources (not part of the C-ABI).
#ifndef PDA_INTERNAL_H
#define PDA_INTERNAL_H

#include <stdint.h>

namespace pda_internal {

// Records a formatted message for pda_last_error() on this thread and
// returns `code`.
__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));

// Clears the thread's message and returns PDA_OK.
__attribute__((visibility("hidden"))) int ok();

// The thread's message.
__attribute__((visibility("hidden"))) const char* last_error();

// Four int8 values (one dword, each byte's sign bit already flipped:
// b + 128) as one fp16 pair, exactly: v_perm places two bytes under the fp16
// exponent byte 0x64, which reads as 1024 + b + 128; subtracting 1152 leaves
// b. `sel` chooses the two bytes (0x04010400: bytes 0, 1; 0x04030402: bytes
// 2, 3).
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2_t bytes_to_f16x2(uint32_t flipped, uint32_t sel) {
  const half2_t biased =
      __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, flipped, sel));
  return biased - half2_t{(_Float16)1152.0f, (_Float16)1152.0f};
}

}  // namespace pda_internal

#endif  // PDA_INTERNAL_H
