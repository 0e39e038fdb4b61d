// Internal helpers shared by the libpda.so sources (not part of the C-ABI).
#ifndef PDA_INTERNAL_H
#define PDA_INTERNAL_H

namespace pda_internal {

// Records a formatted message for pda_last_error() on this thread and
// returns `code`.
__attribute__((visibility("hidden"))) int fail(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));

// Clears the thread's message and returns PDA_OK.
__attribute__((visibility("hidden"))) int ok();

// The thread's message.
__attribute__((visibility("hidden"))) const char* last_error();

}  // namespace pda_internal

#endif  // PDA_INTERNAL_H
