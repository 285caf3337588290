// C-ABI bookkeeping shared by the kernel translation units: version and the
// per-thread last-error text.
#include <stdint.h>

#include "../../include/fp8_blockwise.h"

namespace fp8b {

static thread_local const char* g_last_error = "no error";

void set_error(const char* msg) { g_last_error = msg; }

}  // namespace fp8b

extern "C" int fp8b_version(void) { return 0x000100; }

extern "C" const char* fp8b_last_error(void) { return fp8b::g_last_error; }
