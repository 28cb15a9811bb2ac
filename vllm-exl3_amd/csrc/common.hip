// Host-side error plumbing and library metadata for the C ABI.
#include "exl3_common.h"

#include <cstring>

namespace exl3 {

static thread_local char g_error[1024] = {0};

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

const char* get_error() { return g_error; }

}  // namespace exl3

EXL3_API const char* exl3_last_error(void) { return exl3::get_error(); }

EXL3_API int exl3_abi_version(void) { return 4; }
