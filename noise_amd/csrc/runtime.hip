// Library-wide host state: the per-thread error message and the ABI version.
#include "common.hpp"

namespace noise {
namespace {
thread_local char g_error[1024] = "";
}

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace noise

extern "C" int noise_abi_version(void) { return 2; }

extern "C" const char *noise_last_error(void) { return noise::g_error; }
