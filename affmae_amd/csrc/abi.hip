// Library-wide C entry points: error reporting and ABI version.
#include "common.hpp"

#include <string.h>

#include <mutex>

namespace aff {

static thread_local char g_last_error[512] = "";

aff_status fail(aff_status code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

// CU count of the current device, queried once per device (std::call_once, so
// concurrent first calls from several host threads are ordered).
int device_cu_count() {
    constexpr int MAXDEV = 64;
    static std::once_flag once[MAXDEV];
    static int cache[MAXDEV];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return 256;
    std::call_once(once[dev], [dev] {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    });
    return cache[dev];
}

}  // namespace aff

extern "C" const char *aff_last_error(void) { return aff::g_last_error; }

extern "C" int aff_abi_version(void) { return 8; }
