// Error reporting and version for the ltxk C ABI.
#include <cstdarg>
#include <cstdio>

#include "ltxk_common.h"

namespace ltxk {

static thread_local char g_err[512];

int fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(LTXK_E_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return LTXK_OK;
}

}  // namespace ltxk

extern "C" int ltxk_version(void) { return LTXK_VERSION; }

extern "C" const char *ltxk_last_error(void) { return ltxk::g_err; }
