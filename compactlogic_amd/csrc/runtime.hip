// Error state and version query of the C ABI.
#include "common.h"

#include <string.h>

namespace cl {
namespace {
thread_local char g_error[512] = {0};
}  // namespace

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: HIP error %d (%s)", what, int(e), hipGetErrorString(e));
        return CL_ERR_HIP;
    }
    return CL_OK;
}

}  // namespace cl

extern "C" int cl_abi_version(void) { return 1; }

extern "C" const char* cl_last_error(void) { return cl::g_error; }
