// Error text and HIP status translation shared by every entry point.
#include "common.h"
#include <string.h>

namespace v1 {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return V1_OK;
    set_error("%s: %s", what, hipGetErrorString(e));
    return V1_ERR_HIP;
}

}  // namespace v1

extern "C" const char* v1_last_error(void) { return v1::g_error; }
extern "C" int v1_abi_version(void) { return 1; }
