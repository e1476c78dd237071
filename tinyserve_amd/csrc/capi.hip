// Error plumbing of the C ABI: a per-thread message buffer and launch checking.
#include <stdarg.h>
#include <stdio.h>
#include "common.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return TSM_E_HIP;
    }
    return TSM_OK;
}

int launch_status(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return TSM_E_HIP;
    }
    return TSM_OK;
}
}  // namespace tsm

extern "C" const char* tsm_last_error(void) { return tsm::g_error; }
extern "C" int tsm_abi_version(void) { return 1; }
