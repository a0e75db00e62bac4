// C-ABI runtime pieces: per-thread error message, launch checks, version and target queries.
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace attnlab {

static thread_local char g_error[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(ATTNLAB_ERUNTIME, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return ATTNLAB_OK;
}

}  // namespace attnlab

extern "C" int attnlab_abi_version(void) { return 9; }

extern "C" const char* attnlab_last_error(void) { return attnlab::g_error; }

extern "C" const char* attnlab_target(void) { return "gfx950"; }
