// Library identity and per-thread error reporting of libcresso_hip.so.
#include "common.hpp"

#include <cstdarg>
#include <cstdio>

namespace cresso {
namespace {
thread_local char g_last_error[1024] = "";
}

int32_t fail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

int32_t hip_fail(hipError_t e, const char* what) {
    return fail(CRESSO_E_HIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}
}  // namespace cresso

extern "C" int32_t cresso_hip_abi_version(void) { return CRESSO_HIP_ABI_VERSION; }

extern "C" const char* cresso_hip_last_error(void) { return cresso::g_last_error; }
