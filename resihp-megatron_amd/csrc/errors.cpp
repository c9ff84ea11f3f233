// Per-thread error state of the C ABI and the version query.
#include <hip/hip_runtime.h>

#include <string>

#include "rhp_common.h"

namespace rhp {
namespace {
thread_local std::string g_last_error;
}

int fail(const std::string& msg) {
    g_last_error = msg;
    return 1;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(std::string(what) + ": launch failed: " + hipGetErrorString(e));
    return 0;
}

}  // namespace rhp

extern "C" int rhp_abi_version(void) { return RHP_ABI_VERSION; }

extern "C" const char* rhp_last_error(void) { return rhp::g_last_error.c_str(); }
