// Error plumbing of the C ABI: a thread-local message, no exceptions.
#include <hip/hip_runtime.h>

#include <string>

#include "mtl.h"

namespace mtl {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_last_error = std::string(what) + ": " + hipGetErrorString(e);
        return MTL_EHIP;
    }
    return MTL_OK;
}

}  // namespace mtl

extern "C" const char* mtl_last_error(void) { return mtl::g_last_error.c_str(); }
extern "C" int mtl_abi_version(void) { return 3; }
