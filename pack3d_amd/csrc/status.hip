// Thread-local status of the C ABI: the message of the last failure.
#include "common.hpp"

namespace p3d {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(P3D_EHIP, std::string(what) + ": " + hipGetErrorString(e));
    return P3D_OK;
}

}  // namespace p3d

extern "C" const char* p3d_last_error(void) { return p3d::g_last_error.c_str(); }
extern "C" int p3d_abi_version(void) { return P3D_ABI_VERSION; }
