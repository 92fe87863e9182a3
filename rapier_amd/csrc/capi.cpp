// capi.cpp - error model of the rapier_mi C ABI: every entry point returns a code, the message of the calling
// thread's last failure is kept for rmi_last_error() (the C++ shim in include/rapier_mi.hpp rethrows it).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "rmi_common.h"

namespace rmi {
namespace {
thread_local char g_err[512] = "";
}

void set_error(const char* msg) {
    std::snprintf(g_err, sizeof g_err, "%s", msg ? msg : "");
}

int fail(int code, const char* msg) {
    set_error(msg);
    return code;
}

int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return RMI_OK;
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s launch: %s", what, hipGetErrorString(e));
    return fail(RMI_ERR_LAUNCH, buf);
}

}  // namespace rmi

extern "C" const char* rmi_last_error(void) { return rmi::g_err; }
extern "C" const char* rmi_version(void) { return "rapier_mi 0.1 gfx950"; }
