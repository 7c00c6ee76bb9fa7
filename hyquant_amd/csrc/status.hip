// Status reporting shared by every entry point of libhyq.so.
#include "hyq_common.h"

namespace hyq {
namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(HYQ_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return HYQ_OK;
}

const char* last_error_cstr() { return g_last_error.c_str(); }
}  // namespace hyq

extern "C" const char* hyq_last_error(void) { return hyq::last_error_cstr(); }
extern "C" int hyq_abi_version(void) { return 7; }
