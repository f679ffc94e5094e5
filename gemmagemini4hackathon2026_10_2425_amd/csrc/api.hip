// Library-wide host plumbing: thread-local error text, tunables, ABI version.
#include "common.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <unordered_map>

namespace mxd {

static thread_local char g_err[512] = "";

static void vset(const char* fmt, va_list ap) { vsnprintf(g_err, sizeof(g_err), fmt, ap); }

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vset(fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vset(fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(MXD_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return MXD_OK;
}

static std::mutex g_tun_mu;
static std::unordered_map<std::string, int> g_tun;

int tunable(const char* name, int fallback) {
    std::lock_guard<std::mutex> lk(g_tun_mu);
    auto it = g_tun.find(name);
    return it == g_tun.end() ? fallback : it->second;
}

}  // namespace mxd

extern "C" const char* mxd_last_error(void) { return mxd::g_err; }

extern "C" int mxd_abi_version(void) { return 2; }

extern "C" int mxd_set_tunable(const char* name, int value) {
    if (!name || !*name) return mxd::fail(MXD_ERR_INVALID_ARG, "mxd_set_tunable: empty name");
    std::lock_guard<std::mutex> lk(mxd::g_tun_mu);
    if (value <= 0)
        mxd::g_tun.erase(name);
    else
        mxd::g_tun[name] = value;
    return MXD_OK;
}
