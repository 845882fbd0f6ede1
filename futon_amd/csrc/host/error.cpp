// Thread-local error detail behind fh_last_error (include/futon_hip.h).
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../../include/futon_hip.h"
#include "host_common.h"

namespace fh {
namespace {
thread_local std::string g_err;

std::string vformat(const char *fmt, va_list ap) {
    char buf[2048];
    vsnprintf(buf, sizeof buf, fmt, ap);
    return buf;
}
}  // namespace

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    g_err = vformat(fmt, ap);
    va_end(ap);
    return code;
}

const std::string &last_error() { return g_err; }

void raise(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::string msg = vformat(fmt, ap);
    va_end(ap);
    throw Error(code, msg);
}
}  // namespace fh

extern "C" const char *fh_strerror(int code) {
    switch (code) {
    case FH_OK: return "ok";
    case FH_EINVAL: return "invalid argument";
    case FH_ENOMEM: return "out of memory";
    case FH_EHIP: return "HIP runtime error";
    case FH_ECANCELED: return "canceled";
    case FH_ETOOLONG: return "sequence too long";
    case FH_ENODEV: return "no gfx950 device";
    default: return "unknown error";
    }
}

extern "C" int fh_last_error(char *buf, size_t len) {
    const std::string &e = fh::g_err;
    if (buf && len) {
        size_t n = e.size() < len - 1 ? e.size() : len - 1;
        memcpy(buf, e.data(), n);
        buf[n] = 0;
    }
    return (int)e.size();
}
