// Error reporting shared by the library's host translation units: the text
// hoard_last_error() returns, set together with the status a call returns.
#pragma once

#include <cstdarg>
#include <cstdio>

extern "C" int hoard_set_error(int code, const char *msg);

namespace hoard {

inline int fail_fmt(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return hoard_set_error(code, buf);
}

}  // namespace hoard
