// Host-only helpers shared by every libgrws translation unit: the error
// state of the C ABI and the argument-check macros.  No HIP headers, so the
// host converter (abi.cpp) also builds with a plain C++ compiler (the
// sanitizer build in tests/sanitize/).
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/grws.h"

namespace grws {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define GRWS_CHECK_ARG(cond, ...)                                   \
    do {                                                            \
        if (!(cond)) return ::grws::set_error(GRWS_E_INVALID, __VA_ARGS__); \
    } while (0)

#define GRWS_TRY(call)              \
    do {                            \
        int s_ = (call);            \
        if (s_ != GRWS_OK) return s_; \
    } while (0)

}  // namespace grws
