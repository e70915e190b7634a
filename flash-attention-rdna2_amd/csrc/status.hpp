// status.hpp — per-thread "last error" text behind fable_attn_last_error().
#pragma once
#include <stdarg.h>
#include <stdio.h>

namespace fa {

// Records a formatted message for fable_attn_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);

// Maps the result of a kernel launch to a status code (FA_OK or FA_ERR_LAUNCH).
int launch_status(const char* what);

}  // namespace fa
