// moe_status.h -- the per-thread status message behind gptoss_last_error(),
// shared by the C-ABI source files.
#pragma once

#include <cstdarg>

namespace gxmoe {

// Record a message for `code` on the calling thread and return `code`.
int vset_error(int code, const char* fmt, va_list ap);
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

}  // namespace gxmoe
