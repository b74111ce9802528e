// moe_status.h -- the per-thread status message behind gptoss_last_error(),
// shared by the C-ABI source files.
#pragma once

#include <cstdarg>
#include <exception>
#include <new>

#include "../../include/gptoss_moe.h"

namespace gxmoe {

// Record a message for `code` on the calling thread and return `code`.
int vset_error(int code, const char* fmt, va_list ap);
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Runs f() and turns a C++ exception (host allocation, thread creation)
// into a status code: nothing thrown crosses the C ABI.
template <typename F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const std::bad_alloc&) {
    return set_error(GPTOSS_ERR_OOM, "out of host memory");
  } catch (const std::exception& e) {
    return set_error(GPTOSS_ERR_STATE, "unexpected C++ exception: %s", e.what());
  } catch (...) {
    return set_error(GPTOSS_ERR_STATE, "unexpected C++ exception");
  }
}

}  // namespace gxmoe
