// moe_status.h -- the per-thread status message behind gptoss_last_error(),
// shared by the C-ABI source files.
#pragma once

#include <cstdarg>
#include <cstddef>
#include <exception>
#include <new>

#include "../../include/gptoss_moe.h"

namespace gxmoe {

// Length (1..4) of the well-formed UTF-8 sequence at u, of which `avail`
// bytes are readable, or 0: no overlong forms, surrogates or code points
// past U+10FFFF.
inline int utf8_seq_len(const unsigned char* u, size_t avail) {
  if (avail == 0) return 0;
  const unsigned c = u[0];
  if (c < 0x80) return 1;
  const int n = (c >> 5) == 6 ? 1 : (c >> 4) == 14 ? 2 : (c >> 3) == 30 ? 3 : -1;  // continuation bytes
  if (n < 0 || static_cast<size_t>(n) >= avail) return 0;
  unsigned cp = n == 1 ? c & 0x1f : n == 2 ? c & 0x0f : c & 0x07;
  for (int i = 1; i <= n; ++i) {
    if ((u[i] >> 6) != 2) return 0;
    cp = (cp << 6) | (u[i] & 0x3f);
  }
  if ((n == 1 && cp < 0x80) || (n == 2 && (cp < 0x800 || (cp >= 0xd800 && cp < 0xe000))) ||
      (n == 3 && (cp < 0x10000 || cp > 0x10ffff)))
    return 0;
  return n + 1;
}

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
