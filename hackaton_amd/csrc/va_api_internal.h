// Error reporting shared by the C-ABI translation units.
#pragma once

#include <cstdarg>
#include <cstdio>

namespace va {

// Thread-local message of the last failure (returned by va_last_error).
char* last_error_buffer();

// Formats the message into the thread's buffer and returns `code`.
inline int fail(int code, const char* fmt, ...) {
  char* buf = last_error_buffer();
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, 512, fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace va
