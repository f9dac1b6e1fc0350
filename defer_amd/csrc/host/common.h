// common.h -- error plumbing shared by the host sources.
#pragma once

#include <stdarg.h>
#include <stdio.h>

#include <string>

namespace dh {

std::string& last_error();

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

}  // namespace dh
