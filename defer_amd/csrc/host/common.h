// common.h -- error plumbing shared by the host sources.
#pragma once

#include <stdarg.h>
#include <stddef.h>
#include <stdint.h>
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

// SHA-256 over data fed in pieces (FIPS 180-4; sha256.rs:15-134).
struct Sha256 {
  uint32_t h[8];
  uint8_t buf[64];
  size_t nbuf;
  uint64_t total;
  Sha256();
  void update(const uint8_t* data, size_t n);
  void finish(uint8_t out[32]);
};

}  // namespace dh
