// checkpoint.cpp -- semantic checkpoints (checkpoint.rs:4-136 of the
// reference): the metadata that rebuilds a session by recomputation, as one
// little-endian, CRC-checked file of 112 + 4n bytes, written to a temporary
// name, synced, then renamed.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "common.h"
#include "defer_host.h"

using dh::fail;

namespace {

const char kMagic[8] = {'D', 'E', 'F', 'E', 'R', 'C', 'K', 'P'};
const uint32_t kVersion = 1;
const size_t kFixed = 8 + 4 + 32 + 32 + 4 + 4 + 16 + 8;  // bytes before the tokens

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_u64(std::vector<uint8_t>& b, uint64_t v) {
  for (int i = 0; i < 8; ++i) b.push_back((uint8_t)(v >> (8 * i)));
}
uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
uint64_t get_u64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}

// DeferCheckpoint::to_bytes (checkpoint.rs:44-57).
std::vector<uint8_t> to_bytes(const defer_host_checkpoint_header& h, const uint32_t* tokens,
                              size_t n) {
  std::vector<uint8_t> b(kMagic, kMagic + 8);
  b.reserve(kFixed + 4 * n + 4);
  put_u32(b, kVersion);
  b.insert(b.end(), h.model_signature, h.model_signature + 32);
  b.insert(b.end(), h.base_seed, h.base_seed + 32);
  uint32_t tb;
  memcpy(&tb, &h.temperature, 4);
  put_u32(b, tb);
  put_u32(b, h.prompt_len);
  put_u64(b, h.rng_word_pos);
  put_u64(b, 0);  // high half of the u128 word position
  put_u64(b, (uint64_t)n);
  for (size_t i = 0; i < n; ++i) put_u32(b, tokens[i]);
  put_u32(b, defer_host_crc32(b.data(), b.size()));
  return b;
}

// Path::with_extension("ckpt.tmp"): the file name's extension (after its
// last '.', unless that dot starts the name) replaced, or appended.
std::string tmp_path(const std::string& path) {
  const size_t slash = path.find_last_of('/');
  const size_t name = slash == std::string::npos ? 0 : slash + 1;
  const size_t dot = path.find_last_of('.');
  if (dot != std::string::npos && dot > name) return path.substr(0, dot) + ".ckpt.tmp";
  return path + ".ckpt.tmp";
}

}  // namespace

extern "C" int defer_host_checkpoint_save(const char* path, const defer_host_checkpoint_header* h,
                                          const uint32_t* history, size_t n) {
  if (!path || !h || (n && !history)) return fail(DEFER_HOST_E_INVALID, "null argument");
  if (h->prompt_len > n) return fail(DEFER_HOST_E_INVALID, "prompt_len exceeds history length");
  const std::vector<uint8_t> b = to_bytes(*h, history, n);
  const std::string tmp = tmp_path(path);
  const int fd = open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) return fail(DEFER_HOST_E_IO, "%s: %s", tmp.c_str(), strerror(errno));
  size_t off = 0;
  while (off < b.size()) {
    const ssize_t w = write(fd, b.data() + off, b.size() - off);
    if (w < 0) {
      if (errno == EINTR) continue;
      const int e = errno;
      close(fd);
      return fail(DEFER_HOST_E_IO, "%s: %s", tmp.c_str(), strerror(e));
    }
    off += (size_t)w;
  }
  if (fsync(fd) != 0) {
    const int e = errno;
    close(fd);
    return fail(DEFER_HOST_E_IO, "%s: fsync: %s", tmp.c_str(), strerror(e));
  }
  if (close(fd) != 0) return fail(DEFER_HOST_E_IO, "%s: close: %s", tmp.c_str(), strerror(errno));
  if (rename(tmp.c_str(), path) != 0)
    return fail(DEFER_HOST_E_IO, "rename %s -> %s: %s", tmp.c_str(), path, strerror(errno));
  return DEFER_HOST_OK;
}

// DeferCheckpoint::from_bytes (checkpoint.rs:59-84) on the file's bytes.
extern "C" int defer_host_checkpoint_load(const char* path, defer_host_checkpoint_header* h,
                                          uint32_t* history, size_t* n_history) {
  if (!path || !h || !n_history) return fail(DEFER_HOST_E_INVALID, "null argument");
  FILE* f = fopen(path, "rb");
  if (!f) return fail(DEFER_HOST_E_IO, "%s: %s", path, strerror(errno));
  std::vector<uint8_t> b;
  uint8_t buf[1 << 16];
  size_t got;
  while ((got = fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + got);
  const bool err = ferror(f) != 0;
  fclose(f);
  if (err) return fail(DEFER_HOST_E_IO, "%s: read error", path);
  if (b.size() < kFixed + 4 || memcmp(b.data(), kMagic, 8) != 0)
    return fail(DEFER_HOST_E_CHECKPOINT, "not a defer checkpoint");
  const size_t body = b.size() - 4;
  if (defer_host_crc32(b.data(), body) != get_u32(b.data() + body))
    return fail(DEFER_HOST_E_CHECKPOINT, "checksum mismatch (file corrupt)");
  const uint8_t* p = b.data() + 8;
  if (get_u32(p) != kVersion) return fail(DEFER_HOST_E_CHECKPOINT, "unsupported checkpoint version");
  p += 4;
  defer_host_checkpoint_header hh;
  memcpy(hh.model_signature, p, 32);
  memcpy(hh.base_seed, p + 32, 32);
  p += 64;
  const uint32_t tb = get_u32(p);
  memcpy(&hh.temperature, &tb, 4);
  hh.prompt_len = get_u32(p + 4);
  hh.rng_word_pos = get_u64(p + 8);
  const uint64_t hi = get_u64(p + 16);
  const uint64_t n = get_u64(p + 24);
  if (n > (body - kFixed) / 4 || body != kFixed + 4 * n)
    return fail(DEFER_HOST_E_CHECKPOINT, "length mismatch");
  if (hh.prompt_len > n) return fail(DEFER_HOST_E_CHECKPOINT, "prompt_len exceeds history length");
  if (hi != 0) return fail(DEFER_HOST_E_CHECKPOINT, "rng_word_pos beyond 2^64 words");
  *h = hh;
  if (history) {
    if (*n_history < n) return fail(DEFER_HOST_E_INVALID, "history buffer too small");
    for (uint64_t i = 0; i < n; ++i) history[i] = get_u32(b.data() + kFixed + 4 * i);
  }
  *n_history = (size_t)n;
  return DEFER_HOST_OK;
}
