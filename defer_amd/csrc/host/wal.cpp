// wal.cpp -- the write-ahead log of generated tokens (wal.rs:8-255 of the
// reference): a CRC-checked header with the context prefix, then one
// 29-byte CRC-checked record per sampled token. A torn or corrupt final
// record is dropped on read and cut away on resume.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "common.h"
#include "defer_host.h"

namespace dh {
std::string& last_error() {
  static thread_local std::string e;
  return e;
}
}  // namespace dh

using dh::fail;

extern "C" const char* defer_host_last_error(void) { return dh::last_error().c_str(); }

namespace {

const char kMagic[8] = {'D', 'E', 'F', 'E', 'R', 'W', 'A', 'L'};
const uint32_t kVersion = 1;
const uint8_t kTagToken = 0x01;
const size_t kRecord = 29;
const size_t kFixed = 8 + 4 + 32 + 32 + 4 + 4 + 16 + 4;  // header bytes before the prefix

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
  for (int i = 0; i < 4; ++i) b.push_back((uint8_t)(v >> (8 * i)));
}
void put_u128(std::vector<uint8_t>& b, uint64_t lo) {
  for (int i = 0; i < 8; ++i) b.push_back((uint8_t)(lo >> (8 * i)));
  for (int i = 0; i < 8; ++i) b.push_back(0);
}
uint32_t get_u32(const uint8_t* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
// u128 little-endian; the high half must be zero (positions fit 64 bits).
bool get_u128(const uint8_t* p, uint64_t* lo) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
  for (int i = 8; i < 16; ++i)
    if (p[i]) return false;
  *lo = v;
  return true;
}

std::vector<uint8_t> header_bytes(const defer_host_wal_header& h, const uint32_t* prefix,
                                  size_t n) {
  std::vector<uint8_t> b(kMagic, kMagic + 8);
  put_u32(b, kVersion);
  b.insert(b.end(), h.model_signature, h.model_signature + 32);
  b.insert(b.end(), h.base_seed, h.base_seed + 32);
  uint32_t tb;
  memcpy(&tb, &h.temperature, 4);
  put_u32(b, tb);
  put_u32(b, h.prompt_len);
  put_u128(b, h.start_rng_word_pos);
  put_u32(b, (uint32_t)n);
  for (size_t i = 0; i < n; ++i) put_u32(b, prefix[i]);
  put_u32(b, defer_host_crc32(b.data(), b.size()));
  return b;
}

bool write_all(int fd, const uint8_t* p, size_t n) {
  while (n) {
    const ssize_t w = ::write(fd, p, n);
    if (w < 0) {
      if (errno == EINTR) continue;
      return false;
    }
    p += w;
    n -= (size_t)w;
  }
  return true;
}

struct Parsed {
  defer_host_wal_header h;
  std::vector<uint32_t> prefix;
  std::vector<uint32_t> tokens;
  uint64_t last_rng;
  size_t valid_len;
  bool torn;
};

int parse(const std::vector<uint8_t>& b, Parsed* out) {
  if (b.size() < kFixed + 4 || memcmp(b.data(), kMagic, 8) != 0)
    return fail(DEFER_HOST_E_WAL, "not a defer WAL");
  const uint8_t* p = b.data() + 8;
  if (get_u32(p) != kVersion) return fail(DEFER_HOST_E_WAL, "unsupported WAL version");
  p += 4;
  Parsed r;
  memcpy(r.h.model_signature, p, 32);
  p += 32;
  memcpy(r.h.base_seed, p, 32);
  p += 32;
  const uint32_t tb = get_u32(p);
  memcpy(&r.h.temperature, &tb, 4);
  p += 4;
  r.h.prompt_len = get_u32(p);
  p += 4;
  if (!get_u128(p, &r.h.start_rng_word_pos))
    return fail(DEFER_HOST_E_WAL, "rng word position beyond 64 bits");
  p += 16;
  const uint32_t n = get_u32(p);
  p += 4;
  const size_t header_end = kFixed + 4 * (size_t)n;
  if (b.size() < header_end + 4) return fail(DEFER_HOST_E_WAL, "truncated WAL header");
  r.prefix.resize(n);
  for (uint32_t i = 0; i < n; ++i) r.prefix[i] = get_u32(b.data() + kFixed + 4 * i);
  if (defer_host_crc32(b.data(), header_end) != get_u32(b.data() + header_end))
    return fail(DEFER_HOST_E_WAL, "WAL header checksum mismatch");
  if (r.h.prompt_len > n) return fail(DEFER_HOST_E_WAL, "prompt_len exceeds prefix length");
  size_t off = header_end + 4;
  uint32_t expect_step = n;
  uint64_t expect_rng = r.h.start_rng_word_pos;
  const uint64_t wps = defer_host_words_per_sample(r.h.temperature);
  r.torn = false;
  r.last_rng = r.h.start_rng_word_pos;
  while (off < b.size()) {
    if (b.size() - off < kRecord) {
      r.torn = true;
      break;
    }
    const uint8_t* rec = b.data() + off;
    if (rec[0] != kTagToken || defer_host_crc32(rec, 25) != get_u32(rec + 25)) {
      r.torn = true;
      break;
    }
    const uint32_t step = get_u32(rec + 1), token = get_u32(rec + 5);
    uint64_t rng = 0;
    const bool fits = get_u128(rec + 9, &rng);
    expect_rng += wps;
    if (!fits || step != expect_step || rng != expect_rng)
      return fail(DEFER_HOST_E_WAL,
                  "record %zu is inconsistent (step %u / rng %llu, expected %u / %llu)",
                  r.tokens.size(), step, (unsigned long long)rng, expect_step,
                  (unsigned long long)expect_rng);
    ++expect_step;
    r.tokens.push_back(token);
    r.last_rng = rng;
    off += kRecord;
  }
  r.valid_len = off;
  *out = std::move(r);
  return DEFER_HOST_OK;
}

int read_file(const char* path, std::vector<uint8_t>* b) {
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(DEFER_HOST_E_IO, "open %s: %s", path, strerror(errno));
  uint8_t buf[65536];
  for (;;) {
    const ssize_t r = ::read(fd, buf, sizeof(buf));
    if (r < 0) {
      if (errno == EINTR) continue;
      ::close(fd);
      return fail(DEFER_HOST_E_IO, "read %s: %s", path, strerror(errno));
    }
    if (r == 0) break;
    b->insert(b->end(), buf, buf + r);
  }
  ::close(fd);
  return DEFER_HOST_OK;
}

}  // namespace

struct defer_host_wal {
  int fd;
  uint32_t next_step;
  bool durable;
};

extern "C" int defer_host_wal_create(const char* path, const defer_host_wal_header* h,
                                     const uint32_t* prefix, size_t n_prefix, int durable,
                                     defer_host_wal** out) {
  if (!path || !h || !out || (n_prefix && !prefix)) return fail(DEFER_HOST_E_INVALID, "null argument");
  const int fd = ::open(path, O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return fail(DEFER_HOST_E_IO, "create %s: %s", path, strerror(errno));
  const std::vector<uint8_t> b = header_bytes(*h, prefix, n_prefix);
  if (!write_all(fd, b.data(), b.size()) || ::fsync(fd) != 0) {
    ::close(fd);
    return fail(DEFER_HOST_E_IO, "write %s: %s", path, strerror(errno));
  }
  *out = new defer_host_wal{fd, (uint32_t)n_prefix, durable != 0};
  return DEFER_HOST_OK;
}

extern "C" int defer_host_wal_resume(const char* path, int durable, defer_host_wal** out) {
  if (!path || !out) return fail(DEFER_HOST_E_INVALID, "null argument");
  std::vector<uint8_t> b;
  int rc = read_file(path, &b);
  if (rc) return rc;
  Parsed p;
  if ((rc = parse(b, &p))) return rc;
  const int fd = ::open(path, O_WRONLY);
  if (fd < 0) return fail(DEFER_HOST_E_IO, "open %s: %s", path, strerror(errno));
  if (::ftruncate(fd, (off_t)p.valid_len) != 0 || ::lseek(fd, 0, SEEK_END) < 0 || ::fsync(fd) != 0) {
    ::close(fd);
    return fail(DEFER_HOST_E_IO, "truncate %s: %s", path, strerror(errno));
  }
  *out = new defer_host_wal{fd, (uint32_t)(p.prefix.size() + p.tokens.size()), durable != 0};
  return DEFER_HOST_OK;
}

extern "C" int defer_host_wal_append(defer_host_wal* w, uint32_t token, uint64_t rng_word_pos) {
  if (!w) return fail(DEFER_HOST_E_INVALID, "null WAL");
  std::vector<uint8_t> rec;
  rec.push_back(kTagToken);
  put_u32(rec, w->next_step);
  put_u32(rec, token);
  put_u128(rec, rng_word_pos);
  put_u32(rec, defer_host_crc32(rec.data(), 25));
  if (!write_all(w->fd, rec.data(), rec.size()))
    return fail(DEFER_HOST_E_IO, "WAL append: %s", strerror(errno));
  if (w->durable && ::fdatasync(w->fd) != 0)
    return fail(DEFER_HOST_E_IO, "WAL sync: %s", strerror(errno));
  ++w->next_step;
  return DEFER_HOST_OK;
}

extern "C" uint32_t defer_host_wal_next_step(const defer_host_wal* w) { return w ? w->next_step : 0; }

extern "C" void defer_host_wal_close(defer_host_wal* w) {
  if (!w) return;
  ::close(w->fd);
  delete w;
}

extern "C" int defer_host_wal_read(const char* path, defer_host_wal_header* h, uint32_t* history,
                                   size_t* n_history, uint64_t* rng_word_pos, int* torn_tail) {
  if (!path || !n_history) return fail(DEFER_HOST_E_INVALID, "null argument");
  std::vector<uint8_t> b;
  int rc = read_file(path, &b);
  if (rc) return rc;
  Parsed p;
  if ((rc = parse(b, &p))) return rc;
  const size_t n = p.prefix.size() + p.tokens.size();
  if (history) {
    if (*n_history < n) return fail(DEFER_HOST_E_INVALID, "history buffer too small (%zu < %zu)", *n_history, n);
    for (size_t i = 0; i < p.prefix.size(); ++i) history[i] = p.prefix[i];
    for (size_t i = 0; i < p.tokens.size(); ++i) history[p.prefix.size() + i] = p.tokens[i];
  }
  *n_history = n;
  if (h) *h = p.h;
  if (rng_word_pos) *rng_word_pos = p.last_rng;
  if (torn_tail) *torn_tail = p.torn ? 1 : 0;
  return DEFER_HOST_OK;
}
