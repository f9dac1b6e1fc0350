// hash.cpp -- CRC-32 and SHA-256 for the WAL / checkpoint formats and the
// cache fingerprint (crc32.rs:4-28, sha256.rs:15-134, model.rs:233-242 of
// the reference).
#include <string.h>

#include <vector>

#include "common.h"
#include "defer_host.h"

namespace {

struct Crc32Table {
  uint32_t t[256];
  Crc32Table() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1u) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      t[i] = c;
    }
  }
};
const Crc32Table kCrc;

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

// FIPS 180-4 section 4.2.2: the first 32 bits of the fractional parts of the
// cube roots of the first 64 primes.
const uint32_t kK[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

void sha_block(uint32_t h[8], const uint8_t* p) {
  uint32_t w[64];
  for (int i = 0; i < 16; ++i)
    w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 |
           (uint32_t)p[4 * i + 3];
  for (int i = 16; i < 64; ++i) {
    const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
    const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
  for (int i = 0; i < 64; ++i) {
    const uint32_t t1 = k + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + kK[i] + w[i];
    const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
    k = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + t2;
  }
  h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += k;
}

}  // namespace

extern "C" uint32_t defer_host_crc32(const uint8_t* data, size_t n) {
  uint32_t c = 0xFFFFFFFFu;
  for (size_t i = 0; i < n; ++i) c = kCrc.t[(c ^ data[i]) & 0xFFu] ^ (c >> 8);
  return c ^ 0xFFFFFFFFu;
}

namespace dh {

Sha256::Sha256() : nbuf(0), total(0) {
  // FIPS 180-4 section 5.3.3 initial hash value.
  static const uint32_t h0[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
  memcpy(h, h0, sizeof(h));
}

void Sha256::update(const uint8_t* data, size_t n) {
  total += n;
  if (nbuf) {
    const size_t k = n < 64 - nbuf ? n : 64 - nbuf;
    memcpy(buf + nbuf, data, k);
    nbuf += k;
    data += k;
    n -= k;
    if (nbuf < 64) return;
    sha_block(h, buf);
    nbuf = 0;
  }
  for (; n >= 64; n -= 64, data += 64) sha_block(h, data);
  memcpy(buf, data, n);
  nbuf = n;
}

void Sha256::finish(uint8_t out[32]) {
  const uint64_t bits = total * 8u;
  uint8_t tail[128];
  memcpy(tail, buf, nbuf);
  tail[nbuf] = 0x80;
  const size_t tl = nbuf + 9 <= 64 ? 64 : 128;
  memset(tail + nbuf + 1, 0, tl - nbuf - 1);
  for (int k = 0; k < 8; ++k) tail[tl - 1 - k] = (uint8_t)(bits >> (8 * k));
  for (size_t o = 0; o < tl; o += 64) sha_block(h, tail + o);
  for (int k = 0; k < 8; ++k) {
    out[4 * k] = (uint8_t)(h[k] >> 24);
    out[4 * k + 1] = (uint8_t)(h[k] >> 16);
    out[4 * k + 2] = (uint8_t)(h[k] >> 8);
    out[4 * k + 3] = (uint8_t)h[k];
  }
}

}  // namespace dh

extern "C" void defer_host_sha256(const uint8_t* data, size_t n, uint8_t out[32]) {
  dh::Sha256 s;
  s.update(data, n);
  s.finish(out);
}

// KvCache::fingerprint (model.rs:233-242): SHA-256 of the length as a
// little-endian u64, then for each layer every key, then every value, as
// the little-endian bits of each f32 (positions 0..len, kv_dim per row).
extern "C" int defer_host_cache_fingerprint(const defer_gpu_cache* c, uint8_t out[32]) {
  if (!c || !out) return dh::fail(DEFER_HOST_E_INVALID, "null argument");
  uint32_t layers = 0, kv = 0;
  int rc = defer_gpu_cache_shape(c, &layers, &kv);
  if (rc) return dh::fail(DEFER_HOST_E_GPU, "defer_gpu error %d: %s", rc, defer_gpu_last_error());
  const uint64_t len = defer_gpu_cache_len(c);
  dh::Sha256 h;
  uint8_t lb[8];
  for (int k = 0; k < 8; ++k) lb[k] = (uint8_t)(len >> (8 * k));
  h.update(lb, 8);
  const size_t n = (size_t)len * kv;
  std::vector<float> keys(n), values(n);
  std::vector<uint8_t> bytes(4 * n);
  auto feed = [&](const std::vector<float>& v) {
    for (size_t i = 0; i < n; ++i) {
      uint32_t b;
      memcpy(&b, &v[i], 4);
      for (int k = 0; k < 4; ++k) bytes[4 * i + k] = (uint8_t)(b >> (8 * k));
    }
    h.update(bytes.data(), bytes.size());
  };
  for (uint32_t l = 0; l < layers; ++l) {
    rc = defer_gpu_cache_read(c, l, keys.data(), values.data());
    if (rc) return dh::fail(DEFER_HOST_E_GPU, "defer_gpu error %d: %s", rc, defer_gpu_last_error());
    feed(keys);
    feed(values);
  }
  h.finish(out);
  return DEFER_HOST_OK;
}
