// rng.cpp -- the word source of the sampler: ChaCha8 keyed by the session
// seed (engine.rs:51), and the numeric-seed expansion of engine.rs:19-21.
#include "defer_host.h"

namespace {

inline uint32_t rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

inline void quarter(uint32_t* x, int a, int b, int c, int d) {
  x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
  x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
  x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
  x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
}

// One ChaCha block (RFC 8439 section 2.3) with 8 rounds: constants, the
// 256-bit key, a 64-bit block counter in words 12-13 and a 64-bit stream id
// (0) in words 14-15.
void chacha8_block(const uint32_t key[8], uint64_t counter, uint32_t out[16]) {
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                    key[0], key[1], key[2], key[3], key[4], key[5], key[6], key[7],
                    (uint32_t)counter, (uint32_t)(counter >> 32), 0u, 0u};
  uint32_t x[16];
  for (int i = 0; i < 16; ++i) x[i] = s[i];
  for (int r = 0; r < 8; r += 2) {
    quarter(x, 0, 4, 8, 12);
    quarter(x, 1, 5, 9, 13);
    quarter(x, 2, 6, 10, 14);
    quarter(x, 3, 7, 11, 15);
    quarter(x, 0, 5, 10, 15);
    quarter(x, 1, 6, 11, 12);
    quarter(x, 2, 7, 8, 13);
    quarter(x, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

}  // namespace

extern "C" void defer_host_seed_from_u64(uint64_t state, uint8_t out[32]) {
  // PCG32 (XSH RR): advance, then output the rotated xorshift of the state.
  const uint64_t mul = 6364136223846793005ull, inc = 11634580027462260723ull;
  for (int i = 0; i < 8; ++i) {
    state = state * mul + inc;
    const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
    const uint32_t rot = (uint32_t)(state >> 59);
    const uint32_t v = (xs >> rot) | (xs << ((32 - rot) & 31));
    for (int k = 0; k < 4; ++k) out[4 * i + k] = (uint8_t)(v >> (8 * k));
  }
}

extern "C" void defer_host_chacha8_words(const uint8_t seed[32], uint64_t word_pos, size_t n,
                                         uint32_t* out) {
  uint32_t key[8];
  for (int i = 0; i < 8; ++i)
    key[i] = (uint32_t)seed[4 * i] | (uint32_t)seed[4 * i + 1] << 8 |
             (uint32_t)seed[4 * i + 2] << 16 | (uint32_t)seed[4 * i + 3] << 24;
  uint32_t blk[16];
  uint64_t have = ~0ull;
  for (size_t i = 0; i < n; ++i) {
    const uint64_t w = word_pos + i, b = w / 16;
    if (b != have) {
      chacha8_block(key, b, blk);
      have = b;
    }
    out[i] = blk[w % 16];
  }
}

extern "C" uint32_t defer_host_words_per_sample(float temperature) {
  return temperature == 0.0f ? 0u : 1u;
}
