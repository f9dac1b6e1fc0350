/*
 * abi_test.c -- the C ABI of include/defer_gpu.h exercised from C through
 * the static library (libdefer_gpu.a), as a Rust build.rs would link it,
 * and checked against the CPU oracle (oracle/oracle.c, linked in as the
 * checker only).
 *
 * Model: the reference's tiny test shape (synthetic.rs:12-29: vocab 256,
 * hidden 64, 2 layers, 4/2 heads, head_dim 16, ff 160, untied, theta 1e4)
 * with weights from a fixed xorshift stream, uniform in +-0.05.
 *
 * Checks (exit status 0 when all hold; each failure is printed):
 *   forward:  24 prompt positions, max |logit - oracle| <= 1e-3;
 *   generate: 16 greedy tokens equal the oracle's;
 *   sample:   T = 0.7 draws on the device equal sample_token on the same
 *             logits (sampler.rs:78-109) for 64 words, except at a CDF edge;
 *   replay:   the generated history rebuilds the cache with first_div -1 and
 *             logits bit-identical to the generating cache's;
 *   errors:   an out-of-range token gives DEFER_GPU_E_TOKEN and leaves the
 *             cache length unchanged (model.rs:417-419).
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/defer_gpu.h"
#include "../../oracle/oracle.h"

static int failures = 0;
#define CHECK(cond, ...)                 \
  do {                                   \
    if (!(cond)) {                       \
      fprintf(stderr, "FAIL: " __VA_ARGS__); \
      fprintf(stderr, "\n");             \
      ++failures;                        \
    }                                    \
  } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static float next_weight(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return ((float)(rng_state >> 40) / 16777216.0f - 0.5f) * 0.1f;
}

int main(void) {
  defer_gpu_config cfg = {256, 64, 160, 2, 4, 2, 16, 1e-5f, 10000.0f, 512, 0, 0, 0};
  const uint32_t V = cfg.vocab_size, h = cfg.hidden_size, ff = cfg.intermediate_size;
  const uint32_t q = cfg.num_heads * cfg.head_dim, kv = cfg.num_kv_heads * cfg.head_dim;
  const size_t nt = defer_gpu_model_tensor_count(&cfg);
  float** t = (float**)calloc(nt, sizeof(float*));
  size_t k = 0;
  size_t sizes[64];
  sizes[k++] = (size_t)V * h;
  for (uint32_t l = 0; l < cfg.num_layers; ++l) {
    sizes[k++] = h;               /* attn_norm */
    sizes[k++] = (size_t)q * h;   /* wq */
    sizes[k++] = (size_t)kv * h;  /* wk */
    sizes[k++] = (size_t)kv * h;  /* wv */
    sizes[k++] = (size_t)h * q;   /* wo */
    sizes[k++] = h;               /* ffn_norm */
    sizes[k++] = (size_t)ff * h;  /* gate */
    sizes[k++] = (size_t)ff * h;  /* up */
    sizes[k++] = (size_t)h * ff;  /* down */
  }
  sizes[k++] = h;                 /* norm */
  sizes[k++] = (size_t)V * h;     /* lm_head (untied) */
  if (k != nt) {
    fprintf(stderr, "FAIL: tensor count %zu, expected %zu\n", k, nt);
    return 1;
  }
  for (size_t i = 0; i < nt; ++i) {
    t[i] = (float*)malloc(sizes[i] * sizeof(float));
    for (size_t j = 0; j < sizes[i]; ++j) t[i][j] = (sizes[i] == h) ? 1.0f + next_weight() : next_weight();
  }

  defer_gpu_model* m = NULL;
  int rc = defer_gpu_model_create(&cfg, (const float* const*)t, nt, 0, &m);
  if (rc) {
    fprintf(stderr, "FAIL: model_create %d: %s\n", rc, defer_gpu_last_error());
    return 1;
  }
  oracle_config oc;
  memcpy(&oc, &cfg, sizeof(oc));
  oracle_model* om = oracle_model_create(&oc, (const float* const*)t, nt);
  oracle_cache* ocache = oracle_cache_create(om);
  defer_gpu_cache* c = NULL;
  rc = defer_gpu_cache_create(m, 256, &c);
  CHECK(rc == DEFER_GPU_OK, "cache_create %d", rc);

  /* forward */
  float* lg = (float*)malloc(V * sizeof(float));
  float* lo = (float*)malloc(V * sizeof(float));
  uint32_t prompt[24];
  double worst = 0.0;
  for (int i = 0; i < 24; ++i) {
    prompt[i] = (uint32_t)((i * 97 + 13) % V);
    rc = defer_gpu_forward(m, c, prompt[i], NULL, 0, lg, NULL);
    CHECK(rc == DEFER_GPU_OK, "forward %d: %s", rc, defer_gpu_last_error());
    oracle_forward_ext(om, ocache, prompt[i], NULL, 0, lo, NULL);
    for (uint32_t v = 0; v < V; ++v) worst = fmax(worst, fabs((double)lg[v] - (double)lo[v]));
  }
  CHECK(worst <= 1e-3, "forward max |dlogit| %.3e > 1e-3", worst);

  /* errors before any change */
  rc = defer_gpu_forward(m, c, V, NULL, 0, NULL, NULL);
  CHECK(rc == DEFER_GPU_E_TOKEN, "out-of-range token gave %d", rc);
  CHECK(defer_gpu_cache_len(c) == 24, "cache length %u after a token error", defer_gpu_cache_len(c));

  /* sample on the device vs sample_token on the same logits: identical */
  uint32_t differ = 0;
  rc = defer_gpu_last_logits(c, lg);
  CHECK(rc == DEFER_GPU_OK, "last_logits %d", rc);
  for (uint32_t w = 0; w < 64; ++w) {
    const uint32_t word = (w * 0x9E3779B9u) ^ 0x5bd1e995u;
    uint32_t tok = 0;
    rc = defer_gpu_sample(m, c, 0.7f, word, &tok);
    CHECK(rc == DEFER_GPU_OK, "sample %d", rc);
    const uint32_t ref = oracle_sample_token(lg, V, 0.7f, word);
    if (tok != ref) ++differ;
  }
  CHECK(differ == 0, "%u of 64 device draws differ from sample_token", differ);

  /* generate */
  uint32_t toks[16], otoks[16], n = 0;
  rc = defer_gpu_generate(m, c, 16, 0.0f, NULL, NULL, 0, toks, &n);
  CHECK(rc == DEFER_GPU_OK && n == 16, "generate %d, %u tokens", rc, n);
  uint8_t seed[32] = {0};
  oracle_cache* oc2 = oracle_cache_create(om);
  oracle_generate(om, oc2, seed, 0.0f, prompt, 24, 16, otoks, NULL);
  CHECK(memcmp(toks, otoks, sizeof(toks)) == 0, "greedy tokens differ from the oracle's");

  /* replay */
  uint32_t hist[40];
  memcpy(hist, prompt, sizeof(prompt));
  memcpy(hist + 24, toks, sizeof(toks));
  defer_gpu_cache* r = NULL;
  rc = defer_gpu_cache_create(m, 256, &r);
  CHECK(rc == DEFER_GPU_OK, "cache_create %d: %s", rc, defer_gpu_last_error());
  int64_t first_div = 0;
  uint32_t at = 0;
  rc = defer_gpu_replay(m, r, hist, 40, 24, 0.0f, NULL, &first_div, &at);
  CHECK(rc == DEFER_GPU_OK && first_div == -1, "replay %d, first_div %lld", rc, (long long)first_div);
  rc = defer_gpu_last_logits(r, lo);
  rc |= defer_gpu_last_logits(c, lg);
  CHECK(rc == DEFER_GPU_OK && memcmp(lo, lg, V * sizeof(float)) == 0,
        "replayed logits differ from the generating cache's");

  printf("abi_test (static library): forward max|dlogit| %.3e, %u/64 draws differ from "
         "sample_token, greedy and replay %s\n", worst, differ, failures ? "FAILED" : "ok");
  /* teardown: refused while a cache lives, then the device reset */
  rc = defer_gpu_shutdown();
  CHECK(rc == DEFER_GPU_E_INVALID, "shutdown with live handles gave %d", rc);
  defer_gpu_cache_destroy(r);
  defer_gpu_cache_destroy(c);
  defer_gpu_model_destroy(m);
  rc = defer_gpu_shutdown();
  CHECK(rc == DEFER_GPU_OK, "shutdown %d: %s", rc, defer_gpu_last_error());
  oracle_cache_destroy(oc2);
  oracle_cache_destroy(ocache);
  oracle_model_destroy(om);
  for (size_t i = 0; i < nt; ++i) free(t[i]);
  free(t);
  free(lg);
  free(lo);
  return failures ? 1 : 0;
}
