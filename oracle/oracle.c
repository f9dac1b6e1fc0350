/*
 * oracle.c -- CPU oracle for defer's per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY (the checker for the HIP path; the product never
 * links it). Each function restates one loop of the reference, cited as
 * file:line under the reference's src/. Build flags (oracle/Makefile):
 * -O2 -ffp-contract=off, no fast-math, so every `a * b + c` below is a
 * rounded product followed by a rounded add, exactly like the Rust code.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ ops.rs */

/* ops.rs:9-22 */
void oracle_matmul_sequential(float* out, const float* a, const float* b, size_t m, size_t n,
                              size_t k) {
  for (size_t i = 0; i < m; ++i) {
    for (size_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (size_t p = 0; p < k; ++p) sum += a[i * k + p] * b[p * n + j];
      out[i * n + j] = sum;
    }
  }
}

/* ops.rs:26-71: four independent rows per pass, each a single accumulator in
 * index order; the bias is added after the sum. */
void oracle_linear(float* out, const float* x, const float* w, const float* bias, size_t in_dim,
                   size_t out_dim) {
  const size_t blocks = out_dim / 4;
  for (size_t blk = 0; blk < blocks; ++blk) {
    const size_t o = blk * 4;
    const float* r0 = w + o * in_dim;
    const float* r1 = w + (o + 1) * in_dim;
    const float* r2 = w + (o + 2) * in_dim;
    const float* r3 = w + (o + 3) * in_dim;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (size_t i = 0; i < in_dim; ++i) {
      const float xi = x[i];
      s0 += r0[i] * xi;
      s1 += r1[i] * xi;
      s2 += r2[i] * xi;
      s3 += r3[i] * xi;
    }
    if (bias) {
      s0 += bias[o];
      s1 += bias[o + 1];
      s2 += bias[o + 2];
      s3 += bias[o + 3];
    }
    out[o] = s0;
    out[o + 1] = s1;
    out[o + 2] = s2;
    out[o + 3] = s3;
  }
  for (size_t o = blocks * 4; o < out_dim; ++o) {
    const float* row = w + o * in_dim;
    float sum = 0.0f;
    for (size_t i = 0; i < in_dim; ++i) sum += row[i] * x[i];
    if (bias) sum += bias[o];
    out[o] = sum;
  }
}

/* ops.rs:74-81 */
float oracle_dot(const float* a, const float* b, size_t n) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += a[i] * b[i];
  return sum;
}

/* ops.rs:84-95 */
void oracle_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

/* ops.rs:98-118 */
void oracle_layernorm(float* out, const float* x, const float* w, const float* b, size_t n,
                      float eps) {
  const float nf = (float)n;
  float mean = 0.0f;
  for (size_t i = 0; i < n; ++i) mean += x[i];
  mean /= nf;
  float var = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float d = x[i] - mean;
    var += d * d;
  }
  var /= nf;
  const float inv = 1.0f / sqrtf(var + eps);
  for (size_t i = 0; i < n; ++i) out[i] = (x[i] - mean) * inv * w[i] + b[i];
}

/* ops.rs:120-122 */
float oracle_silu(float x) { return x / (1.0f + expf(-x)); }

/* ops.rs:125-128 (tanh approximation) */
float oracle_gelu(float x) {
  const float c = 0.7978846f;
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

/* ops.rs:130-140 */
void oracle_silu_inplace(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = oracle_silu(x[i]);
}
void oracle_gelu_inplace(float* x, size_t n) {
  for (size_t i = 0; i < n; ++i) x[i] = oracle_gelu(x[i]);
}

/* ops.rs:143-156 */
void oracle_add_inplace(float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) a[i] += b[i];
}
void oracle_mul_inplace(float* a, const float* b, size_t n) {
  for (size_t i = 0; i < n; ++i) a[i] *= b[i];
}

/* ops.rs:159-178 */
void oracle_softmax_inplace(float* x, size_t n) {
  if (n == 0) return;
  float max = -INFINITY;
  for (size_t i = 0; i < n; ++i)
    if (x[i] > max) max = x[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - max);
    sum += x[i];
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) x[i] *= inv;
}

/* ---------------------------------------------------------------- model.rs */

typedef struct {
  const float *attn_norm, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *ffn_norm, *w_gate, *w_up, *w_down;
} oracle_layer;

struct oracle_model {
  oracle_config cfg;
  const float* embed;
  oracle_layer* layers;
  const float* norm;
  const float* lm_head; /* NULL when tied (model.rs:343-347, 516) */
  float* inv_freq;      /* model.rs:348-353 */
};

struct oracle_cache {
  uint32_t num_layers, kv_dim, capacity, len;
  float** keys;   /* [layer][len * kv_dim], model.rs:182-190 */
  float** values;
};

size_t oracle_model_tensor_count(const oracle_config* c) {
  const size_t per_layer = c->has_bias ? 12 : 9;
  return 1 + (size_t)c->num_layers * per_layer + 1 + (c->tie_word_embeddings ? 0 : 1);
}

/* model.rs:301-363 (tensor order of model.rs:322-347) */
oracle_model* oracle_model_create(const oracle_config* cfg, const float* const* t,
                                  size_t n_tensors) {
  if (n_tensors != oracle_model_tensor_count(cfg)) return NULL;
  if (cfg->num_kv_heads == 0 || cfg->num_heads % cfg->num_kv_heads != 0) return NULL;
  if (cfg->head_dim % 2 != 0) return NULL;
  oracle_model* m = (oracle_model*)calloc(1, sizeof(oracle_model));
  m->cfg = *cfg;
  m->layers = (oracle_layer*)calloc(cfg->num_layers, sizeof(oracle_layer));
  size_t k = 0;
  m->embed = t[k++];
  for (uint32_t l = 0; l < cfg->num_layers; ++l) {
    oracle_layer* L = &m->layers[l];
    L->attn_norm = t[k++];
    L->wq = t[k++];
    L->bq = cfg->has_bias ? t[k++] : NULL;
    L->wk = t[k++];
    L->bk = cfg->has_bias ? t[k++] : NULL;
    L->wv = t[k++];
    L->bv = cfg->has_bias ? t[k++] : NULL;
    L->wo = t[k++];
    L->ffn_norm = t[k++];
    L->w_gate = t[k++];
    L->w_up = t[k++];
    L->w_down = t[k++];
  }
  m->norm = t[k++];
  m->lm_head = cfg->tie_word_embeddings ? NULL : t[k++];
  const uint32_t half = cfg->head_dim / 2;
  m->inv_freq = (float*)calloc(half ? half : 1, sizeof(float));
  for (uint32_t i = 0; i < half; ++i) {
    const double exponent = (double)(2 * i) / (double)cfg->head_dim;
    m->inv_freq[i] = (float)(1.0 / pow((double)cfg->rope_theta, exponent));
  }
  return m;
}

void oracle_model_destroy(oracle_model* m) {
  if (!m) return;
  free(m->layers);
  free(m->inv_freq);
  free(m);
}

/* KvCache::new (model.rs:193-200), preallocated to max_seq_len. */
oracle_cache* oracle_cache_create(const oracle_model* m) {
  const oracle_config* c = &m->cfg;
  oracle_cache* kc = (oracle_cache*)calloc(1, sizeof(oracle_cache));
  kc->num_layers = c->num_layers;
  kc->kv_dim = c->num_kv_heads * c->head_dim;
  kc->capacity = c->max_seq_len;
  kc->keys = (float**)calloc(c->num_layers, sizeof(float*));
  kc->values = (float**)calloc(c->num_layers, sizeof(float*));
  for (uint32_t l = 0; l < c->num_layers; ++l) {
    kc->keys[l] = (float*)malloc((size_t)kc->capacity * kc->kv_dim * sizeof(float));
    kc->values[l] = (float*)malloc((size_t)kc->capacity * kc->kv_dim * sizeof(float));
  }
  return kc;
}

void oracle_cache_destroy(oracle_cache* c) {
  if (!c) return;
  for (uint32_t l = 0; l < c->num_layers; ++l) {
    free(c->keys[l]);
    free(c->values[l]);
  }
  free(c->keys);
  free(c->values);
  free(c);
}

uint32_t oracle_cache_len(const oracle_cache* c) { return c->len; }

/* model.rs:211-220 */
void oracle_cache_truncate(oracle_cache* c, uint32_t n) {
  if (n < c->len) c->len = n;
}

void oracle_cache_read(const oracle_cache* c, uint32_t layer, float* keys, float* values) {
  const size_t n = (size_t)c->len * c->kv_dim;
  memcpy(keys, c->keys[layer], n * sizeof(float));
  memcpy(values, c->values[layer], n * sizeof(float));
}

/* Half-split RoPE, model.rs:446-456 */
static void rope(float* v, uint32_t n_heads, uint32_t hd, const float* cs, const float* sn) {
  const uint32_t half = hd / 2;
  for (uint32_t h = 0; h < n_heads; ++h) {
    const uint32_t base = h * hd;
    for (uint32_t i = 0; i < half; ++i) {
      const float x0 = v[base + i];
      const float x1 = v[base + i + half];
      v[base + i] = x0 * cs[i] - x1 * sn[i];
      v[base + i + half] = x1 * cs[i] + x0 * sn[i];
    }
  }
}

/* Model::forward_ext, model.rs:394-520 */
int oracle_forward_ext(const oracle_model* m, oracle_cache* kc, uint32_t token,
                       const uint32_t* masked, size_t n_masked, float* logits_out,
                       float* trace_out) {
  const oracle_config* c = &m->cfg;
  const uint32_t pos = kc->len;
  if (token >= c->vocab_size) return ORACLE_E_TOKEN;      /* 417-419 */
  if (pos >= c->max_seq_len) return ORACLE_E_CONTEXT;      /* 420-422 */
  const uint32_t h = c->hidden_size, hd = c->head_dim, half = hd / 2;
  const uint32_t nh = c->num_heads, nkv = c->num_kv_heads, group = nh / nkv;
  const uint32_t qd = nh * hd, kvd = nkv * hd, ff = c->intermediate_size;
  const float scale = 1.0f / sqrtf((float)hd);

  /* 403-413: skip mask (masks >= pos are ignored) */
  unsigned char* skip = NULL;
  if (n_masked) {
    skip = (unsigned char*)calloc(pos + 1, 1);
    for (size_t i = 0; i < n_masked; ++i)
      if (masked[i] < pos) skip[masked[i]] = 1;
  }

  float* x = (float*)malloc(h * sizeof(float));
  float* xb = (float*)malloc(h * sizeof(float));
  float* q = (float*)malloc(qd * sizeof(float));
  float* k = (float*)malloc(kvd * sizeof(float));
  float* v = (float*)malloc(kvd * sizeof(float));
  float* att = (float*)malloc(qd * sizeof(float));
  float* scores = (float*)malloc((size_t)(pos + 1) * sizeof(float));
  float* gate = (float*)malloc(ff * sizeof(float));
  float* up = (float*)malloc(ff * sizeof(float));
  float* cs = (float*)malloc((half ? half : 1) * sizeof(float));
  float* sn = (float*)malloc((half ? half : 1) * sizeof(float));

  memcpy(x, m->embed + (size_t)token * h, h * sizeof(float)); /* 428 */
  for (uint32_t i = 0; i < half; ++i) {                       /* 438-445 */
    const float angle = (float)pos * m->inv_freq[i];
    cs[i] = cosf(angle);
    sn[i] = sinf(angle);
  }

  for (uint32_t l = 0; l < c->num_layers; ++l) {
    const oracle_layer* L = &m->layers[l];
    oracle_rmsnorm(xb, x, L->attn_norm, h, c->rms_norm_eps); /* 460 */
    oracle_linear(q, xb, L->wq, L->bq, h, qd);                /* 461-463 */
    oracle_linear(k, xb, L->wk, L->bk, h, kvd);
    oracle_linear(v, xb, L->wv, L->bv, h, kvd);
    rope(q, nh, hd, cs, sn); /* 464-465 */
    rope(k, nkv, hd, cs, sn);
    memcpy(kc->keys[l] + (size_t)pos * kvd, k, kvd * sizeof(float)); /* 466-467 */
    memcpy(kc->values[l] + (size_t)pos * kvd, v, kvd * sizeof(float));
    const float* keys = kc->keys[l];
    const float* vals = kc->values[l];

    for (uint32_t hh = 0; hh < nh; ++hh) { /* 471-497 */
      const uint32_t kvh = hh / group;
      const float* qh = q + hh * hd;
      for (uint32_t t = 0; t <= pos; ++t)
        scores[t] = oracle_dot(qh, keys + (size_t)t * kvd + kvh * hd, hd) * scale;
      if (skip)
        for (uint32_t t = 0; t < pos; ++t)
          if (skip[t]) scores[t] = -INFINITY;
      oracle_softmax_inplace(scores, pos + 1);
      if (trace_out)
        memcpy(trace_out + ((size_t)l * nh + hh) * (pos + 1), scores,
               (size_t)(pos + 1) * sizeof(float));
      float* out = att + hh * hd;
      for (uint32_t d = 0; d < hd; ++d) {
        float acc = 0.0f;
        for (uint32_t t = 0; t <= pos; ++t) acc += scores[t] * vals[(size_t)t * kvd + kvh * hd + d];
        out[d] = acc;
      }
    }
    oracle_linear(xb, att, L->wo, NULL, qd, h); /* 498-499 */
    oracle_add_inplace(x, xb, h);

    oracle_rmsnorm(xb, x, L->ffn_norm, h, c->rms_norm_eps); /* 502-511 */
    oracle_linear(gate, xb, L->w_gate, NULL, h, ff);
    oracle_linear(up, xb, L->w_up, NULL, h, ff);
    if (c->activation == 0)
      oracle_silu_inplace(gate, ff);
    else
      oracle_gelu_inplace(gate, ff);
    oracle_mul_inplace(gate, up, ff);
    oracle_linear(xb, gate, L->w_down, NULL, ff, h);
    oracle_add_inplace(x, xb, h);
  }
  kc->len += 1; /* 513 */

  if (logits_out) { /* 515-519 */
    oracle_rmsnorm(xb, x, m->norm, h, c->rms_norm_eps);
    const float* head = m->lm_head ? m->lm_head : m->embed;
    oracle_linear(logits_out, xb, head, NULL, h, c->vocab_size);
  }

  free(skip);
  free(x);
  free(xb);
  free(q);
  free(k);
  free(v);
  free(att);
  free(scores);
  free(gate);
  free(up);
  free(cs);
  free(sn);
  return ORACLE_OK;
}

/* -------------------------------------------------------------- sampler.rs */

/* sampler.rs:24-40 */
uint32_t oracle_argmax(const float* logits, size_t n) {
  size_t best = 0;
  float best_val = -INFINITY;
  int found = 0;
  for (size_t i = 0; i < n; ++i) {
    const float v = logits[i];
    if (isnan(v)) continue;
    if (!found || v > best_val) {
      best = i;
      best_val = v;
      found = 1;
    }
  }
  return (uint32_t)best;
}

/* sampler.rs:43-75 */
void oracle_softmax_with_temperature(const float* logits, size_t n, float temperature,
                                     float* probs) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; ++i) {
    const float s = logits[i] / temperature;
    if (s > max) max = s;
  }
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float s = logits[i] / temperature;
    const float p = isnan(s) ? 0.0f : expf(s - max);
    probs[i] = p;
    sum += p;
  }
  if (!(sum > 0.0f) || !isfinite(sum)) {
    const uint32_t best = oracle_argmax(logits, n);
    for (size_t i = 0; i < n; ++i) probs[i] = 0.0f;
    if (n) probs[best] = 1.0f;
    return;
  }
  const float inv = 1.0f / sum;
  for (size_t i = 0; i < n; ++i) probs[i] *= inv;
}

/* rand 0.8 `Standard` for f32: the top 24 bits of one u32, times 2^-24. */
float oracle_unit_f32(uint32_t word) { return (float)(word >> 8) * (1.0f / 16777216.0f); }

/* The CDF scan of sampler.rs:94-108 over normalised probabilities: the
 * first i with p_i > 0 and r < the sequential float sum of p_0..p_i, else the
 * last i with p_i > 0 (0 if none). *lo / *hi (nullable): the cumulative sum
 * before and after the returned index, in that same float arithmetic. */
static uint32_t cdf_scan(const float* probs, size_t n, float r, float* lo, float* hi) {
  float cumulative = 0.0f;
  size_t last_nonzero = 0;
  float before_last = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    const float p = probs[i];
    if (p > 0.0f) {
      const float before = cumulative;
      last_nonzero = i;
      before_last = before;
      cumulative += p;
      if (r < cumulative) {
        if (lo) *lo = before;
        if (hi) *hi = cumulative;
        return (uint32_t)i;
      }
    }
  }
  if (lo) *lo = before_last;
  if (hi) *hi = cumulative;
  return (uint32_t)last_nonzero;
}

/* sampler.rs:78-109 */
uint32_t oracle_sample_token(const float* logits, size_t n, float temperature, uint32_t word) {
  if (temperature == 0.0f) return oracle_argmax(logits, n);
  float* probs = (float*)malloc(n * sizeof(float));
  oracle_softmax_with_temperature(logits, n, temperature, probs);
  const uint32_t tok = cdf_scan(probs, n, oracle_unit_f32(word), NULL, NULL);
  free(probs);
  return tok;
}

/* sample_token at T > 0 plus how close the draw was: *margin = min(r - lo,
 * hi - r) with lo / hi the cumulative sums around the chosen token in the
 * reference's own arithmetic (sampler.rs:52-75 sums and normalises
 * sequentially in float; 94-106 accumulates the CDF the same way). */
uint32_t oracle_sample_margin(const float* logits, size_t n, float temperature, uint32_t word,
                              float* margin) {
  float* probs = (float*)malloc(n * sizeof(float));
  oracle_softmax_with_temperature(logits, n, temperature, probs);
  const float r = oracle_unit_f32(word);
  float lo = 0.0f, hi = 0.0f;
  const uint32_t tok = cdf_scan(probs, n, r, &lo, &hi);
  free(probs);
  const float a = r - lo, b = hi - r;
  *margin = a < b ? a : b;
  return tok;
}

/* sampler.rs:58-108 on un-normalised terms p (what softmax_with_temperature
 * forms before its sum, 55-57): the sequential float total, inv = 1/total,
 * p_i * inv, then the CDF scan for the draw of `word`. Returns the index;
 * *total gets the sum. Degenerate totals are the caller's business. */
uint32_t oracle_sample_terms(const float* p, size_t n, uint32_t word, float* total) {
  float sum = 0.0f;
  for (size_t i = 0; i < n; ++i) sum += p[i];
  *total = sum;
  const float inv = 1.0f / sum;
  float* probs = (float*)malloc(n * sizeof(float));
  for (size_t i = 0; i < n; ++i) probs[i] = p[i] * inv;
  const uint32_t tok = cdf_scan(probs, n, oracle_unit_f32(word), NULL, NULL);
  free(probs);
  return tok;
}

/* The reference's f32::exp (the platform libm's expf) over an array. */
void oracle_expf_array(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
}

/* ----------------------------------------- rand_chacha 0.3.1 / rand_core 0.6.4 */

static uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

#define QR(a, b, c, d)            \
  do {                            \
    x[a] += x[b];                 \
    x[d] = rotl32(x[d] ^ x[a], 16); \
    x[c] += x[d];                 \
    x[b] = rotl32(x[b] ^ x[c], 12); \
    x[a] += x[b];                 \
    x[d] = rotl32(x[d] ^ x[a], 8);  \
    x[c] += x[d];                 \
    x[b] = rotl32(x[b] ^ x[c], 7);  \
  } while (0)

/* ChaCha block function (Bernstein; RFC 8439 2.3) with a 64-bit block counter
 * in words 12-13 and a 64-bit stream id in words 14-15, as rand_chacha lays
 * them out. `rounds` is 8 for ChaCha8Rng. */
void oracle_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds,
                         uint32_t out[16]) {
  uint32_t s[16];
  s[0] = 0x61707865u;
  s[1] = 0x3320646eu;
  s[2] = 0x79622d32u;
  s[3] = 0x6b206574u;
  for (int i = 0; i < 8; ++i) s[4 + i] = key[i];
  s[12] = (uint32_t)counter;
  s[13] = (uint32_t)(counter >> 32);
  s[14] = (uint32_t)stream;
  s[15] = (uint32_t)(stream >> 32);
  uint32_t x[16];
  memcpy(x, s, sizeof(x));
  for (int r = 0; r < rounds; r += 2) {
    QR(0, 4, 8, 12);
    QR(1, 5, 9, 13);
    QR(2, 6, 10, 14);
    QR(3, 7, 11, 15);
    QR(0, 5, 10, 15);
    QR(1, 6, 11, 12);
    QR(2, 7, 8, 13);
    QR(3, 4, 9, 14);
  }
  for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

/* PCG32 (O'Neill, PCG-XSH-RR 64/32): the LCG step with the standard
 * multiplier, and the output permutation of a state. */
uint64_t oracle_pcg32_step(uint64_t state, uint64_t inc) {
  return state * 6364136223846793005ull + inc;
}
uint32_t oracle_pcg32_output(uint64_t state) {
  const uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
  const uint32_t rot = (uint32_t)(state >> 59);
  return (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
}

/* rand_core 0.6.4 SeedableRng::seed_from_u64: PCG32 output, 4 bytes at a
 * time, state advanced before each output (the increment is rand_core's
 * constant). */
void oracle_seed_from_u64(uint64_t state, uint8_t out[32]) {
  const uint64_t inc = 11634580027462260723ull;
  for (int chunk = 0; chunk < 8; ++chunk) {
    state = oracle_pcg32_step(state, inc);
    const uint32_t v = oracle_pcg32_output(state);
    out[chunk * 4 + 0] = (uint8_t)v;
    out[chunk * 4 + 1] = (uint8_t)(v >> 8);
    out[chunk * 4 + 2] = (uint8_t)(v >> 16);
    out[chunk * 4 + 3] = (uint8_t)(v >> 24);
  }
}

static void seed_key(const uint8_t seed[32], uint32_t key[8]) {
  for (int i = 0; i < 8; ++i)
    key[i] = (uint32_t)seed[4 * i] | ((uint32_t)seed[4 * i + 1] << 8) |
             ((uint32_t)seed[4 * i + 2] << 16) | ((uint32_t)seed[4 * i + 3] << 24);
}

uint32_t oracle_chacha8_word(const uint8_t seed[32], uint64_t index) {
  uint32_t key[8], blk[16];
  seed_key(seed, key);
  oracle_chacha_block(key, index / 16, 0, 8, blk);
  return blk[index % 16];
}

/* Sequential ChaCha8 word stream (ChaCha8Rng::next_u32 / get_word_pos). */
typedef struct {
  uint32_t key[8];
  uint32_t buf[16];
  uint64_t word_pos;
} chacha8_stream;

static uint32_t chacha8_next(chacha8_stream* st) {
  if (st->word_pos % 16 == 0) oracle_chacha_block(st->key, st->word_pos / 16, 0, 8, st->buf);
  return st->buf[st->word_pos++ % 16];
}

/* ---------------------------------------------------------------- engine.rs */

/* Session::new / prompt / generate (engine.rs:44-137) */
int64_t oracle_generate(const oracle_model* m, oracle_cache* c, const uint8_t seed[32],
                        float temperature, const uint32_t* prompt, size_t n_prompt, size_t n_gen,
                        uint32_t* out_tokens, float* last_logits) {
  if (!(temperature >= 0.0f && isfinite(temperature))) return -3;
  const size_t V = m->cfg.vocab_size;
  float* logits = (float*)malloc(V * sizeof(float));
  chacha8_stream st;
  seed_key(seed, st.key);
  st.word_pos = 0;
  int have_logits = 0;
  for (size_t i = 0; i < n_prompt; ++i) { /* prompt -> feed (62-71, 90-102) */
    const int e = oracle_forward_ext(m, c, prompt[i], NULL, 0, logits, NULL);
    if (e) {
      free(logits);
      return -(int64_t)(10 + e);
    }
    have_logits = 1;
  }
  for (size_t g = 0; g < n_gen; ++g) { /* step = sample + feed (104-117) */
    if (!have_logits) {
      free(logits);
      return -4;
    }
    const uint32_t word = temperature == 0.0f ? 0u : chacha8_next(&st);
    const uint32_t tok = oracle_sample_token(logits, V, temperature, word);
    out_tokens[g] = tok;
    const int e = oracle_forward_ext(m, c, tok, NULL, 0, logits, NULL);
    if (e) {
      free(logits);
      return -(int64_t)(10 + e);
    }
  }
  if (last_logits && have_logits) memcpy(last_logits, logits, V * sizeof(float));
  free(logits);
  return (int64_t)st.word_pos;
}

/* Session::checkout's replay (engine.rs:261-271) */
int64_t oracle_checkout(const oracle_model* m, oracle_cache* c, const uint8_t seed[32],
                        float temperature, const uint32_t* history, size_t n_history,
                        size_t prompt_len, uint32_t* sampled_at_div, float* last_logits) {
  if (!(temperature >= 0.0f && isfinite(temperature))) return -3;
  if (prompt_len > n_history) return -5;
  const size_t V = m->cfg.vocab_size;
  float* logits = (float*)malloc(V * sizeof(float));
  chacha8_stream st;
  seed_key(seed, st.key);
  st.word_pos = 0;
  int have_logits = 0;
  for (size_t i = 0; i < n_history; ++i) {
    if (i >= prompt_len) {
      if (!have_logits) {
        free(logits);
        return -4;
      }
      const uint32_t word = temperature == 0.0f ? 0u : chacha8_next(&st);
      const uint32_t sampled = oracle_sample_token(logits, V, temperature, word);
      if (sampled != history[i]) {
        if (sampled_at_div) *sampled_at_div = sampled;
        free(logits);
        return (int64_t)i;
      }
    }
    const int e = oracle_forward_ext(m, c, history[i], NULL, 0, logits, NULL);
    if (e) {
      free(logits);
      return -(int64_t)(10 + e);
    }
    have_logits = 1;
  }
  if (last_logits && have_logits) memcpy(last_logits, logits, V * sizeof(float));
  free(logits);
  return -1;
}

/* attribution.rs:116-148 (ValueNorms::sync, the loop body per layer) */
void oracle_value_norms(const float* wo, const float* vals, uint32_t hidden, uint32_t nh,
                        uint32_t nkv, uint32_t hd, uint32_t t0, uint32_t t1, float* out) {
  const uint32_t q_dim = nh * hd, kv_dim = nkv * hd, group = nh / nkv;
  for (uint32_t t = t0; t < t1; ++t)
    for (uint32_t h = 0; h < nh; ++h) {
      const float* v = vals + (size_t)t * kv_dim + (h / group) * hd;
      float sq = 0.0f;
      for (uint32_t i = 0; i < hidden; ++i) {
        const float* row = wo + (size_t)i * q_dim + h * hd;
        float o = 0.0f;
        for (uint32_t d = 0; d < hd; ++d) o += row[d] * v[d];
        sq += o * o;
      }
      out[(size_t)(t - t0) * nh + h] = sqrtf(sq);
    }
}
