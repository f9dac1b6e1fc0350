/*
 * oracle.h -- CPU oracle for defer's per-token forward pass.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * strictly sequential Rust loops, used as the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product (defer_amd/) never links or calls it.
 *
 * Arithmetic follows the reference exactly: one accumulator walked in index
 * order, products rounded before the add (built with -ffp-contract=off, no
 * fast-math), glibc libm for expf/sinf/cosf/tanhf/pow.
 *
 * Parity pins (what checks each function; see tests/test_oracle_*.py):
 *   ops           -- the reference's own unit-test vectors (ops.rs:190-252),
 *                    brute force against numpy float64.
 *   forward_ext   -- HF transformers LlamaForCausalLM in float64 on the
 *                    reference's tiny config; closed forms (pos 0 RoPE is the
 *                    identity, one-position attention returns V[0] bitwise).
 *   sampler       -- the reference's sampler tests (sampler.rs:116-162) and
 *                    the closed form for uniform logits over 2^k tokens.
 *   chacha core   -- RFC 7539 / 8439 ChaCha20 vectors and the published
 *                    8-round zero-key keystream.
 *   seed_from_u64 -- parity unpinned (rand_core 0.6.4 PCG32 expansion; no
 *                    vector exists outside the crate).
 *   value_norms   -- closed forms: a one-hot value row returns the norm of
 *                    one column of W_o (float64 within 1e-6), scaling v by
 *                    2^k scales every norm by exactly 2^k, zero v gives 0.
 */
#ifndef DEFER_ORACLE_H
#define DEFER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ops.rs ------------------------------------------------------------ */
void oracle_matmul_sequential(float* out, const float* a, const float* b, size_t m, size_t n,
                              size_t k);
void oracle_linear(float* out, const float* x, const float* w, const float* bias, size_t in_dim,
                   size_t out_dim);
float oracle_dot(const float* a, const float* b, size_t n);
void oracle_rmsnorm(float* out, const float* x, const float* w, size_t n, float eps);
void oracle_layernorm(float* out, const float* x, const float* w, const float* b, size_t n,
                      float eps);
float oracle_silu(float x);
float oracle_gelu(float x);
void oracle_silu_inplace(float* x, size_t n);
void oracle_gelu_inplace(float* x, size_t n);
void oracle_add_inplace(float* a, const float* b, size_t n);
void oracle_mul_inplace(float* a, const float* b, size_t n);
void oracle_softmax_inplace(float* x, size_t n);

/* ---- model.rs ---------------------------------------------------------- */
typedef struct oracle_config {
  uint32_t vocab_size;
  uint32_t hidden_size;
  uint32_t intermediate_size;
  uint32_t num_layers;
  uint32_t num_heads;
  uint32_t num_kv_heads;
  uint32_t head_dim;
  float rms_norm_eps;
  float rope_theta;
  uint32_t max_seq_len;
  uint32_t tie_word_embeddings; /* 1: lm_head is the embedding */
  uint32_t activation;          /* 0: silu, 1: gelu (tanh) */
  uint32_t has_bias;            /* q/k/v projection biases present */
} oracle_config;

typedef struct oracle_model oracle_model;
typedef struct oracle_cache oracle_cache;

/* Tensors in canonical order: embed [V,h]; per layer attn_norm [h], wq [q,h],
 * (bq [q]), wk [kv,h], (bk [kv]), wv [kv,h], (bv [kv]), wo [h,q],
 * ffn_norm [h], w_gate [ff,h], w_up [ff,h], w_down [h,ff]; norm [h];
 * (lm_head [V,h] when untied). The model borrows the arrays. */
oracle_model* oracle_model_create(const oracle_config* cfg, const float* const* tensors,
                                  size_t n_tensors);
void oracle_model_destroy(oracle_model* m);
size_t oracle_model_tensor_count(const oracle_config* cfg);

oracle_cache* oracle_cache_create(const oracle_model* m);
void oracle_cache_destroy(oracle_cache* c);
uint32_t oracle_cache_len(const oracle_cache* c);
void oracle_cache_truncate(oracle_cache* c, uint32_t n);
/* Copies layer `layer`'s keys and values, [len, kv_dim] each. */
void oracle_cache_read(const oracle_cache* c, uint32_t layer, float* keys, float* values);

#define ORACLE_OK 0
#define ORACLE_E_TOKEN 1
#define ORACLE_E_CONTEXT 2

/* Model::forward_ext. logits_out [V] may be NULL; trace_out may be NULL, else
 * receives probs[layer][head*(pos+1)+t] laid out [L, nh, pos+1]. */
int oracle_forward_ext(const oracle_model* m, oracle_cache* c, uint32_t token,
                       const uint32_t* masked, size_t n_masked, float* logits_out,
                       float* trace_out);

/* ---- sampler.rs -------------------------------------------------------- */
uint32_t oracle_argmax(const float* logits, size_t n);
void oracle_softmax_with_temperature(const float* logits, size_t n, float temperature,
                                     float* probs);
float oracle_unit_f32(uint32_t word);
/* One ChaCha8 word `word` is consumed iff temperature > 0. */
uint32_t oracle_sample_token(const float* logits, size_t n, float temperature, uint32_t word);
uint32_t oracle_sample_margin(const float* logits, size_t n, float temperature, uint32_t word,
                              float* margin);
uint32_t oracle_sample_terms(const float* p, size_t n, uint32_t word, float* total);
void oracle_expf_array(const float* x, float* y, size_t n);

/* ---- rand_chacha / rand_core (third-party, restated) -------------------- */
void oracle_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream, int rounds,
                         uint32_t out[16]);
uint64_t oracle_pcg32_step(uint64_t state, uint64_t inc);
uint32_t oracle_pcg32_output(uint64_t state);
void oracle_seed_from_u64(uint64_t seed, uint8_t out[32]);
/* Word `index` of the ChaCha8 stream keyed by `seed` (stream 0). */
uint32_t oracle_chacha8_word(const uint8_t seed[32], uint64_t index);

/* ---- engine.rs: prompt + generate, checkout ------------------------------ */
/* Session::new + prompt + generate(n_gen). Writes n_gen tokens; last_logits
 * [V] may be NULL. Returns words consumed (rng_word_pos) or a negative error. */
int64_t oracle_generate(const oracle_model* m, oracle_cache* c, const uint8_t seed[32],
                        float temperature, const uint32_t* prompt, size_t n_prompt, size_t n_gen,
                        uint32_t* out_tokens, float* last_logits);
/* Session::checkout's replay loop. Returns -1 when every recorded token
 * re-samples identically, else the first diverging history index (and the
 * sampled token in *sampled_at_div); negative < -1 on model errors. */
int64_t oracle_checkout(const oracle_model* m, oracle_cache* c, const uint8_t seed[32],
                        float temperature, const uint32_t* history, size_t n_history,
                        size_t prompt_len, uint32_t* sampled_at_div, float* last_logits);

#ifdef __cplusplus
}
#endif
/* ValueNorms::sync (attribution.rs:116-148) for one layer: for positions
 * t in [t0, t1) and query heads h, out[(t - t0) * nh + h] =
 * sqrt(sum_i (sum_d wo[i][h*hd + d] * v[t][kvh*hd + d])^2), kvh = h / group,
 * each sum sequential with the product rounded before the add. wo is
 * [hidden][nh*hd]; vals is the layer's cached values [t][nkv*hd]. */
void oracle_value_norms(const float* wo, const float* vals, uint32_t hidden, uint32_t nh,
                        uint32_t nkv, uint32_t hd, uint32_t t0, uint32_t t1, float* out);

#endif
