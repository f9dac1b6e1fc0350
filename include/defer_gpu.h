/*
 * defer_gpu.h -- C ABI of the MI355X (gfx950) per-token forward pass.
 *
 * This library replaces the hot path of defer's Model::forward_ext and
 * sampler::sample_token with hand-written HIP kernels. The host keeps
 * ownership of every host buffer. Device memory lives behind opaque handles.
 * Every call returns an int status (0 = DEFER_GPU_OK) and returns only once
 * its outputs are visible on the host. Nothing is thrown across the ABI.
 * Handles are not thread-safe, which matches the reference's single-threaded
 * `&mut KvCache` contract.
 *
 * Reference interfaces replaced (paths under the reference's src/):
 *   defer_gpu_model_create   Model::from_safetensors          model.rs:301-363
 *   defer_gpu_cache_*        KvCache::{new,len,truncate,clone} model.rs:182-243
 *   defer_gpu_forward        Model::forward_ext                model.rs:394-520
 *   defer_gpu_sample         sampler::sample_token             sampler.rs:78-109
 *   defer_gpu_step           Session::step                     engine.rs:113-117
 *   defer_gpu_generate       Session::generate                 engine.rs:121-137
 *   defer_gpu_replay         Session::checkout replay loop     engine.rs:261-271
 *   defer_gpu_forward_batch, defer_gpu_step_batch, defer_gpu_model_set_batching,
 *   defer_gpu_model_set_profiling, defer_gpu_batch_stats:
 *                            no counterpart (the reference is batch-1 only)
 */
#ifndef DEFER_GPU_H
#define DEFER_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DEFER_GPU_OK 0
#define DEFER_GPU_E_INVALID 1    /* bad argument, shape or config */
#define DEFER_GPU_E_TOKEN 2      /* token id out of range (model.rs:417-419) */
#define DEFER_GPU_E_CONTEXT 3    /* context length exceeded (model.rs:420-422) */
#define DEFER_GPU_E_HIP 4        /* HIP runtime error (message in last_error) */
#define DEFER_GPU_E_NO_LOGITS 5  /* sample with no forward yet (engine.rs:104-108) */
#define DEFER_GPU_E_TIMEOUT 6    /* a device-side wait exceeded its bound */
#define DEFER_GPU_E_CALLBACK 7   /* an on_token callback returned non-zero */

/* Model::Config (model.rs:23-39), sizes as the reference names them. */
typedef struct defer_gpu_config {
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
  uint32_t tie_word_embeddings; /* 1: lm_head is the embedding table */
  uint32_t activation;          /* 0: silu, 1: gelu (tanh approximation) */
  uint32_t has_bias;            /* q/k/v projection biases present */
} defer_gpu_config;

typedef struct defer_gpu_model defer_gpu_model;
typedef struct defer_gpu_cache defer_gpu_cache;

/* Execution modes for a model's token steps. Every mode runs the same
 * device arithmetic, so results are bit-identical across modes. */
#define DEFER_GPU_EXEC_PERSISTENT 0 /* one cooperative dataflow kernel per call */
#define DEFER_GPU_EXEC_GRAPH 1      /* one captured hipGraph of phase kernels per token */
#define DEFER_GPU_EXEC_EAGER 2      /* phase kernels launched one by one */

/* Model::from_safetensors (model.rs:301-363). `tensors` holds host pointers in
 * the order of model.rs:322-347: embed [V,h]; per layer attn_norm [h],
 * wq [q,h], (bq [q]), wk [kv,h], (bk [kv]), wv [kv,h], (bv [kv]), wo [h,q],
 * ffn_norm [h], w_gate [ff,h], w_up [ff,h], w_down [h,ff]; norm [h];
 * (lm_head [V,h] when untied). The library copies them to HBM and computes
 * RoPE tables on the host as model.rs:348-353 and 438-445 do. `flags` is 0. */
int defer_gpu_model_create(const defer_gpu_config* cfg, const float* const* tensors,
                           size_t n_tensors, uint32_t flags, defer_gpu_model** out);
void defer_gpu_model_destroy(defer_gpu_model* m);
size_t defer_gpu_model_tensor_count(const defer_gpu_config* cfg);
int defer_gpu_model_set_exec(defer_gpu_model* m, uint32_t mode);

/* KvCache::new (model.rs:193-200): device-resident, preallocated to
 * `capacity` positions (0 means the config's max_seq_len). */
int defer_gpu_cache_create(const defer_gpu_model* m, uint32_t capacity, defer_gpu_cache** out);
void defer_gpu_cache_destroy(defer_gpu_cache* c);
uint32_t defer_gpu_cache_len(const defer_gpu_cache* c);          /* KvCache::len   model.rs:202 */
/* Positions the cache was created for (the reference's bound is the config's
 * max_seq_len, model.rs:420-422). */
uint32_t defer_gpu_cache_capacity(const defer_gpu_cache* c);
int defer_gpu_cache_truncate(defer_gpu_cache* c, uint32_t n);    /* model.rs:211-220 */
int defer_gpu_cache_clone(const defer_gpu_cache* c, defer_gpu_cache** out); /* derive(Clone) */
/* The pub `keys` / `values` fields (model.rs:185-188) of one layer, each as a
 * [len, kv_dim] row-major host array. */
int defer_gpu_cache_read(const defer_gpu_cache* c, uint32_t layer, float* keys, float* values);
/* The cache's layer count and its pub `kv_dim` field (model.rs:185-188):
 * the shape of what defer_gpu_cache_read returns per layer. */
int defer_gpu_cache_shape(const defer_gpu_cache* c, uint32_t* layers, uint32_t* kv_dim);

/* ValueNorms::sync (attribution.rs:116-148), the extension step: for cached
 * positions t in [t0, t1), every layer l and query head h,
 * out[(l * (t1 - t0) + t - t0) * num_heads + h] = ||W_o,h . v_{t,kv(h)}||,
 * computed on the device in the reference's order (sequential sums of
 * rounded products, then sqrt), so the values equal the CPU loop's bit for
 * bit. The caller keeps the per-layer arrays and truncates them as
 * ValueNorms::sync does when the cache shrinks. */
int defer_gpu_value_norms(const defer_gpu_cache* c, uint32_t t0, uint32_t t1, float* out);

/* Model::forward_ext (model.rs:394-520). Appends the token's keys/values at
 * position cache_len and keeps the logits on the device. `logits_out` [V]
 * and `trace_out` [L, num_heads, pos+1] may be NULL. `masked` lists earlier
 * positions whose attention logit is forced to -inf; entries >= pos are
 * ignored. Range errors are reported before the cache is touched. */
int defer_gpu_forward(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t token,
                      const uint32_t* masked, size_t n_masked, float* logits_out,
                      float* trace_out);
/* Copies the logits of the cache's last forward to the host. */
int defer_gpu_last_logits(const defer_gpu_cache* c, float* logits_out);

/* The Session's logits (engine.rs:32, `logits: Option<Vec<f32>>`) replaced by
 * the caller's [V] vector, so the next sample / step / generate samples
 * exactly these values with the device sampler (used to pin the sampler's
 * edge cases: ties, NaN, -inf, overflow). Needs a forward on the cache first. */
int defer_gpu_cache_set_logits(defer_gpu_cache* c, const float* logits);

/* sampler::sample_token (sampler.rs:78-109) on the last forward's logits.
 * temperature == 0 is greedy argmax and ignores rng_word; temperature > 0
 * consumes exactly the one ChaCha8 word `rng_word`, r = (rng_word >> 8) * 2^-24. */
int defer_gpu_sample(const defer_gpu_model* m, defer_gpu_cache* c, float temperature,
                     uint32_t rng_word, uint32_t* token_out);

/* Session::step (engine.rs:113-117): sample, then forward the sampled token. */
int defer_gpu_step(const defer_gpu_model* m, defer_gpu_cache* c, float temperature,
                   uint32_t rng_word, uint32_t* token_out);

/* Session::generate (engine.rs:121-137) with no host round trip per token.
 * rng_words[i] is the word the i-th sampled token consumes (unused when
 * temperature == 0; may then be NULL). Generation stops after a token listed
 * in `stop` has been fed. *n_out receives the number of tokens produced. */
int defer_gpu_generate(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t max_tokens,
                       float temperature, const uint32_t* rng_words, const uint32_t* stop,
                       size_t n_stop, uint32_t* tokens_out, uint32_t* n_out);

/* The on_token hook of Session::generate (engine.rs:121-137): called on the
 * calling thread once per generated token, in order, while the device is
 * still generating the later ones (each token is handed over as soon as its
 * forward is committed), e.g. to append and flush a write-ahead log record
 * (main.rs:292-296, wal.rs:241-250). index counts this call's tokens. A
 * non-zero return stops the call there, as an error from the reference's
 * closure does: the call returns DEFER_GPU_E_CALLBACK with *n_out = index + 1
 * and the cache holding exactly those tokens (tokens the device generated
 * past it are truncated away; the logits are then not kept). */
typedef int (*defer_gpu_token_fn)(void* user, uint32_t index, uint32_t token);

/* Device and pinned host allocations the library has made since the process
 * started (a diagnostic with no counterpart in the reference: tests use it
 * to show that defer_gpu_generate_static allocates nothing). */
uint64_t defer_gpu_allocation_count(void);

/* Process teardown (no counterpart in the reference, whose CPU path holds no
 * device state): once every model and cache is destroyed, synchronises and
 * resets (hipDeviceReset) each device the library made a model on, so the HIP
 * runtime's queues are released before the process exits rather than in the
 * runtime's exit handlers. DEFER_GPU_E_INVALID while any handle is live. The
 * reset frees every allocation of the process on those devices, the library's
 * or not: call it last, when nothing else in the process uses them. The
 * library may be used again afterwards. */
int defer_gpu_shutdown(void);

/* defer_gpu_generate with on_token (nullable) called per committed token. */
int defer_gpu_generate_cb(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t max_tokens,
                          float temperature, const uint32_t* rng_words, const uint32_t* stop,
                          size_t n_stop, uint32_t* tokens_out, uint32_t* n_out,
                          defer_gpu_token_fn on_token, void* user);

/* defer_gpu_generate without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc). It launches kernels,
 * synchronises the stream and copies the tokens back, so it must be called
 * outside any stream capture. The rng words, stop list and tokens of the run
 * are staged in a static device array of 513 KB per GPU, kept until the
 * process ends, so a call takes at most 65536 tokens and 256 stop tokens
 * (more is rejected with DEFER_GPU_E_INVALID before anything runs). Same
 * arguments, results and errors as defer_gpu_generate, bit for bit. Calls
 * that overlap on one GPU (from several host threads, on any caches) share
 * that array and race. */
int defer_gpu_generate_static(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t max_tokens,
                              float temperature, const uint32_t* rng_words, const uint32_t* stop,
                              size_t n_stop, uint32_t* tokens_out, uint32_t* n_out);

/* Session::prompt (engine.rs:62-71): forward each token in order. */
int defer_gpu_prompt(const defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* tokens,
                     size_t n_tokens);

/* Session::checkout's replay loop (engine.rs:261-271) on an empty cache:
 * history[0..prompt_len) is fed as prompt; every later token is first
 * re-sampled (consuming rng_words[i - prompt_len]) and compared with the
 * record, then the recorded token is fed. *first_div is -1 when every token
 * matched, else the first diverging history index, with the re-sampled token
 * in *sampled_at_div; the cache then holds the positions before it. */
int defer_gpu_replay(const defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* history,
                     size_t n_history, size_t prompt_len, float temperature,
                     const uint32_t* rng_words, int64_t* first_div, uint32_t* sampled_at_div);

/* ---------------------------------------------------------------- batches
 *
 * Rows run together (no counterpart in the reference, which steps one
 * session at a time, engine.rs:90-137). Every matrix product of a batch is an
 * MFMA GEMM that computes each output in the one-token order, and everything
 * else a row goes through is the one-token arithmetic, so a row's cache
 * entries, logits and tokens are bit-identical to feeding it on its own. */

/* defer_gpu_prompt and defer_gpu_replay run the batched path for at least
 * `min_rows` tokens and feed token by token below that; 0 turns batching
 * off. Results are identical either way. The default is 16. */
int defer_gpu_model_set_batching(defer_gpu_model* m, uint32_t min_rows);

/* Feeds tokens[b] to caches[b] for b < n as if in the order b = 0, 1, ...: a
 * cache listed k times receives k consecutive positions. Each cache keeps the
 * logits of its last row for a following sample/step. logits_out (nullable)
 * receives [n, V]: row b's logits. Range and capacity errors are reported
 * before any cache is touched. */
int defer_gpu_forward_batch(const defer_gpu_model* m, defer_gpu_cache* const* caches,
                            const uint32_t* tokens, uint32_t n, float* logits_out);

/* Session::step (engine.rs:113-117) on n distinct caches in lockstep: each
 * samples its last logits (consuming rng_words[b] when temperature > 0),
 * then the n sampled tokens are fed as one batch. tokens_out [n]. */
int defer_gpu_step_batch(const defer_gpu_model* m, defer_gpu_cache* const* caches, uint32_t n,
                         float temperature, const uint32_t* rng_words, uint32_t* tokens_out);

/* Launch geometry, for tests of the claim that results never depend on it:
 * the persistent kernel and the per-phase kernels run `workgroups`
 * workgroups (0: one per compute unit, capped by the smallest phase's item
 * count), and the batched path shapes its GEMM launches for `gemm_cus`
 * compute units (0: the device's). Must be called before the model's first
 * cache is created. Bits are identical for every setting. */
int defer_gpu_model_set_grid(defer_gpu_model* m, uint32_t workgroups, uint32_t gemm_cus);

/* Instrumentation of the batched path: when on, every batched call times its
 * GEMM and attention launches with HIP events on the library's stream.
 * stats[0..5] = GEMM ms, GEMM flop, GEMM launches, attention ms, attention
 * flop, attention launches, summed since the last reset (reset != 0 clears
 * them after reading). */
int defer_gpu_model_set_profiling(defer_gpu_model* m, uint32_t on);
int defer_gpu_batch_stats(const defer_gpu_model* m, double* stats, uint32_t reset);

/* Thread-local description of the last failing call. */
const char* defer_gpu_last_error(void);

/* Device time (ms) of the last generate / prompt / replay call, measured with
 * HIP events on the library's stream. */
double defer_gpu_last_device_ms(const defer_gpu_model* m);

#ifdef __cplusplus
}
#endif
#endif
