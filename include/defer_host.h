/*
 * defer_host.h -- C ABI of the host side that drives libdefer_gpu: the
 * session (prompt / step / generate / checkout), the ChaCha8 word source the
 * sampler consumes, the write-ahead log and checkpoint formats, and the
 * CRC-32 / SHA-256 they use. Plain C types only; every call returns an int
 * status (0 = DEFER_HOST_OK) unless it cannot fail.
 *
 * Reference interfaces restated (paths under the reference's src/):
 *   defer_host_crc32            crc32::crc32                     crc32.rs:4-28
 *   defer_host_sha256           sha256::sha256                   sha256.rs:15-134
 *   defer_host_cache_fingerprint KvCache::fingerprint            model.rs:233-242
 *   defer_host_seed_from_u64    engine::seed_from_u64            engine.rs:19-21
 *   defer_host_chacha8_words    ChaCha8Rng word stream           engine.rs:51, 213-215
 *   defer_host_words_per_sample sampler::words_per_sample        sampler.rs:15-21
 *   defer_host_wal_*            WalHeader / WalWriter / WalLog   wal.rs:8-255
 *   defer_host_checkpoint_*     DeferCheckpoint                  checkpoint.rs:4-136
 *   defer_host_st_*             SafeTensors::load                safetensors.rs:142-237
 *   defer_host_model_load       Model::load / Config::from_json  model.rs:41-118, 285-347
 *   defer_host_session_*        Session                          engine.rs:23-137, 241-274
 */
#ifndef DEFER_HOST_H
#define DEFER_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "defer_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DEFER_HOST_OK 0
#define DEFER_HOST_E_INVALID 1     /* bad argument */
#define DEFER_HOST_E_IO 2          /* file error (DeferError::Io) */
#define DEFER_HOST_E_WAL 3         /* malformed or inconsistent WAL (DeferError::Wal) */
#define DEFER_HOST_E_CHECKPOINT 4  /* checkpoint does not fit the model (DeferError::Checkpoint) */
#define DEFER_HOST_E_DIVERGENCE 5  /* replay re-sampled another token (DeferError::Divergence) */
#define DEFER_HOST_E_GPU 6         /* a libdefer_gpu call failed (its message is kept) */
#define DEFER_HOST_E_MODEL 7       /* malformed model file or config (DeferError::Model) */

/* Thread-local description of the last failing call. */
const char* defer_host_last_error(void);

/* ---------------------------------------------------------------- hashes */

/* CRC-32 (IEEE 802.3, reflected, init and final xor 0xFFFFFFFF). */
uint32_t defer_host_crc32(const uint8_t* data, size_t n);
/* SHA-256 (FIPS 180-4). */
void defer_host_sha256(const uint8_t* data, size_t n, uint8_t out[32]);
/* KvCache::fingerprint (model.rs:233-242) of a device cache: SHA-256 of
 * len as a little-endian u64, then per layer all keys, then all values, as
 * little-endian f32 bits. Reads the cache to the host (verification only). */
int defer_host_cache_fingerprint(const defer_gpu_cache* c, uint8_t out[32]);

/* -------------------------------------------------------------- randomness */

/* The 32-byte ChaCha8 seed expanded from a numeric seed (rand_core 0.6.4
 * SeedableRng::seed_from_u64: a PCG32 stream fills it 4 bytes at a time). */
void defer_host_seed_from_u64(uint64_t seed, uint8_t out[32]);
/* Words word_pos .. word_pos+n-1 of the ChaCha8 stream keyed by `seed`
 * (rand_chacha 0.3.1: 8 rounds, 64-bit block counter in words 12-13, stream
 * 0; word w is u32 w % 16 of block w / 16). Word w is the one the w-th
 * sampled token consumes. */
void defer_host_chacha8_words(const uint8_t seed[32], uint64_t word_pos, size_t n, uint32_t* out);
/* Words one sampled token consumes: 0 when temperature == 0, else 1. */
uint32_t defer_host_words_per_sample(float temperature);

/* ------------------------------------------------------------ WAL format */

/* WalHeader (wal.rs:46-70). The prefix tokens are passed separately. */
typedef struct defer_host_wal_header {
  uint8_t model_signature[32];
  uint8_t base_seed[32];
  float temperature;
  uint32_t prompt_len;
  uint64_t start_rng_word_pos; /* u128 in the file; the high half is 0 */
} defer_host_wal_header;

typedef struct defer_host_wal defer_host_wal;

/* WalWriter::create (wal.rs:203-211): truncate `path`, write the header with
 * its prefix, flush and sync. With `durable`, every append is synced. */
int defer_host_wal_create(const char* path, const defer_host_wal_header* h, const uint32_t* prefix,
                          size_t n_prefix, int durable, defer_host_wal** out);
/* WalWriter::resume (wal.rs:214-222): parse, cut a torn tail, append after it. */
int defer_host_wal_resume(const char* path, int durable, defer_host_wal** out);
/* WalWriter::append (wal.rs:224-234): one 29-byte record, flushed. */
int defer_host_wal_append(defer_host_wal* w, uint32_t token, uint64_t rng_word_pos);
uint32_t defer_host_wal_next_step(const defer_host_wal* w);
void defer_host_wal_close(defer_host_wal* w);

/* WalLog::parse (wal.rs:115-183) collapsed into a checkpoint
 * (WalLog::to_checkpoint, wal.rs:186-197). Call with history == NULL to learn
 * *n_history, then again with a buffer of that size. *torn_tail tells whether
 * trailing bytes were discarded. */
int defer_host_wal_read(const char* path, defer_host_wal_header* h, uint32_t* history,
                        size_t* n_history, uint64_t* rng_word_pos, int* torn_tail);

/* ------------------------------------------------------ checkpoint format */

/* DeferCheckpoint (checkpoint.rs:26-37); the history is passed separately. */
typedef struct defer_host_checkpoint_header {
  uint8_t model_signature[32];
  uint8_t base_seed[32];
  float temperature;
  uint32_t prompt_len;
  uint64_t rng_word_pos; /* u128 in the file; the high half is 0 */
} defer_host_checkpoint_header;

/* DeferCheckpoint::save (checkpoint.rs:86-97): the 112 + 4n bytes of
 * to_bytes (checkpoint.rs:44-57) written to `path` with its extension
 * replaced by "ckpt.tmp", synced, then renamed over `path`. */
int defer_host_checkpoint_save(const char* path, const defer_host_checkpoint_header* h,
                               const uint32_t* history, size_t n);
/* DeferCheckpoint::load (checkpoint.rs:59-84, 99-101). Call with history ==
 * NULL to learn *n_history, then again with a buffer of that size. */
int defer_host_checkpoint_load(const char* path, defer_host_checkpoint_header* h,
                               uint32_t* history, size_t* n_history);

/* ------------------------------------------------------------ model file */

typedef struct defer_host_st defer_host_st;

/* SafeTensors::load (safetensors.rs:142-237): one front-to-back pass, every
 * byte hashed (SHA-256 = the model signature), F32 / F16 / BF16 / F64
 * tensors converted exactly to f32. The accessors index tensors in on-disk
 * order; the pointers live until defer_host_st_close. */
int defer_host_st_open(const char* path, defer_host_st** out);
void defer_host_st_close(defer_host_st* st);
size_t defer_host_st_count(const defer_host_st* st);
const char* defer_host_st_name(const defer_host_st* st, size_t i);
/* Writes up to max_dims dimensions; returns the rank. */
size_t defer_host_st_shape(const defer_host_st* st, size_t i, uint64_t* dims, size_t max_dims);
const float* defer_host_st_data(const defer_host_st* st, size_t i, size_t* n);
/* The __metadata__ string for `key`, or NULL. */
const char* defer_host_st_meta(const defer_host_st* st, const char* key);
void defer_host_st_signature(const defer_host_st* st, uint8_t out[32]);

/* Model::load (model.rs:285-298): the file's tensors, the config from its
 * "defer.config" metadata or config.json beside it (Config::from_json,
 * model.rs:41-118, with the reference's defaults and inferences), the
 * tensors in the order of model.rs:301-347, then defer_gpu_model_create.
 * max_seq_len != 0 overrides max_position_embeddings. cfg_out and
 * signature (the file's SHA-256) may be NULL. */
int defer_host_model_load(const char* path, uint32_t max_seq_len, defer_gpu_model** out,
                          defer_gpu_config* cfg_out, uint8_t signature[32]);

/* --------------------------------------------------------------- session */

typedef struct defer_host_session defer_host_session;

/* Session::new (engine.rs:44-59) on a device cache of `capacity` positions
 * (0: the model's max_seq_len). The model stays owned by the caller. */
int defer_host_session_create(const defer_gpu_model* m, const uint8_t base_seed[32],
                              float temperature, uint32_t capacity, defer_host_session** out);
void defer_host_session_destroy(defer_host_session* s);
/* Session::prompt (engine.rs:62-71). */
int defer_host_session_prompt(defer_host_session* s, const uint32_t* tokens, size_t n);
/* Session::step (engine.rs:113-117). */
int defer_host_session_step(defer_host_session* s, uint32_t* token_out);
/* Session::generate (engine.rs:121-137), one device launch for the run. */
int defer_host_session_generate(defer_host_session* s, uint32_t max_tokens, const uint32_t* stop,
                                size_t n_stop, uint32_t* tokens_out, uint32_t* n_out);
/* Session::generate with a WAL (main.rs:261-312): each token's record is
 * appended and flushed (synced when the log is durable) as soon as the device
 * commits the token, while later tokens are still being generated, with the
 * rng position after its sample. A failed append stops the call there with
 * the WAL's error, the session holding the tokens up to that one. */
int defer_host_session_generate_logged(defer_host_session* s, uint32_t max_tokens,
                                       const uint32_t* stop, size_t n_stop, defer_host_wal* wal,
                                       uint32_t* tokens_out, uint32_t* n_out);
/* Accessors (engine.rs:194-221). */
size_t defer_host_session_history(const defer_host_session* s, uint32_t* out /* nullable */);
uint32_t defer_host_session_prompt_len(const defer_host_session* s);
uint64_t defer_host_session_rng_word_pos(const defer_host_session* s);
defer_gpu_cache* defer_host_session_cache(defer_host_session* s);
/* Session::checkout (engine.rs:241-274): validate, then rebuild the session
 * by replaying the history on the device; a re-sampled token that differs
 * from the record fails with DEFER_HOST_E_DIVERGENCE and the reference's
 * message. The caller checks the model signature. */
int defer_host_session_checkout(const defer_gpu_model* m, const uint8_t base_seed[32],
                                float temperature, const uint32_t* history, size_t n_history,
                                uint32_t prompt_len, uint64_t rng_word_pos, uint32_t capacity,
                                defer_host_session** out);

/* Session::checkpoint (engine.rs:223-232): the session's header fields with
 * the loaded model's signature (the history: defer_host_session_history). */
int defer_host_session_checkpoint(const defer_host_session* s, const uint8_t model_signature[32],
                                  defer_host_checkpoint_header* h);
/* Session::checkout (engine.rs:241-274) of a checkpoint file: the model
 * signature must match (the reference's "model signature mismatch" message),
 * then defer_host_session_checkout. */
int defer_host_session_checkout_file(const defer_gpu_model* m, const uint8_t model_signature[32],
                                     const char* path, uint32_t capacity,
                                     defer_host_session** out);

#ifdef __cplusplus
}
#endif

#endif /* DEFER_HOST_H */
