// session.cpp -- Session (engine.rs:23-137, 241-274 of the reference) on the
// device path: the cache lives in HBM, the logits never leave it, and the
// rng is the ChaCha8 word stream whose position counts the words consumed
// (one per sampled token at temperature > 0). Multi-token calls draw their
// words on the host first and run as one device launch.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <exception>
#include <vector>

#include "common.h"
#include "defer_host.h"

using dh::fail;

struct defer_host_session {
  const defer_gpu_model* m;
  defer_gpu_cache* c;
  uint8_t seed[32];
  float temperature;
  uint64_t word_pos;
  std::vector<uint32_t> history;
  uint32_t prompt_len;
};

namespace {

int gpu_fail(int rc) {
  return fail(DEFER_HOST_E_GPU, "defer_gpu error %d: %s", rc, defer_gpu_last_error());
}

std::vector<uint32_t> words_for(const defer_host_session* s, size_t n_samples) {
  std::vector<uint32_t> w;
  if (defer_host_words_per_sample(s->temperature)) {
    w.resize(n_samples);
    if (n_samples) defer_host_chacha8_words(s->seed, s->word_pos, n_samples, w.data());
  }
  return w;
}

}  // namespace

extern "C" int defer_host_session_create(const defer_gpu_model* m, const uint8_t base_seed[32],
                                         float temperature, uint32_t capacity,
                                         defer_host_session** out) {
  if (!m || !base_seed || !out) return fail(DEFER_HOST_E_INVALID, "null argument");
  if (!(temperature >= 0.0f && isfinite(temperature)))
    return fail(DEFER_HOST_E_INVALID, "temperature must be finite and >= 0");
  defer_gpu_cache* c = nullptr;
  const int rc = defer_gpu_cache_create(m, capacity, &c);
  if (rc) return gpu_fail(rc);
  defer_host_session* s = new defer_host_session();
  s->m = m;
  s->c = c;
  memcpy(s->seed, base_seed, 32);
  s->temperature = temperature;
  s->word_pos = 0;
  s->prompt_len = 0;
  *out = s;
  return DEFER_HOST_OK;
}

extern "C" void defer_host_session_destroy(defer_host_session* s) {
  if (!s) return;
  defer_gpu_cache_destroy(s->c);
  delete s;
}

extern "C" int defer_host_session_prompt(defer_host_session* s, const uint32_t* tokens, size_t n) {
  if (!s || (n && !tokens)) return fail(DEFER_HOST_E_INVALID, "null argument");
  if (s->history.size() != s->prompt_len)
    return fail(DEFER_HOST_E_INVALID, "cannot add prompt tokens after generation started");
  if (n == 0) return DEFER_HOST_OK;
  const uint32_t before = defer_gpu_cache_len(s->c);
  const int rc = defer_gpu_prompt(s->m, s->c, tokens, n);
  // Tokens fed before an error stay in the history, as feed() leaves them;
  // prompt_len only moves when every token was fed (engine.rs:62-71 returns
  // before setting it), so a failed prompt blocks further prompt calls.
  const uint32_t fed = defer_gpu_cache_len(s->c) - before;
  s->history.insert(s->history.end(), tokens, tokens + fed);
  if (rc) return gpu_fail(rc);
  s->prompt_len = (uint32_t)s->history.size();
  return DEFER_HOST_OK;
}

extern "C" int defer_host_session_generate(defer_host_session* s, uint32_t max_tokens,
                                           const uint32_t* stop, size_t n_stop,
                                           uint32_t* tokens_out, uint32_t* n_out) {
  if (!s || (n_stop && !stop) || (max_tokens && !tokens_out))
    return fail(DEFER_HOST_E_INVALID, "null argument");
  // At most the cache's free positions can be sampled (one more request
  // reports the context error), so no more words than that are drawn. The
  // step that hits the full cache still counts its word, as the reference's
  // does: Session::step samples (one word) before feed fails
  // (engine.rs:113-117, model.rs:420-422).
  const uint32_t room = defer_gpu_cache_capacity(s->c) - defer_gpu_cache_len(s->c);
  std::vector<uint32_t> words;
  try {
    words = words_for(s, std::min<uint32_t>(max_tokens, room));
  } catch (const std::exception& e) {
    return fail(DEFER_HOST_E_INVALID, "cannot draw %u rng words: %s", max_tokens, e.what());
  }
  uint32_t n = 0;
  const int rc = defer_gpu_generate(s->m, s->c, max_tokens, s->temperature,
                                    words.empty() ? nullptr : words.data(), stop, n_stop,
                                    tokens_out, &n);
  s->history.insert(s->history.end(), tokens_out, tokens_out + n);
  s->word_pos += (uint64_t)(n + (rc == DEFER_GPU_E_CONTEXT)) * defer_host_words_per_sample(s->temperature);
  if (n_out) *n_out = n;
  return rc ? gpu_fail(rc) : DEFER_HOST_OK;
}

namespace {
// on_token of a logged generate: the WAL record of the token just committed,
// with the rng position after its sample (main.rs:292-296).
struct WalLogCtx {
  defer_host_wal* wal;
  uint64_t word_pos0;
  uint32_t wps;
  int wal_rc;
};
int wal_on_token(void* user, uint32_t index, uint32_t token) {
  WalLogCtx* x = static_cast<WalLogCtx*>(user);
  x->wal_rc = defer_host_wal_append(x->wal, token, x->word_pos0 + (uint64_t)(index + 1) * x->wps);
  return x->wal_rc;
}
}  // namespace

extern "C" int defer_host_session_generate_logged(defer_host_session* s, uint32_t max_tokens,
                                                  const uint32_t* stop, size_t n_stop,
                                                  defer_host_wal* wal, uint32_t* tokens_out,
                                                  uint32_t* n_out) {
  if (!s || !wal || (n_stop && !stop) || (max_tokens && !tokens_out))
    return fail(DEFER_HOST_E_INVALID, "null argument");
  const uint32_t room = defer_gpu_cache_capacity(s->c) - defer_gpu_cache_len(s->c);
  std::vector<uint32_t> words;
  try {
    words = words_for(s, std::min<uint32_t>(max_tokens, room));
  } catch (const std::exception& e) {
    return fail(DEFER_HOST_E_INVALID, "cannot draw %u rng words: %s", max_tokens, e.what());
  }
  WalLogCtx ctx{wal, s->word_pos, defer_host_words_per_sample(s->temperature), 0};
  uint32_t n = 0;
  const int rc = defer_gpu_generate_cb(s->m, s->c, max_tokens, s->temperature,
                                       words.empty() ? nullptr : words.data(), stop, n_stop,
                                       tokens_out, &n, wal_on_token, &ctx);
  s->history.insert(s->history.end(), tokens_out, tokens_out + n);
  s->word_pos += (uint64_t)(n + (rc == DEFER_GPU_E_CONTEXT)) * ctx.wps;
  if (n_out) *n_out = n;
  if (ctx.wal_rc) return ctx.wal_rc;  // the WAL's error, its message kept
  return rc ? gpu_fail(rc) : DEFER_HOST_OK;
}

extern "C" int defer_host_session_step(defer_host_session* s, uint32_t* token_out) {
  if (!token_out) return fail(DEFER_HOST_E_INVALID, "null argument");
  uint32_t n = 0;
  const int rc = defer_host_session_generate(s, 1, nullptr, 0, token_out, &n);
  if (rc == DEFER_HOST_OK && n != 1) return fail(DEFER_HOST_E_GPU, "step produced no token");
  return rc;
}

extern "C" size_t defer_host_session_history(const defer_host_session* s, uint32_t* out) {
  if (!s) return 0;
  if (out) memcpy(out, s->history.data(), s->history.size() * sizeof(uint32_t));
  return s->history.size();
}

extern "C" uint32_t defer_host_session_prompt_len(const defer_host_session* s) {
  return s ? s->prompt_len : 0;
}

extern "C" uint64_t defer_host_session_rng_word_pos(const defer_host_session* s) {
  return s ? s->word_pos : 0;
}

extern "C" defer_gpu_cache* defer_host_session_cache(defer_host_session* s) {
  return s ? s->c : nullptr;
}

extern "C" int defer_host_session_checkout(const defer_gpu_model* m, const uint8_t base_seed[32],
                                           float temperature, const uint32_t* history,
                                           size_t n_history, uint32_t prompt_len,
                                           uint64_t rng_word_pos, uint32_t capacity,
                                           defer_host_session** out) {
  if (!m || !base_seed || !out || (n_history && !history))
    return fail(DEFER_HOST_E_INVALID, "null argument");
  if (prompt_len > n_history) return fail(DEFER_HOST_E_CHECKPOINT, "prompt_len exceeds history");
  const uint64_t sampled = n_history - prompt_len;
  const uint64_t expected = sampled * defer_host_words_per_sample(temperature);
  if (rng_word_pos != expected)
    return fail(DEFER_HOST_E_CHECKPOINT,
                "rng_word_pos %llu inconsistent with %llu sampled tokens (expected %llu)",
                (unsigned long long)rng_word_pos, (unsigned long long)sampled,
                (unsigned long long)expected);
  defer_host_session* s = nullptr;
  int rc = defer_host_session_create(m, base_seed, temperature, capacity, &s);
  if (rc) return rc;
  std::vector<uint32_t> words;
  try {
    words = words_for(s, sampled);
  } catch (const std::exception& e) {
    defer_host_session_destroy(s);
    return fail(DEFER_HOST_E_INVALID, "cannot draw %llu rng words: %s", (unsigned long long)sampled,
                e.what());
  }
  int64_t first_div = -1;
  uint32_t at_div = 0;
  rc = defer_gpu_replay(m, s->c, history, n_history, prompt_len, temperature,
                        words.empty() ? nullptr : words.data(), &first_div, &at_div);
  if (rc) {
    defer_host_session_destroy(s);
    return gpu_fail(rc);
  }
  if (first_div >= 0) {
    defer_host_session_destroy(s);
    return fail(DEFER_HOST_E_DIVERGENCE,
                "replay sampled token %u at position %lld, checkpoint recorded %u", at_div,
                (long long)first_div, history[first_div]);
  }
  s->history.assign(history, history + n_history);
  s->prompt_len = prompt_len;
  s->word_pos = rng_word_pos;
  *out = s;
  return DEFER_HOST_OK;
}

extern "C" int defer_host_session_checkpoint(const defer_host_session* s,
                                             const uint8_t model_signature[32],
                                             defer_host_checkpoint_header* h) {
  if (!s || !model_signature || !h) return fail(DEFER_HOST_E_INVALID, "null argument");
  memcpy(h->model_signature, model_signature, 32);
  memcpy(h->base_seed, s->seed, 32);
  h->temperature = s->temperature;
  h->prompt_len = s->prompt_len;
  h->rng_word_pos = s->word_pos;
  return DEFER_HOST_OK;
}

extern "C" int defer_host_session_checkout_file(const defer_gpu_model* m,
                                                const uint8_t model_signature[32],
                                                const char* path, uint32_t capacity,
                                                defer_host_session** out) {
  if (!m || !model_signature || !path || !out) return fail(DEFER_HOST_E_INVALID, "null argument");
  defer_host_checkpoint_header h;
  size_t n = 0;
  int rc = defer_host_checkpoint_load(path, &h, nullptr, &n);
  if (rc) return rc;
  std::vector<uint32_t> history(n);
  rc = defer_host_checkpoint_load(path, &h, history.data(), &n);
  if (rc) return rc;
  if (memcmp(h.model_signature, model_signature, 32) != 0) {
    auto hex = [](const uint8_t* b) {
      std::string s;
      char t[3];
      for (int i = 0; i < 32; ++i) {
        snprintf(t, sizeof(t), "%02x", b[i]);
        s += t;
      }
      return s;
    };
    return fail(DEFER_HOST_E_CHECKPOINT, "model signature mismatch: checkpoint %s vs loaded %s",
                hex(h.model_signature).c_str(), hex(model_signature).c_str());
  }
  return defer_host_session_checkout(m, h.base_seed, h.temperature, history.data(), n,
                                     h.prompt_len, h.rng_word_pos, capacity, out);
}
