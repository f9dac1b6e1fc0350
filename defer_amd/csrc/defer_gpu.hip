// defer_gpu.hip -- gfx950 implementation of the C ABI in include/defer_gpu.h.
//
// Three launch modes share the phase functions of phases.h:
//   persistent: one cooperative kernel (one workgroup per CU) runs every op
//               of a call; workgroups hand activations to each other through
//               tagged mailboxes, so there is no grid barrier at all.
//   graph:      one hipGraph per op (sampler, 6 phases x L, lm_head, commit),
//               captured once per cache and replayed per token.
//   eager:      the same kernels launched one by one.
#include <hip/hip_runtime.h>

#include <atomic>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/defer_gpu.h"
#include "phases.h"

using namespace dg;

// Persistent kernels specialised for known model shapes (kernels_*.hip).
#define DG_DECLARE_SPECIALISED(NS)                            \
  namespace NS {                                              \
  struct Args;                                                \
  struct RunDesc;                                             \
  template <bool RANDOM>                                      \
  __global__ void k_persistent(const Args* ap, const RunDesc* run); \
  }
DG_DECLARE_SPECIALISED(dg135)
DG_DECLARE_SPECIALISED(dg360)
DG_DECLARE_SPECIALISED(dg1b)
DG_DECLARE_SPECIALISED(dg8b)
#undef DG_DECLARE_SPECIALISED

// ------------------------------------------------------------------ errors

static thread_local std::string g_last_error;

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                      \
  do {                                                                                     \
    hipError_t e_ = (expr);                                                                \
    if (e_ != hipSuccess)                                                                  \
      return fail(DEFER_GPU_E_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                  __FILE__, __LINE__);                                                     \
  } while (0)

extern "C" const char* defer_gpu_last_error(void) { return g_last_error.c_str(); }

// Every device and pinned host allocation of the library goes through these,
// so defer_gpu_allocation_count can show a call allocated nothing.
static std::atomic<uint64_t> g_allocations{0};
template <class T>
static hipError_t counted_malloc(T** p, size_t n) {
  g_allocations.fetch_add(1, std::memory_order_relaxed);
  return hipMalloc(reinterpret_cast<void**>(p), n);
}
static hipError_t counted_host_malloc(void** p, size_t n, unsigned flags) {
  g_allocations.fetch_add(1, std::memory_order_relaxed);
  return hipHostMalloc(p, n, flags);
}
extern "C" uint64_t defer_gpu_allocation_count(void) { return g_allocations.load(std::memory_order_relaxed); }

// Live models and caches, and the devices models were made on (a bit each):
// defer_gpu_shutdown resets only those devices, and only once nothing is live.
static std::atomic<uint64_t> g_live_models{0}, g_live_caches{0}, g_devices_used{0};

// ------------------------------------------------------------------ kernels

#include "persistent.h"
#include "batch.h"

// Per-run reset of the counters (pos / tick / token are kept).
__global__ void k_begin(DevState* st) {
  st->abort = 0;
  st->halt = 0;
  st->n_done = 0;
  st->op = 0;
  st->first_div = -1;
  st->sampled_div = 0;
}

enum : uint32_t { PH_LM_KERNEL = 100 };

__global__ __launch_bounds__(BLOCK) void k_phase(const Args* __restrict__ ap, uint32_t ph,
                                                 uint32_t layer) {
  const Args& a = *ap;
  const Lds s = lds_init(a.d);
  const DevState* st = a.st;
  if (st->halt) return;
  const uint32_t pos = st->pos, tick = st->tick, token = st->token;
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  const Stager sg = make_stager(a, s, wg, G, false);
  switch (ph) {
    case PH_QKV: phase_qkv(a, layer, tick, pos, token, wg, G, s, sg); break;
    case PH_ATTN: phase_attn(a, layer, tick, pos, wg, G, s); break;
    case PH_COMB: phase_comb(a, layer, tick, pos, wg, G, s); break;
    case PH_O: phase_o(a, layer, tick, pos, token, wg, G, s, sg); break;
    case PH_GU: phase_gu(a, layer, tick, wg, G, s, sg); break;
    case PH_D: phase_d(a, layer, tick, wg, G, s, sg); break;
    case PH_LM_KERNEL:
      lm_prime(a, s);
      phase_lm(a, tick, wg, G, s, sg);
      break;
    default: break;
  }
}

// Sampler stage A for the op in flight (no-op when it does not sample).
__global__ __launch_bounds__(BLOCK) void k_samp_a(const Args* __restrict__ ap,
                                                  const RunDesc* __restrict__ run) {
  const Args& a = *ap;
  const Lds s = lds_init(a.d);
  const DevState* st = a.st;
  if (st->halt) return;
  const uint32_t i = st->op;
  if (i < run->sample_from || run->temperature == 0.0f) return;
  float m;
  uint32_t bi;
  sample_stage_a(a, st->tick, run->samp_tag0 + (i - run->sample_from), run->temperature,
                 blockIdx.x, gridDim.x, s, &m, &bi);
}

// One workgroup: sampler stage B (if the op samples) and the token to feed.
__global__ __launch_bounds__(BLOCK) void k_op(const Args* __restrict__ ap,
                                              const RunDesc* __restrict__ run) {
  const Args& a = *ap;
  const Lds s = lds_init(a.d);
  DevState* st = a.st;
  if (st->halt) return;
  const RunDesc& r = *run;
  const uint32_t i = st->op;
  uint32_t tok;
  if (i >= r.sample_from) {
    const uint32_t word = r.temperature != 0.0f ? r.words[i - r.sample_from] : 0u;
    if (!sample_one_wg(a, st->tick, r.samp_tag0 + (i - r.sample_from), r.temperature, word, s, &tok))
      return;
    if (r.mode == RUN_REPLAY) {
      if (tok != r.tokens[i]) {
        __syncthreads();
        if (threadIdx.x == 0) {
          st->first_div = (long long)i;
          st->sampled_div = tok;
          st->halt = 1;
        }
        return;
      }
      tok = cptr(r.tokens)[i];
    } else if (threadIdx.x == 0) {
      r.out_tokens[i] = tok;
    }
  } else {
    tok = r.tokens[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) st->token = tok;
}

__global__ void k_commit(const Args* __restrict__ ap, const RunDesc* __restrict__ run) {
  DevState* st = ap->st;
  if (st->halt) return;
  if (run->ring && run->mode == RUN_GENERATE) ring_commit(run->ring, st->op, st->token);
  st->pos += 1;
  st->tick += 1;
  st->op += 1;
  st->n_done += 1;
  if (run->mode == RUN_GENERATE && is_stop(*run, st->token)) st->halt = 1;
}

// The attention probabilities of one layer for the forward in flight (the
// trace of forward_ext, model.rs:486-488), written as [nh][pos + 1]: scores
// in phase_attn's order (16-element fma chains per lane group, the group's
// tree, then the scale; masked positions -inf), then p_t = exp(s_t - M) / S
// with M the context's max and S the sum of exp(s_t - M) (thread-strided
// partials in position order, then a fixed tree). One workgroup per head;
// runs after the layer's attention and before the next layer's q/k/v.
__global__ __launch_bounds__(256) void k_trace(const Args* __restrict__ ap, uint32_t l,
                                               float* __restrict__ out) {
  const Args& a = *ap;
  const Dims& d = a.d;
  const uint32_t hh = blockIdx.x, g = hh / d.group, pos = a.st->pos, n = pos + 1;
  const uint32_t hd = d.hd, lps = hd / 16;
  float* o = out + (size_t)hh * n;
  __shared__ float red[256 / WAVE];
  const float* kb = a.kc + ((size_t)l * d.nkv + g) * d.cap * d.kvs;
  float mx = -INFINITY;
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
    float part[16];
    for (uint32_t sb = 0; sb < lps; ++sb) {
      float acc = 0.0f;
      for (uint32_t e = 0; e < 16; ++e) {
        const uint32_t i = sb * 16 + e;
        const float q = __uint_as_float((uint32_t)a.mb_qkv[hh * hd + i]);
        acc = fmaf(q, kb[(size_t)t * d.kvs + i], acc);
      }
      part[sb] = acc;
    }
    for (uint32_t w = 1; w < lps; w <<= 1)
      for (uint32_t sb = 0; sb + w < lps; sb += 2 * w) part[sb] = part[sb] + part[sb + w];
    const bool masked = a.mask && t < pos && ((a.mask[t >> 5] >> (t & 31)) & 1u);
    const float sc = masked ? -INFINITY : part[0] * d.scale;
    o[t] = sc;
    mx = fmaxf(mx, sc);
  }
  mx = wave_max(mx);
  if (threadIdx.x % WAVE == 0) red[threadIdx.x / WAVE] = mx;
  __syncthreads();
  mx = red[0];
  for (uint32_t w = 1; w < blockDim.x / WAVE; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  float sum = 0.0f;
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) {
    const float e = (mx == -INFINITY) ? 0.0f : expf(o[t] - mx);
    o[t] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  if (threadIdx.x % WAVE == 0) red[threadIdx.x / WAVE] = sum;
  __syncthreads();
  float S = 0.0f;
  for (uint32_t w = 0; w < blockDim.x / WAVE; ++w) S += red[w];
  for (uint32_t t = threadIdx.x; t < n; t += blockDim.x) o[t] = o[t] / S;
}

// Length and generation base of many caches at once (batched calls).
struct StateSet {
  DevState* st;
  uint32_t pos, tick;
  // batch commits: the cache's tagged logits and chunk maxima, filled from
  // workspace logits row li
  u64 *logit, *vmax, *varg;
  uint32_t li;
};
__global__ void k_set_state(const StateSet* __restrict__ set, uint32_t n) {
  const uint32_t k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n) return;
  set[k].st->pos = set[k].pos;
  set[k].st->tick = set[k].tick;
}

// Batch commit: cache k's tagged logits and chunk (max, argmax) words from
// the workspace's logits row set[k].li, all caches in one launch (grid y = k).
__global__ void k_commit_rows(const StateSet* __restrict__ set, const u64* __restrict__ logt,
                              const u64* __restrict__ vmax, const u64* __restrict__ varg,
                              uint32_t V, uint32_t nvc) {
  const StateSet e = set[blockIdx.y];
  const size_t li = e.li;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < V + 2 * nvc;
       i += gridDim.x * blockDim.x) {
    if (i < V)
      e.logit[i] = logt[li * V + i];
    else if (i < V + nvc)
      e.vmax[i - V] = vmax[li * nvc + (i - V)];
    else
      e.varg[i - V - nvc] = varg[li * nvc + (i - V - nvc)];
  }
}

// Caller-given logits become the cache's last logits: each word tagged as
// the last forward's lm_head phase tags it, and each vocabulary chunk's
// (max, argmax) formed as phase_lm forms it. One 64-lane block per chunk.
__global__ __launch_bounds__(VCHUNK) void k_set_logits(const Args* __restrict__ ap,
                                                       const float* __restrict__ lg, uint32_t gen) {
  const Args& a = *ap;
  const uint32_t c = blockIdx.x, v = c * VCHUNK + threadIdx.x;
  float bv = -INFINITY;
  uint32_t bi = NO_INDEX;
  if (v < a.d.V) {
    const float y = lg[v];
    mb_put(a.mb_logit + v, y, gen);
    if (!isnan(y)) {
      bv = y;
      bi = v;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o);
    const uint32_t i2 = __shfl_xor(bi, o);
    if (better(v2, i2, bv, bi)) {
      bv = v2;
      bi = i2;
    }
  }
  if (threadIdx.x == 0) {
    mb_put(a.mb_vmax + c, bv, gen);
    mb_put(a.mb_varg + c, __uint_as_float(bi), gen);
  }
}

// Strip the tags of logits (or any tagged vector) into plain floats.
__global__ void k_untag(const u64* src, float* dst, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = __uint_as_float((uint32_t)src[i]);
}

// Head-major cache rows -> the reference's [len, kv_dim] layout.
__global__ void k_kv_gather(const float* src, float* dst, uint32_t len, uint32_t nkv, uint32_t hd,
                            uint32_t cap, uint32_t kvs) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t kvd = nkv * hd;
  if (i >= len * kvd) return;
  const uint32_t t = i / kvd, r = i - t * kvd, g = r / hd, dd = r - g * hd;
  dst[i] = src[((size_t)g * cap + t) * kvs + dd];
}

// ValueNorms::sync (attribution.rs:116-148): ||W_o,h . v_{t,kv(h)}|| for
// positions t0 + blockIdx.y, query head blockIdx.x, layer blockIdx.z. Thread
// i forms o_i = sum_d Wo[i][h*hd + d] * v[d] as a sequential sum of rounded
// products (built without contraction, so no fused multiply-add), the
// squares go to LDS, and one thread adds them in order i = 0, 1, ... before
// the square root -- the reference's loop order exactly.
__global__ __launch_bounds__(256) void k_value_norms(const LayerW* __restrict__ layers,
                                                     const float* __restrict__ vc, Dims d,
                                                     uint32_t cap, uint32_t t0, uint32_t nt,
                                                     float* __restrict__ out) {
  extern __shared__ float vn_lds[];  // [hd] value row, then [h] squares
  const uint32_t h = blockIdx.x, t = t0 + blockIdx.y, l = blockIdx.z;
  const uint32_t kvh = h / d.group, hd = d.hd;
  float* v = vn_lds;
  float* sq = vn_lds + hd;
  const float* vrow = vc + (((size_t)l * d.nkv + kvh) * cap + t) * d.kvs;
  for (uint32_t x = threadIdx.x; x < hd; x += blockDim.x) v[x] = vrow[x];
  __syncthreads();
  const float* wo = layers[l].wo;
  for (uint32_t i = threadIdx.x; i < d.h; i += blockDim.x) {
    const float* row = wo + (size_t)i * d.q + h * hd;
    float o = 0.0f;
    for (uint32_t x = 0; x < hd; ++x) o = o + row[x] * v[x];
    sq[i] = o * o;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (uint32_t i = 0; i < d.h; ++i) s = s + sq[i];
    out[((size_t)l * nt + blockIdx.y) * d.nh + h] = sqrtf(s);
  }
}

// ------------------------------------------------------------------ host side

struct defer_gpu_model {
  defer_gpu_config cfg;
  Dims d;
  int device = 0;
  uint32_t G = 0;  // workgroups per phase (= CUs, capped by the smallest phase)
  uint32_t ncu = 0;  // compute units of the device
  uint32_t gemm_ncu = 0;  // compute units the batched path's GEMM launches are shaped for
  uint32_t n_caches = 0;  // live caches (their argument blocks copy the layout)
  size_t lds_bytes = 0;
  hipStream_t stream = nullptr;
  float* wbuf = nullptr;
  LayerW* d_layers = nullptr;
  std::vector<LayerW> layers;
  const float* embed = nullptr;
  const float* norm = nullptr;
  const float* head = nullptr;
  float2* rope = nullptr;
  uint32_t exec_mode = DEFER_GPU_EXEC_PERSISTENT;
  const void* persistent[2] = {};  // the persistent kernel for this shape: greedy, random
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  double last_ms = 0.0;
  // Batched path (built on first use): weight panels and the workspace.
  uint32_t batch_min = 16;
  uint32_t samp_next = 1;  // tag of the next batched sampling op's chunk sums (workspace)
  size_t lds_rows = 0;  // LDS of the batched kernels that run one-token functions
  size_t lds_attn = 0;  // LDS of k_b_attn_w (the attention's scratch)
  float* panels = nullptr;
  std::vector<const float*> p_qkv, p_o, p_gu, p_d;
  const float* p_lm = nullptr;
  struct BatchWs* bw = nullptr;
  uint64_t coop_refused = 0;  // persistent launches refused and run as per-phase kernels
  // Optional timing of the batched path's GEMM and attention launches.
  bool prof = false;
  std::vector<hipEvent_t> pev;   // event pool; pairs (start, end) per timed launch
  std::vector<int> pcls;         // class of each pair: 0 GEMM, 1 attention
  std::vector<double> pflop;     // algorithmic flop of each pair
  size_t pused = 0;
  double pstat[6] = {0, 0, 0, 0, 0, 0};
};

// k_b_sample's LDS: the rows layout, with the sampler's region (stage A's
// chunk area holds NWA * SAMP_CPW chunks) wherever it runs past that
// layout's end.
static size_t samp_lds_bytes(const defer_gpu_model* m) {
  const Dims& d = m->d;
  const size_t samp_end =
      (size_t)(4 + 64 + d.lds_vec + d.lds_vec2 + samp_lds_floats(d.nvc, NWA * SAMP_CPW, d.lds_vec)) * sizeof(float);
  return std::max(m->lds_rows, samp_end);
}

// A persistent kernel compiled for this exact shape, if there is one. The
// 135M kernel has no streaming path, so it runs only where every kind's rows
// are staged.
static bool has_shape(const Dims& d, const Dims& f) {
  return d.h == f.h && d.nh == f.nh && d.nkv == f.nkv && d.hd == f.hd && d.ff == f.ff &&
         d.V == f.V && d.L == f.L && d.act == f.act && d.has_bias == f.has_bias && d.tied == f.tied;
}
template <bool RANDOM>
static const void* persistent_kernel_for(const Dims& d) {
  if (has_shape(d, fix_shape(d, DG_SHAPE_ARGS_135M)) && d.stg_mask == 0xFu)
    return (const void*)dg135::k_persistent<RANDOM>;
  if (has_shape(d, fix_shape(d, DG_SHAPE_ARGS_360M))) return (const void*)dg360::k_persistent<RANDOM>;
  if (has_shape(d, fix_shape(d, DG_SHAPE_ARGS_1B))) return (const void*)dg1b::k_persistent<RANDOM>;
  if (has_shape(d, fix_shape(d, DG_SHAPE_ARGS_8B))) return (const void*)dg8b::k_persistent<RANDOM>;
  return (const void*)k_persistent<RANDOM>;
}

struct defer_gpu_cache {
  const defer_gpu_model* m = nullptr;
  uint32_t cap = 0;
  float* kc = nullptr;
  float* vc = nullptr;
  u64* mb = nullptr;
  size_t mb_words = 0;
  DevState* st = nullptr;
  RunDesc* d_run = nullptr;
  uint32_t* d_mask = nullptr;
  uint32_t* d_tokens = nullptr;
  uint32_t* d_words = nullptr;
  uint32_t* d_stop = nullptr;
  uint32_t* d_out = nullptr;
  size_t run_cap = 0;   // capacity of d_tokens / d_words / d_out
  size_t stop_cap = 0;
  u64* h_ring = nullptr;  // pinned host words of defer_gpu_generate_cb
  u64* d_ring = nullptr;  // ... as the device addresses them
  size_t ring_cap = 0;
  float* d_logits = nullptr;
  float* d_tmp = nullptr;  // kv gather staging
  float* d_trace = nullptr;   // [L][nh][cap] staging of a traced forward
  float* trace_to = nullptr;  // set during a traced forward: where k_trace writes
  uint32_t pos = 0;        // host mirror of st->pos
  uint32_t tick = 0;
  uint32_t samp_next = 1;  // tag of the next sampling event's chunk sums (RunDesc)
  bool has_logits = false;
  hipGraphExec_t graph = nullptr;
  Args args;       // host copy
  Args* d_args = nullptr;  // device copy the kernels read
};

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// LDS of one gfx950 compute unit, all of which a workgroup may take.
static constexpr size_t LDS_BYTES_MAX = 160 * 1024;

extern "C" size_t defer_gpu_model_tensor_count(const defer_gpu_config* c) {
  const size_t per_layer = c->has_bias ? 12 : 9;
  return 1 + (size_t)c->num_layers * per_layer + 1 + (c->tie_word_embeddings ? 0 : 1);
}

static int validate(const defer_gpu_config* c) {
  if (!c) return fail(DEFER_GPU_E_INVALID, "null config");
  if (!c->vocab_size || !c->hidden_size || !c->intermediate_size || !c->num_layers ||
      !c->num_heads || !c->head_dim || !c->max_seq_len)
    return fail(DEFER_GPU_E_INVALID, "config has a zero size");
  if (c->num_kv_heads == 0 || c->num_heads % c->num_kv_heads != 0)
    return fail(DEFER_GPU_E_INVALID,
                "num_attention_heads must be a multiple of num_key_value_heads");
  if (c->head_dim % 2 != 0) return fail(DEFER_GPU_E_INVALID, "head_dim must be even for RoPE");
  const uint32_t hd = c->head_dim;
  if (hd < 16 || hd > 256 || (hd & (hd - 1)) != 0)
    return fail(DEFER_GPU_E_INVALID, "head_dim %u unsupported (need 16 * 2^k, at most 256)", hd);
  if (c->num_heads / c->num_kv_heads > MAX_GROUP)
    return fail(DEFER_GPU_E_INVALID, "GQA group larger than %u", MAX_GROUP);
  if (c->num_heads > COMB_MAX_HEADS)
    return fail(DEFER_GPU_E_INVALID, "num_attention_heads above %u", COMB_MAX_HEADS);
  if (c->hidden_size % 4 || c->intermediate_size % 4)
    return fail(DEFER_GPU_E_INVALID, "hidden and intermediate sizes must be multiples of 4");
  const uint64_t q = (uint64_t)c->num_heads * hd;
  const uint64_t mx = std::max<uint64_t>({c->hidden_size, q, c->intermediate_size});
  if (mx > 32ull * BLOCK) return fail(DEFER_GPU_E_INVALID, "vector length %llu too large",
                                      (unsigned long long)mx);
  if (c->hidden_size > (uint32_t)NWK * BLOCK)
    return fail(DEFER_GPU_E_INVALID, "hidden_size %u above %u", c->hidden_size, NWK * BLOCK);
  if (c->activation > 1) return fail(DEFER_GPU_E_INVALID, "unsupported activation");
  return DEFER_GPU_OK;
}

// The smallest matvec phase: every workgroup must own work in every phase
// (phases.h), so the persistent grid is at most this many workgroups.
static uint32_t min_phase_items(const Dims& d) {
  return std::min({d.qkv_rows / 2, d.h, d.ff, d.nvc});
}

// Everything that depends on the persistent grid G: the LDS regions (the
// weight staging of the busiest workgroup, the scratch the O phase and
// lm_head size per workgroup), the kernels' LDS attribute and the
// co-residency check. Results never depend on G (an item is computed the same
// way whichever workgroup owns it); only the layout does.
static int apply_layout(defer_gpu_model* m, uint32_t G) {
  Dims& d = m->d;
  d.lds_vec = (std::max({d.h, d.q, d.ff}) + 3) & ~3u;
  d.lds_vec2 = (2 * d.h + 3) & ~3u;
  const uint32_t hs = d.hd + 2;
  const uint32_t rmax = (d.h + G - 1) / G;
  const uint32_t scr_attn = MAX_GROUP * d.hd + 2 * d.hd + 2 * MAX_GROUP +
                            MAX_GROUP * attn_chunk(d.cap - 1) + NCW * d.hd * d.group;
  const uint32_t scr_o = INLINE_COMB_MAX + rmax;
  const uint32_t scr_comb = MAX_ACHUNKS * hs;
  const uint32_t scr_samp = samp_lds_floats(d.nvc, NWA, d.lds_vec);
  const uint32_t scr_lm = ((d.nvc + G - 1) / G) * VCHUNK;
  d.lds_scr = (std::max({scr_attn, scr_o, scr_comb, scr_samp, scr_lm, 2 * NWAVES}) + 3) & ~3u;
  // O rows skip the workgroups that take the attention items at positions
  // below 2 * ACHUNK (2 * nh items, one per query head and chunk, on the
  // first workgroups) where that leaves the busiest workgroup's O rows as
  // they are (135M shape: 576 rows on 238 instead of 256 workgroups, still
  // at most 3 each). Those workgroups' O rows waited for their attention to
  // finish, and every gate/up workgroup waits for the last O row.
  d.o_skip = 0;
  {
    const uint32_t skip = 2 * d.nh;
    if (skip < G && (d.h + G - skip - 1) / (G - skip) == (d.h + G - 1) / G) d.o_skip = skip;
  }
  // Listed results (phases.h: Pub): one entry per matvec result of a phase
  // (four per QKV item), where rows are streamed (the per-phase kernels
  // always).
  {
    const uint32_t per_wg[4] = {4 * ((d.qkv_rows / 2 + G - 1) / G), (d.h + G - 1) / G,
                                (d.ff + G - 1) / G, (d.h + G - 1) / G};
    d.lds_pub = std::max({per_wg[0], per_wg[1], per_wg[2], per_wg[3]});
  }
  // Weight staging for the persistent kernel: each kind's rows of one layer
  // for the workgroup with the most items. Where all four kinds do not fit
  // the CU's LDS, the smallest kinds that fit are staged and the others
  // streamed: a small kind's share per workgroup is a few rows, which a
  // stream pays a memory latency for, while a large kind's stream runs long
  // enough to hide it. With any kind staged the loader waves stage rows, so
  // the streamed phases lose what the loaders do for them when nothing is
  // staged (storing the listed results, warming the L2, streaming beside the
  // compute waves); so a partial staging is kept only where the staged rows
  // are at least as many bytes as the streamed ones (360M shape: QKV, O and
  // down staged, 6.4 % faster than all streamed; 1B shape: O alone would be
  // staged, 5.8 % slower).
  {
    const uint32_t n_items[4] = {d.qkv_rows / 2, d.h, d.ff, d.h};
    const uint32_t rows[4] = {2, 1, 2, 1};
    const uint32_t K[4] = {d.h, d.q, d.h, d.ff};
    size_t need[4], total = 0;
    for (int k = 0; k < 4; ++k) {
      need[k] = (size_t)(n_items[k] + G - 1) / G * rows[k] * K[k];
      total += need[k];
    }
    const size_t base = (size_t)(4 + 64 + d.lds_vec + d.lds_vec2 + d.lds_scr) * sizeof(float) +
                        (size_t)d.lds_pub * 2 * sizeof(u64);
    uint32_t mask = 0;
    if (base + total * sizeof(float) <= LDS_BYTES_MAX) {
      mask = 0xFu;
    } else {
      int order[4] = {0, 1, 2, 3};
      std::stable_sort(order, order + 4, [&](int x, int y) { return need[x] < need[y]; });
      size_t used = 0;
      for (int i = 0; i < 4; ++i) {
        const int k = order[i];
        if (base + (used + need[k]) * sizeof(float) <= LDS_BYTES_MAX) {
          mask |= 1u << k;
          used += need[k];
        }
      }
      if (used < total - used) mask = 0;
    }
    uint32_t stg = 0;
    for (int k = 0; k < 4; ++k) {
      d.stg_off[k] = stg;
      if (mask >> k & 1u) stg += (uint32_t)need[k];
    }
    d.stg_mask = mask;
    d.lds_stg = stg;
  }
  m->persistent[0] = persistent_kernel_for<false>(d);
  m->persistent[1] = persistent_kernel_for<true>(d);
  m->lds_bytes = (size_t)(4 + 64 + d.lds_vec + d.lds_vec2 + d.lds_scr + d.lds_stg) * sizeof(float) +
                 (size_t)d.lds_pub * 2 * sizeof(u64) + (d.lds_stg ? 0 : 1024);
  m->lds_rows = (size_t)(4 + 64 + d.lds_vec + d.lds_vec2 + d.lds_scr) * sizeof(float);
  // k_b_attn_f's combine: the group's chunk partials, their weights and totals.
  const uint32_t scr_fcomb = MAX_GROUP * MAX_ACHUNKS * hs + MAX_GROUP * MAX_ACHUNKS + MAX_GROUP;
  m->lds_attn = (size_t)(4 + 64 + ((std::max(scr_attn, scr_fcomb) + 3) & ~3u)) * sizeof(float);

  m->G = G;
  const void* kernels[] = {m->persistent[0], m->persistent[1], (const void*)k_phase, (const void*)k_samp_a,
                           (const void*)k_op};
  for (const void* kf : kernels) {
    const hipError_t e =
        hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)m->lds_bytes);
    if (e != hipSuccess)
      return fail(DEFER_GPU_E_HIP, "LDS attribute (%zu bytes): %s", m->lds_bytes,
                  hipGetErrorString(e));
  }
  for (const void* kf : {(const void*)k_b_sample}) {
    const hipError_t e =
        hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)samp_lds_bytes(m));
    if (e != hipSuccess)
      return fail(DEFER_GPU_E_HIP, "LDS attribute (%zu bytes): %s", samp_lds_bytes(m),
                  hipGetErrorString(e));
  }
  for (const void* kf : {(const void*)k_b_attn_w, (const void*)k_b_attn_f}) {
    const hipError_t e =
        hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)m->lds_attn);
    if (e != hipSuccess)
      return fail(DEFER_GPU_E_HIP, "LDS attribute (%zu bytes): %s", m->lds_attn, hipGetErrorString(e));
  }
  for (const void* kf : m->persistent) {
    int occ = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kf, BLOCK, m->lds_bytes);
    if (e != hipSuccess || occ < 1)
      return fail(DEFER_GPU_E_HIP, "persistent kernel does not fit a CU (occupancy %d)", occ);
  }
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_model_create(const defer_gpu_config* cfg, const float* const* tensors,
                                      size_t n_tensors, uint32_t flags, defer_gpu_model** out) {
  if (!out) return fail(DEFER_GPU_E_INVALID, "null output handle");
  *out = nullptr;
  int rc = validate(cfg);
  if (rc) return rc;
  (void)flags;
  if (!tensors || n_tensors != defer_gpu_model_tensor_count(cfg))
    return fail(DEFER_GPU_E_INVALID, "expected %zu tensors, got %zu",
                defer_gpu_model_tensor_count(cfg), n_tensors);
  for (size_t i = 0; i < n_tensors; ++i)
    if (!tensors[i]) return fail(DEFER_GPU_E_INVALID, "tensor %zu is null", i);

  defer_gpu_model* m = new defer_gpu_model();
  ++g_live_models;
  m->cfg = *cfg;
  Dims& d = m->d;
  d.h = cfg->hidden_size;
  d.nh = cfg->num_heads;
  d.nkv = cfg->num_kv_heads;
  d.hd = cfg->head_dim;
  d.half = d.hd / 2;
  d.ff = cfg->intermediate_size;
  d.V = cfg->vocab_size;
  d.L = cfg->num_layers;
  d.q = d.nh * d.hd;
  d.kv = d.nkv * d.hd;
  d.qkv_rows = d.q + 2 * d.kv;
  d.group = d.nh / d.nkv;
  d.act = cfg->activation;
  d.has_bias = cfg->has_bias;
  d.tied = cfg->tie_word_embeddings;
  d.kvs = std::max<uint32_t>(d.hd, 32);
  d.nvc = (d.V + VCHUNK - 1) / VCHUNK;
  d.eps = cfg->rms_norm_eps;
  d.scale = 1.0f / sqrtf((float)d.hd);  // model.rs:426
  d.cap = cfg->max_seq_len;

  auto cleanup = [&](int code) {
    defer_gpu_model_destroy(m);
    return code;
  };
  hipError_t e = hipGetDevice(&m->device);
  if (e != hipSuccess) return cleanup(fail(DEFER_GPU_E_HIP, "hipGetDevice: %s", hipGetErrorString(e)));
  if (m->device >= 0 && m->device < 64) g_devices_used |= 1ull << m->device;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, m->device);
  if (e != hipSuccess)
    return cleanup(fail(DEFER_GPU_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e)));
  // Every workgroup must own work in every matvec phase (see phases.h): cap G
  // by the smallest phase.
  const uint32_t min_items = min_phase_items(d);
  m->ncu = (uint32_t)prop.multiProcessorCount;
  m->gemm_ncu = m->ncu;

  // Weight layout: one allocation, each tensor 256-byte aligned; q/k/v rows
  // are stored back to back as one [q + 2kv, h] matrix.
  const size_t h = d.h, q = d.q, kv = d.kv, ff = d.ff, V = d.V;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t o = off;
    off += align256(n * sizeof(float));
    return o;
  };
  const size_t o_embed = take(V * h);
  struct LOff { size_t an, qkv, b, wo, fn, wg, wu, wd; };
  std::vector<LOff> lo(d.L);
  for (uint32_t l = 0; l < d.L; ++l) {
    lo[l].an = take(h);
    lo[l].qkv = take((q + 2 * kv) * h);
    lo[l].b = d.has_bias ? take(q + 2 * kv) : 0;
    lo[l].wo = take(h * q);
    lo[l].fn = take(h);
    lo[l].wg = take(ff * h);
    lo[l].wu = take(ff * h);
    lo[l].wd = take(h * ff);
  }
  const size_t o_norm = take(h);
  const size_t o_head = d.tied ? o_embed : take(V * h);
  const size_t total = off;

  e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return cleanup(fail(DEFER_GPU_E_HIP, "stream: %s", hipGetErrorString(e)));
  e = counted_malloc(&m->wbuf, total);
  if (e != hipSuccess)
    return cleanup(fail(DEFER_GPU_E_HIP, "hipMalloc(%zu) for weights: %s", total,
                        hipGetErrorString(e)));
  char* base = reinterpret_cast<char*>(m->wbuf);
  auto up = [&](size_t o, const float* src, size_t n) {
    return hipMemcpy(base + o, src, n * sizeof(float), hipMemcpyHostToDevice);
  };
  // A matrix that consumes an RMSNorm output is stored with the norm weight
  // folded into its columns, W'[r][j] = W[r][j] * w_norm[j], so the kernels
  // compute (x * inv) * w_norm . W as inv * (W' . x). Unit norm weights leave
  // the matrix bit-identical.
  std::vector<float> stage;
  auto up_folded = [&](size_t o, const float* src, size_t rows, const float* wn) {
    bool unit = true;
    for (size_t j = 0; j < h && unit; ++j) unit = (wn[j] == 1.0f);
    if (unit) return up(o, src, rows * h);
    const size_t chunk_rows = std::max<size_t>(1, (size_t)(4u << 20) / h);
    stage.resize(chunk_rows * h);
    for (size_t r0 = 0; r0 < rows; r0 += chunk_rows) {
      const size_t nr = std::min(chunk_rows, rows - r0);
      for (size_t r = 0; r < nr; ++r)
        for (size_t j = 0; j < h; ++j) stage[r * h + j] = src[(r0 + r) * h + j] * wn[j];
      const hipError_t er = up(o + r0 * h * sizeof(float), stage.data(), nr * h);
      if (er != hipSuccess) return er;
    }
    return hipSuccess;
  };
  size_t k = 0;
  e = up(o_embed, tensors[k++], V * h);
  for (uint32_t l = 0; l < d.L && e == hipSuccess; ++l) {
    const float* an = tensors[k++];
    e = up(lo[l].an, an, h);
    const float* wq = tensors[k++];
    const float* bq = d.has_bias ? tensors[k++] : nullptr;
    const float* wk = tensors[k++];
    const float* bk = d.has_bias ? tensors[k++] : nullptr;
    const float* wv = tensors[k++];
    const float* bv = d.has_bias ? tensors[k++] : nullptr;
    if (e == hipSuccess) e = up_folded(lo[l].qkv, wq, q, an);
    if (e == hipSuccess) e = up_folded(lo[l].qkv + q * h * sizeof(float), wk, kv, an);
    if (e == hipSuccess) e = up_folded(lo[l].qkv + (q + kv) * h * sizeof(float), wv, kv, an);
    if (d.has_bias) {
      if (e == hipSuccess) e = up(lo[l].b, bq, q);
      if (e == hipSuccess) e = up(lo[l].b + q * sizeof(float), bk, kv);
      if (e == hipSuccess) e = up(lo[l].b + (q + kv) * sizeof(float), bv, kv);
    }
    if (e == hipSuccess) e = up(lo[l].wo, tensors[k++], h * q);
    const float* fnw = tensors[k++];
    if (e == hipSuccess) e = up(lo[l].fn, fnw, h);
    if (e == hipSuccess) e = up_folded(lo[l].wg, tensors[k++], ff, fnw);
    if (e == hipSuccess) e = up_folded(lo[l].wu, tensors[k++], ff, fnw);
    if (e == hipSuccess) e = up(lo[l].wd, tensors[k++], h * ff);
  }
  if (e == hipSuccess) e = up(o_norm, tensors[k++], h);
  if (e == hipSuccess && !d.tied) e = up(o_head, tensors[k++], V * h);
  if (e != hipSuccess)
    return cleanup(fail(DEFER_GPU_E_HIP, "weight upload: %s", hipGetErrorString(e)));

  auto at = [&](size_t o) { return reinterpret_cast<const float*>(base + o); };
  m->layers.resize(d.L);
  for (uint32_t l = 0; l < d.L; ++l) {
    LayerW& W = m->layers[l];
    W.attn_norm = at(lo[l].an);
    W.wqkv = at(lo[l].qkv);
    W.bqkv = d.has_bias ? at(lo[l].b) : nullptr;
    W.wo = at(lo[l].wo);
    W.ffn_norm = at(lo[l].fn);
    W.wg = at(lo[l].wg);
    W.wu = at(lo[l].wu);
    W.wd = at(lo[l].wd);
  }
  m->embed = at(o_embed);
  m->norm = at(o_norm);
  m->head = at(o_head);
  e = counted_malloc(&m->d_layers, sizeof(LayerW) * d.L);
  if (e == hipSuccess)
    e = hipMemcpy(m->d_layers, m->layers.data(), sizeof(LayerW) * d.L, hipMemcpyHostToDevice);
  if (e != hipSuccess) return cleanup(fail(DEFER_GPU_E_HIP, "layer table: %s", hipGetErrorString(e)));

  // RoPE tables: inv_freq in f64 then f32 (model.rs:348-353); angle and
  // cos/sin in f32 with the host libm (model.rs:438-445).
  std::vector<float> inv_freq(d.half);
  for (uint32_t i = 0; i < d.half; ++i) {
    const double exponent = (double)(2 * i) / (double)d.hd;
    inv_freq[i] = (float)(1.0 / pow((double)cfg->rope_theta, exponent));
  }
  std::vector<float2> rope((size_t)d.cap * d.half);
  for (uint32_t p = 0; p < d.cap; ++p)
    for (uint32_t i = 0; i < d.half; ++i) {
      const float angle = (float)p * inv_freq[i];
      rope[(size_t)p * d.half + i] = make_float2(cosf(angle), sinf(angle));
    }
  e = counted_malloc(&m->rope, rope.size() * sizeof(float2));
  if (e == hipSuccess)
    e = hipMemcpy(m->rope, rope.data(), rope.size() * sizeof(float2), hipMemcpyHostToDevice);
  if (e != hipSuccess) return cleanup(fail(DEFER_GPU_E_HIP, "rope table: %s", hipGetErrorString(e)));

  rc = apply_layout(m, std::min<uint32_t>(m->ncu, min_items));
  if (rc) return cleanup(rc);
  {
    const void* gk[] = {
        (const void*)k_gemm<1, GO_PLAIN, false>, (const void*)k_gemm<1, GO_RESID, false>,
        (const void*)k_gemm<1, GO_TAG, false>,   (const void*)k_gemm<2, GO_PLAIN, false>,
        (const void*)k_gemm<2, GO_RESID, false>, (const void*)k_gemm<2, GO_TAG, false>,
        (const void*)k_gemm<4, GO_PLAIN, false>, (const void*)k_gemm<4, GO_RESID, false>,
        (const void*)k_gemm<4, GO_TAG, false>,   (const void*)k_gemm<1, GO_PLAIN, true>,
        (const void*)k_gemm<1, GO_RESID, true>,  (const void*)k_gemm<1, GO_TAG, true>,
        (const void*)k_gemm<2, GO_PLAIN, true>,  (const void*)k_gemm<2, GO_RESID, true>,
        (const void*)k_gemm<2, GO_TAG, true>,    (const void*)k_gemm<4, GO_PLAIN, true>,
        (const void*)k_gemm<4, GO_RESID, true>,  (const void*)k_gemm<4, GO_TAG, true>};
    const int tn[] = {1, 1, 1, 2, 2, 2, 4, 4, 4, 1, 1, 1, 2, 2, 2, 4, 4, 4};
    for (int i = 0; i < 18; ++i) {
      e = hipFuncSetAttribute(gk[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)gemm_lds_bytes(tn[i]));
      if (e != hipSuccess)
        return cleanup(fail(DEFER_GPU_E_HIP, "LDS attribute (GEMM): %s", hipGetErrorString(e)));
    }
    const void* gn[] = {(const void*)k_gemm_n<GO_PLAIN, false>, (const void*)k_gemm_n<GO_RESID, false>,
                        (const void*)k_gemm_n<GO_TAG, false>,   (const void*)k_gemm_n<GO_PLAIN, true>,
                        (const void*)k_gemm_n<GO_RESID, true>,  (const void*)k_gemm_n<GO_TAG, true>};
    for (const void* kf : gn) {
      e = hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_n_lds_bytes());
      if (e != hipSuccess)
        return cleanup(fail(DEFER_GPU_E_HIP, "LDS attribute (narrow GEMM): %s", hipGetErrorString(e)));
    }
    for (const void* kf : {(const void*)k_gemm_q<false>, (const void*)k_gemm_q<true>}) {
      e = hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm_q_lds_bytes());
      if (e != hipSuccess)
        return cleanup(fail(DEFER_GPU_E_HIP, "LDS attribute (quarter GEMM): %s", hipGetErrorString(e)));
    }
  }
  e = hipFuncSetAttribute((const void*)k_b_attn_tile, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)attn_tile_lds(MAX_GROUP));
  if (e != hipSuccess)
    return cleanup(fail(DEFER_GPU_E_HIP, "LDS attribute (tiled attention): %s", hipGetErrorString(e)));
  if (hipEventCreate(&m->ev0) != hipSuccess || hipEventCreate(&m->ev1) != hipSuccess)
    return cleanup(fail(DEFER_GPU_E_HIP, "event create"));
  *out = m;
  return DEFER_GPU_OK;
}

static void batch_ws_free(defer_gpu_model* m);

extern "C" void defer_gpu_model_destroy(defer_gpu_model* m) {
  if (!m) return;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  batch_ws_free(m);
  for (hipEvent_t e : m->pev) (void)hipEventDestroy(e);
  (void)hipFree(m->panels);
  (void)hipFree(m->wbuf);
  (void)hipFree(m->d_layers);
  (void)hipFree(m->rope);
  if (m->ev0) (void)hipEventDestroy(m->ev0);
  if (m->ev1) (void)hipEventDestroy(m->ev1);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
  --g_live_models;
}

extern "C" int defer_gpu_model_set_exec(defer_gpu_model* m, uint32_t mode) {
  if (!m || mode > DEFER_GPU_EXEC_EAGER) return fail(DEFER_GPU_E_INVALID, "bad exec mode");
  m->exec_mode = mode;
  return DEFER_GPU_OK;
}

extern "C" double defer_gpu_last_device_ms(const defer_gpu_model* m) { return m ? m->last_ms : 0.0; }

extern "C" int defer_gpu_model_set_grid(defer_gpu_model* m, uint32_t workgroups,
                                        uint32_t gemm_cus) {
  if (!m) return fail(DEFER_GPU_E_INVALID, "null model");
  if (m->n_caches) return fail(DEFER_GPU_E_INVALID, "set the grid before creating caches");
  const uint32_t top = std::min(m->ncu, min_phase_items(m->d));
  const uint32_t G = workgroups ? std::min(workgroups, top) : top;
  const int rc = apply_layout(m, G);
  if (rc) return rc;
  m->gemm_ncu = gemm_cus ? std::min(gemm_cus, m->ncu) : m->ncu;
  return DEFER_GPU_OK;
}

// ------------------------------------------------------------------ caches

static int cache_alloc(const defer_gpu_model* m, uint32_t cap, defer_gpu_cache* c) {
  const Dims& d = m->d;
  c->m = m;
  ++const_cast<defer_gpu_model*>(m)->n_caches;
  ++g_live_caches;
  c->cap = cap;
  const size_t kvn = (size_t)d.L * d.nkv * cap * d.kvs;
  HIP_TRY(counted_malloc(&c->kc, kvn * sizeof(float)));
  HIP_TRY(counted_malloc(&c->vc, kvn * sizeof(float)));
  const size_t hs = d.hd + 2;
  // xo, xd, g: MB_REPS replicas of one block, each on its own 32 KB boundary
  const size_t rep_words = ((size_t)2 * d.h + d.ff + 4095) / 4096 * 4096;
  const size_t base_words = (d.qkv_rows + (size_t)d.nh * MAX_ACHUNKS * hs + d.q + 2 * (size_t)d.V +
                             5 * (size_t)d.nvc + 64 + 4095) / 4096 * 4096;
  const size_t words = base_words + MB_REPS * rep_words;
  c->mb_words = words;
  HIP_TRY(counted_malloc(&c->mb, words * sizeof(u64)));
  HIP_TRY(hipMemset(c->mb, 0, words * sizeof(u64)));
  HIP_TRY(counted_malloc(&c->st, sizeof(DevState)));
  HIP_TRY(hipMemset(c->st, 0, sizeof(DevState)));
  HIP_TRY(counted_malloc(&c->d_run, sizeof(RunDesc)));
  HIP_TRY(counted_malloc(&c->d_mask, ((cap + 31) / 32) * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&c->d_logits, (size_t)d.V * sizeof(float)));
  Args& a = c->args;
  a.d = d;
  a.d.cap = cap;
  a.layers = m->d_layers;
  a.embed = m->embed;
  a.norm = m->norm;
  a.head = m->head;
  a.rope = m->rope;
  a.kc = c->kc;
  a.vc = c->vc;
  u64* p = c->mb;
  a.mb_qkv = p; p += d.qkv_rows;
  a.mb_part = p; p += (size_t)d.nh * MAX_ACHUNKS * hs;
  a.mb_att = p; p += d.q;
  a.mb_logit = p; p += d.V;
  a.mb_vmax = p; p += d.nvc;
  a.mb_varg = p; p += d.nvc;
  a.mb_vsum = p; p += d.nvc;
  a.mb_p = p; p += d.V;
  a.mb_psum = p; p += d.nvc;
  a.mb_qsum = p; p += d.nvc;
  p = c->mb + base_words;
  a.mb_xo = p;
  a.mb_xd = p + d.h;
  a.mb_g = p + 2 * d.h;
  a.rep_words = (uint32_t)rep_words;
  a.st = c->st;
  a.mask = nullptr;
  HIP_TRY(counted_malloc(&c->d_args, sizeof(Args)));
  HIP_TRY(hipMemcpy(c->d_args, &a, sizeof(Args), hipMemcpyHostToDevice));
  return DEFER_GPU_OK;
}

static int sync_args(defer_gpu_cache* c) {
  HIP_TRY(hipMemcpy(c->d_args, &c->args, sizeof(Args), hipMemcpyHostToDevice));
  return DEFER_GPU_OK;
}

static void cache_free(defer_gpu_cache* c) {
  if (!c) return;
  --g_live_caches;  // every cache_free follows a cache_alloc
  if (c->m) --const_cast<defer_gpu_model*>(c->m)->n_caches;
  if (c->m && c->m->stream) (void)hipStreamSynchronize(c->m->stream);
  if (c->graph) (void)hipGraphExecDestroy(c->graph);
  (void)hipFree(c->kc);
  (void)hipFree(c->vc);
  (void)hipFree(c->mb);
  (void)hipFree(c->st);
  (void)hipFree(c->d_run);
  (void)hipFree(c->d_mask);
  (void)hipFree(c->d_tokens);
  (void)hipFree(c->d_words);
  (void)hipFree(c->d_stop);
  (void)hipFree(c->d_out);
  (void)hipFree(c->d_logits);
  (void)hipFree(c->d_tmp);
  (void)hipFree(c->d_trace);
  (void)hipFree(c->d_args);
  if (c->h_ring) (void)hipHostFree(c->h_ring);
}

extern "C" int defer_gpu_cache_create(const defer_gpu_model* m, uint32_t capacity,
                                      defer_gpu_cache** out) {
  if (!m || !out) return fail(DEFER_GPU_E_INVALID, "null argument");
  *out = nullptr;
  const uint32_t cap = capacity ? capacity : m->cfg.max_seq_len;
  if (cap > m->cfg.max_seq_len)
    return fail(DEFER_GPU_E_INVALID, "capacity %u exceeds max_seq_len %u", cap,
                m->cfg.max_seq_len);
  defer_gpu_cache* c = new defer_gpu_cache();
  const int rc = cache_alloc(m, cap, c);
  if (rc) {
    cache_free(c);
    delete c;
    return rc;
  }
  *out = c;
  return DEFER_GPU_OK;
}

extern "C" void defer_gpu_cache_destroy(defer_gpu_cache* c) {
  if (!c) return;
  cache_free(c);
  delete c;
}

extern "C" uint32_t defer_gpu_cache_len(const defer_gpu_cache* c) { return c ? c->pos : 0; }
extern "C" uint32_t defer_gpu_cache_capacity(const defer_gpu_cache* c) { return c ? c->cap : 0; }

static int push_state(defer_gpu_cache* c) {
  DevState h;
  HIP_TRY(hipMemcpy(&h, c->st, sizeof(h), hipMemcpyDeviceToHost));
  h.pos = c->pos;
  h.tick = c->tick;
  HIP_TRY(hipMemcpy(c->st, &h, sizeof(h), hipMemcpyHostToDevice));
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_cache_truncate(defer_gpu_cache* c, uint32_t n) {
  if (!c) return fail(DEFER_GPU_E_INVALID, "null cache");
  if (n >= c->pos) return DEFER_GPU_OK;
  c->pos = n;
  c->has_logits = false;
  return push_state(c);
}

extern "C" int defer_gpu_cache_clone(const defer_gpu_cache* src, defer_gpu_cache** out) {
  if (!src || !out) return fail(DEFER_GPU_E_INVALID, "null argument");
  *out = nullptr;
  defer_gpu_cache* c = new defer_gpu_cache();
  int rc = cache_alloc(src->m, src->cap, c);
  if (rc) {
    cache_free(c);
    delete c;
    return rc;
  }
  const Dims& d = src->m->d;
  const size_t kvn = (size_t)d.L * d.nkv * src->cap * d.kvs;
  hipError_t e = hipMemcpy(c->kc, src->kc, kvn * sizeof(float), hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(c->vc, src->vc, kvn * sizeof(float), hipMemcpyDeviceToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(c->mb, src->mb, src->mb_words * sizeof(u64), hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(c->st, src->st, sizeof(DevState), hipMemcpyDeviceToDevice);
  if (e != hipSuccess) {
    cache_free(c);
    delete c;
    return fail(DEFER_GPU_E_HIP, "cache clone: %s", hipGetErrorString(e));
  }
  c->pos = src->pos;
  c->tick = src->tick;
  c->samp_next = src->samp_next;
  c->has_logits = src->has_logits;
  *out = c;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_cache_read(const defer_gpu_cache* cc, uint32_t layer, float* keys,
                                    float* values) {
  defer_gpu_cache* c = const_cast<defer_gpu_cache*>(cc);
  if (!c) return fail(DEFER_GPU_E_INVALID, "null cache");
  const Dims& d = c->m->d;
  if (layer >= d.L) return fail(DEFER_GPU_E_INVALID, "layer %u out of range", layer);
  const size_t n = (size_t)c->pos * d.kv;
  if (n == 0) return DEFER_GPU_OK;
  if (!c->d_tmp) HIP_TRY(counted_malloc(&c->d_tmp, (size_t)c->cap * d.kv * sizeof(float)));
  const hipStream_t s = c->m->stream;
  const size_t per_layer = (size_t)d.nkv * c->cap * d.kvs;
  for (int which = 0; which < 2; ++which) {
    float* dst = which ? values : keys;
    if (!dst) continue;
    const float* src = (which ? c->vc : c->kc) + layer * per_layer;
    const uint32_t nb = (uint32_t)((n + 255) / 256);
    k_kv_gather<<<nb, 256, 0, s>>>(src, c->d_tmp, c->pos, d.nkv, d.hd, c->cap, d.kvs);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(dst, c->d_tmp, n * sizeof(float), hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
  }
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_cache_shape(const defer_gpu_cache* c, uint32_t* layers, uint32_t* kv_dim) {
  if (!c || !layers || !kv_dim) return fail(DEFER_GPU_E_INVALID, "null argument");
  *layers = c->m->d.L;
  *kv_dim = c->m->d.kv;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_value_norms(const defer_gpu_cache* cc, uint32_t t0, uint32_t t1,
                                     float* out) {
  defer_gpu_cache* c = const_cast<defer_gpu_cache*>(cc);
  if (!c || !out) return fail(DEFER_GPU_E_INVALID, "null cache or output");
  if (t0 > t1 || t1 > c->pos)
    return fail(DEFER_GPU_E_INVALID, "positions [%u, %u) outside the cache's %u", t0, t1, c->pos);
  const defer_gpu_model* m = c->m;
  const Dims& d = m->d;
  const uint32_t nt = t1 - t0;
  if (nt == 0) return DEFER_GPU_OK;
  const size_t n = (size_t)d.L * nt * d.nh;
  float* dout = nullptr;
  HIP_TRY(counted_malloc(&dout, n * sizeof(float)));
  const hipStream_t s = m->stream;
  k_value_norms<<<dim3(d.nh, nt, d.L), 256, (d.hd + d.h) * sizeof(float), s>>>(
      m->d_layers, c->vc, d, c->cap, t0, nt, dout);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(out, dout, n * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(dout);
  if (e != hipSuccess) return fail(DEFER_GPU_E_HIP, "value norms: %s", hipGetErrorString(e));
  return DEFER_GPU_OK;
}

// ------------------------------------------------------------------ runs

static int ensure_run_buffers(defer_gpu_cache* c, size_t n_ops, size_t n_stop) {
  // The capacities are zero while the buffers are being replaced, so a failed
  // allocation leaves no size that a later call would trust.
  if (n_ops > c->run_cap || !c->d_tokens || !c->d_words || !c->d_out) {
    (void)hipFree(c->d_tokens);
    (void)hipFree(c->d_words);
    (void)hipFree(c->d_out);
    c->d_tokens = c->d_words = c->d_out = nullptr;
    c->run_cap = 0;
    const size_t cap = std::max<size_t>(n_ops, 1024);
    HIP_TRY(counted_malloc(&c->d_tokens, cap * sizeof(uint32_t)));
    HIP_TRY(counted_malloc(&c->d_words, cap * sizeof(uint32_t)));
    HIP_TRY(counted_malloc(&c->d_out, cap * sizeof(uint32_t)));
    c->run_cap = cap;
  }
  if (n_stop > c->stop_cap || !c->d_stop) {
    (void)hipFree(c->d_stop);
    c->d_stop = nullptr;
    c->stop_cap = 0;
    const size_t cap = std::max<size_t>(n_stop, 16);
    HIP_TRY(counted_malloc(&c->d_stop, cap * sizeof(uint32_t)));
    c->stop_cap = cap;
  }
  return DEFER_GPU_OK;
}

static int launch_op_kernels(defer_gpu_cache* c, hipStream_t s) {
  const defer_gpu_model* m = c->m;
  const Dims& d = m->d;
  const Args* a = c->d_args;
  const uint32_t G = m->G;
  const size_t lds = m->lds_bytes;
  k_samp_a<<<G, BLOCK, lds, s>>>(a, c->d_run);
  k_op<<<1, BLOCK, lds, s>>>(a, c->d_run);
  for (uint32_t l = 0; l < d.L; ++l) {
    for (uint32_t ph = 0; ph < PH_PER_LAYER; ++ph) {
      k_phase<<<G, BLOCK, lds, s>>>(a, ph, l);
      if (ph == PH_COMB && c->trace_to)
        k_trace<<<d.nh, 256, 0, s>>>(a, l, c->trace_to + (size_t)l * d.nh * (c->pos + 1));
    }
  }
  k_phase<<<G, BLOCK, lds, s>>>(a, PH_LM_KERNEL, 0);
  k_commit<<<1, 1, 0, s>>>(a, c->d_run);
  HIP_TRY(hipGetLastError());
  return DEFER_GPU_OK;
}

// Queues n_ops ops described by `r` (host copy, device pointers filled in)
// on the model's stream; run_finish waits for them.
static int run_launch(defer_gpu_cache* c, RunDesc r, bool force_eager) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(c->m);
  const hipStream_t s = m->stream;
  HIP_TRY(hipMemcpyAsync(c->d_run, &r, sizeof(r), hipMemcpyHostToDevice, s));
  k_begin<<<1, 1, 0, s>>>(c->st);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipEventRecord(m->ev0, s));
  const uint32_t mode = force_eager ? DEFER_GPU_EXEC_EAGER : m->exec_mode;
  if (r.n_ops > 0) {
    if (mode == DEFER_GPU_EXEC_PERSISTENT) {
      const Args* a = c->d_args;
      const RunDesc* dr = c->d_run;
      void* params[] = {&a, &dr};
      const hipError_t e = hipLaunchCooperativeKernel(m->persistent[r.temperature != 0.0f], dim3(m->G),
                                                      dim3(BLOCK), params,
                                                      (unsigned)m->lds_bytes, s);
      if (e != hipSuccess) {
        // Refused at launch (nothing ran): the device grants cooperative
        // launches to one process at a time. The per-phase kernels compute
        // the same bits without one.
        (void)hipGetLastError();
        ++m->coop_refused;
        for (uint32_t i = 0; i < r.n_ops; ++i) {
          const int rc = launch_op_kernels(c, s);
          if (rc) return rc;
        }
      }
    } else if (mode == DEFER_GPU_EXEC_GRAPH) {
      if (!c->graph) {
        hipGraph_t g;
        HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        const int rc = launch_op_kernels(c, s);
        hipError_t e = hipStreamEndCapture(s, &g);
        if (rc) return rc;
        if (e != hipSuccess) return fail(DEFER_GPU_E_HIP, "graph capture: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&c->graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess)
          return fail(DEFER_GPU_E_HIP, "graph instantiate: %s", hipGetErrorString(e));
      }
      for (uint32_t i = 0; i < r.n_ops; ++i) HIP_TRY(hipGraphLaunch(c->graph, s));
    } else {
      for (uint32_t i = 0; i < r.n_ops; ++i) {
        const int rc = launch_op_kernels(c, s);
        if (rc) return rc;
      }
    }
  }
  HIP_TRY(hipEventRecord(m->ev1, s));
  return DEFER_GPU_OK;
}

static int run_finish(defer_gpu_cache* c) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(c->m);
  HIP_TRY(hipStreamSynchronize(m->stream));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->last_ms = ms;
  DevState h;
  HIP_TRY(hipMemcpy(&h, c->st, sizeof(h), hipMemcpyDeviceToHost));
  if (h.abort) {
    c->has_logits = false;
    return fail(DEFER_GPU_E_TIMEOUT, "a device-side wait exceeded its bound; cache state is undefined");
  }
  c->pos = h.pos;
  c->tick = h.tick;
  if (h.n_done > 0) c->has_logits = true;
  return DEFER_GPU_OK;
}

static int run_ops(defer_gpu_cache* c, RunDesc r, bool force_eager) {
  const int rc = run_launch(c, r, force_eager);
  return rc ? rc : run_finish(c);
}

static DevState read_state(defer_gpu_cache* c) {
  DevState h;
  memset(&h, 0, sizeof(h));
  if (hipMemcpy(&h, c->st, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) h.first_div = -2;
  return h;
}

static int check_pair(const defer_gpu_model* m, const defer_gpu_cache* c) {
  if (!m || !c) return fail(DEFER_GPU_E_INVALID, "null model or cache");
  if (c->m != m) return fail(DEFER_GPU_E_INVALID, "cache belongs to another model");
  return DEFER_GPU_OK;
}

static int copy_logits(defer_gpu_cache* c, float* out) {
  const Dims& d = c->m->d;
  const hipStream_t s = c->m->stream;
  k_untag<<<(d.V + 255) / 256, 256, 0, s>>>(c->args.mb_logit, c->d_logits, d.V);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipMemcpyAsync(out, c->d_logits, (size_t)d.V * sizeof(float), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_cache_set_logits(defer_gpu_cache* c, const float* logits) {
  if (!c || !logits) return fail(DEFER_GPU_E_INVALID, "null argument");
  if (c->tick == 0)
    return fail(DEFER_GPU_E_NO_LOGITS, "no forward has run on this cache yet");
  const Dims& d = c->m->d;
  const hipStream_t s = c->m->stream;
  HIP_TRY(hipMemcpyAsync(c->d_logits, logits, (size_t)d.V * sizeof(float), hipMemcpyHostToDevice, s));
  k_set_logits<<<d.nvc, VCHUNK, 0, s>>>(c->d_args, c->d_logits, gen_lm(d, c->tick - 1));
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(s));
  c->has_logits = true;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_last_logits(const defer_gpu_cache* cc, float* logits_out) {
  defer_gpu_cache* c = const_cast<defer_gpu_cache*>(cc);
  if (!c || !logits_out) return fail(DEFER_GPU_E_INVALID, "null argument");
  if (!c->has_logits) return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  return copy_logits(c, logits_out);
}

static int feed_tokens(const defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* tokens,
                       size_t n, bool eager) {
  for (size_t i = 0; i < n; ++i)
    if (tokens[i] >= m->d.V) return fail(DEFER_GPU_E_TOKEN, "token id %u out of range", tokens[i]);
  if ((size_t)c->pos + n > c->cap)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  int rc = ensure_run_buffers(c, n, 0);
  if (rc) return rc;
  if (n) HIP_TRY(hipMemcpy(c->d_tokens, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice));
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = (uint32_t)n;
  r.mode = RUN_FEED;
  r.sample_from = (uint32_t)n;
  r.tokens = c->d_tokens;
  r.words = c->d_words;
  r.stop = c->d_stop;
  r.out_tokens = c->d_out;
  return run_ops(c, r, eager);
}

extern "C" int defer_gpu_forward(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t token,
                                 const uint32_t* masked, size_t n_masked, float* logits_out,
                                 float* trace_out) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  if (token >= m->d.V) return fail(DEFER_GPU_E_TOKEN, "token id %u out of range", token);
  if (c->pos >= c->cap)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  bool use_mask = false;
  if (n_masked) {
    std::vector<uint32_t> bits((c->cap + 31) / 32, 0u);
    for (size_t i = 0; i < n_masked; ++i)
      if (masked[i] < c->pos) {
        bits[masked[i] >> 5] |= 1u << (masked[i] & 31);
        use_mask = true;
      }
    if (use_mask)
      HIP_TRY(hipMemcpy(c->d_mask, bits.data(), bits.size() * sizeof(uint32_t),
                        hipMemcpyHostToDevice));
  }
  if (use_mask) {
    c->args.mask = c->d_mask;
    rc = sync_args(c);
    if (rc) return rc;
  }
  const uint32_t pos0 = c->pos;
  if (trace_out) {
    if (!c->d_trace)
      HIP_TRY(counted_malloc(&c->d_trace, (size_t)m->d.L * m->d.nh * c->cap * sizeof(float)));
    c->trace_to = c->d_trace;
  }
  rc = feed_tokens(m, c, &token, 1, use_mask || trace_out);
  c->trace_to = nullptr;
  if (!rc && trace_out)
    rc = hipMemcpy(trace_out, c->d_trace, (size_t)m->d.L * m->d.nh * (pos0 + 1) * sizeof(float),
                   hipMemcpyDeviceToHost) == hipSuccess
             ? DEFER_GPU_OK
             : fail(DEFER_GPU_E_HIP, "trace copy failed");
  if (use_mask) {
    c->args.mask = nullptr;
    const int rc2 = sync_args(c);
    if (!rc) rc = rc2;
  }
  if (rc) return rc;
  return logits_out ? copy_logits(c, logits_out) : DEFER_GPU_OK;
}

static bool use_batch(const defer_gpu_model* m, size_t n);
static int feed_batched(defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* tokens, size_t n);
static int replay_batched(defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* history,
                          size_t n, size_t plen, float T, const uint32_t* words,
                          int64_t* first_div, uint32_t* sampled_at_div);

// Device time of a host-driven sequence of launches on the model's stream.
template <class F>
static int timed(const defer_gpu_model* mc, F body) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(mc);
  HIP_TRY(hipEventRecord(m->ev0, m->stream));
  const int rc = body();
  if (rc) return rc;
  HIP_TRY(hipEventRecord(m->ev1, m->stream));
  HIP_TRY(hipEventSynchronize(m->ev1));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->last_ms = ms;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_prompt(const defer_gpu_model* m, defer_gpu_cache* c,
                                const uint32_t* tokens, size_t n_tokens) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  if (n_tokens && !tokens) return fail(DEFER_GPU_E_INVALID, "null tokens");
  // Session::prompt feeds token by token (engine.rs:62-71): the tokens before
  // the first one that fails -- out of range (model.rs:417-419), or past the
  // capacity (model.rs:420-422), checked in that order -- are fed and stay
  // in the cache, then the error is returned.
  size_t n_ok = 0;
  int err = DEFER_GPU_OK;
  uint32_t bad = 0;
  for (; n_ok < n_tokens; ++n_ok) {
    if (tokens[n_ok] >= m->d.V) {
      err = DEFER_GPU_E_TOKEN;
      bad = tokens[n_ok];
      break;
    }
    if ((size_t)c->pos + n_ok >= c->cap) {
      err = DEFER_GPU_E_CONTEXT;
      break;
    }
  }
  if (use_batch(m, n_ok))
    rc = timed(m, [&] { return feed_batched(const_cast<defer_gpu_model*>(m), c, tokens, n_ok); });
  else
    rc = feed_tokens(m, c, tokens, n_ok, false);
  if (rc) return rc;
  if (err == DEFER_GPU_E_TOKEN) return fail(err, "token id %u out of range", bad);
  if (err == DEFER_GPU_E_CONTEXT)
    return fail(err, "context length %u exceeded", m->cfg.max_seq_len);
  return DEFER_GPU_OK;
}

static int check_temperature(float t) {
  if (!(t >= 0.0f && isfinite(t)))
    return fail(DEFER_GPU_E_INVALID, "temperature must be finite and >= 0");
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_generate(const defer_gpu_model* m, defer_gpu_cache* c, uint32_t max_tokens,
                                  float temperature, const uint32_t* rng_words,
                                  const uint32_t* stop, size_t n_stop, uint32_t* tokens_out,
                                  uint32_t* n_out) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  if (n_out) *n_out = 0;
  rc = check_temperature(temperature);
  if (rc) return rc;
  if (max_tokens == 0) return DEFER_GPU_OK;
  if (!c->has_logits) return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  // A full cache is a context error before anything else (sampler.rs draws
  // its word first, then forward_ext fails: model.rs:420-422).
  const uint32_t room = c->cap - c->pos;
  const uint32_t n = std::min(max_tokens, room);
  if (n == 0) return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  if (temperature != 0.0f && !rng_words) return fail(DEFER_GPU_E_INVALID, "null rng words");
  if (!tokens_out) return fail(DEFER_GPU_E_INVALID, "null tokens_out");
  rc = ensure_run_buffers(c, n, n_stop);
  if (rc) return rc;
  if (temperature != 0.0f)
    HIP_TRY(hipMemcpy(c->d_words, rng_words, n * sizeof(uint32_t), hipMemcpyHostToDevice));
  if (n_stop) HIP_TRY(hipMemcpy(c->d_stop, stop, n_stop * sizeof(uint32_t), hipMemcpyHostToDevice));
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = n;
  r.mode = RUN_GENERATE;
  r.sample_from = 0;
  r.samp_tag0 = c->samp_next;
  c->samp_next += n;
  r.temperature = temperature;
  r.n_stop = (uint32_t)n_stop;
  r.tokens = c->d_tokens;
  r.words = c->d_words;
  r.stop = c->d_stop;
  r.out_tokens = c->d_out;
  rc = run_ops(c, r, false);
  if (rc) return rc;
  const DevState h = read_state(c);
  if (h.n_done) HIP_TRY(hipMemcpy(tokens_out, c->d_out, h.n_done * sizeof(uint32_t),
                                  hipMemcpyDeviceToHost));
  if (n_out) *n_out = h.n_done;
  if (n < max_tokens && !h.halt)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  return DEFER_GPU_OK;
}

// ------------------------------------------------- generate with on_token

static int ensure_ring(defer_gpu_cache* c, size_t n) {
  if (n <= c->ring_cap && c->h_ring) return DEFER_GPU_OK;
  if (c->h_ring) (void)hipHostFree(c->h_ring);
  c->h_ring = c->d_ring = nullptr;
  c->ring_cap = 0;
  const size_t cap = std::max<size_t>(n, 1024);
  // Coherent pinned memory: the device's system-scope stores land where the
  // host thread polls them while the run goes on.
  HIP_TRY(counted_host_malloc((void**)&c->h_ring, cap * sizeof(u64), hipHostMallocCoherent));
  HIP_TRY(hipHostGetDevicePointer((void**)&c->d_ring, c->h_ring, 0));
  c->ring_cap = cap;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_generate_cb(const defer_gpu_model* m, defer_gpu_cache* c,
                                     uint32_t max_tokens, float temperature,
                                     const uint32_t* rng_words, const uint32_t* stop,
                                     size_t n_stop, uint32_t* tokens_out, uint32_t* n_out,
                                     defer_gpu_token_fn on_token, void* user) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  if (n_out) *n_out = 0;
  rc = check_temperature(temperature);
  if (rc) return rc;
  if (max_tokens == 0) return DEFER_GPU_OK;
  if (!c->has_logits) return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  // A full cache is a context error before anything else (sampler.rs draws
  // its word first, then forward_ext fails: model.rs:420-422).
  const uint32_t room = c->cap - c->pos;
  const uint32_t n = std::min(max_tokens, room);
  if (n == 0) return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  if (temperature != 0.0f && !rng_words) return fail(DEFER_GPU_E_INVALID, "null rng words");
  if (n_stop && !stop) return fail(DEFER_GPU_E_INVALID, "null stop tokens");
  if (!tokens_out) return fail(DEFER_GPU_E_INVALID, "null tokens_out");
  rc = ensure_run_buffers(c, n, n_stop);
  if (rc) return rc;
  rc = ensure_ring(c, n);
  if (rc) return rc;
  memset(c->h_ring, 0, n * sizeof(u64));  // no index tag is 0
  if (temperature != 0.0f)
    HIP_TRY(hipMemcpy(c->d_words, rng_words, n * sizeof(uint32_t), hipMemcpyHostToDevice));
  if (n_stop) HIP_TRY(hipMemcpy(c->d_stop, stop, n_stop * sizeof(uint32_t), hipMemcpyHostToDevice));
  const uint32_t pos0 = c->pos;
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = n;
  r.mode = RUN_GENERATE;
  r.sample_from = 0;
  r.samp_tag0 = c->samp_next;
  c->samp_next += n;
  r.temperature = temperature;
  r.n_stop = (uint32_t)n_stop;
  r.tokens = c->d_tokens;
  r.words = c->d_words;
  r.stop = c->d_stop;
  r.out_tokens = c->d_out;
  r.ring = c->d_ring;
  rc = run_launch(c, r, false);
  if (rc) return rc;
  // Hand each committed token to on_token, in order, as it lands; the run
  // is over once the stream is idle and the slot after the last is unset.
  const hipStream_t s = m->stream;
  uint32_t next = 0;
  int cb_rc = 0;
  bool idle = false;
  while (next < n && cb_rc == 0) {
    const u64 w = __atomic_load_n(c->h_ring + next, __ATOMIC_ACQUIRE);
    if ((uint32_t)(w >> 32) == next + 1) {
      tokens_out[next] = (uint32_t)w;
      if (on_token) cb_rc = on_token(user, next, (uint32_t)w);
      ++next;
      continue;
    }
    if (idle) break;
    const hipError_t q = hipStreamQuery(s);
    if (q == hipSuccess) {
      idle = true;  // every store of the run is visible now: drain, then stop
    } else if (q != hipErrorNotReady) {
      (void)run_finish(c);
      return fail(DEFER_GPU_E_HIP, "generate: %s", hipGetErrorString(q));
    }
  }
  rc = run_finish(c);
  if (rc) return rc;
  const DevState h = read_state(c);
  if (cb_rc != 0) {
    // on_token failed at token next - 1: as the reference's generate returns
    // there, the call ends with the tokens up to it; the ones the device ran
    // past it are dropped from the cache.
    const int trc = defer_gpu_cache_truncate(c, pos0 + next);
    if (n_out) *n_out = next;
    if (trc) return trc;
    return fail(DEFER_GPU_E_CALLBACK, "on_token returned %d at token %u", cb_rc, next - 1);
  }
  if (next < h.n_done) {
    // Tokens whose commit the poll did not see (cannot happen once the
    // stream is idle, kept as a guard): delivered from the run's output.
    HIP_TRY(hipMemcpy(tokens_out + next, c->d_out + next, (h.n_done - next) * sizeof(uint32_t),
                      hipMemcpyDeviceToHost));
    for (; next < h.n_done && cb_rc == 0; ++next)
      if (on_token) cb_rc = on_token(user, next, tokens_out[next]);
    if (cb_rc != 0) {
      const int trc = defer_gpu_cache_truncate(c, pos0 + next);
      if (n_out) *n_out = next;
      if (trc) return trc;
      return fail(DEFER_GPU_E_CALLBACK, "on_token returned %d at token %u", cb_rc, next - 1);
    }
  }
  if (n_out) *n_out = h.n_done;
  if (n < max_tokens && !h.halt)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  return DEFER_GPU_OK;
}

// ------------------------------------------------- allocation-free generate
//
// defer_gpu_generate_static: defer_gpu_generate without any allocation, for
// callers that cannot allocate device memory. The run's staging -- the rng
// words handed in, the stop list and the tokens handed back, which
// defer_gpu_generate keeps in buffers the library allocates on demand --
// lives in `scratch`, a file-scope device array each GPU holds for the life
// of the process. Every call on a GPU shares that GPU's copy: calls that
// overlap on one GPU (from several host threads) race.
constexpr uint32_t STATIC_MAX_TOKENS = 1u << 16;  // tokens per call at most
constexpr uint32_t STATIC_MAX_STOP = 256;          // stop tokens per call at most
constexpr size_t STATIC_WORDS = 2 * (size_t)STATIC_MAX_TOKENS + STATIC_MAX_STOP;
static __device__ __align__(256) uint32_t scratch[STATIC_WORDS];  // 513 KB per GPU

// The array's address on each device. In host code `scratch` names a host
// stand-in, never the device memory: only these pointers are handed to
// kernels and copies.
constexpr int STATIC_MAX_DEVICES = 64;
static uint32_t* g_scratch[STATIC_MAX_DEVICES];

static int scratch_on(int device, uint32_t** out) {
  if (device < 0 || device >= STATIC_MAX_DEVICES)
    return fail(DEFER_GPU_E_INVALID, "device %d beyond the %d the static scratch serves", device,
                STATIC_MAX_DEVICES);
  if (!g_scratch[device]) {
    int cur = 0;
    HIP_TRY(hipGetDevice(&cur));
    if (cur != device) HIP_TRY(hipSetDevice(device));
    uint32_t* p = nullptr;
    const hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (cur != device) HIP_TRY(hipSetDevice(cur));
    if (e != hipSuccess || !p)
      return fail(DEFER_GPU_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return DEFER_GPU_OK;
}

// Process teardown: every device a model was made on is synchronised and
// reset (hipDeviceReset), releasing the HIP runtime's queues, including the
// one it keeps for cooperative launches, while the process is still whole
// rather than in the runtime's exit handlers.
extern "C" int defer_gpu_shutdown(void) {
  const uint64_t nm = g_live_models.load(), nc = g_live_caches.load();
  if (nm || nc)
    return fail(DEFER_GPU_E_INVALID, "%llu models and %llu caches are still live: destroy them first",
                (unsigned long long)nm, (unsigned long long)nc);
  int cur = 0;
  HIP_TRY(hipGetDevice(&cur));
  const uint64_t used = g_devices_used.exchange(0);
  for (int dev = 0; dev < 64; ++dev) {
    if (!(used >> dev & 1u)) continue;
    HIP_TRY(hipSetDevice(dev));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipDeviceReset());
    if (dev < STATIC_MAX_DEVICES) g_scratch[dev] = nullptr;  // the array may move once reloaded
  }
  HIP_TRY(hipSetDevice(cur));
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_generate_static(const defer_gpu_model* m, defer_gpu_cache* c,
                                         uint32_t max_tokens, float temperature,
                                         const uint32_t* rng_words, const uint32_t* stop,
                                         size_t n_stop, uint32_t* tokens_out, uint32_t* n_out) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  if (n_out) *n_out = 0;
  rc = check_temperature(temperature);
  if (rc) return rc;
  if (max_tokens > STATIC_MAX_TOKENS)
    return fail(DEFER_GPU_E_INVALID, "defer_gpu_generate_static: %u tokens exceed the %u a call may take",
                max_tokens, STATIC_MAX_TOKENS);
  if (n_stop > STATIC_MAX_STOP)
    return fail(DEFER_GPU_E_INVALID, "defer_gpu_generate_static: %zu stop tokens exceed the %u a call may take",
                n_stop, STATIC_MAX_STOP);
  if (max_tokens == 0) return DEFER_GPU_OK;
  if (!c->has_logits) return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  // A full cache is a context error before anything else (sampler.rs draws
  // its word first, then forward_ext fails: model.rs:420-422).
  const uint32_t room = c->cap - c->pos;
  const uint32_t n = std::min(max_tokens, room);
  if (n == 0) return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  if (temperature != 0.0f && !rng_words) return fail(DEFER_GPU_E_INVALID, "null rng words");
  if (n_stop && !stop) return fail(DEFER_GPU_E_INVALID, "null stop tokens");
  if (!tokens_out) return fail(DEFER_GPU_E_INVALID, "null tokens_out");
  uint32_t* base = nullptr;
  rc = scratch_on(m->device, &base);
  if (rc) return rc;
  uint32_t* d_words = base;
  uint32_t* d_stop = base + STATIC_MAX_TOKENS;
  uint32_t* d_out = base + STATIC_MAX_TOKENS + STATIC_MAX_STOP;
  const hipStream_t s = m->stream;
  // Every word the kernels read is written here first (words, stop list);
  // the tokens are read back only up to the ops the run completed.
  if (temperature != 0.0f)
    HIP_TRY(hipMemcpyAsync(d_words, rng_words, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  if (n_stop)
    HIP_TRY(hipMemcpyAsync(d_stop, stop, n_stop * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = n;
  r.mode = RUN_GENERATE;
  r.sample_from = 0;
  r.samp_tag0 = c->samp_next;
  c->samp_next += n;
  r.temperature = temperature;
  r.n_stop = (uint32_t)n_stop;
  r.tokens = d_words;  // unused by generate ops
  r.words = d_words;
  r.stop = d_stop;
  r.out_tokens = d_out;
  // A graph would be instantiated (allocated) on first use: in graph mode the
  // same phase kernels run one by one instead (identical bits).
  rc = run_ops(c, r, m->exec_mode == DEFER_GPU_EXEC_GRAPH);
  if (rc) return rc;
  const DevState h = read_state(c);
  if (h.n_done) HIP_TRY(hipMemcpy(tokens_out, d_out, h.n_done * sizeof(uint32_t), hipMemcpyDeviceToHost));
  if (n_out) *n_out = h.n_done;
  if (n < max_tokens && !h.halt)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_sample(const defer_gpu_model* m, defer_gpu_cache* c, float temperature,
                                uint32_t rng_word, uint32_t* token_out) {
  // A sample without the feed: run the sampler kernels alone on the current
  // logits (stage A on all workgroups, stage B on one).
  int rc = check_pair(m, c);
  if (rc) return rc;
  rc = check_temperature(temperature);
  if (rc) return rc;
  if (!c->has_logits) return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  if (!token_out) return fail(DEFER_GPU_E_INVALID, "null token_out");
  rc = ensure_run_buffers(c, 1, 0);
  if (rc) return rc;
  HIP_TRY(hipMemcpy(c->d_words, &rng_word, sizeof(uint32_t), hipMemcpyHostToDevice));
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = 1;
  r.mode = RUN_GENERATE;
  r.sample_from = 0;
  r.samp_tag0 = c->samp_next++;
  r.temperature = temperature;
  r.tokens = c->d_tokens;
  r.words = c->d_words;
  r.stop = c->d_stop;
  r.out_tokens = c->d_out;
  const hipStream_t s = m->stream;
  HIP_TRY(hipMemcpyAsync(c->d_run, &r, sizeof(r), hipMemcpyHostToDevice, s));
  k_begin<<<1, 1, 0, s>>>(c->st);
  k_samp_a<<<m->G, BLOCK, m->lds_bytes, s>>>(c->d_args, c->d_run);
  k_op<<<1, BLOCK, m->lds_bytes, s>>>(c->d_args, c->d_run);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(s));
  const DevState h = read_state(c);
  if (h.abort) return fail(DEFER_GPU_E_TIMEOUT, "a device-side wait exceeded its bound");
  HIP_TRY(hipMemcpy(token_out, c->d_out, sizeof(uint32_t), hipMemcpyDeviceToHost));
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_step(const defer_gpu_model* m, defer_gpu_cache* c, float temperature,
                              uint32_t rng_word, uint32_t* token_out) {
  uint32_t n = 0;
  const int rc = defer_gpu_generate(m, c, 1, temperature, &rng_word, nullptr, 0, token_out, &n);
  if (rc) return rc;
  if (n != 1) return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_replay(const defer_gpu_model* m, defer_gpu_cache* c,
                                const uint32_t* history, size_t n_history, size_t prompt_len,
                                float temperature, const uint32_t* rng_words, int64_t* first_div,
                                uint32_t* sampled_at_div) {
  int rc = check_pair(m, c);
  if (rc) return rc;
  rc = check_temperature(temperature);
  if (rc) return rc;
  if (first_div) *first_div = -1;
  if (prompt_len > n_history) return fail(DEFER_GPU_E_INVALID, "prompt_len exceeds history");
  if (c->pos != 0) return fail(DEFER_GPU_E_INVALID, "replay needs an empty cache");
  if (n_history > prompt_len && prompt_len == 0)
    return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
  if (n_history > prompt_len && temperature != 0.0f && !rng_words)
    return fail(DEFER_GPU_E_INVALID, "null rng words");
  for (size_t i = 0; i < n_history; ++i)
    if (history[i] >= m->d.V) return fail(DEFER_GPU_E_TOKEN, "token id %u out of range", history[i]);
  if (n_history > c->cap)
    return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  if (use_batch(m, n_history))
    return timed(m, [&] {
      return replay_batched(const_cast<defer_gpu_model*>(m), c, history, n_history, prompt_len,
                            temperature, rng_words, first_div, sampled_at_div);
    });
  rc = ensure_run_buffers(c, n_history, 0);
  if (rc) return rc;
  if (n_history)
    HIP_TRY(hipMemcpy(c->d_tokens, history, n_history * sizeof(uint32_t), hipMemcpyHostToDevice));
  const size_t n_sampled = n_history - prompt_len;
  if (n_sampled && temperature != 0.0f)
    HIP_TRY(hipMemcpy(c->d_words, rng_words, n_sampled * sizeof(uint32_t), hipMemcpyHostToDevice));
  RunDesc r;
  memset(&r, 0, sizeof(r));
  r.n_ops = (uint32_t)n_history;
  r.mode = RUN_REPLAY;
  r.sample_from = (uint32_t)prompt_len;
  r.samp_tag0 = c->samp_next;
  c->samp_next += (uint32_t)n_sampled;
  r.temperature = temperature;
  r.tokens = c->d_tokens;
  r.words = c->d_words;
  r.stop = c->d_stop;
  r.out_tokens = c->d_out;
  rc = run_ops(c, r, false);
  if (rc) return rc;
  const DevState h = read_state(c);
  if (h.first_div >= 0) {
    if (first_div) *first_div = h.first_div;
    if (sampled_at_div) *sampled_at_div = h.sampled_div;
  }
  return DEFER_GPU_OK;
}

// ------------------------------------------------------------------ batches

// Rows per batched launch sequence; longer runs go in slices (a slice's
// attention reads the cache the earlier slices wrote).
static constexpr uint32_t BATCH_MAX_ROWS = 2048;

struct BatchWs {
  uint32_t rows = 0, lm = 0;  // capacities
  // X: the residual rows; XP its GEMM panel (written with it); XQ the panel of
  // the other GEMM inputs (attention output, activation, final-norm rows).
  float *X = nullptr, *Y = nullptr, *INV = nullptr, *XP = nullptr, *XQ = nullptr;
  float* LINV = nullptr;
  float* QS = nullptr;  // quarter-split GEMM subtrees [4][B][M], B <= 64, M <= batch_ldy
  u64 *QKVT = nullptr, *PART = nullptr, *LOGT = nullptr, *VMAX = nullptr, *VARG = nullptr,
      *VSUM = nullptr, *VP = nullptr;
  BRow* drows = nullptr;
  Args* rargs = nullptr;
  Args* largs = nullptr;
  uint32_t *sel = nullptr, *lgen = nullptr, *stick = nullptr, *swords = nullptr, *sout = nullptr;
  uint32_t* items = nullptr;  // attention (row, item) list, or tiled attention tasks
  uint32_t* tiles = nullptr;  // tiled attention: first batch row of each tile
  uint32_t* CNT = nullptr;    // [rows][nkv] finished attention items (k_b_attn_f), 0 between launches
  StateSet* sets = nullptr;   // [rows] cache states to set after a batch
  DevState* st = nullptr;
};

static void batch_ws_release(BatchWs* w) {
  if (!w) return;
  void* ps[] = {w->X, w->Y, w->INV, w->XP, w->XQ, w->LINV, w->QS, w->QKVT, w->PART,
                w->LOGT, w->VMAX, w->VARG, w->VSUM, w->VP, w->drows, w->rargs, w->largs, w->sel,
                w->lgen, w->stick, w->swords, w->sout, w->items, w->tiles, w->CNT, w->sets, w->st};
  for (void* p : ps) (void)hipFree(p);
  *w = BatchWs();
}

static void batch_ws_free(defer_gpu_model* m) {
  if (!m->bw) return;
  batch_ws_release(m->bw);
  delete m->bw;
  m->bw = nullptr;
}

static uint32_t batch_ldy(const Dims& d) { return std::max({d.qkv_rows, 2 * d.ff, d.h}); }
static uint32_t part_words(const Dims& d) { return d.nh * MAX_ACHUNKS * (d.hd + 2); }

static int ensure_ws(defer_gpu_model* m, uint32_t rows, uint32_t lm) {
  if (!m->bw) m->bw = new BatchWs();
  BatchWs& w = *m->bw;
  if (rows <= w.rows && lm <= w.lm && w.st) return DEFER_GPU_OK;
  const Dims& d = m->d;
  const uint32_t R = std::max(rows, w.rows), Lm = std::max(lm, w.lm);
  batch_ws_release(&w);
  const uint32_t kmax = std::max({d.h, d.q, d.ff});
  HIP_TRY(counted_malloc(&w.X, (size_t)R * d.h * sizeof(float)));
  HIP_TRY(counted_malloc(&w.Y, (size_t)R * batch_ldy(d) * sizeof(float)));
  HIP_TRY(counted_malloc(&w.QS, (size_t)4 * std::min(R, 64u) * batch_ldy(d) * sizeof(float)));
  HIP_TRY(counted_malloc(&w.INV, (size_t)R * sizeof(float)));
  HIP_TRY(counted_malloc(&w.XP, panel_floats(R, d.h) * sizeof(float)));
  HIP_TRY(counted_malloc(&w.QKVT, (size_t)R * d.qkv_rows * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.PART, (size_t)R * part_words(d) * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.drows, (size_t)R * sizeof(BRow)));
  HIP_TRY(counted_malloc(&w.rargs, (size_t)R * sizeof(Args)));
  HIP_TRY(counted_malloc(&w.items, (size_t)R * d.nkv * MAX_ACHUNKS * d.group * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.tiles, ((size_t)R / 16 + 2) * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.CNT, (size_t)R * d.nkv * sizeof(uint32_t)));
  HIP_TRY(hipMemset(w.CNT, 0, (size_t)R * d.nkv * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.sets, (size_t)R * sizeof(StateSet)));
  const uint32_t L1 = std::max(Lm, 1u);
  HIP_TRY(counted_malloc(&w.XQ, panel_floats(std::max(R, L1), kmax) * sizeof(float)));
  HIP_TRY(counted_malloc(&w.LINV, (size_t)L1 * sizeof(float)));
  HIP_TRY(counted_malloc(&w.LOGT, (size_t)L1 * d.V * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.VMAX, (size_t)L1 * d.nvc * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.VARG, (size_t)L1 * d.nvc * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.VSUM, (size_t)L1 * 3 * d.nvc * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.VP, (size_t)L1 * d.V * sizeof(u64)));
  HIP_TRY(counted_malloc(&w.largs, (size_t)L1 * sizeof(Args)));
  HIP_TRY(counted_malloc(&w.sel, (size_t)L1 * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.lgen, (size_t)L1 * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.stick, (size_t)L1 * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.swords, (size_t)L1 * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.sout, (size_t)L1 * sizeof(uint32_t)));
  HIP_TRY(counted_malloc(&w.st, sizeof(DevState)));
  HIP_TRY(hipMemset(w.st, 0, sizeof(DevState)));
  // Tags start at 1, so zeroed sums never match a wait; sampled tokens
  // start in range.
  HIP_TRY(hipMemset(w.VSUM, 0, (size_t)L1 * 3 * d.nvc * sizeof(u64)));
  HIP_TRY(hipMemset(w.VP, 0, (size_t)L1 * d.V * sizeof(u64)));
  HIP_TRY(hipMemset(w.sout, 0, (size_t)L1 * sizeof(uint32_t)));
  w.rows = R;
  w.lm = Lm;
  return DEFER_GPU_OK;
}

static void launch_panel(hipStream_t s, const float* src0, const float* src1, uint32_t R0,
                         uint32_t R, uint32_t K, uint32_t ld, float* dst) {
  const size_t n = panel_floats(R, K);
  const uint32_t blocks = (uint32_t)std::min<size_t>((n + 255) / 256, 16384);
  k_to_panel<<<blocks, 256, 0, s>>>(src0, src1, R0, R, K, ld, dst);
}

// The weight panels of every matrix, built once per model.
static int ensure_panels(defer_gpu_model* m) {
  if (m->panels) return DEFER_GPU_OK;
  const Dims& d = m->d;
  const size_t pq = panel_floats(d.qkv_rows, d.h), po = panel_floats(d.h, d.q),
               pg = panel_floats(2 * d.ff, d.h), pd = panel_floats(d.h, d.ff),
               pl = panel_floats(d.V, d.h);
  const size_t total = (pq + po + pg + pd) * d.L + pl;
  HIP_TRY(counted_malloc(&m->panels, total * sizeof(float)));
  const hipStream_t s = m->stream;
  float* p = m->panels;
  m->p_qkv.assign(d.L, nullptr);
  m->p_o.assign(d.L, nullptr);
  m->p_gu.assign(d.L, nullptr);
  m->p_d.assign(d.L, nullptr);
  for (uint32_t l = 0; l < d.L; ++l) {
    const LayerW& W = m->layers[l];
    launch_panel(s, W.wqkv, W.wqkv, d.qkv_rows, d.qkv_rows, d.h, d.h, p);
    m->p_qkv[l] = p;
    p += pq;
    launch_panel(s, W.wo, W.wo, d.h, d.h, d.q, d.q, p);
    m->p_o[l] = p;
    p += po;
    launch_panel(s, W.wg, W.wu, d.ff, 2 * d.ff, d.h, d.h, p);
    m->p_gu[l] = p;
    p += pg;
    launch_panel(s, W.wd, W.wd, d.h, d.h, d.ff, d.ff, p);
    m->p_d[l] = p;
    p += pd;
  }
  launch_panel(s, m->head, m->head, d.V, d.V, d.h, d.h, p);
  m->p_lm = p;
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(s));
  return DEFER_GPU_OK;
}

template <int TN, uint32_t OUT>
static void launch_gemm_tn(hipStream_t s, const float* Wp, uint32_t M, uint32_t K, const float* Xp,
                           uint32_t B, float* Y, uint32_t ldy, const float* scale,
                           const uint32_t* gen, uint32_t cbase, uint32_t ncols, uint32_t ncu,
                           float* P) {
  const uint32_t nrg = (M + 63) / 64, ntask = nrg * ((ncols + TN - 1) / TN);
  // One workgroup per CU (two for smaller tasks, whose LDS and registers allow it).
  const uint32_t grid = std::min(ntask, (TN == 4 ? 1 : 2) * ncu);
  const uint32_t threads = GEMM_WAVES * WAVE;
  if (K % 64 == 0)
    k_gemm<TN, OUT, false><<<grid, threads, gemm_lds_bytes(TN), s>>>(Wp, M, K, Xp, B, Y, ldy, scale,
                                                                      gen, cbase, ncols, P);
  else
    k_gemm<TN, OUT, true><<<grid, threads, gemm_lds_bytes(TN), s>>>(Wp, M, K, Xp, B, Y, ldy, scale,
                                                                     gen, cbase, ncols, P);
}
// One workgroup per CU runs at a time (registers and LDS), so a grid whose
// last round would hold only a few workgroups is split: whole rounds of
// four-column-tile workgroups, then the remaining column tiles one per
// workgroup (a quarter of the work each), which finish in a fraction of a
// round. Every output is computed the same way either way.
template <uint32_t OUT>
static bool launch_gemm_out(hipStream_t s, const float* Wp, uint32_t M, uint32_t K, const float* Xp,
                            uint32_t B, float* Y, uint32_t ldy, const float* scale,
                            const uint32_t* gen, uint32_t ncu, float* P, float* QS, size_t qs_floats,
                            float* inv_out, float eps, bool leave_planes) {
  // Returns whether the rows' 1/rms (inv_out) was written as well (GO_RESID),
  // or whether the product was left as QS's four subtree planes and Y not
  // written (GO_PLAIN with leave_planes).
  const uint32_t nct = (B + 15) / 16, nrg = (M + 63) / 64;
  // Narrow batches: four full column tiles and a row group per CU take the
  // four-tile tasks below; fewer row groups split the segments four ways
  // (the subtrees in QS, then combined); otherwise one row tile per task.
  if (nct <= 4 && !(nct == 4 && nrg >= ncu) && QS && nrg < ncu && (size_t)4 * B * M <= qs_floats) {
    const uint32_t per_cu = gemm_q_lds_bytes() <= 80 * 1024 ? 2 : 1;
    const uint32_t grid = std::min(4 * ((M + 31) / 32) * ((nct + 3) / 4), per_cu * ncu);
    if (K % 64 == 0)
      k_gemm_q<false><<<grid, GEMM_WAVES * WAVE, gemm_q_lds_bytes(), s>>>(Wp, M, K, Xp, B, QS);
    else
      k_gemm_q<true><<<grid, GEMM_WAVES * WAVE, gemm_q_lds_bytes(), s>>>(Wp, M, K, Xp, B, QS);
    if (OUT == GO_RESID && inv_out) {
      k_gemm_qcomb_rms<<<B, 256, 0, s>>>(QS, M, B, Y, ldy, P, eps, inv_out);
      return true;
    }
    if (OUT == GO_PLAIN && leave_planes) return true;
    k_gemm_qcomb<OUT><<<dim3((M + 255) / 256, B), 256, 0, s>>>(QS, M, B, Y, ldy, scale, gen, P);
    return false;
  }

  if (nct <= 4 && !(nct == 4 && nrg >= ncu)) {  // narrow: one row tile per task
    const uint32_t grid = std::min((M + 15) / 16, 2 * ncu), threads = GEMM_WAVES * WAVE;
    if (K % 64 == 0)
      k_gemm_n<OUT, false><<<grid, threads, gemm_n_lds_bytes(), s>>>(Wp, M, K, Xp, B, Y, ldy, scale,
                                                                     gen, P);
    else
      k_gemm_n<OUT, true><<<grid, threads, gemm_n_lds_bytes(), s>>>(Wp, M, K, Xp, B, Y, ldy, scale,
                                                                    gen, P);
    return false;
  }
  const uint32_t w4 = nrg * ((nct + 3) / 4), rounds = w4 / ncu, rest = w4 % ncu;
  if (rounds >= 1 && rest > 0 && rest * 4 <= ncu) {
    const uint32_t y4 = rounds * ncu / nrg;  // column groups of 4 in the whole rounds
    if (y4 >= 1 && 4 * y4 < nct) {
      launch_gemm_tn<4, OUT>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, 0, 4 * y4, ncu, P);
      launch_gemm_tn<1, OUT>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, 4 * y4, nct - 4 * y4, ncu, P);
      return false;
    }
  }
  launch_gemm_tn<4, OUT>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, 0, nct, ncu, P);
  return false;
}
// P: GO_RESID's panel of the updated rows (K = M).
// QS / qs_floats: scratch for the quarter-split narrow GEMM (null: not used).
// inv_out (GO_RESID, ldy = M): the updated rows' 1/rms (k_b_rms's order) as
// well; returns whether this launch wrote it (else the caller runs k_b_rms).
// leave_planes (GO_PLAIN): the quarter-split product may stay as QS's
// subtree planes for the consumer to combine; returns whether it did.
static bool launch_gemm(hipStream_t s, uint32_t ncu, uint32_t out, const float* Wp, uint32_t M,
                        uint32_t K, const float* Xp, uint32_t B, float* Y, uint32_t ldy,
                        const float* scale = nullptr, const uint32_t* gen = nullptr,
                        float* P = nullptr, float* QS = nullptr, size_t qs_floats = 0,
                        float* inv_out = nullptr, float eps = 0.0f, bool leave_planes = false) {
  if (out == GO_PLAIN)
    return launch_gemm_out<GO_PLAIN>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, ncu, P, QS,
                                     qs_floats, nullptr, eps, leave_planes);
  if (out == GO_RESID)
    return launch_gemm_out<GO_RESID>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, ncu, P, QS,
                                     qs_floats, inv_out, eps, false);
  return launch_gemm_out<GO_TAG>(s, Wp, M, K, Xp, B, Y, ldy, scale, gen, ncu, P, QS, qs_floats,
                                 nullptr, eps, false);
}

// Timing of one launch (profiling on): events recorded around it on the
// model's stream, read back after the batch's final synchronisation.
struct ProfSpan {
  defer_gpu_model* m;
  int cls;
  double flop;
  size_t at = 0;
  bool on = false;
  ProfSpan(defer_gpu_model* m_, int cls_, double flop_) : m(m_), cls(cls_), flop(flop_) {
    if (!m->prof) return;
    while (m->pev.size() < m->pused + 2) {
      hipEvent_t e;
      if (hipEventCreate(&e) != hipSuccess) return;
      m->pev.push_back(e);
    }
    at = m->pused;
    m->pused += 2;
    on = hipEventRecord(m->pev[at], m->stream) == hipSuccess;
  }
  ~ProfSpan() {
    if (!on) return;
    (void)hipEventRecord(m->pev[at + 1], m->stream);
    m->pcls.push_back(cls);
    m->pflop.push_back(flop);
  }
};

// After a synchronisation: fold the recorded spans into the totals.
static void prof_collect(defer_gpu_model* m) {
  for (size_t i = 0; i < m->pcls.size(); ++i) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, m->pev[2 * i], m->pev[2 * i + 1]) != hipSuccess) continue;
    const int c = m->pcls[i];
    m->pstat[3 * c] += ms;
    m->pstat[3 * c + 1] += m->pflop[i];
    m->pstat[3 * c + 2] += 1.0;
  }
  m->pcls.clear();
  m->pflop.clear();
  m->pused = 0;
}

extern "C" int defer_gpu_model_set_profiling(defer_gpu_model* m, uint32_t on) {
  if (!m) return fail(DEFER_GPU_E_INVALID, "null model");
  m->prof = on != 0;
  return DEFER_GPU_OK;
}

extern "C" int defer_gpu_batch_stats(const defer_gpu_model* mc, double* stats, uint32_t reset) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(mc);
  if (!m || !stats) return fail(DEFER_GPU_E_INVALID, "null argument");
  for (int i = 0; i < 6; ++i) stats[i] = m->pstat[i];
  if (reset)
    for (int i = 0; i < 6; ++i) m->pstat[i] = 0.0;
  return DEFER_GPU_OK;
}

// The one-token kernels' view of a batch row (attention, combine): the
// row cache's arguments with the batch's tagged buffers and no staging.
static Args row_args(const defer_gpu_cache* c, const BatchWs& w, uint32_t b) {
  Args a = c->args;
  a.d.lds_stg = 0;
  a.mb_qkv = w.QKVT + (size_t)b * a.d.qkv_rows;
  a.mb_part = w.PART + (size_t)b * part_words(a.d);
  a.st = w.st;
  a.mask = nullptr;
  return a;
}

// Runs n rows (n <= BATCH_MAX_ROWS) through every layer; logits rows
// sel[0..nl) (batch row indices) get tagged logits and chunk maxima in the
// workspace. Rows must already be validated (tokens, capacity).
// dtok: the rows' tokens on the device (else rows[b].token). deferred: the
// caller synchronises and checks the run state later (and has reset it).
static int batch_run(defer_gpu_model* m, const BRow* rows, defer_gpu_cache* const* rcache,
                     uint32_t n, const uint32_t* sel, uint32_t nl,
                     const uint32_t* dtok = nullptr, bool deferred = false) {
  const Dims& d = m->d;
  const hipStream_t s = m->stream;
  int rc = ensure_panels(m);
  if (rc) return rc;
  rc = ensure_ws(m, n, nl);
  if (rc) return rc;
  BatchWs& w = *m->bw;
  std::vector<Args> ra(n);
  for (uint32_t b = 0; b < n; ++b) ra[b] = row_args(rcache[b], w, b);
  // Attention: tiles of 16 aligned positions when the rows are one cache's
  // consecutive positions (a prefill or a replay) and the shape is the tiled
  // kernel's; otherwise one workgroup per (row, item).
  bool tiled = d.hd == AT_HD && d.kvs == AT_HD && rows[n - 1].pos < ACHUNK * MAX_ACHUNKS;
  for (uint32_t b = 1; b < n && tiled; ++b)
    tiled = rcache[b] == rcache[0] && rows[b].pos == rows[0].pos + b;
  // Rows of distinct caches (a lockstep step) run the attention with its
  // QKV epilogue and combine in one launch (k_b_attn_f): no row reads a
  // cache row that another row's epilogue writes.
  bool fused = !tiled;
  if (fused) {
    std::vector<const defer_gpu_cache*> cs(rcache, rcache + n);
    std::sort(cs.begin(), cs.end());
    fused = std::adjacent_find(cs.begin(), cs.end()) == cs.end();
  }
  std::vector<uint32_t> items, tiles;
  if (tiled) {
    tiles.push_back(0);
    for (uint32_t b = 1; b < n; ++b)
      if (rows[b].pos % 16 == 0) tiles.push_back(b);
    tiles.push_back(n);
    for (uint32_t t = 0; t + 1 < tiles.size(); ++t) {
      const uint32_t nch = attn_nchunks(rows[tiles[t]].pos);
      for (uint32_t c = 0; c < nch; ++c)
        for (uint32_t g = 0; g < d.nkv; ++g) items.push_back(t << 16 | c << 8 | g);
    }
  } else {
    // Grouped items x = (kv head, chunk): every query head of the group in
    // one (rows <= 2048, items < 2^16). Full chunks are listed before each
    // row's last, shorter one, so that the longest items are dispatched
    // first and the short ones fill in behind them.
    items.reserve((size_t)n * d.nkv * 2);
    for (int last = 0; last < 2; ++last)
      for (uint32_t b = 0; b < n; ++b) {
        const uint32_t nch = attn_nchunks(rows[b].pos);
        for (uint32_t g = 0; g < d.nkv; ++g)
          for (uint32_t c = last ? nch - 1 : 0; c < (last ? nch : nch - 1); ++c)
            items.push_back(b << 16 | (g * nch + c));
      }
  }
  // attention flop per layer: scores and weighted values, 2 * hd each per
  // (query head, position)
  double attn_flop = 0.0;
  for (uint32_t b = 0; b < n; ++b) attn_flop += 4.0 * d.nh * d.hd * (rows[b].pos + 1.0);
  std::vector<uint32_t> lgen(nl);
  for (uint32_t i = 0; i < nl; ++i) lgen[i] = gen_lm(d, rows[sel[i]].tick);
  HIP_TRY(hipMemcpyAsync(w.drows, rows, n * sizeof(BRow), hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(w.rargs, ra.data(), n * sizeof(Args), hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(w.items, items.data(), items.size() * sizeof(uint32_t),
                         hipMemcpyHostToDevice, s));
  if (tiled)
    HIP_TRY(hipMemcpyAsync(w.tiles, tiles.data(), tiles.size() * sizeof(uint32_t),
                           hipMemcpyHostToDevice, s));
  if (nl) {
    HIP_TRY(hipMemcpyAsync(w.sel, sel, nl * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    HIP_TRY(hipMemcpyAsync(w.lgen, lgen.data(), nl * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  }
  if (!deferred) k_begin<<<1, 1, 0, s>>>(w.st);
  const uint32_t ldy = batch_ldy(d);
  const size_t qs_n = (size_t)4 * std::min(w.rows, 64u) * ldy;
  k_b_embed<<<n, 256, 0, s>>>(w.drows, dtok, m->embed, d.h, w.X, w.XP);
  // Each layer's residual products also leave the rows' 1/rms for the next
  // product (GO_RESID with inv_out); the embedding rows need their own.
  k_b_rms<<<(n + 3) / 4, 256, 0, s>>>(w.X, n, d.h, d.eps, w.INV);
  for (uint32_t l = 0; l < d.L; ++l) {
    bool planes;
    {
      ProfSpan ps(m, 0, 2.0 * d.qkv_rows * d.h * n);
      planes = launch_gemm(s, m->gemm_ncu, GO_PLAIN, m->p_qkv[l], d.qkv_rows, d.h, w.XP, n, w.Y, ldy,
                           nullptr, nullptr, nullptr, w.QS, qs_n, nullptr, 0.0f, true);
    }
    if (fused) {
      ProfSpan ps(m, 1, attn_flop);
      k_b_attn_f<<<(uint32_t)items.size(), NCW * WAVE, m->lds_attn, s>>>(
          w.rargs, w.drows, w.items, l, w.Y, ldy, planes ? w.QS : nullptr, n, w.INV, w.CNT, w.XQ);
    } else {
      k_b_qkv_epi<<<dim3((d.qkv_rows / 2 + 255) / 256, n), 256, 0, s>>>(
          w.rargs, w.drows, l, w.Y, ldy, w.INV, w.QKVT, d.qkv_rows, planes ? w.QS : nullptr, n);
      {
        ProfSpan ps(m, 1, attn_flop);
        if (tiled)
          k_b_attn_tile<<<(uint32_t)items.size(), 256, attn_tile_lds(d.group), s>>>(
              d, w.drows, w.items, w.tiles, l, w.QKVT, w.PART, part_words(d));
        else
          k_b_attn_w<<<(uint32_t)items.size(), NCW * WAVE, m->lds_attn, s>>>(w.rargs, w.drows,
                                                                              w.items, l);
      }
      k_b_comb<<<dim3(n, (d.nh + COMB_HEADS_PER_BLOCK - 1) / COMB_HEADS_PER_BLOCK), 256, 0, s>>>(
          d, w.drows, w.PART, part_words(d), w.XQ);
    }
    bool inv_done;
    {
      ProfSpan ps(m, 0, 2.0 * d.h * d.q * n);
      inv_done = launch_gemm(s, m->gemm_ncu, GO_RESID, m->p_o[l], d.h, d.q, w.XQ, n, w.X, d.h, nullptr,
                             nullptr, w.XP, w.QS, qs_n, w.INV, d.eps);
    }
    if (!inv_done) k_b_rms<<<(n + 3) / 4, 256, 0, s>>>(w.X, n, d.h, d.eps, w.INV);
    {
      ProfSpan ps(m, 0, 2.0 * 2 * d.ff * d.h * n);
      launch_gemm(s, m->gemm_ncu, GO_PLAIN, m->p_gu[l], 2 * d.ff, d.h, w.XP, n, w.Y, ldy, nullptr,
                  nullptr, nullptr, w.QS, qs_n);
    }
    k_b_act<<<dim3((d.ff + 255) / 256, n), 256, 0, s>>>(w.Y, ldy, w.INV, d.ff, d.act, w.XQ);
    {
      ProfSpan ps(m, 0, 2.0 * d.h * d.ff * n);
      inv_done = launch_gemm(s, m->gemm_ncu, GO_RESID, m->p_d[l], d.h, d.ff, w.XQ, n, w.X, d.h, nullptr,
                             nullptr, w.XP, w.QS, qs_n, w.INV, d.eps);
    }
    if (!inv_done && l + 1 < d.L) k_b_rms<<<(n + 3) / 4, 256, 0, s>>>(w.X, n, d.h, d.eps, w.INV);
  }
  if (nl) {
    k_b_final<<<nl, 64, 0, s>>>(w.X, w.sel, d.h, m->norm, d.eps, w.XQ, w.LINV);
    {
      ProfSpan ps(m, 0, 2.0 * d.V * d.h * nl);
      launch_gemm(s, m->gemm_ncu, GO_TAG, m->p_lm, d.V, d.h, w.XQ, nl, reinterpret_cast<float*>(w.LOGT), d.V,
                  w.LINV, w.lgen, nullptr, w.QS, qs_n);
    }
    k_b_chunkmax<<<dim3((d.nvc + 4 * CM_CPW - 1) / (4 * CM_CPW), nl), 256, 0, s>>>(d, w.LOGT, w.lgen, w.VMAX,
                                                                                   w.VARG, nl);
  }
  HIP_TRY(hipGetLastError());
  if (deferred && !m->prof) return DEFER_GPU_OK;
  HIP_TRY(hipStreamSynchronize(s));
  if (m->prof) prof_collect(m);
  DevState h;
  HIP_TRY(hipMemcpy(&h, w.st, sizeof(h), hipMemcpyDeviceToHost));
  if (h.abort) return fail(DEFER_GPU_E_TIMEOUT, "a device-side wait exceeded its bound");
  return DEFER_GPU_OK;
}

// Sampling ops on logits rows of the workspace: op j samples logits row
// lrow[j] of cache c for generation base tick[j] (the tick of the forward
// that follows the sample) with word words[j].
// deferred: the tokens stay in the workspace (w.sout) and the caller
// synchronises and checks the run state later.
static int batch_sample(defer_gpu_model* m, defer_gpu_cache* const* ocache, const uint32_t* lrow,
                        const uint32_t* tick, const uint32_t* words, uint32_t nops, float T,
                        uint32_t* out, bool own_logits, bool deferred = false) {
  const Dims& d = m->d;
  const hipStream_t s = m->stream;
  // Sampling a batch's logits rows: batch_run sized the workspace for them,
  // so this does not reallocate (which would drop them).
  int rc = ensure_ws(m, 1, nops);
  if (rc) return rc;
  BatchWs& w = *m->bw;
  std::vector<Args> la(nops);
  for (uint32_t j = 0; j < nops; ++j) {
    Args a = ocache[j]->args;
    a.d.lds_stg = 0;
    if (!own_logits) {
      a.mb_logit = w.LOGT + (size_t)lrow[j] * d.V;
      a.mb_vmax = w.VMAX + (size_t)lrow[j] * d.nvc;
      a.mb_varg = w.VARG + (size_t)lrow[j] * d.nvc;
    }
    a.mb_vsum = w.VSUM + (size_t)j * 3 * d.nvc;
    a.mb_psum = a.mb_vsum + d.nvc;
    a.mb_qsum = a.mb_vsum + 2 * d.nvc;
    a.mb_p = w.VP + (size_t)j * d.V;
    a.st = w.st;
    a.mask = nullptr;
    la[j] = a;
  }
  HIP_TRY(hipMemcpyAsync(w.largs, la.data(), nops * sizeof(Args), hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(w.stick, tick, nops * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  if (T != 0.0f)
    HIP_TRY(hipMemcpyAsync(w.swords, words, nops * sizeof(uint32_t), hipMemcpyHostToDevice, s));
  k_begin<<<1, 1, 0, s>>>(w.st);
  const uint32_t tag0 = m->samp_next;
  m->samp_next += nops;
  k_b_sample<<<nops, BLOCK, samp_lds_bytes(m), s>>>(w.largs, w.stick, w.swords, T, tag0, w.sout);
  HIP_TRY(hipGetLastError());
  if (deferred) return DEFER_GPU_OK;
  HIP_TRY(hipMemcpyAsync(out, w.sout, nops * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  DevState h;
  HIP_TRY(hipMemcpy(&h, w.st, sizeof(h), hipMemcpyDeviceToHost));
  if (h.abort) return fail(DEFER_GPU_E_TIMEOUT, "a device-side wait exceeded its bound");
  return DEFER_GPU_OK;
}

// Caches after their batch rows: length, generation base and, from logits
// row li[k] of the workspace, the tagged logits and chunk maxima a following
// sample reads. One kernel copies every cache's words, one sets the device
// states, then one synchronisation.
static int batch_commit_many(defer_gpu_model* m, defer_gpu_cache* const* cs, const uint32_t* li,
                             const uint32_t* pos, const uint32_t* tick, uint32_t n) {
  const Dims& d = m->d;
  const hipStream_t s = m->stream;
  const BatchWs& w = *m->bw;
  std::vector<StateSet> set(n);
  for (uint32_t k = 0; k < n; ++k) {
    defer_gpu_cache* c = cs[k];
    set[k].st = c->st;
    set[k].pos = pos[k];
    set[k].tick = tick[k];
    set[k].logit = c->args.mb_logit;
    set[k].vmax = c->args.mb_vmax;
    set[k].varg = c->args.mb_varg;
    set[k].li = li[k];
  }
  HIP_TRY(hipMemcpyAsync(w.sets, set.data(), n * sizeof(StateSet), hipMemcpyHostToDevice, s));
  if (n > 0) {
    const uint32_t words = d.V + 2 * d.nvc;
    k_commit_rows<<<dim3(std::min((words + 1023) / 1024, 64u), n), 256, 0, s>>>(
        w.sets, w.LOGT, w.VMAX, w.VARG, d.V, d.nvc);
  }
  k_set_state<<<(n + 63) / 64, 64, 0, s>>>(w.sets, n);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(s));
  for (uint32_t k = 0; k < n; ++k) {
    cs[k]->pos = pos[k];
    cs[k]->tick = tick[k];
    cs[k]->has_logits = true;
  }
  return DEFER_GPU_OK;
}
static int batch_commit(defer_gpu_model* m, defer_gpu_cache* c, uint32_t li, uint32_t pos,
                        uint32_t tick) {
  return batch_commit_many(m, &c, &li, &pos, &tick, 1);
}

static BRow make_row(const defer_gpu_cache* c, uint32_t pos, uint32_t tick, uint32_t token) {
  BRow r;
  r.kc = c->kc;
  r.vc = c->vc;
  r.cap = c->cap;
  r.pos = pos;
  r.tick = tick;
  r.token = token;
  return r;
}

static bool use_batch(const defer_gpu_model* m, size_t n) { return m->batch_min && n >= m->batch_min; }

extern "C" int defer_gpu_model_set_batching(defer_gpu_model* m, uint32_t min_rows) {
  if (!m) return fail(DEFER_GPU_E_INVALID, "null model");
  m->batch_min = min_rows;
  return DEFER_GPU_OK;
}

// Feeds tokens[0..n) to one cache in slices; the last slice's last row
// keeps its logits. Range checks are done by the caller.
static int feed_batched(defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* tokens, size_t n) {
  for (size_t o = 0; o < n; o += BATCH_MAX_ROWS) {
    const uint32_t k = (uint32_t)std::min<size_t>(BATCH_MAX_ROWS, n - o);
    std::vector<BRow> rows(k);
    std::vector<defer_gpu_cache*> rc(k, c);
    for (uint32_t j = 0; j < k; ++j) rows[j] = make_row(c, c->pos + j, c->tick + j, tokens[o + j]);
    const bool last = o + k == n;
    const uint32_t sel = k - 1;
    int e = batch_run(m, rows.data(), rc.data(), k, &sel, last ? 1 : 0);
    if (e) return e;
    if (last) {
      e = batch_commit(m, c, 0, c->pos + k, c->tick + k);
      if (e) return e;
    } else {
      c->pos += k;
      c->tick += k;
      c->has_logits = false;
      e = push_state(c);
      if (e) return e;
    }
  }
  return DEFER_GPU_OK;
}

// The batch forward. tokens: host token ids (checked), or null with dtok:
// the tokens on the device (just sampled into the workspace, in range by
// construction), copied to tok_out in the same pass; the run state was
// reset by the sampling, and one synchronisation ends the call.
static int forward_batch_impl(defer_gpu_model* m, defer_gpu_cache* const* caches,
                              const uint32_t* tokens, const uint32_t* dtok, uint32_t* tok_out,
                              uint32_t n, float* logits_out) {
  const Dims& d = m->d;
  const bool deferred = dtok != nullptr;
  // positions: a cache listed k times gets k consecutive positions
  std::vector<uint32_t> add(n, 0);
  std::vector<int> last_of(n, -1);  // per row: is it its cache's last row
  for (uint32_t b = 0; b < n; ++b) {
    int rc = check_pair(m, caches[b]);
    if (rc) return rc;
    if (tokens && tokens[b] >= d.V) return fail(DEFER_GPU_E_TOKEN, "token id %u out of range", tokens[b]);
    for (uint32_t e = 0; e < b; ++e)
      if (caches[e] == caches[b]) ++add[b];
  }
  for (uint32_t b = 0; b < n; ++b) {
    bool later = false;
    for (uint32_t e = b + 1; e < n && !later; ++e) later = caches[e] == caches[b];
    last_of[b] = later ? 0 : 1;
    if (last_of[b] && caches[b]->pos + add[b] + 1 > caches[b]->cap)
      return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
  }
  std::vector<BRow> rows(n);
  for (uint32_t b = 0; b < n; ++b)
    rows[b] = make_row(caches[b], caches[b]->pos + add[b], caches[b]->tick + add[b],
                       tokens ? tokens[b] : 0u);
  std::vector<uint32_t> sel;
  std::vector<uint32_t> li_of(n, 0);
  for (uint32_t b = 0; b < n; ++b)
    if (logits_out || last_of[b]) {
      li_of[b] = (uint32_t)sel.size();
      sel.push_back(b);
    }
  HIP_TRY(hipEventRecord(m->ev0, m->stream));
  int rc = batch_run(m, rows.data(), caches, n, sel.data(), (uint32_t)sel.size(), dtok, deferred);
  if (rc) return rc;
  HIP_TRY(hipEventRecord(m->ev1, m->stream));
  if (deferred)
    HIP_TRY(hipMemcpyAsync(tok_out, dtok, n * sizeof(uint32_t), hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipEventSynchronize(m->ev1));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->last_ms = ms;
  if (deferred) {
    // A wait that ran out leaves the rows undefined: nothing is committed.
    DevState h;
    HIP_TRY(hipMemcpy(&h, m->bw->st, sizeof(h), hipMemcpyDeviceToHost));
    if (h.abort) {
      for (uint32_t b = 0; b < n; ++b) caches[b]->has_logits = false;
      return fail(DEFER_GPU_E_TIMEOUT, "a device-side wait exceeded its bound; cache state is undefined");
    }
  }
  if (logits_out) {
    const BatchWs& w = *m->bw;
    for (uint32_t b = 0; b < n; ++b) {
      float* dst = caches[b]->d_logits;  // [V] staging of the untagged row
      k_untag<<<(d.V + 255) / 256, 256, 0, m->stream>>>(w.LOGT + (size_t)li_of[b] * d.V, dst, d.V);
      HIP_TRY(hipMemcpyAsync(logits_out + (size_t)b * d.V, dst, (size_t)d.V * sizeof(float),
                             hipMemcpyDeviceToHost, m->stream));
      HIP_TRY(hipStreamSynchronize(m->stream));
    }
  }
  std::vector<defer_gpu_cache*> cc;
  std::vector<uint32_t> cli, cpos, ctick;
  for (uint32_t b = 0; b < n; ++b)
    if (last_of[b]) {
      cc.push_back(caches[b]);
      cli.push_back(li_of[b]);
      cpos.push_back(rows[b].pos + 1);
      ctick.push_back(rows[b].tick + 1);
    }
  return batch_commit_many(m, cc.data(), cli.data(), cpos.data(), ctick.data(), (uint32_t)cc.size());
}

extern "C" int defer_gpu_forward_batch(const defer_gpu_model* mc, defer_gpu_cache* const* caches,
                                       const uint32_t* tokens, uint32_t n, float* logits_out) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(mc);
  if (!m) return fail(DEFER_GPU_E_INVALID, "null model");
  if (n == 0) return DEFER_GPU_OK;
  if (!caches || !tokens) return fail(DEFER_GPU_E_INVALID, "null argument");
  if (n > BATCH_MAX_ROWS) return fail(DEFER_GPU_E_INVALID, "at most %u rows per batch", BATCH_MAX_ROWS);
  return forward_batch_impl(m, caches, tokens, nullptr, nullptr, n, logits_out);
}

extern "C" int defer_gpu_step_batch(const defer_gpu_model* mc, defer_gpu_cache* const* caches,
                                    uint32_t n, float temperature, const uint32_t* rng_words,
                                    uint32_t* tokens_out) {
  defer_gpu_model* m = const_cast<defer_gpu_model*>(mc);
  if (!m) return fail(DEFER_GPU_E_INVALID, "null model");
  int rc = check_temperature(temperature);
  if (rc) return rc;
  if (n == 0) return DEFER_GPU_OK;
  if (!caches || !tokens_out) return fail(DEFER_GPU_E_INVALID, "null argument");
  if (temperature != 0.0f && !rng_words) return fail(DEFER_GPU_E_INVALID, "null rng words");
  if (n > BATCH_MAX_ROWS) return fail(DEFER_GPU_E_INVALID, "at most %u rows per batch", BATCH_MAX_ROWS);
  std::vector<uint32_t> tick(n);
  for (uint32_t b = 0; b < n; ++b) {
    rc = check_pair(m, caches[b]);
    if (rc) return rc;
    for (uint32_t e = 0; e < b; ++e)
      if (caches[e] == caches[b]) return fail(DEFER_GPU_E_INVALID, "step_batch needs distinct caches");
    if (!caches[b]->has_logits)
      return fail(DEFER_GPU_E_NO_LOGITS, "no context: provide a non-empty prompt");
    if (caches[b]->pos >= caches[b]->cap)
      return fail(DEFER_GPU_E_CONTEXT, "context length %u exceeded", m->cfg.max_seq_len);
    tick[b] = caches[b]->tick;
  }
  // Sample, forward and commit in one pass with one synchronisation: the
  // sampled tokens stay on the device for the embedding (the workspace is
  // sized first, so the forward does not reallocate it under them).
  rc = ensure_ws(m, n, n);
  if (rc) return rc;
  rc = batch_sample(m, caches, nullptr, tick.data(), rng_words, n, temperature, tokens_out, true,
                    true);
  if (rc) return rc;
  return forward_batch_impl(m, caches, nullptr, m->bw->sout, tokens_out, n, nullptr);
}

// Checkout's replay through batches: every history token is fed (teacher
// forcing, as the loop feeds the recorded token after comparing), each
// sampled position re-sampled from its predecessor's logits and compared.
// The first mismatch ends the replay with the cache holding the positions
// before it, as the token-by-token loop leaves it.
static int replay_batched(defer_gpu_model* m, defer_gpu_cache* c, const uint32_t* history,
                          size_t n, size_t plen, float T, const uint32_t* words,
                          int64_t* first_div, uint32_t* sampled_at_div) {
  const uint32_t tick0 = c->tick;
  for (size_t o = 0; o < n; o += BATCH_MAX_ROWS) {
    const uint32_t k = (uint32_t)std::min<size_t>(BATCH_MAX_ROWS, n - o);
    std::vector<BRow> rows(k);
    std::vector<defer_gpu_cache*> rc(k, c);
    for (uint32_t j = 0; j < k; ++j)
      rows[j] = make_row(c, (uint32_t)(o + j), tick0 + (uint32_t)(o + j), history[o + j]);
    // rows whose logits are sampled (positions >= plen - 1) or kept (the last)
    std::vector<uint32_t> sel;
    for (uint32_t j = 0; j < k; ++j)
      if (o + j + 1 >= plen) sel.push_back(j);
    int e = batch_run(m, rows.data(), rc.data(), k, sel.data(), (uint32_t)sel.size());
    if (e) return e;
    // op i = row + 1 samples logits row `row` (the ops inside the history)
    std::vector<uint32_t> lrow, tk, wd, out;
    std::vector<defer_gpu_cache*> oc;
    for (uint32_t li = 0; li < sel.size(); ++li) {
      const size_t i = o + sel[li] + 1;
      if (i >= n || i < plen) continue;
      lrow.push_back(li);
      tk.push_back(tick0 + (uint32_t)i);
      wd.push_back(T != 0.0f ? words[i - plen] : 0u);
      oc.push_back(c);
    }
    const uint32_t nops = (uint32_t)lrow.size();
    out.resize(nops);
    if (nops) {
      e = batch_sample(m, oc.data(), lrow.data(), tk.data(), wd.data(), nops, T, out.data(), false);
      if (e) return e;
    }
    for (uint32_t j = 0; j < nops; ++j) {
      const size_t i = o + sel[lrow[j]] + 1;
      if (out[j] != history[i]) {
        if (first_div) *first_div = (int64_t)i;
        if (sampled_at_div) *sampled_at_div = out[j];
        return batch_commit(m, c, lrow[j], (uint32_t)i, tick0 + (uint32_t)i);
      }
    }
    if (o + k == n) return batch_commit(m, c, (uint32_t)sel.size() - 1, (uint32_t)n, tick0 + (uint32_t)n);
    c->pos = (uint32_t)(o + k);
    c->tick = tick0 + (uint32_t)(o + k);
    c->has_logits = false;
    e = push_state(c);
    if (e) return e;
  }
  return DEFER_GPU_OK;
}
