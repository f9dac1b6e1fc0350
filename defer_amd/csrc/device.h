// device.h -- device-side building blocks of the gfx950 forward pass.
//
// Tagged mailboxes. Every activation that crosses workgroups is stored as a
// 64-bit word {generation:32, float bits:32} with an agent-scope relaxed
// store (global_store_dwordx2 sc1) and read with agent-scope relaxed loads.
// A consumer polls the words it needs until every tag equals the expected
// generation, so no barrier, fence or read-modify-write atomic is needed:
// the value and its readiness arrive in one access.
//
// Determinism. Every reduction below has a fixed shape that depends only on
// the problem size: lane-strided partials in index order, an xor butterfly
// across the 64 lanes of a wave, then wave partials summed in wave order.
// Which workgroup computes an output never changes how it is computed, so
// the persistent kernel and the per-phase kernels give identical bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// The device code is compiled once generically (namespace dg, every model
// dimension read at run time) and once per specialised model shape (its own
// namespace, DG_NS, with the shape's dimensions as compile-time constants).
#ifndef DG_NS
#define DG_NS dg
#endif

namespace DG_NS {

typedef unsigned long long u64;

constexpr uint32_t WAVE = 64;
constexpr uint32_t BLOCK = 512;
constexpr uint32_t NWAVES = BLOCK / WAVE;
constexpr uint32_t VCHUNK = 64;        // vocabulary rows per sampling chunk
constexpr uint32_t ACHUNK = 128;       // attention positions per chunk (base size)
constexpr uint32_t MAX_ACHUNKS = 16;   // attention chunks per head at most
constexpr uint32_t INLINE_COMB_MAX = 1536;  // floats of partials combined inside the O phase
constexpr uint32_t SPIN_LIMIT = 1u << 21;
constexpr uint32_t NO_INDEX = 0xffffffffu;

// ------------------------------------------------------------------ layout

struct Dims {
  uint32_t h, nh, nkv, hd, half, ff, V, L, q, kv, qkv_rows, group;
  uint32_t act, has_bias, tied;
  uint32_t cap;        // cache capacity (positions)
  uint32_t kvs;        // KV row stride in floats (>= 32: rows never share a 128-byte line)
  uint32_t nvc;        // number of vocabulary chunks
  uint32_t lds_vec;    // floats of the input-vector LDS region
  uint32_t lds_vec2;   // floats of the second vector region (h)
  uint32_t lds_scr;    // floats of the scratch LDS region
  uint32_t lds_stg;    // floats of the weight staging region (0: rows are not staged)
  uint32_t stg_off[4]; // float offset of each item kind's rows in the staging region
  uint32_t lds_pub;    // entries of the publish list
  float eps, scale;
};

struct LayerW {
  const float* attn_norm;
  const float* wqkv;  // [q + 2kv, h]: q rows, then k rows, then v rows
  const float* bqkv;  // [q + 2kv] or null
  const float* wo;    // [h, q]
  const float* ffn_norm;
  const float* wg;    // [ff, h]
  const float* wu;    // [ff, h]
  const float* wd;    // [h, ff]
};

// Phases of one layer, in order; generation numbers are derived from them.
enum Phase : uint32_t { PH_QKV = 0, PH_ATTN = 1, PH_COMB = 2, PH_O = 3, PH_GU = 4, PH_D = 5 };
constexpr uint32_t PH_PER_LAYER = 6;

struct DevState {
  uint32_t pos;      // cache length
  uint32_t tick;     // number of forwards run on this cache (generation base)
  uint32_t token;    // token of the forward in flight (per-phase kernels)
  uint32_t abort;    // set when a wait exceeded SPIN_LIMIT
  uint32_t halt;     // a run stopped early (divergence or stop token)
  uint32_t n_done;   // ops completed in the current run
  uint32_t op;       // op index of the forward in flight (per-phase kernels)
  uint32_t sampled_div;
  long long first_div;
};

// Describes a run of ops: op i optionally samples (i >= sample_from), then
// feeds a token: the sampled one (generate) or tokens[i] (prompt, replay).
enum RunMode : uint32_t { RUN_FEED = 0, RUN_GENERATE = 1, RUN_REPLAY = 2 };

struct RunDesc {
  uint32_t n_ops;
  uint32_t mode;
  uint32_t sample_from;
  float temperature;
  uint32_t n_stop;
  const uint32_t* tokens;
  const uint32_t* words;
  const uint32_t* stop;
  uint32_t* out_tokens;
};

struct Args {
  Dims d;
  const LayerW* layers;
  const float* embed;
  const float* norm;
  const float* head;     // lm_head, or the embedding when tied
  const float2* rope;    // [max_seq][half] (cos, sin)
  float* kc;             // [L][nkv][cap][kvs]
  float* vc;
  u64* mb_qkv;           // [qkv_rows]
  u64* mb_part;          // [nh][MAX_ACHUNKS][hd + 2]  (m, l, acc[hd])
  u64* mb_att;           // [q] combined attention (separate-combine path)
  u64* mb_xo;            // [h] residual after attention
  u64* mb_xd;            // [h] residual after the MLP
  u64* mb_g;             // [ff]
  u64* mb_logit;         // [V]
  u64* mb_vmax;          // [nvc] chunk max logit
  u64* mb_varg;          // [nvc] chunk argmax (index bits)
  u64* mb_vsum;          // [nvc] chunk sum of exp(logit/T - m)
  DevState* st;
  const uint32_t* mask;  // bitmask over positions, or null
  RunDesc run;
};

__host__ __device__ inline uint32_t phases_per_tick(const Dims& d) {
  return d.L * PH_PER_LAYER + 2;
}
__host__ __device__ inline uint32_t gen_of(const Dims& d, uint32_t tick, uint32_t layer,
                                           uint32_t ph) {
  return tick * phases_per_tick(d) + layer * PH_PER_LAYER + ph + 1u;
}
__host__ __device__ inline uint32_t gen_lm(const Dims& d, uint32_t tick) {
  return tick * phases_per_tick(d) + d.L * PH_PER_LAYER + 1u;
}
__host__ __device__ inline uint32_t gen_sums(const Dims& d, uint32_t tick) {
  return tick * phases_per_tick(d) + d.L * PH_PER_LAYER + 2u;
}

// The dimensions device code computes with. In a shape-specialised build the
// model's dimensions are compile-time constants (loops unroll, index
// arithmetic folds); the per-cache and per-launch fields (capacity, LDS
// layout) always come from the arguments. The values are identical either
// way, so specialised and generic kernels produce the same bits.
__device__ __forceinline__ Dims shape_dims(const Dims& r) {
  Dims d = r;
#if defined(DG_SHAPE_SMOLLM2_135M)
  d.h = 576;
  d.nh = 9;
  d.nkv = 3;
  d.hd = 64;
  d.half = 32;
  d.ff = 1536;
  d.V = 49152;
  d.L = 30;
  d.q = 576;
  d.kv = 192;
  d.qkv_rows = 960;
  d.group = 3;
  d.act = 0;
  d.has_bias = 0;
  d.tied = 1;
  d.kvs = 64;
  d.nvc = 768;
#endif
  return d;
}

// Attention chunking: a function of the query position only, so results
// depend on (pos, data) alone.
__host__ __device__ inline uint32_t attn_chunk(uint32_t pos) {
  const uint32_t ctx = pos + 1;
  const uint32_t base = ACHUNK * MAX_ACHUNKS;
  const uint32_t mult = (ctx + base - 1) / base;
  return ACHUNK * (mult ? mult : 1);
}
__host__ __device__ inline uint32_t attn_nchunks(uint32_t pos) {
  const uint32_t ch = attn_chunk(pos);
  return (pos + 1 + ch - 1) / ch;
}
// Attention items of the query at pos: one per (kv head, chunk, query head).
__host__ __device__ inline uint32_t attn_items(const Dims& d, uint32_t pos) {
  return d.nkv * attn_nchunks(pos) * d.group;
}
__host__ __device__ inline bool comb_inline(const Dims& d, uint32_t pos) {
  return d.nh * attn_nchunks(pos) * (d.hd + 2) <= INLINE_COMB_MAX;
}

// --------------------------------------------------------- memory helpers
//
// Explicit address spaces: pointers reach the kernels inside structs, so the
// compiler would otherwise emit flat instructions, which count against both
// the vector-memory and the LDS wait counters; a later LDS access would then
// wait for every outstanding HBM load and undo the prefetching.

#define AS_GLOBAL __attribute__((address_space(1)))
#define AS_CONST __attribute__((address_space(4)))
#define AS_LDS __attribute__((address_space(3)))

// Address-space casts go through an integer: a direct cast from a generic
// pointer is dropped by the front end. A generic LDS address holds the LDS
// offset in its low 32 bits (the same truncation the flat-to-LDS cast does).
template <class T>
__device__ __forceinline__ AS_GLOBAL T* gptr(T* p) {
  return (AS_GLOBAL T*)(uintptr_t)p;
}
// Read-only data the whole kernel shares (the layer table): through the
// constant address space, so wave-uniform reads become scalar loads, which
// never enter the vector-memory counter.
template <class T>
__device__ __forceinline__ const AS_CONST T* cptr(const T* p) {
  return (const AS_CONST T*)(uintptr_t)p;
}
template <class T>
__device__ __forceinline__ AS_LDS T* lptr(T* p) {
  return (AS_LDS T*)(uintptr_t)(uint32_t)(uintptr_t)p;
}

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float4 ldg4(const float* p) {
  const v4f x = *gptr(reinterpret_cast<const v4f*>(p));
  return make_float4(x.x, x.y, x.z, x.w);
}
__device__ __forceinline__ float ldg(const float* p) { return *gptr(p); }
__device__ __forceinline__ float2 ldg2(const float2* p) {
  const v2f x = *gptr(reinterpret_cast<const v2f*>(p));
  return make_float2(x.x, x.y);
}
__device__ __forceinline__ uint32_t ldg_u32(const uint32_t* p) { return *gptr(p); }
__device__ __forceinline__ float4 lds4(const float* p) {
  const v4f x = *lptr(reinterpret_cast<const v4f*>(p));
  return make_float4(x.x, x.y, x.z, x.w);
}
__device__ __forceinline__ float lds_ld(const float* p) { return *lptr(p); }
__device__ __forceinline__ void lds_st(float* p, float v) { *lptr(p) = v; }

__device__ __forceinline__ void mb_put(u64* slot, float v, uint32_t gen) {
  const u64 w = ((u64)gen << 32) | (u64)__float_as_uint(v);
  __hip_atomic_store(gptr(slot), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 mb_load(const u64* slot) {
  return __hip_atomic_load(gptr(const_cast<u64*>(slot)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(gptr(reinterpret_cast<uint32_t*>(p)), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(gptr(const_cast<uint32_t*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// --------------------------------------------------------- reductions

// Lane permutations through DPP (a VALU operand modifier: a few cycles, no
// LDS round trip). Controls: quad_perm [1,0,3,2] and [2,3,0,1], mirror within
// 8 and 16 lanes, and the row broadcasts of lane 15 / 31 into later rows.
enum : uint32_t {
  DPP_QUAD_X1 = 0xB1,
  DPP_QUAD_X2 = 0x4E,
  DPP_HALF_MIRROR = 0x141,
  DPP_MIRROR = 0x140,
  DPP_BCAST15 = 0x142,
  DPP_BCAST31 = 0x143,
};

// v from the lane DPP control CTRL names; lanes of rows outside ROWS get old.
template <uint32_t CTRL, uint32_t ROWS = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROWS, 0xF, false));
}
template <uint32_t CTRL, uint32_t ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_u(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWS, 0xF, false);
}

// Sum over aligned groups of n lanes (n = 1, 2, 4, 8 or 16): a butterfly in
// which the two lanes of each pair add the same two values, so every lane of
// a group ends with the same bits.
__device__ __forceinline__ float group_sum(float v, uint32_t n) {
  if (n >= 2) v += dpp_f<DPP_QUAD_X1>(0.0f, v);
  if (n >= 4) v += dpp_f<DPP_QUAD_X2>(0.0f, v);
  if (n >= 8) v += dpp_f<DPP_HALF_MIRROR>(0.0f, v);
  if (n >= 16) v += dpp_f<DPP_MIRROR>(0.0f, v);
  return v;
}
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, dpp_f<DPP_QUAD_X1>(v, v));
  v = fmaxf(v, dpp_f<DPP_QUAD_X2>(v, v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v, v));
  v = fmaxf(v, dpp_f<DPP_MIRROR>(v, v));
  return v;
}

// Sum over the wave in a fixed tree: rows of 16 (group_sum), then
// row1 += row0, row3 += row2, row3 += row1; lane 63's value, to every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum(v, 16);
  v += dpp_f<DPP_BCAST15, 0xA>(0.0f, v);
  v += dpp_f<DPP_BCAST31, 0xC>(0.0f, v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), WAVE - 1));
}
// wave_sum of N values at once, stage by stage, so the N dependency chains
// interleave (same tree, same bits as wave_sum).
template <int N>
__device__ __forceinline__ void wave_sum_n(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_QUAD_X1>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_QUAD_X2>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_HALF_MIRROR>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_MIRROR>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_BCAST15, 0xA>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_f<DPP_BCAST31, 0xC>(0.0f, v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i)
    v[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), WAVE - 1));
}

__device__ __forceinline__ float wave_max(float v) {
  v = row_max(v);
  v = fmaxf(v, dpp_f<DPP_BCAST15, 0xA>(v, v));
  v = fmaxf(v, dpp_f<DPP_BCAST31, 0xC>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), WAVE - 1));
}

// Sum over the block in a fixed tree; every thread gets the result.
// `red` is LDS scratch of at least NWAVES floats (+1).
__device__ __forceinline__ float block_sum(float v, float* red) {
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) lds_st(red + wave, v);
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (uint32_t w = 0; w < NWAVES; ++w) s += lds_ld(red + w);
  return s;
}

// Row dot products. Lane `lane` owns the float4s at j = 4*lane + 256*k of a
// row; its partial sum runs over them in ascending j with one fused
// multiply-add per element, then wave_sum() adds the 64 partials. That order
// is the same however the loads are scheduled, so the helpers below (all
// loads of a row issued at once, optionally before the row's input vector is
// available) all give identical bits.
constexpr int KF = 6;  // float4 per lane held in registers: rows of up to 1536 floats

template <int NF>
struct RowT {
  float4 v[NF];
};
typedef RowT<KF> Row;

template <int NF>
__device__ __forceinline__ void row_load(RowT<NF>& r, const float* __restrict__ w, uint32_t K,
                                         uint32_t lane) {
#pragma unroll
  for (int k = 0; k < NF; ++k) {
    const uint32_t j = lane * 4 + 256u * k;
    if (j < K) r.v[k] = ldg4(w + j);
  }
}

template <int NF>
__device__ __forceinline__ float row_fma(const RowT<NF>& r, const float* __restrict__ x,
                                         uint32_t K, uint32_t lane, float acc) {
#pragma unroll
  for (int k = 0; k < NF; ++k) {
    const uint32_t j = lane * 4 + 256u * k;
    if (j < K) {
      const float4 xv = lds4(x + j);
      acc = fmaf(r.v[k].x, xv.x, acc);
      acc = fmaf(r.v[k].y, xv.y, acc);
      acc = fmaf(r.v[k].z, xv.z, acc);
      acc = fmaf(r.v[k].w, xv.w, acc);
    }
  }
  return acc;
}

// Lane partial of w . x given the row's first 256*NF floats already loaded
// into `r`; longer rows stream the rest segment by segment through the same
// registers (so `r` is consumed).
template <int NF>
__device__ __forceinline__ float dot_tail(RowT<NF>& r, const float* __restrict__ w,
                                          const float* __restrict__ x, uint32_t K,
                                          uint32_t lane) {
  float acc = row_fma(r, x, K, lane, 0.0f);
  for (uint32_t base = 256u * NF; base < K; base += 256u * NF) {
    row_load(r, w + base, K - base, lane);
    acc = row_fma(r, x + base, K - base, lane, acc);
  }
  return acc;
}

// Lane partials of two rows w0 . x and w1 . x (same K), the loads of each
// next segment issued before the fmas of the current one, so a wave keeps two
// segments of both rows in flight. Same element order as dot_tail.
template <int NF>
__device__ __forceinline__ float2 dot2_stream(const float* __restrict__ w0,
                                              const float* __restrict__ w1,
                                              const float* __restrict__ x, uint32_t K,
                                              uint32_t lane) {
  constexpr uint32_t SEG = 256u * NF;
  RowT<NF> a0, a1, b0, b1;
  row_load(a0, w0, K, lane);
  row_load(a1, w1, K, lane);
  float acc0 = 0.0f, acc1 = 0.0f;
  for (uint32_t base = 0; base < K; base += 2 * SEG) {
    const uint32_t nb = base + SEG;
    if (nb < K) {
      row_load(b0, w0 + nb, K - nb, lane);
      row_load(b1, w1 + nb, K - nb, lane);
    }
    acc0 = row_fma(a0, x + base, K - base, lane, acc0);
    acc1 = row_fma(a1, x + base, K - base, lane, acc1);
    if (nb >= K) break;
    const uint32_t na = nb + SEG;
    if (na < K) {
      row_load(a0, w0 + na, K - na, lane);
      row_load(a1, w1 + na, K - na, lane);
    }
    acc0 = row_fma(b0, x + nb, K - nb, lane, acc0);
    acc1 = row_fma(b1, x + nb, K - nb, lane, acc1);
  }
  return make_float2(acc0, acc1);
}

__device__ __forceinline__ float dot_partial(const float* __restrict__ w,
                                             const float* __restrict__ x, uint32_t K,
                                             uint32_t lane) {
  Row r;
  row_load(r, w, K, lane);
  return dot_tail(r, w, x, K, lane);
}

__device__ __forceinline__ float dot_row(const float* __restrict__ w, const float* __restrict__ x,
                                         uint32_t K, uint32_t lane) {
  return wave_sum(dot_partial(w, x, K, lane));
}

// Norm weights of one vector, the thread's elements i = tid + BLOCK*k.
constexpr int NWK = 8;  // vectors of up to 8 * BLOCK floats
struct NormW {
  float v[NWK];
};
__device__ __forceinline__ void norm_load(NormW& nw, const float* __restrict__ w, uint32_t n) {
#pragma unroll
  for (int k = 0; k < NWK; ++k) {
    const uint32_t i = threadIdx.x + BLOCK * k;
    if (i < n) nw.v[k] = ldg(w + i);
  }
}

// ----------------------------------------------------------- activation

__device__ __forceinline__ float act_fn(float x, uint32_t act) {
  if (act == 0) return x / (1.0f + expf(-x));  // silu, ops.rs:120-122
  const float c = 0.7978846f;                  // gelu (tanh), ops.rs:125-128
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// ------------------------------------------------------------- waiting

// Shared between the polling helpers of one block (phases.h: wait_gather).
struct WaitCtl {
  int abort_seen;
};

}  // namespace DG_NS
