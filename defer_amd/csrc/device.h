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
// the problem size: chains of fused multiply-adds over fixed element sets in
// index order, then a fixed tree (an xor butterfly over lanes, wave partials
// in wave order).
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
// The dispatcher places workgroup w on XCD w % NXCD.
constexpr uint32_t NXCD = 8;
// Replicas of the all-to-all mailboxes (xo, xd, g): one per XCD, so the
// 32 workgroups of an XCD poll their own copy.
constexpr uint32_t MB_REPS = NXCD;
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
  uint32_t stg_mask;   // bit k: item kind k's rows are staged (the rest are streamed)
  uint32_t stg_off[4]; // float offset of each staged kind's rows in the staging region
  uint32_t lds_pub;    // entries of the listed results (rows streamed)
  uint32_t o_skip;     // workgroups 0 .. o_skip-1 own no O rows (they run attention items)
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
  // Tag of the first sampling op's chunk sums (mb_vsum); op i uses
  // samp_tag0 + (i - sample_from). The host hands out tags from a per-cache
  // counter that starts at 1 and only grows, so no two sampling events of a
  // cache share one.
  uint32_t samp_tag0;
  float temperature;
  uint32_t n_stop;
  const uint32_t* tokens;
  const uint32_t* words;
  const uint32_t* stop;
  uint32_t* out_tokens;
  // Generate runs only, nullable: pinned host words the host reads while the
  // run goes on; op i's token is committed as ((i + 1) << 32) | token.
  u64* ring;
};

// Commits op i's token to the host ring with one 64-bit system-scope store
// (its index in the high half, so a reader needs no separate count).
__device__ __forceinline__ void ring_commit(u64* ring, uint32_t i, uint32_t tok) {
  __hip_atomic_store(ring + i, ((u64)(i + 1u) << 32) | tok, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}

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
  // xo, xd and g have MB_REPS replicas, rep_words apart: a word is
  // published to every replica and a workgroup reads its XCD's (wg % 8)
  u64* mb_xo;            // [h] residual after attention
  u64* mb_xd;            // [h] residual after the MLP
  u64* mb_g;             // [ff]
  uint32_t rep_words;
  u64* mb_logit;         // [V]
  u64* mb_vmax;          // [nvc] chunk max logit
  u64* mb_varg;          // [nvc] chunk argmax (index bits)
  u64* mb_vsum;          // [nvc] chunk sum of exp(logit/T - m)
  u64* mb_p;             // [V] exp(logit/T - m) of the sampling event in flight
  u64* mb_psum;          // [nvc] chunk summary words of the sequential total (exact sampler)
  u64* mb_qsum;          // [nvc] chunk summary words of the sequential CDF (exact sampler)
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

// The dimensions device code computes with. In a shape-specialised build the
// model's dimensions are compile-time constants (loops unroll, index
// arithmetic folds); the per-cache and per-launch fields (capacity, LDS
// layout) always come from the arguments. The values are identical either
// way, so specialised and generic kernels produce the same bits.
// The shapes with a specialised persistent kernel: hidden, heads, kv heads,
// head_dim, intermediate, vocabulary, layers, tied head (SwiGLU, no biases).
#define DG_SHAPE_ARGS_135M 576, 9, 3, 64, 1536, 49152, 30, 1
#define DG_SHAPE_ARGS_360M 960, 15, 5, 64, 2560, 49152, 32, 1
#define DG_SHAPE_ARGS_1B 2048, 32, 8, 64, 8192, 128256, 16, 1
#define DG_SHAPE_ARGS_8B 4096, 32, 8, 128, 14336, 128256, 32, 0
#if defined(DG_SHAPE_SMOLLM2_135M)
#define DG_FIXED_SHAPE DG_SHAPE_ARGS_135M
#elif defined(DG_SHAPE_SMOLLM2_360M)
#define DG_FIXED_SHAPE DG_SHAPE_ARGS_360M
#elif defined(DG_SHAPE_LLAMA32_1B)
#define DG_FIXED_SHAPE DG_SHAPE_ARGS_1B
#elif defined(DG_SHAPE_LLAMA3_8B)
#define DG_FIXED_SHAPE DG_SHAPE_ARGS_8B
#endif
// The derived fields follow the host's model set-up (defer_gpu.hip).
__host__ __device__ constexpr Dims fix_shape(Dims d, uint32_t h, uint32_t nh, uint32_t nkv,
                                             uint32_t hd, uint32_t ff, uint32_t V, uint32_t L,
                                             uint32_t tied) {
  d.h = h;
  d.nh = nh;
  d.nkv = nkv;
  d.hd = hd;
  d.half = hd / 2;
  d.ff = ff;
  d.V = V;
  d.L = L;
  d.q = nh * hd;
  d.kv = nkv * hd;
  d.qkv_rows = nh * hd + 2 * nkv * hd;
  d.group = nh / nkv;
  d.act = 0;
  d.has_bias = 0;
  d.tied = tied;
  d.kvs = hd > 32 ? hd : 32;
  d.nvc = (V + VCHUNK - 1) / VCHUNK;
  return d;
}
__device__ __forceinline__ Dims shape_dims(const Dims& r) {
#if defined(DG_FIXED_SHAPE)
  return fix_shape(r, DG_FIXED_SHAPE);
#else
  return r;
#endif
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

// p, hidden from the optimiser where it is used: addresses formed from it
// there (p + constant) are not hoisted into registers kept across the
// kernel, and their constant parts fold into the LDS instruction's offset.
__device__ __forceinline__ const float* pin(const float* p) {
  asm volatile("" : "+v"(p));
  return p;
}

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

// Row dot products: the one order every matvec of the model uses, whoever
// computes it (a decode workgroup from LDS or from HBM, or the batched
// GEMM). A row of K elements is 16 segments, segment s holding the elements
// 64*i + 4*s + c (i ascending, c = 0..3); each segment is a chain of fused
// multiply-adds from +0, and the row's value is the complete binary tree over
// the 16 segment sums. In a wave, lane 16*r + s computes segment s of row r
// of a quad pass (four rows at once), and group_sum over 16 lanes is the tree.
__device__ __forceinline__ uint32_t qrow(uint32_t lane) { return lane >> 4; }
__device__ __forceinline__ uint32_t qseg(uint32_t lane) { return lane & 15u; }

// NF consecutive chunks of one segment held in registers.
template <int NF>
struct SegT {
  float4 v[NF];
};

// Loads and fmas of whole chunks (every lane's four elements inside the
// row) carry no per-lane condition, so the compiler counts the loads in
// flight exactly: a use waits only for the loads its values need. A
// per-lane condition around a load instead makes every later use wait for
// all loads in flight, which serialises a double-buffered stream.

// Chunks i0 .. i0+NF-1 of segment s of the global row w, all whole chunks.
template <int NF>
__device__ __forceinline__ void seg_load_in(SegT<NF>& r, const float* __restrict__ w, uint32_t s,
                                            uint32_t i0) {
  const float* wb = w + 64u * i0 + 4u * s;
#pragma unroll
  for (int k = 0; k < NF; ++k) r.v[k] = ldg4(wb + 64 * k);
}

// The fmas of whole chunks i0 .. i0+n-1 (n <= NF, wave-uniform) held in r,
// against the LDS vector x, in chunk order. ORDERED keeps each chunk's x
// read next to its fmas (a compiler barrier between chunks), so no more than
// one chunk of x is live: for callers at the edge of the register budget.
template <int NF, bool ORDERED = false>
__device__ __forceinline__ float seg_fma_in(const SegT<NF>& r, const float* x, uint32_t s,
                                            uint32_t i0, float acc, int n = NF) {
  const float* xb = pin(x + 64u * i0 + 4u * s);
#pragma unroll
  for (int k = 0; k < NF; ++k)
    if (k < n) {
      if (ORDERED) asm volatile("" ::: "memory");
      const float4 xv = lds4(xb + 64 * k);
      acc = fmaf(r.v[k].x, xv.x, acc);
      acc = fmaf(r.v[k].y, xv.y, acc);
      acc = fmaf(r.v[k].z, xv.z, acc);
      acc = fmaf(r.v[k].w, xv.w, acc);
    }
  return acc;
}

// Chunks i0 .. i0+NF-1 of segment s of the global row w (those below K).
template <int NF>
__device__ __forceinline__ void seg_load(SegT<NF>& r, const float* __restrict__ w, uint32_t K,
                                         uint32_t s, uint32_t i0) {
#pragma unroll
  for (int k = 0; k < NF; ++k) {
    const uint32_t j = 64u * (i0 + k) + 4u * s;
    if (j < K) r.v[k] = ldg4(w + j);
  }
}

// The fmas of chunks i0 .. i0+NF-1 (held in r) against the LDS vector x.
template <int NF>
__device__ __forceinline__ float seg_fma(const SegT<NF>& r, const float* x, uint32_t K, uint32_t s,
                                         uint32_t i0, float acc) {
  const float* xb = pin(x + 64u * i0 + 4u * s);
#pragma unroll
  for (int k = 0; k < NF; ++k) {
    const uint32_t j = 64u * (i0 + k) + 4u * s;
    if (j < K) {
      const float4 xv = lds4(xb + 64 * k);
      acc = fmaf(r.v[k].x, xv.x, acc);
      acc = fmaf(r.v[k].y, xv.y, acc);
      acc = fmaf(r.v[k].z, xv.z, acc);
      acc = fmaf(r.v[k].w, xv.w, acc);
    }
  }
  return acc;
}

// The chunks of segment s of row w from i on that are not whole blocks of
// NF: the whole chunks with clamped (always issued) loads, then a partial
// last chunk with per-lane tests.
template <int NF>
__device__ __forceinline__ float seg_rest(const float* __restrict__ w, const float* x, uint32_t K,
                                          uint32_t s, uint32_t i, float acc) {
  const uint32_t nwhole = K / 64;
  if (i < nwhole) {
    const int n = (int)(nwhole - i);  // < NF whole chunks
    SegT<NF> r;
    const float* wb = w + 4u * s;
#pragma unroll
    for (int k = 0; k < NF; ++k) r.v[k] = ldg4(wb + 64u * min(i + k, nwhole - 1));
    acc = seg_fma_in(r, x, s, i, acc, n);
    i = nwhole;
  }
  if (64u * i < K) {
    SegT<1> r;
    seg_load(r, w, K, s, i);
    acc = seg_fma(r, x, K, s, i, acc);
  }
  return acc;
}

// Segment s of the global row w from chunk i0 on, NF chunks at a time with
// the next NF in flight, added to acc.
template <int NF>
__device__ __forceinline__ float seg_stream(const float* __restrict__ w, const float* x, uint32_t K,
                                            uint32_t s, uint32_t i0, float acc) {
  const uint32_t nwhole = K / 64;
  const uint32_t nb = nwhole > i0 ? (nwhole - i0) / NF : 0;  // whole blocks
  uint32_t i = i0;
  if (nb > 0) {
    SegT<NF> a, b;
    seg_load_in(a, w, s, i);
    uint32_t blk = 0;
    // Not unrolled: in a shape-specialised build nb is a constant, and the
    // unrolled blocks' loads, hoisted together, spill registers.
#pragma unroll 1
    for (; blk + 2 < nb; blk += 2) {  // both following blocks exist
      seg_load_in(b, w, s, i + NF);
      acc = seg_fma_in(a, x, s, i, acc);
      seg_load_in(a, w, s, i + 2 * NF);
      acc = seg_fma_in(b, x, s, i + NF, acc);
      i += 2 * NF;
    }
    if (blk + 2 == nb) {
      seg_load_in(b, w, s, i + NF);
      acc = seg_fma_in(a, x, s, i, acc);
      acc = seg_fma_in(b, x, s, i + NF, acc);
      i += 2 * NF;
    } else {
      acc = seg_fma_in(a, x, s, i, acc);
      i += NF;
    }
  }
  return seg_rest<NF>(w, x, K, s, i, acc);
}

// LDS segment reads four chunks at a time: group g holds the chunks at
// elements j, j + 64, j + 128, j + 192 (those below K).
struct SegGroup {
  float4 w[4], x[4];
};
__device__ __forceinline__ void seg_group_load(SegGroup& g, const float* w, const float* x,
                                               uint32_t K, uint32_t j) {
  const float* wb = pin(w + j);
  const float* xb = pin(x + j);
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (j + 64 * k < K) {
      g.w[k] = lds4(wb + 64 * k);
      g.x[k] = lds4(xb + 64 * k);
    }
}
__device__ __forceinline__ float seg_group_fma(const SegGroup& g, uint32_t K, uint32_t j, float acc) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (j + 64 * k < K) {
      acc = fmaf(g.w[k].x, g.x[k].x, acc);
      acc = fmaf(g.w[k].y, g.x[k].y, acc);
      acc = fmaf(g.w[k].z, g.x[k].z, acc);
      acc = fmaf(g.w[k].w, g.x[k].w, acc);
    }
  return acc;
}

// Segment s of the LDS row w from element j on (j = 64*i0 + 4*s), given
// the group at j already loaded into a; each next group's reads are issued
// before the current group's fmas.
__device__ __forceinline__ float seg_lds_from(SegGroup& a, const float* w, const float* x,
                                              uint32_t K, uint32_t j, float acc) {
  SegGroup b;
#pragma unroll 1
  for (; j < K; j += 512) {
    if (j + 256 < K) seg_group_load(b, w, x, K, j + 256);
    acc = seg_group_fma(a, K, j, acc);
    if (j + 256 >= K) break;
    if (j + 512 < K) seg_group_load(a, w, x, K, j + 512);
    acc = seg_group_fma(b, K, j + 256, acc);
  }
  return acc;
}

// Segment s of the LDS row w from chunk i0 on, added to acc.
__device__ __forceinline__ float seg_lds(const float* w, const float* x, uint32_t K, uint32_t s,
                                         uint32_t i0, float acc) {
  const uint32_t j = 64u * i0 + 4u * s;
  if (j >= K) return acc;
  SegGroup a;
  seg_group_load(a, w, x, K, j);
  return seg_lds_from(a, w, x, K, j, acc);
}

// Segment s of the global row w given its first NF chunks already in r;
// longer rows stream the rest double-buffered (seg_stream).
template <int NF>
__device__ __forceinline__ float seg_tail(SegT<NF>& r, const float* __restrict__ w, const float* x,
                                          uint32_t K, uint32_t s) {
  if (64u * NF <= K) {
    const float acc = seg_fma_in<NF, true>(r, x, s, 0, 0.0f);
    return seg_stream<NF>(w, x, K, s, NF, acc);
  }
  return seg_fma(r, x, K, s, 0, 0.0f);
}

// The four row values of a quad pass from the lanes' segment sums: y[r] is
// row r's, the same in every lane.
__device__ __forceinline__ void quad_sums(float p, float (&y)[4]) {
  const float v = group_sum(p, 16);
#pragma unroll
  for (int r = 0; r < 4; ++r) y[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * r));
}

constexpr int KF = 8;  // chunks a streamed segment keeps in flight per buffer (two buffers)

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
