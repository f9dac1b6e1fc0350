// phases.h -- the phases of one token's forward pass and the sampler, as
// workgroup-level device functions. Each takes (wg, G): the calling
// workgroup and how many workgroups share the phase. The persistent kernel
// runs them back to back; the per-phase kernels run one each. Work items are
// dealt in contiguous blocks (item_of), and an item is always computed the
// same way whoever computes it.
//
// Roles inside a workgroup (BLOCK = 512 threads = 8 waves):
//  * pollers (waves 0..NPOLL-1) read mailboxes; in the matvec phases the
//    compute waves poll beside them (NWA waves), since they have no load in
//    flight there, while in the attention and the lm_head, where they do,
//    the pollers poll alone, so a poll round waits for nothing but its own
//    words;
//  * compute waves (the next NCW) compute the matvec items dealt to them
//    and store each result as soon as they have it (where rows are streamed
//    from memory instead of staged, a phase with more passes than NCW takes
//    every wave after its poll, and the results are listed in LDS and
//    stored after the phase: mv_waves, Pub);
//  * loaders (the last NLOAD waves) stage weight rows into LDS with direct
//    global->LDS loads (persistent kernel only, when a layer's share of the
//    workgroup fits): each kind's rows for the next layer are requested as
//    soon as this layer's rows of that kind have been used, and a loader
//    waits for them (exact vector-memory counts) only at the barrier before
//    their use. Loaders issue no other memory instruction, so those counts
//    hold, and no other wave ever waits for a weight load. Where rows are
//    streamed instead, the loaders pull the first blocks of the compute
//    waves' first pass into the L2 during the poll (prefetch_first) and
//    store the listed results after the phase (pub_flush).
// Attention, lm_head and the sampler run on pollers and compute waves.
#pragma once

#include <type_traits>

#include "device.h"
#include "exact.h"

namespace DG_NS {

// A kernel specialised for one model shape runs only where that shape's
// weight rows are staged in LDS (the host picks the generic kernel
// otherwise), so its streaming matvec path is compiled out.
#if defined(DG_SHAPE_SMOLLM2_135M)
constexpr bool STAGED_ONLY = true;
#else
constexpr bool STAGED_ONLY = false;
#endif

constexpr uint32_t NPOLL = 2;
// Words a polling lane owns per round in the per-layer gathers, sized so the
// specialised shape's vectors (576 and 1536 words) take one round of NWA
// polling waves; larger shapes take a few rounds.
constexpr uint32_t PW_H = STAGED_ONLY ? 2 : 4;  // hidden-size gathers
constexpr uint32_t PW_F = STAGED_ONLY ? 4 : 6;  // intermediate-size gathers
constexpr uint32_t NCW = 4;
constexpr uint32_t NLOAD = NWAVES - NPOLL - NCW;
constexpr uint32_t NWA = NPOLL + NCW;  // waves 0..NWA-1 compute attention, lm_head, sampler
static_assert(NLOAD == 2, "two loader waves");

struct Lds {
  WaitCtl* ctl;
  float* red;   // 64 floats
  float* vec;   // d.lds_vec floats: the matvec input vector
  float* vec2;  // d.lds_vec2 floats: the normalised lm_head input
  float* scr;   // d.lds_scr floats
  float* stg;   // d.lds_stg floats: staged weight rows (persistent kernel)
  u64* pub;     // d.lds_pub entries of {word, address}: listed results (Pub)
  float* trash; // 1 KB that direct-to-LDS prefetches land in (streamed kernels)
};

__device__ inline Lds lds_layout(float* base, const Dims& d) {
  Lds s;
  s.ctl = reinterpret_cast<WaitCtl*>(base);
  s.red = base + 4;
  s.vec = base + 4 + 64;
  s.vec2 = s.vec + d.lds_vec;
  s.scr = s.vec2 + d.lds_vec2;
  s.stg = s.scr + d.lds_scr;
  s.pub = reinterpret_cast<u64*>(s.stg + d.lds_stg);
  s.trash = reinterpret_cast<float*>(s.pub + 2 * d.lds_pub);
  return s;
}

// One strided gather of tagged words: element e < seg_len * n_seg comes from
// src[(e / seg_len) * src_stride + e % seg_len] and goes to dst[e].
struct Gather {
  const u64* src;
  uint32_t seg_len, n_seg, src_stride, gen;
  float* dst;
};

__device__ __forceinline__ Gather gather_strided(const u64* src, uint32_t seg_len, uint32_t n_seg,
                                                 uint32_t src_stride, uint32_t gen, float* dst) {
  Gather g;
  g.src = src;
  g.seg_len = seg_len;
  g.n_seg = n_seg;
  g.src_stride = src_stride;
  g.gen = gen;
  g.dst = dst;
  return g;
}
__device__ __forceinline__ Gather gather_vec(const u64* src, uint32_t n, uint32_t gen, float* dst) {
  return gather_strided(src, n, 1, 0, gen, dst);
}
__device__ __forceinline__ Gather no_gather() { return gather_strided(nullptr, 0, 0, 0, 0, nullptr); }


// Word offset of element e of a gather from its source.
__device__ __forceinline__ uint32_t gather_off(const Gather& g, uint32_t e) {
  if (g.n_seg <= 1) return e;
  const uint32_t seg = e / g.seg_len;
  return seg * g.src_stride + (e - seg * g.seg_len);
}

// One polling round of gather g for this lane: P words in flight.
template <uint32_t P>
struct PollState {
  uint32_t pend;
  u64 w[P > 0 ? P : 1];
};

template <uint32_t P>
__device__ __forceinline__ void poll_init(PollState<P>& ps, const Gather& g, uint32_t n,
                                          uint32_t base, uint32_t tid, uint32_t npl) {
  ps.pend = 0;
#pragma unroll
  for (uint32_t k = 0; k < P; ++k)
    if (base + tid + k * npl < n) ps.pend |= 1u << k;
}
// Every lane loads all P of its slots (a slot past the gather's end re-reads
// the gather's last word, and is never pending), so the loads carry no
// per-lane condition and the compiler counts them exactly: a check waits for
// its own round only, not for a round issued after it.
template <uint32_t P>
__device__ __forceinline__ void poll_issue(u64 (&w)[P > 0 ? P : 1], const Gather& g, uint32_t n,
                                           uint32_t base, uint32_t tid, uint32_t npl) {
  if (P == 0 || n == 0) return;
#pragma unroll
  for (uint32_t k = 0; k < P; ++k) w[k] = mb_load(g.src + gather_off(g, min(base + tid + k * npl, n - 1)));
}
template <uint32_t P>
__device__ __forceinline__ void poll_check(PollState<P>& ps, const u64 (&w)[P > 0 ? P : 1],
                                           const Gather& g, uint32_t base, uint32_t tid,
                                           uint32_t npl) {
#pragma unroll
  for (uint32_t k = 0; k < P; ++k)
    if ((ps.pend & (1u << k)) && (uint32_t)(w[k] >> 32) == g.gen) {
      lds_st(g.dst + base + tid + k * npl, __uint_as_float((uint32_t)w[k]));
      ps.pend &= ~(1u << k);
    }
}

__device__ __forceinline__ uint32_t rounds_for(uint32_t n, uint32_t per_round) {
  return per_round ? (n + per_round - 1) / per_round : (n ? 0xffffffffu : 0u);
}

// Work other waves do around a poll's barriers: pre_b1 runs before the first
// (the barrier after which the previous phase's compute is over), post_b1
// after it, while the pollers poll, and post_b2 after the last (the input is
// in LDS).
struct NoHook {
  __device__ __forceinline__ void pre_b1() const {}
  __device__ __forceinline__ void post_b1() const {}
  __device__ __forceinline__ void post_b2() const {}
};

// Wait until every element of up to three gathers carries its generation and
// copy the values to LDS. Only the first `npoll_waves` waves read memory; a
// polling lane owns P0 + P1 + P2 words per round (sized to the call site)
// and keeps two polls of them in flight: the second is issued a fraction of
// a memory round trip after the first, and each is re-issued as soon as it
// has been checked, so a word that becomes current is seen about one round
// trip later rather than up to two. The lane loops until its own words are
// all current, and the block then meets at a barrier. Returns false
// (uniformly) if the run was aborted.
constexpr uint32_t POLL_STAGGER = 8;  // s_sleep units (64 cycles) between the two polls
template <uint32_t P0, uint32_t P1 = 0, uint32_t P2 = 0, class H = NoHook>
__device__ __forceinline__ bool poll_gather(const Gather& g0, const Gather& g1, const Gather& g2,
                                            uint32_t npoll_waves, DevState* st, WaitCtl* ctl,
                                            const H& hook = H()) {
  const uint32_t tid = threadIdx.x;
  const uint32_t npl = npoll_waves * WAVE;
  hook.pre_b1();
  // The destination LDS may still be read by the previous phase.
  __syncthreads();
  hook.post_b1();
  if (tid < npl) {
    const uint32_t n0 = g0.seg_len * g0.n_seg, n1 = g1.seg_len * g1.n_seg;
    const uint32_t n2 = g2.seg_len * g2.n_seg;
    const uint32_t rounds = max(max(rounds_for(n0, P0 * npl), rounds_for(n1, P1 * npl)),
                                rounds_for(n2, P2 * npl));
    for (uint32_t r = 0; r < rounds; ++r) {
      const uint32_t b0 = r * P0 * npl, b1 = r * P1 * npl, b2 = r * P2 * npl;
      PollState<P0> s0;
      PollState<P1> s1;
      PollState<P2> s2;
      poll_init(s0, g0, n0, b0, tid, npl);
      poll_init(s1, g1, n1, b1, tid, npl);
      poll_init(s2, g2, n2, b2, tid, npl);
      u64 x0[P0 > 0 ? P0 : 1], x1[P1 > 0 ? P1 : 1], x2[P2 > 0 ? P2 : 1];  // the second poll
      poll_issue<P0>(s0.w, g0, n0, b0, tid, npl);
      poll_issue<P1>(s1.w, g1, n1, b1, tid, npl);
      poll_issue<P2>(s2.w, g2, n2, b2, tid, npl);
      __builtin_amdgcn_s_sleep(POLL_STAGGER);
      poll_issue<P0>(x0, g0, n0, b0, tid, npl);
      poll_issue<P1>(x1, g1, n1, b1, tid, npl);
      poll_issue<P2>(x2, g2, n2, b2, tid, npl);
      for (uint32_t spins = 0;; ++spins) {
        poll_check(s0, s0.w, g0, b0, tid, npl);
        poll_check(s1, s1.w, g1, b1, tid, npl);
        poll_check(s2, s2.w, g2, b2, tid, npl);
        if (__all((s0.pend | s1.pend | s2.pend) == 0)) break;
        poll_issue<P0>(s0.w, g0, n0, b0, tid, npl);
        poll_issue<P1>(s1.w, g1, n1, b1, tid, npl);
        poll_issue<P2>(s2.w, g2, n2, b2, tid, npl);
        poll_check(s0, x0, g0, b0, tid, npl);
        poll_check(s1, x1, g1, b1, tid, npl);
        poll_check(s2, x2, g2, b2, tid, npl);
        if (__all((s0.pend | s1.pend | s2.pend) == 0)) break;
        poll_issue<P0>(x0, g0, n0, b0, tid, npl);
        poll_issue<P1>(x1, g1, n1, b1, tid, npl);
        poll_issue<P2>(x2, g2, n2, b2, tid, npl);
        if (spins >= SPIN_LIMIT) {
          st_coherent_u32(&st->abort, 1u);
          ctl->abort_seen = 1;
          break;
        }
        if ((spins & 63) == 63 && ld_coherent_u32(&st->abort)) {
          ctl->abort_seen = 1;
          break;
        }
      }
      if (ctl->abort_seen) break;
    }
  }
  __syncthreads();
  hook.post_b2();
  return ctl->abort_seen == 0;
}

template <uint32_t P0, uint32_t P1, class H = NoHook>
__device__ __forceinline__ bool poll_gather(const Gather& g0, const Gather& g1, uint32_t npw,
                                            DevState* st, WaitCtl* ctl, const H& hook = H()) {
  return poll_gather<P0, P1, 0, H>(g0, g1, no_gather(), npw, st, ctl, hook);
}
template <uint32_t P0, class H = NoHook>
__device__ __forceinline__ bool poll_gather(const Gather& g0, uint32_t npw, DevState* st,
                                            WaitCtl* ctl, const H& hook = H()) {
  return poll_gather<P0, 0, 0, H>(g0, no_gather(), no_gather(), npw, st, ctl, hook);
}

// Number of the n items of a phase dealt to workgroup wg: n / G, plus one for
// the first n % G workgroups.
__device__ __forceinline__ uint32_t rows_owned(uint32_t n, uint32_t wg, uint32_t G) {
  return wg < n ? (n - wg + G - 1) / G : 0;
}
// Item k (k < rows_owned) of workgroup wg. Each workgroup's items are
// contiguous, so its results fill whole mailbox lines and a reader's line
// holds the words of one or two writers, not of eight.
__device__ __forceinline__ uint32_t item_of(uint32_t n, uint32_t wg, uint32_t G, uint32_t k) {
  const uint32_t q = n / G, r = n - q * G;
  return wg * q + min(wg, r) + k;
}

// ------------------------------------------------------------ publishing
//
// Where weight rows are staged in LDS, a compute wave stores each result as
// soon as it has it: a tagged mailbox word (agent-scope relaxed 64-bit
// store, lane 0), the eight replicas of a replicated mailbox (lanes 0..7,
// one each), or a plain float to the K/V cache (lane 0); no barrier ends the
// phase, the next phase's first barrier orders the reuse of its LDS.
// (Handing the results over through LDS for other waves to store after a
// phase-end barrier cost 25 us per token more at 135M.) Where rows are
// streamed from HBM, a store would sit in the compute wave's in-order
// vector-memory counter ahead of its next loads and polls while HBM is
// saturated, so results are listed in LDS instead ({word, address | kind},
// entry i per result) and, after a phase-end barrier, the loader waves --
// idle when nothing is staged -- store them (pub_flush).
struct Pub {
  bool list;  // wave-uniform: list the results (rows streamed) or store them now
  u64* ent;   // LDS entries
};
__device__ __forceinline__ Pub pub_for(bool staged, const Lds& s) {
  Pub p;
  p.list = !(STAGED_ONLY || staged);
  p.ent = s.pub;
  return p;
}
// Result i: a tagged mailbox word.
__device__ __forceinline__ void pub_word(const Pub& p, uint32_t i, u64* slot, float v, uint32_t gen,
                                         uint32_t lane) {
  if (lane != 0) return;
  if (p.list) {
    AS_LDS u64* e = lptr(p.ent + 2 * i);
    e[0] = ((u64)gen << 32) | (u64)__float_as_uint(v);
    e[1] = (u64)(uintptr_t)slot;
  } else {
    mb_put(slot, v, gen);
  }
}
// Result i: a plain float (address bit 0 marks the kind in a list).
__device__ __forceinline__ void pub_float(const Pub& p, uint32_t i, float* ptr, float v, uint32_t lane) {
  if (lane != 0) return;
  if (p.list) {
    AS_LDS u64* e = lptr(p.ent + 2 * i);
    e[0] = (u64)__float_as_uint(v);
    e[1] = (u64)(uintptr_t)ptr | 1u;
  } else {
    st_coherent(ptr, v);
  }
}
// Result i: nothing (a list entry that stores nothing).
__device__ __forceinline__ void pub_none(const Pub& p, uint32_t i, uint32_t lane) {
  if (p.list && lane == 0) lptr(p.ent + 2 * i)[1] = 0;
}
// Result i: the same word in every replica of a replicated mailbox (replicas
// rep_words apart; address bit 1 marks the kind in a list).
__device__ __forceinline__ void pub_word_rep(const Pub& p, uint32_t i, u64* slot, float v,
                                             uint32_t gen, uint32_t rep_words, uint32_t lane) {
  const u64 w = ((u64)gen << 32) | (u64)__float_as_uint(v);
  if (p.list) {
    if (lane == 0) {
      AS_LDS u64* e = lptr(p.ent + 2 * i);
      e[0] = w;
      e[1] = (u64)(uintptr_t)slot | 2u;
    }
  } else if (lane < MB_REPS) {
    __hip_atomic_store(gptr(slot + (size_t)lane * rep_words), w, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}
// A workgroup's replica of a replicated mailbox.
__device__ __forceinline__ const u64* rep_of(const Args& a, const u64* base, uint32_t wg) {
  return base + (size_t)(wg % MB_REPS) * a.rep_words;
}

// A listed phase's end: a barrier, then the loader waves store entries
// [0, n).
__device__ __forceinline__ void pub_flush(const Pub& p, uint32_t n, uint32_t rep_words = 0) {
  if (!p.list) return;
  __syncthreads();
  if (threadIdx.x < NWA * WAVE) return;
  for (uint32_t i = threadIdx.x - NWA * WAVE; i < n; i += NLOAD * WAVE) {
    const AS_LDS u64* e = lptr(p.ent + 2 * i);
    const u64 w = e[0], addr = e[1];
    if (addr & 1u) {
      st_coherent(reinterpret_cast<float*>((uintptr_t)(addr & ~(u64)1)), __uint_as_float((uint32_t)w));
    } else if (addr & 2u) {
      u64* q = reinterpret_cast<u64*>((uintptr_t)(addr & ~(u64)2));
#pragma unroll
      for (uint32_t r = 0; r < MB_REPS; ++r)
        __hip_atomic_store(gptr(q + (size_t)r * rep_words), w, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else if (addr) {
      __hip_atomic_store(gptr(reinterpret_cast<u64*>((uintptr_t)addr)), w, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------- matvec items

enum ItemKind : uint32_t { IK_QKV = 0, IK_O = 1, IK_GU = 2, IK_D = 3 };

// Items of each kind: QKV pairs (rows i, i + hd/2 of one head, so RoPE needs
// no exchange), O rows, GU pairs (gate row j, up row j), D rows. Item k of a
// kind owned by workgroup wg is number own_item(d, kind, wg, G, k); compute wave
// k % NCW computes it and loader k % NLOAD stages it.
__device__ __forceinline__ uint32_t kind_items(const Dims& d, uint32_t kind) {
  return kind == IK_QKV ? d.qkv_rows / 2 : (kind == IK_GU ? d.ff : d.h);
}
__device__ __forceinline__ uint32_t kind_k(const Dims& d, uint32_t kind) {
  return kind == IK_O ? d.q : (kind == IK_D ? d.ff : d.h);
}
__device__ __forceinline__ uint32_t kind_rows(uint32_t kind) {
  return (kind == IK_QKV || kind == IK_GU) ? 2u : 1u;
}

// The workgroups' items of a kind. O rows skip the first d.o_skip
// workgroups, which take the attention items of the usual positions: their
// O rows would wait for their attention to finish, and every gate/up
// workgroup waits for the last O row.
__device__ __forceinline__ uint32_t own_count(const Dims& d, uint32_t kind, uint32_t wg, uint32_t G) {
  if (kind == IK_O) return wg < d.o_skip ? 0u : rows_owned(d.h, wg - d.o_skip, G - d.o_skip);
  return rows_owned(kind_items(d, kind), wg, G);
}
__device__ __forceinline__ uint32_t own_item(const Dims& d, uint32_t kind, uint32_t wg, uint32_t G,
                                             uint32_t k) {
  if (kind == IK_O) return item_of(d.h, wg - d.o_skip, G - d.o_skip, k);
  return item_of(kind_items(d, kind), wg, G, k);
}

// The layer table entry of layer l (scalar loads: see cptr).
__device__ __forceinline__ LayerW layer_w(const Args& a, uint32_t l) {
  const AS_CONST LayerW* p = cptr(a.layers) + l;
  LayerW W;
  W.attn_norm = p->attn_norm;
  W.wqkv = p->wqkv;
  W.bqkv = p->bqkv;
  W.wo = p->wo;
  W.ffn_norm = p->ffn_norm;
  W.wg = p->wg;
  W.wu = p->wu;
  W.wd = p->wd;
  return W;
}

// Row pointers and length of item k of a kind in layer l.
struct ItemRows {
  const float* w0;
  const float* w1;  // null for single-row kinds
  uint32_t K;
};

__device__ __forceinline__ ItemRows item_rows(const Args& a, uint32_t kind, uint32_t l, uint32_t k,
                                              uint32_t wg, uint32_t G) {
  const Dims d = shape_dims(a.d);
  const LayerW W = layer_w(a, l);
  const uint32_t it = own_item(d, kind, wg, G, k);
  ItemRows r;
  if (kind == IK_QKV) {
    const uint32_t hb = it / d.half, i = it - hb * d.half;
    const uint32_t r0 = hb * d.hd + i;
    r.w0 = W.wqkv + (size_t)r0 * d.h;
    r.w1 = W.wqkv + (size_t)(r0 + d.half) * d.h;
    r.K = d.h;
  } else if (kind == IK_O) {
    r.w0 = W.wo + (size_t)it * d.q;
    r.w1 = nullptr;
    r.K = d.q;
  } else if (kind == IK_GU) {
    r.w0 = W.wg + (size_t)it * d.h;
    r.w1 = W.wu + (size_t)it * d.h;
    r.K = d.h;
  } else {
    r.w0 = W.wd + (size_t)it * d.ff;
    r.w1 = nullptr;
    r.K = d.ff;
  }
  return r;
}

// Offset of kind X's rows in the staging region, by selects rather than an
// indexed load (a run-time index into the Dims copy would put it on the
// stack).
__device__ __forceinline__ uint32_t stg_off_of(const Dims& d, uint32_t kind) {
  return kind == 0 ? d.stg_off[0] : kind == 1 ? d.stg_off[1] : kind == 2 ? d.stg_off[2] : d.stg_off[3];
}

// Staging of the workgroup's rows in LDS (persistent kernel). Kind X's items
// sit back to back at s.stg + d.stg_off[X], item k's rows contiguous.
struct Stager {
  bool on;             // some kind's rows are staged: the loader waves stage them
  uint32_t mask;       // bit k: kind k's rows are staged (else compute waves stream them)
  const Args* a;
  float* stg;
  uint32_t wg, G, ld;  // ld: this wave's loader index (loaders only)
  bool loader;
  // Loads a loader may leave in flight when kind X's rows must have landed:
  // at the first barrier of X's phase, the batches requested after X's are
  // those of the two kinds whose phases came since (the kind before X is
  // requested only after that barrier).
  uint32_t wait[4];
};
// Kind X's rows are staged in LDS (a wave-uniform test).
__device__ __forceinline__ bool staged(const Stager& sg, uint32_t kind) {
  return STAGED_ONLY || (sg.mask >> kind & 1u);
}

// 16 bytes per lane from global memory straight into LDS: lane i's bytes
// land at LDS byte address lds_base + 16*i (lds_base is wave-uniform). M0,
// which the instruction takes the LDS address from, is saved and restored.
// The compiler does not see this load, so it never waits for it: loaders
// wait explicitly (stage_wait).
__device__ __forceinline__ void dma16(const float* src, uint32_t lds_base) {
  uint32_t m0_saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(m0_saved)
      : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds_base))
      : "memory");
}

// s_waitcnt vmcnt(n) for a run-time n (clamped to the counter's 63).
__device__ __forceinline__ void stage_wait(uint32_t n) {
#define DG_VMW(N) \
  case N:         \
    asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); \
    break;
  switch (n < 63u ? n : 63u) {
    DG_VMW(0) DG_VMW(1) DG_VMW(2) DG_VMW(3) DG_VMW(4) DG_VMW(5) DG_VMW(6) DG_VMW(7)
    DG_VMW(8) DG_VMW(9) DG_VMW(10) DG_VMW(11) DG_VMW(12) DG_VMW(13) DG_VMW(14) DG_VMW(15)
    DG_VMW(16) DG_VMW(17) DG_VMW(18) DG_VMW(19) DG_VMW(20) DG_VMW(21) DG_VMW(22) DG_VMW(23)
    DG_VMW(24) DG_VMW(25) DG_VMW(26) DG_VMW(27) DG_VMW(28) DG_VMW(29) DG_VMW(30) DG_VMW(31)
    DG_VMW(32) DG_VMW(33) DG_VMW(34) DG_VMW(35) DG_VMW(36) DG_VMW(37) DG_VMW(38) DG_VMW(39)
    DG_VMW(40) DG_VMW(41) DG_VMW(42) DG_VMW(43) DG_VMW(44) DG_VMW(45) DG_VMW(46) DG_VMW(47)
    DG_VMW(48) DG_VMW(49) DG_VMW(50) DG_VMW(51) DG_VMW(52) DG_VMW(53) DG_VMW(54) DG_VMW(55)
    DG_VMW(56) DG_VMW(57) DG_VMW(58) DG_VMW(59) DG_VMW(60) DG_VMW(61) DG_VMW(62)
    default:
      asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
      break;
  }
#undef DG_VMW
}

// Loads one loader wave issues for its items of a kind: 1 KB per load.
__device__ __forceinline__ uint32_t stage_loads(const Dims& d, uint32_t kind, uint32_t wg,
                                                uint32_t G, uint32_t ld) {
  const uint32_t cnt = own_count(d, kind, wg, G);
  const uint32_t mine = cnt > ld ? (cnt - ld + NLOAD - 1) / NLOAD : 0;
  return mine * kind_rows(kind) * ((kind_k(d, kind) + 255) / 256);
}

__device__ __forceinline__ Stager make_stager(const Args& a, const Lds& s, uint32_t wg, uint32_t G,
                                              bool on) {
  Stager sg;
  sg.mask = STAGED_ONLY ? 0xFu : (on ? a.d.stg_mask : 0u);
  sg.on = sg.mask != 0;
  sg.a = &a;
  sg.stg = s.stg;
  sg.wg = wg;
  sg.G = G;
  const uint32_t wave = threadIdx.x / WAVE;
  sg.loader = wave >= NWA;
  sg.ld = sg.loader ? wave - NWA : 0;
  uint32_t n[4], tot = 0;
  for (uint32_t k = 0; k < 4; ++k) {
    n[k] = (sg.mask >> k & 1u) ? stage_loads(shape_dims(a.d), k, wg, G, sg.ld) : 0u;
    tot += n[k];
  }
  for (uint32_t k = 0; k < 4; ++k) sg.wait[k] = tot - n[k] - n[(k + 3) % 4];
  return sg;
}

// Loader: request this wave's items of `kind`, layer l.
__device__ __forceinline__ void stage_issue(const Stager& sg, uint32_t kind, uint32_t l) {
  const Args& a = *sg.a;
  const Dims d = shape_dims(a.d);
  const uint32_t lane = threadIdx.x % WAVE;
  const uint32_t cnt = own_count(d, kind, sg.wg, sg.G);
  const uint32_t K = kind_k(d, kind), nr = kind_rows(kind), nseg = (K + 255) / 256;
  const uint32_t base = (uint32_t)(uintptr_t)(sg.stg + stg_off_of(d, kind));
  for (uint32_t k = sg.ld; k < cnt; k += NLOAD) {
    const ItemRows r = item_rows(a, kind, l, k, sg.wg, sg.G);
    for (uint32_t row = 0; row < nr; ++row) {
      const float* src = row ? r.w1 : r.w0;
      const uint32_t dst = base + ((k * nr + row) * K) * 4u;
      for (uint32_t sgm = 0; sgm < nseg; ++sgm) {
        const uint32_t rem = K - sgm * 256;
        if (rem >= 256 || lane * 4 < rem) dma16(src + sgm * 256 + lane * 4, dst + sgm * 1024);
      }
    }
  }
}

// What the loader waves do at a matvec phase's first barrier: before it,
// wait until at most `wait` of their loads are in flight (none if NO_WAIT);
// after it, request kind `issue` of layer `layer` (none if issue >= 4).
constexpr uint32_t NO_WAIT = 0xffffffffu;
struct LoadOp {
  uint32_t issue, layer, wait;
};
__device__ __forceinline__ LoadOp no_load() {
  LoadOp o;
  o.issue = 4;
  o.layer = 0;
  o.wait = NO_WAIT;
  return o;
}

// Staged rows of item k of a kind (pairs: second row at +K).
__device__ __forceinline__ const float* staged_item(const Stager& sg, uint32_t kind, uint32_t k) {
  const Dims d = shape_dims(sg.a->d);
  return sg.stg + stg_off_of(d, kind) + k * kind_rows(kind) * kind_k(d, kind);
}

// Lane partial of x . x over the elements 4*lane + 256*i of a length-K
// vector (i ascending).
__device__ __forceinline__ float sumsq_lane(const float* x, uint32_t K, uint32_t lane) {
  float ss = 0.0f;
  uint32_t j = lane * 4;
  // Four reads in flight, then the fmas in order.
  for (; j + 768 < K; j += 1024) {
    const float4 v0 = lds4(x + j), v1 = lds4(x + j + 256), v2 = lds4(x + j + 512),
                 v3 = lds4(x + j + 768);
    ss = fmaf(v0.x, v0.x, ss); ss = fmaf(v0.y, v0.y, ss); ss = fmaf(v0.z, v0.z, ss); ss = fmaf(v0.w, v0.w, ss);
    ss = fmaf(v1.x, v1.x, ss); ss = fmaf(v1.y, v1.y, ss); ss = fmaf(v1.z, v1.z, ss); ss = fmaf(v1.w, v1.w, ss);
    ss = fmaf(v2.x, v2.x, ss); ss = fmaf(v2.y, v2.y, ss); ss = fmaf(v2.z, v2.z, ss); ss = fmaf(v2.w, v2.w, ss);
    ss = fmaf(v3.x, v3.x, ss); ss = fmaf(v3.y, v3.y, ss); ss = fmaf(v3.z, v3.z, ss); ss = fmaf(v3.w, v3.w, ss);
  }
  for (; j < K; j += 256) {
    const float4 v = lds4(x + j);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  return ss;
}

// 1/rms of the length-n vector in LDS (ops.rs:84-95: 1/sqrt(ss/n + eps)).
// The RMSNorm weight is folded into the consuming matrix columns at load
// time, so the normalised dot product is inv * (W' . x).
__device__ __forceinline__ float rms_inv(const float* x, uint32_t n, float eps, uint32_t lane) {
  const float ss = wave_sum(sumsq_lane(x, n, lane));
  return 1.0f / sqrtf(ss / (float)n + eps);
}

// Matvec passes. A compute wave takes the rows of its items four at a time
// (a quad pass, device.h): lane 16*r + s computes segment s of row slot r.
// Pair kinds put items k and k + n in the slots (gate/up or the two RoPE
// rows of each), single-row kinds items k, k + n, k + 2n, k + 3n, where n is
// the number of waves that share the phase's items (NCW where rows are
// staged, every wave where they are streamed); a wave's passes start at
// items cw, cw + n * pass_items, ...
__host__ __device__ constexpr uint32_t pass_items(bool pair) { return pair ? 2u : 4u; }
__device__ __forceinline__ uint32_t slot_item(bool pair, uint32_t k, uint32_t r, uint32_t n = NCW) {
  return k + n * (pair ? r / 2 : r);
}

// A compute wave's first pass of a staged matvec phase: the lane's
// PRE_F4 first chunks of its segment, read from LDS into registers while the
// pollers wait for the phase's input, so only the input vector is read after
// the barrier; longer rows read the rest from LDS later.
constexpr int PRE_F4 = 9;
struct Preload {
  float4 w[PRE_F4];
  bool any;  // the wave has an item
};

// Staged row of slot r of the pass starting at item k (nullptr: no item).
__device__ __forceinline__ const float* staged_slot(const Stager& sg, uint32_t kind, uint32_t k,
                                                    uint32_t r, uint32_t cnt) {
  const bool pair = kind_rows(kind) == 2;
  const uint32_t it = slot_item(pair, k, r);
  if (it >= cnt) return nullptr;
  const float* w = staged_item(sg, kind, it);
  return pair && (r & 1u) ? w + kind_k(shape_dims(sg.a->d), kind) : w;
}

__device__ __forceinline__ void preload_rows(Preload& P, const Stager& sg, uint32_t kind,
                                             uint32_t cw, uint32_t lane) {
  const Dims d = shape_dims(sg.a->d);
  const uint32_t cnt = own_count(d, kind, sg.wg, sg.G);
  const uint32_t K = kind_k(d, kind), s = qseg(lane);
  P.any = cw < cnt;
  if (!P.any) return;
  const float* w = staged_slot(sg, kind, cw, qrow(lane), cnt);
  if (!w) return;
  const float* wb = pin(w + 4u * s);
#pragma unroll
  for (int i = 0; i < PRE_F4; ++i) {
    const uint32_t j = 64u * i + 4u * s;
    if (j < K) P.w[i] = lds4(wb + 64 * i);
  }
}

// The lane's segment of the first pass: the preloaded chunks, then (longer
// rows) the rest from LDS. Every read of x, and the first group of the rest,
// is issued before the first fma.
__device__ __forceinline__ float pass_pre(const Preload& P, const float* w, const float* x,
                                          uint32_t K, uint32_t s) {
  if (!w) return 0.0f;
  const float* xb = pin(x + 4u * s);
  float4 xv[PRE_F4];
#pragma unroll
  for (int i = 0; i < PRE_F4; ++i) {
    const uint32_t j = 64u * i + 4u * s;
    if (j < K) xv[i] = lds4(xb + 64 * i);
  }
  const uint32_t jr = 64u * PRE_F4 + 4u * s;
  SegGroup g;
  if (jr < K) seg_group_load(g, w, x, K, jr);
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < PRE_F4; ++i) {
    const uint32_t j = 64u * i + 4u * s;
    if (j < K) {
      acc = fmaf(P.w[i].x, xv[i].x, acc);
      acc = fmaf(P.w[i].y, xv[i].y, acc);
      acc = fmaf(P.w[i].z, xv[i].z, acc);
      acc = fmaf(P.w[i].w, xv[i].w, acc);
    }
  }
  return jr < K ? seg_lds_from(g, w, x, K, jr, acc) : acc;
}

// Barrier work of a staged matvec phase: loaders wait for this kind's rows
// before the first barrier and request the previous kind's once the poll is
// over (requested while the pollers poll, that burst of weight reads competes
// with the poll's reads); compute waves preload their first pass while the
// pollers poll.
struct MvHook {
  const Stager* sg;
  LoadOp op;
  Preload* pre;
  uint32_t kind;
  __device__ __forceinline__ void pre_b1() const {
    if (sg->on && sg->loader && op.wait != NO_WAIT) stage_wait(op.wait);
  }
  __device__ __forceinline__ void post_b1() const {
    if (!staged(*sg, kind)) return;
    const uint32_t wave = threadIdx.x / WAVE;
    if (!sg->loader && wave >= NPOLL) preload_rows(*pre, *sg, kind, wave - NPOLL, threadIdx.x % WAVE);
  }
  __device__ __forceinline__ void post_b2() const {
    if (sg->on && sg->loader && op.issue < 4) stage_issue(*sg, op.issue, op.layer);
  }
};

__device__ __forceinline__ MvHook mv_hook(const Stager& sg, LoadOp op, Preload& P, uint32_t kind) {
  MvHook h;
  h.sg = &sg;
  h.op = op;
  h.pre = &P;
  h.kind = kind;
  return h;
}

// The waves that compute a matvec phase's items: the NCW compute waves
// where its rows are staged in LDS (the pollers and loaders have their own
// work then). Where each lane streams its rows from memory nothing else runs
// after the poll, and a phase of more passes than NCW waves but no more than
// NWAVES takes every wave (one round of passes instead of two; with more
// passes, twice the waves only compete for the same bandwidth). An item's
// arithmetic does not depend on which wave takes it. (The phases test the
// staged-only kernel's compute waves directly before calling this: the same
// test made through it costs that kernel a spilled register.)
struct MvWaves {
  bool on;       // this wave computes items
  uint32_t cw;   // its index among them
  uint32_t n;    // how many there are
};
__device__ __forceinline__ MvWaves mv_waves(const Stager& sg, uint32_t wave, const Args& a,
                                            uint32_t kind, uint32_t wg, uint32_t G) {
  MvWaves m;
  bool all = false;
  if (!(STAGED_ONLY || sg.on)) {
    const uint32_t cnt = own_count(shape_dims(a.d), kind, wg, G);
    const uint32_t per = pass_items(kind_rows(kind) == 2);
    const uint32_t passes = (cnt + per - 1) / per;
    all = passes > NCW && passes <= NWAVES;
  }
  m.on = all || (wave >= NPOLL && wave < NWA);
  m.cw = all ? wave : wave - NPOLL;
  m.n = all ? NWAVES : NCW;
  return m;
}

// Streamed phases whose items take only the compute waves: while the input
// is polled for, the loader waves pull the first 1024 elements (the first
// two blocks a lane streams) of the rows of every compute wave's first pass
// into the L2 (direct-to-LDS loads into a line nothing reads; no wave waits
// for them), so the compute waves' first loads after the poll hit the L2
// instead of HBM.
__device__ __forceinline__ void prefetch_first(const Args& a, uint32_t kind, uint32_t l, uint32_t wg,
                                               uint32_t G, const Lds& s, uint32_t lw, uint32_t lane) {
  const Dims d = shape_dims(a.d);
  if (d.lds_stg) return;  // the 1 KB line exists only in layouts without staged rows
  const uint32_t cnt = own_count(d, kind, wg, G);
  const bool pair = kind_rows(kind) == 2;
  const uint32_t nit = min(cnt, NCW * pass_items(pair));
  const uint32_t K = kind_k(d, kind), lim = min(K, 1024u);
  const uint32_t trash = (uint32_t)(uintptr_t)s.trash;
  for (uint32_t k = lw; k < nit; k += NLOAD) {
    const ItemRows rw = item_rows(a, kind, l, k, wg, G);
    for (uint32_t off = 0; off + 256 <= lim; off += 256) {
      dma16(rw.w0 + off + lane * 4, trash);
      if (pair) dma16(rw.w1 + off + lane * 4, trash);
    }
  }
}

// body(k, y0, y1) for every item k of `kind` dealt to wave mw.cw of mw.n,
// with its dot products against the LDS vector x (y1 = 0 for single-row
// kinds), wave-uniform. Staged: the preloaded first pass, then further
// passes read from LDS. Otherwise each lane streams its segment of its row
// from memory.
template <class F>
__device__ __forceinline__ void items_dot(const Args& a, uint32_t kind, MvWaves mw, uint32_t l,
                                          const Stager& sg, const Preload& P, const float* x,
                                          uint32_t wg, uint32_t G, uint32_t lane, F body) {
  const uint32_t cw = mw.cw;
  const Dims dd = shape_dims(a.d);
  const uint32_t cnt = own_count(dd, kind, wg, G);
  const uint32_t K = kind_k(dd, kind);
  const bool pair = kind_rows(kind) == 2;
  const uint32_t r = qrow(lane), s = qseg(lane);
  // The results of the pass at item k, whose slots are nw items apart.
  auto emit = [&](uint32_t k, float acc, uint32_t nw) {
    float y[4];
    quad_sums(acc, y);
    if (pair) {
      body(k, y[0], y[1]);
      if (k + nw < cnt) body(k + nw, y[2], y[3]);
    } else {
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u)
        if (k + nw * u < cnt) body(k + nw * u, y[u], 0.0f);
    }
  };
  if (staged(sg, kind)) {
    if (!P.any) return;
    const uint32_t step = NCW * pass_items(pair);
    emit(cw, pass_pre(P, staged_slot(sg, kind, cw, r, cnt), x, K, s), NCW);
    for (uint32_t k = cw + step; k < cnt; k += step) {
      const float* w = staged_slot(sg, kind, k, r, cnt);
      emit(k, w ? seg_lds(w, x, K, s, 0, 0.0f) : 0.0f, NCW);
    }
    return;
  }
  const uint32_t nw = mw.n, step = nw * pass_items(pair);
  for (uint32_t k = cw; k < cnt; k += step) {
    const uint32_t it = slot_item(pair, k, r, nw);
    float acc = 0.0f;
    if (it < cnt) {
      const ItemRows rw = item_rows(a, kind, l, it, wg, G);
      acc = seg_stream<KF>(pair && (r & 1u) ? rw.w1 : rw.w0, x, K, s, 0, 0.0f);
    }
    emit(k, acc, nw);
  }
}

constexpr uint32_t MAX_GROUP = 4;
constexpr uint32_t KU_DEF = 2;  // score passes whose K rows a lane keeps in flight
constexpr uint32_t VU_DEF = 8;  // V float4 a lane keeps in flight

// Lane geometry of the attention (head_dim = 16 * 2^k, at most 256). The
// attention math runs on the NCW compute waves (attention wave w = wave -
// NPOLL) while the pollers wait for q/k/v, so the compute waves can have the
// chunk's K/V rows in flight during the poll without delaying it (a wave's
// loads complete in order). Every lane holds float4 pieces of rows:
//  score pass: lps = head_dim/16 lanes per position, 4 float4 each; a wave
//              scores pw = WAVE/lps positions, the block NCW*pw per pass;
//  value pass: lv = head_dim/4 lanes per position, 1 float4 each; a wave
//              takes pv = WAVE/lv positions per step.
struct AttGeo {
  uint32_t lps, pw, lv, pv;
};
__device__ __forceinline__ AttGeo att_geo(uint32_t hd) {
  AttGeo g;
  g.lps = hd / 16;
  g.pw = WAVE / g.lps;
  g.lv = hd / 4;
  g.pv = WAVE / g.lv;
  return g;
}

// ------------------------------------------------------------------ QKV

// What the QKV epilogue of item k needs from memory: the RoPE rotation
// (cos, sin) and the biases of its two rows.
__device__ __forceinline__ float4 qkv_epi_load(const Args& a, uint32_t l, uint32_t pos, uint32_t k,
                                               uint32_t wg, uint32_t G) {
  const Dims d = shape_dims(a.d);
  const uint32_t p = item_of(d.qkv_rows / 2, wg, G, k);
  const uint32_t hb = p / d.half, i = p - hb * d.half;
  const uint32_t r0 = hb * d.hd + i;
  float4 e = make_float4(1.0f, 0.0f, 0.0f, 0.0f);
  if (hb < d.nh + d.nkv) {
    const float2 cs = ldg2(a.rope + (size_t)pos * d.half + i);
    e.x = cs.x;
    e.y = cs.y;
  }
  const float* b = (cptr(a.layers) + l)->bqkv;
  if (b) {
    e.z = ldg(b + r0);
    e.w = ldg(b + r0 + d.half);
  }
  return e;
}

constexpr uint32_t QKV_PRE = 2;  // epilogue inputs a compute wave loads before the wait

// rmsnorm -> q/k/v rows (+bias) -> RoPE on q and k (model.rs:460-465) ->
// k, v appended to the cache at `pos` (model.rs:466-467).
__device__ __forceinline__ bool phase_qkv(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                          uint32_t token, uint32_t wg, uint32_t G, const Lds& s,
                                          const Stager& sg) {
  const Dims d = shape_dims(a.d);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const MvWaves mw = mv_waves(sg, wave, a, IK_QKV, wg, G);
  if (!(STAGED_ONLY || sg.on) && mw.n == NCW && wave >= NWA) prefetch_first(a, IK_QKV, l, wg, G, s, wave - NWA, lane);
  const bool compute = mw.on;
  const uint32_t cw = mw.cw;  // meaningful for computing waves only
  const uint32_t cnt = rows_owned(d.qkv_rows / 2, wg, G);
  // The epilogue inputs of the wave's first items are loaded before the wait.
  float4 pre[QKV_PRE];
  if (compute) {
#pragma unroll
    for (uint32_t u = 0; u < QKV_PRE; ++u) {
      const uint32_t k = cw + mw.n * u;
      if (k < cnt) pre[u] = qkv_epi_load(a, l, pos, k, wg, G);
    }
  }
  Preload P;
  const Pub pub = pub_for(sg.on, s);
  LoadOp op = no_load();
  if (staged(sg, IK_D)) {
    op.issue = IK_D;  // the previous layer's D rows are used: this layer's
    op.layer = l;
  }
  if (staged(sg, IK_QKV)) op.wait = sg.wait[IK_QKV];
  const MvHook hk = mv_hook(sg, op, P, IK_QKV);
  if (l == 0) {
    // The embedding row (model.rs:428), read by the pollers only.
    hk.pre_b1();
    __syncthreads();
    hk.post_b1();
    const float* e = a.embed + (size_t)token * d.h;
    for (uint32_t i = threadIdx.x; i < d.h && threadIdx.x < NPOLL * WAVE; i += NPOLL * WAVE)
      lds_st(s.vec + i, ldg(e + i));
    __syncthreads();
    hk.post_b2();
  } else if (!poll_gather<PW_H>(gather_vec(rep_of(a, a.mb_xd, wg), d.h, gen_of(d, tick, l - 1, PH_D), s.vec), NWA,
                             a.st, s.ctl, hk)) {
    return false;
  }
  if (compute && cnt > 0) {
    const float inv = rms_inv(s.vec, d.h, d.eps, lane);
    const uint32_t gen = gen_of(d, tick, l, PH_QKV);
    items_dot(a, IK_QKV, mw, l, sg, P, s.vec, wg, G, lane, [&](uint32_t k, float y0, float y1) {
      const uint32_t u = (k - cw) / mw.n;
      float4 e;
      if (u == 0)
        e = pre[0];
      else if (u == 1)
        e = pre[1];
      else
        e = qkv_epi_load(a, l, pos, k, wg, G);
      const uint32_t p = item_of(d.qkv_rows / 2, wg, G, k);
      const uint32_t hb = p / d.half, i = p - hb * d.half;
      const uint32_t r0 = hb * d.hd + i, r1 = r0 + d.half;
      y0 = y0 * inv + e.z;
      y1 = y1 * inv + e.w;
      float a0 = y0, a1 = y1;
      if (hb < d.nh + d.nkv) {
        a0 = y0 * e.x - y1 * e.y;
        a1 = y1 * e.x + y0 * e.y;
      }
      if (hb >= d.nh) {  // the cache rows first: attention reads them a token later
        const bool is_k = hb < d.nh + d.nkv;
        const uint32_t g = is_k ? hb - d.nh : hb - d.nh - d.nkv;
        float* row = (is_k ? a.kc : a.vc) + (((size_t)l * d.nkv + g) * d.cap + pos) * d.kvs;
        pub_float(pub, 4 * k, row + i, a0, lane);
        pub_float(pub, 4 * k + 1, row + i + d.half, a1, lane);
      } else {
        pub_none(pub, 4 * k, lane);
        pub_none(pub, 4 * k + 1, lane);
      }
      pub_word(pub, 4 * k + 2, a.mb_qkv + r0, a0, gen, lane);
      pub_word(pub, 4 * k + 3, a.mb_qkv + r1, a1, gen, lane);
    });
  }
  pub_flush(pub, 4 * cnt);
  return true;
}

// ------------------------------------------------------------ attention

// Split-context attention for one (kv head, chunk, query head) item
// (model.rs:471-497): the chunk's softmax partials of query head j,
// m = max score, l = sum exp(score - m), acc = sum exp(score - m) v.
//  1. scores of every position of the chunk into LDS;
//  2. one wave: m, exp in place, l (lane-strided partials, wave tree);
//  3. exp-weighted V rows: position group (w, pl) chains positions
//     t0 + pv*w + pl + NCW*pv*k (k ascending); the groups of a wave are
//     folded by an xor butterfly over pl, then the waves summed in order.
// Every order above depends on (pos, head_dim) only.
// GROUPED = false: one query head per item (items (kv head, chunk, query
// head); the decode spreads them over the most workgroups). GROUPED = true:
// the group's query heads in one item (items (kv head, chunk); the batched
// path, whose rows bring workgroups enough, reads each K/V row once per item
// instead of once per head). The heads of a GQA group share K/V rows but
// nothing else, so both give each head the same arithmetic, bit for bit.
// AW0: the first attention wave (the persistent kernel's waves 0..NPOLL-1
// poll while the attention waves load; a workgroup of the NCW attention
// waves alone passes 0). NPW: the waves that poll q/k/v and publish the
// partials. KU, VU: the loads in flight. None of these changes the
// arithmetic.
// FillFn: where q/k/v come from. NoFill polls the tagged words of the QKV
// phase; otherwise fill(g, qs, kn, vn) writes kv group g's query rows, k and
// v into LDS itself (all threads call it; it ends with a barrier).
struct NoFill {};
template <bool GROUPED = false, uint32_t AW0 = NPOLL, uint32_t NPW = NPOLL, uint32_t KU = KU_DEF,
          uint32_t VU = VU_DEF, class FillFn = NoFill>
__device__ __forceinline__ bool phase_attn(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                           uint32_t wg, uint32_t G, const Lds& s,
                                           const FillFn& fill = FillFn()) {
  const Dims d = shape_dims(a.d);
  const uint32_t nch = attn_nchunks(pos), CH = attn_chunk(pos);
  const uint32_t n_items = GROUPED ? d.nkv * nch : attn_items(d, pos);
  const uint32_t gen_in = gen_of(d, tick, l, PH_QKV);
  const uint32_t gen_out = gen_of(d, tick, l, PH_ATTN);
  constexpr uint32_t MH = GROUPED ? MAX_GROUP : 1;  // query heads per item, at most
  const uint32_t hd = d.hd, grp = d.group, hs = hd + 2;
  const uint32_t NH1 = GROUPED ? grp : 1;  // query heads per item
  const AttGeo ge = att_geo(hd);
  float* qs = s.scr;                      // [MAX_GROUP*hd] (rows >= grp: don't care)
  float* kn = qs + MAX_GROUP * hd;        // [hd]
  float* vn = kn + hd;                    // [hd]
  float* ml = vn + hd;                    // [2*MAX_GROUP]
  float* sc = ml + 2 * MAX_GROUP;         // [MAX_GROUP][CH]
  float* wp = sc + MAX_GROUP * CH;        // [NCW][grp][hd]
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t ps = lane / ge.lps, sub = lane % ge.lps;
  const uint32_t pl = lane / ge.lv, dl = lane % ge.lv;
  const uint32_t sstep = NCW * ge.pw, vstep = NCW * ge.pv;
  // pollers and loaders only meet the barriers
  const bool att = wave >= AW0 && wave < AW0 + NCW;
  const uint32_t aw = att ? wave - AW0 : 0;  // attention wave
  const uint32_t tw = aw * ge.pw + ps;  // this lane's position offset in a score pass
  const uint32_t vw = aw * ge.pv + pl;  // ... and in a value step
  // One query head per item: the items of one (kv head, chunk) read the same
  // K/V rows. With at least NXCD such pairs they take slots NXCD apart --
  // workgroups on one XCD -- so the rows are fetched into one L2 rather than
  // one per head: slot NXCD * (grp * b + j0) + x is pair gc = NXCD * b + x,
  // query head j0, and slots past the last pair are empty (360M shape, 4096
  // tokens: 1.8 % faster, K/V fetched once instead of three times). Fewer
  // pairs take consecutive slots (slot = gc * grp + j0), as do all in the
  // staged-only kernel, whose decode the placement made 1 % slower.
  const uint32_t ngc = GROUPED ? n_items : d.nkv * nch;
  const bool by_xcd = !GROUPED && !STAGED_ONLY && ngc >= NXCD;
  const uint32_t n_slots = by_xcd ? NXCD * grp * ((ngc + NXCD - 1) / NXCD) : n_items;
  for (uint32_t slot = wg; slot < n_slots; slot += G) {
    uint32_t gc = slot, j0 = 0;
    if (by_xcd) {
      const uint32_t x = slot % NXCD, b = slot / NXCD;
      j0 = b % grp;
      gc = (b / grp) * NXCD + x;
      if (gc >= ngc) continue;
    } else if (!GROUPED) {
      gc = slot / grp;
      j0 = slot - gc * grp;
    }
    const uint32_t g = gc / nch, c = gc - g * nch;
    const uint32_t t0 = c * CH;
    const uint32_t t1 = min(t0 + CH, pos + 1);
    const float* kb = a.kc + ((size_t)l * d.nkv + g) * d.cap * d.kvs + sub * 16;
    const float* vb = a.vc + ((size_t)l * d.nkv + g) * d.cap * d.kvs + dl * 4;
    // The chunk's K rows of the first KU score passes and V rows of the
    // first VU value steps (a whole 128-position chunk at head_dim 64) are
    // requested before waiting for this token's q/k/v, all in one straight
    // run, so no load of the history sits on the critical path; later
    // passes and steps keep KU / VU in flight. Rows at or past pos are
    // clamped to row pos - 1 and never used (row pos comes from the poll):
    // a row is never read before the token that writes it, so no XCD's
    // cache can hold a copy older than its agent-scope store.
    float4 kr[KU][4], vr[VU];
    if (att && pos > 0) {
#pragma unroll
      for (uint32_t u = 0; u < KU; ++u) {
        const float* r = kb + (size_t)min(t0 + tw + u * sstep, pos - 1) * d.kvs;
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) kr[u][i] = ldg4(r + 4 * i);
      }
#pragma unroll
      for (uint32_t u = 0; u < VU; ++u)
        vr[u] = ldg4(vb + (size_t)min(t0 + vw + u * vstep, pos - 1) * d.kvs);
    }
    bool got;
    if constexpr (std::is_same<FillFn, NoFill>::value)
      got = poll_gather<GROUPED ? 8 / NPW : 1, 1, 1>(
          gather_vec(a.mb_qkv + (size_t)(g * grp + j0) * hd, NH1 * hd, gen_in, qs),
          gather_vec(a.mb_qkv + d.q + g * hd, hd, gen_in, kn),
          gather_vec(a.mb_qkv + d.q + d.kv + g * hd, hd, gen_in, vn), NPW, a.st, s.ctl);
    else
      got = fill(g, qs, kn, vn);
    if (!got) return false;
    // 1. scores, KU passes per round (pass u of a round uses kr[u], then
    // requests the pass KU later into it)
    for (uint32_t pb0 = t0; att && pb0 < t1; pb0 += KU * sstep) {
#pragma unroll
      for (uint32_t u = 0; u < KU; ++u) {
        const uint32_t ts = pb0 + u * sstep + tw;
        const bool live = ts < t1;
        if (ts == pos) {
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) kr[u][i] = lds4(kn + sub * 16 + 4 * i);
        }
        const bool masked = live && a.mask && ts < pos &&
                            ((ldg_u32(a.mask + (ts >> 5)) >> (ts & 31)) & 1u);
        // One head at a time keeps the live registers to this lane's K piece.
#pragma unroll 1
        for (uint32_t j = 0; j < NH1; ++j) {
          float acc = 0.0f;
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) {
            const float4 qq = lds4(qs + j * hd + sub * 16 + 4 * i);
            acc = fmaf(qq.x, kr[u][i].x, acc);
            acc = fmaf(qq.y, kr[u][i].y, acc);
            acc = fmaf(qq.z, kr[u][i].z, acc);
            acc = fmaf(qq.w, kr[u][i].w, acc);
          }
          const float v = group_sum(acc, ge.lps);
          if (live && sub == 0) lds_st(sc + j * CH + (ts - t0), masked ? -INFINITY : v * d.scale);
        }
        const uint32_t tn = ts + KU * sstep;
        if (tn < t1 && tn < pos) {
          const float* r = kb + (size_t)tn * d.kvs;
#pragma unroll
          for (uint32_t i = 0; i < 4; ++i) kr[u][i] = ldg4(r + 4 * i);
        }
      }
    }
    __syncthreads();
    // 2. softmax statistics, one attention wave per query head
    const uint32_t n = t1 - t0;
    if (att && aw < NH1) {
      float* sh = sc + aw * CH;
      float m = -INFINITY;
      for (uint32_t i = lane; i < n; i += WAVE) m = fmaxf(m, lds_ld(sh + i));
      m = wave_max(m);
      float ls = 0.0f;
      for (uint32_t i = lane; i < n; i += WAVE) {
        const float e = (m == -INFINITY) ? 0.0f : expf(lds_ld(sh + i) - m);
        lds_st(sh + i, e);
        ls += e;
      }
      ls = wave_sum(ls);
      if (lane == 0) {
        lds_st(ml + 2 * aw, m);
        lds_st(ml + 2 * aw + 1, ls);
      }
    }
    __syncthreads();
    // 3. exp-weighted V rows: positions t0 + vw + k*vstep, k = 0, 1, ...
    float4 acc[MH];
#pragma unroll
    for (uint32_t j = 0; j < MH; ++j) acc[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const uint32_t nk = att && t0 + vw < t1 ? (t1 - t0 - vw + vstep - 1) / vstep : 0;
    for (uint32_t k0 = 0; k0 < nk; k0 += VU) {
#pragma unroll
      for (uint32_t u = 0; u < VU; ++u) {
        const uint32_t k = k0 + u;
        if (k < nk) {
          const uint32_t t = t0 + vw + k * vstep;
          const float4 v = (t == pos) ? lds4(vn + dl * 4) : vr[u];
          const uint32_t tf = t + VU * vstep;
          if (k + VU < nk && tf < pos) vr[u] = ldg4(vb + (size_t)tf * d.kvs);
#pragma unroll
          for (uint32_t j = 0; j < MH; ++j) {
            if (j >= NH1) break;
            const float p = lds_ld(sc + j * CH + (t - t0));
            acc[j].x = fmaf(p, v.x, acc[j].x);
            acc[j].y = fmaf(p, v.y, acc[j].y);
            acc[j].z = fmaf(p, v.z, acc[j].z);
            acc[j].w = fmaf(p, v.w, acc[j].w);
          }
        }
      }
    }
    // The wave's position groups (lanes lv apart) in a butterfly, then one
    // partial per wave.
    for (uint32_t o = ge.lv; o < WAVE; o <<= 1) {
#pragma unroll
      for (uint32_t j = 0; j < MH; ++j) {
        if (j >= NH1) break;
        acc[j].x += __shfl_xor(acc[j].x, o);
        acc[j].y += __shfl_xor(acc[j].y, o);
        acc[j].z += __shfl_xor(acc[j].z, o);
        acc[j].w += __shfl_xor(acc[j].w, o);
      }
    }
#pragma unroll
    for (uint32_t j = 0; j < MH; ++j)
      if (j < NH1 && att && pl == 0) {
        float* dst = wp + (aw * NH1 + j) * hd + dl * 4;
        lds_st(dst + 0, acc[j].x);
        lds_st(dst + 1, acc[j].y);
        lds_st(dst + 2, acc[j].z);
        lds_st(dst + 3, acc[j].w);
      }
    __syncthreads();
    for (uint32_t u = threadIdx.x; threadIdx.x < NPW * WAVE && u < NH1 * hd; u += NPW * WAVE) {
      const uint32_t j = u / hd, dd = u - j * hd;
      float pw[NCW];
#pragma unroll
      for (uint32_t w = 0; w < NCW; ++w) pw[w] = lds_ld(wp + (w * NH1 + j) * hd + dd);
      float A = 0.0f;
#pragma unroll
      for (uint32_t w = 0; w < NCW; ++w) A += pw[w];
      const uint32_t hh = g * grp + j0 + j;
      u64* out = a.mb_part + ((size_t)hh * MAX_ACHUNKS + c) * hs;
      mb_put(out + 2 + dd, A, gen_out);
      if (dd == 0) {
        mb_put(out + 0, lds_ld(ml + 2 * j), gen_out);
        mb_put(out + 1, lds_ld(ml + 2 * j + 1), gen_out);
      }
    }
  }
  return true;
}

// Combine the chunk partials of one head (in chunk order) into its output:
// att[d] = sum_c acc_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M).
// ld(i): float i of the head's partials [nch][hs] (m, l, acc[hd]).
// combine_scales: the chunks' weights sc[c] = exp(m_c - M) and their
// weighted total l; combine_value: one output dim. Together they are
// combine_with.
template <class LD>
__device__ __forceinline__ float combine_scales(LD ld, uint32_t nch, uint32_t hs, float* sc) {
  if (nch == 1) return ld(1) * 1.0f;  // one chunk: its own max, weight exp(0) = 1
  float M = -INFINITY;
  for (uint32_t c = 0; c < nch; ++c) M = fmaxf(M, ld(c * hs));
  float Ls = 0.0f;
  for (uint32_t c = 0; c < nch; ++c) {
    const float mc = ld(c * hs);
    sc[c] = (mc == -INFINITY) ? 0.0f : expf(mc - M);
    Ls = Ls + ld(c * hs + 1) * sc[c];
  }
  return Ls;
}
template <class LD>
__device__ __forceinline__ float combine_value(LD ld, uint32_t nch, uint32_t hs, uint32_t dd,
                                               const float* sc, float Ls) {
  if (nch == 1) return (ld(2 + dd) * 1.0f) / Ls;
  float A = 0.0f;
  for (uint32_t c = 0; c < nch; ++c) A = A + ld(c * hs + 2 + dd) * sc[c];
  return A / Ls;
}
template <class LD>
__device__ __forceinline__ float combine_with(LD ld, uint32_t nch, uint32_t hs, uint32_t dd) {
  float sc[MAX_ACHUNKS];
  const float Ls = combine_scales(ld, nch, hs, sc);
  return combine_value(ld, nch, hs, dd, sc, Ls);
}
__device__ __forceinline__ float combine_one(const float* part, uint32_t nch, uint32_t hs,
                                             uint32_t dd) {
  return combine_with([&](uint32_t i) { return lds_ld(part + i); }, nch, hs, dd);
}

// Separate combine (used when the partials of all heads do not fit the O
// phase's LDS budget): item = one query head.
__device__ __forceinline__ bool phase_comb(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                           uint32_t wg, uint32_t G, const Lds& s) {
  const Dims d = shape_dims(a.d);
  if (comb_inline(d, pos)) return true;
  const uint32_t nch = attn_nchunks(pos), hs = d.hd + 2;
  const uint32_t gen_in = gen_of(d, tick, l, PH_ATTN), gen_out = gen_of(d, tick, l, PH_COMB);
  for (uint32_t hh = wg; hh < d.nh; hh += G) {
    if (!poll_gather<4>(gather_vec(a.mb_part + (size_t)hh * MAX_ACHUNKS * hs, nch * hs, gen_in, s.scr),
                     NPOLL, a.st, s.ctl))
      return false;
    for (uint32_t dd = threadIdx.x; dd < d.hd; dd += BLOCK)
      mb_put(a.mb_att + hh * d.hd + dd, combine_one(s.scr, nch, hs, dd), gen_out);
  }
  return true;
}

// ------------------------------------------------------------ O projection

// x_o = x + Wo . att (model.rs:498-499), with the attention combine done
// after the poll when it fits.
__device__ __forceinline__ bool phase_o(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                        uint32_t token, uint32_t wg, uint32_t G, const Lds& s,
                                        const Stager& sg) {
  const Dims d = shape_dims(a.d);
  const uint32_t nch = attn_nchunks(pos), hs = d.hd + 2;
  const bool inl = comb_inline(d, pos);
  const uint32_t R = own_count(d, IK_O, wg, G);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  float* part = s.scr;
  float* xres = s.scr + (inl ? d.nh * nch * hs : 0);
  // A workgroup without O rows only meets the barriers (its loaders' work).
  const Gather ga =
      R == 0 ? no_gather()
      : inl  ? gather_strided(a.mb_part, nch * hs, d.nh, MAX_ACHUNKS * hs, gen_of(d, tick, l, PH_ATTN),
                              part)
             : gather_vec(a.mb_att, d.q, gen_of(d, tick, l, PH_COMB), s.vec);
  const Gather gr = (l > 0 && R > 0)
                        ? gather_vec(rep_of(a, a.mb_xd, wg) + own_item(d, IK_O, wg, G, 0), R, gen_of(d, tick, l - 1, PH_D), xres)
                        : no_gather();
  // Layer 0's residual is the embedding row: its words are loaded before the
  // wait (pollers, one word per thread).
  float emb = 0.0f;
  if (l == 0 && threadIdx.x < R) emb = ldg(a.embed + (size_t)token * d.h + own_item(d, IK_O, wg, G, threadIdx.x));
  Preload P;
  const Pub pub = pub_for(sg.on, s);
  // The QKV rows are used: the next layer's are requested -- after the
  // combine's barrier below, not at the poll's end as in the other phases,
  // where no barrier follows: here every wave would wait at that barrier
  // for the loaders to finish issuing (1.3 us per layer at 135M).
  LoadOp op = no_load();
  if (staged(sg, IK_O)) op.wait = sg.wait[IK_O];
  {
    const MvWaves m0 = mv_waves(sg, wave, a, IK_O, wg, G);
    if (!(STAGED_ONLY || sg.on) && m0.n == NCW && wave >= NWA) prefetch_first(a, IK_O, l, wg, G, s, wave - NWA, lane);
  }
  if (!poll_gather<4, 1>(ga, gr, NWA, a.st, s.ctl, mv_hook(sg, op, P, IK_O))) return false;
  if (l == 0 && threadIdx.x < R) lds_st(xres + threadIdx.x, emb);
  if (inl && R > 0)
    for (uint32_t u = threadIdx.x; u < d.q && threadIdx.x < NWA * WAVE; u += NWA * WAVE) {
      const uint32_t hh = u / d.hd, dd = u - hh * d.hd;
      lds_st(s.vec + u, combine_one(part + hh * nch * hs, nch, hs, dd));
    }
  __syncthreads();
  if (sg.on && sg.loader && staged(sg, IK_QKV)) stage_issue(sg, IK_QKV, l + 1 < d.L ? l + 1 : 0);
  if (STAGED_ONLY ? (wave >= NPOLL && wave < NWA) : mv_waves(sg, wave, a, IK_O, wg, G).on) {
    const MvWaves mw = mv_waves(sg, wave, a, IK_O, wg, G);
    const uint32_t gen = gen_of(d, tick, l, PH_O);
    items_dot(a, IK_O, mw, l, sg, P, s.vec, wg, G, lane, [&](uint32_t k, float y, float) {
      pub_word_rep(pub, k, a.mb_xo + own_item(d, IK_O, wg, G, k), lds_ld(xres + k) + y, gen, a.rep_words, lane);
    });
  }
  pub_flush(pub, R, a.rep_words);
  return true;
}

// ------------------------------------------------------------ MLP

// rmsnorm -> g = act(Wg.x) * (Wu.x) (model.rs:502-509).
__device__ __forceinline__ bool phase_gu(const Args& a, uint32_t l, uint32_t tick, uint32_t wg,
                                         uint32_t G, const Lds& s, const Stager& sg) {
  const Dims d = shape_dims(a.d);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  Preload P;
  const Pub pub = pub_for(sg.on, s);
  LoadOp op = no_load();
  if (staged(sg, IK_O)) {
    op.issue = IK_O;
    op.layer = l + 1 < d.L ? l + 1 : 0;
  }
  if (staged(sg, IK_GU)) op.wait = sg.wait[IK_GU];
  {
    const MvWaves m0 = mv_waves(sg, wave, a, IK_GU, wg, G);
    if (!(STAGED_ONLY || sg.on) && m0.n == NCW && wave >= NWA) prefetch_first(a, IK_GU, l, wg, G, s, wave - NWA, lane);
  }
  if (!poll_gather<PW_H>(gather_vec(rep_of(a, a.mb_xo, wg), d.h, gen_of(d, tick, l, PH_O), s.vec), NWA, a.st, s.ctl,
                      mv_hook(sg, op, P, IK_GU)))
    return false;
  if (STAGED_ONLY ? (wave >= NPOLL && wave < NWA) : mv_waves(sg, wave, a, IK_GU, wg, G).on) {
    const MvWaves mw = mv_waves(sg, wave, a, IK_GU, wg, G);
    const float inv = rms_inv(s.vec, d.h, d.eps, lane);
    const uint32_t gen = gen_of(d, tick, l, PH_GU);
    items_dot(a, IK_GU, mw, l, sg, P, s.vec, wg, G, lane,
              [&](uint32_t k, float gate, float up) {
                pub_word_rep(pub, k, a.mb_g + item_of(d.ff, wg, G, k), act_fn(gate * inv, d.act) * (up * inv), gen, a.rep_words, lane);
              });
  }
  pub_flush(pub, rows_owned(d.ff, wg, G), a.rep_words);
  return true;
}

// x_d = x_o + Wd . g (model.rs:510-511).
__device__ __forceinline__ bool phase_d(const Args& a, uint32_t l, uint32_t tick, uint32_t wg,
                                        uint32_t G, const Lds& s, const Stager& sg) {
  const Dims d = shape_dims(a.d);
  const uint32_t R = rows_owned(d.h, wg, G);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const Gather gr = R > 0 ? gather_vec(rep_of(a, a.mb_xo, wg) + item_of(d.h, wg, G, 0), R, gen_of(d, tick, l, PH_O), s.scr)
                          : no_gather();
  Preload P;
  const Pub pub = pub_for(sg.on, s);
  LoadOp op = no_load();
  if (staged(sg, IK_GU)) {
    op.issue = IK_GU;
    op.layer = l + 1 < d.L ? l + 1 : 0;
  }
  if (staged(sg, IK_D)) op.wait = sg.wait[IK_D];
  {
    const MvWaves m0 = mv_waves(sg, wave, a, IK_D, wg, G);
    if (!(STAGED_ONLY || sg.on) && m0.n == NCW && wave >= NWA) prefetch_first(a, IK_D, l, wg, G, s, wave - NWA, lane);
  }
  if (!poll_gather<PW_F, 1>(gather_vec(rep_of(a, a.mb_g, wg), d.ff, gen_of(d, tick, l, PH_GU), s.vec), gr, NWA,
                          a.st, s.ctl, mv_hook(sg, op, P, IK_D)))
    return false;
  if (STAGED_ONLY ? (wave >= NPOLL && wave < NWA) : mv_waves(sg, wave, a, IK_D, wg, G).on) {
    const MvWaves mw = mv_waves(sg, wave, a, IK_D, wg, G);
    const uint32_t gen = gen_of(d, tick, l, PH_D);
    items_dot(a, IK_D, mw, l, sg, P, s.vec, wg, G, lane, [&](uint32_t k, float y, float) {
      pub_word_rep(pub, k, a.mb_xd + item_of(d.h, wg, G, k), lds_ld(s.scr + k) + y, gen, a.rep_words, lane);
    });
  }
  pub_flush(pub, R, a.rep_words);
  return true;
}

// ------------------------------------------------------------ lm_head

// argmax order: non-NaN beats missing, larger beats smaller, then the lower
// index wins (sampler.rs:24-40). A total order, so any tree gives one answer.
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  if (i == NO_INDEX) return false;
  if (bi == NO_INDEX) return true;
  return v > bv || (v == bv && i < bi);
}

constexpr int LMF = 9;  // chunks of a lane's lm_head segment held in registers (h <= 576 in one go)

// The final RMSNorm weight, kept in LDS for the kernel's lifetime (the
// lm_head may be the tied embedding, so it cannot be folded into the rows).
__device__ __forceinline__ void lm_prime(const Args& a, const Lds& s) {
  const uint32_t h = shape_dims(a.d).h;
  for (uint32_t i = threadIdx.x; i < h && threadIdx.x < NPOLL * WAVE; i += NPOLL * WAVE)
    lds_st(s.vec2 + h + i, ldg(a.norm + i));
  __syncthreads();
}

// rmsnorm(final) -> logits = H . x (model.rs:515-519), plus each vocabulary
// chunk's (max, argmax) for the sampler. The workgroup owns chunks
// c = wg + G*k; every wave computes quad passes of four rows, with the next
// four rows in flight. logit = inv * (H . (x * w_norm)).
__device__ __forceinline__ bool phase_lm(const Args& a, uint32_t tick, uint32_t wg, uint32_t G,
                                         const Lds& s, const Stager& sg) {
  const Dims d = shape_dims(a.d);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < d.nvc ? (d.nvc - wg + G - 1) / G : 0;
  const uint32_t nrows = nown * VCHUNK;  // local rows r -> chunk r / VCHUNK
  float* lg = s.scr;                     // [nrows] logits of this workgroup
  float* xs = s.vec2;                    // x * w_norm
  const float* nrm = s.vec2 + d.h;       // final norm weight (lm_prime)
  auto vocab_row = [&](uint32_t r) { return (wg + G * (r / VCHUNK)) * VCHUNK + r % VCHUNK; };
  const uint32_t sgm = qseg(lane);
  SegT<LMF> A, B;
  // The loader waves only meet the barriers where they stage rows; where
  // nothing is staged every wave streams lm_head rows.
  const uint32_t nlm = (STAGED_ONLY || sg.on) ? NWA : NWAVES;
  const bool lmw = wave < nlm;
  // Quad q: local rows 4q .. 4q+3, this lane's 4q + qrow(lane).
  auto live = [&](uint32_t q) {
    const uint32_t rr = 4 * q + qrow(lane);
    return rr < nrows && vocab_row(rr) < d.V;
  };
  // Rows past the vocabulary (or past the workgroup's rows) are clamped to
  // the last row and computed but never used, so every load is issued
  // unconditionally (seg_load_in) and counted exactly.
  auto row_of = [&](uint32_t q) {
    return a.head + (size_t)min(vocab_row(4 * q + qrow(lane)), d.V - 1) * d.h;
  };
  auto first = [&](SegT<LMF>& r, uint32_t q) {
    if (64u * LMF <= d.h)
      seg_load_in(r, row_of(q), sgm, 0);
    else
      seg_load(r, row_of(q), d.h, sgm, 0);
  };
  if (lmw) first(A, wave);
  if (!poll_gather<5>(gather_vec(rep_of(a, a.mb_xd, wg), d.h, gen_of(d, tick, d.L - 1, PH_D), s.vec), NPOLL, a.st,
                      s.ctl))
    return false;
  for (uint32_t i = threadIdx.x; i < d.h; i += BLOCK) lds_st(xs + i, lds_ld(s.vec + i) * lds_ld(nrm + i));
  __syncthreads();
  const float inv = rms_inv(s.vec, d.h, d.eps, lane);
  const uint32_t gen = gen_lm(d, tick);
  for (uint32_t q = wave; lmw && 4 * q < nrows; q += nlm) {
    first(B, q + nlm);
    const bool lv = live(q);
    const float acc = seg_tail(A, row_of(q), xs, d.h, sgm);
    const float y = inv * group_sum(acc, 16);
    if (lv && sgm == 0) {
      const uint32_t rr = 4 * q + qrow(lane);
      lds_st(lg + rr, y);
      mb_put(a.mb_logit + vocab_row(rr), y, gen);
    }
    A = B;
  }
  __syncthreads();
  // Chunk (max, argmax): one wave per chunk, one lane per row.
  for (uint32_t k = wave; lmw && k < nown; k += nlm) {
    const uint32_t c = wg + G * k;
    const uint32_t v = c * VCHUNK + lane;
    float bv = -INFINITY;
    uint32_t bi = NO_INDEX;
    if (v < d.V) {
      const float y = lds_ld(lg + k * VCHUNK + lane);
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
    if (lane == 0) {
      mb_put(a.mb_vmax + c, bv, gen);
      mb_put(a.mb_varg + c, __uint_as_float(bi), gen);
    }
  }
  return true;
}

// ------------------------------------------------------------ sampler

// Global (max, argmax) over the chunk partials already in LDS.
__device__ __forceinline__ void global_argmax(const float* vmx, const float* varg, uint32_t nvc, float* red,
                              float* bv_out, uint32_t* bi_out) {
  float bv = -INFINITY;
  uint32_t bi = NO_INDEX;
  for (uint32_t c = threadIdx.x; c < nvc; c += BLOCK) {
    const float v = vmx[c];
    const uint32_t i = __float_as_uint(varg[c]);
    if (better(v, i, bv, bi)) { bv = v; bi = i; }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(bv, o);
    const uint32_t i2 = __shfl_xor(bi, o);
    if (better(v2, i2, bv, bi)) { bv = v2; bi = i2; }
  }
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  __syncthreads();
  if (lane == 0) {
    red[wave] = bv;
    reinterpret_cast<uint32_t*>(red)[NWAVES + wave] = bi;
  }
  __syncthreads();
  float cv = -INFINITY;
  uint32_t ci = NO_INDEX;
  for (uint32_t w = 0; w < NWAVES; ++w) {
    const float wv = red[w];
    const uint32_t wi = reinterpret_cast<const uint32_t*>(red)[NWAVES + w];
    if (better(wv, wi, cv, ci)) { cv = wv; ci = wi; }
  }
  __syncthreads();
  *bv_out = cv;
  *bi_out = ci;
}

__device__ __forceinline__ float unit_f32(uint32_t word) {
  return (float)(word >> 8) * (1.0f / 16777216.0f);
}

// ------------------------------------------------------------ exact sampler
//
// sample_token (sampler.rs:78-109) for T > 0 with the reference's
// arithmetic: p_v = exp(l_v/T - m) (exact.h's expf), the sequential float
// total of the p_v, inv = 1/total, q_v = p_v * inv, and the first v with
// r < (the sequential float sum of q_0..q_v), else the last v with q_v > 0.
// Both sequential sums are formed as exact.h describes, in stages that every
// participating workgroup runs (G of them, workgroup wg owning the chunks
// c = wg + G*k):
//   A   the chunk maxima give m; each owner forms its chunks' p_v (kept in
//       LDS where they fit) and publishes them and each chunk's float sum;
//   A2  every workgroup reads all chunk sums and forms the same approximate
//       prefix; owners publish each chunk's total in units of the float
//       spacing the running sum is expected to have there (a summary word,
//       or "term by term" where a spacing change or a tie falls inside);
//       every workgroup fetches the terms of the chunks expected to change
//       spacing while the others finish;
//   W1  every workgroup reads the summaries and walks them (exact_walk):
//       the exact total, hence inv;
//   C   owners publish the summaries of q_v = p_v * inv in the spacing the
//       CDF is expected to have; the terms of the chunks around spacing
//       changes and around r are fetched;
//   W2  every workgroup walks those: the token.
// A summary is used only where the exact running sum is in the spacing it
// was formed for and stays there, so a wrong guess costs time, never bits;
// every workgroup computes the same token. With G = 1 one workgroup does it
// all (the batched sampler, the per-phase kernels).

constexpr double SAMP_MARGIN = 1.0 / 16384;  // relative slack of the spacing guesses
constexpr uint32_t OWN_MAX = 16;             // owned chunks whose p_v stay in LDS
constexpr uint32_t NEV_MAX = 36;             // term-by-term chunks fetched ahead of a walk
static_assert(NEV_MAX % NWA == 0, "fetch slots split evenly over the waves");
constexpr uint16_t NO_SLOT = 0xFFFF;

// The sampler's LDS (from s.scr): stage A's chunk maxima and logits, then
// the state that lives from stage A2 to the token.
struct SampLds {
  float* ownp;    // [OWN_MAX * VCHUNK] this workgroup's p_v
  float* vmx;     // stage A: [nvc] chunk maxima, [nvc] argmaxes, then the
  float* varg;    //   logits of the chunks in flight (overlapping A ..)
  float* chunk;
  float* A;       // [nvc] chunk sums of p
  float* pre;     // [nvc] approximate exclusive prefix of the chunk sums
  uint32_t* sw;   // [nvc] summary words of the walk in hand
  uint32_t* PI;   // [nvc] build_segments: the integer total of chunk c's segment from c on
  uint16_t* nxt;  // [nvc] the first segment start after chunk c
  uint32_t* nev;  // number of fetched chunks
  uint32_t* evc;  // [NEV_MAX] the chunk in each fetch slot
  uint16_t* slot; // [nvc] where chunk c's p_v are in evp (NO_SLOT: not fetched)
  float* evp;     // [NEV_MAX * VCHUNK] p_v of the fetched chunks
  uint32_t* pw;   // [NEV_MAX][2][VCHUNK] their terms' prefix words in grids E and E + 1 (pack_prefix)
  int32_t* slE;   // [NEV_MAX] the grid E each fetched chunk's prefix words are for
  double* dred;   // [NWAVES]
  uint32_t* res;  // [4]
};
// A and pre live in the matvec input region (s.vec, free from the lm_head
// to the next token's first gather) where they fit, else after the rest.
__host__ __device__ inline bool samp_ap_in_vec(uint32_t nvc, uint32_t lds_vec) { return 2 * nvc <= lds_vec; }
__host__ __device__ inline uint32_t samp_lds_floats(uint32_t nvc, uint32_t stage_a_chunks, uint32_t lds_vec) {
  const uint32_t a = OWN_MAX * VCHUNK + 2 * nvc + stage_a_chunks * VCHUNK;
  const uint32_t w = OWN_MAX * VCHUNK + 2 * nvc + 2 * ((nvc + 1) / 2) + 1 + NEV_MAX + 3 * NEV_MAX * VCHUNK +
                     NEV_MAX + 1 + 2 * NWAVES + 4 + (samp_ap_in_vec(nvc, lds_vec) ? 0 : 2 * nvc);
  return a > w ? a : w;
}
__device__ __forceinline__ SampLds samp_lds(const Lds& s, uint32_t nvc, uint32_t lds_vec) {
  SampLds L;
  float* b = s.scr;
  L.ownp = b;
  b += OWN_MAX * VCHUNK;
  // stage A: chunk maxima, argmaxes, then the logits of the chunks in flight
  L.vmx = b;
  L.varg = b + nvc;
  L.chunk = b + 2 * nvc;
  // from stage A2 on
  L.sw = reinterpret_cast<uint32_t*>(b);
  b += nvc;
  L.PI = reinterpret_cast<uint32_t*>(b);
  b += nvc;
  L.nxt = reinterpret_cast<uint16_t*>(b);
  b += (nvc + 1) / 2;
  L.nev = reinterpret_cast<uint32_t*>(b);
  b += 1;
  L.evc = reinterpret_cast<uint32_t*>(b);
  b += NEV_MAX;
  L.slot = reinterpret_cast<uint16_t*>(b);
  b += (nvc + 1) / 2;
  L.evp = b;
  b += NEV_MAX * VCHUNK;
  L.pw = reinterpret_cast<uint32_t*>(b);
  b += 2 * NEV_MAX * VCHUNK;
  L.slE = reinterpret_cast<int32_t*>(b);
  b += NEV_MAX;
  b += (uint32_t)((uintptr_t)b & 4u) ? 1 : 0;  // 8-byte alignment (s.scr is 16-byte aligned)
  L.dred = reinterpret_cast<double*>(b);
  b += 2 * NWAVES;
  L.res = reinterpret_cast<uint32_t*>(b);
  b += 4;
  float* ap = samp_ap_in_vec(nvc, lds_vec) ? s.vec : b;
  L.A = ap;
  L.pre = ap + nvc;
  return L;
}

// Sampler stage A (temperature > 0): the global max m from the chunk maxima
// (*m and the argmax *bi out; every workgroup forms the same), then, for
// this workgroup's chunks, every p_v with the reference's exp, kept in LDS
// where they fit and published, and each chunk's sum of them (any order:
// only the spacing guesses use it). Everything is published under the tag
// gsum, unique to one sampling event (a per-cache or per-workspace sequence
// number handed in by the host), so values an earlier sample left in the
// mailboxes never carry the tag a later stage waits for.
// CPW: chunks per polling/computing wave per round; PA: words per lane per
// poll round.
template <uint32_t CPW = 1, uint32_t PA = 2>
__device__ __forceinline__ bool sample_stage_a(const Args& a, uint32_t tick, uint32_t gsum, float T,
                                               uint32_t wg, uint32_t G, const Lds& s, float* m_out,
                                               uint32_t* bi_out) {
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u);
  const SampLds L = samp_lds(s, nvc, a.d.lds_vec);
  if (!poll_gather<2, 2>(gather_vec(a.mb_vmax, nvc, gl, L.vmx), gather_vec(a.mb_varg, nvc, gl, L.varg),
                         NWA, a.st, s.ctl))
    return false;
  float bv;
  uint32_t bi;
  global_argmax(L.vmx, L.varg, nvc, s.red, &bv, &bi);
  const float m = (bi == NO_INDEX) ? -INFINITY : bv / T;
  *m_out = m;
  *bi_out = bi;
  if (!isfinite(m)) return true;  // the reference falls back to argmax
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < nvc ? (nvc - wg + G - 1) / G : 0;
  for (uint32_t k0 = 0; k0 < nown; k0 += NWA * CPW) {
    const uint32_t nb = min(NWA * CPW, nown - k0);
    // chunks wg + G*(k0 + b), b < nb; the last one may be short
    const u64* src0 = a.mb_logit + (size_t)(wg + G * k0) * VCHUNK;
    const uint32_t clast = wg + G * (k0 + nb - 1);
    // a short last chunk is gathered separately so no slot past V is read
    const bool short_last = (clast + 1) * VCHUNK > d.V;
    const Gather ga = gather_strided(src0, VCHUNK, short_last ? nb - 1 : nb, G * VCHUNK, gl, L.chunk);
    const Gather gb = short_last ? gather_vec(a.mb_logit + (size_t)clast * VCHUNK,
                                              d.V - clast * VCHUNK, gl, L.chunk + (nb - 1) * VCHUNK)
                                 : no_gather();
    if (!poll_gather<PA, 1>(ga, gb, NWA, a.st, s.ctl)) return false;
    for (uint32_t b = wave; wave < NWA && b < nb; b += NWA) {
      const uint32_t c = wg + G * (k0 + b);
      const uint32_t v = c * VCHUNK + lane;
      const float e = (v < d.V) ? prob_term(L.chunk[b * VCHUNK + lane], T, m) : 0.0f;
      if (v < d.V) mb_put(a.mb_p + v, e, gsum);
      if (nown <= OWN_MAX) L.ownp[(k0 + b) * VCHUNK + lane] = e;
      const float S = wave_sum(e);
      if (lane == 0) mb_put(a.mb_vsum + c, S, gsum);
    }
    __syncthreads();
  }
  return true;
}

// This lane's words ptr[k] (k < N) once each carries `tag`; false (uniform
// over the wave) if the run was aborted meanwhile.
template <int N>
__device__ __forceinline__ bool load_tagged(const u64* const (&ptr)[N], uint32_t tag, float (&v)[N],
                                            DevState* st, WaitCtl* ctl) {
  uint32_t pend = 0;
  u64 w[N];
#pragma unroll
  for (int k = 0; k < N; ++k) w[k] = mb_load(ptr[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) {
    if ((uint32_t)(w[k] >> 32) == tag) v[k] = __uint_as_float((uint32_t)w[k]);
    else pend |= 1u << k;
  }
  for (uint32_t spins = 0; __any(pend != 0); ++spins) {
    if (spins >= SPIN_LIMIT) {
      st_coherent_u32(&st->abort, 1u);
      ctl->abort_seen = 1;
      return false;
    }
    if ((spins & 63) == 63 && ld_coherent_u32(&st->abort)) {
      ctl->abort_seen = 1;
      return false;
    }
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (pend & (1u << k)) {
        const u64 x = mb_load(ptr[k]);
        if ((uint32_t)(x >> 32) == tag) {
          v[k] = __uint_as_float((uint32_t)x);
          pend &= ~(1u << k);
        }
      }
  }
  return true;
}

// The block-wide approximate exclusive prefix of the chunk sums A (float
// partials in a fixed tree: a few roundings of 2^-24, far inside the
// guesses' margin), in pre. Thread t owns a contiguous run of chunks.
__device__ __forceinline__ void approx_prefix(const float* A, float* pre, uint32_t nvc, float* wred) {
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t cpt = (nvc + BLOCK - 1) / BLOCK;
  const uint32_t ca = min(threadIdx.x * cpt, nvc), cb = min(ca + cpt, nvc);
  float own = 0.0f;
  for (uint32_t c = ca; c < cb; ++c) own += A[c];
  const float incl = wave_scan_f32(own);
  __syncthreads();
  if (lane == WAVE - 1) wred[wave] = incl;
  __syncthreads();
  float p = incl - own;
  for (uint32_t w = 0; w < wave; ++w) p += wred[w];
  for (uint32_t c = ca; c < cb; ++c) {
    pre[c] = p;
    p += A[c];
  }
  __syncthreads();
}

// The spacing guess of chunk c for the terms x = p * scale: the grid its
// running sum is expected to start in, and whether a spacing change is
// expected inside it (then it goes term by term).
__device__ __forceinline__ int chunk_guess(const SampLds& L, uint32_t c, float scale, bool* change) {
  const double lo = (double)L.pre[c] * scale * (1.0 - SAMP_MARGIN);
  const double hi = ((double)L.pre[c] + (double)L.A[c]) * scale * (1.0 + SAMP_MARGIN);
  const int E = grid_of((float)lo);
  *change = E != grid_of((float)hi);
  return E;
}

// Owned chunks' summary words of x = p (FIND false) or p * inv, published
// to `dst` under gsum: one wave per chunk, a lane per term. own_in_lds: this
// kernel ran stage A with the same (wg, G), so the owned p_v are in LDS
// where they fit; else they are read back from the mailbox. Chunks starting
// past r (FIND) are not needed by a walk that finds r and are published as
// term-by-term without being formed.
template <bool FIND>
__device__ __forceinline__ bool publish_summaries(const Args& a, u64* dst, uint32_t gsum, float inv, float r,
                                                  uint32_t wg, uint32_t G, bool own_in_lds, const SampLds& L,
                                                  const Lds& s) {
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc, V = d.V;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < nvc ? (nvc - wg + G - 1) / G : 0;
  // The 135M kernel runs only at its full grid, where the owned p_v fit.
  const bool lds_p = STAGED_ONLY || (own_in_lds && nown <= OWN_MAX);
  // chunk k's summary word from its terms pk (one wave, a lane per term)
  auto one = [&](uint32_t k, float pk) {
    const uint32_t c = wg + G * k;
    bool change;
    const int E = chunk_guess(L, c, FIND ? inv : 1.0f, &change);
    const bool past = FIND && (double)L.pre[c] * inv * (1.0 - SAMP_MARGIN) > (double)r;
    uint32_t w = sum_word(E, SUM_EVENT);
    if (!change && !past) {
      const uint32_t v = c * VCHUNK + lane;
      const float x = v < V ? (FIND ? pk * inv : pk) : 0.0f;
      const GridTerm g = grid_term(x, E);
      const uint32_t tot = lane_u32(wave_scan_u32(g.big ? 0u : g.rho), 63);
      const bool flag = __ballot(g.big || g.tie) != 0;
      w = sum_word(E, flag ? SUM_EVENT : tot);
    }
    if (lane == 0) mb_put(dst + c, __uint_as_float(w), gsum);
  };
  bool ok = true;
  if (lds_p) {
    // from LDS: one chunk per wave at a time, the chunks spread over the waves
    for (uint32_t k = wave; wave < NWA && k < nown; k += NWA) one(k, L.ownp[k * VCHUNK + lane]);
  } else {
    constexpr uint32_t B = 4;  // chunks per wave in flight from the mailbox
    for (uint32_t k0 = wave * B; wave < NWA && k0 < nown; k0 += NWA * B) {
      float p[B];
      const u64* ptr[B];
#pragma unroll
      for (uint32_t e = 0; e < B; ++e) ptr[e] = a.mb_p + min((wg + G * min(k0 + e, nown - 1)) * VCHUNK + lane, V - 1);
      if (!load_tagged<B>(ptr, gsum, p, a.st, s.ctl)) {
        ok = false;
        break;
      }
#pragma unroll
      for (uint32_t e = 0; e < B; ++e)
        if (k0 + e < nown) one(k0 + e, p[e]);
    }
  }
  if (!ok && lane == 0) s.ctl->abort_seen = 1;
  __syncthreads();
  return s.ctl->abort_seen == 0;
}

// A chunk's terms in grid E, summarised per lane j in one word: bits 0-29
// the inclusive prefix sum of rho over lanes <= j, bit 30 whether term j
// rounds up (rho = a + 1, so the crossing test k + Pex + a is k + P - bit),
// bit 31 whether term j leaves the region by itself or is a tie. Lanes at
// or past n hold zero terms.
constexpr uint32_t PW_P = 0x3FFFFFFFu, PW_UP = 1u << 30, PW_BAD = 1u << 31;
__device__ __forceinline__ uint32_t pack_prefix(float x, int E) {
  const GridTerm g = grid_term(x, E);
  const uint32_t rho = g.big ? 0u : g.rho;
  const uint32_t P = wave_scan_u32(rho);
  return P | (!g.big && g.rho != g.a ? PW_UP : 0u) | (g.big || g.tie ? PW_BAD : 0u);
}

// The p_v of the chunks a walk is expected to sum term by term, fetched
// into LDS (at most NEV_MAX chunks; a walk reads any other from the
// mailbox). Round 0 (while the other workgroups finish their summaries):
// the chunks with a spacing change expected inside, and their neighbours,
// where a guess off by a little puts the change; FIND also the chunks
// around r. Round 1 (once the summary words are in L.sw): every chunk whose
// word says term by term and that round 0 did not fetch. The slot map
// L.slot says where each fetched chunk went.
template <bool FIND>
__device__ __forceinline__ bool fetch_events(const Args& a, uint32_t gsum, float inv, float r, uint32_t round,
                                             const SampLds& L, const Lds& s) {
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc, V = d.V;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t cpt = (nvc + BLOCK - 1) / BLOCK;
  const uint32_t ca = min(threadIdx.x * cpt, nvc), cb = min(ca + cpt, nvc);
  auto past = [&](uint32_t c) {
    return FIND && (double)L.pre[c] * inv * (1.0 - SAMP_MARGIN) > (double)r;
  };
  auto change = [&](uint32_t c) {
    bool ch;
    (void)chunk_guess(L, c, FIND ? inv : 1.0f, &ch);
    if (FIND) {
      const double lo = (double)L.pre[c] * inv, hi = ((double)L.pre[c] + (double)L.A[c]) * inv;
      ch = ch || (lo * (1.0 - SAMP_MARGIN) <= (double)r && hi * (1.0 + SAMP_MARGIN) >= (double)r);
    }
    return ch;
  };
  // Round 0: each chunk's change flag, formed once into L.sw (free until the
  // summary words arrive), read for the chunk and its neighbours.
  auto wanted = [&](uint32_t c) {
    if (past(c)) return false;
    if (round == 0) return L.sw[c] != 0 || (c > 0 && L.sw[c - 1] != 0) || (c + 1 < nvc && L.sw[c + 1] != 0);
    return L.slot[c] == NO_SLOT && sum_total(L.sw[c]) == SUM_EVENT;
  };
  if (round == 0) {
    for (uint32_t c = ca; c < cb; ++c) {
      L.slot[c] = NO_SLOT;
      L.sw[c] = change(c) ? 1u : 0u;
    }
    __syncthreads();
  }
  const uint32_t base_n = round == 0 ? 0u : *L.nev;
  uint32_t cnt = 0;
  for (uint32_t c = ca; c < cb; ++c) cnt += wanted(c) ? 1u : 0u;
  const uint32_t incl = wave_scan_u32(cnt);
  uint32_t* wtot = reinterpret_cast<uint32_t*>(L.dred);
  __syncthreads();
  if (lane == WAVE - 1) wtot[wave] = incl;
  __syncthreads();
  uint32_t pos = base_n + incl - cnt, total = 0;
  for (uint32_t w = 0; w < NWAVES; ++w) {
    if (w < wave) pos += wtot[w];
    total += wtot[w];
  }
  for (uint32_t c = ca; c < cb; ++c)
    if (wanted(c)) {
      if (pos < NEV_MAX) {
        L.slot[c] = (uint16_t)pos;
        L.evc[pos] = c;
      }
      ++pos;
    }
  const uint32_t n_after = min(base_n + total, NEV_MAX);
  __syncthreads();
  if (threadIdx.x == 0) *L.nev = n_after;
  // The fetch: slots base_n .. n_after-1, a lane per term, FB slots per wave
  // in flight (NWA * FB = NEV_MAX: one round).
  constexpr uint32_t FB = NEV_MAX / NWA;
  bool ok = true;
  const uint32_t s0 = base_n + wave * FB;
  if (wave < NWA && s0 < n_after) {
    const u64* ptr[FB];
    float t[FB];
#pragma unroll
    for (uint32_t e = 0; e < FB; ++e)
      ptr[e] = a.mb_p + min(L.evc[min(s0 + e, n_after - 1)] * VCHUNK + lane, V - 1);
    ok = load_tagged<FB>(ptr, gsum, t, a.st, s.ctl);
#pragma unroll
    for (uint32_t e = 0; e < FB; ++e) {
      const uint32_t sl = s0 + e;
      if (!ok || sl >= n_after) break;
      L.evp[sl * VCHUNK + lane] = t[e];
      // the terms' prefix words in the grid the chunk is expected to start
      // in and the next one, off the walk's path
      const uint32_t c = L.evc[sl];
      bool ch;
      const int E = chunk_guess(L, c, FIND ? inv : 1.0f, &ch);
      const float x = c * VCHUNK + lane < V ? (FIND ? t[e] * inv : t[e]) : 0.0f;
      L.pw[(2 * sl) * VCHUNK + lane] = pack_prefix(x, E);
      L.pw[(2 * sl + 1) * VCHUNK + lane] = pack_prefix(x, E + 1);
      if (lane == 0) L.slE[sl] = E;
    }
  }
  if (!ok && lane == 0) s.ctl->abort_seen = 1;
  __syncthreads();
  return s.ctl->abort_seen == 0;
}

// The terms of one chunk (n <= 64 of them, lane j the j-th, x), added to the
// exact running sum s one rounded step at a time, in parallel: with s in
// grid E, the steps before the first term that leaves the region (or is a
// tie) are an integer prefix sum; that term is one float addition; repeat.
// FIND: stops at the first term j with r < the sum after it (hit = j; 64 if
// none). Wave-uniform.
template <bool FIND>
__device__ __forceinline__ void chunk_exact(float x, uint32_t n, float r, float& s, uint32_t& hit,
                                            uint32_t jstart = 0) {
  const uint32_t lane = threadIdx.x % WAVE;
  hit = 64;
  int E = grid_of(s);
  GridTerm g = grid_term(x, E);
  // Where several terms leave the running sum's region at once, or the
  // terms add up to several times the sum (the first chunk, whose sum starts
  // at 0: a spacing change every doubling, and a tie is likely for a term
  // not far below the sum's spacing), one float addition per term is
  // cheaper than a restart per term. The terms are read into scalar
  // registers 16 at a time, ahead of their additions, so the chain of
  // additions waits on nothing else.
  const float rest = lane_f32(wave_scan_f32(lane >= jstart && lane < n ? x : 0.0f), 63);
  if (rest > 4.0f * s || __popcll(__ballot(lane >= jstart && lane < n && (g.big || g.tie))) >= 4) {
    // Past n (and past lane 63) the batch adds zeros, which leave s as it is.
    const float xm = lane < n ? x : 0.0f;
    for (uint32_t j0 = jstart; j0 < n; j0 += 16) {
      float t[16];
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) t[q] = j0 + q < WAVE ? lane_f32(xm, min(j0 + q, WAVE - 1)) : 0.0f;
      const float s0 = s;
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) s = s + t[q];
      if (FIND && r < s) {  // r falls in this batch: the same additions, checked one by one
        s = s0;
        for (uint32_t q = 0; q < 16; ++q) {
          s = s + t[q];
          if (r < s) {
            hit = j0 + q;
            return;
          }
        }
      }
    }
    return;
  }
  // Each round forms the terms in grid E and in the next grid E + 1 (where
  // the sum goes when it leaves E upwards), so a chunk whose sum changes
  // spacing once is done in one round.
  for (;;) {
    const uint32_t k = grid_units(s, E);
    const bool act = lane >= jstart && lane < n;
    const GridTerm h = grid_term(x, E + 1);
    const uint32_t rho = (act && !g.big) ? g.rho : 0u, aa = (act && !g.big) ? g.a : 0u;
    const uint32_t rho1 = (act && !h.big) ? h.rho : 0u;
    const uint32_t P = wave_scan_u32(rho), P1 = wave_scan_u32(rho1);
    const uint32_t Pex = P - rho;
    const bool bad = act && (g.big || g.tie || k + Pex + aa >= GRID_TOP);
    const uint32_t jb = first_lane(__ballot(bad));
    if (FIND) {
      const bool hh = act && lane < jb && r < __builtin_ldexpf((float)(k + P), E);
      const uint32_t jh = first_lane(__ballot(hh));
      if (jh < 64) {
        hit = jh;
        s = __builtin_ldexpf((float)(k + lane_u32(P, jh)), E);
        return;
      }
    }
    if (jb >= 64) {
      s = __builtin_ldexpf((float)(k + lane_u32(P, 63)), E);
      return;
    }
    s = __builtin_ldexpf((float)(k + lane_u32(Pex, jb)), E);
    s = s + lane_f32(x, jb);
    if (FIND && r < s) {
      hit = jb;
      return;
    }
    jstart = jb + 1;
    if (jstart >= n) return;
    const int E2 = grid_of(s);
    if (E2 == E + 1) {
      // the terms after jb in grid E + 1, from the same round
      const uint32_t k2 = grid_units(s, E2), base = lane_u32(P1, jb);
      const bool act2 = lane >= jstart && lane < n;
      const uint32_t Q = P1 - base, Qex = Q - rho1;
      const bool bad2 = act2 && (h.big || h.tie || k2 + Qex + (h.big ? 0u : h.a) >= GRID_TOP);
      const uint32_t jb2 = first_lane(__ballot(bad2));
      if (FIND) {
        const bool hh = act2 && lane < jb2 && r < __builtin_ldexpf((float)(k2 + Q), E2);
        const uint32_t jh = first_lane(__ballot(hh));
        if (jh < 64) {
          hit = jh;
          s = __builtin_ldexpf((float)(k2 + lane_u32(Q, jh)), E2);
          return;
        }
      }
      if (jb2 >= 64) {
        s = __builtin_ldexpf((float)(k2 + lane_u32(Q, 63)), E2);
        return;
      }
      s = __builtin_ldexpf((float)(k2 + lane_u32(Qex, jb2)), E2);
      s = s + lane_f32(x, jb2);
      if (FIND && r < s) {
        hit = jb2;
        return;
      }
      jstart = jb2 + 1;
      if (jstart >= n) return;
    }
    E = grid_of(s);
    g = grid_term(x, E);
  }
}

// The terms of a fetched chunk from lane j0 on, added to the running sum s
// with the chunk's prefix words in grid E (wE) and grid E + 1 (wE1): while s
// lies in one of those two grids, the terms up to the next that leaves it
// (or is a tie there) are one integer step and that term one float
// addition, as often as the chunk needs. Returns the lane from which
// chunk_exact must go on once s is in neither grid (64 when the chunk is
// done).
template <bool FIND>
__device__ __forceinline__ uint32_t chunk_words(uint32_t wE, uint32_t wE1, float x, uint32_t n, int E, float r,
                                                float& s, uint32_t& hit, uint32_t j0 = 0) {
  const uint32_t lane = threadIdx.x % WAVE;
  hit = 64;
  for (;;) {
    const int Ec = grid_of(s);
    if (Ec != E && Ec != E + 1) return j0;
    const uint32_t w = Ec == E ? wE : wE1;
    const uint32_t k = grid_units(s, Ec);
    const uint32_t P = w & PW_P;
    const uint32_t Q = P - (j0 ? lane_u32(P, j0 - 1) : 0u);  // from lane j0 on
    const bool act = lane >= j0 && lane < n;
    const bool bad = act && ((w & PW_BAD) || k + Q - ((w & PW_UP) ? 1u : 0u) >= GRID_TOP);
    const uint32_t jb = first_lane(__ballot(bad));
    if (FIND) {
      const uint32_t jh = first_lane(__ballot(act && lane < jb && r < __builtin_ldexpf((float)(k + Q), Ec)));
      if (jh < 64) {
        hit = jh;
        s = __builtin_ldexpf((float)(k + lane_u32(Q, jh)), Ec);
        return 64;
      }
    }
    if (jb >= 64) {  // lanes at or past n hold zero terms
      s = __builtin_ldexpf((float)(k + lane_u32(Q, 63)), Ec);
      return 64;
    }
    s = __builtin_ldexpf((float)(k + (jb > j0 ? lane_u32(Q, jb - 1) : 0u)), Ec);
    s = s + lane_f32(x, jb);
    if (FIND && r < s) {
      hit = jb;
      return 64;
    }
    j0 = jb + 1;
    if (j0 >= n) return 64;
  }
}

// Segments of the summary words in L.sw: a segment is a maximal run of
// usable chunks (an integer total) in one grid, and each term-by-term chunk
// is one of its own. L.PI gets the inclusive prefix of the usable totals, so
// a segment's total is a difference of two entries; L.nxt[c] the first
// segment start after c (nvc past the last). A walk at a segment's start
// whose running sum is in the segment's grid and stays there takes the whole
// segment as one integer step.
__device__ __forceinline__ void build_segments(const SampLds& L, uint32_t nvc) {
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t cpt = (nvc + BLOCK - 1) / BLOCK;
  const uint32_t ca = min(threadIdx.x * cpt, nvc), cb = min(ca + cpt, nvc);
  auto ev = [&](uint32_t c) { return sum_total(L.sw[c]) == SUM_EVENT; };
  auto start = [&](uint32_t c) {
    return c == 0 || ev(c) || ev(c - 1) || sum_grid(L.sw[c]) != sum_grid(L.sw[c - 1]);
  };
  uint32_t own = 0, first = nvc;
  for (uint32_t c = ca; c < cb; ++c) {
    own += ev(c) ? 0u : sum_total(L.sw[c]);
    if (first == nvc && start(c)) first = c;
  }
  // exclusive prefix of the totals over threads; suffix minimum of the
  // first starts over the following threads
  const uint32_t incl = wave_scan_u32(own);
  uint32_t later;  // first start in the following lanes and waves
  {
    uint32_t m = first;  // suffix minimum including this lane
#pragma unroll
    for (uint32_t o = 1; o < WAVE; o <<= 1) {
      const uint32_t y = __shfl_down(m, o);
      if (lane + o < WAVE) m = min(m, y);
    }
    later = __shfl_down(m, 1);
    if (lane == WAVE - 1) later = nvc;
    uint32_t* wsum = reinterpret_cast<uint32_t*>(L.dred);  // [NWAVES] totals, [NWAVES] minima
    __syncthreads();
    if (lane == WAVE - 1) wsum[wave] = incl;
    if (lane == 0) wsum[NWAVES + wave] = m;
    __syncthreads();
    uint32_t base = incl - own;
    for (uint32_t w = 0; w < wave; ++w) base += wsum[w];
    for (uint32_t w = wave + 1; w < NWAVES; ++w) later = min(later, wsum[NWAVES + w]);
    uint32_t run = base;
    for (uint32_t c = ca; c < cb; ++c) {
      run += ev(c) ? 0u : sum_total(L.sw[c]);
      L.PI[c] = run;
    }
    uint32_t nx = later;
    for (uint32_t c = cb; c-- > ca;) {
      L.nxt[c] = (uint16_t)nx;
      if (start(c)) nx = c;
    }
  }
  __syncthreads();
  // PI[c] becomes the total of c's segment from c on: PI[nxt - 1] - PI[c - 1]
  // (read by every thread before any is overwritten)
  constexpr uint32_t CPT_MAX = 4;  // chunks per thread: nvc <= 2048
  uint32_t rest[CPT_MAX];
#pragma unroll
  for (uint32_t q = 0; q < CPT_MAX; ++q) {
    const uint32_t c = ca + q;
    rest[q] = c < cb ? L.PI[L.nxt[c] - 1] - (c ? L.PI[c - 1] : 0u) : 0u;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t q = 0; q < CPT_MAX; ++q)
    if (ca + q < cb) L.PI[ca + q] = rest[q];
  __syncthreads();
}

// One chunk summed term by term at the running sum: from its fetch slot sc
// with the prefix words (the sum starting in the grid they were formed for
// or the next), else from the mailbox. FIND: *hit the lane where r falls.
template <bool FIND>
__device__ __forceinline__ bool walk_chunk(const Args& a, uint32_t gsum, float inv, float r, const SampLds& L,
                                           const Lds& s, uint32_t c, uint32_t sc, uint32_t V, float& sum,
                                           uint32_t& hit) {
  const uint32_t lane = threadIdx.x % WAVE;
  const uint32_t base = c * VCHUNK, n = min(VCHUNK, V - base);
  float p;
  uint32_t from = 0;  // the lane chunk_exact goes on from
  hit = 64;
  if (sc != NO_SLOT) {
    p = L.evp[sc * VCHUNK + lane];
    const uint32_t w0s = L.pw[(2 * sc) * VCHUNK + lane], w1s = L.pw[(2 * sc + 1) * VCHUNK + lane];
    const int Es = L.slE[sc], Eg = grid_of(sum);
    const float xf = lane < n ? (FIND ? p * inv : p) : 0.0f;
    if (Eg == Es || Eg == Es + 1) from = chunk_words<FIND>(w0s, w1s, xf, n, Es, r, sum, hit);
  } else {
    const u64* ptr[1] = {a.mb_p + base + min(lane, n - 1)};
    float t[1];
    if (!load_tagged<1>(ptr, gsum, t, a.st, s.ctl)) return false;
    p = t[0];
  }
  const float x = lane < n ? (FIND ? p * inv : p) : 0.0f;
  if (hit == 64 && from < n) chunk_exact<FIND>(x, n, r, sum, hit, from);
  return true;
}

// One walk over the summary words L.sw (wave 0; the block waits): the total
// of the terms (FIND false: *out = its bits) or the index sample_token
// returns (FIND true). The expected path visits the segment starts in order:
// a segment (its grid the running sum's, no crossing inside) is one integer
// step, a term-by-term chunk goes through walk_chunk. The path is read a
// window of 64 chunks at a time into registers (the starts as a ballot, each
// start's summary, segment total and fetch slot in a lane), so a step reads
// no LDS but the chunk's terms. Where a step does not hold (a spacing guess
// off, a segment whose total overflows the grid, r inside a segment) the
// walk goes on from that chunk chunk by chunk: windows of 64 summaries whose
// usable prefix is one integer sum, the first unusable chunk term by term.
template <bool FIND>
__device__ __forceinline__ bool exact_walk(const Args& a, uint32_t gsum, float inv, float r, const SampLds& L,
                                           const Lds& s, uint32_t* out) {
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc, V = d.V;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  if (wave == 0) {
    float sum = 0.0f;
    uint32_t found = NO_INDEX;
    bool ok = true;
    uint32_t c0 = nvc;  // where the chunk-by-chunk walk starts (nvc: not needed)
    for (uint32_t wb = 0; wb < nvc; wb += WAVE) {
      const uint32_t c = wb + lane;
      const bool in = c < nvc;
      const uint32_t vW = in ? L.sw[c] : 0u;
      const uint32_t vT = in ? L.PI[c] : 0u;
      const uint32_t vS = in ? L.slot[c] : NO_SLOT;
      unsigned long long starts = __ballot(in && (c == 0 || L.nxt[c - 1] == c));
      bool stop = false;
      while (starts) {
        const uint32_t j = first_lane(starts);
        starts &= starts - 1;
        const uint32_t cc = wb + j;
        const uint32_t w = lane_u32(vW, j);
        const int E = grid_of(sum);
        const uint32_t k = grid_units(sum, E);
        if (sum_total(w) != SUM_EVENT) {
          const uint32_t T = lane_u32(vT, j);
          if (sum_grid(w) == E && T < GRID_TOP && k + T < GRID_TOP &&
              !(FIND && r < __builtin_ldexpf((float)(k + T), E))) {
            sum = __builtin_ldexpf((float)(k + T), E);
            continue;
          }
          c0 = cc;
          stop = true;
          break;
        }
        uint32_t hit;
        if (!walk_chunk<FIND>(a, gsum, inv, r, L, s, cc, lane_u32(vS, j), V, sum, hit)) {
          ok = false;
          stop = true;
          break;
        }
        if (FIND && hit < 64) {
          found = cc * VCHUNK + hit;
          stop = true;
          break;
        }
      }
      if (stop) break;
    }
    while (ok && found == NO_INDEX && c0 < nvc) {
      const int E = grid_of(sum);
      const uint32_t k = grid_units(sum, E);
      const uint32_t w0 = L.sw[c0];
      const uint32_t e = L.nxt[c0];
      const uint32_t T = L.PI[c0];
      if (sum_total(w0) != SUM_EVENT && sum_grid(w0) == E && T < GRID_TOP && k + T < GRID_TOP &&
          !(FIND && r < __builtin_ldexpf((float)(k + T), E))) {
        // the rest of c0's segment as one integer step
        sum = __builtin_ldexpf((float)(k + T), E);
        c0 = e;
        continue;
      }
      uint32_t fb = 0;
      if (sum_total(w0) != SUM_EVENT) {
        const uint32_t c = c0 + lane;
        const uint32_t w = c < nvc ? L.sw[c] : SUM_EVENT;
        const uint32_t I = sum_total(w);
        bool use = c < nvc && I != SUM_EVENT && sum_grid(w) == E;
        const uint32_t P = wave_scan_u32(use ? I : 0u);
        use = use && k + P < GRID_TOP;
        bool stop = !use;
        if (FIND) stop = stop || r < __builtin_ldexpf((float)(k + P), E);
        fb = first_lane(__ballot(stop));
        const uint32_t pre = fb ? lane_u32(P, fb - 1) : 0u;
        sum = __builtin_ldexpf((float)(k + pre), E);
        c0 += fb;
      }
      if (fb < 64 && c0 < nvc) {
        uint32_t hit;
        if (!walk_chunk<FIND>(a, gsum, inv, r, L, s, c0, L.slot[c0], V, sum, hit)) {
          ok = false;
          break;
        }
        if (FIND && hit < 64) {
          found = c0 * VCHUNK + hit;
          break;
        }
        ++c0;
      }
    }
    // No crossing (the rounded total stayed at or below r): the last v with
    // q_v > 0 (sampler.rs:103-108), 0 if none.
    for (uint32_t cc = nvc; FIND && ok && found == NO_INDEX && cc-- > 0;) {
      const uint32_t base = cc * VCHUNK, n = min(VCHUNK, V - base);
      const u64* ptr[1] = {a.mb_p + base + min(lane, n - 1)};
      float t[1];
      if (!load_tagged<1>(ptr, gsum, t, a.st, s.ctl)) {
        ok = false;
        break;
      }
      const unsigned long long nz = __ballot(lane < n && t[0] * inv > 0.0f);
      if (nz) found = base + 63u - (uint32_t)__clzll((long long)nz);
    }
    if (FIND && ok && found == NO_INDEX) found = 0;
    if (lane == 0) {
      L.res[0] = FIND ? found : __float_as_uint(sum);
      L.res[1] = ok ? 1u : 0u;
    }
  }
  __syncthreads();
  const bool ok = L.res[1] != 0;
  *out = L.res[0];
  __syncthreads();
  return ok;
}

// Stages A2 to W2 (stage A has run on every participating workgroup; m and
// the argmax bi are its results): the token sample_token returns (and, if
// total_bits is given, the bits of the sequential total). Where m is not
// finite the reference's total is NaN or 0 and it falls back to argmax
// (sampler.rs:60-69).
__device__ __forceinline__ bool sample_exact(const Args& a, uint32_t gsum, float m, uint32_t bi, uint32_t word,
                                             uint32_t wg, uint32_t G, bool own_in_lds, const Lds& s,
                                             uint32_t* tok_out, uint32_t* total_bits = nullptr) {
  if (!isfinite(m)) {
    *tok_out = (bi == NO_INDEX) ? 0u : bi;
    return true;
  }
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc;
  const SampLds L = samp_lds(s, nvc, a.d.lds_vec);
  // A2
  if (!poll_gather<2>(gather_vec(a.mb_vsum, nvc, gsum, L.A), NWA, a.st, s.ctl)) return false;
  approx_prefix(L.A, L.pre, nvc, reinterpret_cast<float*>(L.dred));
  if (!publish_summaries<false>(a, a.mb_psum, gsum, 1.0f, 0.0f, wg, G, own_in_lds, L, s)) return false;
  if (!fetch_events<false>(a, gsum, 1.0f, 0.0f, 0, L, s)) return false;
  // W1
  if (!poll_gather<2>(gather_vec(a.mb_psum, nvc, gsum, reinterpret_cast<float*>(L.sw)), NWA, a.st, s.ctl))
    return false;
  if (!fetch_events<false>(a, gsum, 1.0f, 0.0f, 1, L, s)) return false;
  build_segments(L, nvc);
  uint32_t sum_bits;
  if (!exact_walk<false>(a, gsum, 1.0f, 0.0f, L, s, &sum_bits)) return false;
  if (total_bits) *total_bits = sum_bits;
  const float inv = 1.0f / __uint_as_float(sum_bits);
  const float r = unit_f32(word);
  // C
  if (!publish_summaries<true>(a, a.mb_qsum, gsum, inv, r, wg, G, own_in_lds, L, s)) return false;
  if (!fetch_events<true>(a, gsum, inv, r, 0, L, s)) return false;
  // W2
  if (!poll_gather<2>(gather_vec(a.mb_qsum, nvc, gsum, reinterpret_cast<float*>(L.sw)), NWA, a.st, s.ctl))
    return false;
  if (!fetch_events<true>(a, gsum, inv, r, 1, L, s)) return false;
  build_segments(L, nvc);
  return exact_walk<true>(a, gsum, inv, r, L, s, tok_out);
}

// The greedy token: the global argmax of the chunk maxima (0 when every
// logit is NaN), on every workgroup that calls it.
__device__ __forceinline__ bool sample_greedy(const Args& a, uint32_t tick, const Lds& s, uint32_t* tok_out) {
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u);
  float* vmx = s.scr;
  float* varg = vmx + nvc;
  if (!poll_gather<2, 2>(gather_vec(a.mb_vmax, nvc, gl, vmx), gather_vec(a.mb_varg, nvc, gl, varg), NWA,
                         a.st, s.ctl))
    return false;
  float bv;
  uint32_t bi;
  global_argmax(vmx, varg, nvc, s.red, &bv, &bi);
  *tok_out = (bi == NO_INDEX) ? 0u : bi;
  return true;
}

// The whole sampler on one workgroup after stage A ran on G workgroups (the
// per-phase kernels): m from the chunk maxima, then stages A2 to W2 with this
// workgroup owning every chunk.
__device__ __forceinline__ bool sample_one_wg(const Args& a, uint32_t tick, uint32_t gsum, float T, uint32_t word,
                                              const Lds& s, uint32_t* tok_out) {
  if (T == 0.0f) return sample_greedy(a, tick, s, tok_out);
  const Dims d = shape_dims(a.d);
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u);
  const SampLds L = samp_lds(s, nvc, a.d.lds_vec);
  if (!poll_gather<2, 2>(gather_vec(a.mb_vmax, nvc, gl, L.vmx), gather_vec(a.mb_varg, nvc, gl, L.varg), NWA,
                         a.st, s.ctl))
    return false;
  float bv;
  uint32_t bi;
  global_argmax(L.vmx, L.varg, nvc, s.red, &bv, &bi);
  const float m = (bi == NO_INDEX) ? -INFINITY : bv / T;
  return sample_exact(a, gsum, m, bi, word, 0, 1, false, s, tok_out);
}

}  // namespace DG_NS
