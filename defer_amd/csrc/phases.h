// phases.h -- the phases of one token's forward pass and the sampler, as
// workgroup-level device functions. Each takes (wg, G): the calling
// workgroup and how many workgroups share the phase. The persistent kernel
// runs them back to back; the per-phase kernels run one each. Work items are
// dealt round-robin (item = wg + G*k), and an item is always computed the
// same way whoever computes it.
//
// Roles inside a workgroup (BLOCK = 512 threads = 8 waves):
//  * waves 0..NPOLL-1 are pollers: in the matvec phases they alone read
//    mailboxes, so their in-order load counter never holds a weight load
//    and a poll completes as soon as its data is there;
//  * waves NPOLL.. are compute waves: each owns the matvec items dealt to it
//    and keeps the rows of its first NSLOT items in register slots, each
//    refilled for the next layer right after use (persistent kernel only),
//    so the weights of a phase are in registers before its inputs arrive.
#pragma once

#include "device.h"

namespace dg {

constexpr uint32_t NPOLL = 2;
constexpr uint32_t NCW = NWAVES - NPOLL;
constexpr uint32_t NSLOT = 2;
constexpr int KS = 3;  // float4 per lane in half a slot: 768 floats

struct Lds {
  WaitCtl* ctl;
  float* red;   // 64 floats
  float* vec;   // d.lds_vec floats: the matvec input vector
  float* vec2;  // d.lds_vec2 floats: the normalised lm_head input
  float* scr;   // d.lds_scr floats
};

__device__ inline Lds lds_layout(float* base, const Dims& d) {
  Lds s;
  s.ctl = reinterpret_cast<WaitCtl*>(base);
  s.red = base + 4;
  s.vec = base + 4 + 64;
  s.vec2 = s.vec + d.lds_vec;
  s.scr = s.vec2 + d.lds_vec2;
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
template <uint32_t P>
__device__ __forceinline__ void poll_issue(PollState<P>& ps, const Gather& g, uint32_t base,
                                           uint32_t tid, uint32_t npl) {
#pragma unroll
  for (uint32_t k = 0; k < P; ++k)
    if (ps.pend & (1u << k)) ps.w[k] = mb_load(g.src + gather_off(g, base + tid + k * npl));
}
template <uint32_t P>
__device__ __forceinline__ void poll_check(PollState<P>& ps, const Gather& g, uint32_t base,
                                           uint32_t tid, uint32_t npl) {
#pragma unroll
  for (uint32_t k = 0; k < P; ++k)
    if ((ps.pend & (1u << k)) && (uint32_t)(ps.w[k] >> 32) == g.gen) {
      lds_st(g.dst + base + tid + k * npl, __uint_as_float((uint32_t)ps.w[k]));
      ps.pend &= ~(1u << k);
    }
}

__device__ __forceinline__ uint32_t rounds_for(uint32_t n, uint32_t per_round) {
  return per_round ? (n + per_round - 1) / per_round : (n ? 0xffffffffu : 0u);
}

// Wait until every element of up to three gathers carries its generation and
// copy the values to LDS. Only the first `npoll_waves` waves read memory; a
// polling lane keeps P0 + P1 + P2 words in flight per round (sized to the call
// site), loops until its own words are all current, and the block then meets
// at a barrier. Returns false (uniformly) if the run was aborted.
template <uint32_t P0, uint32_t P1 = 0, uint32_t P2 = 0>
__device__ __forceinline__ bool poll_gather(const Gather& g0, const Gather& g1, const Gather& g2,
                                            uint32_t npoll_waves, DevState* st, WaitCtl* ctl) {
  const uint32_t tid = threadIdx.x;
  const uint32_t npl = npoll_waves * WAVE;
  // The destination LDS may still be read by the previous phase.
  __syncthreads();
  if (tid < npl) {
    const uint32_t n0 = g0.seg_len * g0.n_seg, n1 = g1.seg_len * g1.n_seg;
    const uint32_t n2 = g2.seg_len * g2.n_seg;
    const uint32_t rounds = max(max(rounds_for(n0, P0 * npl), rounds_for(n1, P1 * npl)),
                                rounds_for(n2, P2 * npl));
    for (uint32_t r = 0; r < rounds; ++r) {
      PollState<P0> s0;
      PollState<P1> s1;
      PollState<P2> s2;
      poll_init(s0, g0, n0, r * P0 * npl, tid, npl);
      poll_init(s1, g1, n1, r * P1 * npl, tid, npl);
      poll_init(s2, g2, n2, r * P2 * npl, tid, npl);
      for (uint32_t spins = 0;; ++spins) {
        poll_issue(s0, g0, r * P0 * npl, tid, npl);
        poll_issue(s1, g1, r * P1 * npl, tid, npl);
        poll_issue(s2, g2, r * P2 * npl, tid, npl);
        poll_check(s0, g0, r * P0 * npl, tid, npl);
        poll_check(s1, g1, r * P1 * npl, tid, npl);
        poll_check(s2, g2, r * P2 * npl, tid, npl);
        if (__all((s0.pend | s1.pend | s2.pend) == 0)) break;
        if (spins >= SPIN_LIMIT) {
          st_coherent_u32(&st->abort, 1u);
          ctl->abort_seen = 1;
          break;
        }
        if ((spins & 63) == 63 && ld_coherent_u32(&st->abort)) {
          ctl->abort_seen = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (ctl->abort_seen) break;
    }
  }
  __syncthreads();
  return ctl->abort_seen == 0;
}

template <uint32_t P0, uint32_t P1>
__device__ __forceinline__ bool poll_gather(const Gather& g0, const Gather& g1, uint32_t npw,
                                            DevState* st, WaitCtl* ctl) {
  return poll_gather<P0, P1, 0>(g0, g1, no_gather(), npw, st, ctl);
}
template <uint32_t P0>
__device__ __forceinline__ bool poll_gather(const Gather& g0, uint32_t npw, DevState* st,
                                            WaitCtl* ctl) {
  return poll_gather<P0, 0, 0>(g0, no_gather(), no_gather(), npw, st, ctl);
}

// Number of items i = wg + G*k below n owned by this workgroup.
__device__ __forceinline__ uint32_t rows_owned(uint32_t n, uint32_t wg, uint32_t G) {
  return wg < n ? (n - wg + G - 1) / G : 0;
}

// ------------------------------------------------------------- matvec items

enum ItemKind : uint32_t { IK_QKV = 0, IK_O = 1, IK_GU = 2, IK_D = 3 };

// The workgroup's items of every kind, numbered in order QKV, O, GU, D; item
// number r belongs to compute wave r % NCW and lives in its slot r / NCW
// (items with r / NCW >= NSLOT are loaded when used).
struct Deal {
  uint32_t base[4], cnt[4];
};

__device__ __forceinline__ Deal deal_of(const Dims& d, uint32_t wg, uint32_t G) {
  Deal q;
  q.cnt[IK_QKV] = rows_owned(d.qkv_rows / 2, wg, G);
  q.cnt[IK_O] = rows_owned(d.h, wg, G);
  q.cnt[IK_GU] = rows_owned(d.ff, wg, G);
  q.cnt[IK_D] = rows_owned(d.h, wg, G);
  q.base[0] = 0;
  q.base[1] = q.cnt[0];
  q.base[2] = q.base[1] + q.cnt[1];
  q.base[3] = q.base[2] + q.cnt[2];
  return q;
}

// Registers holding the first 1536 floats of one item: two rows of up to 768
// (pairs) or one row split in halves.
struct Slot {
  RowT<KS> a, b;
};

// Row pointers and length of item k of a kind in layer l. Pairs give two
// rows (QKV: rows i and i + hd/2 of one head; GU: gate and up row j).
struct ItemRows {
  const float* w0;
  const float* w1;  // null for single-row kinds
  uint32_t K;
};

__device__ __forceinline__ ItemRows item_rows(const Args& a, uint32_t kind, uint32_t l, uint32_t k,
                                              uint32_t wg, uint32_t G) {
  const Dims& d = a.d;
  const LayerW& W = a.layers[l];
  const uint32_t it = wg + G * k;
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

__device__ __forceinline__ void slot_load(Slot& S, const ItemRows& r, uint32_t lane) {
  row_load(S.a, r.w0, r.K, lane);
  if (r.w1)
    row_load(S.b, r.w1, r.K, lane);
  else if (r.K > 256u * KS)
    row_load(S.b, r.w0 + 256u * KS, r.K - 256u * KS, lane);
}

// Lane partial of w . x over a row whose first 256*KS floats are in `first`
// and, when `second` is given, the next 256*KS in `second`; the rest streams.
// Ascending j, one fma per element.
__device__ __forceinline__ float dot_slot(RowT<KS>& first, RowT<KS>* second, const float* w,
                                          const float* x, uint32_t K, uint32_t lane) {
  float acc = row_fma(first, x, K, lane, 0.0f);
  uint32_t base = 256u * KS;
  if (second && base < K) {
    acc = row_fma(*second, x + base, K - base, lane, acc);
    base += 256u * KS;
  }
  for (; base < K; base += 256u * KS) {
    row_load(first, w + base, K - base, lane);
    acc = row_fma(first, x + base, K - base, lane, acc);
  }
  return acc;
}

// Lane partial of x . x over the lane's elements of a length-K vector, in
// the order the dot products visit them.
__device__ __forceinline__ float sumsq_lane(const float* x, uint32_t K, uint32_t lane) {
  float ss = 0.0f;
  for (uint32_t j = lane * 4; j < K; j += 256) {
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

// Runs body(k, si) for every item of `kind` dealt to compute wave cw, in item
// order; si is the item's slot (>= NSLOT: no slot).
template <class F>
__device__ __forceinline__ void for_items(const Deal& q, uint32_t kind, uint32_t cw, F body) {
  const uint32_t b = q.base[kind], n = q.cnt[kind];
  uint32_t k = (cw + NCW - b % NCW) % NCW;  // first k with (b + k) % NCW == cw
  for (; k < n; k += NCW) body(k, (b + k) / NCW);
}

struct SlotSet {
  Slot s[NSLOT];
};

// Calls f(slot si) with a statically indexed slot (so slots stay in
// registers).
template <class F>
__device__ __forceinline__ void with_slot(SlotSet& SS, uint32_t si, F f) {
  static_assert(NSLOT >= 1 && NSLOT <= 3, "with_slot covers up to three slots");
  if (si == 0)
    f(SS.s[0]);
  else if (NSLOT >= 2 && si == 1)
    f(SS.s[NSLOT >= 2 ? 1 : 0]);
  else if (NSLOT >= 3)
    f(SS.s[NSLOT >= 3 ? 2 : 0]);
}

// Prefetch state of the calling wave.
struct Pf {
  bool on;              // the slots hold this layer's rows (persistent kernel)
  SlotSet* SS;          // this wave's slots
  uint32_t next_layer;  // layer the refills load
};

// Refill the slots of compute wave cw that hold items of `kind` with layer
// l's rows (persistent kernel, right after they were consumed).
__device__ __forceinline__ void slot_refill(const Args& a, const Deal& q, const Pf& pf, uint32_t cw,
                                            uint32_t kind, uint32_t wg, uint32_t G, uint32_t lane) {
  if (!pf.on) return;
  for_items(q, kind, cw, [&](uint32_t k, uint32_t si) {
    if (si >= NSLOT) return;
    const ItemRows r = item_rows(a, kind, pf.next_layer, k, wg, G);
    with_slot(*pf.SS, si, [&](Slot& S) { slot_load(S, r, lane); });
  });
}

// Dot products of one item whose rows are in S against the LDS vector x:
// y0 (and y1 for pairs). S is consumed.
__device__ __forceinline__ void slot_dot(Slot& S, const ItemRows& r, const float* x, uint32_t lane,
                                         float* y0, float* y1) {
  if (r.w1) {
    *y0 = wave_sum(dot_slot(S.a, nullptr, r.w0, x, r.K, lane));
    *y1 = wave_sum(dot_slot(S.b, nullptr, r.w1, x, r.K, lane));
  } else {
    *y0 = wave_sum(dot_slot(S.a, &S.b, r.w0, x, r.K, lane));
    *y1 = 0.0f;
  }
}

// Item k of a kind: from its prefetched slot, or loaded now.
__device__ __forceinline__ void item_dot(const Args& a, uint32_t kind, uint32_t l, uint32_t k,
                                         uint32_t si, const Pf& pf, const float* x, uint32_t wg,
                                         uint32_t G, uint32_t lane, float* y0, float* y1) {
  const ItemRows r = item_rows(a, kind, l, k, wg, G);
  if (pf.on && si < NSLOT) {
    with_slot(*pf.SS, si, [&](Slot& S) { slot_dot(S, r, x, lane, y0, y1); });
  } else {
    Slot T;
    slot_load(T, r, lane);
    slot_dot(T, r, x, lane, y0, y1);
  }
}

// Fill the calling compute wave's slots with their items' rows of layer l
// (persistent kernel start).
__device__ __forceinline__ void slot_prime(const Args& a, SlotSet& SS, uint32_t l, uint32_t wg,
                                           uint32_t G) {
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  if (wave < NPOLL) return;
  const Deal q = deal_of(a.d, wg, G);
  Pf pf;
  pf.on = true;
  pf.SS = &SS;
  pf.next_layer = l;
  for (uint32_t kind = 0; kind < 4; ++kind) slot_refill(a, q, pf, wave - NPOLL, kind, wg, G, lane);
}

// ------------------------------------------------------------------ QKV

// rmsnorm -> q/k/v rows (+bias) -> RoPE on q and k (model.rs:460-465) ->
// k, v appended to the cache at `pos` (model.rs:466-467). Item = a pair of
// rows (i, i + hd/2) of one head, so RoPE needs no exchange.
__device__ __forceinline__ bool phase_qkv(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                          uint32_t token, uint32_t wg, uint32_t G, const Lds& s,
                                          const Pf& pf) {
  const Dims& d = a.d;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  if (l == 0) {
    // The embedding row (model.rs:428), read by the pollers only.
    __syncthreads();
    const float* e = a.embed + (size_t)token * d.h;
    for (uint32_t i = threadIdx.x; i < d.h && threadIdx.x < NPOLL * WAVE; i += NPOLL * WAVE)
      lds_st(s.vec + i, ldg(e + i));
    __syncthreads();
  } else if (!poll_gather<8>(gather_vec(a.mb_xd, d.h, gen_of(d, tick, l - 1, PH_D), s.vec), NPOLL,
                          a.st, s.ctl)) {
    return false;
  }
  if (wave < NPOLL) return true;
  const uint32_t cw = wave - NPOLL;
  const Deal q = deal_of(d, wg, G);
  if (q.cnt[IK_QKV] == 0) return true;
  const float inv = rms_inv(s.vec, d.h, d.eps, lane);
  const uint32_t gen = gen_of(d, tick, l, PH_QKV);
  const LayerW& W = a.layers[l];
  const float2* rp = a.rope + (size_t)pos * d.half;
  for_items(q, IK_QKV, cw, [&](uint32_t k, uint32_t si) {
    float y0, y1;
    item_dot(a, IK_QKV, l, k, si, pf, s.vec, wg, G, lane, &y0, &y1);
    const uint32_t p = wg + G * k;
    const uint32_t hb = p / d.half, i = p - hb * d.half;
    const uint32_t r0 = hb * d.hd + i, r1 = r0 + d.half;
    y0 *= inv;
    y1 *= inv;
    if (W.bqkv) {
      y0 += ldg(W.bqkv + r0);
      y1 += ldg(W.bqkv + r1);
    }
    if (hb < d.nh + d.nkv) {
      const float2 cs = ldg2(rp + i);
      const float a0 = y0 * cs.x - y1 * cs.y;
      const float a1 = y1 * cs.x + y0 * cs.y;
      y0 = a0;
      y1 = a1;
    }
    if (lane == 0) {
      mb_put(a.mb_qkv + r0, y0, gen);
      mb_put(a.mb_qkv + r1, y1, gen);
    }
    if (hb >= d.nh && lane == 1) {
      const bool is_k = hb < d.nh + d.nkv;
      const uint32_t g = is_k ? hb - d.nh : hb - d.nh - d.nkv;
      float* row = (is_k ? a.kc : a.vc) + (((size_t)l * d.nkv + g) * d.cap + pos) * d.kvs;
      st_coherent(row + i, y0);
      st_coherent(row + i + d.half, y1);
    }
  });
  return true;
}

// ------------------------------------------------------------ attention

constexpr uint32_t MAX_GROUP = 4;
constexpr uint32_t ATT_PF = 4;  // position iterations whose K/V rows a lane holds at once
// Waves that compute attention (all of them; a fixed number, so the merge
// order does not depend on the launch).
constexpr uint32_t NWA = NWAVES;

// K/V rows (this lane's float4) of positions t, t + stride, ... for ATT_PF
// iterations; rows at or past `pos` come from LDS, not the cache.
__device__ __forceinline__ void load_kv(const float* kb, const float* vb, float4* kr, float4* vr,
                                        uint32_t t, uint32_t stride, uint32_t t1, uint32_t pos,
                                        uint32_t kvs, uint32_t sub) {
#pragma unroll
  for (uint32_t it = 0; it < ATT_PF; ++it) {
    const uint32_t tt = t + stride * it;
    if (tt < t1 && tt < pos) {
      kr[it] = ldg4(kb + (size_t)tt * kvs + sub * 4);
      vr[it] = ldg4(vb + (size_t)tt * kvs + sub * 4);
    }
  }
}

// Online-softmax state of one query head over this lane group's positions.
struct AttState {
  float m, l, acc[4];
};

// Folds ATT_PF iterations (positions t0 + gi + NG*(base + it)) into st.
__device__ __forceinline__ void att_batch(AttState& st, const float4* kr, const float4* vr,
                                          const float* qh, const float* kn, const float* vn,
                                          const uint32_t* mask, float scale, uint32_t t_first,
                                          uint32_t NG, uint32_t t1, uint32_t pos, uint32_t sub,
                                          uint32_t LP) {
#pragma unroll
  for (uint32_t it = 0; it < ATT_PF; ++it) {
    const uint32_t t = t_first + NG * it;
    if (t >= t1) continue;
    const bool cur = (t == pos);
    const float4 kk = cur ? lds4(kn + sub * 4) : kr[it];
    const float4 vv = cur ? lds4(vn + sub * 4) : vr[it];
    const bool masked = mask && t < pos && ((ldg_u32(mask + (t >> 5)) >> (t & 31)) & 1u);
    const float4 qq = lds4(qh + sub * 4);
    float p = qq.x * kk.x;
    p = fmaf(qq.y, kk.y, p);
    p = fmaf(qq.z, kk.z, p);
    p = fmaf(qq.w, kk.w, p);
    for (uint32_t o = LP / 2; o > 0; o >>= 1) p += __shfl_xor(p, o);
    const float sc = masked ? -INFINITY : p * scale;
    if (sc > st.m) {
      const float r = (st.m == -INFINITY) ? 0.0f : expf(st.m - sc);
      st.l *= r;
      st.acc[0] *= r;
      st.acc[1] *= r;
      st.acc[2] *= r;
      st.acc[3] *= r;
      st.m = sc;
    }
    const float e = (sc == -INFINITY) ? 0.0f : expf(sc - st.m);
    st.l += e;
    st.acc[0] = fmaf(e, vv.x, st.acc[0]);
    st.acc[1] = fmaf(e, vv.y, st.acc[1]);
    st.acc[2] = fmaf(e, vv.z, st.acc[2]);
    st.acc[3] = fmaf(e, vv.w, st.acc[3]);
  }
}

// Split-context attention for one (kv head, chunk) item: scores, softmax
// partials (max m, sum l, unnormalised acc) for each query head of the GQA
// group (model.rs:471-497). A chunk's K/V rows are loaded once and reused for
// every head of the group when they fit the lane's registers; longer chunks
// stream them again per head.
__device__ __forceinline__ bool phase_attn(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                           uint32_t wg, uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  const uint32_t nch = attn_nchunks(pos), CH = attn_chunk(pos);
  const uint32_t n_items = d.nkv * nch;
  const uint32_t gen_in = gen_of(d, tick, l, PH_QKV);
  const uint32_t gen_out = gen_of(d, tick, l, PH_ATTN);
  const uint32_t hd = d.hd, grp = d.group, hs = hd + 2;
  float* qs = s.scr;            // [grp*hd]
  float* kn = qs + grp * hd;    // [hd]
  float* vn = kn + hd;          // [hd]
  float* wp = vn + hd;          // [NWA][grp][hd+2]
  const uint32_t LP = hd / 4, PPI = WAVE / LP, NG = NWA * PPI;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t sub = lane % LP;
  const uint32_t gi = wave * PPI + lane / LP;
  for (uint32_t item = wg; item < n_items; item += G) {
    const uint32_t g = item / nch, c = item - g * nch;
    const uint32_t t0 = c * CH;
    const uint32_t t1 = min(t0 + CH, pos + 1);
    const float* kb = a.kc + ((size_t)l * d.nkv + g) * d.cap * d.kvs;
    const float* vb = a.vc + ((size_t)l * d.nkv + g) * d.cap * d.kvs;
    // The first batch of historical K/V rows is issued before waiting for
    // this token's q/k/v.
    float4 kr[ATT_PF], vr[ATT_PF];
    load_kv(kb, vb, kr, vr, t0 + gi, NG, t1, pos, d.kvs, sub);
    if (!poll_gather<2, 1, 1>(gather_vec(a.mb_qkv + (size_t)g * grp * hd, grp * hd, gen_in, qs),
                              gather_vec(a.mb_qkv + d.q + g * hd, hd, gen_in, kn),
                              gather_vec(a.mb_qkv + d.q + d.kv + g * hd, hd, gen_in, vn), NPOLL,
                              a.st, s.ctl))
      return false;
    const uint32_t n_iter = (t1 - t0 + NG - 1) / NG;
    for (uint32_t j = 0; j < grp; ++j) {
      AttState st;
      st.m = -INFINITY;
      st.l = 0.0f;
      st.acc[0] = st.acc[1] = st.acc[2] = st.acc[3] = 0.0f;
      for (uint32_t base = 0; base < n_iter; base += ATT_PF) {
        if (n_iter > ATT_PF && (base > 0 || j > 0))
          load_kv(kb, vb, kr, vr, t0 + gi + NG * base, NG, t1, pos, d.kvs, sub);
        att_batch(st, kr, vr, qs + j * hd, kn, vn, a.mask, d.scale, t0 + gi + NG * base, NG, t1,
                  pos, sub, LP);
      }
      // Merge the position groups of this wave (lanes with the same `sub`).
      for (uint32_t o = LP; o < WAVE; o <<= 1) {
        const float m2 = __shfl_xor(st.m, o), l2 = __shfl_xor(st.l, o);
        const float b0 = __shfl_xor(st.acc[0], o), b1 = __shfl_xor(st.acc[1], o);
        const float b2 = __shfl_xor(st.acc[2], o), b3 = __shfl_xor(st.acc[3], o);
        const float mn = fmaxf(st.m, m2);
        const float s1 = (st.m == -INFINITY) ? 0.0f : expf(st.m - mn);
        const float s2 = (m2 == -INFINITY) ? 0.0f : expf(m2 - mn);
        st.l = st.l * s1 + l2 * s2;
        st.acc[0] = st.acc[0] * s1 + b0 * s2;
        st.acc[1] = st.acc[1] * s1 + b1 * s2;
        st.acc[2] = st.acc[2] * s1 + b2 * s2;
        st.acc[3] = st.acc[3] * s1 + b3 * s2;
        st.m = mn;
      }
      if (lane < LP) {
        float* dst = wp + (wave * grp + j) * hs;
        if (lane == 0) {
          lds_st(dst + 0, st.m);
          lds_st(dst + 1, st.l);
        }
        lds_st(dst + 2 + sub * 4 + 0, st.acc[0]);
        lds_st(dst + 2 + sub * 4 + 1, st.acc[1]);
        lds_st(dst + 2 + sub * 4 + 2, st.acc[2]);
        lds_st(dst + 2 + sub * 4 + 3, st.acc[3]);
      }
    }
    __syncthreads();
    // Merge the waves in wave order and publish the chunk's partials.
    for (uint32_t u = threadIdx.x; u < grp * hd; u += BLOCK) {
      const uint32_t j = u / hd, dd = u - j * hd;
      float M = -INFINITY;
      for (uint32_t w = 0; w < NWA; ++w) M = fmaxf(M, lds_ld(wp + (w * grp + j) * hs));
      float Ls = 0.0f, A = 0.0f;
      for (uint32_t w = 0; w < NWA; ++w) {
        const float* src = wp + (w * grp + j) * hs;
        const float mw = lds_ld(src);
        const float sw = (mw == -INFINITY) ? 0.0f : expf(mw - M);
        Ls = Ls + lds_ld(src + 1) * sw;
        A = A + lds_ld(src + 2 + dd) * sw;
      }
      const uint32_t hh = g * grp + j;
      u64* out = a.mb_part + ((size_t)hh * MAX_ACHUNKS + c) * hs;
      mb_put(out + 2 + dd, A, gen_out);
      if (dd == 0) {
        mb_put(out + 0, M, gen_out);
        mb_put(out + 1, Ls, gen_out);
      }
    }
  }
  return true;
}

// Combine the chunk partials of one head (in chunk order) into its output:
// att[d] = sum_c acc_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M).
__device__ __forceinline__ float combine_one(const float* part, uint32_t nch, uint32_t hs,
                                             uint32_t dd) {
  float M = -INFINITY;
  for (uint32_t c = 0; c < nch; ++c) M = fmaxf(M, lds_ld(part + c * hs));
  float Ls = 0.0f, A = 0.0f;
  for (uint32_t c = 0; c < nch; ++c) {
    const float* p = part + c * hs;
    const float mc = lds_ld(p);
    const float sc = (mc == -INFINITY) ? 0.0f : expf(mc - M);
    Ls = Ls + lds_ld(p + 1) * sc;
    A = A + lds_ld(p + 2 + dd) * sc;
  }
  return A / Ls;
}

// Separate combine (used when the partials of all heads do not fit the O
// phase's LDS budget): item = one query head.
__device__ __forceinline__ bool phase_comb(const Args& a, uint32_t l, uint32_t tick, uint32_t pos,
                                           uint32_t wg, uint32_t G, const Lds& s) {
  const Dims& d = a.d;
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
                                        const Pf& pf) {
  const Dims& d = a.d;
  const uint32_t nch = attn_nchunks(pos), hs = d.hd + 2;
  const bool inl = comb_inline(d, pos);
  const Deal q = deal_of(d, wg, G);
  const uint32_t R = q.cnt[IK_O];
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  float* part = s.scr;
  float* xres = s.scr + (inl ? d.nh * nch * hs : 0);
  const Gather ga =
      inl ? gather_strided(a.mb_part, nch * hs, d.nh, MAX_ACHUNKS * hs, gen_of(d, tick, l, PH_ATTN),
                           part)
          : gather_vec(a.mb_att, d.q, gen_of(d, tick, l, PH_COMB), s.vec);
  const Gather gr = (l > 0 && R > 0)
                        ? gather_strided(a.mb_xd + wg, 1, R, G, gen_of(d, tick, l - 1, PH_D), xres)
                        : no_gather();
  if (!poll_gather<12, 1>(ga, gr, NPOLL, a.st, s.ctl)) return false;
  // QKV slots were consumed before the attention; refill them now that the
  // attention's K/V reads are done (next layer, or the next token's layer 0).
  if (pf.on && wave >= NPOLL)
    slot_refill(a, q, pf, wave - NPOLL, IK_QKV, wg, G, lane);
  if (l == 0)
    for (uint32_t k = threadIdx.x; k < R; k += BLOCK)
      lds_st(xres + k, ldg(a.embed + (size_t)token * d.h + wg + G * k));
  if (inl)
    for (uint32_t u = threadIdx.x; u < d.q; u += BLOCK) {
      const uint32_t hh = u / d.hd, dd = u - hh * d.hd;
      lds_st(s.vec + u, combine_one(part + hh * nch * hs, nch, hs, dd));
    }
  __syncthreads();
  if (wave < NPOLL) return true;
  const uint32_t cw = wave - NPOLL;
  const uint32_t gen = gen_of(d, tick, l, PH_O);
  for_items(q, IK_O, cw, [&](uint32_t k, uint32_t si) {
    float y, unused;
    item_dot(a, IK_O, l, k, si, pf, s.vec, wg, G, lane, &y, &unused);
    if (lane == 0) mb_put(a.mb_xo + wg + G * k, lds_ld(xres + k) + y, gen);
  });
  slot_refill(a, q, pf, cw, IK_O, wg, G, lane);
  return true;
}

// ------------------------------------------------------------ MLP

// rmsnorm -> g = act(Wg.x) * (Wu.x) (model.rs:502-509).
__device__ __forceinline__ bool phase_gu(const Args& a, uint32_t l, uint32_t tick, uint32_t wg,
                                         uint32_t G, const Lds& s, const Pf& pf) {
  const Dims& d = a.d;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  if (!poll_gather<8>(gather_vec(a.mb_xo, d.h, gen_of(d, tick, l, PH_O), s.vec), NPOLL, a.st, s.ctl))
    return false;
  if (wave < NPOLL) return true;
  const uint32_t cw = wave - NPOLL;
  const Deal q = deal_of(d, wg, G);
  const float inv = rms_inv(s.vec, d.h, d.eps, lane);
  const uint32_t gen = gen_of(d, tick, l, PH_GU);
  for_items(q, IK_GU, cw, [&](uint32_t k, uint32_t si) {
    float gate, up;
    item_dot(a, IK_GU, l, k, si, pf, s.vec, wg, G, lane, &gate, &up);
    if (lane == 0) mb_put(a.mb_g + wg + G * k, act_fn(gate * inv, d.act) * (up * inv), gen);
  });
  slot_refill(a, q, pf, cw, IK_GU, wg, G, lane);
  return true;
}

// x_d = x_o + Wd . g (model.rs:510-511).
__device__ __forceinline__ bool phase_d(const Args& a, uint32_t l, uint32_t tick, uint32_t wg,
                                        uint32_t G, const Lds& s, const Pf& pf) {
  const Dims& d = a.d;
  const Deal q = deal_of(d, wg, G);
  const uint32_t R = q.cnt[IK_D];
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const Gather gr = R > 0 ? gather_strided(a.mb_xo + wg, 1, R, G, gen_of(d, tick, l, PH_O), s.scr)
                          : no_gather();
  if (!poll_gather<12, 1>(gather_vec(a.mb_g, d.ff, gen_of(d, tick, l, PH_GU), s.vec), gr, NPOLL, a.st,
                   s.ctl))
    return false;
  if (wave < NPOLL) return true;
  const uint32_t cw = wave - NPOLL;
  const uint32_t gen = gen_of(d, tick, l, PH_D);
  for_items(q, IK_D, cw, [&](uint32_t k, uint32_t si) {
    float y, unused;
    item_dot(a, IK_D, l, k, si, pf, s.vec, wg, G, lane, &y, &unused);
    if (lane == 0) mb_put(a.mb_xd + wg + G * k, lds_ld(s.scr + k) + y, gen);
  });
  slot_refill(a, q, pf, cw, IK_D, wg, G, lane);
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

constexpr int LMF = 4;  // float4 per lane per lm_head row held in registers (h <= 1024 in one go)

// The final RMSNorm weight, kept in LDS for the kernel's lifetime (the
// lm_head may be the tied embedding, so it cannot be folded into the rows).
__device__ __forceinline__ void lm_prime(const Args& a, const Lds& s) {
  for (uint32_t i = threadIdx.x; i < a.d.h && threadIdx.x < NPOLL * WAVE; i += NPOLL * WAVE)
    lds_st(s.vec2 + a.d.h + i, ldg(a.norm + i));
  __syncthreads();
}

// rmsnorm(final) -> logits = H . x (model.rs:515-519), plus each vocabulary
// chunk's (max, argmax) for the sampler. The workgroup owns chunks
// c = wg + G*k; every wave computes rows, two at a time, with the next two
// rows in flight. logit = inv * (H . (x * w_norm)).
__device__ __forceinline__ bool phase_lm(const Args& a, uint32_t tick, uint32_t wg, uint32_t G,
                                         const Lds& s) {
  const Dims& d = a.d;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < d.nvc ? (d.nvc - wg + G - 1) / G : 0;
  const uint32_t nrows = nown * VCHUNK;  // local rows r -> chunk r / VCHUNK
  float* lg = s.scr;                     // [nrows] logits of this workgroup
  float* xs = s.vec2;                    // x * w_norm
  const float* nrm = s.vec2 + d.h;       // final norm weight (lm_prime)
  auto vocab_row = [&](uint32_t r) { return (wg + G * (r / VCHUNK)) * VCHUNK + r % VCHUNK; };
  RowT<LMF> A0, A1, B0, B1;
  auto load_pair = [&](RowT<LMF>& x0, RowT<LMF>& x1, uint32_t r0) {
    const uint32_t r1 = r0 + NWAVES;
    if (r0 < nrows && vocab_row(r0) < d.V)
      row_load(x0, a.head + (size_t)vocab_row(r0) * d.h, d.h, lane);
    if (r1 < nrows && vocab_row(r1) < d.V)
      row_load(x1, a.head + (size_t)vocab_row(r1) * d.h, d.h, lane);
  };
  load_pair(A0, A1, wave);
  if (!poll_gather<8>(gather_vec(a.mb_xd, d.h, gen_of(d, tick, d.L - 1, PH_D), s.vec), NPOLL, a.st,
                   s.ctl))
    return false;
  for (uint32_t i = threadIdx.x; i < d.h; i += BLOCK) lds_st(xs + i, lds_ld(s.vec + i) * lds_ld(nrm + i));
  __syncthreads();
  const float inv = rms_inv(s.vec, d.h, d.eps, lane);
  const uint32_t gen = gen_lm(d, tick);
  for (uint32_t r0 = wave; r0 < nrows; r0 += 2 * NWAVES) {
    const uint32_t r1 = r0 + NWAVES;
    load_pair(B0, B1, r0 + 2 * NWAVES);
    const uint32_t v0 = vocab_row(r0), v1 = vocab_row(r1);
    if (v0 < d.V) {
      const float y = inv * wave_sum(dot_tail(A0, a.head + (size_t)v0 * d.h, xs, d.h, lane));
      if (lane == 0) {
        lds_st(lg + r0, y);
        mb_put(a.mb_logit + v0, y, gen);
      }
    }
    if (r1 < nrows && v1 < d.V) {
      const float y = inv * wave_sum(dot_tail(A1, a.head + (size_t)v1 * d.h, xs, d.h, lane));
      if (lane == 0) {
        lds_st(lg + r1, y);
        mb_put(a.mb_logit + v1, y, gen);
      }
    }
    A0 = B0;
    A1 = B1;
  }
  __syncthreads();
  // Chunk (max, argmax): one wave per chunk, one lane per row.
  for (uint32_t k = wave; k < nown; k += NWAVES) {
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

// p_v before normalisation: exp(l/T - m), NaN -> 0 (sampler.rs:55-57).
__device__ __forceinline__ float exp_term(float logit, float T, float m) {
  const float sv = logit / T;
  return isnan(sv) ? 0.0f : expf(sv - m);
}

// Sampler stage A (temperature > 0): the global max m from the chunk maxima,
// then exp-sums of this workgroup's chunks, published for stage B.
__device__ __forceinline__ bool sample_stage_a(const Args& a, uint32_t tick, float T, uint32_t wg, uint32_t G,
                               const Lds& s) {
  const Dims& d = a.d;
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u), gsum = gen_sums(d, tick);
  float* vmx = s.scr;
  float* varg = vmx + nvc;
  float* chunk = varg + nvc;  // [NWAVES][VCHUNK]
  if (!poll_gather<4, 4>(gather_vec(a.mb_vmax, nvc, gl, vmx), gather_vec(a.mb_varg, nvc, gl, varg),
                   NWAVES, a.st, s.ctl))
    return false;
  float bv;
  uint32_t bi;
  global_argmax(vmx, varg, nvc, s.red, &bv, &bi);
  const float m = (bi == NO_INDEX) ? -INFINITY : bv / T;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < nvc ? (nvc - wg + G - 1) / G : 0;
  for (uint32_t k0 = 0; k0 < nown; k0 += NWAVES) {
    const uint32_t nb = min(NWAVES, nown - k0);
    // chunks wg + G*(k0 + b), b < nb; the last one may be short
    const u64* src0 = a.mb_logit + (size_t)(wg + G * k0) * VCHUNK;
    const uint32_t clast = wg + G * (k0 + nb - 1);
    // a short last chunk is gathered separately so no slot past V is read
    const bool short_last = (clast + 1) * VCHUNK > d.V;
    const Gather ga = gather_strided(src0, VCHUNK, short_last ? nb - 1 : nb, G * VCHUNK, gl, chunk);
    const Gather gb = short_last ? gather_vec(a.mb_logit + (size_t)clast * VCHUNK,
                                              d.V - clast * VCHUNK, gl, chunk + (nb - 1) * VCHUNK)
                                 : no_gather();
    if (!poll_gather<2, 1>(ga, gb, NWAVES, a.st, s.ctl)) return false;
    if (wave < nb) {
      const uint32_t c = wg + G * (k0 + wave);
      const uint32_t v = c * VCHUNK + lane;
      const float e = (v < d.V) ? exp_term(chunk[wave * VCHUNK + lane], T, m) : 0.0f;
      const float S = wave_sum(e);
      if (lane == 0) mb_put(a.mb_vsum + c, S, gsum);
    }
    __syncthreads();
  }
  return true;
}

// Inclusive scan over the 64 lanes (fixed Hillis-Steele steps).
__device__ __forceinline__ float wave_scan(float x) {
  const uint32_t lane = threadIdx.x % WAVE;
#pragma unroll
  for (uint32_t o = 1; o < WAVE; o <<= 1) {
    const float y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

// Sampler stage B: the token (sampler.rs:78-109). Greedy is the global argmax
// (0 when every logit is NaN). With T > 0 the chunk exp-sums give the total
// and a chunk-level scan of the CDF; the chunk holding the crossing is then
// scanned element by element, p_v = exp(l_v/T - m) * (1/total), returning
// the first v with p_v > 0 and r < cumulative, else the last v with p_v > 0.
// A degenerate total (not > 0, or not finite) falls back to argmax.
__device__ __forceinline__ bool sample_stage_b(const Args& a, uint32_t tick, float T, uint32_t word,
                               const Lds& s, uint32_t* tok_out) {
  const Dims& d = a.d;
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u), gsum = gen_sums(d, tick);
  float* vmx = s.scr;
  float* varg = vmx + nvc;
  float* vsum = varg + nvc;
  float* chunk = vsum + nvc;  // [VCHUNK]
  float* wtot = chunk + VCHUNK;  // [NWAVES + 2]
  if (!poll_gather<4, 4, 4>(gather_vec(a.mb_vmax, nvc, gl, vmx), gather_vec(a.mb_varg, nvc, gl, varg),
                   T != 0.0f ? gather_vec(a.mb_vsum, nvc, gsum, vsum) : no_gather(), NWAVES, a.st,
                   s.ctl))
    return false;
  float bv;
  uint32_t bi;
  global_argmax(vmx, varg, nvc, s.red, &bv, &bi);
  const uint32_t greedy = (bi == NO_INDEX) ? 0u : bi;
  if (T == 0.0f) {
    *tok_out = greedy;
    return true;
  }
  const float m = (bi == NO_INDEX) ? -INFINITY : bv / T;
  // total = fixed-tree sum of the chunk sums
  float part = 0.0f;
  for (uint32_t c = threadIdx.x; c < nvc; c += BLOCK) part += vsum[c];
  const float total = block_sum(part, s.red);
  if (!(total > 0.0f) || !isfinite(total)) {
    *tok_out = greedy;
    return true;
  }
  const float inv = 1.0f / total;
  const float r = unit_f32(word);
  // Chunk-level exclusive prefix of P_c = S_c * inv: each thread owns a
  // contiguous run of chunks, then lanes, then waves, in fixed order.
  const uint32_t per = (nvc + BLOCK - 1) / BLOCK;
  const uint32_t c0 = threadIdx.x * per, c1 = min(c0 + per, nvc);
  float own = 0.0f;
  for (uint32_t c = c0; c < c1; ++c) own += vsum[c] * inv;
  const float incl = wave_scan(own);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  __syncthreads();
  if (lane == WAVE - 1) wtot[wave] = incl;
  __syncthreads();
  float base = 0.0f;
  for (uint32_t w = 0; w < wave; ++w) base += wtot[w];
  float cum = base + (incl - own);
  uint32_t first = NO_INDEX;
  float first_cum = 0.0f;
  for (uint32_t c = c0; c < c1; ++c) {
    const float pc = vsum[c] * inv;
    if (vsum[c] > 0.0f && r < cum + pc) {
      first = c;
      first_cum = cum;
      break;
    }
    cum += pc;
  }
  // lowest chunk index with a crossing, and its starting cumulative value
  uint32_t fc = first;
  for (int o = 32; o > 0; o >>= 1) fc = min(fc, (uint32_t)__shfl_xor(fc, o));
  __syncthreads();
  if (lane == 0) reinterpret_cast<uint32_t*>(wtot)[wave] = fc;
  __syncthreads();
  uint32_t cstar = NO_INDEX;
  for (uint32_t w = 0; w < NWAVES; ++w) cstar = min(cstar, reinterpret_cast<uint32_t*>(wtot)[w]);
  __syncthreads();
  if (first != NO_INDEX && first == cstar) wtot[NWAVES] = first_cum;
  __syncthreads();
  float run = (cstar != NO_INDEX) ? wtot[NWAVES] : 0.0f;
  __syncthreads();
  // Element scan from chunk cstar onwards (normally one chunk).
  for (uint32_t c = cstar; c < nvc; ++c) {
    const uint32_t v0 = c * VCHUNK, nv = min(VCHUNK, d.V - v0);
    if (!poll_gather<1>(gather_vec(a.mb_logit + v0, nv, gl, chunk), NWAVES, a.st, s.ctl)) return false;
    const float p = (lane < nv) ? exp_term(chunk[lane], T, m) * inv : 0.0f;
    const float sc = wave_scan(p > 0.0f ? p : 0.0f);
    const bool hit = p > 0.0f && r < run + sc;
    const unsigned long long hits = __ballot(hit);
    if (hits) {
      *tok_out = v0 + (uint32_t)__ffsll((long long)hits) - 1u;
      __syncthreads();
      return true;
    }
    run = run + __shfl(sc, WAVE - 1);
    __syncthreads();
  }
  // No crossing (rounding): the last token with p > 0.
  for (uint32_t cc = nvc; cc-- > 0;) {
    if (!(vsum[cc] > 0.0f)) continue;
    const uint32_t v0 = cc * VCHUNK, nv = min(VCHUNK, d.V - v0);
    if (!poll_gather<1>(gather_vec(a.mb_logit + v0, nv, gl, chunk), NWAVES, a.st, s.ctl)) return false;
    const float p = (lane < nv) ? exp_term(chunk[lane], T, m) * inv : 0.0f;
    const unsigned long long nz = __ballot(p > 0.0f);
    __syncthreads();
    if (nz) {
      *tok_out = v0 + 63u - (uint32_t)__clzll((long long)nz);
      return true;
    }
  }
  *tok_out = 0;
  return true;
}

}  // namespace dg
