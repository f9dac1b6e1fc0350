// persistent.h -- the persistent kernel (every op of a call in one launch)
// and the LDS set-up the other kernels share. Included once per device
// namespace: generically (dg) and per specialised model shape.
#pragma once

#include "phases.h"

namespace DG_NS {

__device__ __forceinline__ Lds lds_init(const Dims& d) {
  extern __shared__ float lds_raw[];
  Lds s = lds_layout(lds_raw, d);
  if (threadIdx.x == 0) s.ctl->abort_seen = 0;
  __syncthreads();
  return s;
}

__device__ __forceinline__ bool forward_all(const Args& a, uint32_t tok, uint32_t pos, uint32_t tick,
                                            uint32_t wg, uint32_t G, const Lds& s,
                                            const Stager& sg) {
  const uint32_t L = shape_dims(a.d).L;
  for (uint32_t l = 0; l < L; ++l) {
    // Hidden from the optimiser per layer, so values derived from the
    // workgroup index (item numbers, mailbox and cache addresses) are
    // recomputed where they are used instead of being hoisted out of the
    // layer loop and spilled.
    uint32_t wgl = wg;
    asm volatile("" : "+s"(wgl));
    const uint32_t wg = wgl;
    if (!phase_qkv(a, l, tick, pos, tok, wg, G, s, sg)) return false;
    if (!phase_attn(a, l, tick, pos, wg, G, s)) return false;
    if (!phase_comb(a, l, tick, pos, wg, G, s)) return false;
    if (!phase_o(a, l, tick, pos, tok, wg, G, s, sg)) return false;
    if (!phase_gu(a, l, tick, wg, G, s, sg)) return false;
    if (!phase_d(a, l, tick, wg, G, s, sg)) return false;
  }
  return phase_lm(a, tick, wg, G, s, sg);
}

__device__ __forceinline__ bool is_stop(const RunDesc& r, uint32_t tok) {
  for (uint32_t k = 0; k < r.n_stop; ++k)
    if (cptr(r.stop)[k] == tok) return true;
  return false;
}

// Every op of a run in one launch. Every workgroup samples (same inputs, same
// code, same token), so no broadcast is needed. RANDOM: the run samples at a
// temperature above 0 (the host launches the instance that matches the run's
// temperature); the greedy instance holds none of the random sampler's code,
// whose registers would otherwise crowd the forward's.
template <bool RANDOM>
__global__ __launch_bounds__(BLOCK) void k_persistent(const Args* __restrict__ ap,
                                                      const RunDesc* __restrict__ run) {
  const Args& a = *ap;
  const Lds s = lds_init(a.d);
  const RunDesc r = *run;
  DevState* st = a.st;
  uint32_t pos = cptr(st)->pos, tick = cptr(st)->tick;
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  lm_prime(a, s);
  // The kinds whose rows of a layer fit in LDS are staged there: the loaders
  // request layer 0's QKV, O and GU rows now, where staged (the D rows follow
  // at the first QKV phase, as in every later layer).
  const Stager sg = make_stager(a, s, wg, G, a.d.lds_stg != 0);
  if (sg.on && sg.loader)
    for (uint32_t k = 0; k < 3; ++k)
      if (staged(sg, k)) stage_issue(sg, k, 0);
  uint32_t i = 0;
  uint32_t halted = 0;
  for (; i < r.n_ops; ++i) {
    uint32_t tok;
    if (i >= r.sample_from) {
      if constexpr (RANDOM) {
        const uint32_t word = cptr(r.words)[i - r.sample_from];
        const uint32_t gsum = r.samp_tag0 + (i - r.sample_from);
        float m;
        uint32_t bi;
        if (!sample_stage_a(a, tick, gsum, r.temperature, wg, G, s, &m, &bi)) break;
        if (!sample_exact(a, gsum, m, bi, word, wg, G, true, s, &tok)) break;
      } else if (!sample_greedy(a, tick, s, &tok)) {
        break;
      }
      if (r.mode == RUN_REPLAY) {
        if (tok != cptr(r.tokens)[i]) {
          if (wg == 0 && threadIdx.x == 0) {
            st->first_div = (long long)i;
            st->sampled_div = tok;
          }
          halted = 1;
          break;
        }
        tok = cptr(r.tokens)[i];
      } else if (wg == 0 && threadIdx.x == 0) {
        r.out_tokens[i] = tok;
      }
    } else {
      tok = cptr(r.tokens)[i];
    }
    if constexpr (RANDOM) {
      // The forward's LDS layout and stager formed afresh per token from
      // values the optimiser cannot see through, so nothing derived from
      // them is held across the sampler (whose registers would push it to
      // scratch, reloaded inside the forward).
      Dims dl = a.d;
      uint32_t wgt = wg;
      asm volatile("" : "+s"(dl.lds_vec), "+s"(dl.lds_vec2), "+s"(dl.lds_scr), "+s"(dl.lds_stg),
                   "+s"(dl.lds_pub), "+s"(wgt));
      extern __shared__ float lds_raw[];
      const Lds sf = lds_layout(lds_raw, dl);
      const Stager sgt = make_stager(a, sf, wgt, G, a.d.lds_stg != 0);
      if (!forward_all(a, tok, pos, tick, wgt, G, sf, sgt)) break;
    } else if (!forward_all(a, tok, pos, tick, wg, G, s, sg)) {
      break;
    }
    ++pos;
    ++tick;
    if (r.ring && r.mode == RUN_GENERATE && wg == 0 && threadIdx.x == 0) ring_commit(r.ring, i, tok);
    if (r.mode == RUN_GENERATE && is_stop(r, tok)) {
      ++i;
      halted = 1;
      break;
    }
  }
  if (wg == 0 && threadIdx.x == 0) {
    st->pos = pos;
    st->tick = tick;
    st->n_done = i;
    st->halt = halted;
  }
  // Staged loads of a layer that will not run land before the wave ends.
  if (sg.on && sg.loader) stage_wait(0);
}
template __global__ void k_persistent<false>(const Args* __restrict__, const RunDesc* __restrict__);
template __global__ void k_persistent<true>(const Args* __restrict__, const RunDesc* __restrict__);

}  // namespace DG_NS
