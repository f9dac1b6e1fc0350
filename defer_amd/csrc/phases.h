// phases.h -- the phases of one token's forward pass and the sampler, as
// workgroup-level device functions. Each takes (wg, G): the calling
// workgroup and how many workgroups share the phase. The persistent kernel
// runs them back to back; the per-phase kernels run one each. Work items are
// dealt round-robin (item = wg + G*k), and an item is always computed the
// same way whoever computes it.
#pragma once

#include "device.h"

namespace dg {

struct Lds {
  WaitCtl* ctl;
  float* red;  // 64 floats
  float* vec;  // d.lds_vec floats: the matvec input vector
  float* scr;  // d.lds_scr floats
};

__device__ inline Lds lds_layout(float* base, const Dims& d) {
  Lds s;
  s.ctl = reinterpret_cast<WaitCtl*>(base);
  s.red = base + 4;
  s.vec = base + 4 + 64;
  s.scr = s.vec + d.lds_vec;
  return s;
}

// One strided gather of tagged words: element e < seg_len * n_seg comes from
// src[(e / seg_len) * src_stride + e % seg_len] and goes to dst[e].
struct Gather {
  const u64* src;
  uint32_t seg_len, n_seg, src_stride, gen;
  float* dst;
};

__device__ inline Gather gather_vec(const u64* src, uint32_t n, uint32_t gen, float* dst) {
  Gather g;
  g.src = src;
  g.seg_len = n;
  g.n_seg = 1;
  g.src_stride = 0;
  g.gen = gen;
  g.dst = dst;
  return g;
}

// Block-wide wait for up to three gathers at once (one polling loop, so the
// round trips overlap). Returns false, uniformly, if the run was aborted.
__device__ bool wait_gather(const Gather* gs, uint32_t ng, DevState* st, WaitCtl* ctl) {
  const uint32_t tid = threadIdx.x;
  // The destination LDS may still be read by slower waves of the previous
  // phase: no wave writes it before every wave has arrived here.
  __syncthreads();
  uint32_t n[3] = {0, 0, 0};
  uint32_t total = 0;
  for (uint32_t k = 0; k < ng; ++k) {
    n[k] = gs[k].seg_len * gs[k].n_seg;
    total += n[k];
  }
  const uint32_t nk = (total + BLOCK - 1) / BLOCK;
  uint32_t pend = 0;
  for (uint32_t k = 0; k < nk && k < 32; ++k)
    if (tid + k * BLOCK < total) pend |= 1u << k;
  for (uint32_t spins = 0;; ++spins) {
    for (uint32_t k = 0; k < nk && k < 32; ++k) {
      if (!(pend & (1u << k))) continue;
      uint32_t e = tid + k * BLOCK;
      uint32_t which = 0;
      while (which + 1 < ng && e >= n[which]) {
        e -= n[which];
        ++which;
      }
      const Gather& g = gs[which];
      const uint32_t seg = e / g.seg_len, off = e - seg * g.seg_len;
      const u64 w = mb_load(g.src + (size_t)seg * g.src_stride + off);
      if ((uint32_t)(w >> 32) == g.gen) {
        g.dst[e] = __uint_as_float((uint32_t)w);
        pend &= ~(1u << k);
      }
    }
    if (tid == 0) {
      if (spins >= SPIN_LIMIT) {
        st_coherent_u32(&st->abort, 1u);
        ctl->abort_seen = 1;
      } else if ((spins & 63) == 63 && ld_coherent_u32(&st->abort)) {
        ctl->abort_seen = 1;
      }
    }
    const int pending = __syncthreads_count(pend != 0);
    if (ctl->abort_seen) return false;
    if (pending == 0) {
      __syncthreads();
      return true;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// In-place RMSNorm of v[0..n) in LDS (ops.rs:84-95): inv = 1/sqrt(ss/n + eps),
// out = x * inv * w. ss is a fixed-tree sum.
__device__ void rmsnorm_lds(float* v, const float* __restrict__ w, uint32_t n, float eps,
                            float* red) {
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < n; i += BLOCK) ss = fmaf(v[i], v[i], ss);
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n; i += BLOCK) v[i] = v[i] * inv * w[i];
  __syncthreads();
}

// x entering layer l: the embedding row (model.rs:428) or the last MLP output.
__device__ bool load_x(const Args& a, uint32_t l, uint32_t tick, uint32_t token, float* dst,
                       const Lds& s) {
  const Dims& d = a.d;
  if (l == 0) {
    __syncthreads();  // dst may still be read by the previous phase
    const float* e = a.embed + (size_t)token * d.h;
    for (uint32_t i = threadIdx.x; i < d.h; i += BLOCK) dst[i] = e[i];
    __syncthreads();
    return true;
  }
  Gather g = gather_vec(a.mb_xd, d.h, gen_of(d, tick, l - 1, PH_D), dst);
  return wait_gather(&g, 1, a.st, s.ctl);
}

// ------------------------------------------------------------------ QKV

// rmsnorm -> q/k/v rows (+bias) -> RoPE on q and k (model.rs:460-465) ->
// k, v appended to the cache at `pos` (model.rs:466-467). Work item = a pair
// of rows (i, i + hd/2) of one head, so RoPE needs no exchange.
__device__ bool phase_qkv(const Args& a, uint32_t l, uint32_t tick, uint32_t pos, uint32_t token,
                          uint32_t wg, uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  const LayerW& W = a.layers[l];
  if (!load_x(a, l, tick, token, s.vec, s)) return false;
  rmsnorm_lds(s.vec, W.attn_norm, d.h, d.eps, s.red);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t P = d.qkv_rows / 2;
  const uint32_t gen = gen_of(d, tick, l, PH_QKV);
  const float2* rp = a.rope + (size_t)pos * d.half;
  for (uint32_t k = wave; wg + G * k < P; k += NWAVES) {
    const uint32_t p = wg + G * k;
    const uint32_t hb = p / d.half, i = p - hb * d.half;
    const uint32_t r0 = hb * d.hd + i, r1 = r0 + d.half;
    const float p0 = dot_partial(W.wqkv + (size_t)r0 * d.h, s.vec, d.h, lane);
    const float p1 = dot_partial(W.wqkv + (size_t)r1 * d.h, s.vec, d.h, lane);
    float y0 = wave_sum(p0), y1 = wave_sum(p1);
    if (W.bqkv) {
      y0 += W.bqkv[r0];
      y1 += W.bqkv[r1];
    }
    if (hb < d.nh + d.nkv) {
      const float2 cs = rp[i];
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
  }
  return true;
}

// ------------------------------------------------------------ attention

constexpr uint32_t MAX_GROUP = 8;

// Split-context attention for one (kv head, chunk) item: scores, softmax
// partials (max m, sum l, unnormalised acc) for each query head of the GQA
// group (model.rs:471-497). K/V rows of the chunk are read once per group.
__device__ bool phase_attn(const Args& a, uint32_t l, uint32_t tick, uint32_t pos, uint32_t wg,
                           uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  const uint32_t nch = attn_nchunks(pos), CH = attn_chunk(pos);
  const uint32_t n_items = d.nkv * nch;
  const uint32_t gen_in = gen_of(d, tick, l, PH_QKV);
  const uint32_t gen_out = gen_of(d, tick, l, PH_ATTN);
  const uint32_t hd = d.hd, grp = d.group, hs = hd + 2;
  float* qs = s.scr;            // [grp*hd]
  float* kn = qs + grp * hd;    // [hd]
  float* vn = kn + hd;          // [hd]
  float* wp = vn + hd;          // [NWAVES][grp][hd+2]
  const uint32_t LP = hd / 4, PPI = WAVE / LP, NG = NWAVES * PPI;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t sub = lane % LP;
  const uint32_t gi = wave * PPI + lane / LP;
  for (uint32_t item = wg; item < n_items; item += G) {
    const uint32_t g = item / nch, c = item - g * nch;
    const uint32_t t0 = c * CH;
    const uint32_t t1 = min(t0 + CH, pos + 1);
    Gather gs[3];
    gs[0] = gather_vec(a.mb_qkv + (size_t)g * grp * hd, grp * hd, gen_in, qs);
    gs[1] = gather_vec(a.mb_qkv + d.q + g * hd, hd, gen_in, kn);
    gs[2] = gather_vec(a.mb_qkv + d.q + d.kv + g * hd, hd, gen_in, vn);
    if (!wait_gather(gs, 3, a.st, s.ctl)) return false;
    const float* kb = a.kc + ((size_t)l * d.nkv + g) * d.cap * d.kvs;
    const float* vb = a.vc + ((size_t)l * d.nkv + g) * d.cap * d.kvs;
    float m[MAX_GROUP], ls[MAX_GROUP], acc[MAX_GROUP][4];
#pragma unroll
    for (uint32_t j = 0; j < MAX_GROUP; ++j) {
      m[j] = -INFINITY;
      ls[j] = 0.0f;
      acc[j][0] = acc[j][1] = acc[j][2] = acc[j][3] = 0.0f;
    }
    for (uint32_t t = t0 + gi; t < t1; t += NG) {
      const bool cur = (t == pos);
      const float4 kk = cur ? ld4(kn + sub * 4) : ld4(kb + (size_t)t * d.kvs + sub * 4);
      const float4 vv = cur ? ld4(vn + sub * 4) : ld4(vb + (size_t)t * d.kvs + sub * 4);
      const bool masked = a.mask && t < pos && ((a.mask[t >> 5] >> (t & 31)) & 1u);
#pragma unroll
      for (uint32_t j = 0; j < MAX_GROUP; ++j) {
        if (j >= grp) break;
        const float4 qq = ld4(qs + j * hd + sub * 4);
        float p = qq.x * kk.x;
        p = fmaf(qq.y, kk.y, p);
        p = fmaf(qq.z, kk.z, p);
        p = fmaf(qq.w, kk.w, p);
        for (uint32_t o = LP / 2; o > 0; o >>= 1) p += __shfl_xor(p, o);
        const float sc = masked ? -INFINITY : p * d.scale;
        if (sc > m[j]) {
          const float r = (m[j] == -INFINITY) ? 0.0f : expf(m[j] - sc);
          ls[j] *= r;
          acc[j][0] *= r;
          acc[j][1] *= r;
          acc[j][2] *= r;
          acc[j][3] *= r;
          m[j] = sc;
        }
        const float e = (sc == -INFINITY) ? 0.0f : expf(sc - m[j]);
        ls[j] += e;
        acc[j][0] = fmaf(e, vv.x, acc[j][0]);
        acc[j][1] = fmaf(e, vv.y, acc[j][1]);
        acc[j][2] = fmaf(e, vv.z, acc[j][2]);
        acc[j][3] = fmaf(e, vv.w, acc[j][3]);
      }
    }
    // Merge the position groups of this wave (lanes with the same `sub`).
#pragma unroll
    for (uint32_t j = 0; j < MAX_GROUP; ++j) {
      if (j >= grp) break;
      for (uint32_t o = LP; o < WAVE; o <<= 1) {
        const float m2 = __shfl_xor(m[j], o), l2 = __shfl_xor(ls[j], o);
        const float b0 = __shfl_xor(acc[j][0], o), b1 = __shfl_xor(acc[j][1], o);
        const float b2 = __shfl_xor(acc[j][2], o), b3 = __shfl_xor(acc[j][3], o);
        const float mn = fmaxf(m[j], m2);
        const float s1 = (m[j] == -INFINITY) ? 0.0f : expf(m[j] - mn);
        const float s2 = (m2 == -INFINITY) ? 0.0f : expf(m2 - mn);
        ls[j] = ls[j] * s1 + l2 * s2;
        acc[j][0] = acc[j][0] * s1 + b0 * s2;
        acc[j][1] = acc[j][1] * s1 + b1 * s2;
        acc[j][2] = acc[j][2] * s1 + b2 * s2;
        acc[j][3] = acc[j][3] * s1 + b3 * s2;
        m[j] = mn;
      }
      if (lane < LP) {
        float* dst = wp + (wave * grp + j) * hs;
        if (lane == 0) {
          dst[0] = m[j];
          dst[1] = ls[j];
        }
        dst[2 + sub * 4 + 0] = acc[j][0];
        dst[2 + sub * 4 + 1] = acc[j][1];
        dst[2 + sub * 4 + 2] = acc[j][2];
        dst[2 + sub * 4 + 3] = acc[j][3];
      }
    }
    __syncthreads();
    // Merge the waves in wave order and publish the chunk's partials.
    for (uint32_t u = threadIdx.x; u < grp * hd; u += BLOCK) {
      const uint32_t j = u / hd, dd = u - j * hd;
      float M = -INFINITY;
      for (uint32_t w = 0; w < NWAVES; ++w) M = fmaxf(M, wp[(w * grp + j) * hs]);
      float Ls = 0.0f, A = 0.0f;
      for (uint32_t w = 0; w < NWAVES; ++w) {
        const float* src = wp + (w * grp + j) * hs;
        const float sw = (src[0] == -INFINITY) ? 0.0f : expf(src[0] - M);
        Ls = Ls + src[1] * sw;
        A = A + src[2 + dd] * sw;
      }
      const uint32_t hh = g * grp + j;
      u64* out = a.mb_part + ((size_t)hh * MAX_ACHUNKS + c) * hs;
      mb_put(out + 2 + dd, A, gen_out);
      if (dd == 0) {
        mb_put(out + 0, M, gen_out);
        mb_put(out + 1, Ls, gen_out);
      }
    }
    __syncthreads();
  }
  return true;
}

// Combine the chunk partials of one head (in chunk order) into its output:
// att[d] = sum_c acc_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M).
__device__ __forceinline__ float combine_one(const float* part, uint32_t nch, uint32_t hs,
                                             uint32_t dd) {
  float M = -INFINITY;
  for (uint32_t c = 0; c < nch; ++c) M = fmaxf(M, part[c * hs]);
  float Ls = 0.0f, A = 0.0f;
  for (uint32_t c = 0; c < nch; ++c) {
    const float* p = part + c * hs;
    const float sc = (p[0] == -INFINITY) ? 0.0f : expf(p[0] - M);
    Ls = Ls + p[1] * sc;
    A = A + p[2 + dd] * sc;
  }
  return A / Ls;
}

// Separate combine (used when the partials of all heads do not fit the O
// phase's LDS budget): item = one query head.
__device__ bool phase_comb(const Args& a, uint32_t l, uint32_t tick, uint32_t pos, uint32_t wg,
                           uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  if (comb_inline(d, pos)) return true;
  const uint32_t nch = attn_nchunks(pos), hs = d.hd + 2;
  const uint32_t gen_in = gen_of(d, tick, l, PH_ATTN), gen_out = gen_of(d, tick, l, PH_COMB);
  for (uint32_t hh = wg; hh < d.nh; hh += G) {
    Gather g = gather_vec(a.mb_part + (size_t)hh * MAX_ACHUNKS * hs, nch * hs, gen_in, s.scr);
    if (!wait_gather(&g, 1, a.st, s.ctl)) return false;
    for (uint32_t dd = threadIdx.x; dd < d.hd; dd += BLOCK)
      mb_put(a.mb_att + hh * d.hd + dd, combine_one(s.scr, nch, hs, dd), gen_out);
    __syncthreads();
  }
  return true;
}

// Number of rows r = wg + G*k below n owned by this workgroup.
__device__ __forceinline__ uint32_t rows_owned(uint32_t n, uint32_t wg, uint32_t G) {
  return wg < n ? (n - wg + G - 1) / G : 0;
}

// ------------------------------------------------------------ O projection

// x_o = x + Wo . att (model.rs:498-499), with the attention combine done
// in the prologue when it fits.
__device__ bool phase_o(const Args& a, uint32_t l, uint32_t tick, uint32_t pos, uint32_t token,
                        uint32_t wg, uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  const LayerW& W = a.layers[l];
  const uint32_t nch = attn_nchunks(pos), hs = d.hd + 2;
  const bool inl = comb_inline(d, pos);
  const uint32_t R = rows_owned(d.h, wg, G);
  float* part = s.scr;
  float* xres = s.scr + (inl ? d.nh * nch * hs : 0);
  Gather gs[2];
  uint32_t ng = 0;
  if (inl)
    gs[ng++] = {a.mb_part, nch * hs, d.nh, MAX_ACHUNKS * hs, gen_of(d, tick, l, PH_ATTN), part};
  else
    gs[ng++] = gather_vec(a.mb_att, d.q, gen_of(d, tick, l, PH_COMB), s.vec);
  if (l > 0 && R > 0) gs[ng++] = {a.mb_xd + wg, 1, R, G, gen_of(d, tick, l - 1, PH_D), xres};
  if (!wait_gather(gs, ng, a.st, s.ctl)) return false;
  if (l == 0)
    for (uint32_t k = threadIdx.x; k < R; k += BLOCK)
      xres[k] = a.embed[(size_t)token * d.h + wg + G * k];
  if (inl)
    for (uint32_t u = threadIdx.x; u < d.q; u += BLOCK) {
      const uint32_t hh = u / d.hd, dd = u - hh * d.hd;
      s.vec[u] = combine_one(part + hh * nch * hs, nch, hs, dd);
    }
  __syncthreads();
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t gen = gen_of(d, tick, l, PH_O);
  for (uint32_t k = wave; k < R; k += NWAVES) {
    const uint32_t i = wg + G * k;
    const float y = dot_row(W.wo + (size_t)i * d.q, s.vec, d.q, lane);
    if (lane == 0) mb_put(a.mb_xo + i, xres[k] + y, gen);
  }
  return true;
}

// ------------------------------------------------------------ MLP

// rmsnorm -> g = act(Wg.x) * (Wu.x) (model.rs:502-509).
__device__ bool phase_gu(const Args& a, uint32_t l, uint32_t tick, uint32_t wg, uint32_t G,
                         const Lds& s) {
  const Dims& d = a.d;
  const LayerW& W = a.layers[l];
  Gather g = gather_vec(a.mb_xo, d.h, gen_of(d, tick, l, PH_O), s.vec);
  if (!wait_gather(&g, 1, a.st, s.ctl)) return false;
  rmsnorm_lds(s.vec, W.ffn_norm, d.h, d.eps, s.red);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t gen = gen_of(d, tick, l, PH_GU);
  for (uint32_t k = wave; wg + G * k < d.ff; k += NWAVES) {
    const uint32_t j = wg + G * k;
    const float pg = dot_partial(W.wg + (size_t)j * d.h, s.vec, d.h, lane);
    const float pu = dot_partial(W.wu + (size_t)j * d.h, s.vec, d.h, lane);
    const float gate = wave_sum(pg), up = wave_sum(pu);
    if (lane == 0) mb_put(a.mb_g + j, act_fn(gate, d.act) * up, gen);
  }
  return true;
}

// x_d = x_o + Wd . g (model.rs:510-511).
__device__ bool phase_d(const Args& a, uint32_t l, uint32_t tick, uint32_t wg, uint32_t G,
                        const Lds& s) {
  const Dims& d = a.d;
  const LayerW& W = a.layers[l];
  const uint32_t R = rows_owned(d.h, wg, G);
  Gather gs[2];
  uint32_t ng = 0;
  gs[ng++] = gather_vec(a.mb_g, d.ff, gen_of(d, tick, l, PH_GU), s.vec);
  if (R > 0) gs[ng++] = {a.mb_xo + wg, 1, R, G, gen_of(d, tick, l, PH_O), s.scr};
  if (!wait_gather(gs, ng, a.st, s.ctl)) return false;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t gen = gen_of(d, tick, l, PH_D);
  for (uint32_t k = wave; k < R; k += NWAVES) {
    const uint32_t i = wg + G * k;
    const float y = dot_row(W.wd + (size_t)i * d.ff, s.vec, d.ff, lane);
    if (lane == 0) mb_put(a.mb_xd + i, s.scr[k] + y, gen);
  }
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

// rmsnorm(final) -> logits = H . x (model.rs:515-519), plus each vocabulary
// chunk's (max, argmax) for the sampler.
__device__ bool phase_lm(const Args& a, uint32_t tick, uint32_t wg, uint32_t G, const Lds& s) {
  const Dims& d = a.d;
  Gather g = gather_vec(a.mb_xd, d.h, gen_of(d, tick, d.L - 1, PH_D), s.vec);
  if (!wait_gather(&g, 1, a.st, s.ctl)) return false;
  rmsnorm_lds(s.vec, a.norm, d.h, d.eps, s.red);
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t gen = gen_lm(d, tick);
  float* wbest = s.scr;  // [NWAVES] values, then [NWAVES] indices
  for (uint32_t c = wg; c < d.nvc; c += G) {
    const uint32_t v0 = c * VCHUNK, v1 = min(v0 + VCHUNK, d.V);
    float bv = -INFINITY;
    uint32_t bi = NO_INDEX;
    uint32_t v = v0 + wave;
    for (; v + 3 * NWAVES < v1; v += 4 * NWAVES) {
      const float p0 = dot_partial(a.head + (size_t)v * d.h, s.vec, d.h, lane);
      const float p1 = dot_partial(a.head + (size_t)(v + NWAVES) * d.h, s.vec, d.h, lane);
      const float p2 = dot_partial(a.head + (size_t)(v + 2 * NWAVES) * d.h, s.vec, d.h, lane);
      const float p3 = dot_partial(a.head + (size_t)(v + 3 * NWAVES) * d.h, s.vec, d.h, lane);
      const float y0 = wave_sum(p0), y1 = wave_sum(p1), y2 = wave_sum(p2), y3 = wave_sum(p3);
      if (lane == 0) {
        mb_put(a.mb_logit + v, y0, gen);
        mb_put(a.mb_logit + v + NWAVES, y1, gen);
        mb_put(a.mb_logit + v + 2 * NWAVES, y2, gen);
        mb_put(a.mb_logit + v + 3 * NWAVES, y3, gen);
      }
      if (!isnan(y0) && better(y0, v, bv, bi)) { bv = y0; bi = v; }
      if (!isnan(y1) && better(y1, v + NWAVES, bv, bi)) { bv = y1; bi = v + NWAVES; }
      if (!isnan(y2) && better(y2, v + 2 * NWAVES, bv, bi)) { bv = y2; bi = v + 2 * NWAVES; }
      if (!isnan(y3) && better(y3, v + 3 * NWAVES, bv, bi)) { bv = y3; bi = v + 3 * NWAVES; }
    }
    for (; v < v1; v += NWAVES) {
      const float y = dot_row(a.head + (size_t)v * d.h, s.vec, d.h, lane);
      if (lane == 0) mb_put(a.mb_logit + v, y, gen);
      if (!isnan(y) && better(y, v, bv, bi)) { bv = y; bi = v; }
    }
    if (lane == 0) {
      wbest[wave] = bv;
      reinterpret_cast<uint32_t*>(wbest)[NWAVES + wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float cv = -INFINITY;
      uint32_t ci = NO_INDEX;
      for (uint32_t w = 0; w < NWAVES; ++w) {
        const float wv = wbest[w];
        const uint32_t wi = reinterpret_cast<const uint32_t*>(wbest)[NWAVES + w];
        if (better(wv, wi, cv, ci)) { cv = wv; ci = wi; }
      }
      mb_put(a.mb_vmax + c, cv, gen);
      mb_put(a.mb_varg + c, __uint_as_float(ci), gen);
    }
    __syncthreads();
  }
  return true;
}

// ------------------------------------------------------------ sampler

// Global (max, argmax) over the chunk partials already in LDS.
__device__ void global_argmax(const float* vmx, const float* varg, uint32_t nvc, float* red,
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
__device__ bool sample_stage_a(const Args& a, uint32_t tick, float T, uint32_t wg, uint32_t G,
                               const Lds& s) {
  const Dims& d = a.d;
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u), gsum = gen_sums(d, tick);
  float* vmx = s.scr;
  float* varg = vmx + nvc;
  float* chunk = varg + nvc;  // [NWAVES][VCHUNK]
  Gather gs[2] = {gather_vec(a.mb_vmax, nvc, gl, vmx), gather_vec(a.mb_varg, nvc, gl, varg)};
  if (!wait_gather(gs, 2, a.st, s.ctl)) return false;
  float bv;
  uint32_t bi;
  global_argmax(vmx, varg, nvc, s.red, &bv, &bi);
  const float m = (bi == NO_INDEX) ? -INFINITY : bv / T;
  const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint32_t nown = wg < nvc ? (nvc - wg + G - 1) / G : 0;
  for (uint32_t k0 = 0; k0 < nown; k0 += NWAVES) {
    const uint32_t nb = min(NWAVES, nown - k0);
    // chunks wg + G*(k0 + b), b < nb; the last one may be short
    Gather g = {a.mb_logit + (size_t)(wg + G * k0) * VCHUNK, VCHUNK, nb, G * VCHUNK, gl, chunk};
    const uint32_t clast = wg + G * (k0 + nb - 1);
    if ((clast + 1) * VCHUNK > d.V) {
      // short last chunk: gather it separately so no slot past V is read
      Gather g2[2];
      uint32_t ng = 0;
      if (nb > 1) g2[ng++] = {g.src, VCHUNK, nb - 1, G * VCHUNK, gl, chunk};
      g2[ng++] = gather_vec(a.mb_logit + (size_t)clast * VCHUNK, d.V - clast * VCHUNK, gl,
                            chunk + (nb - 1) * VCHUNK);
      if (!wait_gather(g2, ng, a.st, s.ctl)) return false;
    } else if (!wait_gather(&g, 1, a.st, s.ctl)) {
      return false;
    }
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
__device__ bool sample_stage_b(const Args& a, uint32_t tick, float T, uint32_t word,
                               const Lds& s, uint32_t* tok_out) {
  const Dims& d = a.d;
  const uint32_t nvc = d.nvc;
  const uint32_t gl = gen_lm(d, tick - 1u), gsum = gen_sums(d, tick);
  float* vmx = s.scr;
  float* varg = vmx + nvc;
  float* vsum = varg + nvc;
  float* chunk = vsum + nvc;  // [VCHUNK]
  float* wtot = chunk + VCHUNK;  // [NWAVES + 2]
  Gather gs[3];
  uint32_t ng = 0;
  gs[ng++] = gather_vec(a.mb_vmax, nvc, gl, vmx);
  gs[ng++] = gather_vec(a.mb_varg, nvc, gl, varg);
  if (T != 0.0f) gs[ng++] = gather_vec(a.mb_vsum, nvc, gsum, vsum);
  if (!wait_gather(gs, ng, a.st, s.ctl)) return false;
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
    Gather g = gather_vec(a.mb_logit + v0, nv, gl, chunk);
    if (!wait_gather(&g, 1, a.st, s.ctl)) return false;
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
    Gather g = gather_vec(a.mb_logit + v0, nv, gl, chunk);
    if (!wait_gather(&g, 1, a.st, s.ctl)) return false;
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
