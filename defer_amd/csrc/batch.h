// batch.h -- the batched forward: B rows, each a (cache, position, token),
// step through the model together and every matrix product is an MFMA GEMM.
//
// Batch invariance. Every output element of every matrix product is computed
// in the one order the one-token path uses (device.h, "Row dot products"):
// 16 segments s, segment s holding the elements 64*i + 4*s + c (i
// ascending, c = 0..3), each segment a chain of fused multiply-adds from +0,
// then the complete binary tree over the 16 segment sums.
// v_mfma_f32_16x16x4_f32 computes, for each output, exactly
// fma(a3,b3,fma(a2,b2,fma(a1,b1,fma(a0,b0,c)))) -- four links of such a
// chain -- so chaining one MFMA per chunk reproduces a segment's sum bit for
// bit, and the tree is then formed from the 16 segment accumulators. The
// result of a row depends on that row's inputs only: not on B, not on the
// other rows, not on the tiling. Everything else a row goes through
// (RMSNorm, RoPE, attention, combine, residuals, activation, sampling) runs
// the same expressions as the one-token path, or the very same functions.
#pragma once

#include "phases.h"

namespace dg {

typedef float f4v __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ panel layout
//
// GEMM operands are stored as panels: a matrix of R rows and K columns
// becomes [ceil(R/16)][nch = ceil(K/64)][4 quarters][64 lanes][4 floats],
// float u of quarter q of lane l = r + 16c in chunk i of tile T holding
// element (16*T + r, 64*i + 4*(4q + u) + c), zero outside the matrix. Lane l's
// float u of quarter q is its MFMA operand (A for weights, B for activations)
// of segment 4q + u; a (tile, chunk) is 4 KB, each quarter 1 KB contiguous,
// so one 16-byte-per-lane load moves a quarter, and lanes read LDS copies of
// it at consecutive addresses.

constexpr uint32_t PANEL_TILE = 1024;  // floats per (16-row tile, chunk)

__host__ __device__ inline uint32_t panel_chunks(uint32_t K) { return (K + 63) / 64; }
__host__ __device__ inline size_t panel_floats(uint32_t R, uint32_t K) {
  return (size_t)((R + 15) / 16) * panel_chunks(K) * PANEL_TILE;
}

// Position of element (row r, column k) in a panel of nch chunks.
__host__ __device__ inline size_t panel_at(uint32_t r, uint32_t k, uint32_t nch) {
  const uint32_t i = k / 64, s = (k % 64) / 4, c = k % 4;
  return (((size_t)(r / 16) * nch + i) * 4 + s / 4) * 256 + ((r % 16) + 16 * c) * 4 + s % 4;
}

// Rows [0, R0) from src0, rows [R0, R) from src1 (row r - R0): a stacked
// matrix without a stacked copy. ld: row stride of both sources.
__global__ void k_to_panel(const float* __restrict__ src0, const float* __restrict__ src1,
                           uint32_t R0, uint32_t R, uint32_t K, uint32_t ld,
                           float* __restrict__ dst) {
  const size_t n = panel_floats(R, K);
  const uint32_t nch = panel_chunks(K);
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < n;
       e += (size_t)gridDim.x * blockDim.x) {
    const uint32_t u = (uint32_t)(e % 4), l = (uint32_t)((e / 4) % 64),
                   q = (uint32_t)((e / 256) % 4);
    const size_t rest = e / PANEL_TILE;
    const uint32_t i = (uint32_t)(rest % nch);
    const size_t r = (rest / nch) * 16 + l % 16;
    const uint32_t k = 64 * i + 4 * (4 * q + u) + l / 16;
    float v = 0.0f;
    if (r < R && k < K) v = r < R0 ? src0[r * ld + k] : src1[(r - R0) * ld + k];
    dst[e] = v;
  }
}

// ------------------------------------------------------------------ GEMM

enum GemmOut : uint32_t {
  GO_PLAIN = 0,  // Y[b][o] = y
  GO_RESID = 1,  // Y[b][o] = Y[b][o] + y   (the residual stream, in place; also into panel P)
  GO_TAG = 2,    // T[b][o] = tag(gen[b], scale[b] * y)  (tagged logits)
};

// Complete binary tree over 16 values in index order.
__device__ __forceinline__ f4v tree16(const f4v* a) {
  f4v p[8], q[4];
#pragma unroll
  for (int k = 0; k < 8; ++k) p[k] = a[2 * k] + a[2 * k + 1];
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = p[2 * k] + p[2 * k + 1];
  return (q[0] + q[1]) + (q[2] + q[3]);
}

// Chunks of operands in flight through LDS, and the LDS a launch needs.
// Four-tile tasks take a CU's LDS alone; smaller ones fit two workgroups
// per CU with three stages.
__host__ __device__ constexpr uint32_t gemm_stages(uint32_t tn) { return tn == 4 ? 4 : 3; }
__host__ __device__ constexpr uint32_t gemm_lds_bytes(uint32_t tn) {
  return gemm_stages(tn) * (4 + tn) * PANEL_TILE * 4;
}
constexpr uint32_t GEMM_WAVES = 8;

// Y[b][o] = W[o] . X[b] for o < M, b < B, K columns. A task (x, y) covers
// row tiles 4x .. 4x+3 and column tiles cbase + y*TN .. cbase + y*TN+TN-1.
// Eight waves, two per SIMD, so one wave's MFMAs run while the other waits
// for its operands: wave w owns row tile 4x + w%4 and column tiles
// (w/4)*TN/2 .. of the task (TN = 1: the waves w < 4 only), all 16
// segments of each of its outputs in its own accumulators, reduced with
// tree16 at the end. A chunk's operands (the four row tiles and the TN
// column tiles, 4 KB each) are copied into LDS by the waves together (16
// bytes per lane straight from memory into LDS), gemm_stages(TN) - 1 chunks
// ahead of their use, so each tile is read from memory once per workgroup.
// The kernel is persistent: workgroup k takes tasks k, k + gridDim.x, ...,
// and the copies run ahead across task boundaries. PARTIAL: K may end
// inside a chunk.
template <int TN, uint32_t OUT, bool PARTIAL>
__global__ __launch_bounds__(512) void k_gemm(const float* __restrict__ Wp, uint32_t M, uint32_t K,
                                              const float* __restrict__ Xp, uint32_t B,
                                              float* __restrict__ Y, uint32_t ldy,
                                              const float* __restrict__ scale,
                                              const uint32_t* __restrict__ gen, uint32_t cbase,
                                              uint32_t ncols, float* __restrict__ P) {
  extern __shared__ float4 gsm[];  // [stages][4 + TN tiles][4 quarters][64 lanes]
  constexpr uint32_t GEMM_STAGES = gemm_stages(TN);
  constexpr uint32_t NT = 4 + TN;                    // tiles per stage
  constexpr uint32_t WN = TN >= 2 ? TN / 2 : 1;      // column tiles per wave
  constexpr uint32_t NQ = 4 * NT;                    // 1 KB copies per stage
  // The wave index is uniform: scalar registers and branches for it.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
  const uint32_t rt = wave % 4, half = wave / 4;
  const bool mfma_wave = TN >= 2 || half == 0;
  const uint32_t nld = (NQ - wave + GEMM_WAVES - 1) / GEMM_WAVES;  // this wave's copies per stage
  const uint32_t gdx = gridDim.x;  // kept in a register (a reload would wait for every LDS read)
  const uint32_t nch = panel_chunks(K), nrt = (M + 15) / 16, nct = (B + 15) / 16;
  const uint32_t nrg = (nrt + 3) / 4, ngy = (ncols + TN - 1) / TN, ntask = nrg * ngy;
  const uint32_t mine = blockIdx.x < ntask ? (ntask - blockIdx.x + gdx - 1) / gdx : 0;
  const uint32_t total = mine * nch;  // chunks of this workgroup's tasks, in order
  const uint32_t lds0 = (uint32_t)(uintptr_t)gsm;
  // The copies run ahead of the MFMAs through the workgroup's chunks in
  // order: chunk ci of task ct is next. A wave's copies of a stage are
  // entries wave, wave + 8, ... of the stage's (tile, quarter) list; cb[j]
  // is the tile of its copy j in task ct (tiles past the last one load a
  // real tile, never used, so a wave issues the same number of copies for
  // every chunk). Only a new task divides.
  constexpr uint32_t MAXJ = (NQ + GEMM_WAVES - 1) / GEMM_WAVES;
  uint32_t ct = blockIdx.x, ci = 0;
  const float* cb[MAXJ];
  auto set_task = [&]() {
    const uint32_t x = ct % nrg, C0 = cbase + (ct / nrg) * TN;
#pragma unroll
    for (uint32_t j = 0; j < MAXJ; ++j) {
      const uint32_t tile = (wave + GEMM_WAVES * j) / 4;
      cb[j] = tile < 4 ? Wp + (size_t)min(4 * x + tile, nrt - 1) * nch * PANEL_TILE
                       : Xp + (size_t)min(C0 + tile - 4, nct - 1) * nch * PANEL_TILE;
    }
  };
  set_task();
  // The next chunk into stage st.
  auto issue = [&](uint32_t st) {
    const uint32_t sb = lds0 + st * NT * PANEL_TILE * 4;
#pragma unroll
    for (uint32_t j = 0; j < MAXJ; ++j) {
      const uint32_t f = wave + GEMM_WAVES * j;
      if (f < NQ) dma16(cb[j] + (size_t)ci * PANEL_TILE + (f % 4) * 256 + lane * 4, sb + f * 1024);
    }
    if (++ci == nch) {
      ci = 0;
      ct += gdx;
      set_task();
    }
  };
  for (uint32_t g = 0; g + 1 < GEMM_STAGES && g < total; ++g) issue(g);
  for (uint32_t k = 0; k < mine; ++k) {
    f4v acc[WN][16];
#pragma unroll
    for (int t = 0; t < (int)WN; ++t)
#pragma unroll
      for (int s = 0; s < 16; ++s) acc[t][s] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    // Chunk i of this task from its stage, once it has landed: chunk g has
    // landed once at most the later chunks' copies are in flight; the
    // barrier makes that true of every wave, and every wave is then done
    // with chunk g - 1's stage, which the next request overwrites.
    auto operands = [&](uint32_t i, float4 (&a)[4], float4 (&b)[WN][4]) {
      const uint32_t g = k * nch + i;
      stage_wait(min(GEMM_STAGES - 2, total - 1 - g) * nld);
      __syncthreads();
      if (g + GEMM_STAGES - 1 < total) issue((g + GEMM_STAGES - 1) % GEMM_STAGES);
      const float4* sa = gsm + (g % GEMM_STAGES) * NT * 256;
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] = sa[(rt * 4 + q) * 64 + lane];
#pragma unroll
      for (int t = 0; t < (int)WN; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) b[t][q] = sa[((4 + half * WN + t) * 4 + q) * 64 + lane];
    };
    const uint32_t nfull = K / 64;
    for (uint32_t i = 0; i < nfull; ++i) {
      float4 a[4], b[WN][4];
      operands(i, a, b);
      if (!mfma_wave) continue;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float av = (&a[s / 4].x)[s % 4];
#pragma unroll
        for (int t = 0; t < (int)WN; ++t)
          acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, (&b[t][s / 4].x)[s % 4], acc[t][s],
                                                           0, 0, 0);
      }
    }
    if (PARTIAL && nfull < nch) {
      // A last, partial chunk: the segments past K are left alone (their
      // zero padding would still turn a -0 sum into +0).
      float4 a[4], b[WN][4];
      operands(nfull, a, b);
      const uint32_t ns = (K - 64 * nfull) / 4;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        if ((uint32_t)s < ns && mfma_wave) {
          const float av = (&a[s / 4].x)[s % 4];
#pragma unroll
          for (int t = 0; t < (int)WN; ++t)
            acc[t][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, (&b[t][s / 4].x)[s % 4],
                                                             acc[t][s], 0, 0, 0);
        }
      }
    }
    // The task's outputs, one tile at a time.
    const uint32_t tk = blockIdx.x + gdx * k;
    const uint32_t T = 4 * (tk % nrg) + rt, C0 = cbase + (tk / nrg) * TN + half * WN;
#pragma unroll
    for (int t = 0; t < (int)WN; ++t) {
      __builtin_amdgcn_sched_barrier(0);
      const f4v r = tree16(acc[t]);
      const uint32_t b = (C0 + t) * 16 + lane % 16;
      const uint32_t o = T * 16 + 4 * (lane / 16);
      if (!mfma_wave || T >= nrt || C0 + t >= cbase + ncols || b >= B) continue;
      const size_t at = (size_t)b * ldy + o;
      const uint32_t nchp = panel_chunks(M);  // the residual's panel: K = M
      if (OUT != GO_TAG && o + 4 <= M && (at & 3) == 0) {
        float4* y4 = reinterpret_cast<float4*>(Y + at);
        float4 v = make_float4(r[0], r[1], r[2], r[3]);
        if (OUT == GO_RESID) {
          const float4 old = *y4;
          v = make_float4(old.x + r[0], old.y + r[1], old.z + r[2], old.w + r[3]);
          P[panel_at(b, o, nchp)] = v.x;
          P[panel_at(b, o + 1, nchp)] = v.y;
          P[panel_at(b, o + 2, nchp)] = v.z;
          P[panel_at(b, o + 3, nchp)] = v.w;
        }
        *y4 = v;
        continue;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (o + j >= M) continue;
        if (OUT == GO_PLAIN) {
          Y[at + j] = r[j];
        } else if (OUT == GO_RESID) {
          const float v = Y[at + j] + r[j];
          Y[at + j] = v;
          P[panel_at(b, o + j, nchp)] = v;
        } else {
          const float v = scale[b] * r[j];
          reinterpret_cast<u64*>(Y)[at + j] = ((u64)gen[b] << 32) | (u64)__float_as_uint(v);
        }
      }
    }
  }
}

// The same product for narrow batches (at most four column tiles, B <= 64):
// a task is one row tile with every column tile, so there are enough tasks
// to stream the weights through every CU. Wave w computes column tile w % 4
// over segments 8h .. 8h+7 (h = w / 4) and forms their subtree; the two
// halves meet in LDS as (s0..s7) + (s8..s15) -- the same tree16.
constexpr uint32_t GEMMN_STAGES = 3;  // two workgroups per CU
__host__ __device__ constexpr uint32_t gemm_n_lds_bytes() {
  return GEMMN_STAGES * 5 * PANEL_TILE * 4 + 4 * 64 * 16;
}
template <uint32_t OUT, bool PARTIAL>
__global__ __launch_bounds__(512) void k_gemm_n(const float* __restrict__ Wp, uint32_t M,
                                                uint32_t K, const float* __restrict__ Xp,
                                                uint32_t B, float* __restrict__ Y, uint32_t ldy,
                                                const float* __restrict__ scale,
                                                const uint32_t* __restrict__ gen,
                                                float* __restrict__ P) {
  extern __shared__ float4 gsm[];  // [stages][5 tiles][4 quarters][64 lanes], then [4][64] f4v
  constexpr uint32_t NT = 5, NQ = 4 * NT;
  f4v* half_sum = reinterpret_cast<f4v*>(gsm + GEMMN_STAGES * NT * 256);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
  const uint32_t gdx = gridDim.x;  // kept in a register (a reload would wait for every LDS read)
  const uint32_t ct = wave % 4, h = wave / 4;
  const uint32_t nch = panel_chunks(K), nrt = (M + 15) / 16, nct = (B + 15) / 16;
  const uint32_t nld = (NQ - wave + GEMM_WAVES - 1) / GEMM_WAVES;
  const uint32_t mine = blockIdx.x < nrt ? (nrt - blockIdx.x + gdx - 1) / gdx : 0;
  const uint32_t total = mine * nch;
  const uint32_t lds0 = (uint32_t)(uintptr_t)gsm;
  auto issue = [&](uint32_t g, uint32_t st) {
    const uint32_t T = blockIdx.x + gdx * (g / nch), i = g % nch;
    const uint32_t sb = lds0 + st * NT * PANEL_TILE * 4;
#pragma unroll
    for (uint32_t f = wave; f < NQ; f += GEMM_WAVES) {
      const uint32_t tile = f / 4, q = f % 4;
      const float* src = tile == 0 ? Wp + ((size_t)T * nch + i) * PANEL_TILE
                                   : Xp + ((size_t)min(tile - 1, nct - 1) * nch + i) * PANEL_TILE;
      dma16(src + q * 256 + lane * 4, sb + f * 1024);
    }
  };
  for (uint32_t g = 0; g + 1 < GEMMN_STAGES && g < total; ++g) issue(g, g);
  for (uint32_t k = 0; k < mine; ++k) {
    f4v acc[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) acc[s] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t i = 0; i < nch; ++i) {
      const uint32_t g = k * nch + i;
      stage_wait(min(GEMMN_STAGES - 2, total - 1 - g) * nld);
      __syncthreads();
      if (g + GEMMN_STAGES - 1 < total)
        issue(g + GEMMN_STAGES - 1, (g + GEMMN_STAGES - 1) % GEMMN_STAGES);
      const float4* sa = gsm + (g % GEMMN_STAGES) * NT * 256;
      float4 a[2], b[2];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        a[qq] = sa[(2 * h + qq) * 64 + lane];
        b[qq] = sa[((1 + ct) * 4 + 2 * h + qq) * 64 + lane];
      }
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        // A last, partial chunk: the segments past K are left alone (their
        // zero padding would still turn a -0 sum into +0).
        if (PARTIAL && 64 * i + 4 * (8 * h + s) >= K) continue;
        acc[s] = __builtin_amdgcn_mfma_f32_16x16x4f32((&a[s / 4].x)[s % 4], (&b[s / 4].x)[s % 4],
                                                      acc[s], 0, 0, 0);
      }
    }
    // Subtree of this wave's eight segments; the upper half hands its own to
    // the lower half through LDS.
    f4v p4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p4[u] = acc[2 * u] + acc[2 * u + 1];
    const f4v t8 = (p4[0] + p4[1]) + (p4[2] + p4[3]);
    if (h == 1) half_sum[ct * 64 + lane] = t8;
    __syncthreads();
    const uint32_t T = blockIdx.x + gdx * k;
    if (h == 0 && ct < nct) {
      const f4v r = t8 + half_sum[ct * 64 + lane];
      const uint32_t b = ct * 16 + lane % 16;
      const uint32_t o = T * 16 + 4 * (lane / 16);
      if (b < B) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (o + j >= M) continue;
          const size_t at = (size_t)b * ldy + o + j;
          if (OUT == GO_PLAIN) {
            Y[at] = r[j];
          } else if (OUT == GO_RESID) {
            const float v = Y[at] + r[j];
            Y[at] = v;
            P[panel_at(b, o + j, panel_chunks(M))] = v;
          } else {
            const float v = scale[b] * r[j];
            reinterpret_cast<u64*>(Y)[at] = ((u64)gen[b] << 32) | (u64)__float_as_uint(v);
          }
        }
      }
    }
    // half_sum is rewritten by the next task only after this barrier.
    __syncthreads();
  }
}

// Narrow batches (B <= 64) with few row groups: the segments split four
// ways. Quarter q of tree16 is ((s_4q + s_4q+1) + (s_4q+2 + s_4q+3)), a
// subtree of its own, and it needs only quarter q of every chunk (one
// contiguous 1 KB block per tile and chunk in the panel layout), so a task
// is (pair of row tiles, quarter q, four column tiles): it reads a quarter
// of the rows' weights and of four column tiles' panel, and writes its
// subtree to plane q of Q ([4][B][M]); k_gemm_qcomb forms (t_0 + t_1) +
// (t_2 + t_3), the same tree16, and applies OUT. With all four column tiles
// of B <= 64 in one task, each weight quarter is read by one task only.
// Eight waves: wave w owns row tile w % 2 and column tile w / 2. A chunk's
// six 1 KB blocks (two row tiles, four column tiles) take one copy each
// from waves 0..5; a stage holds GEMMQ_CPB chunks (one barrier per stage),
// GEMMQ_STAGES - 1 stages ahead.
constexpr uint32_t GEMMQ_CPB = 8, GEMMQ_STAGES = 3;
__host__ __device__ constexpr uint32_t gemm_q_lds_bytes() {
  return GEMMQ_STAGES * GEMMQ_CPB * 6 * 1024;
}
template <bool PARTIAL>
__global__ __launch_bounds__(512) void k_gemm_q(const float* __restrict__ Wp, uint32_t M, uint32_t K,
                                                const float* __restrict__ Xp, uint32_t B,
                                                float* __restrict__ Q) {
  extern __shared__ float4 gsm[];  // [stages][GEMMQ_CPB chunks][6 blocks][64 lanes]
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
  const uint32_t gdx = gridDim.x;  // kept in a register (a reload would wait for every LDS read)
  const uint32_t rt = wave % 2, ct = wave / 2;
  const uint32_t nch = panel_chunks(K), nrt = (M + 15) / 16, nct = (B + 15) / 16;
  const uint32_t nsc = (nch + GEMMQ_CPB - 1) / GEMMQ_CPB;  // stages of chunks per task
  const uint32_t nrg = (nrt + 1) / 2, ncg = (nct + 3) / 4, ntask = 4 * nrg * ncg;
  const uint32_t mine = blockIdx.x < ntask ? (ntask - blockIdx.x + gdx - 1) / gdx : 0;
  const uint32_t total = mine * nsc;
  const uint32_t nld = wave < 6 ? GEMMQ_CPB : 0u;  // copies per stage
  const uint32_t lds0 = (uint32_t)(uintptr_t)gsm;
  // Task t = (x * 4 + q) * ncg + cg. Stage g's chunks into LDS stage st:
  // block `wave` of each is row tile 2x + wave (waves 0, 1) or column tile
  // 4cg + wave - 2, quarter q. Tiles and chunks past the last load a real
  // one (never used), so every copying wave issues GEMMQ_CPB per stage.
  auto issue = [&](uint32_t g, uint32_t st) {
    const uint32_t t = blockIdx.x + gdx * (g / nsc), i0 = (g % nsc) * GEMMQ_CPB;
    const uint32_t cg = t % ncg, xq = t / ncg, x = xq / 4, q = xq % 4;
    if (wave >= 6) return;
    const float* src = wave < 2 ? Wp + (size_t)min(2 * x + wave, nrt - 1) * nch * PANEL_TILE
                                : Xp + (size_t)min(4 * cg + wave - 2, nct - 1) * nch * PANEL_TILE;
#pragma unroll
    for (uint32_t c = 0; c < GEMMQ_CPB; ++c)
      dma16(src + (size_t)min(i0 + c, nch - 1) * PANEL_TILE + q * 256 + lane * 4,
            lds0 + ((st * GEMMQ_CPB + c) * 6 + wave) * 1024);
  };
  for (uint32_t g = 0; g + 1 < GEMMQ_STAGES && g < total; ++g) issue(g, g);
  for (uint32_t k = 0; k < mine; ++k) {
    const uint32_t t = blockIdx.x + gdx * k;
    const uint32_t cg = t % ncg, xq = t / ncg, x = xq / 4, q = xq % 4;
    f4v acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t j = 0; j < nsc; ++j) {
      const uint32_t g = k * nsc + j;
      // Stage g has landed once at most the later stages' copies are in
      // flight; after the barrier every wave is done with stage g - 1's
      // LDS, which the next request overwrites.
      stage_wait(min(GEMMQ_STAGES - 2, total - 1 - g) * nld);
      __syncthreads();
      if (g + GEMMQ_STAGES - 1 < total) issue(g + GEMMQ_STAGES - 1, (g + GEMMQ_STAGES - 1) % GEMMQ_STAGES);
      const float4* sa = gsm + (g % GEMMQ_STAGES) * GEMMQ_CPB * 6 * 64;
      float4 a[GEMMQ_CPB], b[GEMMQ_CPB];
#pragma unroll
      for (uint32_t c = 0; c < GEMMQ_CPB; ++c) {
        a[c] = sa[(c * 6 + rt) * 64 + lane];
        b[c] = sa[(c * 6 + 2 + ct) * 64 + lane];
      }
#pragma unroll
      for (uint32_t c = 0; c < GEMMQ_CPB; ++c) {
        const uint32_t i = j * GEMMQ_CPB + c;
        if (i >= nch) break;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // A last, partial chunk: the segments past K are left alone.
          if (PARTIAL && 64 * i + 4 * (4 * q + u) >= K) continue;
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32((&a[c].x)[u], (&b[c].x)[u], acc[u], 0, 0, 0);
        }
      }
    }
    const uint32_t T = 2 * x + rt, o = T * 16 + 4 * (lane / 16);
    const f4v r = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const uint32_t bc = (4 * cg + ct) * 16 + lane % 16;
    if (T < nrt && bc < B) {
      float* dst = Q + ((size_t)q * B + bc) * M + o;
      if (o + 4 <= M && (((size_t)q * B + bc) * M + o) % 4 == 0) {
        *reinterpret_cast<float4*>(dst) = make_float4(r[0], r[1], r[2], r[3]);
      } else {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          if (o + jj < M) dst[jj] = r[jj];
      }
    }
  }
}

// 1/rms of one row of n floats, by one wave: lane partials over the float4s
// at 4*lane + 256*i (i ascending), then the wave tree.
__device__ __forceinline__ float rms_row_inv(const float* __restrict__ x, uint32_t n, float eps,
                                             uint32_t lane) {
  float ss = 0.0f;
  for (uint32_t j = lane * 4; j < n; j += 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + j);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  ss = wave_sum(ss);
  return 1.0f / sqrtf(ss / (float)n + eps);
}

// The residual output of k_gemm_q (x += tree16 of the four subtrees, and
// its panel) for one row per workgroup, then the row's 1/rms (k_b_rms's
// order) for the next matrix product's normalisation: one launch instead of
// two.
__global__ __launch_bounds__(256) void k_gemm_qcomb_rms(const float* __restrict__ Q, uint32_t M,
                                                        uint32_t B, float* __restrict__ Y,
                                                        uint32_t ldy, float* __restrict__ P,
                                                        float eps, float* __restrict__ inv) {
  const uint32_t b = blockIdx.x;
  const size_t plane = (size_t)B * M;
  for (uint32_t o = threadIdx.x; o < M; o += blockDim.x) {
    const size_t e = (size_t)b * M + o;
    const float r = (Q[e] + Q[plane + e]) + (Q[2 * plane + e] + Q[3 * plane + e]);
    const size_t at = (size_t)b * ldy + o;
    const float v = Y[at] + r;
    Y[at] = v;
    P[panel_at(b, o, panel_chunks(M))] = v;
  }
  // The row's new values, written by the whole workgroup, are visible to it
  // after the barrier.
  __syncthreads();
  if (threadIdx.x < WAVE) {
    const float r = rms_row_inv(Y + (size_t)b * ldy, M, eps, threadIdx.x);
    if (threadIdx.x == 0) inv[b] = r;
  }
}

// The four quarter subtrees of k_gemm_q into tree16 and the output: thread
// (b, o) for o < M, b < B.
template <uint32_t OUT>
__global__ void k_gemm_qcomb(const float* __restrict__ Q, uint32_t M, uint32_t B,
                             float* __restrict__ Y, uint32_t ldy, const float* __restrict__ scale,
                             const uint32_t* __restrict__ gen, float* __restrict__ P) {
  const uint32_t o = blockIdx.x * blockDim.x + threadIdx.x, b = blockIdx.y;
  if (o >= M || b >= B) return;
  const size_t plane = (size_t)B * M, e = (size_t)b * M + o;
  const float r = (Q[e] + Q[plane + e]) + (Q[2 * plane + e] + Q[3 * plane + e]);
  const size_t at = (size_t)b * ldy + o;
  if (OUT == GO_PLAIN) {
    Y[at] = r;
  } else if (OUT == GO_RESID) {
    const float v = Y[at] + r;
    Y[at] = v;
    P[panel_at(b, o, panel_chunks(M))] = v;
  } else {
    const float v = scale[b] * r;
    reinterpret_cast<u64*>(Y)[at] = ((u64)gen[b] << 32) | (u64)__float_as_uint(v);
  }
}

// ------------------------------------------------------------- rows

// One row of a batch: the cache it extends, at which position and
// generation base, with which token.
struct BRow {
  float* kc;
  float* vc;
  uint32_t cap, pos, tick, token;
};

// X[b] = E[token_b] (model.rs:428), and its panel XP; token_b from dtok
// (device, e.g. just sampled) when given, else from the row.
__global__ void k_b_embed(const BRow* __restrict__ rows, const uint32_t* __restrict__ dtok,
                          const float* __restrict__ embed, uint32_t h,
                          float* __restrict__ X, float* __restrict__ XP) {
  const uint32_t b = blockIdx.x, nch = panel_chunks(h);
  const float* e = embed + (size_t)(dtok ? dtok[b] : rows[b].token) * h;
  for (uint32_t i = threadIdx.x; i < h; i += blockDim.x) {
    const float v = e[i];
    X[(size_t)b * h + i] = v;
    XP[panel_at(b, i, nch)] = v;
  }
}

// inv[b] = 1/rms(X[b]) in the order of rms_inv: each lane's elements
// 4*lane + 256*k ascending, then wave_sum. One wave per row.
__global__ __launch_bounds__(256) void k_b_rms(const float* __restrict__ X, uint32_t B, uint32_t n,
                                               float eps, float* __restrict__ inv) {
  const uint32_t b = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  if (b >= B) return;
  const float r = rms_row_inv(X + (size_t)b * n, n, eps, lane);
  if (lane == 0) inv[b] = r;
}

// QKV epilogue of the one-token path (phase_qkv) for pair i of head block
// hb of batch row b: the product's rows r0 = hb * hd + i and r1 = r0 + half
// (from Y, or combined from k_gemm_q's four subtree planes QS ([4][nb]
// [qkv_rows]) as k_gemm_qcomb would), scaled by the row's 1/rms, biased,
// and rotated (q and k heads) -- phase_qkv's expressions.
__device__ __forceinline__ float2 qkv_epi_pair(const Args& a, uint32_t l, uint32_t pos, uint32_t b,
                                               uint32_t hb, uint32_t i, const float* __restrict__ Y,
                                               uint32_t ldy, const float* __restrict__ QS,
                                               uint32_t nb, float iv) {
  const Dims& d = a.d;
  const uint32_t r0 = hb * d.hd + i, r1 = r0 + d.half;
  float4 e = make_float4(1.0f, 0.0f, 0.0f, 0.0f);
  if (hb < d.nh + d.nkv) {
    const float2 cs = a.rope[(size_t)pos * d.half + i];
    e.x = cs.x;
    e.y = cs.y;
  }
  const float* bias = a.layers[l].bqkv;
  if (bias) {
    e.z = bias[r0];
    e.w = bias[r0 + d.half];
  }
  float y0, y1;
  if (QS) {
    const size_t plane = (size_t)nb * d.qkv_rows, e0 = (size_t)b * d.qkv_rows + r0, e1 = e0 + d.half;
    y0 = (QS[e0] + QS[plane + e0]) + (QS[2 * plane + e0] + QS[3 * plane + e0]);
    y1 = (QS[e1] + QS[plane + e1]) + (QS[2 * plane + e1] + QS[3 * plane + e1]);
  } else {
    y0 = Y[(size_t)b * ldy + r0];
    y1 = Y[(size_t)b * ldy + r1];
  }
  y0 = y0 * iv + e.z;
  y1 = y1 * iv + e.w;
  float a0 = y0, a1 = y1;
  if (hb < d.nh + d.nkv) {
    a0 = y0 * e.x - y1 * e.y;
    a1 = y1 * e.x + y0 * e.y;
  }
  return make_float2(a0, a1);
}

// k (hb < nh + nkv) or v rows of head block hb into the row's cache at its
// position (model.rs:466-467).
__device__ __forceinline__ void qkv_epi_cache(const Dims& d, const BRow& r, uint32_t l, uint32_t hb,
                                              uint32_t i, float2 v) {
  const bool is_k = hb < d.nh + d.nkv;
  const uint32_t gi = is_k ? hb - d.nh : hb - d.nh - d.nkv;
  float* row = (is_k ? r.kc : r.vc) + (((size_t)l * d.nkv + gi) * r.cap + r.pos) * d.kvs;
  row[i] = v.x;
  row[i + d.half] = v.y;
}

// QKV epilogue per (row, pair): q/k/v words tagged for the attention items;
// k, v into the row's cache at its position.
__global__ void k_b_qkv_epi(const Args* __restrict__ ap, const BRow* __restrict__ rows, uint32_t l,
                            const float* __restrict__ Y, uint32_t ldy, const float* __restrict__ inv,
                            u64* __restrict__ qkvt, uint32_t ldq, const float* __restrict__ QS,
                            uint32_t nb) {
  const Dims& d = ap->d;
  const uint32_t b = blockIdx.y;
  const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= d.qkv_rows / 2) return;
  const BRow r = rows[b];
  const uint32_t hb = p / d.half, i = p - hb * d.half;
  const uint32_t r0 = hb * d.hd + i, r1 = r0 + d.half;
  const float2 v = qkv_epi_pair(*ap, l, r.pos, b, hb, i, Y, ldy, QS, nb, inv[b]);
  const u64 g = (u64)gen_of(d, r.tick, l, PH_QKV) << 32;
  qkvt[(size_t)b * ldq + r0] = g | __float_as_uint(v.x);
  qkvt[(size_t)b * ldq + r1] = g | __float_as_uint(v.y);
  if (hb >= d.nh) qkv_epi_cache(d, r, l, hb, i, v);
}

// LDS of the batched kernels that run one-token functions: no weight
// staging (lds_stg = 0 in the row Args).
__device__ __forceinline__ Lds lds_init_rows(const Dims& d) {
  extern __shared__ float lds_raw[];
  Lds s = lds_layout(lds_raw, d);
  if (threadIdx.x == 0) s.ctl->abort_seen = 0;
  __syncthreads();
  return s;
}

// LDS of the attention-only workgroups: the wait control words, then the
// attention's scratch.
__device__ __forceinline__ Lds lds_init_attn() {
  extern __shared__ float lds_raw[];
  Lds s;
  s.ctl = reinterpret_cast<WaitCtl*>(lds_raw);
  s.red = lds_raw + 4;
  s.vec = s.vec2 = s.stg = nullptr;
  s.scr = lds_raw + 4 + 64;
  s.pub = nullptr;
  if (threadIdx.x == 0) s.ctl->abort_seen = 0;
  __syncthreads();
  return s;
}

// Attention items of every row, one per workgroup: entry x of `items` is
// (row, item) packed as row << 16 | item, and the workgroup runs that item
// with the one-token path's phase_attn in its grouped form (item = (kv head,
// chunk) with all the group's query heads; each head's arithmetic is the
// one-token path's), reading the row's tagged q/k/v and writing its tagged
// partials. The workgroups are the NCW attention waves alone (they also
// poll and publish) with only the attention's LDS, so that several items
// share a CU: one row's chunk is a chain of dependent loads and barriers
// that a lone workgroup cannot keep the CU busy with. One score pass and
// four value steps in flight per lane keep the kernel within 128 VGPRs,
// four workgroups per CU.
__global__ __launch_bounds__(NCW * WAVE) __attribute__((amdgpu_waves_per_eu(4))) void k_b_attn_w(
    const Args* __restrict__ rargs, const BRow* __restrict__ rows,
    const uint32_t* __restrict__ items, uint32_t l) {
  const uint32_t e = items[blockIdx.x], b = e >> 16, x = e & 0xffffu;
  const Args& a = rargs[b];
  const Lds s = lds_init_attn();
  const BRow r = rows[b];
  phase_attn<true, 0, NCW, 1, 4>(a, l, r.tick, r.pos, x, 0x10000u, s);
}

// The same attention items of rows with distinct caches (a lockstep step)
// with the QKV epilogue before and the chunk combine after, so that one
// launch replaces three. Each item forms its kv group's q/k/v from the QKV
// product itself (qkv_epi_pair; the chunk-0 item also writes k and v into
// the cache: no item of the step reads that row, as position pos comes from
// LDS), runs phase_attn, and counts itself done in cnt[b][g] (an
// agent-scope add); the group's last item waits for the tags of the group's
// chunk partials, combines them (combine_scales / combine_value, as
// k_b_comb) into the attention panel and sets the count back to 0.
__global__ __launch_bounds__(NCW * WAVE) __attribute__((amdgpu_waves_per_eu(4))) void k_b_attn_f(
    const Args* __restrict__ rargs, const BRow* __restrict__ rows,
    const uint32_t* __restrict__ items, uint32_t l, const float* __restrict__ Y, uint32_t ldy,
    const float* __restrict__ QS, uint32_t nb, const float* __restrict__ inv,
    uint32_t* __restrict__ cnt, float* __restrict__ attp) {
  const uint32_t e = items[blockIdx.x], b = e >> 16, x = e & 0xffffu;
  const Args& a = rargs[b];
  const Lds s = lds_init_attn();
  const BRow r = rows[b];
  const Dims& d = a.d;
  const uint32_t nch = attn_nchunks(r.pos), g = x / nch, c = x - g * nch;
  const float iv = inv[b];
  auto fill = [&](uint32_t gg, float* qs, float* kn, float* vn) {
    for (uint32_t u = threadIdx.x; u < (d.group + 2) * d.half; u += blockDim.x) {
      const uint32_t j = u / d.half, i = u - j * d.half;
      const uint32_t hb = j < d.group ? gg * d.group + j : (j == d.group ? d.nh + gg : d.nh + d.nkv + gg);
      const float2 v = qkv_epi_pair(a, l, r.pos, b, hb, i, Y, ldy, QS, nb, iv);
      float* dst = j < d.group ? qs + j * d.hd : (j == d.group ? kn : vn);
      lds_st(dst + i, v.x);
      lds_st(dst + i + d.half, v.y);
      if (j >= d.group && c == 0) qkv_epi_cache(d, r, l, hb, i, v);
    }
    __syncthreads();
    return true;
  };
  phase_attn<true, 0, NCW, 1, 4>(a, l, r.tick, r.pos, x, 0x10000u, s, fill);
  // Every wave has issued its partials' stores. No fence: the last item
  // waits for the partials' tags instead (a device-scope fence would write
  // back and invalidate the whole L2 of the XCD).
  __syncthreads();
  AS_LDS uint32_t* last = lptr(reinterpret_cast<uint32_t*>(s.red));
  if (threadIdx.x == 0) {
    uint32_t* cg = cnt + (size_t)b * d.nkv + g;
    const uint32_t done = __hip_atomic_fetch_add(cg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = done + 1 == nch;
    if (done + 1 == nch) __hip_atomic_store(cg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*last) return;
  const uint32_t hs = d.hd + 2, grp = d.group, n1 = nch * hs;
  float* part = s.scr;                      // [grp][nch][hs]
  float* sc = part + MAX_GROUP * MAX_ACHUNKS * hs;  // [MAX_GROUP][MAX_ACHUNKS]
  float* ls = sc + MAX_GROUP * MAX_ACHUNKS;  // [MAX_GROUP]
  if (!poll_gather<4>(gather_strided(a.mb_part + (size_t)g * grp * MAX_ACHUNKS * hs, n1, grp,
                                     MAX_ACHUNKS * hs, gen_of(d, r.tick, l, PH_ATTN), part),
                      NCW, a.st, s.ctl))
    return;
  for (uint32_t k = threadIdx.x; k < grp; k += blockDim.x)
    ls[k] = combine_scales([&](uint32_t i) { return lds_ld(part + k * n1 + i); }, nch, hs,
                           sc + k * MAX_ACHUNKS);
  __syncthreads();
  for (uint32_t v = threadIdx.x; v < grp * d.hd; v += blockDim.x) {
    const uint32_t k = v / d.hd, dd = v - k * d.hd, u = (g * grp + k) * d.hd + dd;
    attp[panel_at(b, u, panel_chunks(d.q))] =
        combine_value([&](uint32_t i) { return lds_ld(part + k * n1 + i); }, nch, hs, dd,
                      sc + k * MAX_ACHUNKS, ls[k]);
  }
}

// ----------------------------------------------------- tiled attention
//
// Rows of one cache at consecutive positions (a prefill or a replay) share
// their K/V rows, so their attention runs as tiles: a workgroup takes 16
// consecutive query positions (aligned to 16), one chunk of 128 key
// positions and one kv head, stages the chunk's K and V rows in LDS once, and
// computes every query's chunk partials (m, l, acc) in the order phase_attn
// uses (head_dim 64, chunk 128, positions < 2048), with MFMA chains where
// phase_attn has fma chains:
//  * score(q, t): 4 chains over 16 elements each (the lanes of a position),
//    then ((c0 + c1) + (c2 + c3)) * scale;
//  * softmax: phase_attn's sums -- lane slot L = 0..63 adds positions L,
//    L + 64 from +0, then the wave tree over the 64 slots -- with 16 lanes
//    per (query, head), lane s holding slots s + 16v, so a wave takes four
//    (query, head) rows at once;
//  * value[d]: 16 position groups (attention wave w, group pl: positions
//    4w + pl + 16k, k ascending), each a chain, then per w the tree over its
//    four groups and the sum w = 0..3 in order, from +0.
// Positions past a query's own (t > pos) carry probability +0 and zero V
// rows, which leave an accumulator unchanged (a chain started at +0 never
// holds -0). The scores reuse the LDS of K and Q once every wave is done
// with them, so with three query heads per kv head two workgroups fit a CU.

constexpr uint32_t AT_HD = 64, AT_CH = 128, AT_VROWS = 128;  // 16 groups x 8 positions
constexpr int AT_VG = 16;  // value position groups (phase_attn: NCW waves x 4)
static_assert(AT_VG == NCW * 4, "the value groups are phase_attn's");
constexpr uint32_t AT_KP = 65, AT_VP = 66, AT_QP = 65, AT_SP = 193;  // LDS row pitches (floats)

// Floats of the K + Q region, which the scores then take.
__host__ __device__ inline size_t attn_tile_kq(uint32_t grp) {
  const size_t kq = (size_t)AT_CH * AT_KP + (size_t)grp * 16 * AT_QP;
  const size_t sc = (size_t)grp * 16 * AT_SP;
  return kq > sc ? kq : sc;
}
__host__ __device__ inline size_t attn_tile_lds(uint32_t grp) {
  return sizeof(float) * (attn_tile_kq(grp) + (size_t)AT_CH * AT_VP + grp * 32);
}

// tasks[x] = tile << 16 | chunk << 8 | kv head; tiles[m] .. tiles[m + 1] are
// the batch rows of tile m. rows: the batch (one cache, consecutive
// positions); qkvt: tagged q/k/v words per row; part: tagged partials.
__global__ __launch_bounds__(256, 2) void k_b_attn_tile(const Dims d, const BRow* __restrict__ rows,
                                                     const uint32_t* __restrict__ tasks,
                                                     const uint32_t* __restrict__ tiles, uint32_t l,
                                                     const u64* __restrict__ qkvt,
                                                     u64* __restrict__ part, uint32_t part_w) {
  extern __shared__ float at_lds[];
  const uint32_t grp = d.group, hs = AT_HD + 2;
  float* Ks = at_lds;                       // [AT_CH][AT_KP]
  float* Qs = Ks + AT_CH * AT_KP;           // [grp][16][AT_QP]
  float* Ss = at_lds;                       // [grp][16][AT_SP]: scores, then probabilities
  float* Vs = at_lds + attn_tile_kq(grp);   // [AT_CH][AT_VP]
  float* ML = Vs + AT_CH * AT_VP;           // [grp][16][2]: m, l
  const uint32_t task = tasks[blockIdx.x];
  const uint32_t m = task >> 16, c = (task >> 8) & 0xffu, g = task & 0xffu;
  const uint32_t rb0 = tiles[m], nq = tiles[m + 1] - rb0;
  const BRow r0 = rows[rb0];
  const uint32_t p_last = r0.pos + nq - 1;
  const uint32_t t0 = c * AT_CH;
  const uint32_t nk = min(AT_CH, p_last + 1 - t0);
  const uint32_t tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const float* kb = r0.kc + ((size_t)l * d.nkv + g) * r0.cap * d.kvs;
  const float* vb = r0.vc + ((size_t)l * d.nkv + g) * r0.cap * d.kvs;
  // 1. K rows, V rows and Q words of the chunk: each thread issues all its
  // loads before its first LDS store (16 threads per K/V row).
  constexpr int NR = AT_CH * 16 / 256;                 // K/V float4 per thread: 8
  constexpr int NQ = MAX_GROUP * 16 * AT_HD / 256;     // Q words per thread: 16
  float4 kr[NR], vr[NR];
  u64 qw[NQ];
  // Generation tags of this lane's output queries 4*lc + rr (values stage).
  const uint32_t lr = lane % 16, lc = lane / 16;
  u64 gtag[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const uint32_t q = 4 * lc + rr;
    gtag[rr] = q < nq ? (u64)gen_of(d, rows[rb0 + q].tick, l, PH_ATTN) << 32 : 0;
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint32_t e = tid + 256 * k, t = e / 16, q4 = (e % 16) * 4;
    kr[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    vr[k] = kr[k];
    if (t < nk) {
      kr[k] = *reinterpret_cast<const float4*>(kb + (size_t)(t0 + t) * d.kvs + q4);
      vr[k] = *reinterpret_cast<const float4*>(vb + (size_t)(t0 + t) * d.kvs + q4);
    }
  }
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const uint32_t e = tid + 256 * k, j = e / (16 * AT_HD), q = (e / AT_HD) % 16, dd = e % AT_HD;
    qw[k] = 0;
    if (j < grp && q < nq) qw[k] = qkvt[(size_t)(rb0 + q) * d.qkv_rows + (g * grp + j) * AT_HD + dd];
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const uint32_t e = tid + 256 * k, t = e / 16, q4 = (e % 16) * 4;
    float* kd = Ks + t * AT_KP + q4;
    float* vd = Vs + t * AT_VP + q4;
    kd[0] = kr[k].x;
    kd[1] = kr[k].y;
    kd[2] = kr[k].z;
    kd[3] = kr[k].w;
    vd[0] = vr[k].x;
    vd[1] = vr[k].y;
    vd[2] = vr[k].z;
    vd[3] = vr[k].w;
  }
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const uint32_t e = tid + 256 * k, j = e / (16 * AT_HD), q = (e / AT_HD) % 16, dd = e % AT_HD;
    if (j < grp) Qs[(j * 16 + q) * AT_QP + dd] = __uint_as_float((uint32_t)qw[k]);
  }
  __syncthreads();
  // 2. scores: wave w takes key tiles w and w + 4, kept in registers until
  // every wave is done with K and Q, whose LDS the scores then take. The
  // (head, sub) chains of a key tile run interleaved.
  const uint32_t nkt = (nk + 15) / 16;
  float qa[MAX_GROUP][4][4];  // element 16*sub + 4*i + lc of query lr, head j
#pragma unroll
  for (uint32_t j = 0; j < MAX_GROUP; ++j)
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        qa[j][sub][i] = j < grp ? Qs[(j * 16 + lr) * AT_QP + 16 * sub + 4 * i + lc] : 0.0f;
  f4v sreg[2][MAX_GROUP];
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t kt = wave + 4 * u;
    if (kt >= nkt) continue;
    float ka[4][4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) ka[sub][i] = Ks[(kt * 16 + lr) * AT_KP + 16 * sub + 4 * i + lc];
    f4v acc[MAX_GROUP][4];
#pragma unroll
    for (uint32_t j = 0; j < MAX_GROUP; ++j)
#pragma unroll
      for (int sub = 0; sub < 4; ++sub) acc[j][sub] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (uint32_t j = 0; j < MAX_GROUP; ++j) {
        if (j >= grp) continue;
#pragma unroll
        for (int sub = 0; sub < 4; ++sub)
          acc[j][sub] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[j][sub][i], ka[sub][i], acc[j][sub],
                                                             0, 0, 0);
      }
#pragma unroll
    for (uint32_t j = 0; j < MAX_GROUP; ++j)
      sreg[u][j] = (acc[j][0] + acc[j][1]) + (acc[j][2] + acc[j][3]);
  }
  __syncthreads();
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t kt = wave + 4 * u;
#pragma unroll
    for (uint32_t j = 0; j < MAX_GROUP; ++j) {
      if (kt >= nkt || j >= grp) continue;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)  // query 4*lc + rr, key kt*16 + lr
        Ss[(j * 16 + 4 * lc + rr) * AT_SP + kt * 16 + lr] = sreg[u][j][rr] * d.scale;
    }
  }
  __syncthreads();
  // 3. softmax statistics and probabilities, 16 lanes per (query, head):
  // lane sub holds phase_attn's lane slots L = sub + 16v (v = 0..3), each
  // the sum of positions L, L + 64 from +0; the slots' tree is group_sum
  // over the 16 lanes of each v, then (R3 + R2) + (R1 + R0) as wave_sum.
  // A lane's eight positions sub + 16k are read at once; positions from n
  // on (up to AT_VROWS) get probability +0.
  {
    const uint32_t sub = lane % 16;
    for (uint32_t u0 = 4 * wave; u0 < grp * 16; u0 += 16) {
      const uint32_t u = u0 + lane / 16;
      const uint32_t j = u / 16, q = u % 16;
      float* sh = Ss + u * AT_SP;
      const uint32_t n = q < nq ? min(AT_CH, r0.pos + q + 1 - t0) : 0;
      float sv[8];
#pragma unroll
      for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t i = sub + 16 * k;
        sv[k] = i < n ? sh[i] : -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (uint32_t k = 0; k < 8; ++k) mx = fmaxf(mx, sv[k]);
      mx = row_max(mx);
      float e[8];
#pragma unroll
      for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t i = sub + 16 * k;
        e[k] = (i < n && mx != -INFINITY) ? expf(sv[k] - mx) : 0.0f;
        sh[i] = e[k];
      }
#pragma unroll
      for (uint32_t k = 8; k < AT_VROWS / 16; ++k) sh[sub + 16 * k] = 0.0f;
      float R[4];
#pragma unroll
      for (uint32_t v = 0; v < 4; ++v) R[v] = group_sum((0.0f + e[v]) + e[v + 4], 16);
      const float lsum = (R[3] + R[2]) + (R[1] + R[0]);
      if (sub == 0) {
        ML[(j * 16 + q) * 2] = mx;
        ML[(j * 16 + q) * 2 + 1] = lsum;
      }
    }
  }
  __syncthreads();
  // 4. values: wave w computes dims 16w..16w+15 of every head; the V
  // operands are read once for all heads.
  float vop[AT_VG][2];
#pragma unroll
  for (int gi = 0; gi < AT_VG; ++gi)
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const uint32_t pos = gi + AT_VG * (4 * mm + lc);  // group gi = 4*w' + pl
      vop[gi][mm] = pos < AT_CH ? Vs[pos * AT_VP + 16 * wave + lr] : 0.0f;
    }
  for (uint32_t j = 0; j < grp; ++j) {
    float pop[AT_VG][2];
#pragma unroll
    for (int gi = 0; gi < AT_VG; ++gi)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) pop[gi][mm] = Ss[(j * 16 + lr) * AT_SP + gi + AT_VG * (4 * mm + lc)];
    f4v acc[AT_VG];
#pragma unroll
    for (int gi = 0; gi < AT_VG; ++gi) acc[gi] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int gi = 0; gi < AT_VG; ++gi)
        acc[gi] = __builtin_amdgcn_mfma_f32_16x16x4f32(pop[gi][mm], vop[gi][mm], acc[gi], 0, 0, 0);
    f4v A = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w4 = 0; w4 < AT_VG / 4; ++w4) {
      const f4v W = (acc[4 * w4] + acc[4 * w4 + 1]) + (acc[4 * w4 + 2] + acc[4 * w4 + 3]);
      A = A + W;
    }
    const uint32_t hh = g * grp + j;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {  // query 4*lc + rr, dim 16*wave + lr
      const uint32_t q = 4 * lc + rr;
      if (q >= nq) continue;
      u64* out = part + (size_t)(rb0 + q) * part_w + ((size_t)hh * MAX_ACHUNKS + c) * hs;
      out[2 + 16 * wave + lr] = gtag[rr] | __float_as_uint(A[rr]);
      if (wave == 0 && lr == 0) {
        out[0] = gtag[rr] | __float_as_uint(ML[(j * 16 + q) * 2]);
        out[1] = gtag[rr] | __float_as_uint(ML[(j * 16 + q) * 2 + 1]);
      }
    }
  }
}

// Combine of the chunk partials (combine_scales / combine_value, as the O
// phase does) into the panel of att[b][q]: one workgroup per row and group of
// heads; the weights of a head's chunks are formed once in LDS (a wave per
// head, a lane per chunk), then a thread per (head, dim). The
// partials were written by earlier launches on the same stream, so their
// values are read directly (the low half of each tagged word).
constexpr uint32_t COMB_MAX_HEADS = 64;
constexpr uint32_t COMB_HEADS_PER_BLOCK = 4;  // grid y: groups of heads
__global__ __launch_bounds__(256) void k_b_comb(const Dims d, const BRow* __restrict__ rows,
                                                const u64* __restrict__ part, uint32_t part_w,
                                                float* __restrict__ attp) {
  __shared__ float sc[COMB_HEADS_PER_BLOCK][MAX_ACHUNKS];
  __shared__ float ls[COMB_HEADS_PER_BLOCK];
  const uint32_t b = blockIdx.x, h0 = blockIdx.y * COMB_HEADS_PER_BLOCK;
  const uint32_t nh = min(COMB_HEADS_PER_BLOCK, d.nh - h0);
  const uint32_t nch = attn_nchunks(rows[b].pos), hs = d.hd + 2;
  const u64* pb = part + (size_t)b * part_w;
  const uint32_t wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  auto val = [](const u64* p) { return __uint_as_float((uint32_t)*p); };
  // combine_scales for head h0 + wave, one lane per chunk: M is a maximum
  // (the same in any order, NaN maxima dropped as fmaxf from -inf drops
  // them), each weight the same expf, and the weighted total summed in
  // chunk order by lane 0 from the lanes' products (no contraction).
  if (wave < nh) {
    const u64* p = pb + (size_t)(h0 + wave) * MAX_ACHUNKS * hs;
    if (nch == 1) {
      if (lane == 0) ls[wave] = val(p + 1) * 1.0f;
    } else {
      const float mc = lane < nch ? val(p + lane * hs) : -INFINITY;
      const float lc = lane < nch ? val(p + lane * hs + 1) : 0.0f;
      float M = fmaxf(-INFINITY, mc);
      for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
      const float w = (mc == -INFINITY) ? 0.0f : expf(mc - M);
      const float prod = lc * w;
      if (lane < nch) sc[wave][lane] = w;
      float Ls = 0.0f;
      for (uint32_t c = 0; c < nch; ++c) Ls = Ls + __shfl(prod, c);
      if (lane == 0) ls[wave] = Ls;
    }
  }
  __syncthreads();
  // combine_value, with the chunks' values loaded before the sum (the same
  // sum in chunk order).
  for (uint32_t v = threadIdx.x; v < nh * d.hd; v += blockDim.x) {
    const uint32_t k = v / d.hd, dd = v - k * d.hd, u = (h0 + k) * d.hd + dd;
    const u64* p = pb + (size_t)(h0 + k) * MAX_ACHUNKS * hs + 2 + dd;
    float x[MAX_ACHUNKS];
#pragma unroll
    for (uint32_t c = 0; c < MAX_ACHUNKS; ++c) x[c] = c < nch ? val(p + c * hs) : 0.0f;
    float out;
    if (nch == 1) {
      out = (x[0] * 1.0f) / ls[k];
    } else {
      float A = 0.0f;
#pragma unroll
      for (uint32_t c = 0; c < MAX_ACHUNKS; ++c)
        if (c < nch) A = A + x[c] * sc[k][c];
      out = A / ls[k];
    }
    attp[panel_at(b, u, panel_chunks(d.q))] = out;
  }
}

// g = act(gate * inv) * (up * inv) (phase_gu), into the panel GP; Y holds
// gate rows then up rows.
__global__ void k_b_act(const float* __restrict__ Y, uint32_t ldy, const float* __restrict__ inv,
                        uint32_t ff, uint32_t act, float* __restrict__ GP) {
  const uint32_t b = blockIdx.y;
  const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= ff) return;
  const float iv = inv[b];
  const float gate = Y[(size_t)b * ldy + j], up = Y[(size_t)b * ldy + ff + j];
  GP[panel_at(b, j, panel_chunks(ff))] = act_fn(gate * iv, act) * (up * iv);
}

// Final norm of the rows that need logits (phase_lm): xs = x * w_norm and
// inv = 1/rms(x) in rms_inv's order; xs goes into the panel XSP. One wave
// per logits row; sel[i] is its batch row.
__global__ __launch_bounds__(64) void k_b_final(const float* __restrict__ X,
                                                const uint32_t* __restrict__ sel, uint32_t h,
                                                const float* __restrict__ nrm, float eps,
                                                float* __restrict__ XSP, float* __restrict__ linv) {
  const uint32_t i = blockIdx.x, lane = threadIdx.x, nch = panel_chunks(h);
  const float* x = X + (size_t)sel[i] * h;
  float ss = 0.0f;
  for (uint32_t j = lane * 4; j < h; j += 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + j);
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
    XSP[panel_at(i, j, nch)] = v.x * nrm[j];
    XSP[panel_at(i, j + 1, nch)] = v.y * nrm[j + 1];
    XSP[panel_at(i, j + 2, nch)] = v.z * nrm[j + 2];
    XSP[panel_at(i, j + 3, nch)] = v.w * nrm[j + 3];
  }
  ss = wave_sum(ss);
  if (lane == 0) linv[i] = 1.0f / sqrtf(ss / (float)h + eps);
}

// Chunk (max, argmax) of the tagged logits of each logits row, tagged for
// the sampler (phase_lm's chunk step; argmax is a total order, so any tree
// gives its answer). One wave per (chunk, row).
// Chunk (max, argmax) of every logits row: each wave takes CM_CPW
// consecutive chunks, one lane per row of a chunk, with all its loads issued
// before the first reduction (the same reduction per chunk as the lm_head
// phase's, so the same values).
constexpr uint32_t CM_CPW = 4;
__global__ __launch_bounds__(256) void k_b_chunkmax(const Dims d, const u64* __restrict__ logt,
                                                    const uint32_t* __restrict__ gen,
                                                    u64* __restrict__ vmax, u64* __restrict__ varg,
                                                    uint32_t nlm) {
  const uint32_t c0 = (blockIdx.x * 4 + threadIdx.x / WAVE) * CM_CPW, lane = threadIdx.x % WAVE;
  const uint32_t i = blockIdx.y;
  if (c0 >= d.nvc || i >= nlm) return;
  u64 raw[CM_CPW];
#pragma unroll
  for (uint32_t u = 0; u < CM_CPW; ++u) {
    const uint32_t v = (c0 + u) * VCHUNK + lane;
    raw[u] = (c0 + u < d.nvc && v < d.V) ? logt[(size_t)i * d.V + v] : 0;
  }
  const u64 g = (u64)gen[i] << 32;
#pragma unroll
  for (uint32_t u = 0; u < CM_CPW; ++u) {
    const uint32_t c = c0 + u;
    if (c >= d.nvc) break;
    const uint32_t v = c * VCHUNK + lane;
    float bv = -INFINITY;
    uint32_t bi = NO_INDEX;
    if (v < d.V) {
      const float y = __uint_as_float((uint32_t)raw[u]);
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
      vmax[(size_t)i * d.nvc + c] = g | __float_as_uint(bv);
      varg[(size_t)i * d.nvc + c] = g | bi;
    }
  }
}

// Chunks per wave and round of k_b_sample's stage A: the one workgroup of an
// op walks all the row's chunks, so rounds of NWA chunks would each wait a
// full memory latency. Its LDS holds NWA * SAMP_CPW chunks past the rows
// layout's scratch start (samp_lds_bytes).
constexpr uint32_t SAMP_CPW = 8;

// One sampling op per workgroup (the one-token sampler, stages A and B on
// one workgroup): op j samples logits row lrow[j] for generation base
// tick[j] with rng word words[j]; the token goes to out[j].
__global__ __launch_bounds__(BLOCK) void k_b_sample(const Args* __restrict__ largs,
                                                    const uint32_t* __restrict__ tick,
                                                    const uint32_t* __restrict__ words, float T,
                                                    uint32_t tag0, uint32_t* __restrict__ out) {
  const uint32_t j = blockIdx.x;
  const Args& a = largs[j];
  const Lds s = lds_init_rows(a.d);
  // A row whose wait runs out still leaves a token in range (0), so a
  // following batched embedding never reads outside the table.
  if (threadIdx.x == 0) out[j] = 0u;
  uint32_t tok = 0;
  if (T != 0.0f) {
    float m;
    uint32_t bi;
    if (!sample_stage_a<SAMP_CPW, 8>(a, tick[j], tag0 + j, T, 0, 1, s, &m, &bi)) return;
    if (!sample_exact(a, tag0 + j, m, bi, words[j], 0, 1, true, s, &tok)) return;
  } else if (!sample_greedy(a, tick[j], s, &tok)) {
    return;
  }
  if (threadIdx.x == 0) out[j] = tok;
}

}  // namespace dg
