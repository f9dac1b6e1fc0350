// exact.h -- the arithmetic sample_token (sampler.rs:43-109) does on the CPU,
// reproduced bit for bit on the device.
//
// 1. expf. The reference's `f32::exp` is the platform libm's expf (glibc
//    2.35 here). glibc uses the published algorithm of Arm's optimized-
//    routines (Szabolcs Nagy, MIT / Apache-2.0): x * 32/ln2 = k + r with k
//    the nearest integer, exp(x) = 2^(k/32) * 2^(r/32), the first factor from
//    a 32-entry table of 2^(i/32) and the second a degree-3 polynomial, all in
//    double precision, rounded to float once. On x86-64 CPUs with FMA, glibc
//    runs the build of that code compiled with fused multiply-adds: the
//    polynomial's three a*b+c steps and the reduction r = x*32/ln2 - k are
//    each one rounding. expf_ref below does exactly those operations; an
//    exhaustive comparison over all 2^32 inputs against the libm expf of the
//    build container finds no difference (tests/test_exact.py keeps a
//    strided sweep of it).
//
// 2. Sequential float sums. sample_token sums probabilities one at a time in
//    index order (sampler.rs:52-59, 94-106). While a running sum s stays in
//    one "grid region" -- the floats that are multiples of u = 2^E below
//    2^(E+24) -- every rounded step s + x is s plus x rounded to a multiple
//    of u (ties to an even multiple), so a stretch of steps is an integer
//    prefix sum in units of u and can be formed in parallel. A step whose
//    exact sum reaches 2^(E+24) (the grid coarsens) or whose x lies exactly
//    half way between two multiples (the tie depends on s) is done as the
//    one float addition it is. Which region a chunk of 64 terms starts in is
//    guessed from an approximate prefix and checked against the exact
//    running sum before the chunk's integer total is used, so a wrong guess
//    costs time, never bits.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

namespace DG_NS {

// ------------------------------------------------------------------ expf

// 2^(i/32) rounded to the nearest double, stored as its bit pattern minus
// i << 47, so that adding k << 47 for k = 32q + i scales it by 2^q.
__host__ __device__ inline uint64_t exp2_32_bits(uint32_t i) {
  static constexpr uint64_t tab[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
      0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
      0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
      0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
      0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
      0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
  };
  return tab[i & 31];
}

// expf as the reference's libm computes it (see the header comment). Also
// built for the host, where the tests compare it with the libm expf.
__host__ __device__ inline float expf_ref(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  const uint32_t abstop = (bits >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88, or x is inf or NaN
    if (bits == 0xff800000u) return 0.0f;           // -inf
    if (abstop >= 0x7f8) return x + x;              // +inf, NaN
    if (x > 0x1.62e42ep6f) return INFINITY;         // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;            // underflow
  }
  constexpr double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
  constexpr double shift = 0x1.8p+52;
  constexpr double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  constexpr double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  constexpr double c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  const double z = inv_ln2_32 * xd;
  double kd = z + shift;
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= shift;
  const double r = fma(inv_ln2_32, xd, -kd);
  const uint64_t t = exp2_32_bits((uint32_t)ki) + (ki << 47);
  double s;
  memcpy(&s, &t, 8);
  const double p = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(p, r2, y);
  y = y * s;
  return (float)y;
}

// sampler.rs:53-57: p = exp(l/T - m), 0 where l/T is NaN.
__device__ __forceinline__ float prob_term(float logit, float T, float m) {
  const float sv = logit / T;
  return isnan(sv) ? 0.0f : expf_ref(sv - m);
}

// ------------------------------------------------------------ grid regions

constexpr int GRID_MIN = -149;         // the subnormal spacing
constexpr uint32_t GRID_TOP = 1u << 24;  // multiples of u below 2^(E+24)
constexpr uint32_t SUM_EVENT = 0xFFFFFFu;  // chunk summary: no integer total

// Region of s >= 0: u = 2^E with s < 2^(E+24), s >= 2^(E+23) unless E is the
// smallest. s's float spacing is u throughout the region.
__device__ __forceinline__ int grid_of(float s) {
  const uint32_t ex = __float_as_uint(s) >> 23;
  return ex <= 1 ? GRID_MIN : (int)ex - 150;
}
// s in units of 2^E (exact: s is such a multiple, below 2^24 of them).
__device__ __forceinline__ uint32_t grid_units(float s, int E) {
  return (uint32_t)__builtin_ldexpf(s, -E);
}

// One term in the units of grid E: rho = x / u rounded to nearest even, a =
// floor(x / u); tie: x / u is exactly half way; big: x >= 2^(E+24) (the step
// always leaves the region).
struct GridTerm {
  uint32_t rho, a;
  bool tie, big;
};
__device__ __forceinline__ GridTerm grid_term(float x, int E) {
  GridTerm g;
  g.big = !(x < __builtin_ldexpf(1.0f, E + 24));
  const float t = g.big ? 0.0f : __builtin_ldexpf(x, -E);
  const float fl = floorf(t);
  g.rho = (uint32_t)rintf(t);
  g.a = (uint32_t)fl;
  g.tie = (t - fl) == 0.5f;
  return g;
}

// Summary word of a chunk whose running sum is expected in grid E: bits
// 31..24 hold E - GRID_MIN, bits 23..0 the chunk's total in units of 2^E, or
// SUM_EVENT where the chunk must be summed term by term.
__device__ __forceinline__ uint32_t sum_word(int E, uint32_t total) {
  return ((uint32_t)(E - GRID_MIN) << 24) | (total < SUM_EVENT ? total : SUM_EVENT);
}
__device__ __forceinline__ int sum_grid(uint32_t w) { return (int)(w >> 24) + GRID_MIN; }
__device__ __forceinline__ uint32_t sum_total(uint32_t w) { return w & 0xFFFFFFu; }

// ------------------------------------------------------------ wave helpers

// Inclusive prefix sum of a u32 over the 64 lanes: Hillis-Steele shifts
// within rows of 16, then row 0's total into row 1 and row 2's into row 3,
// then lane 31's into rows 2 and 3.
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, true);  // row_shr:8
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// The same scan of a float: a fixed tree of additions (the lanes' order of
// summation is set by the shifts), for approximate prefixes only.
__device__ __forceinline__ float wave_scan_f32(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
  return v;
}

__device__ __forceinline__ uint32_t lane_u32(uint32_t v, uint32_t lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)lane);
}
__device__ __forceinline__ float lane_f32(float v, uint32_t lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)lane));
}
// Lowest set lane of a ballot, 64 if none.
__device__ __forceinline__ uint32_t first_lane(unsigned long long m) {
  return m ? (uint32_t)__ffsll((long long)m) - 1u : 64u;
}

}  // namespace DG_NS
