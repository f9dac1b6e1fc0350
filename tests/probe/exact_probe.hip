// exact_probe.hip -- TEST INFRASTRUCTURE: entry points into the exact
// sampler's device code (defer_amd/csrc/exact.h, phases.h) on arbitrary
// inputs, for tests/test_exact.py. Not part of the library or its ABI.
//
//   probe_expf_sweep   host build of expf_ref against the libm expf, over
//                      every stride-th float bit pattern from first on;
//   probe_expf_device  the device expf_ref on an array;
//   probe_scan_device  wave_scan_u32 on 64-lane groups of an array;
//   probe_walk         the exact sampler's stages A2 to W2 (sample_exact,
//                      one workgroup) on an arbitrary term sequence p: the
//                      sequential float total of p, and the index
//                      sample_token's scan returns over q = p * (1/total)
//                      for the draw r = (word >> 8) * 2^-24.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../defer_amd/csrc/phases.h"

using namespace dg;

extern "C" int probe_expf_sweep(uint32_t first, uint64_t count, uint32_t stride, uint64_t* n_diff,
                                uint32_t* first_diff) {
  uint64_t nd = 0;
  uint32_t fd = 0;
  uint64_t u = first;
  for (uint64_t i = 0; i < count; ++i, u += stride) {
    const uint32_t w = (uint32_t)u;
    float x;
    memcpy(&x, &w, 4);
    const float a = expf(x), b = expf_ref(x);
    uint32_t ab, bb;
    memcpy(&ab, &a, 4);
    memcpy(&bb, &b, 4);
    if (ab != bb && !(isnan(a) && isnan(b))) {
      if (!nd) fd = w;
      ++nd;
    }
  }
  *n_diff = nd;
  *first_diff = fd;
  return 0;
}

__global__ void k_expf(const float* x, float* y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = expf_ref(x[i]);
}

extern "C" int probe_expf_device(const float* x, float* y, size_t n) {
  float *dx = nullptr, *dy = nullptr;
  if (hipMalloc(&dx, n * 4) || hipMalloc(&dy, n * 4)) return 1;
  (void)hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice);
  k_expf<<<(unsigned)((n + 255) / 256), 256>>>(dx, dy, n);
  const int rc = hipMemcpy(y, dy, n * 4, hipMemcpyDeviceToHost) != hipSuccess;
  (void)hipFree(dx);
  (void)hipFree(dy);
  return rc;
}

__global__ void k_scan(const uint32_t* x, uint32_t* y, uint32_t n) {
  const uint32_t i = blockIdx.x * 64 + threadIdx.x;
  const uint32_t v = i < n ? x[i] : 0u;
  const uint32_t s = wave_scan_u32(v);
  if (i < n) y[i] = s;
}

extern "C" int probe_scan_device(const uint32_t* x, uint32_t* y, uint32_t n) {
  uint32_t *dx = nullptr, *dy = nullptr;
  if (hipMalloc(&dx, n * 4) || hipMalloc(&dy, n * 4)) return 1;
  (void)hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice);
  k_scan<<<(n + 63) / 64, 64>>>(dx, dy, n);
  const int rc = hipMemcpy(y, dy, n * 4, hipMemcpyDeviceToHost) != hipSuccess;
  (void)hipFree(dx);
  (void)hipFree(dy);
  return rc;
}

// One workgroup: the sampler's stages A2 to W2 (sample_exact) on terms p
// already published with their chunk sums, as the batched sampler runs them.
__global__ __launch_bounds__(BLOCK) void k_walk(const Args* __restrict__ ap, uint32_t tag, uint32_t word,
                                                uint32_t* out) {
  extern __shared__ float lds_raw[];
  const Args& a = *ap;
  Lds s;
  memset(&s, 0, sizeof(s));
  s.ctl = reinterpret_cast<WaitCtl*>(lds_raw);
  s.red = lds_raw + 4;
  s.scr = lds_raw + 4 + 64;
  if (threadIdx.x == 0) s.ctl->abort_seen = 0;
  __syncthreads();
  uint32_t sum_bits = 0, tok = 0;
  if (!sample_exact(a, tag, 0.0f, 0u, word, 0, 1, false, s, &tok, &sum_bits)) return;
  if (threadIdx.x == 0) {
    out[0] = sum_bits;
    out[1] = tok;
  }
}

// p: n terms >= 0 (finite); words: n_words draws, each its own sampling
// event (its own tag). For each draw: out[2i] the total's bits, out[2i + 1]
// the index.
extern "C" int probe_walk(const float* p, uint32_t n, const uint32_t* words, uint32_t n_words, uint32_t* out) {
  const uint32_t nvc = (n + VCHUNK - 1) / VCHUNK;
  std::vector<u64> hp(n), hs(nvc);
  std::vector<uint32_t> sums(nvc), bits(n);
  for (uint32_t c = 0; c < nvc; ++c) {
    float sum = 0.0f;  // any order: only the spacing guesses use it
    for (uint32_t j = c * VCHUNK; j < n && j < (c + 1) * VCHUNK; ++j) sum += p[j];
    memcpy(&sums[c], &sum, 4);
  }
  memcpy(bits.data(), p, (size_t)n * 4);
  u64 *dp = nullptr, *ds = nullptr;  // p words; chunk sums, then the two summary arrays
  DevState* st = nullptr;
  Args* da = nullptr;
  uint32_t* dout = nullptr;
  int rc = 1;
  if (hipMalloc(&dp, (size_t)n * 8) || hipMalloc(&ds, 3 * (size_t)nvc * 8) ||
      hipMalloc(&st, sizeof(DevState)) || hipMalloc(&da, sizeof(Args)) || hipMalloc(&dout, 8))
    goto done;
  {
    Args a;
    memset(&a, 0, sizeof(a));
    a.d.V = n;
    a.d.nvc = nvc;
    a.mb_p = dp;
    a.mb_vsum = ds;
    a.mb_psum = ds + nvc;
    a.mb_qsum = ds + 2 * nvc;
    a.st = st;
    (void)hipMemset(ds, 0, 3 * (size_t)nvc * 8);
    (void)hipMemset(st, 0, sizeof(DevState));
    (void)hipMemcpy(da, &a, sizeof(Args), hipMemcpyHostToDevice);
    const size_t lds = (4 + 64 + samp_lds_floats(nvc, 0, 0)) * sizeof(float);
    for (uint32_t i = 0; i < n_words; ++i) {
      const u64 tag = 7 + i;
      for (uint32_t c = 0; c < nvc; ++c) hs[c] = (tag << 32) | sums[c];
      for (uint32_t j = 0; j < n; ++j) hp[j] = (tag << 32) | bits[j];
      (void)hipMemcpy(dp, hp.data(), (size_t)n * 8, hipMemcpyHostToDevice);
      (void)hipMemcpy(ds, hs.data(), (size_t)nvc * 8, hipMemcpyHostToDevice);
      (void)hipMemset(dout, 0xff, 8);
      k_walk<<<1, BLOCK, lds>>>(da, (uint32_t)tag, words[i], dout);
      if (hipMemcpy(out + 2 * i, dout, 8, hipMemcpyDeviceToHost) != hipSuccess) goto done;
    }
    DevState h;
    (void)hipMemcpy(&h, st, sizeof(h), hipMemcpyDeviceToHost);
    rc = h.abort ? 2 : 0;
  }
done:
  (void)hipFree(dp);
  (void)hipFree(ds);
  (void)hipFree(st);
  (void)hipFree(da);
  (void)hipFree(dout);
  return rc;
}
