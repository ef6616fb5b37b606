// Exact emulation of a sequential f32 running sum, computed by a whole
// workgroup in parallel.
//
// The reference sampler accumulates f32 sums one element at a time in a
// fixed order (softmax sum in index order, top-p cumulative sum in sorted
// order, inverse-CDF walk in index order). A parallel tree sum rounds
// differently, so this routine reproduces the sequential result bit-exactly.
//
// Facts it relies on, for non-negative summands and a running sum C >= 0:
//  * Inside one binade [2^e, 2^(e+1)) every representable value is a
//    multiple of the grid g = ulp(2^e), and the bit pattern of C grows by
//    exactly n when C grows by n*g (this also holds across the subnormal
//    range and into the first normal binade, where g = 2^-149 throughout).
//  * fl(C + x) for x >= 0 with C + x still inside the binade is C plus x
//    rounded onto the grid, ties to even on the integer C/g. The rounding
//    therefore depends only on the binade and on the parity of C/g, which
//    is the lowest bit of C's encoding.
//  * So a thread can run its own segment starting from the binade base B0
//    (even) and from B0 + g (odd) with ordinary hardware f32 adds: both runs
//    round exactly as the real sum would, provided the real sum stays inside
//    the binade. Each run yields an integer increment (in grid steps) as a
//    function of the incoming parity; these 2-entry maps compose
//    associatively, so a block scan gives every thread its exact start.
//  * When the real sum leaves the binade (at most once per binade, a few
//    dozen times per row), the thread containing the crossing replays its
//    segment with real adds from its exact start, and the threads after it
//    are redone with the new binade.
// Optional search: find the first element whose post-add sum satisfies
// `theta < C` (inverse-CDF walk) or `C >= theta` (top-p crossing).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lumen {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kSat = 1u << 30;

enum EcssMode : int { kEcssSum = 0, kEcssFindGt = 1, kEcssFindGe = 2 };

struct PMap {
  uint32_t a0, a1;  // grid-step increment when the incoming parity is 0 / 1
};

__device__ __forceinline__ PMap pm_combine(PMap L, PMap R) {
  PMap o;
  uint32_t c0 = L.a0 + ((L.a0 & 1u) ? R.a1 : R.a0);
  uint32_t c1 = L.a1 + ((L.a1 & 1u) ? R.a0 : R.a1);
  o.a0 = c0 > kSat ? kSat : c0;
  o.a1 = c1 > kSat ? kSat : c1;
  return o;
}

struct EcssShared {
  PMap wave_tot[kWaves];
  PMap wave_pre[kWaves];
  int red_b[kWaves];
  int red_h[kWaves];
  float bc_c;
  int bc_found;
  int bc_pos;
  float bc_before;
  float bc_at;
};

struct EcssResult {
  float c;       // running sum after the processed elements (or at the hit)
  int found;     // search hit in this chunk
  int pos;       // chunk-relative element index of the hit
  float before;  // running sum just before the hit element
};

__device__ __forceinline__ bool ecss_cond(int mode, float c, float theta) {
  return mode == kEcssFindGt ? (theta < c) : (c >= theta);
}

// Exclusive block scan of parity maps (identity = {0,0}).
__device__ __forceinline__ PMap block_excl_scan(PMap v, EcssShared& sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  PMap inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    PMap L;
    L.a0 = __shfl_up(inc.a0, d, 64);
    L.a1 = __shfl_up(inc.a1, d, 64);
    if (lane >= d) inc = pm_combine(L, inc);
  }
  if (lane == 63) sh.wave_tot[w] = inc;
  __syncthreads();
  if (w == 0) {
    PMap t = (lane < kWaves) ? sh.wave_tot[lane] : PMap{0u, 0u};
    PMap ti = t;
#pragma unroll
    for (int d = 1; d < kWaves; d <<= 1) {
      PMap L;
      L.a0 = __shfl_up(ti.a0, d, 64);
      L.a1 = __shfl_up(ti.a1, d, 64);
      if (lane >= d) ti = pm_combine(L, ti);
    }
    PMap ex;
    ex.a0 = __shfl_up(ti.a0, 1, 64);
    ex.a1 = __shfl_up(ti.a1, 1, 64);
    if (lane == 0) ex = PMap{0u, 0u};
    if (lane < kWaves) sh.wave_pre[lane] = ex;
  }
  __syncthreads();
  PMap ex;
  ex.a0 = __shfl_up(inc.a0, 1, 64);
  ex.a1 = __shfl_up(inc.a1, 1, 64);
  if (lane == 0) ex = PMap{0u, 0u};
  return pm_combine(sh.wave_pre[w], ex);
}

// One chunk: thread t holds x[0..M) = chunk elements t*M .. t*M+M-1, all
// finite and >= 0 (zero for padding). `c` is the exact sequential sum of
// everything before the chunk. Uniform result across the block.
template <int M>
__device__ __forceinline__ EcssResult ecss_chunk(float c, const float (&x)[M], int mode, float theta,
                                 EcssShared& sh) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int t0 = 0;
  for (;;) {
    const uint32_t cb = __float_as_uint(c);
    const uint32_t b0 = cb & 0xff800000u;
    const uint32_t ub = b0 + 0x00800000u;
    PMap m{0u, 0u};
    if (t >= t0) {
      float y0 = __uint_as_float(b0), y1 = __uint_as_float(b0 | 1u);
#pragma unroll
      for (int j = 0; j < M; ++j) {
        y0 = __fadd_rn(y0, x[j]);
        y1 = __fadd_rn(y1, x[j]);
      }
      uint32_t n0 = __float_as_uint(y0) - b0, n1 = __float_as_uint(y1) - (b0 | 1u);
      m.a0 = n0 > kSat ? kSat : n0;
      m.a1 = n1 > kSat ? kSat : n1;
    }
    PMap ex = block_excl_scan(m, sh);
    const uint32_t par0 = cb & 1u;
    const uint32_t before = par0 ? ex.a1 : ex.a0;
    const uint32_t par_t = (par0 ^ before) & 1u;
    const uint32_t own = par_t ? m.a1 : m.a0;
    const uint32_t sbits = cb + before;  // <= 0x7f800000 + 2^30: no wrap
    const uint32_t ebits = sbits + own;  // <= 0x7f800000 + 2^31: no wrap
    const bool act = t >= t0;
    const bool cross = act && (before >= kSat || ebits >= ub);
    const bool hit = act && !cross && mode != kEcssSum && ecss_cond(mode, __uint_as_float(ebits), theta);
    // first crossing / first hit thread
    unsigned long long bm = __ballot(cross), hm = __ballot(hit);
    if (lane == 0) {
      sh.red_b[w] = bm ? (w * 64 + __ffsll((long long)bm) - 1) : kThreads;
      sh.red_h[w] = hm ? (w * 64 + __ffsll((long long)hm) - 1) : kThreads;
    }
    __syncthreads();
    int tb = kThreads, th = kThreads;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      tb = min(tb, sh.red_b[i]);
      th = min(th, sh.red_h[i]);
    }
    EcssResult res;
    if (th < tb) {
      // the search target lies inside thread th, whose start is exact
      if (t == th) {
        float y = __uint_as_float(sbits), prev = y;
        int j = M;
#pragma unroll
        for (int q = 0; q < M; ++q) {
          if (j == M) {
            prev = y;
            y = __fadd_rn(y, x[q]);
            if (ecss_cond(mode, y, theta)) j = q;
          }
        }
        sh.bc_found = 1;
        sh.bc_pos = th * M + j;
        sh.bc_c = y;
        sh.bc_before = prev;
      }
      __syncthreads();
      res.c = sh.bc_c;
      res.found = 1;
      res.pos = sh.bc_pos;
      res.before = sh.bc_before;
      __syncthreads();
      return res;
    }
    if (tb == kThreads) {
      if (t == kThreads - 1) sh.bc_c = __uint_as_float(ebits);
      __syncthreads();
      res.c = sh.bc_c;
      res.found = 0;
      res.pos = -1;
      res.before = 0.f;
      __syncthreads();
      return res;
    }
    // binade crossing inside thread tb: replay it exactly
    if (t == tb) {
      float y = __uint_as_float(sbits), prev = y;
      int f = 0, j = M;
#pragma unroll
      for (int q = 0; q < M; ++q) {
        if (!f) {
          prev = y;
          y = __fadd_rn(y, x[q]);
          if (mode != kEcssSum && ecss_cond(mode, y, theta)) {
            f = 1;
            j = q;
          }
        }
      }
      sh.bc_c = y;
      sh.bc_found = f;
      sh.bc_pos = tb * M + j;
      sh.bc_before = prev;
    }
    __syncthreads();
    c = sh.bc_c;
    if (sh.bc_found) {
      res.c = c;
      res.found = 1;
      res.pos = sh.bc_pos;
      res.before = sh.bc_before;
      __syncthreads();
      return res;
    }
    __syncthreads();
    t0 = tb + 1;
    if (t0 >= kThreads) {
      res.c = c;
      res.found = 0;
      res.pos = -1;
      res.before = 0.f;
      return res;
    }
  }
}

}  // namespace lumen
