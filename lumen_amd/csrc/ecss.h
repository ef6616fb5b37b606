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

#include "wave.h"

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
  const PMap id{0u, 0u};
  const PMap inc = wave_scan_incl(v, id, pm_combine);
  if (lane == 63) sh.wave_tot[w] = inc;
  __syncthreads();
  if (w == 0) {
    const PMap t = (lane < kWaves) ? sh.wave_tot[lane] : id;
    const PMap ex = wave_shr1(wave_scan_incl(t, id, pm_combine), id);
    if (lane < kWaves) sh.wave_pre[lane] = ex;
  }
  __syncthreads();
  return pm_combine(sh.wave_pre[w], wave_shr1(inc, id));
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

// ---------------------------------------------------------------------------
// One-wave variant for short lists: lane l holds elements l*M .. l*M+M-1.
// The same parity-map method with a DPP wave scan instead of a block scan,
// so a binade crossing costs one wave scan and no workgroup barrier. Must
// be called by all 64 lanes of one wave; the result is uniform across it.
template <int M>
__device__ __forceinline__ EcssResult wave_ecss(float c, const float (&x)[M], int mode, float theta) {
  const int lane = threadIdx.x & 63;
  int t0 = 0;
  EcssResult res;
  for (;;) {
    const uint32_t cb = __float_as_uint(c);
    const uint32_t b0 = cb & 0xff800000u;
    const uint32_t ub = b0 + 0x00800000u;
    PMap m{0u, 0u};
    if (lane >= t0) {
      float y0 = __uint_as_float(b0), y1 = __uint_as_float(b0 | 1u);
#pragma unroll
      for (int j = 0; j < M; ++j) {
        y0 = __fadd_rn(y0, x[j]);
        y1 = __fadd_rn(y1, x[j]);
      }
      const uint32_t n0 = __float_as_uint(y0) - b0, n1 = __float_as_uint(y1) - (b0 | 1u);
      m.a0 = n0 > kSat ? kSat : n0;
      m.a1 = n1 > kSat ? kSat : n1;
    }
    const PMap id{0u, 0u};
    const PMap ex = wave_shr1(wave_scan_incl(m, id, pm_combine), id);
    const uint32_t par0 = cb & 1u;
    const uint32_t before = par0 ? ex.a1 : ex.a0;
    const uint32_t own = ((par0 ^ before) & 1u) ? m.a1 : m.a0;
    const uint32_t sbits = cb + before;
    const uint32_t ebits = sbits + own;
    const bool act = lane >= t0;
    const bool cross = act && (before >= kSat || ebits >= ub);
    const bool hit = act && !cross && mode != kEcssSum && ecss_cond(mode, __uint_as_float(ebits), theta);
    const unsigned long long bm = __ballot(cross), hm = __ballot(hit);
    const int tb = bm ? __ffsll((long long)bm) - 1 : 64;
    const int th = hm ? __ffsll((long long)hm) - 1 : 64;
    if (th < tb || tb < 64) {
      // lane r (the hit, or the crossing) replays its elements from its exact start
      const int r = th < tb ? th : tb;
      float y = __uint_as_float(sbits), prev = y;
      int j = M;
#pragma unroll
      for (int q = 0; q < M; ++q) {
        if (j == M) {
          prev = y;
          y = __fadd_rn(y, x[q]);
          if (mode != kEcssSum && ecss_cond(mode, y, theta)) j = q;
        }
      }
      const int jr = __builtin_amdgcn_readlane(j, r);
      const float yr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(y), r));
      if (jr < M) {
        res.c = yr;
        res.found = 1;
        res.pos = r * M + jr;
        res.before = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prev), r));
        return res;
      }
      c = yr;
      t0 = r + 1;
      if (t0 < 64) continue;
      res.c = c;
    } else {
      res.c = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)ebits, 63));
    }
    res.found = 0;
    res.pos = -1;
    res.before = 0.f;
    return res;
  }
}

// ---------------------------------------------------------------------------
// Estimate-guided variant: no block scan per binade crossing.
//
// ecss_chunk pays one block scan each time the running sum changes binade,
// and a sum that starts small changes binade dozens of times. Here each
// thread also has an f64 estimate of the running sum at its start, so the
// threads whose segment may see a binade change are known in advance
// ("boundary" threads); every other thread's binade is known and it builds
// its parity map for that binade only. One segmented block scan (runs of
// non-boundary threads) composes the maps; then one thread walks the runs
// and boundaries in order: a run advances the sum through its composed map,
// a boundary thread is replayed with real f32 adds from its exact start.
// Every step is checked (the sum must be in the run's binade and must not
// leave it); a failed check makes the caller fall back to ecss_chunk, so the
// estimates decide speed only, never the result.

constexpr int kEstMaxB = 128;    // boundary threads per chunk
constexpr int kEstBx = 1024;     // boundary summands kept in LDS
constexpr uint32_t kEmptyRun = 0xffffffffu;

struct EstShared {
  int nb;
  int fail;
  int hit_seg;      // search hit inside run hit_seg (-1: none)
  int hit_pos;      // or at this chunk element, inside a boundary thread (-1: none)
  float c_out;      // sum after the chunk (or at the hit)
  float c_seg;      // exact sum at the start of run hit_seg
  float before;     // sum before the hit element
  uint32_t wave_head[2 * kWaves];
  uint32_t wave_lastb[kWaves];
  uint32_t wave_lastbin[kWaves];
  uint16_t bpos[kEstMaxB];
  uint32_t seg_bin[kEstMaxB + 1];
  PMap seg_tot[kEstMaxB + 1];
  float bx[kEstBx];
  // ecss_chunk4: per-wave summaries and their exclusive prefixes
  uint32_t xw[4][kWaves];
  PMap xm[kWaves];
  uint32_t pxh[kWaves], pxc[kWaves];
  PMap pxm[kWaves];
};

struct SegVal {
  uint32_t head;  // 1: a boundary thread (runs restart after it)
  PMap m;
};

__device__ __forceinline__ SegVal seg_combine(SegVal L, SegVal R) {
  if (R.head) return R;
  SegVal o;
  o.head = L.head;
  o.m = pm_combine(L.m, R.m);
  return o;
}

__device__ __forceinline__ uint32_t est_binade(double x) {
  float f = __double2float_rz(x > 0.0 ? x : 0.0);
  return __float_as_uint(f) & 0xff800000u;
}

// Inclusive segmented block scan; *prev receives the inclusive value of the
// previous thread (identity for thread 0).
__device__ __forceinline__ SegVal seg_scan_incl(SegVal v, EcssShared& sh, EstShared& es,
                                                SegVal* prev) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const SegVal id{0u, PMap{0u, 0u}};
  const SegVal inc = wave_scan_incl(v, id, seg_combine);
  if (lane == 63) {
    sh.wave_tot[w] = inc.m;
    es.wave_head[w] = inc.head;
  }
  __syncthreads();
  if (w == 0) {
    SegVal t;
    t.head = lane < kWaves ? es.wave_head[lane] : 0u;
    t.m = lane < kWaves ? sh.wave_tot[lane] : PMap{0u, 0u};
    const SegVal ex = wave_shr1(wave_scan_incl(t, id, seg_combine), id);
    if (lane < kWaves) {
      sh.wave_pre[lane] = ex.m;
      es.wave_head[kWaves + lane] = ex.head;
    }
  }
  __syncthreads();
  SegVal pre;
  pre.head = es.wave_head[kWaves + w];
  pre.m = sh.wave_pre[w];
  const SegVal in_w = wave_shr1(inc, id);
  const SegVal r = seg_combine(pre, inc);
  *prev = seg_combine(pre, in_w);
  __syncthreads();
  return r;
}

struct EstThread {
  uint32_t boundary;
  uint32_t bin;   // binade base of a non-boundary thread
  PMap own;       // its parity map for that binade
  PMap excl;      // composition of its run before it
  int run;        // index of its run (= boundaries before it)
};

// Builds runs and boundaries. x: this thread's M summands; p_start / d_self:
// estimated sum at the thread's start and of its own summands; rel_err: the
// assumed relative error of p_start. Returns false (uniform) if the result
// does not fit the LDS budget (the caller then uses ecss_chunk).
template <int M>
__device__ __forceinline__ bool est_prepare(const float (&x)[M], double p_start, double d_self,
                                            double rel_err, EcssShared& sh, EstShared& es,
                                            EstThread& et, int nact = kThreads) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const uint32_t blo = est_binade(p_start * (1.0 - rel_err));
  const uint32_t bhi = est_binade((p_start + d_self) * (1.0 + rel_err));
  // threads from nact on hold only zero padding: identity maps, never
  // boundaries, and the last run ends at thread nact - 1
  et.boundary = (blo != bhi && t < nact) ? 1u : 0u;
  et.bin = blo;
  et.own = PMap{0u, 0u};
  if (!et.boundary) {
    float y0 = __uint_as_float(blo), y1 = __uint_as_float(blo | 1u);
#pragma unroll
    for (int j = 0; j < M; ++j) {
      y0 = __fadd_rn(y0, x[j]);
      y1 = __fadd_rn(y1, x[j]);
    }
    const uint32_t n0 = __float_as_uint(y0) - blo, n1 = __float_as_uint(y1) - (blo | 1u);
    et.own.a0 = n0 > kSat ? kSat : n0;
    et.own.a1 = n1 > kSat ? kSat : n1;
  }
  const unsigned long long bm = __ballot(et.boundary != 0u);
  if (lane == 0) sh.red_b[w] = __popcll(bm);
  if (lane == 63) {
    es.wave_lastb[w] = et.boundary;
    es.wave_lastbin[w] = et.bin;
  }
  __syncthreads();
  int before_w = 0, nb = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    before_w += (i < w) ? sh.red_b[i] : 0;
    nb += sh.red_b[i];
  }
  et.run = before_w + __popcll(bm & ((1ull << lane) - 1ull));
  SegVal v{et.boundary, et.own};
  SegVal prev;
  SegVal inc = seg_scan_incl(v, sh, es, &prev);

  et.excl = (t == 0) ? PMap{0u, 0u} : prev.m;
  const bool fits = nb <= kEstMaxB && nb * M <= kEstBx;
  if (fits) {
    // predecessor's boundary flag and binade
    uint32_t pb = wave_shr1(et.boundary, 0u), pbin = wave_shr1(et.bin, 0u);
    if (lane == 0 && w > 0) {
      pb = es.wave_lastb[w - 1];
      pbin = es.wave_lastbin[w - 1];
    }
    if (et.boundary) {
      const int k = et.run;
      es.bpos[k] = (uint16_t)t;
      const bool empty = (t == 0) || pb;
      es.seg_tot[k] = empty ? PMap{0u, 0u} : prev.m;
      es.seg_bin[k] = empty ? kEmptyRun : pbin;
#pragma unroll
      for (int j = 0; j < M; ++j) es.bx[k * M + j] = x[j];
    }
    if (t == nact - 1) {
      es.nb = nb;
      es.seg_tot[nb] = et.boundary ? PMap{0u, 0u} : inc.m;
      es.seg_bin[nb] = et.boundary ? kEmptyRun : et.bin;
    }
  }
  __syncthreads();
  return fits;
}

// Sequential walk over runs and boundaries (thread 0), then the exact search
// inside a run when the hit lies there. Returns false (uniform) when a check
// failed. On success *res holds the chunk result.
template <int M>
__device__ __forceinline__ bool est_resolve(float c_in, const float (&x)[M], int mode, float theta,
                                            const EstThread& et, EcssShared& sh, EstShared& es,
                                            EcssResult* res) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  if (w == 0) {
    const int nb = es.nb;
    // Up to 63 boundaries: lane k holds run k and boundary k in registers
    // (one LDS round trip), and the walk reads them with v_readlane, so the
    // sequential part has no memory latency. All lanes run the walk (the
    // values are uniform); lane 0 publishes it.
    const bool regs = nb < 64;
    uint32_t sb_r = 0, a0_r = 0, a1_r = 0, bp_r = 0;
    float bx_r[M];
#pragma unroll
    for (int q = 0; q < M; ++q) bx_r[q] = 0.f;
    if (regs) {
      if (lane <= nb) {
        sb_r = es.seg_bin[lane];
        a0_r = es.seg_tot[lane].a0;
        a1_r = es.seg_tot[lane].a1;
      }
      if (lane < nb) {
        bp_r = es.bpos[lane];
#pragma unroll
        for (int q = 0; q < M; ++q) bx_r[q] = es.bx[lane * M + q];
      }
    }
    float c = c_in;
    int fail = 0, hit_seg = -1, hit_pos = -1;
    float before = 0.f, cseg = 0.f;
    if (regs) {
      // Branch-free walk. The only dependent chain per boundary is the
      // parity-selected run increment and the M sequential adds; the checks
      // and the first stop (failure, hit inside a run, hit inside a
      // boundary) are recorded with selects off that chain.
      bool stopped = false;
      for (int k = 0; k <= nb; ++k) {
        const uint32_t sb = (uint32_t)__builtin_amdgcn_readlane((int)sb_r, k);
        const uint32_t m0 = (uint32_t)__builtin_amdgcn_readlane((int)a0_r, k);
        const uint32_t m1 = (uint32_t)__builtin_amdgcn_readlane((int)a1_r, k);
        const uint32_t cb = __float_as_uint(c);
        const uint32_t inc = (cb & 1u) ? m1 : m0;
        const uint32_t nbits = cb + inc;
        const bool run = sb != kEmptyRun;
        const bool bad = run && ((cb & 0xff800000u) != sb || inc >= kSat || nbits >= sb + 0x00800000u);
        const bool hs = run && !bad && mode != kEcssSum && ecss_cond(mode, __uint_as_float(nbits), theta);
        if (!stopped && bad) fail = 1;
        if (!stopped && hs) {
          hit_seg = k;
          cseg = c;
        }
        stopped = stopped || bad || hs;
        const float cr = run ? __uint_as_float(nbits) : c;
        float ys[M];
        float y = cr;
#pragma unroll
        for (int q = 0; q < M; ++q) {
          y = __fadd_rn(y, __int_as_float(__builtin_amdgcn_readlane(
                              __float_as_int(bx_r[q]), k < nb ? k : 0)));
          ys[q] = y;
        }
        if (mode != kEcssSum && k < nb) {
          int j = M;
#pragma unroll
          for (int q = M - 1; q >= 0; --q) j = ecss_cond(mode, ys[q], theta) ? q : j;
          if (!stopped && j < M) {
            hit_pos = (int)__builtin_amdgcn_readlane((int)bp_r, k) * M + j;
            float pb = cr;
#pragma unroll
            for (int q = 1; q < M; ++q) pb = (q == j) ? ys[q - 1] : pb;
            before = pb;
            float yh = ys[0];
#pragma unroll
            for (int q = 1; q < M; ++q) yh = (q == j) ? ys[q] : yh;
            c = yh;
            stopped = true;
          }
        }
        if (!stopped) c = k < nb ? y : cr;
      }
    } else {
      for (int k = 0; k <= nb && !fail && hit_seg < 0 && hit_pos < 0; ++k) {
        const uint32_t sb = es.seg_bin[k];
        if (sb != kEmptyRun) {
          const uint32_t cb = __float_as_uint(c);
          if ((cb & 0xff800000u) != sb) {
            fail = 1;
            break;
          }
          const uint32_t inc = (cb & 1u) ? es.seg_tot[k].a1 : es.seg_tot[k].a0;
          const uint32_t nbits = cb + inc;
          if (inc >= kSat || nbits >= sb + 0x00800000u) {
            fail = 1;
            break;
          }
          if (mode != kEcssSum && ecss_cond(mode, __uint_as_float(nbits), theta)) {
            hit_seg = k;
            cseg = c;
            break;
          }
          c = __uint_as_float(nbits);
        }
        if (k == nb) break;
        float y = c, p = c;
        int j = M;
#pragma unroll
        for (int q = 0; q < M; ++q) {
          if (j == M) {
            p = y;
            y = __fadd_rn(y, es.bx[k * M + q]);
            if (mode != kEcssSum && ecss_cond(mode, y, theta)) j = q;
          }
        }
        c = y;
        if (j < M) {
          hit_pos = (int)es.bpos[k] * M + j;
          before = p;
        }
      }
    }
    if (lane == 0) {
      es.fail = fail;
      es.hit_seg = hit_seg;
      es.hit_pos = hit_pos;
      es.c_out = c;
      es.c_seg = cseg;
      es.before = before;
    }
  }
  __syncthreads();
  const int fail = es.fail, hit_seg = es.hit_seg, hit_pos = es.hit_pos;
  res->c = es.c_out;
  res->before = es.before;
  res->found = hit_pos >= 0 ? 1 : 0;
  res->pos = hit_pos;
  if (fail) {
    __syncthreads();
    return false;
  }
  if (hit_seg >= 0) {
    // exact starts inside the run, then the first thread whose end meets the target
    const float cs = es.c_seg;
    const uint32_t cb = __float_as_uint(cs);
    const bool in = !et.boundary && et.run == hit_seg;
    uint32_t sbits = 0, ebits = 0;
    if (in) {
      const uint32_t b = (cb & 1u) ? et.excl.a1 : et.excl.a0;
      sbits = cb + b;
      const uint32_t own = ((cb ^ b) & 1u) ? et.own.a1 : et.own.a0;
      ebits = sbits + own;
    }
    const bool h = in && ecss_cond(mode, __uint_as_float(ebits), theta);
    const unsigned long long hm = __ballot(h);
    if (lane == 0) sh.red_h[w] = hm ? (w * 64 + __ffsll((long long)hm) - 1) : kThreads;
    __syncthreads();
    int th = kThreads;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) th = min(th, sh.red_h[i]);
    if (t == th) {
      float y = __uint_as_float(sbits), p = y;
      int j = M;
#pragma unroll
      for (int q = 0; q < M; ++q) {
        if (j == M) {
          p = y;
          y = __fadd_rn(y, x[q]);
          if (ecss_cond(mode, y, theta)) j = q;
        }
      }
      es.hit_pos = th * M + j;
      es.c_out = y;
      es.before = p;
    }
    __syncthreads();
    res->found = 1;
    res->pos = es.hit_pos;
    res->c = es.c_out;
    res->before = es.before;
  }
  __syncthreads();
  return true;
}

// Full chunk with the estimate-guided method and the exact fallback. The
// estimates come from the summands: p(t) = c + sum of the summands before
// thread t in this chunk, exact enough that only threads within the chunk's
// worst-case rounding drift of a binade edge become boundaries.
template <int M>
__device__ __forceinline__ EcssResult ecss_fast_chunk(float c, const float (&x)[M], int mode,
                                                      float theta, EcssShared& sh, EstShared& es,
                                                      double* wsum, int nact = kThreads) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  double d = 0.0;
#pragma unroll
  for (int j = 0; j < M; ++j) d += (double)x[j];
  // exclusive f64 block scan of d
  const double inc = wave_scan_incl(d, 0.0, [](double l, double r) { return l + r; });
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  double pre = 0.0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) pre += i < w ? wsum[i] : 0.0;
  __syncthreads();
  const double p_start = (double)c + pre + inc - d;
  const double rel = (double)((t + 1) * M) * 0x1.0p-24 * 1.01 + 1e-9;
  EstThread et;
  EcssResult r;
  if (!est_prepare<M>(x, p_start, d, rel, sh, es, et, nact)) {
    if (t == 0) es.fail = 2;  // structure did not fit (diagnostic only)
    return ecss_chunk<M>(c, x, mode, theta, sh);
  }
  if (est_resolve<M>(c, x, mode, theta, et, sh, es, &r)) {
    return r;
  }
  return ecss_chunk<M>(c, x, mode, theta, sh);
}

// ---------------------------------------------------------------------------
// The estimate-guided method for one chunk of at most 4 * kThreads summands
// (thread t holds x[4] = chunk elements 4t .. 4t+3, zero past the end; the
// first nact threads hold any), from the exact running sum c. Same method as
// ecss_fast_chunk, with each cross-wave step (the f64 prefix, the segmented
// composition of runs, the boundary ordinals) done once by wave 0 instead
// of by every thread, and the runs, boundaries and their summands gathered
// so that the walk on wave 0 reads them from its registers. The drift bound
// is rigorous (each add rounds by at most 2^-24 of the running sum, which
// never decreases), so the estimate only decides which threads are replayed;
// a walk check that fails anyway falls back to ecss_chunk.
__device__ __forceinline__ double dadd(double l, double r) { return l + r; }

__device__ __forceinline__ EcssResult ecss_chunk4(float c, const float (&x)[4], int mode,
                                                  float theta, int nact, EcssShared& sh,
                                                  EstShared& es) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const bool act = t < nact;
  // 1. f64 estimate of the running sum at each thread's start
  const double d = ((double)x[0] + (double)x[1]) + ((double)x[2] + (double)x[3]);
  const double winc = wave_scan_incl(d, 0.0, dadd);
  double* dw = reinterpret_cast<double*>(sh.wave_tot);
  double* dp = reinterpret_cast<double*>(sh.wave_pre);
  if (lane == 63) dw[w] = winc;
  __syncthreads();
  if (w == 0) {
    const double v = lane < kWaves ? dw[lane] : 0.0;
    const double vi = wave_scan_incl(v, 0.0, dadd);
    if (lane < kWaves) dp[lane] = vi - v;
  }
  __syncthreads();
  const double P = (double)c + dp[w] + (winc - d);

  const double rel = (double)(4 * t + 4) * 0x1.0p-24 * 1.001 + 1e-12;
  const uint32_t lo = est_binade(P * (1.0 - rel));
  const uint32_t hi = est_binade((P + d) * (1.0 + rel));
  const bool bnd = act && lo != hi;
  PMap m{0u, 0u};
  if (act && !bnd) {
    float y0 = __uint_as_float(lo), y1 = __uint_as_float(lo | 1u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      y0 = __fadd_rn(y0, x[j]);
      y1 = __fadd_rn(y1, x[j]);
    }
    const uint32_t n0 = __float_as_uint(y0) - lo, n1 = __float_as_uint(y1) - (lo | 1u);
    m.a0 = n0 > kSat ? kSat : n0;
    m.a1 = n1 > kSat ? kSat : n1;
  }
  // 2. runs of certain threads between boundary threads
  const SegVal id{0u, PMap{0u, 0u}};
  const SegVal inc = wave_scan_incl(SegVal{bnd ? 1u : 0u, m}, id, seg_combine);
  const unsigned long long bm = __ballot(bnd);
  if (lane == 63) {
    es.xw[0][w] = inc.head;
    es.xm[w] = inc.m;
    es.xw[1][w] = (uint32_t)__popcll(bm);
    es.xw[2][w] = bnd ? 1u : 0u;
    es.xw[3][w] = lo;
  }
  __syncthreads();
  if (w == 0) {
    const SegVal v = lane < kWaves ? SegVal{es.xw[0][lane], es.xm[lane]} : id;
    const SegVal ex = wave_shr1(wave_scan_incl(v, id, seg_combine), id);
    const uint32_t cn = lane < kWaves ? es.xw[1][lane] : 0u;
    const uint32_t ci = wave_scan_incl(cn, 0u, [](uint32_t l, uint32_t r) { return l + r; });
    if (lane < kWaves) {
      es.pxh[lane] = ex.head;
      es.pxm[lane] = ex.m;
      es.pxc[lane] = ci - cn;
    }
    if (lane == kWaves - 1) es.nb = (int)ci;
  }
  __syncthreads();
  const SegVal ex = seg_combine(SegVal{es.pxh[w], es.pxm[w]}, wave_shr1(inc, id));
  const uint32_t bidx = es.pxc[w] + (uint32_t)__popcll(bm & ((1ull << lane) - 1ull));
  const int nb = es.nb;

  if (nb > 63) {
    __syncthreads();
    return ecss_chunk<4>(c, x, mode, theta, sh);
  }
  uint32_t pb = wave_shr1(bnd ? 1u : 0u, 1u), plo = wave_shr1(lo, 0u);
  if (lane == 0) {
    pb = w > 0 ? es.xw[2][w - 1] : 1u;
    plo = w > 0 ? es.xw[3][w - 1] : 0u;
  }
  if (bnd) {
    es.seg_bin[bidx] = pb ? kEmptyRun : plo;
    es.seg_tot[bidx] = pb ? PMap{0u, 0u} : ex.m;
    es.bpos[bidx] = (uint16_t)t;
#pragma unroll
    for (int j = 0; j < 4; ++j) es.bx[4u * bidx + (uint32_t)j] = x[j];
  }
  if (t == nact - 1) {
    es.seg_bin[nb] = bnd ? kEmptyRun : lo;
    es.seg_tot[nb] = bnd ? PMap{0u, 0u} : seg_combine(ex, SegVal{0u, m}).m;
  }
  __syncthreads();

  // 3. the walk over runs and boundaries, on wave 0 (uniform values)
  if (w == 0) {
    uint32_t sb_r = kEmptyRun, a0_r = 0, a1_r = 0, bp_r = 0;
    float bx_r[4] = {0.f, 0.f, 0.f, 0.f};
    if (lane <= nb) {
      sb_r = es.seg_bin[lane];
      a0_r = es.seg_tot[lane].a0;
      a1_r = es.seg_tot[lane].a1;
    }
    if (lane < nb) {
      bp_r = es.bpos[lane];
#pragma unroll
      for (int j = 0; j < 4; ++j) bx_r[j] = es.bx[4 * lane + j];
    }
    uint32_t cb = __float_as_uint(c);
    int fail = 0, hit_seg = -1, hit_pos = -1;
    uint32_t cseg = 0, bef = 0;
    for (int k = 0; k <= nb; ++k) {
      const uint32_t sb = (uint32_t)__builtin_amdgcn_readlane((int)sb_r, k);
      if (sb != kEmptyRun) {
        const uint32_t m0 = (uint32_t)__builtin_amdgcn_readlane((int)a0_r, k);
        const uint32_t m1 = (uint32_t)__builtin_amdgcn_readlane((int)a1_r, k);
        const uint32_t ic = (cb & 1u) ? m1 : m0;
        const uint32_t nbits = cb + ic;
        if ((cb & 0xff800000u) != sb || ic >= kSat || nbits >= sb + 0x00800000u) {
          fail = 1;
          break;
        }
        if (mode != kEcssSum && ecss_cond(mode, __uint_as_float(nbits), theta)) {
          hit_seg = k;
          cseg = cb;
          break;
        }
        cb = nbits;
      }
      if (k == nb) break;
      // the boundary thread's summands, with the running sum kept uniform
      // (scalar registers) between the adds
      float ys[4];
      float y = __uint_as_float(cb);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx_r[q]), k));
        y = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__fadd_rn(y, xq))));
        ys[q] = y;
      }
      int j = 4;
      if (mode != kEcssSum) {
#pragma unroll
        for (int q = 3; q >= 0; --q) j = ecss_cond(mode, ys[q], theta) ? q : j;
      }
      if (j < 4) {
        hit_pos = 4 * __builtin_amdgcn_readlane((int)bp_r, k) + j;
        bef = j ? __float_as_uint(ys[j > 0 ? j - 1 : 0]) : cb;
        cb = __float_as_uint(ys[j]);
        break;
      }
      cb = __float_as_uint(y);
    }
    if (lane == 0) {
      es.fail = fail;
      es.hit_seg = hit_seg;
      es.hit_pos = hit_pos;
      es.c_out = __uint_as_float(cb);
      es.c_seg = __uint_as_float(cseg);
      es.before = __uint_as_float(bef);
    }
  }
  __syncthreads();
  EcssResult r;
  r.c = es.c_out;
  r.before = es.before;
  r.found = es.hit_pos >= 0 ? 1 : 0;
  r.pos = es.hit_pos;
  const int fail = es.fail, hit_seg = es.hit_seg;
  __syncthreads();
  if (fail) return ecss_chunk<4>(c, x, mode, theta, sh);
  if (hit_seg < 0) return r;
  // 4. the hit is inside run hit_seg: exact starts of its threads, then the
  // first thread whose end meets the condition replays its summands
  {
    const uint32_t cs = __float_as_uint(r.c);  // c_out holds the run start here
    const uint32_t c0 = __float_as_uint(es.c_seg);
    (void)cs;
    const bool in = act && !bnd && bidx == (uint32_t)hit_seg;
    uint32_t sbits = 0, ebits = 0;
    if (in) {
      const uint32_t bfr = (c0 & 1u) ? ex.m.a1 : ex.m.a0;
      sbits = c0 + bfr;
      ebits = sbits + (((c0 ^ bfr) & 1u) ? m.a1 : m.a0);
    }
    const bool h = in && ecss_cond(mode, __uint_as_float(ebits), theta);
    const unsigned long long hm = __ballot(h);
    if (lane == 0) sh.red_h[w] = hm ? (w * 64 + __ffsll((long long)hm) - 1) : kThreads;
    __syncthreads();
    int th = kThreads;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) th = min(th, sh.red_h[i]);
    if (t == th) {
      float y = __uint_as_float(sbits), p = y;
      int j = 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (j == 4) {
          p = y;
          y = __fadd_rn(y, x[q]);
          if (ecss_cond(mode, y, theta)) j = q;
        }
      }
      es.hit_pos = 4 * th + j;
      es.c_out = y;
      es.before = p;
    }
    __syncthreads();
    r.found = 1;
    r.pos = es.hit_pos;
    r.c = es.c_out;
    r.before = es.before;
    __syncthreads();
    return r;
  }
}

}  // namespace lumen
