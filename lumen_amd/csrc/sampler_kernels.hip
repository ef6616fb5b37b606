// gfx950 token-sampling engine: one workgroup (1024 threads, 16 wave64s)
// per [V]-row of logits, all stages of Lumen's CPU sampler in one launch.
//
// Reference semantics: crates/lumen-runtime/src/sampling.rs:452-527
//   penalties (:850-900) -> top-k (:904-933) -> top-p on T=1 logits
//   (:942-967) -> min-p (:976-994) -> temperature (:516-520) -> softmax
//   (:207-231) -> inverse-CDF draw (:1003-1014); greedy rows take
//   penalties -> argmax (:468-476, :538-547).
//
// Exactness: every f32 operation of the reference is performed as the same
// single IEEE operation (this file is compiled with -ffp-contract=off and
// uses explicit _rn intrinsics on the penalty/temperature/division paths);
// expf is the glibc restatement in expf_glibc.h; every sequential f32 sum of
// the reference is reproduced bit-exactly by ecss.h. Orderings use the
// total_cmp key (sign-flipped bits) with lowest-index tie breaks.
//
// Data flow per row:
//   * penalized rows are first materialized into a scratch row (the input
//     logits are never modified);
//   * top-k: radix descent on 11/11/10-bit digits of the key with LDS
//     histograms; once the candidates above the current digit fit the LDS
//     list (8192 entries) they are compacted and the cutoff is finished with
//     an LDS bitonic sort. All ties at the cutoff survive (k == 1 keeps the
//     lowest-index maximum);
//   * small path: everything after top-k runs on the LDS list (index order),
//     with LDS sorts for the top-p order;
//   * large path (no top-k, or too many survivors): streaming passes over the
//     row; top-p walks the probability order in windows of at most 8192
//     candidates, each window compacted into LDS and sorted, carrying the
//     exact cumulative sum across windows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "expf_glibc.h"
#include "kernel_abi.h"


// Phase timestamps for development code objects (-DLUMEN_TIMING, devtrace.h);
// in the shipped code object every tick compiles to nothing.
#ifdef LUMEN_TIMING
#include "devtrace.h"
#else
#define LUMEN_TICK(label, b) do { } while (0)
#define LUMEN_TICK_INIT() do { } while (0)
#define LUMEN_TICK_SLOT(row, sl) do { } while (0)
#define LUMEN_TICK_RESET(b) do { } while (0)
#define LUMEN_TICK_DUMP(b) do { } while (0)
#define LUMEN_ROW_TIMES(tr) do { } while (0)
#endif

#include "ecss.h"

namespace lumen {

constexpr int kCap = 8192;          // LDS list capacity (entries)
constexpr int kCapWindow = kCap - 512;  // planned window size (margin for equal-probability spill)
constexpr float kNegInf = -__builtin_huge_valf();

struct Smem {
  uint64_t A[kCap];
  uint64_t Bk[kCap];
  uint32_t H[4096];   // histograms (radix sort: 256 digits x 16 waves)
  uint32_t H0[2048];  // window planner histogram, kept across windows
  EcssShared ecss;
  EstShared est;
  double wsum[kWaves];
  uint32_t red_a[kWaves];
  uint32_t red_b[kWaves];
  float red_f[kWaves];
  uint32_t cnt;
  uint32_t finisher;  // this workgroup arrived last on its row's counter
  int misc_i[4];
  uint32_t misc_u[4];
};

// ---------------------------------------------------------------- helpers

__device__ __forceinline__ uint32_t tkey(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
__device__ __forceinline__ bool is_nan(float f) { return (__float_as_uint(f) & 0x7fffffffu) > 0x7f800000u; }
__device__ __forceinline__ bool is_finite(float f) { return (__float_as_uint(f) & 0x7f800000u) != 0x7f800000u; }
// f32::max: a NaN operand yields the other operand.
__device__ __forceinline__ float rmax(float a, float b) {
  if (is_nan(b)) return a;
  if (is_nan(a)) return b;
  return a > b ? a : b;
}

// Loads and stores through global-memory pointers. The row and workspace
// pointers reach the noinline per-row functions as generic pointers, for
// which the compiler emits flat instructions: those count against the LDS
// wait counter too, so every LDS wait also drains the outstanding row loads.
// The casts give global_load / global_store.
// (Scalars and clang vector types only: a HIP_vector_type goes through its
// copy constructor, whose generic reference loses the address space.)
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <class T>
__device__ __forceinline__ T gld(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
template <class T>
__device__ __forceinline__ void gst(T* p, T v) {
  *(__attribute__((address_space(1))) T*)p = v;
}

struct Row {
  const float* f;
  const uint16_t* h;
  uint32_t V;
  bool vec;
  __device__ __forceinline__ float at(uint32_t i) const {
    return f ? gld(f + i) : __uint_as_float((uint32_t)gld(h + i) << 16);
  }
  // elements i..i+3 (i % 4 == 0); out-of-range lanes are left untouched
  __device__ __forceinline__ void load4(uint32_t i, float (&v)[4]) const {
    if (vec && i + 3 < V) {
      if (f) {
        const f32x4 q = gld(reinterpret_cast<const f32x4*>(f + i));
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
      } else {
        const u16x4 q = gld(reinterpret_cast<const u16x4*>(h + i));
        v[0] = __uint_as_float((uint32_t)q.x << 16);
        v[1] = __uint_as_float((uint32_t)q.y << 16);
        v[2] = __uint_as_float((uint32_t)q.z << 16);
        v[3] = __uint_as_float((uint32_t)q.w << 16);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i + j < V) v[j] = at(i + j);
    }
  }
};

// f(i, v) for every element of the row; each thread handles 4 groups of 4
// consecutive elements per iteration to keep several loads in flight.
template <class F>
__device__ __forceinline__ void row_foreach(const Row& r, F&& f) {
  const uint32_t V = r.V;
  uint32_t g0 = threadIdx.x;
  // whole groups of 4 x 4 elements on aligned rows: no per-element checks
  if (r.vec) {
    for (; (g0 + 3u * kThreads) * 4u + 3u < V; g0 += 4u * kThreads) {
      float v[4][4];
      if (r.f) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f32x4 q = gld(reinterpret_cast<const f32x4*>(r.f) + g0 + u * kThreads);
          v[u][0] = q.x; v[u][1] = q.y; v[u][2] = q.z; v[u][3] = q.w;
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u16x4 q = gld(reinterpret_cast<const u16x4*>(r.h) + g0 + u * kThreads);
          v[u][0] = __uint_as_float((uint32_t)q.x << 16);
          v[u][1] = __uint_as_float((uint32_t)q.y << 16);
          v[u][2] = __uint_as_float((uint32_t)q.z << 16);
          v[u][3] = __uint_as_float((uint32_t)q.w << 16);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t i = (g0 + u * kThreads) * 4u;
#pragma unroll
        for (int j = 0; j < 4; ++j) f(i + j, v[u][j]);
      }
    }
  }
  for (; g0 * 4u < V; g0 += 4u * kThreads) {
    float v[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t i = (g0 + u * kThreads) * 4u;
      if (i < V) r.load4(i, v[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t i = (g0 + u * kThreads) * 4u;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i + j < V) f(i + j, v[u][j]);
    }
  }
}

// f(i, v) for every element of [lo, hi).
template <class F>
__device__ __forceinline__ void range_foreach(const Row& r, uint32_t lo, uint32_t hi, F&& f) {
  if (lo >= hi) return;
  for (uint32_t g0 = lo / 4u + threadIdx.x; g0 * 4u < hi; g0 += 4u * kThreads) {
    float v[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t i = (g0 + u * kThreads) * 4u;
      if (i < hi) r.load4(i, v[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t i = (g0 + u * kThreads) * 4u;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (i + j >= lo && i + j < hi) f(i + j, v[u][j]);
    }
  }
}

__device__ __forceinline__ uint32_t op_add_u32(uint32_t l, uint32_t r) { return l + r; }
__device__ __forceinline__ uint32_t op_or_u32(uint32_t l, uint32_t r) { return l | r; }
__device__ __forceinline__ uint64_t op_max_u64(uint64_t l, uint64_t r) { return l > r ? l : r; }

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return wave_reduce(v, 0u, op_add_u32); }

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum_u32(v);
  if (lane == 0) s.red_a[w] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += s.red_a[i];
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, 0u, [](uint32_t l, uint32_t r) { return l > r ? l : r; });
  if (lane == 0) s.red_a[w] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r = s.red_a[i] > r ? s.red_a[i] : r;
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t block_or_u32(uint32_t v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, 0u, op_or_u32);
  if (lane == 0) s.red_a[w] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r |= s.red_a[i];
  __syncthreads();
  return r;
}

// max of a 64-bit value carried as (hi, lo)
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, (uint64_t)0, op_max_u64);
  if (lane == 0) {
    s.red_a[w] = (uint32_t)(v >> 32);
    s.red_b[w] = (uint32_t)v;
  }
  __syncthreads();
  uint64_t r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    uint64_t u = ((uint64_t)s.red_a[i] << 32) | s.red_b[i];
    r = u > r ? u : r;
  }
  __syncthreads();
  return r;
}

// fold(-inf, f32::max) over the block; NaN inputs are ignored
__device__ __forceinline__ float block_rmax(float v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, kNegInf, rmax);
  if (lane == 0) s.red_f[w] = v;
  __syncthreads();
  float r = kNegInf;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r = rmax(r, s.red_f[i]);
  __syncthreads();
  return r;
}

// block_rmax together with a NaN flag (one barrier pair).
__device__ __forceinline__ float block_rmax_nan(float v, bool nan, Smem& s, bool* any_nan) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, kNegInf, rmax);
  const bool wn = __ballot(nan) != 0ull;
  if (lane == 0) {
    s.red_f[w] = v;
    s.red_b[w] = wn ? 1u : 0u;
  }
  __syncthreads();
  float r = kNegInf;
  uint32_t n = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    r = rmax(r, s.red_f[i]);
    n |= s.red_b[i];
  }
  __syncthreads();
  *any_nan = n != 0u;
  return r;
}

__device__ __forceinline__ uint32_t block_incl_scan_u32(uint32_t v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_scan_incl(v, 0u, op_add_u32);
  if (lane == 63) s.red_a[w] = v;
  __syncthreads();
  uint32_t pre = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) pre += i < w ? s.red_a[i] : 0u;
  __syncthreads();
  return v + pre;
}

// Histogram search from the top digit down: returns d with
// above(d) < need <= above(d) + H[d], above(d) = sum of H over digits > d.
// d = -1 when the total is below `need` (then *above = total).
__device__ __forceinline__ int find_from_top(const uint32_t* H, int nb, uint32_t need, uint32_t* above, Smem& s) {
  const int t = threadIdx.x;
  const int per = nb / kThreads;  // 1 or 2
  uint32_t loc = 0;
  for (int q = 0; q < per; ++q) loc += H[nb - 1 - per * t - q];
  uint32_t incl = block_incl_scan_u32(loc, s);
  uint32_t ex = incl - loc;
  if (t == 0) {
    s.misc_i[0] = -1;
    s.misc_u[0] = 0;
  }
  __syncthreads();
  uint32_t acc = ex;
  for (int q = 0; q < per; ++q) {
    int d = nb - 1 - per * t - q;
    uint32_t h = H[d];
    if (acc < need && need <= acc + h) {
      s.misc_i[0] = d;
      s.misc_u[0] = acc;
    }
    acc += h;
  }
  if (t == kThreads - 1 && incl < need) s.misc_u[1] = incl;
  __syncthreads();
  int d = s.misc_i[0];
  *above = d >= 0 ? s.misc_u[0] : s.misc_u[1];
  __syncthreads();
  return d;
}

__device__ __forceinline__ void clear_hist(uint32_t* H, int nb) {
  for (int i = threadIdx.x; i < nb; i += kThreads) H[i] = 0;
}

// Key of 0-based rank r in descending order among key(j), j < n (n > r):
// three LDS histogram rounds over 11/11/10-bit digits.
// With levels < 3 the result is the lower edge of the bucket holding the
// r-th largest key: a lower bound with at least r + 1 keys at or above it.
template <class K>
__device__ __forceinline__ uint32_t select_desc(uint32_t n, K&& key, uint32_t r, Smem& s,
                                                int levels = 3) {
  uint32_t prefix = 0, pmask = 0, need = r + 1u;
  for (int lvl = 0; lvl < levels; ++lvl) {
    const int sh = lvl == 0 ? 21 : (lvl == 1 ? 10 : 0);
    const int nb = lvl == 2 ? 1024 : 2048;
    const uint32_t dm = (uint32_t)nb - 1u;
    clear_hist(s.H, nb);
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
      const uint32_t k = key(j);
      if ((k & pmask) == prefix) atomicAdd(&s.H[(k >> sh) & dm], 1u);
    }
    __syncthreads();
    uint32_t ab = 0;
    const int d = find_from_top(s.H, nb, need, &ab, s);
    need -= ab;
    prefix |= (uint32_t)d << sh;
    pmask |= dm << sh;
  }
  return prefix;
}

// Lanes of the wave whose 8-bit digit equals this lane's (among `valid`).
__device__ __forceinline__ uint64_t match_digit8(uint32_t d, bool valid) {
  uint64_t m = __ballot(valid);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (d >> b) & 1u;
    const uint64_t bb = __ballot(bit);
    m &= bit ? bb : ~bb;
  }
  return m;
}

// One stable counting pass on the 8-bit digit at `shift`: src -> dst. Wave w
// owns the contiguous range [w * per_w, (w + 1) * per_w) and walks it in
// 64-entry tiles; the 256 x 16 counters (digit-major, wave-minor) are
// scanned so that equal digits keep wave order, tile order and lane order.
__device__ __forceinline__ void radix_pass(const uint64_t* src, uint64_t* dst, uint32_t n,
                                           uint32_t shift, Smem& s) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  uint32_t* hist = s.H;
  const uint32_t per_w = ((n + kThreads - 1u) / kThreads) * 64u;
  const uint32_t wlo = min(n, w * per_w), whi = min(n, wlo + per_w);
  const uint64_t lt = (1ull << lane) - 1ull;
  for (uint32_t i = t; i < 4096u; i += kThreads) hist[i] = 0u;
  __syncthreads();
  // only this wave touches column w, and the leaders of one tile hold
  // distinct digits: plain LDS read-modify-writes suffice
  for (uint32_t base = wlo; base < whi; base += 64u) {
    const uint32_t i = base + lane;
    const bool valid = i < whi;
    const uint32_t d = valid ? (uint32_t)(src[i] >> shift) & 255u : 0u;
    const uint64_t m = match_digit8(d, valid);
    if (valid && (m & lt) == 0ull) hist[d * 16u + w] += (uint32_t)__popcll(m);
  }
  __syncthreads();
  // exclusive scan over the 4096 counters; thread t owns [4t, 4t + 4)
  uint32_t h[4], sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = hist[4u * t + j];
    sum += h[j];
  }
  const uint32_t inc = wave_scan_incl(sum, 0u, op_add_u32);
  if (lane == 63u) s.red_a[w] = inc;
  __syncthreads();
  uint32_t pre = inc - sum;
  for (uint32_t i = 0; i < w; ++i) pre += s.red_a[i];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    hist[4u * t + j] = pre;
    pre += h[j];
  }
  __syncthreads();
  for (uint32_t base = wlo; base < whi; base += 64u) {
    const uint32_t i = base + lane;
    const bool valid = i < whi;
    const uint64_t e = valid ? src[i] : 0ull;
    const uint32_t d = (uint32_t)(e >> shift) & 255u;
    const uint64_t m = match_digit8(d, valid);
    if (valid) {
      const uint32_t off = hist[d * 16u + w];
      const uint32_t r = (uint32_t)__popcll(m & lt);
      dst[off + r] = e;
      if (r == 0u) hist[d * 16u + w] = off + (uint32_t)__popcll(m);
    }
  }
  __syncthreads();
}

// Ascending LSD radix sort of a[0..n) with tmp[0..n) as the second buffer
// (both in LDS). Only the bits in which the keys differ are sorted, in 8-bit
// digits starting at the lowest differing bit, so the cost is about one read
// and one write of the list per 8 varying bits.
__device__ __forceinline__ void radix_sort_u64(uint64_t* a, uint64_t* tmp, uint32_t n, Smem& s) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  uint64_t o = 0ull, an = ~0ull;
  for (uint32_t j = t; j < n; j += kThreads) {
    o |= a[j];
    an &= a[j];
  }
  o = wave_reduce(o, (uint64_t)0, [](uint64_t l, uint64_t r) { return l | r; });
  an = wave_reduce(an, ~(uint64_t)0, [](uint64_t l, uint64_t r) { return l & r; });
  uint64_t* red = reinterpret_cast<uint64_t*>(s.wsum);
  if (lane == 0u) red[w] = o;
  __syncthreads();
  uint64_t ro = 0ull;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) ro |= red[i];
  __syncthreads();
  if (lane == 0u) red[w] = an;
  __syncthreads();
  uint64_t ra = ~0ull;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) ra &= red[i];
  __syncthreads();
  uint64_t diff = ro ^ ra;
  uint64_t* src = a;
  uint64_t* dst = tmp;
  while (diff) {
    const uint32_t shift = (uint32_t)(__ffsll((long long)diff) - 1);
    radix_pass(src, dst, n, shift, s);
    uint64_t* x = src;
    src = dst;
    dst = x;
    diff = shift >= 56u ? 0ull : (diff & ~((1ull << (shift + 8u)) - 1ull));
  }
  if (src != a) {
    for (uint32_t j = t; j < n; j += kThreads) a[j] = src[j];
    __syncthreads();
  }
}

// Ascending sort of a[0..n) in LDS (keys unique or order among equal keys
// irrelevant). n <= 256: every key counts the keys below it and is written
// to its rank (one pass, two barriers). Larger n: bitonic network, one LDS
// barrier per cross-wave stage.
__device__ __forceinline__ void sort_u64_bitonic(uint64_t* a, uint32_t n) {
  const uint32_t t = threadIdx.x;
  if (n <= 256u) {
    uint64_t mine = 0;
    uint32_t rank = 0;
    if (t < n) {
      mine = a[t];
      for (uint32_t j = 0; j < n; ++j) {
        const uint64_t o = a[j];
        rank += (o < mine || (o == mine && j < t)) ? 1u : 0u;
      }
    }
    __syncthreads();
    if (t < n) a[rank] = mine;
    __syncthreads();
    return;
  }
  uint32_t np = 512;
  while (np < n) np <<= 1;
  for (uint32_t i = n + t; i < np; i += kThreads) a[i] = ~0ull;
  __syncthreads();
  // wave w owns the 512-key chunks w, w + 16, ...; a stage whose partner
  // distance j is below 512 stays inside a chunk and needs only a
  // wave-level LDS fence
  const uint32_t lane = t & 63u, w = t >> 6;
  const uint32_t nchunks = np / 512u;
  for (uint32_t k = 2; k <= np; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0; j >>= 1) {
      if (j < 512u) {
        for (uint32_t ch = w; ch < nchunks; ch += kWaves) {
#pragma unroll
          for (uint32_t e = 0; e < 8u; ++e) {
            const uint32_t i = ch * 512u + e * 64u + lane, ixj = i ^ j;
            if (ixj > i) {
              const uint64_t x = a[i], y = a[ixj];
              const bool up = (i & k) == 0;
              if ((x > y) == up) {
                a[i] = y;
                a[ixj] = x;
              }
            }
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
      } else {
        __syncthreads();
        for (uint32_t i = t; i < np; i += kThreads) {
          const uint32_t ixj = i ^ j;
          if (ixj > i) {
            const uint64_t x = a[i], y = a[ixj];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              a[i] = y;
              a[ixj] = x;
            }
          }
        }
        __syncthreads();
      }
    }
  }
  __syncthreads();
}

constexpr uint32_t kBucketMax = 256;  // largest bucket ranked by direct counting

// Ascending sort of a[0..n) (LDS) through tmp[0..n) (LDS). The keys are
// spread over 4096 buckets by the 12 highest bits in which they differ
// (bucket order is key order); every key then counts the keys of its own
// bucket that sort before it, which gives its final position whatever
// order the atomic scatter left inside the bucket. When a bucket holds
// more than kBucketMax keys the radix sort takes over.
__device__ __forceinline__ void bucket_sort_u64(uint64_t* a, uint64_t* tmp, uint32_t n,
                                                          uint64_t diff_hint, Smem& s) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  uint64_t diff = diff_hint;  // a superset of the bits in which keys differ, or 0
  if (!diff) {
  uint64_t o = 0ull, an = ~0ull;
  for (uint32_t j = t; j < n; j += kThreads) {
    o |= a[j];
    an &= a[j];
  }
  o = wave_reduce(o, (uint64_t)0, [](uint64_t l, uint64_t r) { return l | r; });
  an = wave_reduce(an, ~(uint64_t)0, [](uint64_t l, uint64_t r) { return l & r; });
  uint64_t* red = reinterpret_cast<uint64_t*>(s.wsum);
  if (lane == 0u) red[w] = o;
  __syncthreads();
  uint64_t ro = 0ull;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) ro |= red[i];
  __syncthreads();
  if (lane == 0u) red[w] = an;
  __syncthreads();
  uint64_t ra = ~0ull;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) ra &= red[i];
  __syncthreads();
  diff = ro ^ ra;     // bits that differ between some keys
  if (!diff) return;  // all keys equal
  }
  const uint32_t hb = 63u - (uint32_t)__clzll((long long)diff);
  const uint32_t sh = hb >= 11u ? hb - 11u : 0u;
  uint32_t* H = s.H;
  for (uint32_t i = t; i < 4096u; i += kThreads) H[i] = 0u;
  __syncthreads();
  for (uint32_t j = t; j < n; j += kThreads) atomicAdd(&H[(uint32_t)(a[j] >> sh) & 4095u], 1u);
  __syncthreads();
  // exclusive scan of the bucket counts (thread t owns [4t, 4t + 4)) and
  // the largest bucket
  uint32_t h[4], sum = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = H[4u * t + j];
    sum += h[j];
    mx = max(mx, h[j]);
  }
  const uint32_t inc = wave_scan_incl(sum, 0u, op_add_u32);
  mx = wave_reduce(mx, 0u, [](uint32_t l, uint32_t r) { return l > r ? l : r; });
  if (lane == 63u) {
    s.red_a[w] = inc;
    s.red_b[w] = mx;
  }
  __syncthreads();
  uint32_t pre = inc - sum, bmax = 0;
#pragma unroll
  for (uint32_t i = 0; i < (uint32_t)kWaves; ++i) {
    pre += i < w ? s.red_a[i] : 0u;
    bmax = max(bmax, s.red_b[i]);
  }
  if (bmax > kBucketMax) {
    __syncthreads();
    radix_sort_u64(a, tmp, n, s);
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    H[4u * t + j] = pre;
    pre += h[j];
  }
  __syncthreads();
  for (uint32_t j = t; j < n; j += kThreads) {
    const uint64_t e = a[j];
    tmp[atomicAdd(&H[(uint32_t)(e >> sh) & 4095u], 1u)] = e;
  }
  __syncthreads();
  // H[b] is now the end of bucket b
  for (uint32_t i = t; i < n; i += kThreads) {
    const uint64_t e = tmp[i];
    const uint32_t bk = (uint32_t)(e >> sh) & 4095u;
    const uint32_t lo = bk ? H[bk - 1u] : 0u, hi = H[bk];
    uint32_t r = 0;
    for (uint32_t k = lo; k < hi; ++k) {
      const uint64_t q = tmp[k];
      r += (q < e || (q == e && k < i)) ? 1u : 0u;
    }
    a[lo + r] = e;
  }
  __syncthreads();
}

// Ascending sort of a[0..n) in LDS. With a free second buffer `tmp` (n
// entries) lists above 256 entries take the bucket sort.
__device__ __forceinline__ void sort_u64_asc(uint64_t* a, uint32_t n, uint64_t* tmp, Smem& s,
                                             uint64_t diff_hint = 0) {
  if (n > 256u && tmp) {
    bucket_sort_u64(a, tmp, n, diff_hint, s);
    return;
  }
  sort_u64_bitonic(a, n);
}

// All-ones mask covering every value below n (n >= 1).
__device__ __forceinline__ uint32_t span_mask(uint32_t n) {
  return n <= 1u ? 0u : 0xffffffffu >> __clz(n - 1u);
}

// Wave-aggregated append into an LDS list; returns nothing, counts all.
__device__ __forceinline__ void list_push(uint64_t* list, uint32_t* cnt, bool p, uint64_t val) {
  unsigned long long m = __ballot(p);
  if (!m) return;
  const int lane = threadIdx.x & 63;
  uint32_t base = 0;
  int leader = __ffsll((long long)m) - 1;
  if (lane == leader) base = atomicAdd(cnt, (uint32_t)__popcll(m));
  base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);
  if (p) {
    uint32_t off = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
    if (off < (uint32_t)kCap) list[off] = val;
  }
}

// ECSS over a row of V elements, x(i, v) for i < V; 16 contiguous elements
// per thread per chunk.
template <class X>
__device__ __forceinline__ EcssResult row_ecss(const Row& r, X&& xf, int mode, float theta, Smem& s) {
  constexpr int M = 16;
  const uint32_t V = r.V;
  float c = 0.f;
  for (uint32_t base = 0; base < V; base += (uint32_t)kThreads * M) {
    const uint32_t i0 = base + threadIdx.x * M;
    float x[M];
#pragma unroll
    for (int q = 0; q < M / 4; ++q) {
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      uint32_t i = i0 + 4 * q;
      if (i < V) r.load4(i, v);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * q + j] = (i + j < V) ? xf(i + j, v[j]) : 0.f;
    }
    LUMEN_TICK("ecss_x", LUMEN_TIMING_ROW);
    EcssResult e = ecss_fast_chunk<M>(c, x, mode, theta, s.ecss, s.est, s.wsum,
                                      (int)min((uint32_t)kThreads, ((V - base) + (uint32_t)M - 1u) / (uint32_t)M));
    LUMEN_TICK("ecss_chunk", LUMEN_TIMING_ROW);
    if (e.found) {
      e.pos += (int)base;
      return e;
    }
    c = e.c;
  }
  EcssResult e;
  e.c = c;
  e.found = 0;
  e.pos = -1;
  e.before = 0.f;
  return e;
}

// Position of element j in a padded float array: one spare word after every
// 16, so the lanes of a wave reading 16 consecutive elements each (17 words
// apart) hit different LDS banks.
__device__ __forceinline__ uint32_t pad16(uint32_t j) { return j + (j >> 4); }

// The one-wave method on a list, in parts of 1024 elements (16 per lane);
// the exact sum carries from part to part (wave 0 only).
template <class X>
__device__ __forceinline__ EcssResult list_ecss_wave(uint32_t n, X&& xf, int mode, float theta, float c0) {
  const uint32_t lane = threadIdx.x & 63u;
  float c = c0;
  for (uint32_t base = 0; base < n; base += 1024u) {
    float x[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const uint32_t j = base + lane * 16u + (uint32_t)q;
      x[q] = j < n ? xf(j) : 0.f;
    }
    EcssResult r = wave_ecss<16>(c, x, mode, theta);
    if (r.found) {
      r.pos += (int)base;
      return r;
    }
    c = r.c;
  }
  EcssResult r;
  r.c = c;
  r.found = 0;
  r.pos = -1;
  r.before = 0.f;
  return r;
}

template <class X>
__device__ __forceinline__ EcssResult list_ecss(uint32_t n, X&& xf, int mode, float theta, float c0, Smem& s) {
  {
    // one wave, no workgroup barrier inside
    if (threadIdx.x < 64u) {
      const EcssResult r = list_ecss_wave(n, xf, mode, theta, c0);
      if (threadIdx.x == 0) {
        s.est.c_out = r.c;
        s.est.before = r.before;
        s.est.hit_pos = r.found ? r.pos : -1;
        s.est.fail = 0;
      }
    }
    __syncthreads();
    EcssResult e;
    e.c = s.est.c_out;
    e.before = s.est.before;
    e.pos = s.est.hit_pos;
    e.found = e.pos >= 0 ? 1 : 0;
    __syncthreads();
    return e;
  }
}

// The same on the whole workgroup, 4096 elements at a time (thread t holds
// elements 4t .. 4t+3 of a chunk), with the estimate-guided chunk method of
// ecss.h: each chunk starts from the exact running sum, so its drift bound
// is rigorous, and one segmented scan plus a short walk over the few
// threads near a binade edge replaces a wave scan per edge.
template <class X>
__device__ __forceinline__ EcssResult list_ecss_block(uint32_t n, X&& xf, int mode, float theta,
                                                      float c0, Smem& s) {
  constexpr int M = 4;
  float c = c0;
  for (uint32_t base = 0; base < n; base += (uint32_t)kThreads * M) {
    float x[M];
#pragma unroll
    for (int q = 0; q < M; ++q) {
      const uint32_t j = base + threadIdx.x * M + (uint32_t)q;
      x[q] = j < n ? xf(j) : 0.f;
    }
    EcssResult e = ecss_chunk4(c, x, mode, theta,
                               (int)min((uint32_t)kThreads, (n - base + (uint32_t)M - 1u) / (uint32_t)M),
                               s.ecss, s.est);
    if (e.found) {
      e.pos += (int)base;
      return e;
    }
    c = e.c;
  }
  EcssResult e;
  e.c = c;
  e.found = 0;
  e.pos = -1;
  e.before = 0.f;
  return e;
}

// Walk over V tokens that all carry the same probability u (the uniform
// branch of softmax, sampling.rs:211-214 and :224-227).
__device__ __forceinline__ EcssResult const_ecss(uint32_t V, float u, int mode, float theta, Smem& s) {
  constexpr int M = 16;
  float c = 0.f;
  for (uint32_t base = 0; base < V; base += (uint32_t)kThreads * M) {
    const uint32_t i0 = base + threadIdx.x * M;
    float x[M];
#pragma unroll
    for (int j = 0; j < M; ++j) x[j] = (i0 + j < V) ? u : 0.f;
    LUMEN_TICK("ecss_x", LUMEN_TIMING_ROW);
    EcssResult e = ecss_fast_chunk<M>(c, x, mode, theta, s.ecss, s.est, s.wsum,
                                      (int)min((uint32_t)kThreads, ((V - base) + (uint32_t)M - 1u) / (uint32_t)M));
    LUMEN_TICK("ecss_chunk", LUMEN_TIMING_ROW);
    if (e.found) {
      e.pos += (int)base;
      return e;
    }
    c = e.c;
  }
  EcssResult e;
  e.c = c;
  e.found = 0;
  e.pos = -1;
  e.before = 0.f;
  return e;
}

__device__ __forceinline__ float penalize(float v, uint32_t count, const RowParams& P) {
  // sampling.rs:881-900, one IEEE operation per step
  float nv = v;
  if (P.flags & kRep) nv = (v > 0.f) ? __fdiv_rn(v, P.rep) : __fmul_rn(v, P.rep);
  nv = __fsub_rn(nv, P.presence);
  nv = __fsub_rn(nv, __fmul_rn(P.freq, __uint2float_rn(count)));
  return nv;
}

// --------------------------------------------------------------- the kernel

struct Final {  // what the final stage needs to know about the list
  uint32_t n;
};

__device__ __forceinline__ void init_trace(RowTrace& tr, uint32_t V) {
  tr.status = 0; tr.path = 0; tr.topk_cutoff_key = 0; tr.topk_survivors = V; tr.topp_sum = 0.f;
  tr.topp_kept = 0; tr.topp_cum = 0.f; tr.windows = 0; tr.final_max = 0.f; tr.final_sum = 0.f;
  tr.cdf_before = 0.f; tr.cdf_at = 0.f; tr.token = 0; tr.passes = 0; tr.pad[0] = tr.pad[1] = 0;
}

__device__ __forceinline__ Row make_row(const KernelArgs& a, int b) {
  Row row;
  if (a.dtype == 0) {
    row.f = reinterpret_cast<const float*>(a.logits) + (uint64_t)b * a.row_stride;
    row.h = nullptr;
    row.vec = ((reinterpret_cast<uintptr_t>(row.f) & 15u) == 0);
  } else {
    row.f = nullptr;
    row.h = reinterpret_cast<const uint16_t*>(a.logits) + (uint64_t)b * a.row_stride;
    row.vec = ((reinterpret_cast<uintptr_t>(row.h) & 7u) == 0);
  }
  row.V = a.vocab;
  return row;
}

// Xorshift64::next_u64 / next_f32 (sampling.rs:90-104): x ^= x << 13,
// x ^= x >> 7, x ^= x << 17; the draw is the top 24 bits times 2^-24.
__device__ __forceinline__ uint64_t xorshift_step(uint64_t x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

// The draw of row b: a caller uniform, or next_f32 of the row's device RNG
// state (not advanced here: the row's finisher stores the advanced state).
__device__ __forceinline__ float row_draw(const KernelArgs& a, int b) {
  if (a.rng_dev) return (float)(xorshift_step(a.rng_dev[b]) >> 40) * 0x1.0p-24f;
  return a.inline_draws ? a.inline_uniforms[b] : a.uniforms[b];
}

// End of row b's penalty counts (hist_off[b] is the start).
__device__ __forceinline__ uint32_t hist_hi(const KernelArgs& a, int b) {
  return a.hist_end ? a.hist_end[b] : a.hist_off[b + 1];
}

__device__ __forceinline__ void write_result(const KernelArgs& a, int b, uint32_t token, RowTrace& tr) {
  LUMEN_TICK("write", b);
  LUMEN_TICK_DUMP(b);
  if (threadIdx.x == 0) {
    if (a.ring) {
      if (a.hist_off[b] == kHistBad) {
        // the penalty window did not fit the ring (lumen_hist_window)
        token = kTokenError;
        tr.status = kStatusHistOverflow;
      } else if (token != kTokenError) {
        // SamplerState::record (sampling.rs:381-384) into the device ring
        const uint32_t n = a.ring_len[b];
        a.ring[(uint64_t)b * a.ring_cap + n % a.ring_cap] = token;
        a.ring_len[b] = n + 1u;
      }
    }
    a.tokens[b] = token;
    if (a.trace) {
      LUMEN_ROW_TIMES(tr);
      tr.token = token;
      a.trace[b] = tr;
    }
    if (a.rng_dev) {
      // exactly one draw per sampled row with a non-empty vocabulary
      const RowParams& P = a.inline_rows ? a.inline_params[b] : a.params[b];
      if (!(P.flags & kGreedy) && a.vocab > 0) a.rng_dev[b] = xorshift_step(a.rng_dev[b]);
    }
    if (a.tokens_mapped) {
      a.tokens_mapped[b] = token;
      __hip_atomic_fetch_add(a.done_mapped, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
}

// Final stage over the LDS list A (entries (idx << 32) | key, ascending idx,
// n entries, every entry alive). Applies min-p, temperature, softmax, draw.
// known_max: the largest logit of the list when the caller knows it (the
// list is NaN-free then), NaN otherwise.
// With pre_exp, list entries carry exp(v - known_max) in place of the key:
// the caller computed them exactly (expf_glibc) and guarantees inv_temp == 1,
// no min-p, and a finite known_max equal to the list maximum, so the
// summands of the final softmax are those values themselves.
__device__ __forceinline__ uint32_t final_on_list(const KernelArgs& a, const RowParams P, uint32_t n, float r,
                                  Smem& s, RowTrace& tr, float known_max, bool pre_exp = false) {
  const uint32_t V = a.vocab;
  auto lv = [&](uint32_t j) -> float { return key2f((uint32_t)s.A[j]); };
  if (pre_exp) {
    float* xs = reinterpret_cast<float*>(s.Bk);
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) xs[j] = __uint_as_float((uint32_t)s.A[j]);
    __syncthreads();
    tr.final_max = known_max;
    LUMEN_TICK("f_copy", LUMEN_TIMING_ROW);
    const EcssResult S = list_ecss_block(n, [&](uint32_t j) { return xs[j]; }, kEcssSum, 0.f, 0.f, s);
    const float S3 = S.c;
    LUMEN_TICK("f_S", LUMEN_TIMING_ROW);
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) xs[j] = __fdiv_rn(xs[j], S3);
    __syncthreads();
    LUMEN_TICK("f_div", LUMEN_TIMING_ROW);
    tr.final_sum = S3;
    const EcssResult e = list_ecss_block(n, [&](uint32_t j) { return xs[j]; }, kEcssFindGt, r, 0.f, s);
    LUMEN_TICK("f_find", LUMEN_TIMING_ROW);
    tr.cdf_before = e.found ? e.before : e.c;
    tr.cdf_at = e.c;
    if (e.found) return (uint32_t)(s.A[e.pos] >> 32);
    return V - 1;
  }
  // min-p (sampling.rs:976-994)
  bool mmask = false;
  float bound = 0.f;
  const bool known = !is_nan(known_max);
  if (P.flags & kMinP) {
    float m = known_max;
    if (!known) {
      m = kNegInf;
      for (uint32_t j = threadIdx.x; j < n; j += kThreads) m = rmax(m, lv(j));
      m = block_rmax(m, s);
    }
    if (is_finite(m)) {
      mmask = true;
      bound = __fadd_rn(m, P.log_min_p);
    }
  }
  auto wv = [&](uint32_t j) -> float {
    float v = lv(j);
    if (mmask && v < bound) v = kNegInf;
    return __fmul_rn(v, P.inv_temp);
  };
  float m3 = kNegInf;
  uint32_t nan3 = 0;
  if (known && !(mmask && known_max < bound)) {
    // x -> x * inv_temp (inv_temp > 0) is monotone under rounding
    m3 = __fmul_rn(known_max, P.inv_temp);
  } else {
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
      float w = wv(j);
      m3 = rmax(m3, w);
      nan3 |= is_nan(w) ? 1u : 0u;
    }
    // tokens outside the list are -inf * inv_temp: they only matter when the
    // list has no finite value at all (uniform branch over all V tokens)
    m3 = block_rmax(m3, s);
    nan3 = block_or_u32(nan3, s);
  }
  LUMEN_TICK("fin_m3", LUMEN_TIMING_ROW);
  tr.final_max = m3;
  if (!is_finite(m3)) {
    tr.path |= 16u;
    float u = __fdiv_rn(1.0f, __uint2float_rn(V));
    EcssResult e = const_ecss(V, u, kEcssFindGt, r, s);
    tr.final_sum = 0.f;
    tr.cdf_before = e.found ? e.before : e.c;
    tr.cdf_at = e.c;
    return e.found ? (uint32_t)e.pos : V - 1;
  }
  if (nan3) {
    // the sum is NaN, so every probability and every CDF value is NaN and the
    // walk falls through to the last index (sampling.rs:1013)
    tr.path |= 32u;
    tr.final_sum = __uint_as_float(0x7fc00000u);
    tr.cdf_before = tr.cdf_at = __uint_as_float(0x7fc00000u);
    return V - 1;
  }
  // the summands, then the probabilities, computed by the whole workgroup
  // into LDS (list B is free here); the exact sums read them back
  float* xs = reinterpret_cast<float*>(s.Bk);
  for (uint32_t j = threadIdx.x; j < n; j += kThreads) xs[j] = expf_glibc(__fsub_rn(wv(j), m3));
  __syncthreads();
  LUMEN_TICK("fin_exps", LUMEN_TIMING_ROW);
  EcssResult S = list_ecss_block(n, [&](uint32_t j) { return xs[j]; }, kEcssSum, 0.f, 0.f, s);
  const float S3 = S.c;
  for (uint32_t j = threadIdx.x; j < n; j += kThreads) xs[j] = __fdiv_rn(xs[j], S3);
  __syncthreads();
  LUMEN_TICK(s.est.fail == 2 ? "S3_nofit" : s.est.fail ? "S3_failed" : "S3_ok", LUMEN_TIMING_ROW);
  tr.final_sum = S3;
  EcssResult e = list_ecss_block(n, [&](uint32_t j) { return xs[j]; }, kEcssFindGt, r, 0.f, s);
  LUMEN_TICK(s.est.fail == 2 ? "walk_nofit" : s.est.fail ? "walk_failed" : "walk_ok", LUMEN_TIMING_ROW);
  LUMEN_TICK("fin_walk", LUMEN_TIMING_ROW);
  tr.cdf_before = e.found ? e.before : e.c;
  tr.cdf_at = e.c;
  if (e.found) return (uint32_t)(s.A[e.pos] >> 32);
  return V - 1;
}

// One-wave small path: everything after top-k for a list of at most
// kWaveList entries (s.A, (idx << 32) | key, ascending idx) whose maximum is
// finite and that holds no NaN. Lane l holds entries 4l .. 4l + 3, so the
// lane-major order is index order. The list top-p sorts by (p desc, idx
// asc) through ranks (each lane counts the keys below its own, read as LDS
// broadcasts), and every sequential sum is the one-wave exact method.
// Returns false (uniform), having written nothing, when the list needs the
// general path (uniform branches, NaN, or a non-finite temperature product).
constexpr uint32_t kWaveList = 256;

// The reference's own sequential f32 loop over xs[0..n) (LDS, 16-byte
// aligned, zero from n up to the next multiple of 32), run by every lane of
// the wave on broadcast reads. The running sum never decreases, so a search
// first adds whole blocks of 32 (the next block's loads in flight meanwhile)
// and stops at the first block whose end meets the condition, then repeats
// that block one element at a time. For short lists this is cheaper than
// the parity-map method, whose cost grows with the binades the sum crosses.
__device__ __forceinline__ EcssResult seq_ecss(const float* xs, uint32_t n, int mode, float theta) {
  const float4* x4 = reinterpret_cast<const float4*>(xs);
  const uint32_t nb = (n + 31u) >> 5;
  float c = 0.f;
  uint32_t hit = nb;
  for (uint32_t bk = 0; bk < nb; ++bk) {
    float4 cur[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) cur[m] = x4[8u * bk + (uint32_t)m];
    float y = c;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      y = __fadd_rn(y, cur[m].x);
      y = __fadd_rn(y, cur[m].y);
      y = __fadd_rn(y, cur[m].z);
      y = __fadd_rn(y, cur[m].w);
    }
    if (mode != kEcssSum && ecss_cond(mode, y, theta)) {
      hit = bk;
      break;
    }
    c = y;
  }
  EcssResult r;
  r.c = c;
  r.found = 0;
  r.pos = -1;
  r.before = 0.f;
  if (hit == nb) return r;
  // the hit block again: lane q keeps the sum before and after element q
  const uint32_t lane = threadIdx.x & 63u;
  float4 hb[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) hb[m] = x4[8u * hit + (uint32_t)m];
  float y = c, mine = 0.f, pre = 0.f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float xq[4] = {hb[m].x, hb[m].y, hb[m].z, hb[m].w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float y1 = __fadd_rn(y, xq[u]);
      pre = lane == (uint32_t)(4 * m + u) ? y : pre;
      mine = lane == (uint32_t)(4 * m + u) ? y1 : mine;
      y = y1;
    }
  }
  const unsigned long long hm = __ballot(lane < 32u && ecss_cond(mode, mine, theta));
  const int q = __ffsll((long long)hm) - 1;  // the block end met the condition: q >= 0
  r.c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), q));
  r.before = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pre), q));
  r.found = 1;
  r.pos = (int)(32u * hit) + q;
  return r;
}


// f32::max folded in index order (NaN excluded by the caller): between equal
// values (+0 and -0) the later one wins, as in fold(-inf, f32::max).
__device__ __forceinline__ float op_maxl(float l, float r) { return r >= l ? r : l; }

// Maximum (f32::max in index order, NaN skipped) and NaN flag of one value
// per thread over the first nw waves; every thread gets the result. Waves
// at or past nw contribute nothing but must call it (two barriers).
__device__ __forceinline__ float small_max(float v, bool valid, uint32_t nw, Smem& s, bool* any_nan) {
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  if (w < nw) {
    const bool nn = valid && is_nan(v);
    const float m = wave_reduce(nn || !valid ? kNegInf : v, kNegInf, op_maxl);
    const bool wn = __ballot(nn) != 0ull;
    if (lane == 0) {
      s.red_f[w] = m;
      s.red_b[w] = wn ? 1u : 0u;
    }
  }
  __syncthreads();
  float r = kNegInf;
  uint32_t f = 0;
  for (uint32_t i = 0; i < nw; ++i) {
    r = op_maxl(r, s.red_f[i]);
    f |= s.red_b[i];
  }
  __syncthreads();
  *any_nan = f != 0u;
  return r;
}

// Everything after top-k for a list of at most kWaveList entries (s.A,
// (idx << 32) | key, ascending idx) whose maximum is finite and that holds
// no NaN: thread j < n holds entry j (only the first nw = ceil(n / 64) waves
// work, the others wait at the barriers); the four sequential sums run on
// wave 0 (seq_ecss). Returns false (uniform), having written nothing and
// left s.A as it was, when the list needs the general path (uniform
// branches, NaN, or a non-finite temperature product).
__device__ __forceinline__ bool wave_small_path(const KernelArgs& a, int b, const RowParams& P,
                                                uint32_t n, bool topp_done, float r, Smem& s,
                                                RowTrace& tr) {
  const uint32_t t = threadIdx.x, V = a.vocab, lane = t & 63u, w = t >> 6;
  const uint32_t nw = (n + 63u) >> 6;
  const bool wact = w < nw;
  float* xs = reinterpret_cast<float*>(s.Bk);  // [kWaveList] summands in index order
  float* sp = xs + kWaveList;                   // [kWaveList] p by rank
  float* pv = sp + kWaveList;                   // [kWaveList] p by index
  uint32_t* rank = reinterpret_cast<uint32_t*>(pv + kWaveList);  // [kWaveList]
  float* res = reinterpret_cast<float*>(rank + kWaveList);       // [8] results of wave 0
  const bool act = t < n;
  float v = kNegInf;
  if (wact) {
    if (act) v = key2f((uint32_t)s.A[t]);
    // seq_ecss reads whole blocks of 32: zeros past the list
    if (t >= n && t < ((n + 31u) & ~31u)) {
      xs[t] = 0.f;
      sp[t] = 0.f;
    }
    rank[t] = 0u;
  }
  bool nan;
  const float m = small_max(v, act, nw, s, &nan);
  if (!is_finite(m) || nan) return false;
  bool kept = act;
  float tp_sum = 0.f, tp_cum = 0.f;
  uint32_t tp_kept = 0;
  const bool do_topp = (P.flags & kTopP) && !topp_done;
  if (do_topp) {
    // top-p on the list (sampling.rs:942-967): softmax at T = 1 in index
    // order, then the cumulative sum in (p desc, idx asc) order
    float ex = 0.f;
    if (wact) {
      ex = act ? expf_glibc(__fsub_rn(v, m)) : 0.f;
      if (act) xs[t] = ex;
    }
    __syncthreads();
    if (t < 64u) {
      const float S1w = seq_ecss(xs, n, kEcssSum, 0.f).c;
      if (lane == 0) res[0] = S1w;
    }
    __syncthreads();
    const float S1 = res[0];
    const float p = act ? __fdiv_rn(ex, S1) : 0.f;
    if (act) pv[t] = p;
    if (wact && t >= n) pv[t] = 0.f;
    __syncthreads();
    // rank of entry j in (p desc, idx asc) order: keys (~p << 32) | j (the
    // list is in idx order), four threads per entry, each over a quarter
    // of the list, 16 keys at a time
    {
      const uint32_t j = t & (kWaveList - 1u), g = t / kWaveList;
      const uint32_t i0 = g * (kWaveList / 4u), i1 = min(n, i0 + kWaveList / 4u);
      if (j < ((n + 63u) & ~63u) && i0 < i1) {
        const uint64_t kj = ((uint64_t)(~__float_as_uint(j < n ? pv[j] : 0.f)) << 32) | j;
        uint32_t c = 0;
        for (uint32_t ib = i0; ib < i1; ib += 16u) {
          const float4* p4 = reinterpret_cast<const float4*>(pv + ib);
          float4 q[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) q[u] = p4[u];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const float qq[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t i = ib + 4u * (uint32_t)u + (uint32_t)e;
              const uint64_t ki = ((uint64_t)(~__float_as_uint(qq[e])) << 32) | (i < i1 ? i : 0xffffffffu);
              c += ki < kj ? 1u : 0u;
            }
          }
        }
        if (c && j < n) atomicAdd(&rank[j], c);
      }
    }
    __syncthreads();
    const uint32_t rk = act ? rank[t] : 0u;
    if (act) sp[rk] = p;
    __syncthreads();
    if (t < 64u) {
      const EcssResult wr = seq_ecss(sp, n, kEcssFindGe, P.top_p);
      if (lane == 0) {
        res[1] = wr.c;
        reinterpret_cast<int*>(res)[2] = wr.found ? wr.pos : -1;
      }
    }
    __syncthreads();
    const int wpos = reinterpret_cast<const int*>(res)[2];
    tp_sum = S1;
    tp_cum = res[1];
    tp_kept = wpos >= 0 ? (uint32_t)wpos + 1u : V;
    if (wpos >= 0) kept = act && rk <= (uint32_t)wpos;
  }
  // min-p (sampling.rs:976-994): the bound comes from the surviving
  // maximum, which top-p always keeps (it has the largest p)
  if (P.flags & kMinP) {
    const float bound = __fadd_rn(m, P.log_min_p);
    kept = kept && !(v < bound);
  }
  // temperature, softmax, inverse-CDF draw (sampling.rs:516-526, 1003-1014)
  const float wv = kept ? __fmul_rn(v, P.inv_temp) : kNegInf;
  bool nan3 = false;
  // Without min-p the kept set holds the list maximum m (top-p keeps the
  // largest p), and x -> x * inv_temp is monotone under rounding for
  // inv_temp > 0, so its maximum is m * inv_temp; a non-finite product
  // (inv_temp = inf) takes the general path below.
  const float m3 = (P.flags & kMinP) ? small_max(wv, kept, nw, s, &nan3) : __fmul_rn(m, P.inv_temp);
  if (!is_finite(m3) || nan3) return false;  // list and s.A untouched: the general path redoes it
  float e3 = 0.f;
  if (wact) {
    e3 = kept ? expf_glibc(__fsub_rn(wv, m3)) : 0.f;
    if (act) xs[t] = e3;
  }
  __syncthreads();
  if (t < 64u) {
    const float S3w = seq_ecss(xs, n, kEcssSum, 0.f).c;
    if (lane == 0) res[3] = S3w;
  }
  __syncthreads();
  const float S3 = res[3];
  if (act) xs[t] = kept ? __fdiv_rn(e3, S3) : 0.f;
  __syncthreads();
  if (t < 64u) {
    const EcssResult ec = seq_ecss(xs, n, kEcssFindGt, r);
    if (lane == 0) {
      res[4] = ec.found ? ec.before : ec.c;
      res[5] = ec.c;
      reinterpret_cast<uint32_t*>(res)[6] = ec.found ? (uint32_t)(s.A[ec.pos] >> 32) : V - 1u;
    }
  }
  __syncthreads();
  tr.path |= 2u;
  if (do_topp) {
    tr.topp_sum = tp_sum;
    tr.topp_kept = tp_kept;
    tr.topp_cum = tp_cum;
  }
  tr.final_max = m3;
  tr.final_sum = S3;
  tr.cdf_before = res[4];
  tr.cdf_at = res[5];
  write_result(a, b, reinterpret_cast<const uint32_t*>(res)[6], tr);
  return true;
}

// Everything after top-k for a row whose survivors are in s.A as
// (idx << 32) | key, ascending idx (sampling.rs:502-526): top-p on the list
// (unless already applied), min-p, temperature, softmax, draw.
__device__ __forceinline__ void small_path(const KernelArgs& a, int b, const RowParams& P, uint32_t nlist,
                           bool topp_done, float rdraw, Smem& s, RowTrace& tr,
                           float known_max = __builtin_nanf("")) {
  if (nlist <= kWaveList && wave_small_path(a, b, P, nlist, topp_done, rdraw, s, tr)) return;
  const int t = threadIdx.x;
  const uint32_t V = a.vocab;
  tr.path |= 2u;
  // top-p on the list (sampling.rs:942-967)
  bool lpred = false;  // list-level top-p predicate active
  bool lunif = false;
  uint32_t lplim = 0;
  float lpstar = 0.f, lm1 = 0.f, lS1 = 1.f;
  uint32_t ljstar = 0;
  const uint32_t n = nlist;
  auto lv = [&](uint32_t j) -> float { return key2f((uint32_t)s.A[j]); };
  if ((P.flags & kTopP) && !topp_done) {
    float m = kNegInf;
    uint32_t nan = 0;
    for (uint32_t j = t; j < n; j += kThreads) {
      m = rmax(m, lv(j));
      nan |= is_nan(lv(j)) ? 1u : 0u;
    }
    m = block_rmax(m, s);
    nan = block_or_u32(nan, s);
    lm1 = m;
    if (!is_finite(m)) {
      tr.path |= 8u;
      float u = __fdiv_rn(1.0f, __uint2float_rn(V));
      EcssResult e = const_ecss(V, u, kEcssFindGe, P.top_p, s);
      if (e.found) {
        lunif = true;
        lplim = (uint32_t)e.pos;
        tr.topp_kept = lplim + 1;
      } else {
        tr.topp_kept = V;
      }
      tr.topp_cum = e.c;
    } else if (nan) {
      tr.topp_sum = __uint_as_float(0x7fc00000u);
      tr.topp_kept = V;
    } else {
      EcssResult e = list_ecss(
          n, [&](uint32_t j) { return expf_glibc(__fsub_rn(lv(j), lm1)); }, kEcssSum, 0.f, 0.f, s);
      lS1 = e.c;
      tr.topp_sum = lS1;
      for (uint32_t j = t; j < n; j += kThreads) {
        float p = __fdiv_rn(expf_glibc(__fsub_rn(lv(j), lm1)), lS1);
        s.Bk[j] = ((uint64_t)(~__float_as_uint(p)) << 32) | j;
      }
      __syncthreads();
      sort_u64_asc(s.Bk, n, 2u * n <= (uint32_t)kCap ? s.Bk + n : nullptr, s);
      EcssResult w = list_ecss(
          n, [&](uint32_t j) { return __uint_as_float(~(uint32_t)(s.Bk[j] >> 32)); },
          kEcssFindGe, P.top_p, 0.f, s);
      if (w.found) {
        lpred = true;
        lpstar = __uint_as_float(~(uint32_t)(s.Bk[w.pos] >> 32));
        ljstar = (uint32_t)s.Bk[w.pos];
        tr.topp_kept = (uint32_t)w.pos + 1u;
      } else {
        tr.topp_kept = V;
      }
      tr.topp_cum = w.c;
    }
  }
  // compact the list to the entries that survive top-p
  if (lpred || lunif) {
    if (t == 0) s.cnt = 0;
    __syncthreads();
    // entries are kept in index order: process in order with a block scan
    for (uint32_t base = 0; base < n; base += kThreads) {
      const uint32_t j = base + t;
      bool keep = false;
      uint64_t e = 0;
      if (j < n) {
        e = s.A[j];
        if (lunif) {
          keep = (uint32_t)(e >> 32) <= lplim;
        } else {
          float p = __fdiv_rn(expf_glibc(__fsub_rn(lv(j), lm1)), lS1);
          keep = p > lpstar || (p == lpstar && j <= ljstar);
        }
      }
      uint32_t inc = block_incl_scan_u32(keep ? 1u : 0u, s);
      const uint32_t c0 = s.cnt;
      __syncthreads();
      if (keep) s.Bk[c0 + inc - 1] = e;
      if (t == kThreads - 1) s.cnt = c0 + inc;
      __syncthreads();
    }
    const uint32_t nk = s.cnt;
    for (uint32_t j = t; j < nk; j += kThreads) s.A[j] = s.Bk[j];
    __syncthreads();
    nlist = nk;
  }
  LUMEN_TICK("small_before_final", b);
  uint32_t tok = final_on_list(a, P, nlist, rdraw, s, tr, known_max);
  LUMEN_TICK("small_after_final", b);
  write_result(a, b, tok, tr);
}

// ---- anti-restate candidates (sampling.rs:563-603) -------------------------
// guarded_argmax probes the raw argmax, then argmax_excluding over the finite
// values: at most 8 probes, so the raw argmax and the 8 largest finite keys
// ((total_cmp key << 32) | ~id: value desc, id asc) decide every outcome.
struct Top8 {
  uint64_t t[8];  // descending; 0 = empty (no real key is 0: ids are < 2^32 - 1)
};

__device__ __forceinline__ void top8_init(Top8& x) {
#pragma unroll
  for (int q = 0; q < 8; ++q) x.t[q] = 0ull;
}

__device__ __forceinline__ void top8_push(Top8& x, uint64_t k) {
  if (k <= x.t[7]) return;
#pragma unroll
  for (int q = 7; q > 0; --q) x.t[q] = k > x.t[q - 1] ? x.t[q - 1] : (k > x.t[q] ? k : x.t[q]);
  x.t[0] = k > x.t[0] ? k : x.t[0];
}

// The wave's 8 largest keys (the same in every lane) from per-lane sorted
// lists: 8 rounds of a wave maximum over the heads, the owner popping its head.
__device__ __forceinline__ void wave_top8(Top8& x, uint64_t out[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const uint64_t m = wave_reduce(x.t[0], (uint64_t)0, op_max_u64);
    out[r] = m;
    if (m != 0ull && x.t[0] == m) {
#pragma unroll
      for (int q = 0; q < 7; ++q) x.t[q] = x.t[q + 1];
      x.t[7] = 0ull;
    }
  }
}

// The block's 8 largest keys, returned in LDS (s.Bk[128 .. 135]). Uses
// s.Bk[0 .. 135]; starts with a barrier, so s.Bk may be in use before.
__device__ __forceinline__ const uint64_t* block_top8(Top8& x, Smem& s) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  uint64_t out[8];
  wave_top8(x, out);
  __syncthreads();
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < 8; ++r) s.Bk[w * 8u + (uint32_t)r] = out[r];
  }
  __syncthreads();
  if (t < 64u) {
    Top8 y;
    top8_init(y);
    static_assert(kWaves * 8 <= 128, "two entries per lane");
    top8_push(y, s.Bk[2u * lane]);
    top8_push(y, s.Bk[2u * lane + 1u]);
    wave_top8(y, out);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 8; ++r) s.Bk[128 + r] = out[r];
    }
  }
  __syncthreads();
  return s.Bk + 128;
}

__device__ __forceinline__ void write_guard(const KernelArgs& a, int b, uint32_t raw,
                                            const uint64_t* top) {
  if (threadIdx.x != 0) return;
  uint32_t g[kGuardWords];
  g[0] = raw;
#pragma unroll
  for (int r = 0; r < 8; ++r) g[1 + r] = top[r] ? ~(uint32_t)top[r] : kGuardNone;
  if (a.guard)
#pragma unroll
    for (int r = 0; r < kGuardWords; ++r) a.guard[(uint64_t)b * kGuardWords + r] = g[r];
  if (a.guard_mapped)
#pragma unroll
    for (int r = 0; r < kGuardWords; ++r) a.guard_mapped[(uint64_t)b * kGuardWords + r] = g[r];
}

// ---- top-p over distinct values (bf16 rows) ---------------------------------
// A bf16 row holds at most 65536 distinct values, and equal values have equal
// probabilities, so the cumulative sum of apply_top_p_on_logits
// (sampling.rs:942-967) in (p desc, id asc) order is a walk over the distinct
// values in descending order, each value's p added once per occurrence.
// Adding one summand p c times inside a binade of the running sum is closed
// form on the grid (the facts of ecss.h): with p = (q + f) grid steps, every
// add moves q steps (f < 1/2) or q + 1 (f > 1/2); for f = 1/2 the first add
// rounds to the even neighbour and every later one moves by the even of
// q and q + 1. So a distinct value is one parity map, and the walk is the
// one-wave parity-map scan of wave_ecss with values in place of elements.

// occurrences of the value whose total_cmp key has the upper half pk, from u16 counts
__device__ __forceinline__ uint32_t vcount(const uint32_t* cw, uint32_t pk) {
  return (cw[pk >> 1] >> ((pk & 1u) << 4)) & 0xffffu;
}

// Increment map (grid steps, by incoming parity) of adding p c times inside
// the binade with exponent field E; {kSat, kSat} when one add may leave it.
__device__ __forceinline__ PMap rep_map(float p, uint32_t c, uint32_t E) {
  if (c == 0u) return PMap{0u, 0u};
  const double pu = ldexp((double)p, 150 - (int)(E ? E : 1u));
  if (!(pu < 16777216.0)) return PMap{kSat, kSat};
  const uint64_t q = (uint64_t)pu;
  const double f = pu - (double)q;
  uint64_t a0, a1;
  if (f < 0.5) {
    a0 = a1 = (uint64_t)c * q;
  } else if (f > 0.5) {
    a0 = a1 = (uint64_t)c * (q + 1u);
  } else if (!(q & 1u)) {
    a0 = (uint64_t)c * q;
    a1 = a0 + 1u;
  } else {
    a0 = (uint64_t)c * (q + 1u);
    a1 = a0 - 1u;
  }
  return PMap{(uint32_t)(a0 > kSat ? kSat : a0), (uint32_t)(a1 > kSat ? kSat : a1)};
}

// c adds of p to y in sequence from y's exact value: closed form inside each
// binade, one real add for each add that changes binade. With `find`, stops
// at the first add whose result is >= theta: returns true, j = its 0-based
// index, prev = the sum before it.
__device__ __forceinline__ bool rep_replay(float& y, float& prev, float p, uint32_t c, float theta,
                                           bool find, uint32_t& j) {
  uint32_t done = 0;
  prev = y;
  while (done < c) {
    const uint32_t cb = __float_as_uint(y);
    const uint32_t E = cb >> 23;
    const uint32_t ub = (cb & 0xff800000u) + 0x00800000u;
    const double pu = ldexp((double)p, 150 - (int)(E ? E : 1u));
    uint32_t i0 = 0, d = 0;
    bool real = !(pu < 16777216.0);
    if (!real) {
      const uint32_t q = (uint32_t)pu;
      const double f = pu - (double)q;
      if (f < 0.5) {
        i0 = d = q;
      } else if (f > 0.5) {
        i0 = d = q + 1u;
      } else {
        i0 = (((cb & 1u) + q) & 1u) ? q + 1u : q;
        d = q + (q & 1u);
      }
      if (i0 > ub - 1u - cb) real = true;
    }
    if (real) {
      prev = y;
      y = __fadd_rn(y, p);
      if (find && y >= theta) {
        j = done;
        return true;
      }
      ++done;
      continue;
    }
    if (i0 == 0u && d == 0u) return false;  // no add moves y any more
    const uint32_t room = ub - 1u - cb;
    const uint64_t fit = d ? 1u + (uint64_t)(room - i0) / d : (uint64_t)c;
    const uint32_t n = (uint32_t)(fit < (uint64_t)(c - done) ? fit : (uint64_t)(c - done));
    auto val = [&](uint32_t k) { return __uint_as_float(cb + i0 + (k - 1u) * d); };  // after k adds
    if (find && val(n) >= theta) {
      uint32_t lo = 1u, hi = n;
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (val(mid) >= theta) hi = mid; else lo = mid + 1u;
      }
      prev = lo > 1u ? val(lo - 1u) : y;
      y = val(lo);
      j = done + lo - 1u;
      return true;
    }
    prev = n > 1u ? val(n - 1u) : y;
    y = val(n);
    done += n;
  }
  return false;
}

struct ValHit {
  bool found;
  uint32_t lane;  // lane of the value holding the crossing
  uint32_t j;     // 0-based occurrence of that value at the crossing
  float c;        // running sum after the crossing add (or after the chunk)
};

// One chunk of 64 distinct values (lane order = walk order), on one wave.
// c: the running sum, updated. Uniform result.
__device__ __forceinline__ ValHit wave_values(float& c, float p, uint32_t cnt, float theta) {
  const int lane = threadIdx.x & 63;
  int t0 = 0;
  for (;;) {
    const uint32_t cb = __float_as_uint(c);
    const uint32_t ub = (cb & 0xff800000u) + 0x00800000u;
    const bool act = lane >= t0;
    const PMap m = act ? rep_map(p, cnt, cb >> 23) : PMap{0u, 0u};
    const PMap id{0u, 0u};
    const PMap ex = wave_shr1(wave_scan_incl(m, id, pm_combine), id);
    const uint32_t par0 = cb & 1u;
    const uint32_t before = par0 ? ex.a1 : ex.a0;
    const uint32_t own = ((par0 ^ before) & 1u) ? m.a1 : m.a0;
    const uint32_t sbits = cb + before;
    const uint32_t ebits = sbits + own;
    const bool cross = act && (before >= kSat || ebits >= ub);
    const bool hit = act && !cross && cnt && __uint_as_float(ebits) >= theta;
    const unsigned long long bm = __ballot(cross), hm = __ballot(hit);
    const int tb = bm ? __ffsll((long long)bm) - 1 : 64;
    const int th = hm ? __ffsll((long long)hm) - 1 : 64;
    if (th < 64 || tb < 64) {
      const int r = th < tb ? th : tb;
      float y = __uint_as_float(sbits), prev = y;
      uint32_t j = 0;
      bool f = false;
      if (lane == r) f = rep_replay(y, prev, p, cnt, theta, true, j);
      const bool fr = __builtin_amdgcn_readlane((int)f, r) != 0;
      const float yr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(y), r));
      if (fr) {
        c = yr;
        return ValHit{true, (uint32_t)r, (uint32_t)__builtin_amdgcn_readlane((int)j, r), yr};
      }
      c = yr;
      t0 = r + 1;
      if (t0 < 64) continue;
    } else {
      c = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)ebits, 63));
    }
    return ValHit{false, 0u, 0u, c};
  }
}

// Counts of a bf16 row by value, taken during the top-p max pass: u16
// counts of every bf16 value in s.A / s.Bk (by the upper half of its
// total_cmp key), and per block of 256 values in s.H[0 .. 255].
__device__ __forceinline__ uint32_t* bv_counts(Smem& s) { return reinterpret_cast<uint32_t*>(s.A); }

__device__ __forceinline__ void bv_clear(Smem& s) {
  static_assert(sizeof(s.A) + sizeof(s.Bk) == 65536 * 2, "u16 counts of every bf16 value");
  uint32_t* cw = bv_counts(s);  // s.A and s.Bk are adjacent
  for (uint32_t i = threadIdx.x; i < 32768u; i += kThreads) cw[i] = 0u;
  for (uint32_t i = threadIdx.x; i < 256u; i += kThreads) s.H[i] = 0u;
}

__device__ __forceinline__ void bv_count(float x, Smem& s) {
  const uint32_t pk = tkey(x) >> 16;
  atomicAdd(&bv_counts(s)[pk >> 1], 1u << ((pk & 1u) << 4));
}

// Per block of 256 values, the sum of the u16 counts into s.H[0 .. 255] and
// the number of distinct values present into s.H[256 .. 511];
// returns (uniformly) whether the counts are exact: a u16 count that
// overflowed lost 65535 or 65536 (its carry goes to the neighbour or out of
// the word), so the counts are exact iff they add up to the n elements
// counted.
__device__ __forceinline__ bool bv_blocks(uint32_t n, Smem& s) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  const uint32_t* cw = bv_counts(s);
  // wave w sums blocks 16w .. 16w+15 (128 words each), its lanes reading
  // consecutive words (no bank conflicts)
  uint32_t part = 0;
#pragma unroll 2
  for (uint32_t j = 0; j < 16u; ++j) {
    const uint32_t w0 = cw[(16u * w + j) * 128u + lane], w1 = cw[(16u * w + j) * 128u + 64u + lane];
    const uint32_t c = (w0 & 0xffffu) + (w0 >> 16) + (w1 & 0xffffu) + (w1 >> 16);
    const uint32_t d = ((w0 & 0xffffu) != 0u ? 1u : 0u) + ((w0 >> 16) != 0u ? 1u : 0u) +
                       ((w1 & 0xffffu) != 0u ? 1u : 0u) + ((w1 >> 16) != 0u ? 1u : 0u);
    const uint32_t cs = wave_reduce(c, 0u, op_add_u32), ds = wave_reduce(d, 0u, op_add_u32);
    if (lane == 0) {
      s.H[16u * w + j] = cs;
      s.H[256u + 16u * w + j] = ds;
    }
    part += c;
  }
  const uint32_t tot = block_sum_u32(part, s);
  return tot == n;
}

__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, Smem& s, uint32_t* total);
__device__ __forceinline__ double block_excl_scan_f64(double v, Smem& s, double* total);

// The value with key upper half pk: a negative value's key carries ones in
// its low 16 bits.
__device__ __forceinline__ float bv_value(uint32_t pk) {
  return key2f((pk << 16) | ((pk & 0x8000u) ? 0u : 0xffffu));
}

// Top-p of a bf16 row by distinct value, after bv_count over every element
// (x = vf(i, v), bf16-exact). m1 / S1: the row max and softmax sum at T = 1.
// Returns -1 when a value may occur 65536 times or more (the caller takes
// the window path), 0 when the cumulative sum never reaches top_p (every
// token kept), else 1 with the kept set
//   {x : key(x) >> 16 > pk_hi} + {x : pk_lo <= key(x) >> 16 <= pk_hi, id <= istar},
// [pk_lo, pk_hi] being the values whose p equals the crossing's. Sets the
// top-p trace fields. Uses s.A, s.Bk and s.H.
// The row and the top-k mask (kmask: keys below kcut read as -inf) come by
// value: in a non-inlined function, state reached through references would
// be reloaded from private memory on every element.
template <bool V2>
__device__ __attribute__((noinline)) int topp_by_value(const Row row, bool kmask, uint32_t kcut,
                                                       float m1, float S1,
                                                       float top_p, Smem& s, RowTrace& tr,
                                                       uint32_t& pk_lo, uint32_t& pk_hi,
                                                       uint32_t& istar, uint32_t ncount) {
  const uint32_t t = threadIdx.x, V = row.V;
  const uint32_t* cw = bv_counts(s);
  auto vf = [kmask, kcut](uint32_t, float v) -> float {
    return (kmask && tkey(v) < kcut) ? kNegInf : v;
  };
  if (V > (1u << 22) || !bv_blocks(ncount, s)) return -1;
  __syncthreads();
  auto pof = [&](uint32_t pk) { return __fdiv_rn(expf_glibc(__fsub_rn(bv_value(pk), m1)), S1); };
  // The walk in rounds of at most 1024 present values (descending), every
  // wave taking 64 of them: the parity map of its 64 values' adds for the
  // binade its start is estimated in (f64 prefix of count x p), then wave 0
  // composes the waves in order from the exact running sum, taking a wave's
  // map whenever the exact sum starts in that binade and ends in it below
  // top_p, and replaying the wave value by value (wave_values) otherwise.
  uint32_t* const list = s.H + 512;               // [1024] (pk << 16) | count
  float* const pl = reinterpret_cast<float*>(s.H + 1536);  // [1024] p
  uint32_t* const wv = s.H + 2560;                // [16][4] binade, a0, a1, count sum
  const uint32_t lane = t & 63u, w = t >> 6;
  float c = 0.f;
  uint32_t wrank = 0, pks = 0;
  float ph = 0.f;
  bool hit = false;
  int bh = 255;  // next block (of 256 values) to take, descending
  while (bh >= 0 && !hit) {
    // plan: whole blocks while their distinct values fit in 1024
    if (t < 64u) {
      uint32_t take = 0, tot = 0;
      for (int base = bh; base >= 0; base -= 64) {
        const int blk = base - (int)lane;
        const uint32_t d = blk >= 0 ? s.H[256 + blk] : 0u;
        const uint32_t inc = wave_scan_incl(d, 0u, op_add_u32);
        const unsigned long long fit = __ballot(blk >= 0 && tot + inc <= 1024u);
        // blocks are taken while the running total fits (a prefix of lanes)
        const uint32_t nfit = fit == ~0ull ? 64u : (uint32_t)__ffsll((long long)~fit) - 1u;
        take += nfit;
        if (nfit > 0u) tot += (uint32_t)__builtin_amdgcn_readlane((int)inc, (int)nfit - 1);
        if (nfit < 64u) break;
      }
      if (take == 0u) take = 1u;  // a block never holds more than 256 values
      if (lane == 0) {
        s.misc_i[0] = bh - (int)take;  // the round covers blocks (bh - take, bh]
        s.misc_u[0] = tot;
      }
    }
    __syncthreads();
    const int bl = s.misc_i[0];
    __syncthreads();
    LUMEN_TICK("bv_plan", LUMEN_TIMING_ROW);
    uint32_t n;
    if (V2) {
    // compaction of the present values of blocks (bl, bh], descending: wave
    // w takes the key offsets [w * wspan, (w + 1) * wspan) below khi, 512
    // per step, each lane 8 consecutive keys (one 16-byte read of 4 count
    // words), placed by a wave scan of the lanes' counts
    const uint32_t khi = (uint32_t)(bh + 1) * 256u, klo = (uint32_t)(bl + 1) * 256u;
    const uint32_t span = khi - klo, wspan = (span + 512u * kWaves - 1u) / (512u * kWaves) * 512u;
    auto group = [&](uint32_t off0) -> u32x4 {  // the 4 words of keys khi-1-off0 .. khi-8-off0
      return off0 < span ? *reinterpret_cast<const u32x4*>(cw + ((khi - 8u - off0) >> 1))
                         : u32x4{0u, 0u, 0u, 0u};
    };
    auto nz = [](uint32_t x) { return ((x & 0xffffu) != 0u ? 1u : 0u) + ((x >> 16) != 0u ? 1u : 0u); };
    uint32_t mine = 0;
    for (uint32_t q = 0; q < wspan; q += 512u) {
      const u32x4 g = group(w * wspan + q + 8u * lane);
      mine += wave_reduce(nz(g.x) + nz(g.y) + nz(g.z) + nz(g.w), 0u, op_add_u32);
    }
    uint32_t at = block_excl_scan_u32(lane == 0 ? mine : 0u, s, &n);
    at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at);
    for (uint32_t q = 0; q < wspan && mine; q += 512u) {
      const uint32_t off0 = w * wspan + q + 8u * lane;
      const u32x4 g = group(off0);
      const uint32_t cl = nz(g.x) + nz(g.y) + nz(g.z) + nz(g.w);
      const uint32_t incl = wave_scan_incl(cl, 0u, op_add_u32);
      uint32_t pos = at + incl - cl;
      const uint32_t wd[4] = {g.w, g.z, g.y, g.x};  // descending keys: high word, high half first
#pragma unroll
      for (uint32_t k = 0; k < 8u; ++k) {
        const uint32_t cnt = (wd[k >> 1] >> ((1u - (k & 1u)) << 4)) & 0xffffu;
        if (cnt) {
          if (pos < 1024u) list[pos] = ((khi - 1u - off0 - k) << 16) | cnt;
          ++pos;
        }
      }
      at += (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    }
    __syncthreads();
    } else {
    // compaction of the present values of blocks (bl, bh], descending: wave
    // w takes keys khi - 1 - [w * wspan, (w + 1) * wspan), 64 consecutive
    // keys per step (one per lane), and places them by ballot
    const uint32_t khi = (uint32_t)(bh + 1) * 256u, klo = (uint32_t)(bl + 1) * 256u;
    const uint32_t span = khi - klo, wspan = (span + 64u * kWaves - 1u) / (64u * kWaves) * 64u;
    uint32_t mine = 0;
    for (uint32_t q = 0; q < wspan; q += 64u) {
      const uint32_t off = w * wspan + q + lane;
      mine += (uint32_t)__popcll(__ballot(off < span && vcount(cw, khi - 1u - off) != 0u));
    }
    uint32_t at = block_excl_scan_u32(lane == 0 ? mine : 0u, s, &n);
    at = (uint32_t)__builtin_amdgcn_readfirstlane((int)at);
    for (uint32_t q = 0; q < wspan && mine; q += 64u) {
      const uint32_t off = w * wspan + q + lane;
      const uint32_t pk = khi - 1u - off;
      const uint32_t cnt = off < span ? vcount(cw, pk) : 0u;
      const unsigned long long bm = __ballot(cnt != 0u);
      const uint32_t pos = at + (uint32_t)__popcll(bm & ((1ull << lane) - 1ull));
      if (cnt && pos < 1024u) list[pos] = (pk << 16) | cnt;
      at += (uint32_t)__popcll(bm);
    }
    __syncthreads();
    }
    if (n > 1024u) n = 1024u;  // cannot happen: the plan bounds the round
    LUMEN_TICK("bv_list", LUMEN_TIMING_ROW);
    // every wave: its values' p, the f64 estimate of its start, its map
    const uint32_t e = t < n ? list[t] : 0u;
    const uint32_t cnt = e & 0xffffu;
    const float p = cnt ? pof(e >> 16) : 0.f;
    pl[t] = p;
    double tot_d;
    const double pre = block_excl_scan_f64((double)cnt * (double)p, s, &tot_d);
    const double st = (double)c + __shfl(pre, 0);
    const uint32_t E = est_binade(st) >> 23;
    const PMap m = rep_map(p, cnt, E);
    const PMap mt = wave_read(wave_scan_incl(m, PMap{0u, 0u}, pm_combine), 63);
    const uint32_t cs = wave_reduce(cnt, 0u, op_add_u32);
    if (lane == 0) {
      wv[4 * w] = E;
      wv[4 * w + 1] = mt.a0;
      wv[4 * w + 2] = mt.a1;
      wv[4 * w + 3] = cs;
    }
    __syncthreads();
    LUMEN_TICK("bv_maps", LUMEN_TIMING_ROW);
    if (t < 64u) {
      for (uint32_t ww = 0; ww < (n + 63u) / 64u; ++ww) {
        const uint32_t cb = __float_as_uint(c);
        const uint32_t ub = (cb & 0xff800000u) + 0x00800000u;
        const uint32_t wE = wv[4 * ww], a0 = wv[4 * ww + 1], a1 = wv[4 * ww + 2], wc = wv[4 * ww + 3];
        const uint32_t st2 = (cb & 1u) ? a1 : a0;
        if ((cb >> 23) == wE && st2 < kSat && st2 < ub - cb && __uint_as_float(cb + st2) < top_p) {
          c = __uint_as_float(cb + st2);
          wrank += wc;
          continue;
        }
        LUMEN_TICK("bv_fb", LUMEN_TIMING_ROW);
        const uint32_t k = 64u * ww + lane;
        const uint32_t ck = k < n ? (list[k] & 0xffffu) : 0u;
        const float pk_p = k < n ? pl[k] : 0.f;
        const ValHit h = wave_values(c, pk_p, ck, top_p);
        if (h.found) {
          wrank += wave_reduce(lane < h.lane ? ck : 0u, 0u, op_add_u32) + h.j + 1u;
          ph = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pk_p), (int)h.lane));
          pks = (uint32_t)__builtin_amdgcn_readlane((int)(list[64u * ww + h.lane] >> 16), 0);
          hit = true;
          break;
        }
        wrank += wc;
      }
      if (lane == 0) {
        s.misc_u[1] = hit ? 1u : 0u;
        s.red_f[1] = c;
        s.misc_u[2] = wrank;
        s.misc_u[3] = pks;
        s.red_f[2] = ph;
      }
    }
    __syncthreads();
    hit = s.misc_u[1] != 0u;
    c = s.red_f[1];
    wrank = s.misc_u[2];
    pks = s.misc_u[3];
    ph = s.red_f[2];
    __syncthreads();
    bh = bl;
  }
  LUMEN_TICK("bv_cross", LUMEN_TIMING_ROW);
  if (t < 64u) {
    const ValHit h{hit, 0u, 0u, c};
    // the values around the crossing's with the same p (p is monotone in
    // the value, so they are adjacent among the values present)
    uint32_t hi = pks, lo = pks;
    if (h.found) {
      for (uint32_t base = pks + 1u; base <= 0xffffu; base += 64u) {
        const uint32_t pk = base + lane;
        const uint32_t cnt = pk <= 0xffffu ? vcount(cw, pk) : 0u;
        const bool other = cnt && pof(pk) != ph;
        const unsigned long long om = __ballot(other);
        const unsigned long long em = __ballot(cnt && !other) &
                                      (om ? ((1ull << (__ffsll((long long)om) - 1)) - 1ull) : ~0ull);
        if (em) hi = base + 63u - (uint32_t)__clzll((long long)em);
        if (om) break;
      }
      for (int base = (int)pks - 1; base >= 0; base -= 64) {
        const int pk = base - (int)lane;
        const uint32_t cnt = pk >= 0 ? vcount(cw, (uint32_t)pk) : 0u;
        const bool other = cnt && pof((uint32_t)pk) != ph;
        const unsigned long long om = __ballot(other);
        const unsigned long long em = __ballot(cnt && !other) &
                                      (om ? ((1ull << (__ffsll((long long)om) - 1)) - 1ull) : ~0ull);
        if (em) lo = (uint32_t)(base - (63 - __clzll((long long)em)));
        if (om) break;
      }
    }
    if (lane == 0) {
      s.misc_u[0] = h.found ? 1u : 0u;
      s.misc_u[1] = wrank;
      s.misc_u[2] = lo;
      s.misc_u[3] = hi;
      s.red_f[0] = c;
    }
  }
  __syncthreads();
  const bool found = s.misc_u[0] != 0u;
  const uint32_t rank = s.misc_u[1];
  // the group bounds in registers: the loops below must not re-read them
  // through the output references (their stores may alias LDS atomics)
  const uint32_t glo = s.misc_u[2], ghi = s.misc_u[3];
  pk_lo = glo;
  pk_hi = ghi;
  tr.topp_cum = s.red_f[0];
  __syncthreads();
  LUMEN_TICK("bv_walk", LUMEN_TIMING_ROW);
  if (!found) {
    tr.topp_kept = V;
    return 0;
  }
  tr.topp_kept = rank;
  // tokens with a larger p: the counts of the values above pk_hi
  uint32_t gt = 0;
  for (uint32_t pk = ghi + 1u + t; pk <= 0xffffu; pk += kThreads) gt += vcount(cw, pk);
  gt = block_sum_u32(gt, s);
  LUMEN_TICK("bv_gt", LUMEN_TIMING_ROW);
  // the kept set ends at the (rank - gt)-th id, in id order, of the tokens
  // valued in [pk_lo, pk_hi]: an id histogram (lowest ids at the top) finds
  // its bin, then a bitmap of that bin its id
  const uint32_t k = rank - gt;
  uint32_t sh = 0;
  while ((V - 1u) >> sh >= 2048u) ++sh;  // bins of at most 2048 ids (V <= 2^22)
  clear_hist(s.H, 2048);
  __syncthreads();
  row_foreach(row, [&](uint32_t i, float v) {
    const uint32_t pk = tkey(vf(i, v)) >> 16;
    if (pk >= glo && pk <= ghi) atomicAdd(&s.H[2047u - (i >> sh)], 1u);
  });
  __syncthreads();  // every wave's counts are in before the search reads them
  tr.passes++;
  LUMEN_TICK("bv_idhist", LUMEN_TIMING_ROW);
  uint32_t ab = 0;
  const int d = find_from_top(s.H, 2048, k, &ab, s);
  const uint32_t lo = (2047u - (uint32_t)d) << sh, hi = min(V, lo + (1u << sh));
  const uint32_t kk = k - ab;
  LUMEN_TICK("bv_find", LUMEN_TIMING_ROW);
  uint32_t* bits = s.H + 2048;  // one bit per id of the bin
  for (uint32_t i = t; i < 64u; i += kThreads) bits[i] = 0u;
  __syncthreads();
  range_foreach(row, lo, hi, [&](uint32_t i, float v) {
    const uint32_t pk = tkey(vf(i, v)) >> 16;
    if (pk >= glo && pk <= ghi) atomicOr(&bits[(i - lo) >> 5], 1u << ((i - lo) & 31u));
  });
  __syncthreads();
  if (t == 0) {
    uint32_t left = kk, id = lo;
    for (uint32_t w = 0; w < 64u; ++w) {
      const uint32_t n = __popc(bits[w]);
      if (left <= n) {
        uint32_t m = bits[w];
        for (uint32_t q = 1; q < left; ++q) m &= m - 1u;
        id = lo + w * 32u + (uint32_t)(__ffs(m) - 1);
        break;
      }
      left -= n;
    }
    s.misc_u[2] = id;
  }
  __syncthreads();
  istar = s.misc_u[2];
  __syncthreads();
  LUMEN_TICK("bv_istar", LUMEN_TIMING_ROW);
  return 1;
}

// The k-th smallest id (k >= 1) among the tokens i with pred(i, x), x the
// token's value through vf: an id histogram (lowest ids at the top of s.H)
// finds the bin, a bitmap of the bin (s.H + 2048) the id. Two passes.
template <class VF, class Pred>
__device__ __forceinline__ uint32_t kth_id_where(const Row& row, VF&& vf, Pred&& pred, uint32_t k,
                                                 Smem& s) {
  const uint32_t t = threadIdx.x, V = row.V;
  uint32_t sh = 0;
  while ((V - 1u) >> sh >= 2048u) ++sh;  // bins of at most 2048 ids (V <= 2^22)
  clear_hist(s.H, 2048);
  __syncthreads();
  row_foreach(row, [&](uint32_t i, float v) {
    if (pred(i, vf(i, v))) atomicAdd(&s.H[2047u - (i >> sh)], 1u);
  });
  __syncthreads();  // every wave's counts are in before the search reads them
  uint32_t ab = 0;
  const int d = find_from_top(s.H, 2048, k, &ab, s);
  const uint32_t lo = (2047u - (uint32_t)(d < 0 ? 0 : d)) << sh, hi = min(V, lo + (1u << sh));
  uint32_t* bits = s.H + 2048;
  for (uint32_t i = t; i < 64u; i += kThreads) bits[i] = 0u;
  __syncthreads();
  range_foreach(row, lo, hi, [&](uint32_t i, float v) {
    if (pred(i, vf(i, v))) atomicOr(&bits[(i - lo) >> 5], 1u << ((i - lo) & 31u));
  });
  __syncthreads();
  if (t == 0) {
    uint32_t left = k - ab, id = lo;
    for (uint32_t w = 0; w < 64u; ++w) {
      const uint32_t n = __popc(bits[w]);
      if (left <= n) {
        uint32_t m = bits[w];
        for (uint32_t q = 1; q < left; ++q) m &= m - 1u;
        id = lo + w * 32u + (uint32_t)(__ffs(m) - 1);
        break;
      }
      left -= n;
    }
    s.misc_u[2] = id;
  }
  __syncthreads();
  const uint32_t id = s.misc_u[2];
  __syncthreads();
  return id;
}

template <bool FIND, class XF>
__device__ __forceinline__ EcssResult row_rec_sum(const KernelArgs& a, int b, const Row& row,
                                                  XF&& xf, float probe, Smem& s, bool& ok);

// exp(x - m), out of line: the rare elements of a table-driven sum that
// fall outside the table (inlined into every unrolled summand, its code
// made the single-workgroup sampler spill in its hot loops)
__device__ __attribute__((noinline)) float exp_sub_outline(float x, float m) {
  return expf_glibc(__fsub_rn(x, m));
}

// The whole sampler for row b, run by one workgroup: row_single<false> is the
// fallback of the split paths inside lumen_sample_rows, row_single<true> the
// body of lumen_sample_rows_single (one workgroup per row), whose full-row
// exact sums take the record method (row_rec_sum). Two instantiations keep
// the register allocation of the split kernel independent of the latter.
template <bool V2>
__device__ __forceinline__ void row_single_body(const KernelArgs& a, int b, Smem& s) {
  const int t = threadIdx.x;
  const RowParams P = a.inline_rows ? a.inline_params[b] : a.params[b];
  const uint32_t V = a.vocab;
  RowTrace tr;
  init_trace(tr, V);
  LUMEN_TICK("rs_start", b);

  Row row = make_row(a, b);

  // ---- penalties: materialize the penalized row (sampling.rs:850-879) ----
  const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
  if ((P.flags & kPen) && h1 > h0) {
    float* dst = a.pen_scratch + (uint64_t)b * a.pen_stride;
    row_foreach(row, [&](uint32_t i, float v) { gst(dst + i, v); });
    __syncthreads();
    for (uint32_t j = h0 + t; j < h1; j += kThreads) {
      uint32_t id = a.hist_ids[j];
      if (id < V) dst[id] = penalize(row.at(id), a.hist_cnt[j], P);
    }
    __syncthreads();
    row.f = dst;
    row.h = nullptr;
    row.vec = true;
    tr.passes++;
  }
  if (a.pen_out) {
    float* po = a.pen_out + (uint64_t)b * V;
    row_foreach(row, [&](uint32_t i, float v) { gst(po + i, v); });
  }

  // ---- greedy (sampling.rs:468-476) ----
  if (P.flags & kGreedy) {
    uint64_t best = 0;
    if (P.flags & kAnti) {
      // the guard's candidates (sampling.rs:563-603)
      Top8 x;
      top8_init(x);
      row_foreach(row, [&](uint32_t i, float v) {
        const uint64_t k = ((uint64_t)tkey(v) << 32) | (uint64_t)(0xffffffffu - i);
        best = k > best ? k : best;
        if (is_finite(v)) top8_push(x, k);
      });
      best = block_max_u64(best, s);
      write_guard(a, b, 0xffffffffu - (uint32_t)best, block_top8(x, s));
    } else {
      row_foreach(row, [&](uint32_t i, float v) {
        uint64_t k = ((uint64_t)tkey(v) << 32) | (uint64_t)(0xffffffffu - i);
        best = k > best ? k : best;
      });
      best = block_max_u64(best, s);
    }
    tr.path |= 1u;
    tr.passes++;
    write_result(a, b, 0xffffffffu - (uint32_t)best, tr);
    return;
  }

  const float rdraw = row_draw(a, b);
  bool small = false;   // survivors in s.A as (idx << 32) | key, ascending idx
  uint32_t nlist = 0;
  bool topp_done = false;
  bool kmask = false;   // large path with a top-k cutoff mask
  uint32_t kcut = 0;

  // ---- top-k (sampling.rs:904-933) ----
  if (P.flags & kTopK) {
    const uint32_t k = P.top_k;
    if (k == 1) {
      uint64_t best = 0;
      row_foreach(row, [&](uint32_t i, float v) {
        uint64_t kk = ((uint64_t)tkey(v) << 32) | (uint64_t)(0xffffffffu - i);
        best = kk > best ? kk : best;
      });
      best = block_max_u64(best, s);
      tr.passes++;
      const uint32_t idx = 0xffffffffu - (uint32_t)best, key = (uint32_t)(best >> 32);
      if (t == 0) s.A[0] = ((uint64_t)idx << 32) | key;
      __syncthreads();
      nlist = 1;
      small = true;
      tr.topk_cutoff_key = key;
      tr.topk_survivors = 1;
    } else {
      uint32_t prefix = 0, pmask = 0, above = 0;
      for (int lvl = 0; lvl < 3 && !small; ++lvl) {
        const int sh = lvl == 0 ? 21 : (lvl == 1 ? 10 : 0);
        const int nb = lvl == 2 ? 1024 : 2048;
        const uint32_t dm = (uint32_t)nb - 1u;
        clear_hist(s.H, nb);
        __syncthreads();
        row_foreach(row, [&](uint32_t i, float v) {
          uint32_t kk = tkey(v);
          if ((kk & pmask) == prefix) atomicAdd(&s.H[(kk >> sh) & dm], 1u);
        });
        __syncthreads();
        tr.passes++;
        uint32_t ab = 0;
        int d = find_from_top(s.H, nb, k - above, &ab, s);
        above += ab;
        prefix |= (uint32_t)d << sh;
        pmask |= dm << sh;
        const uint32_t cnt_ge = above + s.H[d];
        __syncthreads();
        if (cnt_ge <= (uint32_t)kCap) {
          // compact all keys >= prefix (the smallest key on this digit path)
          if (t == 0) s.cnt = 0;
          __syncthreads();
          row_foreach(row, [&](uint32_t i, float v) {
            uint32_t kk = tkey(v);
            list_push(s.A, &s.cnt, kk >= prefix, ((uint64_t)(~kk) << 32) | i);
          });
          __syncthreads();
          tr.passes++;
          const uint32_t n = s.cnt;
          sort_u64_asc(s.A, n, s.Bk, s);  // descending key
          const uint32_t cut = ~(uint32_t)(s.A[k - 1] >> 32);
          // survivors: every entry with key >= cut is a prefix of the list
          uint32_t ns = 0;
          for (uint32_t j = t; j < n; j += kThreads) ns += (~(uint32_t)(s.A[j] >> 32) >= cut) ? 1u : 0u;
          ns = block_sum_u32(ns, s);
          for (uint32_t j = t; j < ns; j += kThreads) {
            uint64_t e = s.A[j];
            s.A[j] = ((uint64_t)(uint32_t)e << 32) | (uint64_t)(~(uint32_t)(e >> 32));
          }
          __syncthreads();
          sort_u64_asc(s.A, ns, s.Bk, s);  // ascending index
          nlist = ns;
          small = true;
          tr.topk_cutoff_key = cut;
          tr.topk_survivors = ns;
        } else if (lvl == 2) {
          kmask = true;
          kcut = prefix;
          tr.topk_cutoff_key = prefix;
          tr.topk_survivors = cnt_ge;
        }
      }
    }
  }

  // value after the top-k mask (large path)
  auto v1f = [&](float v) -> float { return (kmask && tkey(v) < kcut) ? kNegInf : v; };

  int pmode = 0;        // 0 none, 1 uniform index prefix, 2 probability threshold, 3 value threshold
  uint32_t plim = 0;    // pmode 1: keep idx <= plim
  float m1 = 0.f, S1 = 1.f, pstar = 0.f;
  uint32_t istar = 0;   // pmode 2: keep p > pstar or (p == pstar and idx <= istar)
  uint32_t pk_lo = 0, pk_hi = 0;  // pmode 3 (bf16 by value): keep value > pk_hi, or in
                                  // [pk_lo, pk_hi] with idx <= istar (keys' upper halves)

  if (!small) tr.path |= 4u;

  // ---- top-p on the large path (sampling.rs:942-967) ----
  if ((P.flags & kTopP) && !small) {
    float m = kNegInf;
    uint32_t nan = 0;
    // bf16 rows also count their values (top-p by distinct value): here,
    // or (lumen_sample_rows_single, whose softmax sum takes lists A and B
    // for its exp table) in a pass of their own after that sum
    const bool bf = !row.f;
    const bool count_now = bf && !V2;
    if (count_now) {
      bv_clear(s);
      __syncthreads();
    }
    if (V2 && bf && !kmask) {
      // lumen_sample_rows_single, bf16 without a top-k mask: the largest
      // total_cmp key of the non-NaN values (integer max, no NaN cases); a
      // maximum of +-0 is then taken again with f32::max semantics
      uint32_t kmax = 0x007fu;  // -inf
      row_foreach(row, [&](uint32_t, float v) {
        const uint32_t p = __float_as_uint(v) >> 16;
        const uint32_t sg = (uint32_t)((int32_t)(p << 16) >> 31);
        const uint32_t k = (p ^ (sg | 0x8000u)) & 0xffffu;
        const bool isn = (p & 0x7fffu) > 0x7f80u;
        nan |= isn ? 1u : 0u;
        kmax = isn ? kmax : max(kmax, k);
      });
      kmax = block_max_u32(kmax, s);
      nan = block_or_u32(nan, s);
      m = bv_value(kmax);
      if (m == 0.f) {
        m = kNegInf;
        row_foreach(row, [&](uint32_t, float v) { m = rmax(m, v); });
        m = block_rmax(m, s);
      }
    } else {
      row_foreach(row, [&](uint32_t i, float v) {
        float x = v1f(v);
        m = rmax(m, x);
        nan |= is_nan(x) ? 1u : 0u;
        if (count_now) bv_count(x, s);
      });
      m = block_rmax(m, s);
      nan = block_or_u32(nan, s);
    }
    tr.passes++;
    LUMEN_TICK("rs_topp_max", b);
    m1 = m;
    topp_done = true;
    if (!is_finite(m1)) {
      tr.path |= 8u;
      float u = __fdiv_rn(1.0f, __uint2float_rn(V));
      EcssResult e = const_ecss(V, u, kEcssFindGe, P.top_p, s);
      tr.topp_sum = 0.f;
      if (e.found) {
        pmode = 1;
        plim = (uint32_t)e.pos;
        tr.topp_kept = plim + 1;
      } else {
        tr.topp_kept = V;
      }
      tr.topp_cum = e.c;
    } else if (nan) {
      tr.topp_sum = __uint_as_float(0x7fc00000u);
      tr.topp_kept = V;
    } else {
      // softmax sum at T = 1 and, for the window path, a key histogram of the
      // positive-probability tokens (bf16 rows walk their value counts
      // instead, and build it only if that walk cannot run)
      // bf16 rows of lumen_sample_rows_single: exp(x - m1) from an LDS table
      // (list A) over 64 binades of |value| per sign; live summands have x
      // >= m1 - 128, so |x| <= W = max(|m1|, |m1 - 128|) and patterns above
      // the window are zero, patterns below it take the direct computation
      const bool tab1 = V2 && bf;
      float* const T1 = reinterpret_cast<float*>(s.A);
      uint32_t* const cc1 = reinterpret_cast<uint32_t*>(s.Bk);  // [8192]
      uint32_t wlo1 = 0, whi1 = 0;
      if (tab1) {
        const float W = fmaxf(fabsf(m1), fabsf(__fsub_rn(m1, 128.f)));
        uint32_t emax = ((__float_as_uint(W) >> 23) & 0xffu) + 1u;
        emax = emax > 254u ? 254u : (emax < 63u ? 63u : emax);
        wlo1 = (emax - 63u) << 7;
        whi1 = (emax + 1u) << 7;
#pragma unroll 1
        for (uint32_t j = t; j < 16384u; j += kThreads) {
          const float v = __uint_as_float((((j >> 13) << 15) | (wlo1 + (j & 8191u))) << 16);
          T1[j] = expf_glibc(__fsub_rn(v1f(v), m1));
        }
        for (uint32_t j = t; j < 8192u; j += kThreads) cc1[j] = 0u;
        __syncthreads();
      }
      // Without a top-k mask the sum also counts the values it reads, as u16
      // pairs by table entry (list B): patterns above the window are zero
      // summands (never part of the walk), and any live pattern below it
      // makes the row count in a pass of its own.
      const bool fuse = tab1 && !kmask;
      uint32_t ndead = 0, ntiny = 0;
      auto e1f = [&](uint32_t, float v) -> float {
        if (tab1) {
          const uint32_t p = __float_as_uint(v) >> 16, q = (p & 0x7fffu) - wlo1;
          if (q < 8192u) {
            const uint32_t j = q + ((p >> 15) << 13);
            if (fuse) atomicAdd(&cc1[j >> 1], 1u << ((j & 1u) << 4));
            return T1[j];
          }
          if ((p & 0x7fffu) >= whi1) {
            ndead += fuse ? 1u : 0u;
            return 0.f;
          }
          ntiny += fuse ? 1u : 0u;
        }
        return V2 ? exp_sub_outline(v1f(v), m1) : expf_glibc(__fsub_rn(v1f(v), m1));
      };
      bool rec_ok = false;
      EcssResult e{0.f, 0, -1, 0.f};
      if (V2 && bf) e = row_rec_sum<false>(a, b, row, e1f, 0.f, s, rec_ok);
      // (the chunked method below reads the same summands; its counts are
      // not used)
      if (!rec_ok) {
        clear_hist(s.H0, 2048);
        __syncthreads();
        e = row_ecss(
            row,
            [&](uint32_t i, float v) {
              float x = e1f(i, v);
              if (!bf && x > 0.f) atomicAdd(&s.H0[tkey(v) >> 21], 1u);
              return x;
            },
            kEcssSum, 0.f, s);
      }
      __syncthreads();
      tr.passes++;
      S1 = e.c;
      tr.topp_sum = S1;
      LUMEN_TICK("rs_S1", b);
      uint32_t ncount = V;  // elements the value counts hold
      if (bf && !count_now) {
        bool fused = false;
        if (fuse && rec_ok) {
          ndead = block_sum_u32(ndead, s);
          fused = block_sum_u32(ntiny, s) == 0u;
        }
        if (fused) {
          // the table-entry counts, moved to the layout of the value walk
          uint32_t w8[8];
#pragma unroll
          for (uint32_t k = 0; k < 8u; ++k) w8[k] = cc1[8u * t + k];
          __syncthreads();
          bv_clear(s);
          __syncthreads();
          uint32_t* cw = bv_counts(s);
#pragma unroll
          for (uint32_t k = 0; k < 16u; ++k) {
            const uint32_t c = (w8[k >> 1] >> ((k & 1u) << 4)) & 0xffffu;
            if (c) {
              const uint32_t j = 16u * t + k;
              const uint32_t pat = ((j >> 13) << 15) | (wlo1 + (j & 8191u));
              const uint32_t pk = (pat ^ ((uint32_t)((int32_t)(pat << 16) >> 31) | 0x8000u)) & 0xffffu;
              atomicAdd(&cw[pk >> 1], c << ((pk & 1u) << 4));
            }
          }
          __syncthreads();
          ncount = V - ndead;
        } else {
          bv_clear(s);
          __syncthreads();
          row_foreach(row, [&](uint32_t, float v) { bv_count(v1f(v), s); });
          __syncthreads();
          tr.passes++;
        }
        LUMEN_TICK("rs_count", b);
      }
      float c = 0.f;
      bool found = false;
      // bf16 rows: the walk over distinct values
      const int byval = !bf ? -1
                            : topp_by_value<V2>(row, kmask, kcut, m1, S1, P.top_p, s, tr, pk_lo, pk_hi,
                                            istar, ncount);
      LUMEN_TICK("rs_byval", b);
      if (bf && byval < 0) {
        // the window path's key histogram, skipped above
        clear_hist(s.H0, 2048);
        __syncthreads();
        row_foreach(row, [&](uint32_t i, float v) {
          if (expf_glibc(__fsub_rn(v1f(v), m1)) > 0.f) atomicAdd(&s.H0[tkey(v) >> 21], 1u);
        });
        __syncthreads();
        tr.passes++;
      }
      if (byval >= 0) {
        tr.windows = 1;
        c = tr.topp_cum;
        found = byval == 1;
        if (found) pmode = 3;
      }
      // otherwise walk the probability order window by window
      uint64_t key_hi = 1ull << 32;
      float p_hi = __uint_as_float(0x7f800000u);
      uint32_t ranks = 0;
      for (; byval < 0;) {
        // plan the next window [L, key_hi) of at most kCapWindow keys
        uint32_t L = 0;
        bool empty = false, overflow = false;
        uint32_t gkey = 0;  // overflow: the one key that holds more than a window
        {
          uint32_t pre = 0, pm = 0;
          bool decided = false;
          for (int lvl = 0; lvl < 3 && !decided; ++lvl) {
            const int sh = lvl == 0 ? 21 : (lvl == 1 ? 10 : 0);
            const int nb = lvl == 2 ? 1024 : 2048;
            const uint32_t dm = (uint32_t)nb - 1u;
            uint32_t* H = s.H;
            if (lvl == 0 && (key_hi & 0x1fffffull) == 0) {
              // level-0 counts of the remaining keys come from the saved histogram
              const uint32_t top = (uint32_t)(key_hi >> 21);
              for (int i = t; i < 2048; i += kThreads) s.H[i] = (uint32_t)i < top ? s.H0[i] : 0u;
              __syncthreads();
            } else {
              clear_hist(H, nb);
              __syncthreads();
              const float lo_cut = __fsub_rn(m1, 104.f);
              row_foreach(row, [&](uint32_t i, float v) {
                float x = v1f(v);
                uint32_t kk = tkey(x);
                if ((uint64_t)kk < key_hi && (kk & pm) == pre && x >= lo_cut)
                  atomicAdd(&H[(kk >> sh) & dm], 1u);
              });
              __syncthreads();
              tr.passes++;
            }
            uint32_t ab = 0;
            int d = find_from_top(H, nb, (uint32_t)kCapWindow + 1u, &ab, s);
            if (d < 0) {
              // everything that remains under this prefix fits
              if (ab == 0 && lvl == 0) empty = true;
              L = pre;
              decided = true;
            } else if (ab > 0) {
              L = pre | (((uint32_t)d + 1u) << sh);
              decided = true;
            } else {
              pre |= (uint32_t)d << sh;
              pm |= dm << sh;
            }
            __syncthreads();
          }
          if (!decided) {
            overflow = true;  // more than a window of one exact key
            gkey = pre;
          }
        }
        if (empty) break;
        if ((!overflow && (uint64_t)L >= key_hi) || tr.windows >= 4096u) {
          tr.status = kStatusTieOverflow;  // no progress: never loop
          break;
        }
        bool as_group = overflow;
        float p_lo = 0.f;
        uint32_t n = 0;
        if (!as_group) {
          // probability window [p_lo, p_hi)
          const float vH = key_hi >= (1ull << 32) ? __uint_as_float(0x7f800000u) : key2f((uint32_t)key_hi);
          const float dh = __fadd_rn(__fmul_rn(fabsf(vH) + fabsf(m1), 0x1p-12f), 0x1p-20f);
          const float hi_v = __fadd_rn(vH, dh);
          for (;;) {
            const float vL = key2f(L);
            p_lo = (L == 0u) ? 0.f : __fdiv_rn(expf_glibc(__fsub_rn(vL, m1)), S1);
            const float dl = __fadd_rn(__fmul_rn(fabsf(vL) + fabsf(m1), 0x1p-12f), 0x1p-20f);
            const float lo_v = (L == 0u) ? kNegInf : __fsub_rn(vL, dl);
            if (t == 0) s.cnt = 0;
            __syncthreads();
            row_foreach(row, [&](uint32_t i, float v) {
              float x = v1f(v);
              bool in = false;
              uint32_t pb = 0;
              if (x >= lo_v && x <= hi_v) {
                float p = __fdiv_rn(expf_glibc(__fsub_rn(x, m1)), S1);
                in = p > 0.f && p >= p_lo && p < p_hi;
                pb = __float_as_uint(p);
              }
              list_push(s.Bk, &s.cnt, in, ((uint64_t)(~pb) << 32) | i);
            });
            __syncthreads();
            tr.passes++;
            n = s.cnt;
            if (n <= (uint32_t)kCap || L == 0u) break;
            // The tokens with p == p_lo reach below the planned edge L (values
            // under vL whose probability rounds to the same p, such as the
            // subnormals around zero): move the edge up to the first key whose
            // p exceeds p_lo, which leaves that whole group to the next window.
            if (t == 0) {
              uint64_t lo = (uint64_t)L + 1u, hi = key_hi;
              while (lo < hi) {
                const uint64_t mid = (lo + hi) >> 1;
                const float pm = __fdiv_rn(expf_glibc(__fsub_rn(key2f((uint32_t)mid), m1)), S1);
                if (pm > p_lo) hi = mid; else lo = mid + 1u;
              }
              s.misc_u[0] = lo < key_hi ? (uint32_t)lo : 0u;
            }
            __syncthreads();
            const uint32_t up = s.misc_u[0];
            __syncthreads();
            if (up == 0u) {
              // every key of the window shares one p: a probability group
              // larger than a window, summed as repeated adds below
              as_group = true;
              gkey = L;
              break;
            }
            L = up;
          }
          if (!as_group && n > (uint32_t)kCap) {
            tr.status = kStatusListOverflow;
            break;
          }
        }
        if (as_group) {
          // The top remaining probability group (one key, or neighbouring
          // keys whose p rounds equal) holds more tokens than a window: the
          // group is one summand repeated (rep_replay), and a crossing inside
          // it keeps the group's lowest ids (sampling.rs:948-960: ties in p
          // are sorted by id).
          const float vK = key2f(gkey);
          const float pg = __fdiv_rn(expf_glibc(__fsub_rn(vK, m1)), S1);
          if (!(pg > 0.f)) break;  // zero probabilities never reach top_p
          const float dK = __fadd_rn(__fmul_rn(fabsf(vK) + fabsf(m1), 0x1p-12f), 0x1p-20f);
          const float glo = __fsub_rn(vK, dK), ghi = __fadd_rn(vK, dK);
          const uint64_t khi = key_hi;
          auto ingroup = [&](uint32_t, float x) {
            return x >= glo && x <= ghi && (uint64_t)tkey(x) < khi &&
                   __fdiv_rn(expf_glibc(__fsub_rn(x, m1)), S1) == pg;
          };
          uint32_t ng = 0, kmin = 0xffffffffu;
          row_foreach(row, [&](uint32_t i, float v) {
            const float x = v1f(v);
            if (ingroup(i, x)) {
              ++ng;
              kmin = min(kmin, tkey(x));
            }
          });
          tr.passes++;
          ng = block_sum_u32(ng, s);
          kmin = ~(uint32_t)block_max_u64((uint64_t)(~kmin), s);
          if (!(pg < p_hi)) {
            // the group was summed with the window above (it gathers by p)
            key_hi = kmin;
            continue;
          }
          if (t < 64u) {
            float y = c, prev = c;
            uint32_t j = 0;
            const bool f = rep_replay(y, prev, pg, ng, P.top_p, true, j);
            if (t == 0) {
              s.red_f[0] = y;
              s.misc_u[0] = f ? 1u : 0u;
              s.misc_u[1] = j;
            }
          }
          __syncthreads();
          const float y = s.red_f[0];
          const bool hitg = s.misc_u[0] != 0u;
          const uint32_t jg = s.misc_u[1];
          __syncthreads();
          tr.windows++;
          if (hitg) {
            found = true;
            pstar = pg;
            istar = kth_id_where(row, [&](uint32_t, float v) { return v1f(v); }, ingroup, jg + 1u, s);
            tr.topp_kept = ranks + jg + 1u;
            tr.topp_cum = y;
            pmode = 2;
            break;
          }
          c = y;
          ranks += ng;
          key_hi = kmin;
          p_hi = pg;
          continue;
                }
        tr.windows++;
        sort_u64_asc(s.Bk, n, s.A, s);
        EcssResult w = list_ecss(
            n, [&](uint32_t j) { return __uint_as_float(~(uint32_t)(s.Bk[j] >> 32)); },
            kEcssFindGe, P.top_p, c, s);
        if (w.found) {
          found = true;
          pstar = __uint_as_float(~(uint32_t)(s.Bk[w.pos] >> 32));
          istar = (uint32_t)s.Bk[w.pos];
          tr.topp_kept = ranks + (uint32_t)w.pos + 1u;
          tr.topp_cum = w.c;
          if (tr.windows == 1) {
            // the whole nucleus is in LDS: continue on the small path
            const uint32_t nk = (uint32_t)w.pos + 1u;
            for (uint32_t j = t; j < nk; j += kThreads) {
              uint32_t idx = (uint32_t)s.Bk[j];
              s.A[j] = ((uint64_t)idx << 32) | tkey(v1f(row.at(idx)));
            }
            __syncthreads();
            sort_u64_asc(s.A, nk, s.Bk, s);
            nlist = nk;
            small = true;
          } else {
            pmode = 2;
          }
          break;
        }
        c = w.c;
        ranks += n;
        if (L == 0u) break;
        key_hi = L;
        p_hi = p_lo;
      }
      if (!found) {
        tr.topp_kept = V;
        tr.topp_cum = c;
      }
      if (tr.status) {
        write_result(a, b, 0xffffffffu, tr);
        return;
      }
    }
  }

  if (small) {
    small_path(a, b, P, nlist, topp_done, rdraw, s, tr);
    return;
  }

  // ---- large path: min-p, temperature, softmax, draw over the whole row ----
  // The masks' state as values: some of it went out by reference, and the
  // per-element passes below must not re-read it from memory.
  const bool c_kmask = kmask;
  const uint32_t c_kcut = kcut, c_plim = plim, c_istar = istar, c_pk_lo = pk_lo, c_pk_hi = pk_hi;
  const int c_pmode = pmode;
  const float c_m1 = m1, c_S1 = S1, c_pstar = pstar;
  auto v2f = [=](uint32_t i, float v) -> float {
    float x = (c_kmask && tkey(v) < c_kcut) ? kNegInf : v;
    if (c_pmode == 1) {
      if (i > c_plim) x = kNegInf;
    } else if (c_pmode == 2) {
      float p = __fdiv_rn(expf_glibc(__fsub_rn(x, c_m1)), c_S1);
      if (!(p > c_pstar || (p == c_pstar && i <= c_istar))) x = kNegInf;
    } else if (c_pmode == 3) {
      const uint32_t pk = tkey(x) >> 16;
      if (!(pk > c_pk_hi || (pk >= c_pk_lo && i <= c_istar))) x = kNegInf;
    }
    return x;
  };
  bool mmask = false;
  float bound = 0.f;
  if (P.flags & kMinP) {
    float m = kNegInf;
    row_foreach(row, [&](uint32_t i, float v) { m = rmax(m, v2f(i, v)); });
    m = block_rmax(m, s);
    tr.passes++;
    LUMEN_TICK("rs_minp_max", b);
    if (is_finite(m)) {
      mmask = true;
      bound = __fadd_rn(m, P.log_min_p);
    }
  }
  const float c_bound = bound, c_inv_temp = P.inv_temp;
  const bool c_mmask = mmask;
  auto wf = [=](uint32_t i, float v) -> float {
    float x = v2f(i, v);
    if (c_mmask && x < c_bound) x = kNegInf;
    return __fmul_rn(x, c_inv_temp);
  };
  float m3 = kNegInf;
  uint32_t nan3 = 0;
  if (pmode == 3 && !mmask && !(P.flags & kMinP) && P.inv_temp == 1.0f &&
      (tkey(m1) >> 16) > pk_hi) {
    // The value walk ran on a NaN-free row with a finite maximum m1, and every
    // element whose value pattern lies above the boundary group is kept: the
    // kept set holds m1, and x * 1.0f == x, so its maximum is m1.
    m3 = m1;
  } else {
    row_foreach(row, [&](uint32_t i, float v) {
      float w = wf(i, v);
      m3 = rmax(m3, w);
      nan3 |= is_nan(w) ? 1u : 0u;
    });
    m3 = block_rmax(m3, s);
    nan3 = block_or_u32(nan3, s);
    tr.passes++;
  }
  LUMEN_TICK("rs_m3", b);
  tr.final_max = m3;
  uint32_t tok;
  if (!is_finite(m3)) {
    tr.path |= 16u;
    float u = __fdiv_rn(1.0f, __uint2float_rn(V));
    EcssResult e = const_ecss(V, u, kEcssFindGt, rdraw, s);
    tr.cdf_before = e.found ? e.before : e.c;
    tr.cdf_at = e.c;
    tok = e.found ? (uint32_t)e.pos : V - 1;
  } else if (nan3) {
    tr.path |= 32u;
    tr.final_sum = __uint_as_float(0x7fc00000u);
    tr.cdf_before = tr.cdf_at = __uint_as_float(0x7fc00000u);
    tok = V - 1;
  } else {
    // bf16 rows of lumen_sample_rows_single: a summand is a function of
    // the element's bit pattern and of whether its index lies past the
    // masks' index split (pmode 1: plim, 2 and 3: istar), so the sums read
    // it from two LDS tables (lists A and B: index <= split, index > split)
    // over a window of 64 binades of |value| per sign. Live summands have
    // |w| <= W = max(|m3|, |m3 - 128|) (below m3 - 128, exp gives 0), so
    // every pattern above the window (|v| >= 2^(emax - 126) > 2 W / inv_temp)
    // is zero; patterns below it (|v| < 2^(emax - 190)) take the direct
    // computation.
    const bool ftab = V2 && row.h != nullptr;
    float* const TA = reinterpret_cast<float*>(s.A);
    float* const TB = reinterpret_cast<float*>(s.Bk);
    static_assert(sizeof(s.A) == 16384 * sizeof(float) && sizeof(s.Bk) == sizeof(s.A),
                  "two tables of 2 x 64 x 128 entries");
    uint32_t wlo = 0, whi = 0;
    const uint32_t isplit = c_pmode == 1 ? c_plim : (c_pmode >= 2 ? c_istar : 0xffffffffu);
    if (ftab) {
      const float W = fmaxf(fabsf(m3), fabsf(__fsub_rn(m3, 128.f)));
      const float vm = __fdiv_rn(W, c_inv_temp);
      uint32_t emax = ((__float_as_uint(vm) >> 23) & 0xffu) + 1u;
      emax = emax > 254u ? 254u : (emax < 63u ? 63u : emax);
      wlo = (emax - 63u) << 7;
      whi = (emax + 1u) << 7;
      // value counts still in lists A and B (the by-value walk ran on exact
      // counts): patterns the row does not hold get no exp
      const bool counted = c_pmode == 3;
      uint32_t present = 0xffffu;
      if (counted) {
        const uint32_t* cw = bv_counts(s);
        present = 0u;
#pragma unroll
        for (uint32_t k = 0; k < 16u; ++k) {
          const uint32_t j = threadIdx.x + k * kThreads;
          const uint32_t pat = ((j >> 13) << 15) | (wlo + (j & 8191u));
          if (vcount(cw, tkey(__uint_as_float(pat << 16)) >> 16) != 0u) present |= 1u << k;
        }
        __syncthreads();
      }
#pragma unroll 1
      for (uint32_t k = 0; k < 16u; ++k) {
        const uint32_t j = threadIdx.x + k * kThreads;
        float ea = 0.f, eb = 0.f;
        if ((present >> k) & 1u) {
          const float v = __uint_as_float((((j >> 13) << 15) | (wlo + (j & 8191u))) << 16);
          float x = (c_kmask && tkey(v) < c_kcut) ? kNegInf : v;
          bool ka = true, kb = true;  // kept at an index <= / > the split
          if (c_pmode == 1) {
            kb = false;
          } else if (c_pmode == 2) {
            const float pp = __fdiv_rn(expf_glibc(__fsub_rn(x, c_m1)), c_S1);
            ka = pp >= c_pstar;
            kb = pp > c_pstar;
          } else if (c_pmode == 3) {
            const uint32_t pk = tkey(x) >> 16;
            ka = pk >= c_pk_lo;
            kb = pk > c_pk_hi;
          }
          if (c_mmask && x < c_bound) x = kNegInf;
          const float w = __fmul_rn(x, c_inv_temp);
          const float e = w == kNegInf ? 0.f : expf_glibc(__fsub_rn(w, m3));
          ea = ka ? e : 0.f;
          eb = kb ? e : 0.f;
        }
        TA[j] = ea;
        TB[j] = eb;
      }
      __syncthreads();
    }
    auto e3f = [&](uint32_t i, float v) -> float {
      if (ftab) {
        const uint32_t p = __float_as_uint(v) >> 16, q = (p & 0x7fffu) - wlo;
        if (q < 8192u) return (i <= isplit ? TA : TB)[q + ((p >> 15) << 13)];
        if ((p & 0x7fffu) >= whi) return 0.f;
      }
      const float w = wf(i, v);
      return w == kNegInf ? 0.f : V2 ? exp_sub_outline(w, m3) : expf_glibc(__fsub_rn(w, m3));
    };
    bool rec_ok = false;
    EcssResult S{0.f, 0, -1, 0.f};
    if (V2) S = row_rec_sum<false>(a, b, row, e3f, 0.f, s, rec_ok);
    if (!rec_ok) S = row_ecss(row, e3f, kEcssSum, 0.f, s);
    tr.passes++;
    LUMEN_TICK("rs_S3", b);
    const float S3 = S.c;
    tr.final_sum = S3;
    if (ftab) {
      // each thread divides the entries it wrote
#pragma unroll 1
      for (uint32_t k = 0; k < 16u; ++k) {
        const uint32_t j = threadIdx.x + k * kThreads;
        TA[j] = __fdiv_rn(TA[j], S3);
        TB[j] = __fdiv_rn(TB[j], S3);
      }
      __syncthreads();
    }
    auto p3f = [&](uint32_t i, float v) -> float {
      if (ftab) {
        const uint32_t p = __float_as_uint(v) >> 16, q = (p & 0x7fffu) - wlo;
        if (q < 8192u) return (i <= isplit ? TA : TB)[q + ((p >> 15) << 13)];
        if ((p & 0x7fffu) >= whi) return 0.f;
      }
      const float w = wf(i, v);
      return __fdiv_rn(w == kNegInf ? 0.f : V2 ? exp_sub_outline(w, m3) : expf_glibc(__fsub_rn(w, m3)), S3);
    };
    EcssResult e{0.f, 0, -1, 0.f};
    rec_ok = false;
    if (V2) e = row_rec_sum<true>(a, b, row, p3f, rdraw, s, rec_ok);
    if (!rec_ok) e = row_ecss(row, p3f, kEcssFindGt, rdraw, s);
    tr.passes++;
    LUMEN_TICK("rs_cdf", b);
    tr.cdf_before = e.found ? e.before : e.c;
    tr.cdf_at = e.c;
    tok = e.found ? (uint32_t)e.pos : V - 1;
  }
  write_result(a, b, tok, tr);
}

// The split kernel's fallback: out of line, so that its registers do not
// weigh on the split paths. lumen_sample_rows_single inlines the body.
template <bool V2>
__device__ __attribute__((noinline)) void row_single(const KernelArgs& a, int b, Smem& s) {
  row_single_body<V2>(a, b, s);
}


// ------------------------------------------------------------ row groups
//
// With G > 1 workgroups per row, workgroup `sl` owns the slice
// [sl*per, (sl+1)*per) of its row (per a multiple of 16). The row's workgroups
// coordinate through a RowWs block in device memory:
//  * greedy and top-k rows use a last-arriver pattern (no waiting);
//  * top-p rows use one row barrier and a chain in which slice sl waits for
//    the exact running sum of slice sl-1. Every wait is bounded; on timeout
//    the row reports a failure instead of waiting further.
// The launch is an ordinary one (cooperative only with LUMEN_SAMPLER_COOP):
// the host sizes the grid to the resident capacity (one workgroup per CU),
// so a row's workgroups are co-resident unless other streams' kernels hold
// CUs. Then a waiting workgroup gives up after KernelArgs::wait_ticks of the
// 100 MHz wall clock (lumen_sampler_set_wait_limit; 2 ms by default), counts
// the timeout in *KernelArgs::timeouts, and its row takes the exact
// single-workgroup path: correct, slower, and visible to the caller.

constexpr uint32_t kSampleN = 4096;
// bar value of a top-p row whose finisher stopped waiting for the S1 walker
constexpr uint32_t kAbandoned = 1u << 24;

struct Slice {
  uint32_t lo, hi;
};

__device__ __forceinline__ uint32_t sc_len_max(uint32_t V, uint32_t G) {
  return ((V + G - 1u) / G + 15u) & ~15u;
}

__device__ __forceinline__ Slice slice_bounds(uint32_t V, uint32_t G, uint32_t sl) {
  uint32_t per = ((V + G - 1u) / G + 15u) & ~15u;
  uint32_t lo = min(V, sl * per), hi = min(V, lo + per);
  return Slice{lo, hi};
}

// Makes this workgroup's global writes visible at device scope and arrives on
// *ctr; returns the previous count (uniform across the workgroup). The
// arrival is a release only: an acquire at device scope invalidates the
// whole L2 of this XCD (every workgroup there loses its cached lines), so it
// is paid only by the workgroup that arrives last (old == last), which goes
// on to read what the others wrote.
__device__ __forceinline__ uint32_t wg_arrive(uint32_t* ctr, uint32_t last, Smem& s) {
  // every wave's stores have reached L2 once it passes the barrier; one
  // device-scope release by thread 0 then covers the workgroup
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    if (old == last) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      s.finisher = 1u;
    }
    s.misc_u[2] = old;
  }
  __syncthreads();
  const uint32_t old = s.misc_u[2];
  __syncthreads();
  return old;
}

// Waits until *ctr >= target, then acquires. Returns false when a.wait_ticks
// of the 100 MHz wall clock (s_memrealtime) pass first, or at once when
// wait_ticks is 0 (a host-forced give-up), and then counts the timeout in
// *a.timeouts. The counter is polled with relaxed loads (they read past this
// XCD's L2 without invalidating it); the one acquire comes after the wait.
__device__ __forceinline__ bool wg_wait_geq(const KernelArgs& a, uint32_t* ctr, uint32_t target,
                                            Smem& s) {
  if (threadIdx.x == 0) {
    uint32_t ok = 0;
    const uint64_t limit = a.wait_ticks;
    if (limit) {
      const uint64_t t0 = wall_clock64();
      for (;;) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) {
          ok = 1;
          break;
        }
        if (wall_clock64() - t0 > limit) break;
        __builtin_amdgcn_s_sleep(1);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (!ok && a.timeouts) __hip_atomic_fetch_add(a.timeouts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s.misc_u[3] = ok;
  }
  __syncthreads();
  const bool ok = s.misc_u[3] != 0;
  __syncthreads();
  return ok;
}

// Appends this workgroup's candidates, gathered in s.A[0..s.cnt) by
// list_push, to the row's global buffer with a single atomic. The count is
// always added in full, so an overflow (of LDS or of the buffer) shows up as
// a total above the capacity.
__device__ __forceinline__ void flush_candidates(uint64_t* cand, uint32_t* gcnt, Smem& s,
                                                 uint32_t cap = (uint32_t)kCandCap) {
  __syncthreads();
  const uint32_t n = s.cnt;
  if (threadIdx.x == 0)
    s.misc_u[1] = n ? __hip_atomic_fetch_add(gcnt, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
  __syncthreads();
  const uint32_t base = s.misc_u[1];
  const uint32_t m = min(n, (uint32_t)kCap);
  for (uint32_t j = threadIdx.x; j < m; j += kThreads)
    if (base + j < cap) cand[base + j] = s.A[j];
  __syncthreads();
}

// Key threshold such that about `target` keys of the row are >= it,
// estimated from a fixed strided sample, so every workgroup of the row
// computes the same value. 0 selects everything.
__device__ __forceinline__ uint32_t sample_threshold(const Row& row, uint32_t V, uint32_t target, Smem& s) {
  if (V <= kSampleN || target >= V) return 0u;
  const uint32_t r = (uint32_t)(((uint64_t)target * kSampleN + V - 1) / V);
  if (r == 0u || r > kSampleN) return 0u;
  // kSampleN / 32 aligned runs of 32 consecutive logits (one 128-byte line
  // each) spread over the row: the same sample size as single elements,
  // with 32 times fewer lines read
  uint32_t* keys = reinterpret_cast<uint32_t*>(s.A);
  constexpr uint32_t kRuns = kSampleN / 32u;
  for (uint32_t j = threadIdx.x; j < kSampleN; j += kThreads) {
    const uint32_t c = j >> 5;
    const uint32_t base = (uint32_t)(((uint64_t)c * (V - 32u)) / (kRuns - 1u)) & ~31u;
    keys[j] = tkey(row.at(base + (j & 31u)));
  }
  __syncthreads();
  const uint32_t tau = select_desc(kSampleN, [&](uint32_t j) { return keys[j]; }, r - 1u, s);
  __syncthreads();
  return tau;
}

// LDS bitmap of the history ids that fall in [lo, hi) (bit i - lo), kept in
// the Bk area, which is free during slice passes.
__device__ __forceinline__ uint32_t* slice_bitmap(const KernelArgs& a, int b, Slice sc, Smem& s) {
  uint32_t* bm = reinterpret_cast<uint32_t*>(s.Bk);
  const uint32_t nw = (sc.hi - sc.lo + 31u) / 32u;
  for (uint32_t i = threadIdx.x; i < nw; i += kThreads) bm[i] = 0u;
  __syncthreads();
  const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
  for (uint32_t j = h0 + threadIdx.x; j < h1; j += kThreads) {
    uint32_t id = a.hist_ids[j];
    if (id >= sc.lo && id < sc.hi) atomicOr(&bm[(id - sc.lo) >> 5], 1u << ((id - sc.lo) & 31u));
  }
  __syncthreads();
  return bm;
}

__device__ __forceinline__ bool bm_test(const uint32_t* bm, uint32_t off) {
  return (bm[off >> 5] >> (off & 31u)) & 1u;
}

// Debug copy of the penalized logits of the slice.
__device__ __forceinline__ void slice_pen_out(const KernelArgs& a, int b, const Row& row, Slice sc,
                              const RowParams& P, bool pen) {
  float* po = a.pen_out + (uint64_t)b * a.vocab;
  range_foreach(row, sc.lo, sc.hi, [&](uint32_t i, float v) { po[i] = v; });
  __threadfence();
  __syncthreads();
  if (pen) {
    const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
    for (uint32_t j = h0 + threadIdx.x; j < h1; j += kThreads) {
      uint32_t id = a.hist_ids[j];
      if (id >= sc.lo && id < sc.hi) po[id] = penalize(row.at(id), a.hist_cnt[j], P);
    }
  }
}

// Per-row values every path needs, derived from the arguments inside each
// path function (so the kernel entry passes only scalars to it).
#define ROW_CONTEXT(a, b)                                                             \
  const RowParams P = (a).inline_rows ? (a).inline_params[b] : (a).params[b];         \
  const float rdraw = row_draw((a), (b));                                             \
  RowWs& ws = (a).ws[b];                                                              \
  uint64_t* cand = (a).cand + (uint64_t)(b) * kCandStride;                            \
  const Row row = make_row((a), (b));                                                 \
  (void)rdraw;                                                                        \
  (void)cand

// Greedy with the anti-restate guard, split over G workgroups: the argmax as
// in greedy_split, and each slice's 8 largest finite penalized keys; the
// finisher merges them.
__device__ __forceinline__ void greedy_guard_split(const KernelArgs& a, int b, uint32_t sl,
                                                   uint32_t G, Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t V = a.vocab;
  const Slice sc = slice_bounds(V, G, sl);
  const bool pen = (P.flags & kPen) && hist_hi(a, b) > a.hist_off[b];
  if (a.pen_out) slice_pen_out(a, b, row, sc, P, pen);
  const uint32_t* bm = pen ? slice_bitmap(a, b, sc, s) : nullptr;
  uint64_t best = 0;
  Top8 x;
  top8_init(x);
  range_foreach(row, sc.lo, sc.hi, [&](uint32_t i, float v) {
    if (pen && bm_test(bm, i - sc.lo)) return;
    const uint64_t k = ((uint64_t)tkey(v) << 32) | (uint64_t)(0xffffffffu - i);
    best = k > best ? k : best;
    if (is_finite(v)) top8_push(x, k);
  });
  if (pen) {
    const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
    for (uint32_t j = h0 + threadIdx.x; j < h1; j += kThreads) {
      const uint32_t id = a.hist_ids[j];
      if (id >= sc.lo && id < sc.hi) {
        const float pv = penalize(row.at(id), a.hist_cnt[j], P);
        const uint64_t k = ((uint64_t)tkey(pv) << 32) | (uint64_t)(0xffffffffu - id);
        best = k > best ? k : best;
        if (is_finite(pv)) top8_push(x, k);
      }
    }
  }
  best = block_max_u64(best, s);
  const uint64_t* top = block_top8(x, s);
  if (threadIdx.x == 0) {
    ws.part_arg[sl] = best;
#pragma unroll
    for (int r = 0; r < 8; ++r) ws.part_top[sl][r] = top[r];
  }
  const uint32_t old = wg_arrive(&ws.arrive, G - 1u, s);
  if (old != G - 1u) return;
  if (threadIdx.x < 64u) {
    const uint32_t lane = threadIdx.x;
    uint64_t m = 0;
    for (uint32_t i = 0; i < G; ++i) {
      const uint64_t u = __hip_atomic_load(&ws.part_arg[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      m = u > m ? u : m;
    }
    Top8 y;
    top8_init(y);
    uint64_t* pt = &ws.part_top[0][0];
#pragma unroll
    for (uint32_t q = 0; q < 2u; ++q)
      if (2u * lane + q < G * 8u)
        top8_push(y, __hip_atomic_load(&pt[2u * lane + q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    uint64_t out[8];
    wave_top8(y, out);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < 8; ++r) s.Bk[r] = out[r];
      s.Bk[8] = m;
    }
  }
  __syncthreads();
  const uint64_t m = s.Bk[8];
  write_guard(a, b, 0xffffffffu - (uint32_t)m, s.Bk);
  RowTrace tr;
  init_trace(tr, V);
  tr.path = 1u;
  tr.passes = 1;
  write_result(a, b, 0xffffffffu - (uint32_t)m, tr);
}

// Greedy: per-slice argmax, the last workgroup to arrive combines.
__device__ __forceinline__ void greedy_split(const KernelArgs& a, int b, uint32_t sl, uint32_t G,
                                                      Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t V = a.vocab;
  const Slice sc = slice_bounds(V, G, sl);
  const bool pen = (P.flags & kPen) && hist_hi(a, b) > a.hist_off[b];
  if (a.pen_out) slice_pen_out(a, b, row, sc, P, pen);
  const uint32_t* bm = pen ? slice_bitmap(a, b, sc, s) : nullptr;
  uint64_t best = 0;
  range_foreach(row, sc.lo, sc.hi, [&](uint32_t i, float v) {
    if (pen && bm_test(bm, i - sc.lo)) return;
    uint64_t k = ((uint64_t)tkey(v) << 32) | (uint64_t)(0xffffffffu - i);
    best = k > best ? k : best;
  });
  if (pen) {
    const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
    for (uint32_t j = h0 + threadIdx.x; j < h1; j += kThreads) {
      uint32_t id = a.hist_ids[j];
      if (id >= sc.lo && id < sc.hi) {
        uint64_t k = ((uint64_t)tkey(penalize(row.at(id), a.hist_cnt[j], P)) << 32) |
                     (uint64_t)(0xffffffffu - id);
        best = k > best ? k : best;
      }
    }
  }
  best = block_max_u64(best, s);
  if (threadIdx.x == 0) ws.part_arg[sl] = best;
  const uint32_t old = wg_arrive(&ws.arrive, G - 1u, s);
  if (old != G - 1u) return;
  uint64_t m = 0;
  for (uint32_t i = 0; i < G; ++i) {
    uint64_t u = __hip_atomic_load(&ws.part_arg[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    m = u > m ? u : m;
  }
  RowTrace tr;
  init_trace(tr, V);
  tr.path = 1u;
  tr.passes = 1;
  write_result(a, b, 0xffffffffu - (uint32_t)m, tr);
}

// Candidates of a short top-k slice (at most 16 elements per thread) without
// sampling: with the slice in registers, every thread's largest
// non-history key is found, and two radix levels over those kThreads keys
// give a lower bound tau of their k-th largest (k <= kThreads). At least k
// elements of the slice have keys >= tau, so tau is at most the slice's
// k-th largest key, which is at most the row's: every key of the row's top
// k is >= tau. Non-history elements with keys >= tau are appended to list A
// (history ids are handled by the caller with their penalized values). Key
// 0 stands for "not a candidate".
__device__ __forceinline__ uint32_t topk_collect16(const Row& row, Slice sc, const uint32_t* bm,
                                                   uint32_t k, Smem& s) {
  const uint32_t t = threadIdx.x;
  uint32_t kk[4][4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t i = sc.lo + ((uint32_t)q * kThreads + t) * 4u;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (i < sc.hi) row.load4(i, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) kk[q][j] = i + (uint32_t)j < sc.hi ? tkey(v[j]) : 0u;
  }
  uint32_t tm = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = sc.lo + ((uint32_t)q * kThreads + t) * 4u + (uint32_t)j;
      if (bm && kk[q][j] != 0u && bm_test(bm, i - sc.lo)) kk[q][j] = 0u;
      tm = max(tm, kk[q][j]);
    }
  uint32_t* tk = reinterpret_cast<uint32_t*>(s.A);
  tk[t] = tm;
  __syncthreads();
  const uint32_t tau = select_desc((uint32_t)kThreads, [&](uint32_t j) { return tk[j]; }, k - 1u, s, 2);
  if (t == 0) s.cnt = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = sc.lo + ((uint32_t)q * kThreads + t) * 4u + (uint32_t)j;
      list_push(s.A, &s.cnt, kk[q][j] != 0u && kk[q][j] >= tau, ((uint64_t)(~kk[q][j]) << 32) | i);
    }
  return tau;
}

// Top-k: a sampled threshold, one compaction pass per slice into the row's
// candidate buffer, and the last workgroup finishes on the LDS list. If the
// sample missed (fewer than k or more than the buffer holds), the finisher
// runs the exact single-workgroup path.
__device__ __forceinline__ void topk_split(const KernelArgs& a, int b, uint32_t sl, uint32_t G,
                                                    Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t V = a.vocab;
  const uint32_t k = P.top_k;
  const Slice sc = slice_bounds(V, G, sl);
  const bool pen = (P.flags & kPen) && hist_hi(a, b) > a.hist_off[b];
  if (a.pen_out) slice_pen_out(a, b, row, sc, P, pen);
  LUMEN_TICK("topk_start", b);
  uint32_t tau;
  const uint32_t* bm;
  if (k <= (uint32_t)kThreads && sc_len_max(V, G) <= 16u * kThreads) {
    // short slices: the bound comes from the slice's own values
    bm = pen ? slice_bitmap(a, b, sc, s) : nullptr;
    tau = topk_collect16(row, sc, bm, k, s);
    LUMEN_TICK("topk_sampled", b);
  } else {
    // k up to 2048: 3k + 256 candidates; larger k use the whole row stride
    // of the candidate buffer, aiming at 2.5k + 256
    const uint32_t target = k <= 2048u ? min(3u * k + 256u, (uint32_t)(kCandCap * 3 / 4))
                                       : min(5u * k / 2u + 256u, (uint32_t)kTopKCandCap * 3u / 4u);
    tau = sample_threshold(row, V, target, s);
    LUMEN_TICK("topk_sampled", b);
    bm = pen ? slice_bitmap(a, b, sc, s) : nullptr;
    if (threadIdx.x == 0) s.cnt = 0;
    __syncthreads();
    range_foreach(row, sc.lo, sc.hi, [&](uint32_t i, float v) {
      const uint32_t kk = tkey(v);
      const bool in = kk >= tau && !(pen && bm_test(bm, i - sc.lo));
      list_push(s.A, &s.cnt, in, ((uint64_t)(~kk) << 32) | i);
    });
  }
  if (pen) {
    const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
    for (uint32_t base = h0; base < h1; base += kThreads) {
      const uint32_t j = base + threadIdx.x;
      bool in = false;
      uint32_t kk = 0, id = 0;
      if (j < h1) {
        id = a.hist_ids[j];
        if (id >= sc.lo && id < sc.hi) {
          kk = tkey(penalize(row.at(id), a.hist_cnt[j], P));
          in = kk >= tau;
        }
      }
      list_push(s.A, &s.cnt, in, ((uint64_t)(~kk) << 32) | id);
    }
  }
  flush_candidates(cand, &ws.cand_n, s, kTopKCandCap);
  LUMEN_TICK("topk_compacted", b);
  const uint32_t old = wg_arrive(&ws.arrive, G - 1u, s);
  if (old != G - 1u) return;
  LUMEN_TICK("topk_finisher", b);
  const uint32_t n = __hip_atomic_load(&ws.cand_n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (n < k || n > kTopKCandCap) {
    row_single<false>(a, b, s);
    return;
  }
  RowTrace tr;
  init_trace(tr, V);
  tr.passes = 1;
  // up to kTopKCandCap entries: list A continues into list B (adjacent)
  uint64_t* const CL = s.A;
  for (uint32_t j = threadIdx.x; j < n; j += kThreads) CL[j] = cand[j];
  __syncthreads();
  LUMEN_TICK("topk_loaded", b);
  // candidate entries are (~key << 32) | idx
  auto ckey = [&](uint32_t j) { return ~(uint32_t)(CL[j] >> 32); };
  uint32_t cut, ns;
  if (k == 1) {
    // sampling.rs:913-921: exactly the lowest-index maximum
    uint64_t best = 0;
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
      const uint64_t e = CL[j];
      const uint64_t kk = ((uint64_t)(~(uint32_t)(e >> 32)) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
      best = kk > best ? kk : best;
    }
    best = block_max_u64(best, s);
    cut = (uint32_t)(best >> 32);
    if (threadIdx.x == 0) s.A[0] = ((uint64_t)(0xffffffffu - (uint32_t)best) << 32) | cut;
    ns = 1;
    __syncthreads();
  } else {
    cut = select_desc(n, ckey, k - 1u, s);
    // survivors (every key >= cut, ties included) as (idx << 32) | key,
    // compacted in place: a chunk's entries are all read before any write,
    // and a survivor never moves past its own position
    if (threadIdx.x == 0) s.cnt = 0;
    __syncthreads();
    for (uint32_t base = 0; base < n; base += kThreads) {
      const uint32_t j = base + threadIdx.x;
      bool in = false;
      uint64_t e = 0;
      if (j < n) {
        const uint32_t kk = ckey(j);
        in = kk >= cut;
        e = ((uint64_t)(uint32_t)CL[j] << 32) | kk;
      }
      __syncthreads();
      list_push(CL, &s.cnt, in, e);
    }
    __syncthreads();
    ns = s.cnt;
    if (ns > (uint32_t)kCap) {
      // more tied survivors than a list holds
      row_single<false>(a, b, s);
      return;
    }
  }
  LUMEN_TICK("topk_sort1", b);
  sort_u64_asc(s.A, ns, s.Bk, s);  // ascending index
  tr.topk_cutoff_key = cut;
  tr.topk_survivors = ns;
  LUMEN_TICK("topk_sorted", b);
  small_path(a, b, P, ns, false, rdraw, s, tr);
  LUMEN_TICK("topk_done", b);
}

__device__ __forceinline__ double block_excl_scan_f64(double v, Smem& s, double* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const double inc = wave_scan_incl(v, 0.0, [](double l, double r) { return l + r; });
  __shared__ double wt[kWaves];
  if (lane == 63) wt[w] = inc;
  __syncthreads();
  double pre = 0.0, tot = 0.0;
  for (int i = 0; i < kWaves; ++i) {
    if (i < w) pre += wt[i];
    tot += wt[i];
  }
  __syncthreads();
  *total = tot;
  return pre + inc - v;
}

// Lower bound of the binade holding a non-negative value, as f32 bits.
__device__ __forceinline__ uint32_t binade_bits(double x) {
  float f = __double2float_rz(x > 0.0 ? x : 0.0);
  return __float_as_uint(f) & 0xff800000u;
}

// Exact T = 1 softmax sum across the slices of a row, without a chain of
// waits. Each workgroup cuts its slice into sub-chunks of kThreads * M
// elements (thread t owns M consecutive ones), computes the summands and an
// f64 estimate of the running sum at every thread (its slice's estimated
// prefix plus the summands before it), builds the run/boundary structure of
// est_prepare and parks it in device memory. The last workgroup to arrive
// then walks all structures in row order (est_resolve), exactly; a
// sub-chunk whose structure failed a check is recomputed and summed by the
// iterative method instead.

template <int M>
__device__ __forceinline__ void chain_load(const Row& row, Slice sc, uint32_t i0, float m1,
                                           float (&x)[M]) {
#pragma unroll
  for (int q = 0; q < M / 4; ++q) {
    float v[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
    const uint32_t i = i0 + 4u * q;
    if (i < sc.hi) row.load4(i, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[4 * q + j] = expf_glibc(__fsub_rn((i + j < sc.hi) ? v[j] : kNegInf, m1));
  }
}

// ---------------------------------------------------------------- records
// Run records of the exact softmax sum, one per wave segment. In pass 2 a
// sub-chunk of kThreads * M elements gives thread t elements t M .. t M + M
// - 1, so wave w holds a segment of 64 M consecutive elements. Each wave
// parks that segment's record (the parity-map method of ecss.h at wave
// scope, guided by the f64 estimate of the running sum):
//   [0]                    nb (boundary lanes), or kRecNotParked
//   [1 + 3k .. 3 + 3k]     run k (k = 0..nb): binade bits, map a0, map a1
//   [4 + 3nb ..]           the M summands of every boundary lane, in order
// A lane is a boundary when its estimated running sum, widened by `rel`,
// touches two binades; every other lane builds its parity map in its
// binade, and a segmented wave scan composes the runs between boundaries.
// Records with more than kRecMaxB boundary lanes are not parked; the walk
// sums such a segment again on one wave.
constexpr uint32_t kRecMaxB = 32;
constexpr uint32_t kRecNotParked = 0xffffffffu;
constexpr uint32_t kRecSlots = (uint32_t)kMaxSlices * (uint32_t)kChainMaxQ * (uint32_t)kWaves;
static_assert(kRecSlots == (uint32_t)kRowRecs, "record slots per row");
static_assert(4u + 35u * kRecMaxB <= (uint32_t)kRecWords, "record slot too small");

template <int M>
__device__ __forceinline__ uint32_t rec_words(uint32_t nb) {
  return 4u + (3u + (uint32_t)M) * nb;
}

__device__ __forceinline__ uint32_t* rec_slot(const KernelArgs& a, int b, uint32_t slot) {
  return a.est + ((uint64_t)b * kRowRecs + slot) * kRecWords;
}

template <int M>
__device__ __forceinline__ void wave_park(const float (&x)[M], double p_start, double d_self,
                                          double rel, uint32_t nact, uint32_t* rec) {
  const uint32_t lane = threadIdx.x & 63u;
  const bool live = lane < nact;
  const uint32_t blo = est_binade(p_start * (1.0 - rel));
  const uint32_t bhi = est_binade((p_start + d_self) * (1.0 + rel));
  const bool bd = live && blo != bhi;
  const unsigned long long bm = __ballot(bd);
  const uint32_t nb = (uint32_t)__popcll(bm);
  if (nb > kRecMaxB) {
    if (lane == 0) rec[0] = kRecNotParked;
    return;
  }
  PMap own{0u, 0u};
  if (live && !bd) {
    float y0 = __uint_as_float(blo), y1 = __uint_as_float(blo | 1u);
#pragma unroll
    for (int j = 0; j < M; ++j) {
      y0 = __fadd_rn(y0, x[j]);
      y1 = __fadd_rn(y1, x[j]);
    }
    const uint32_t n0 = __float_as_uint(y0) - blo, n1 = __float_as_uint(y1) - (blo | 1u);
    own.a0 = n0 > kSat ? kSat : n0;
    own.a1 = n1 > kSat ? kSat : n1;
  }
  const uint32_t k = (uint32_t)__popcll(bm & ((1ull << lane) - 1ull));
  const SegVal id{0u, PMap{0u, 0u}};
  const SegVal inc = wave_scan_incl(SegVal{bd ? 1u : 0u, own}, id, seg_combine);
  const SegVal prev = wave_shr1(inc, id);
  const uint32_t pbd = wave_shr1(bd ? 1u : 0u, 0u);
  const uint32_t pbin = wave_shr1(blo, 0u);
  if (bd) {
    const bool empty = lane == 0u || pbd != 0u;
    rec[1u + 3u * k] = empty ? kEmptyRun : pbin;
    rec[2u + 3u * k] = empty ? 0u : prev.m.a0;
    rec[3u + 3u * k] = empty ? 0u : prev.m.a1;
    uint32_t* bx = rec + 4u + 3u * nb + k * (uint32_t)M;
#pragma unroll
    for (int j = 0; j < M; ++j) bx[j] = __float_as_uint(x[j]);
  }
  if (lane == nact - 1u) {
    rec[0] = nb;
    rec[1u + 3u * nb] = bd ? kEmptyRun : blo;
    rec[2u + 3u * nb] = bd ? 0u : inc.m.a0;
    rec[3u + 3u * nb] = bd ? 0u : inc.m.a1;
  }
}

// Applies run (sb, a0, a1) to the exact running sum c; false when the sum
// is not in the run's binade or would leave it (the estimate was wrong).
__device__ __forceinline__ bool run_apply(float& c, uint32_t sb, uint32_t a0, uint32_t a1) {
  if (sb == kEmptyRun) return true;
  const uint32_t cb = __float_as_uint(c);
  const uint32_t inc = (cb & 1u) ? a1 : a0;
  const uint32_t nbits = cb + inc;
  if ((cb & 0xff800000u) != sb || inc >= kSat || nbits >= sb + 0x00800000u) return false;
  c = __uint_as_float(nbits);
  return true;
}

template <int M>
__device__ __forceinline__ bool rec_walk(const uint32_t* rec, float& c) {
  const uint32_t nb = rec[0];
  float y = c;
  for (uint32_t k = 0; k <= nb; ++k) {
    if (!run_apply(y, rec[1u + 3u * k], rec[2u + 3u * k], rec[3u + 3u * k])) return false;
    if (k < nb) {
      const uint32_t* bx = rec + 4u + 3u * nb + (uint32_t)M * k;
      float xs[M];
#pragma unroll
      for (int q = 0; q < M; ++q) xs[q] = __uint_as_float(bx[q]);
#pragma unroll
      for (int q = 0; q < M; ++q) y = __fadd_rn(y, xs[q]);
    }
  }
  c = y;
  return true;
}

// Row range of record slot `slot` = (slice, sub-chunk, wave); empty when the
// segment lies beyond its slice.
template <int M>
__device__ __forceinline__ Slice rec_range(uint32_t V, uint32_t G, uint32_t slot) {
  const uint32_t w = slot % (uint32_t)kWaves, sq = slot / (uint32_t)kWaves;
  const Slice si = slice_bounds(V, G, sq / (uint32_t)kChainMaxQ);
  const uint32_t lo = si.lo + (sq % (uint32_t)kChainMaxQ) * (uint32_t)kThreads * M + w * 64u * M;
  return Slice{min(lo, si.hi), min(si.hi, lo + 64u * M)};
}

// Exact sum of one segment from the exact running sum c, by the calling wave.
template <int M>
__device__ __forceinline__ float seg_recompute(const Row& row, Slice r, float m1, float c) {
  const uint32_t i0 = r.lo + (threadIdx.x & 63u) * M;
  float x[M];
#pragma unroll
  for (int q = 0; q < M / 4; ++q) {
    float v[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
    const uint32_t i = i0 + 4u * q;
    if (i < r.hi) row.load4(i, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) x[4 * q + j] = (i + j < r.hi) ? expf_glibc(__fsub_rn(v[j], m1)) : 0.f;
  }
  return wave_ecss<M>(c, x, kEcssSum, 0.f).c;
}

// Pass 2 of a top-p row: the exact summands exp(v - m1) of this slice, per
// sub-chunk, with one record per wave segment. The incoming sum of the
// slice is the f64 estimate p_slice.
template <int M>
__device__ __forceinline__ void chain_prepare(const KernelArgs& a, int b, uint32_t sl,
                                              const Row& row, Slice sc, float m1,
                                              double p_slice, Smem& s) {
  const uint32_t chunk = (uint32_t)kThreads * M;
  const uint32_t nq = (sc.hi - sc.lo + chunk - 1u) / chunk;
  const uint32_t t = threadIdx.x, w = t >> 6;
  double pre = p_slice;
  for (uint32_t q = 0; q < nq; ++q) {
    const uint32_t i0 = sc.lo + q * chunk + t * M;
    float x[M];
    chain_load<M>(row, sc, i0, m1, x);
    double d = 0.0;
#pragma unroll
    for (int j = 0; j < M; ++j) d += (double)x[j];
    double tot;
    const double pt = pre + block_excl_scan_f64(d, s, &tot);
    pre += tot;
    // The exact f32 running sum drifts below its f64 estimate: addends are
    // rounded onto the accumulator's grid, and the small ones are lost. The
    // drift reaches ~5e-4 relative after 250K summands in logit rows, so the
    // boundary margin grows with the position in the row. A wrong guess
    // only costs one wave's recomputation in the walk.
    const double rel = 4e-5 + 3e-9 * (double)(sc.lo + q * chunk);
    const uint32_t nthr = (sc.hi - (sc.lo + q * chunk) + (uint32_t)M - 1u) / (uint32_t)M;
    if (w * 64u < nthr)
      wave_park<M>(x, pt, d, rel, min(64u, nthr - w * 64u),
                   rec_slot(a, b, (sl * (uint32_t)kChainMaxQ + q) * (uint32_t)kWaves + w));
  }
}

// Record gather of the finisher, issued right after its candidate loads so
// that both travel in one round trip: every record's first kSpec words (its
// head and one boundary lane) into the record area (s.Bk as words); records
// with more boundary lanes take a second trip, one wave per record.
// woff[slot] = LDS word offset, kSlotAbsent (no such segment) or
// kSlotMissing (not in LDS, or not parked: summed again by the walk).
constexpr uint32_t kSlotAbsent = 0xfffffffeu;
constexpr uint32_t kSlotMissing = 0xffffffffu;

template <int M>
__device__ __forceinline__ void rec_gather(const KernelArgs& a, int b, uint32_t G, Smem& s) {
  constexpr uint32_t kSpec = (4u + 3u + (uint32_t)M + 3u) & ~3u;  // nb <= 1, whole uint4s
  const uint32_t t = threadIdx.x, V = a.vocab;
  uint32_t* woff = s.H + 1024;
  uint32_t* longs = s.H + 1536;
  uint32_t* words = reinterpret_cast<uint32_t*>(s.Bk);
  constexpr uint32_t kCapWords = 2u * kCap;
  uint4 rq[kSpec / 4];
  uint32_t size = 0;
  bool valid = false;
  if (t < kRecSlots) {
    const Slice r = rec_range<M>(V, G, t);
    valid = t / ((uint32_t)kWaves * (uint32_t)kChainMaxQ) < G && r.lo < r.hi;
    if (valid) {
      const uint4* rec = reinterpret_cast<const uint4*>(rec_slot(a, b, t));
#pragma unroll
      for (int q = 0; q < (int)(kSpec / 4); ++q) rq[q] = rec[q];
    }
  }
  LUMEN_TICK("g_heads_issued", b);
  const bool parked = valid && rq[0].x != kRecNotParked;
  if (parked) size = rec_words<M>(rq[0].x);
  const uint32_t inc = block_incl_scan_u32(size, s);
  LUMEN_TICK("g_heads_in", b);
  const uint32_t off = inc - size;
  const bool fits = parked && inc <= kCapWords;
  if (t < kRecSlots) woff[t] = !valid ? kSlotAbsent : fits ? off : kSlotMissing;
  if (t == 0) s.misc_u[2] = 0;
  if (fits) {
#pragma unroll
    for (int q = 0; q < (int)(kSpec / 4); ++q) {
      const uint32_t o = 4u * (uint32_t)q;
      if (o < size) words[off + o] = rq[q].x;
      if (o + 1u < size) words[off + o + 1u] = rq[q].y;
      if (o + 2u < size) words[off + o + 2u] = rq[q].z;
      if (o + 3u < size) words[off + o + 3u] = rq[q].w;
    }
  }
  __syncthreads();
  if (fits && size > kSpec) longs[atomicAdd(&s.misc_u[2], 1u)] = t | (off << 9);
  __syncthreads();
  const uint32_t nl = s.misc_u[2], lane = t & 63u;
  LUMEN_TICK("g_heads_stored", b);
  for (uint32_t k = t >> 6; k < nl; k += (uint32_t)kWaves) {
    const uint32_t slot = longs[k] & 511u, o = longs[k] >> 9;
    const uint32_t* rec = rec_slot(a, b, slot);
    const uint32_t sz = rec_words<M>(words[o]);
    for (uint32_t q0 = kSpec; q0 < sz; q0 += 256u) {
      uint32_t tv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t q = q0 + 64u * (uint32_t)u + lane;
        if (q < sz) tv[u] = rec[q];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t q = q0 + 64u * (uint32_t)u + lane;
        if (q < sz) words[o + q] = tv[u];
      }
    }
  }
}

// Exact softmax sum of the row from the gathered records, on wave 0. A
// record with a single run is a parity map in a known binade, so 64 such
// records compose with one wave scan (the one-wave method of ecss.h with
// records in place of elements); a record with boundary lanes, a run in
// another binade, a crossing or a missing record stops the scan there and
// is handled on its own. Returns the sum; *nre counts segments summed again.
template <int M>
__device__ __forceinline__ float chain_walk(const KernelArgs& a, int b, uint32_t G, const Row& row,
                                            float m1, uint32_t* nre_out, Smem& s) {
  const uint32_t t = threadIdx.x, V = a.vocab;
  const uint32_t nslots = G * (uint32_t)kChainMaxQ * (uint32_t)kWaves;
  const uint32_t* words = reinterpret_cast<const uint32_t*>(s.Bk);
  const uint32_t* woff = s.H + 1024;
  // Wave 0 walks from slot `from` until the end or a record it cannot use;
  // such a segment is then summed again by the whole workgroup, and the
  // walk resumes after it.
  uint32_t from = 0, nre = 0, nbw = 0;
  float c = 0.f;
  for (;;) {
    if (t < 64u) {
      const uint32_t lane = t;
      uint32_t stop = 0xffffffffu;
      for (uint32_t s0 = from; s0 < nslots && stop == 0xffffffffu; s0 += 64u) {
        const uint32_t sj = s0 + lane;
        uint32_t wo = kSlotAbsent, nb = 0, sb = kEmptyRun, a0 = 0, a1 = 0;
        if (sj < nslots) {
          wo = woff[sj];
          if (wo < kSlotAbsent) {
            nb = words[wo];
            sb = words[wo + 1];
            a0 = words[wo + 2];
            a1 = words[wo + 3];
          }
        }
        const bool present = wo != kSlotAbsent;
        const bool simple = wo < kSlotAbsent && nb == 0u;
        uint32_t t0 = 0;
        for (;;) {
          const uint32_t cb = __float_as_uint(c);
          const uint32_t bin = cb & 0xff800000u;
          const uint32_t ub = bin + 0x00800000u;
          const bool act = lane >= t0 && present;
          // an empty run (all-zero segment) is the identity in any binade
          const bool fit = simple && (sb == bin || sb == kEmptyRun);
          PMap m{0u, 0u};
          if (act && fit && sb != kEmptyRun) m = PMap{a0, a1};
          const PMap id{0u, 0u};
          const PMap ex = wave_shr1(wave_scan_incl(m, id, pm_combine), id);
          const uint32_t before = (cb & 1u) ? ex.a1 : ex.a0;
          const uint32_t own = ((cb ^ before) & 1u) ? m.a1 : m.a0;
          const uint32_t sbits = cb + before;
          const uint32_t ebits = sbits + own;
          const bool bad = act && (!fit || before >= kSat || own >= kSat || ebits >= ub);
          const unsigned long long bm = __ballot(bad);
          if (!bm) {
            c = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)ebits, 63));
            break;
          }
          const int tb = __ffsll((long long)bm) - 1;
          c = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)sbits, tb));
          const uint32_t wt = (uint32_t)__builtin_amdgcn_readlane((int)wo, tb);
          float y = c;
          ++nbw;
          if (wt < kSlotAbsent && rec_walk<M>(words + wt, y)) {
            c = y;
          } else {
            stop = s0 + (uint32_t)tb;  // c is its exact start
            break;
          }
          t0 = (uint32_t)tb + 1u;
          if (t0 >= 64u) break;
        }
      }
      if (lane == 0) {
        s.red_f[0] = c;
        s.misc_u[3] = stop;
        s.misc_u[2] = nbw;
      }
    }
    __syncthreads();
    c = s.red_f[0];
    const uint32_t stop = s.misc_u[3];
    __syncthreads();
    if (stop == 0xffffffffu) break;
    // the segment again, by the whole workgroup: two summands per thread
    const Slice r = rec_range<M>(V, G, stop);
    static_assert(64 * M <= 2 * kThreads, "a segment fits two summands per thread");
    float x[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t i = r.lo + 2u * t + (uint32_t)q;
      x[q] = i < r.hi ? expf_glibc(__fsub_rn(row.at(i), m1)) : 0.f;
    }
    c = ecss_fast_chunk<2>(c, x, kEcssSum, 0.f, s.ecss, s.est, s.wsum,
                           (int)min((uint32_t)kThreads, (r.hi - r.lo + 1u) / 2u)).c;
    ++nre;
    LUMEN_TICK("walk_recomputed", b);
    from = stop + 1u;
  }
  *nre_out = nre | (s.misc_u[2] << 8);
  return c;
}

// After the row barrier (m1 known): this workgroup's candidates, still in
// list A as (~key << 32) | id, are rewritten to the row's candidate buffer as
// (exp(v - m1) bits << 32) | id, and their exp-mass is binned by logit over
// [tau, m1] into this slice's histogram (used to size the top-p window).
__device__ __forceinline__ void slice_candidates(const KernelArgs& a, int b, uint32_t sl,
                                                 uint64_t* cand, uint32_t base, uint32_t n,
                                                 float m1, uint32_t tau, Smem& s) {
  const uint32_t t = threadIdx.x;
  float* hloc = reinterpret_cast<float*>(s.H);
  for (uint32_t i = t; i < (uint32_t)kMassBins; i += kThreads) hloc[i] = 0.f;
  __syncthreads();
  const float tv = tau ? key2f(tau) : kNegInf;
  const float span = tau ? __fsub_rn(m1, tv) : 0.f;
  const float inv_w = span > 0.f ? __fdiv_rn((float)kMassBins, span) : 0.f;
  for (uint32_t j = t; j < n; j += kThreads) {
    const uint64_t e = s.A[j];
    const float v = key2f(~(uint32_t)(e >> 32));
    const float x = expf_glibc(__fsub_rn(v, m1));
    if (base + j < (uint32_t)kCandCap) cand[base + j] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)e;
    if (inv_w > 0.f && v >= tv)
      atomicAdd(&hloc[min((uint32_t)kMassBins - 1u, (uint32_t)(__fsub_rn(m1, v) * inv_w))], x);
  }
  __syncthreads();
  float* hg = a.hist + ((uint64_t)b * kMaxSlices + sl) * kMassBins;
  for (uint32_t i = t; i < (uint32_t)kMassBins; i += kThreads) hg[i] = hloc[i];
}

__device__ __forceinline__ void topp_window(const KernelArgs& a, int b, const RowParams P,
                                                     const Row row, float m1, float S1, uint32_t tau,
                                                     uint32_t ncand, float rdraw, Smem& s, RowTrace tr);

// Top-p without top-k or penalties. Pass 1 (all slices): slice max, an
// exp-sum estimate, and the candidates above a sampled logit threshold.
// Row barrier. Pass 2: exact T = 1 softmax sum chained across the slices.
// The last slice then walks the candidates in probability order (window 1 of
// the reference's sorted order); if the crossing is not inside it, the exact
// single-workgroup path takes over.
__device__ __forceinline__ void topp_split(const KernelArgs& a, int b, uint32_t sl, uint32_t G,
                                                    Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t V = a.vocab;
  const Slice sc = slice_bounds(V, G, sl);
  if (a.pen_out) slice_pen_out(a, b, row, sc, P, false);
  LUMEN_TICK("p_start", b);
  const uint32_t tau = sample_threshold(row, V, 6000u, s);
  LUMEN_TICK("p_sampled", b);
  const float tv = tau ? key2f(tau) : kNegInf;
  const float lo_v = tau ? __fsub_rn(tv, __fmul_rn(fabsf(tv) + 64.f, 0x1p-10f)) : kNegInf;
  float mt = kNegInf;
  double et = 0.0;
  uint32_t nan = 0;
  if (threadIdx.x == 0) s.cnt = 0;
  __syncthreads();
  range_foreach(row, sc.lo, sc.hi, [&](uint32_t i, float v) {
    const bool isn = is_nan(v);
    nan |= isn ? 1u : 0u;
    if (!isn && v != kNegInf) {
      if (v > mt) {
        et = et * (double)__expf(mt - v) + 1.0;
        mt = v;
      } else {
        et += (double)__expf(v - mt);
      }
    }
    list_push(s.A, &s.cnt, !isn && (tau == 0u || v >= lo_v), ((uint64_t)(~tkey(v)) << 32) | i);
  });
  flush_candidates(cand, &ws.cand_n, s);
  const uint32_t my_base = s.misc_u[1];
  const uint32_t my_n = min(s.cnt, (uint32_t)kCap);
  const float ms = block_rmax(mt, s);
  nan = block_or_u32(nan, s);
  double es = (mt == kNegInf) ? 0.0 : et * exp((double)mt - (double)ms);
  double es_tot;
  (void)block_excl_scan_f64(es, s, &es_tot);
  if (threadIdx.x == 0) {
    ws.part_max[sl] = ms;
    ws.part_nan[sl] = nan;
    ws.part_e[sl] = es_tot;
  }
  LUMEN_TICK("p_pass1", b);
  wg_arrive(&ws.bar, 0xffffffffu, s);
  const bool ok = wg_wait_geq(a, &ws.bar, G, s);
  if (!ok && threadIdx.x == 0)
    __hip_atomic_fetch_or(&ws.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  LUMEN_TICK("p_barrier", b);
  float m1 = kNegInf;
  uint32_t anynan = 0;
  double p_slice = 0.0;
  for (uint32_t i = 0; i < G; ++i) {
    const float mi = ws.part_max[i];
    m1 = rmax(m1, mi);
    anynan |= ws.part_nan[i];
  }
  for (uint32_t i = 0; i < sl; ++i)
    if (ws.part_max[i] != kNegInf) p_slice += exp((double)ws.part_max[i] - (double)m1) * ws.part_e[i];
  const uint32_t ncand = __hip_atomic_load(&ws.cand_n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // NaN / infinite rows and oversized candidate sets take the exact single
  // path (uniform across the row once the barrier has completed)
  const bool single = anynan || !is_finite(m1) || ncand > (uint32_t)kCandCap;
  const bool m16 = sc_len_max(V, G) <= 16u * kThreads;
  if (ok && !single) {
    slice_candidates(a, b, sl, cand, my_base, my_n, m1, tau, s);
    if (m16) chain_prepare<16>(a, b, sl, row, sc, m1, p_slice, s);
    else chain_prepare<32>(a, b, sl, row, sc, m1, p_slice, s);
  }
  LUMEN_TICK("p_prepared", b);
  if (wg_arrive(&ws.arrive, G - 1u, s) != G - 1u) {
    LUMEN_TICK("p_not_finisher", b);
    LUMEN_TICK_DUMP(b);
    return;
  }
  LUMEN_TICK("p_finisher", b);
  if (!ok || single ||
      __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
    row_single<false>(a, b, s);
    return;
  }
  // Inputs from the other workgroups, fetched with as few dependent round
  // trips as possible: the candidates (exp already applied) into list A, the
  // summed mass histogram into H, then the parked records into list B.
  {
    const uint32_t t = threadIdx.x;
    const uint32_t nc = min(ncand, (uint32_t)kCap);
    LUMEN_TICK("g_status_read", b);
    uint64_t c[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t j = (uint32_t)q * kThreads + t;
      c[q] = j < nc ? cand[j] : 0ull;
    }
    LUMEN_TICK("g_cands_issued", b);
    float hsum = 0.f;
    if (t < (uint32_t)kMassBins) {
      const float* hp = a.hist + (uint64_t)b * kMaxSlices * kMassBins + t;
      float hv[kMaxSlices];
#pragma unroll
      for (uint32_t i = 0; i < (uint32_t)kMaxSlices; ++i) hv[i] = i < G ? hp[(uint64_t)i * kMassBins] : 0.f;
#pragma unroll
      for (uint32_t i = 0; i < (uint32_t)kMaxSlices; ++i) hsum += hv[i];
    }
    LUMEN_TICK("g_hist_in", b);
    if (m16) rec_gather<16>(a, b, G, s);
    else rec_gather<32>(a, b, G, s);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t j = (uint32_t)q * kThreads + t;
      if (j < nc) s.A[j] = c[q];
    }
    if (t < (uint32_t)kMassBins) reinterpret_cast<float*>(s.H)[t] = hsum;
    __syncthreads();
  }
  LUMEN_TICK("p_gathered", b);
  uint32_t nre;
  const float S1 = m16 ? chain_walk<16>(a, b, G, row, m1, &nre, s)
                       : chain_walk<32>(a, b, G, row, m1, &nre, s);
  LUMEN_TICK("p_chain", b);
  RowTrace tr;
  init_trace(tr, V);
  tr.path = 4u;
  tr.passes = 2;
  tr.topp_sum = S1;
  tr.pad[0] = nre;  // diagnostics: segments summed again | records walked one by one << 8
  topp_window(a, b, P, row, m1, S1, tau, ncand, rdraw, s, tr);
}

// Window 1 of the top-p order: the candidates with p >= p(tau), sorted by
// (p desc, index asc), walked with the exact cumulative sum; the kept prefix
// continues on the small path in index order. A crossing outside the window
// hands the row to the exact single-workgroup path.
__device__ __forceinline__ void topp_window(const KernelArgs& a, int b, const RowParams P,
                                                     const Row row, float m1, float S1, uint32_t tau,
                                                     uint32_t ncand, float rdraw, Smem& s, RowTrace tr) {
  const uint32_t t = threadIdx.x;
  const float tv = tau ? key2f(tau) : kNegInf;
  // The candidates hold every logit >= tau (and a margin below). Their
  // exp-mass per logit bin, accumulated from the top, gives the lowest bin
  // whose cumulative mass already exceeds top_p * S1 with a margin; window 1
  // then only needs the candidates from that bin's lower edge up (never below
  // tau). The bin masses only steer the window size: the crossing itself is
  // found exactly on the sorted window, and a window that misses it hands
  // the row to the exact path.
  constexpr uint32_t kBins = (uint32_t)kMassBins;
  const float* hmass = reinterpret_cast<const float*>(s.H);
  const float span = tau ? __fsub_rn(m1, tv) : 0.f;
  const bool binned = tau && span > 0.f;
  const uint32_t nc = min(ncand, (uint32_t)kCap);
  float v_thr = tv;
  if (binned) {
    // first bin (from the top) where the running mass reaches the target
    if (t < 64u) {
      const float target = fminf(__fmul_rn(__fmul_rn(P.top_p, S1), 1.004f), S1);
      float run = 0.f;
      uint32_t hit = kBins;
      for (uint32_t base = 0; base < kBins && hit == kBins; base += 64u) {
        const float m =
            wave_scan_incl(hmass[base + t], 0.f, [](float l, float r) { return l + r; });
        const unsigned long long hm = __ballot(run + m >= target);
        if (hm) hit = base + (uint32_t)(__ffsll((long long)hm) - 1);
        run += wave_read(m, 63);
      }
      if (t == 0) s.misc_u[2] = hit;
    }
    __syncthreads();
    const uint32_t hit = s.misc_u[2];
    if (hit + 2u < kBins) {
      // one spare bin below: binning rounds (m1 - v) / w
      const float edge = __fsub_rn(m1, __fmul_rn((float)(hit + 2u), __fdiv_rn(span, (float)kBins)));
      v_thr = fmaxf(tv, edge);
    }
  }
  LUMEN_TICK("p_threshold", b);
  const float p_lo = tau ? __fdiv_rn(expf_glibc(__fsub_rn(v_thr, m1)), S1) : 0.f;
  if (t == 0) s.cnt = 0;
  __syncthreads();
  for (uint32_t base = 0; base < nc; base += kThreads) {
    const uint32_t j = base + t;
    bool in = false;
    uint64_t e = 0;
    if (j < nc) {
      const uint64_t c = s.A[j];
      const float p = __fdiv_rn(__uint_as_float((uint32_t)(c >> 32)), S1);
      in = p > 0.f && p >= p_lo;
      e = ((uint64_t)(~__float_as_uint(p)) << 32) | (uint32_t)c;
    }
    list_push(s.Bk, &s.cnt, in, e);
  }
  __syncthreads();
  const uint32_t n = s.cnt;
  LUMEN_TICK("p_window_built", b);
  {
    // keys (~p bits << 32) | id with p in [p_lo, 1/S1]: their common high
    // bits are known without a reduction
    const uint32_t khi = ~__float_as_uint(__fdiv_rn(1.0f, S1)), klo = ~__float_as_uint(p_lo);
    const uint64_t hint = p_lo > 0.f ? ((uint64_t)(khi ^ klo) << 32) | span_mask(a.vocab) : 0ull;
    sort_u64_asc(s.Bk, n, s.A, s, hint);
  }
  LUMEN_TICK("p_window_sorted", b);
  // the sorted probabilities into a padded float array (list A is free
  // after the sort)
  float* ps = reinterpret_cast<float*>(s.A);
  for (uint32_t j = threadIdx.x; j < n; j += kThreads)
    ps[pad16(j)] = __uint_as_float(~(uint32_t)(s.Bk[j] >> 32));
  __syncthreads();
  EcssResult wk = list_ecss(n, [&](uint32_t j) { return ps[pad16(j)]; }, kEcssFindGe, P.top_p, 0.f, s);
  LUMEN_TICK(s.est.fail == 2 ? "p_walk_nofit" : s.est.fail ? "p_walk_failed" : "p_walk_ok", b);
  if (!wk.found) {
    row_single<false>(a, b, s);
    return;
  }
  tr.windows = 1;
  tr.topp_kept = (uint32_t)wk.pos + 1u;
  tr.topp_cum = wk.c;
  const uint32_t nk = (uint32_t)wk.pos + 1u;
  for (uint32_t j = threadIdx.x; j < nk; j += kThreads) {
    const uint32_t idx = (uint32_t)s.Bk[j];
    s.A[j] = ((uint64_t)idx << 32) | tkey(row.at(idx));
  }
  __syncthreads();
  sort_u64_asc(s.A, nk, s.Bk, s, ((uint64_t)span_mask(a.vocab) << 32) | 0xffffffffull);
  LUMEN_TICK("p_kept_sorted", b);
  // the kept set holds the row maximum m1
  small_path(a, b, P, nk, true, rdraw, s, tr, m1);
}

}  // namespace lumen

#include "resident.h"
#include "plain.h"
#include "rowsum.h"

namespace lumen {

// Row and slice of this workgroup. With xcd_rows, blocks are dispatched to
// the 8 XCDs round-robin: a row's slices stay on one XCD so its
// coordination traffic stays in that XCD's L2.
__device__ __forceinline__ void block_row(const KernelArgs& a, uint32_t& b, uint32_t& sl,
                                          uint32_t& G) {
  if (a.blk_map) {
    const uint32_t m = a.blk_map[blockIdx.x];
    if (m == kIdleBlock) {
      b = 0xffffffffu;
      sl = 0;
      G = 1;
      return;
    }
    b = m >> 10;
    G = (m >> 5) & 31u;
    sl = m & 31u;
    return;
  }
  G = a.slices;
  if (a.xcd_rows) {
    const uint32_t xcd = blockIdx.x & 7u, j = blockIdx.x >> 3;
    b = xcd + 8u * (j / G);
    sl = j % G;
  } else {
    b = blockIdx.x / G;
    sl = blockIdx.x % G;
  }
}

// The workgroup that arrived last on its row's counter restores the row's
// coordination block once it is done. Every other workgroup of the row has
// arrived before it and no longer touches the block; the next launch sees
// the cleared block (kernel boundary). One exception: a top-p finisher that
// gave up waiting for its S1 walker leaves the reset to the walker
// (res_s1_walker), whose release is then the block's last access.
__device__ __forceinline__ void row_reset(const KernelArgs& a, uint32_t b, Smem& s) {
  __syncthreads();
  if (threadIdx.x == 0 && s.finisher) {
    RowWs& ws = a.ws[b];
    ws.arrive = 0;
    ws.bar = 0;
    ws.cand_n = 0;
    ws.status = 0;
  }
}

// The layout stamp the host library checks when it loads this code object.
extern "C" __device__ __attribute__((used)) const uint32_t lumen_kernel_abi = kAbiStamp;

extern "C" __global__ void __launch_bounds__(1024) lumen_sample_rows(KernelArgs args) {
  // Device functions receive the arguments by reference. Referencing the
  // by-value parameter would make every thread copy it to private memory;
  // the kernarg segment already holds it (it is the only argument), so the
  // reference points there instead.
  (void)args;
  const KernelArgs& a =
      *reinterpret_cast<const KernelArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
  __shared__ Smem s;
  LUMEN_TICK_INIT();
  if (threadIdx.x == 0) s.finisher = 0u;
  expf_table_init();
  __syncthreads();
  uint32_t b, sl, G;
  block_row(a, b, sl, G);
  if (b >= a.batch) return;

  LUMEN_TICK_SLOT(b, sl);
  __syncthreads();
  if (G == 1u) {
    row_single<false>(a, (int)b, s);
    return;
  }
  {
    const RowParams& P = a.inline_rows ? a.inline_params[b] : a.params[b];
    const uint32_t flags = P.flags;
    const uint64_t top_k = P.top_k;
    const uint32_t per = ((a.vocab + G - 1u) / G + 15u) & ~15u;
    if (flags & kGreedy) {
      if (flags & kAnti)
        greedy_guard_split(a, (int)b, sl, G, s);
      else
        greedy_split(a, (int)b, sl, G, s);
    } else if ((flags & kTopK) && top_k <= kTopKSplitMax) {
      topk_split(a, (int)b, sl, G, s);
    } else if (!(flags & kTopK) && ((flags & kTopP) || !(flags & kMinP)) && a.vocab >= 64u &&
               make_row(a, (int)b).vec && res_chunks(a.vocab, G) != 0u) {
      // register-resident rows: top-p, or plain temperature
      const uint32_t q = res_chunks(a.vocab, G);
      if (flags & kTopP) {
        if (q == 1u) {
          if (a.dtype == 0)
            topp_res<false, false>(a, (int)b, sl, G, q, s);
          else
            topp_res<true, false>(a, (int)b, sl, G, q, s);
        } else if (a.dtype == 0) {
          topp_res<false, true>(a, (int)b, sl, G, q, s);
        } else {
          topp_res<true, true>(a, (int)b, sl, G, q, s);
        }
      } else if (q == 1u) {
        if (a.dtype == 0)
          temp_res<false, false>(a, (int)b, sl, G, q, s);
        else
          temp_res<true, false>(a, (int)b, sl, G, q, s);
      } else if (a.dtype == 0) {
        temp_res<false, true>(a, (int)b, sl, G, q, s);
      } else {
        temp_res<true, true>(a, (int)b, sl, G, q, s);
      }
    } else if ((flags & kTopP) && !(flags & (kTopK | kPen)) &&
               per <= 32u * kThreads * kChainMaxQ) {
      topp_split(a, (int)b, sl, G, s);
    } else if (sl == 0) {
      row_single<false>(a, (int)b, s);
    }
  }
  row_reset(a, b, s);
}

// One workgroup per row (launches that do not split rows): the whole
// sampler of row blockIdx.x.
extern "C" __global__ void __launch_bounds__(1024) lumen_sample_rows_single(KernelArgs args) {
  (void)args;
  const KernelArgs& a =
      *reinterpret_cast<const KernelArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
  __shared__ Smem s;
  LUMEN_TICK_INIT();
  if (threadIdx.x == 0) s.finisher = 0u;
  expf_table_init();
  __syncthreads();
  const uint32_t b = blockIdx.x;
  if (b >= a.batch) return;
  LUMEN_TICK_SLOT(b, 0u);
  __syncthreads();
  row_single_body<true>(a, (int)b, s);
}

// Penalty window counts from the device history ring, one workgroup per row
// (sampling.rs:858-878: the last `window` tokens, or the whole history when
// window is 0, counted per distinct id). Runs before lumen_sample_rows on the
// same stream. Counts go through an LDS hash table (2 * kRingMaxCap slots,
// linear probing), then out as (id, count) pairs in slot order, which the
// sampler does not depend on. Counts that follow the history token by token
// (one token recorded since they were made) are updated in place instead,
// which also carries a whole-history window (or any window from which
// nothing leaves) past the ring's capacity. A window that must be counted
// again but is longer than the ring cannot be: hist_off[b] = kHistBad (an
// empty range, since hist_end[b] is below it) and the row's token becomes
// LUMEN_TOKEN_ERROR with kStatusHistOverflow when it is written.
constexpr uint32_t kHashSlots = 2u * kRingMaxCap;
constexpr uint32_t kHashEmpty = 0xffffffffu;
static_assert(kHashSlots == (1u << 14), "the hash takes the top 14 bits");

extern "C" __global__ void __launch_bounds__(1024) lumen_hist_window(KernelArgs args) {
  (void)args;
  const KernelArgs& a =
      *reinterpret_cast<const KernelArgs*>(__builtin_amdgcn_kernarg_segment_ptr());
  __shared__ uint32_t hkey[kHashSlots];
  __shared__ uint32_t hcnt[kHashSlots];
  __shared__ uint32_t nout;
  __shared__ uint32_t pout_s;
  const uint32_t b = blockIdx.x, t = threadIdx.x;
  if (b >= a.batch) return;
  const RowParams& P = a.inline_rows ? a.inline_params[b] : a.params[b];
  const uint32_t cap = a.ring_cap, ccap = a.count_cap;
  const uint64_t rbase = (uint64_t)b * cap;   // the row's ring
  const uint32_t base = b * ccap;             // the row's counts
  uint32_t* off = const_cast<uint32_t*>(a.hist_off);
  uint32_t* ids = const_cast<uint32_t*>(a.hist_ids);
  uint32_t* cnt = const_cast<uint32_t*>(a.hist_cnt);
  const uint32_t len = a.ring_len[b];
  const uint32_t w = (P.window > 0u && P.window < len) ? P.window : len;
  uint32_t* st = a.hist_state + (uint64_t)b * 8u;
  const uint64_t rid = (uint64_t)(uintptr_t)a.ring;
  auto set_state = [&](uint32_t l) {
    if (t == 0) {
      st[0] = l;
      st[1] = P.window;
      st[2] = (uint32_t)rid;
      st[3] = (uint32_t)(rid >> 32);
      st[4] = cap;
      st[5] = a.ring_epoch;
      st[6] = ccap;
    }
  };
  if (!(P.flags & kPen) || w == 0u) {
    if (t == 0) {
      off[b] = base;
      a.hist_end[b] = base;
    }
    set_state((P.flags & kPen) ? len : 0xffffffffu);
    return;
  }
  // the counts were made for this ring, window and layout
  const bool same = st[0] != 0xffffffffu && st[1] == P.window && st[2] == (uint32_t)rid &&
                    st[3] == (uint32_t)(rid >> 32) && st[4] == cap && st[5] == a.ring_epoch &&
                    st[6] == ccap && off[b] == base;
  // ... and already reflect this history (seeded, or nothing recorded since)
  if (same && st[0] == len) return;
  // A token that leaves the window sits at len - 1 - window; the ring still
  // holds it (the new token has not overwritten it) only when window < cap.
  const bool leaves = P.window > 0u && len - 1u >= P.window;
  const bool follows = same && st[0] + 1u == len && (!leaves || P.window < cap);
  if (follows) {
    // one token recorded since the counts were made (by the sampler): add
    // it, and take out the token that left a full window
    const uint32_t* ring = a.ring + rbase;
    const uint32_t tin = ring[(len - 1u) % cap];
    const uint32_t tout = leaves ? ring[(len - 1u - P.window) % cap] : kHashEmpty;
    const uint32_t n0 = a.hist_end[b] - base;
    if (t == 0) {
      nout = kHashEmpty;   // position of tin
      pout_s = kHashEmpty;  // position of tout
    }
    __syncthreads();
    if (tin != tout)
      for (uint32_t j = t; j < n0; j += blockDim.x) {
        const uint32_t id = ids[base + j];
        if (id == tin) nout = j;
        if (leaves && id == tout) pout_s = j;
      }
    __syncthreads();
    const uint32_t pin = nout, pout = pout_s;
    const bool grows = tin != tout && pin == kHashEmpty;
    if (!(tin != tout && leaves && pout == kHashEmpty) && !(grows && n0 >= ccap)) {
      if (t == 0) {
        uint32_t n = n0;
        if (tin != tout) {
          if (pin != kHashEmpty) {
            cnt[base + pin] += 1u;
          } else {
            ids[base + n] = tin;
            cnt[base + n] = 1u;
            ++n;
          }
          if (leaves) {
            const uint32_t c = cnt[base + pout] - 1u;
            if (c) {
              cnt[base + pout] = c;
            } else {
              // the last entry takes the freed place
              --n;
              ids[base + pout] = ids[base + n];
              cnt[base + pout] = cnt[base + n];
            }
          }
        }
        off[b] = base;
        a.hist_end[b] = base + n;
        st[0] = len;
      }
      return;
    }
    // the counts do not hold the leaving token: count the window again
    __syncthreads();
  }
  if (w > cap) {
    // the ring no longer holds the window: no counts (an empty range); the
    // row's finisher reports the overflow
    if (t == 0) {
      off[b] = kHistBad;
      a.hist_end[b] = base;
    }
    set_state(0xffffffffu);
    return;
  }
  for (uint32_t i = t; i < kHashSlots; i += blockDim.x) {
    hkey[i] = kHashEmpty;
    hcnt[i] = 0u;
  }
  if (t == 0) nout = 0u;
  __syncthreads();
  const uint32_t* ring = a.ring + rbase;
  for (uint32_t j = t; j < w; j += blockDim.x) {
    const uint32_t id = ring[(len - w + j) % cap];
    uint32_t h = (id * 2654435761u) >> (32 - 14);  // Fibonacci hashing into 2^14 slots
    for (;;) {
      const uint32_t old = atomicCAS(&hkey[h], kHashEmpty, id);
      if (old == kHashEmpty || old == id) {
        atomicAdd(&hcnt[h], 1u);
        break;
      }
      h = (h + 1u) & (kHashSlots - 1u);
    }
  }
  __syncthreads();
  for (uint32_t i = t; i < kHashSlots; i += blockDim.x) {
    if (hkey[i] != kHashEmpty) {
      const uint32_t k = atomicAdd(&nout, 1u);
      ids[base + k] = hkey[i];
      cnt[base + k] = hcnt[i];
    }
  }
  __syncthreads();
  if (t == 0) {
    off[b] = base;
    a.hist_end[b] = base + nout;
  }
  set_state(len);
}
// Token 0 for every row of an empty vocabulary (sampling.rs:458-460),
// recorded into the row's device history ring when there is one
// (SamplerState::record, sampling.rs:381-384).
extern "C" __global__ void __launch_bounds__(256) lumen_zero_tokens(ZeroArgs z) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= z.n) return;
  z.tokens[i] = 0u;
  if (z.ring) {
    const uint32_t n = z.ring_len[i];
    z.ring[(uint64_t)i * z.ring_cap + n % z.ring_cap] = 0u;
    z.ring_len[i] = n + 1u;
  }
}

}  // namespace lumen
