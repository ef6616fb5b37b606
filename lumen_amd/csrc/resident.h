// Register-resident split path for top-p rows (included by sampler_kernels.hip).
//
// Reference semantics: apply_top_p_on_logits (crates/lumen-runtime/src/
// sampling.rs:942-967) after the penalties (:850-900) and before min-p,
// temperature, softmax and the draw (:510-526, :207-231, :1003-1014).
//
// Each of the G workgroups of a row owns a slice of at most kResSlice logits
// and reads it from HBM exactly once: thread t keeps slice elements
// 32t .. 32t+31 in registers (contiguous, so a thread's part of any
// sequential sum is one run of adds). The loads are coalesced; an LDS
// transpose hands each thread its own run. Then:
//
//  phase A  penalties (patched in the LDS copy), the slice maximum, an
//           exp-sum estimate, and the candidates: every logit at or above a
//           threshold sampled from the row (the same in every slice), written
//           in index order to the row's candidate buffer;
//  barrier  the row maximum m1 and each slice's exp-sum estimate;
//  phase B  the exact summands exp(v - m1) and the slice's record of the
//           exact sequential f32 softmax sum (runs of whole threads as parity
//           maps of ecss.h, plus the raw summands of the few threads whose
//           binade the estimate cannot fix);
//  finisher the last workgroup to arrive walks the G records in order (the
//           exact S1), takes the candidates in index order, sorts the window
//           that holds the nucleus by (p desc, id asc), walks the exact
//           cumulative sum to the crossing, keeps the nucleus in index order
//           and runs the final stage (min-p, temperature, softmax, draw).
//
// Every estimate only decides speed: a record run is applied only after
// checking that the exact running sum sits inside its binade and stays
// there, and any check that fails, a candidate set that misses the
// crossing, or a timeout hands the row to the exact single-workgroup path.
#pragma once

namespace lumen {

constexpr uint32_t kResK = 32;                                    // logits per thread
constexpr uint32_t kResSlice = kResK * (uint32_t)kThreads;        // logits per slice
constexpr uint32_t kResPitch = kResK + 4u;                        // LDS words per thread
constexpr uint32_t kResCandTarget = 5000;                         // candidates aimed at per row
constexpr uint32_t kResItemCap = 4096;                            // record items per slice
constexpr uint32_t kResRawOff = 4u * kResItemCap;                 // word offset of the raw area
constexpr uint32_t kResSliceWords = 32u * (uint32_t)kRecWords;    // record words per slice
constexpr uint32_t kResRawCap = (kResSliceWords - kResRawOff) / kResK;  // uncertain threads per slice
constexpr uint32_t kNoRaw = 0xffffffffu;
constexpr uint32_t kResWindowCap = (uint32_t)kCap / 2u;          // sorted in place with its own spare half
static_assert((uint32_t)kMaxSlices * 32u <= (uint32_t)kRowRecs, "slice record areas fit the row");


__device__ __forceinline__ float* res_buf(Smem& s) { return reinterpret_cast<float*>(s.A); }

__device__ __forceinline__ uint32_t* res_rec(const KernelArgs& a, int b, uint32_t sl) {
  return a.est + ((uint64_t)b * kRowRecs + (uint64_t)sl * 32u) * kRecWords;
}


// Issues the coalesced loads of this thread's share of its wave's block:
// wave w covers slice elements [2048 w, 2048 (w + 1)), lane l loads elements
// 256 q + 4 l .. +3 of it. The row must be vector aligned (Row::vec) and
// hold at least 8 logits. Addresses are clamped into the row and elements at
// or past sc.hi read as -inf, with no branch; when the row length is not a
// multiple of 4 the partial group at its end is not loaded here (res_tail
// patches it in the LDS copy).
template <bool BF16>
__device__ __forceinline__ void res_issue(const Row& row, Slice sc, float (&v)[8][4]) {
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t base = sc.lo + w * (64u * kResK) + 4u * lane;
  const uint32_t last4 = (row.V - 4u) & ~3u;  // start of the last whole group of 4
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint32_t i = base + 256u * (uint32_t)q;
    const uint32_t ic = min(i, last4);
    float f[4];
    if (BF16) {
      const ushort4 h = *reinterpret_cast<const ushort4*>(row.h + ic);
      f[0] = __uint_as_float((uint32_t)h.x << 16);
      f[1] = __uint_as_float((uint32_t)h.y << 16);
      f[2] = __uint_as_float((uint32_t)h.z << 16);
      f[3] = __uint_as_float((uint32_t)h.w << 16);
    } else {
      const float4 g = *reinterpret_cast<const float4*>(row.f + ic);
      f[0] = g.x;
      f[1] = g.y;
      f[2] = g.z;
      f[3] = g.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) v[q][j] = (i == ic && i + (uint32_t)j < sc.hi) ? f[j] : kNegInf;
  }
}

// The partial group at the end of a row whose length is not a multiple of
// 4, into the LDS copy of the slice that holds it.
__device__ __forceinline__ bool res_has_tail(const Row& row, Slice sc) {
  return (row.V & 3u) != 0u && sc.hi == row.V && sc.hi > sc.lo;
}

// LDS word of slice element o in the transposed copy.
__device__ __forceinline__ uint32_t res_slot(uint32_t o) { return (o >> 5) * kResPitch + (o & 31u); }

__device__ __forceinline__ void res_tail(const Row& row, Slice sc, float* L) {
  const uint32_t t0 = max(sc.lo, row.V & ~3u);
  if (threadIdx.x < sc.hi - t0) L[res_slot(t0 + threadIdx.x - sc.lo)] = row.at(t0 + threadIdx.x);
}

// Moves the loaded block through LDS so that thread t holds slice elements
// 32t .. 32t+31 in x[]. With `patched`, patch(L) runs on the whole LDS copy
// (all waves) between the store and the read-back. The LDS copy stays valid
// until the caller writes LDS again. Starts and ends with a barrier.
template <class Patch>
__device__ __forceinline__ void res_transpose(const float (&v)[8][4], float (&x)[kResK], Smem& s,
                                              bool patched, Patch&& patch) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  float* L = res_buf(s);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const uint32_t e = 256u * (uint32_t)q + 4u * lane;  // element in the wave's block
    const uint32_t owner = w * 64u + (e >> 5);
    *reinterpret_cast<float4*>(L + owner * kResPitch + (e & 31u)) =
        make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
  }
  __syncthreads();
  if (patched) {
    patch(L);
    __syncthreads();
  }
  // pitch 36 words: 16 consecutive lanes read 16 distinct 4-bank groups
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float4 f = *reinterpret_cast<const float4*>(L + t * kResPitch + 4u * (uint32_t)m);
    x[4 * m] = f.x;
    x[4 * m + 1] = f.y;
    x[4 * m + 2] = f.z;
    x[4 * m + 3] = f.w;
  }
}

__device__ __forceinline__ float block_maxl(float v, Smem& s) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_reduce(v, kNegInf, op_maxl);
  if (lane == 0) s.red_f[w] = v;
  __syncthreads();
  float r = kNegInf;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r = op_maxl(r, s.red_f[i]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ double block_sum_f64(double v, Smem& s) {
  double tot;
  (void)block_excl_scan_f64(v, s, &tot);
  return tot;
}

// Exclusive block scan of a u32 with the total (uniform).
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, Smem& s, uint32_t* total) {
  const uint32_t inc = block_incl_scan_u32(v, s);
  if (threadIdx.x == kThreads - 1) s.misc_u[0] = inc;
  __syncthreads();
  *total = s.misc_u[0];
  __syncthreads();
  return inc - v;
}

struct RecCount {
  uint32_t items, raws;
  bool ok;
};

// Record of the exact sequential f32 sum of this slice's summands (thread t
// reads its slice elements 32t .. 32t+31 at et, in LDS; nthr threads hold
// any), entered
// with a running sum of about p_slice (f64). Thread t's running sum starts
// near P_t = p_slice + (sum of the summands before it); its binade is
// certain unless P_t widened by `rel` (the f32 sum drifts from its f64
// estimate as summands are rounded onto its grid, by up to ~4e-9 per
// element in logit rows) touches another binade. Items (4 words each):
//   {bin, a0, a1, kNoRaw}  a run of consecutive certain threads in binade
//                          bin: grid steps added for an even / odd start;
//   {bin, a0, a1, r}       one uncertain thread: its map inside bin (used
//                          when the exact sum is inside bin at its start and
//                          stays there), else its 32 summands at raw slot r.
// Items start at rec[0]; raw slot r at rec[kResRawOff + 32 r].
// FIND (inverse-CDF records): a thread whose running-sum range may hold the
// draw `probe` is made uncertain too, so a search for the first sum above
// the probe always ends inside a raw; raw items carry their thread index in
// bits 16..25 of the last word.
template <bool FIND = false>
__device__ __forceinline__ RecCount res_record(const float* et, double p_slice, uint32_t pos0,
                                               uint32_t nthr, uint32_t* rec, Smem& s,
                                               float probe = 0.f, float lb = 0.f) {
  const uint32_t t = threadIdx.x;
  const bool live = t < nthr;
  const float4* e4 = reinterpret_cast<const float4*>(et);  // this thread's 32 summands (LDS)
  double d = 0.0;
#pragma unroll
  for (int m = 0; m < (int)kResK / 4; ++m) {
    const float4 f = e4[m];
    d += (double)f.x;
    d += (double)f.y;
    d += (double)f.z;
    d += (double)f.w;
  }
  // the f64 prefix of the thread totals (the estimated running sum at the
  // thread's start) and, with it, a floor for the exact running sum there:
  // a sum of non-negative f32 terms is never below any term added so far,
  // so max(lb, the largest summand of the threads before) bounds it (a
  // row's maximum adds exactly 1.0, a binade edge the estimate straddles)
  float mx = 0.f;
#pragma unroll
  for (int m = 0; m < (int)kResK; ++m) mx = fmaxf(mx, et[m]);
  const uint32_t lane = t & 63u, w = t >> 6;
  const double dinc = wave_scan_incl(d, 0.0, [](double l, double r) { return l + r; });
  const float minc = wave_scan_incl(mx, 0.f, [](float l, float r) { return fmaxf(l, r); });
  double* wsum_d = s.wsum;
  float* wsum_m = s.red_f;
  if (lane == 63u) {
    wsum_d[w] = dinc;
    wsum_m[w] = minc;
  }
  __syncthreads();
  double pre = 0.0, tot = 0.0;
  float mpre = 0.f;
#pragma unroll
  for (uint32_t i = 0; i < (uint32_t)kWaves; ++i) {
    const double x = wsum_d[i];
    if (i < w) {
      pre += x;
      mpre = fmaxf(mpre, wsum_m[i]);
    }
    tot += x;
  }
  __syncthreads();
  const double P = p_slice + pre + (dinc - d);
  const double floor_t = (double)fmaxf(fmaxf(lb, mpre), wave_shr1(minc, 0.f));
  LUMEN_TICK("rr_scan", LUMEN_TIMING_ROW);
  // the probe's margin is the drift of a probability sum from its estimate
  // (the exact softmax sum divided out, from the slice's exact start):
  // observed up to ~3e-5 of it; a sum estimated from the row start drifts
  // by up to ~4e-9 of it per element
  constexpr double kProbeRel = 1e-4;
  const double rel = FIND ? kProbeRel : 5e-5 + 4e-9 * (double)(pos0 + t * kResK + kResK);
  const uint32_t blo = est_binade(fmax(P * (1.0 - rel), floor_t));
  const uint32_t bhi = est_binade((P + d) * (1.0 + rel));
  // a search: a thread whose running sum surely starts above the probe
  // cannot hold the hit and records nothing (a walk that then finds no hit
  // fails, and the caller takes the chunked method)
  const bool past = FIND && live && P * (1.0 - 1e-4) > (double)probe;
  const bool act = live && !past;
  bool unc = act && blo != bhi;
  if (FIND)
    unc = unc || (act && P * (1.0 - kProbeRel) <= (double)probe && (double)probe <= (P + d) * (1.0 + kProbeRel));
  const uint32_t bin = unc ? est_binade(P + 0.5 * d) : blo;
  float y0 = __uint_as_float(bin), y1 = __uint_as_float(bin | 1u);
#pragma unroll
  for (int m = 0; m < (int)kResK / 4; ++m) {
    const float4 f = e4[m];
    y0 = __fadd_rn(y0, f.x);
    y1 = __fadd_rn(y1, f.x);
    y0 = __fadd_rn(y0, f.y);
    y1 = __fadd_rn(y1, f.y);
    y0 = __fadd_rn(y0, f.z);
    y1 = __fadd_rn(y1, f.z);
    y0 = __fadd_rn(y0, f.w);
    y1 = __fadd_rn(y1, f.w);
  }
  const uint32_t n0 = __float_as_uint(y0) - bin, n1 = __float_as_uint(y1) - (bin | 1u);
  const PMap own{n0 > kSat ? kSat : n0, n1 > kSat ? kSat : n1};
  // neighbours' classes: a binade (low 23 bits zero), uncertain or absent
  constexpr uint32_t kUnc = 1u, kDead = 2u;
  uint32_t* cls = s.H0;
  const uint32_t code = !act ? kDead : unc ? kUnc : bin;
  cls[t] = code;
  __syncthreads();
  const uint32_t prv = t > 0 ? cls[t - 1] : kDead;
  const uint32_t nxt = t + 1 < (uint32_t)kThreads ? cls[t + 1] : kDead;
  // a run starts after anything else (certain threads never change binade
  // without an uncertain thread between them) and ends before anything else
  const bool head = act && (unc || prv != code);
  const bool last = act && !unc && nxt != code;
  LUMEN_TICK("rr_maps", LUMEN_TIMING_ROW);
  SegVal prev;
  const SegVal inc = seg_scan_incl(SegVal{head ? 1u : 0u, (act && !unc) ? own : PMap{0u, 0u}},
                                   s.ecss, s.est, &prev);
  const uint32_t packed = ((unc || last) ? 1u : 0u) | ((unc ? 1u : 0u) << 16);
  uint32_t ptot;
  const uint32_t pos = block_excl_scan_u32(packed, s, &ptot);
  RecCount rc{ptot & 0xffffu, ptot >> 16, true};
  LUMEN_TICK("rr_scans", LUMEN_TIMING_ROW);
  if (rc.items > kResItemCap || rc.raws > kResRawCap) {
    rc.ok = false;
    return rc;
  }
  const uint32_t ip = pos & 0xffffu, rp = pos >> 16;
  if (unc) {
    *reinterpret_cast<uint4*>(rec + 4u * ip) = make_uint4(bin, own.a0, own.a1, FIND ? rp | (t << 16) : rp);
    uint4* raw = reinterpret_cast<uint4*>(rec + kResRawOff + kResK * rp);
    const uint4* u4 = reinterpret_cast<const uint4*>(et);
#pragma unroll
    for (int m = 0; m < (int)kResK / 4; ++m) raw[m] = u4[m];
  } else if (last) {
    *reinterpret_cast<uint4*>(rec + 4u * ip) = make_uint4(bin, inc.m.a0, inc.m.a1, kNoRaw);
  }
  return rc;
}

// Mass bins of the window planner, on the bits of e = exp(v - m1) in (0, 1]:
// bin 0 holds the largest values; the shift makes [e_lo, 1] span at most
// kMassBins bins (e_lo: the smallest candidate value, 0 for all values).
__device__ __forceinline__ uint32_t res_bin_shift(float e_lo) {
  const uint32_t span = 0x3f800000u - (__float_as_uint(e_lo) & 0x7fffffffu);
  uint32_t sh = 0;
  while ((span >> sh) >= (uint32_t)kMassBins) ++sh;
  return sh;
}
__device__ __forceinline__ uint32_t res_bin(float e, uint32_t sh) {
  const uint32_t d = 0x3f800000u - min(__float_as_uint(e), 0x3f800000u);
  return min((uint32_t)kMassBins - 1u, d >> sh);
}
// Lower edge of bin h (values of bin h are >= it).
__device__ __forceinline__ float res_bin_lo(uint32_t h, uint32_t sh) {
  const uint64_t d = ((uint64_t)(h + 1u) << sh) - 1u;
  return d >= 0x3f800000ull ? 0.f : __uint_as_float(0x3f800000u - (uint32_t)d);
}

// Sampled key threshold (the rule of sample_threshold): the sample loads
// are issued first (res_sample_issue), the slice loads after them, and the
// selection (res_sample_select) then waits only for the sample.
__device__ __forceinline__ void res_sample_issue(const Row& row, float (&smp)[4]) {
  const uint32_t V = row.V;
  constexpr uint32_t kRuns = kSampleN / 32u;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t j = threadIdx.x + (uint32_t)q * kThreads;
    const uint32_t c = j >> 5;
    const uint32_t base = V > kSampleN ? (uint32_t)(((uint64_t)c * (V - 32u)) / (kRuns - 1u)) & ~31u : 0u;
    smp[q] = V > kSampleN ? row.at(base + (j & 31u)) : 0.f;
  }
}

__device__ __forceinline__ uint32_t res_sample_select(const float (&smp)[4], uint32_t V,
                                                      uint32_t target, Smem& s) {
  if (V <= kSampleN || target >= V) return 0u;
  const uint32_t r = (uint32_t)(((uint64_t)target * kSampleN + V - 1) / V);
  if (r == 0u || r > kSampleN) return 0u;
  uint32_t* keys = reinterpret_cast<uint32_t*>(s.A);
#pragma unroll
  for (int q = 0; q < 4; ++q) keys[threadIdx.x + (uint32_t)q * kThreads] = tkey(smp[q]);
  __syncthreads();
  // two digit levels: the lower edge of the bucket holding the r-th key
  const uint32_t tau = select_desc(kSampleN, [&](uint32_t j) { return keys[j]; }, r - 1u, s, 2);
  __syncthreads();
  return tau;
}

// The records of the row's G slices gathered into LDS (s.Bk as words): items
// of slice i from ib[i], raw slots of slice i from rb[i] (ib, rb in s.H0 +
// [0, 64)); returns false when they do not fit or a slice failed to record.
__device__ __forceinline__ bool res_gather(const KernelArgs& a, int b, uint32_t G, Smem& s,
                                           uint32_t* nit_out, uint32_t* rawbase_out) {
  RowWs& ws = a.ws[b];
  const uint32_t t = threadIdx.x, lane = t & 63u;
  uint32_t* ib = s.H0;
  uint32_t* rb = s.H0 + 32;
  if (t < 64u) {
    const bool in = lane < G;
    const uint32_t ni = in ? ws.part_nrec[lane] : 0u;
    const uint32_t nr = in ? ws.part_nraw[lane] : 0u;
    const bool failed = __ballot(in && ni == 0xffffffffu) != 0ull;
    const uint32_t ei = wave_scan_incl(failed ? 0u : ni, 0u, op_add_u32);
    const uint32_t er = wave_scan_incl(nr, 0u, op_add_u32);
    const uint32_t pi = wave_shr1(ei, 0u), pr = wave_shr1(er, 0u);
    if (lane <= G) {
      ib[lane] = pi;
      rb[lane] = pr;
    }
    if (lane == 0) s.misc_u[3] = failed ? 1u : 0u;
  }
  __syncthreads();
  const uint32_t nit = ib[G], nrw = rb[G];
  const uint32_t rawbase = 4u * nit;
  const uint32_t nw = rawbase + kResK * nrw;
  const bool ok = s.misc_u[3] == 0u && nw <= 2u * (uint32_t)kCap;
  __syncthreads();
  if (!ok) return false;
  uint32_t* words = reinterpret_cast<uint32_t*>(s.Bk);
  auto src_of = [&](uint32_t f) -> const uint32_t* {
    uint32_t i = 0;
    if (f < rawbase) {
      const uint32_t it = f >> 2;
      while (i + 1u < G && ib[i + 1] <= it) ++i;
      return res_rec(a, b, i) + 4u * (it - ib[i]) + (f & 3u);
    }
    const uint32_t r = (f - rawbase) / kResK;
    while (i + 1u < G && rb[i + 1] <= r) ++i;
    return res_rec(a, b, i) + kResRawOff + kResK * (r - rb[i]) + (f - rawbase) % kResK;
  };
  for (uint32_t f0 = 0; f0 < nw; f0 += 4u * kThreads) {
    uint32_t wv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t f = f0 + t + (uint32_t)q * kThreads;
      wv[q] = f < nw ? *src_of(f) : 0u;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t f = f0 + t + (uint32_t)q * kThreads;
      if (f < nw) words[f] = wv[q];
    }
  }
  __syncthreads();
  *nit_out = nit;
  *rawbase_out = rawbase;
  return true;
}

// Walk of the gathered records on wave 0 from a running sum of 0.
//  sum mode (FIND false): the exact total; starts[i] (LDS) receives the exact
//    running sum at the start of slice i.
//  find mode: the first element whose running sum exceeds r (strictly,
//    sampling.rs:1008-1011); it must lie in a raw (the records made every
//    thread that may hold it uncertain).
// Results in s.misc_u / s.red_f: [0] good, [1] found, [2] item, [3] element
// in the raw; red_f[0] final or hit sum, red_f[1] the sum before the hit.
template <bool FIND>
__device__ __forceinline__ void res_walk_at(uint32_t G, uint32_t nit, uint32_t rawbase, float r,
                                            const uint32_t* words, Smem& s,
                                            float* starts = nullptr) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t* ib = s.H0;
  const uint32_t* rb = s.H0 + 32;
  const uint4* items = reinterpret_cast<const uint4*>(words);
  const float* raws = reinterpret_cast<const float*>(words + rawbase);
  uint32_t cb = 0u;
  uint32_t good = 1, found = 0, hit_k = 0, hit_j = 0, before = 0u;
  uint32_t ns = 0;  // next slice whose start is still to be recorded
  for (uint32_t k0 = 0; k0 < nit && good && !found; k0 += 64u) {
    const uint32_t k = k0 + lane;
    uint4 it = make_uint4(0u, 0u, 0u, kNoRaw);
    uint32_t roff = kNoRaw;
    if (k < nit) {
      it = items[k];
      if (it.w != kNoRaw) {
        uint32_t i = 0;
        while (i + 1u < G && ib[i + 1] <= k) ++i;
        roff = kResK * (rb[i] + (it.w & 0xffffu));
      }
    }
    const uint32_t cnt = min(64u, nit - k0);
    for (uint32_t q = 0; q < cnt; ++q) {
      if (!FIND && starts) {
        while (ns < G && ib[ns] <= k0 + q) {
          if (lane == 0) starts[ns] = __uint_as_float(cb);
          ++ns;
        }
      }
      const uint32_t bin = (uint32_t)__builtin_amdgcn_readlane((int)it.x, (int)q);
      const uint32_t a0 = (uint32_t)__builtin_amdgcn_readlane((int)it.y, (int)q);
      const uint32_t a1 = (uint32_t)__builtin_amdgcn_readlane((int)it.z, (int)q);
      const uint32_t ro = (uint32_t)__builtin_amdgcn_readlane((int)roff, (int)q);
      const uint32_t inc = (cb & 1u) ? a1 : a0;
      if (ro == kNoRaw) {
        if ((cb & 0xff800000u) == bin && inc < kSat && cb + inc < bin + 0x00800000u) {
          // a run: the crossing cannot lie in it
          if (FIND && r < __uint_as_float(cb + inc)) {
            good = 0;
            break;
          }
          cb += inc;
        } else {
          good = 0;
          break;
        }
        continue;
      }
      // an uncertain thread: its map when the exact sum is inside its binade
      // and stays there (and, searching, stays at or below r), else its raw
      // summands from the exact start
      if ((cb & 0xff800000u) == bin && inc < kSat && cb + inc < bin + 0x00800000u &&
          !(FIND && r < __uint_as_float(cb + inc))) {
        cb += inc;
        continue;
      }
      const float4* r4 = reinterpret_cast<const float4*>(raws + ro);
      float4 f[kResK / 4];
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) f[m] = r4[m];
      float c = __uint_as_float(cb);
      uint32_t hj = kResK;
      float cbef = c;
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) {
        const float xq[4] = {f[m].x, f[m].y, f[m].z, f[m].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float y = __fadd_rn(c, xq[u]);
          if (FIND && hj == kResK && r < y) {
            hj = 4u * (uint32_t)m + (uint32_t)u;
            cbef = c;
          }
          c = y;
        }
      }
      if (FIND && hj < kResK) {
        // recompute the hit sum (the loop ran past it)
        const float hit = __fadd_rn(cbef, reinterpret_cast<const float*>(r4)[hj]);
        found = 1;
        hit_k = k0 + q;
        hit_j = hj;
        before = (uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(cbef));
        cb = (uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(hit));
        break;
      }
      cb = (uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(c));
    }
  }
  if (!FIND && good && starts) {
    while (ns < G) {
      if (lane == 0) starts[ns] = __uint_as_float(cb);
      ++ns;
    }
  }
  if (lane == 0) {
    s.misc_u[0] = good;
    s.misc_u[1] = found;
    s.misc_u[2] = hit_k;
    s.misc_u[3] = hit_j;
    s.red_f[0] = __uint_as_float(cb);
    s.red_f[1] = __uint_as_float(before);
  }
}

// The S1 walk of res_walk_at (sum mode) arranged for latency: every lane
// loads its item of the current 64 (and the raw summands of an uncertain
// thread) up front, and the items are applied 8 at a time without a taken
// branch: a run, or an uncertain thread whose map applies, is one parity
// select and one add with its checks; only an uncertain thread that must be
// replayed leaves the straight line, and is replayed by all lanes at once,
// each on its own item's summands from the same exact start, lane q's
// result being the one kept. Same results and outputs as res_walk_at<false>
// without slice starts; failed checks accumulate into a flag tested once per
// 64 items.
__device__ __forceinline__ void res_walk_sum(uint32_t G, uint32_t nit, uint32_t rawbase,
                                             const uint32_t* words, Smem& s) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t* ib = s.H0;
  const uint32_t* rb = s.H0 + 32;
  const uint4* items = reinterpret_cast<const uint4*>(words);
  const float* raws = reinterpret_cast<const float*>(words + rawbase);
  uint32_t cb = 0u, bad = 0u;
  for (uint32_t k0 = 0; k0 < nit; k0 += 64u) {
    const uint32_t k = k0 + lane;
    uint4 it = make_uint4(0u, 0u, 0u, kNoRaw);
    uint32_t roff = kNoRaw;
    if (k < nit) {
      it = items[k];
      if (it.w != kNoRaw) {
        uint32_t i = 0;
        while (i + 1u < G && ib[i + 1] <= k) ++i;
        roff = kResK * (rb[i] + (it.w & 0xffffu));
      }
    }
    float xr[kResK];
    {
      const float4* r4 = reinterpret_cast<const float4*>(raws + (roff == kNoRaw ? 0u : roff));
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) {
        const float4 f = roff == kNoRaw ? make_float4(0.f, 0.f, 0.f, 0.f) : r4[m];
        xr[4 * m] = f.x;
        xr[4 * m + 1] = f.y;
        xr[4 * m + 2] = f.z;
        xr[4 * m + 3] = f.w;
      }
    }
    LUMEN_TICK("wk_loaded", LUMEN_TIMING_ROW);
    const uint32_t cnt = min(64u, nit - k0);
    for (uint32_t q0 = 0; q0 < cnt; q0 += 8u) {
#pragma unroll
      for (uint32_t u = 0; u < 8u; ++u) {
        const uint32_t q = q0 + u;
        const bool valid = q < cnt;
        const uint32_t bin = (uint32_t)__builtin_amdgcn_readlane((int)it.x, (int)q);
        const uint32_t a0 = (uint32_t)__builtin_amdgcn_readlane((int)it.y, (int)q);
        const uint32_t a1 = (uint32_t)__builtin_amdgcn_readlane((int)it.z, (int)q);
        const uint32_t ro = (uint32_t)__builtin_amdgcn_readlane((int)roff, (int)q);
        const uint32_t inc = (cb & 1u) ? a1 : a0;
        // the map applies: the exact sum is inside its binade and stays there
        const bool fits = (cb & 0xff800000u) == bin && inc < kSat && cb + inc < bin + 0x00800000u;
        // a run cannot hold a binade change: a map that does not apply fails
        bad |= (valid && ro == kNoRaw && !fits) ? 1u : 0u;
        cb = (valid && fits) ? cb + inc : cb;
        if (__builtin_expect(valid && ro != kNoRaw && !fits, 0)) {
          // an uncertain thread replayed from the exact start
          float c = __uint_as_float(cb);
#pragma unroll
          for (int j = 0; j < (int)kResK; ++j) c = __fadd_rn(c, xr[j]);
          cb = (uint32_t)__builtin_amdgcn_readlane(__float_as_int(c), (int)q);
        }
      }
    }
    LUMEN_TICK("wk_batch", LUMEN_TIMING_ROW);
    if (bad) break;
  }
  if (lane == 0) {
    s.misc_u[0] = bad ? 0u : 1u;
    s.red_f[0] = __uint_as_float(cb);
  }
}

// res_walk_at over the records gathered into s.Bk (res_gather).
template <bool FIND>
__device__ __forceinline__ void res_walk(uint32_t G, uint32_t nit, uint32_t rawbase, float r,
                                         float* starts, Smem& s) {
  res_walk_at<FIND>(G, nit, rawbase, r, reinterpret_cast<const uint32_t*>(s.Bk), s, starts);
}

// Loads virtual slice sc into x (thread t: elements 32t .. 32t+31) with the
// penalties applied (sampling.rs:881-900, each history id once). The loads
// v must have been issued for sc (res_issue).
template <bool BF16>
__device__ __forceinline__ void res_load(const KernelArgs& a, int b, const RowParams& P,
                                         const Row& row, Slice sc, bool pen,
                                         const float (&v)[8][4], float (&x)[kResK], Smem& s) {
  const uint32_t t = threadIdx.x;
  const bool tail = res_has_tail(row, sc);
  res_transpose(v, x, s, pen || tail, [&](float* L) {
    if (tail) {
      res_tail(row, sc, L);
      if (pen) __syncthreads();
    }
    if (!pen) return;
    const uint32_t h0 = a.hist_off[b], h1 = hist_hi(a, b);
    for (uint32_t j = h0 + t; j < h1; j += kThreads) {
      const uint32_t id = a.hist_ids[j];
      if (id >= sc.lo && id < sc.hi) {
        float& y = L[res_slot(id - sc.lo)];
        y = penalize(y, a.hist_cnt[j], P);
      }
    }
  });
}

// Chunks per workgroup of a register-resident row with G workgroups: the
// fewest q (at most 4, G * q <= kMaxSlices) whose G * q virtual slices each
// fit kResSlice logits; 0 when none does.
__device__ __forceinline__ uint32_t res_chunks(uint32_t V, uint32_t G) {
  for (uint32_t q = 1; q <= 4u && G * q <= (uint32_t)kMaxSlices; ++q)
    if ((((V + G * q - 1u) / (G * q) + 15u) & ~15u) <= kResSlice) return q;
  return 0u;
}

// The second-to-last workgroup of a split top-p row to arrive: it waits for
// the last (every slice's records are then complete), walks the records of
// the Gv virtual slices to the exact softmax sum S1 and publishes it in the
// row's block (unused0), releasing it by raising the spin barrier from G to
// 2G. On any failure it sets a status bit instead; it always releases, so
// the finisher never waits past the timeout.
__device__ __forceinline__ void res_s1_walker(const KernelArgs& a, int b, uint32_t G, uint32_t Gv,
                                              Smem& s) {
  RowWs& ws = a.ws[b];
  LUMEN_TICK("w_start", b);
  const bool ok = wg_wait_geq(a, &ws.arrive, G, s);
  LUMEN_TICK("w_waited", b);
  uint32_t nit = 0, rawbase = 0;
  bool good = ok && __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u &&
              res_gather(a, b, Gv, s, &nit, &rawbase);
  LUMEN_TICK("w_gathered", b);
  if (good) {
    if (threadIdx.x < 64u) res_walk_sum(Gv, nit, rawbase, reinterpret_cast<const uint32_t*>(s.Bk), s);
    __syncthreads();
    good = s.misc_u[0] != 0u;
  }
  LUMEN_TICK("w_walked", b);
  if (threadIdx.x == 0) {
    if (good)
      ws.unused0 = __float_as_uint(s.red_f[0]);
    else
      __hip_atomic_fetch_or(&ws.status, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t old = __hip_atomic_fetch_add(&ws.bar, G, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old >= kAbandoned) {
      // the finisher stopped waiting (a timed-out wait) and went on alone;
      // this release is the row's last access to its block, so the walker
      // restores it for the next call
      ws.arrive = 0;
      ws.bar = 0;
      ws.cand_n = 0;
      ws.status = 0;
    }
  }
}

// Top-p (no top-k) over register-resident slices; see the header comment.
// Workgroup sl owns the q virtual slices sl*q .. sl*q+q-1 of the row's G*q;
// with q > 1 each is read again (from cache) in phase B.
template <bool BF16, bool MULTI>
__device__ __forceinline__ void topp_res(const KernelArgs& a, int b, uint32_t sl, uint32_t G,
                                         uint32_t q_rt, Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t q = MULTI ? q_rt : 1u;  // one chunk: straight-line code
  const uint32_t V = a.vocab, t = threadIdx.x, lane = t & 63u;
  const uint32_t Gv = G * q;
  const bool pen = (P.flags & kPen) && hist_hi(a, b) > a.hist_off[b];
  LUMEN_TICK("r_start", b);

  // ---- phase A ----
  float smp[4];
  res_sample_issue(row, smp);
  float v[8][4];
  res_issue<BF16>(row, slice_bounds(V, Gv, sl * q), v);
  const uint32_t tau = res_sample_select(smp, V, kResCandTarget, s);
  const float tv = tau ? key2f(tau) : kNegInf;
  float x[kResK];
  uint32_t cmask = 0, coff = 0;
  for (uint32_t j = 0; j < q; ++j) {
    const uint32_t vs = sl * q + j;
    const Slice sc = slice_bounds(V, Gv, vs);
    if (j > 0) res_issue<BF16>(row, sc, v);
    res_load<BF16>(a, b, P, row, sc, pen, v, x, s);
    LUMEN_TICK("r_loaded", b);
    if (a.pen_out) {
      float* po = a.pen_out + (uint64_t)b * V + sc.lo + t * kResK;
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k)
        if (sc.lo + t * kResK + (uint32_t)k < sc.hi) po[k] = x[k];
    }
    float mt = kNegInf;
    cmask = 0;
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k) {
      mt = op_maxl(mt, x[k]);
      cmask |= (x[k] >= tv ? 1u : 0u) << k;  // NaN never qualifies
    }
    uint32_t ctot;
    coff = block_excl_scan_u32((uint32_t)__popc(cmask), s, &ctot);
    const float ms = block_maxl(mt, s);
    float et = 0.f;  // NaN in the slice makes the estimate NaN
    if (ms != kNegInf) {
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k) et += __expf(x[k] - ms);
    }
    const double es = block_sum_f64((double)et, s);
    if (t == 0) {
      ws.part_max[vs] = ms;
      ws.part_e[vs] = es;
      ws.part_cn[vs] = ctot;
    }
  }
  LUMEN_TICK("r_phaseA", b);
  wg_arrive(&ws.bar, 0xffffffffu, s);
  const bool ok = wg_wait_geq(a, &ws.bar, G, s);
  if (!ok && t == 0) __hip_atomic_fetch_or(&ws.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  LUMEN_TICK("r_barrier", b);

  // ---- phase B ----
  // the last chunk first: its logits are still in registers
  constexpr uint32_t kBins = (uint32_t)kMassBins;
  bool bad = false;
  float m1 = 0.f;
  for (uint32_t jj = 0; jj < q; ++jj) {
    const uint32_t j = q - 1u - jj;
    const uint32_t vs = sl * q + j;
    const Slice sc = slice_bounds(V, Gv, vs);
    if (jj > 0) {
      res_issue<BF16>(row, sc, v);
      res_load<BF16>(a, b, P, row, sc, pen, v, x, s);
      cmask = 0;
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k) cmask |= (x[k] >= tv ? 1u : 0u) << k;
      uint32_t ctot;
      coff = block_excl_scan_u32((uint32_t)__popc(cmask), s, &ctot);
    }
    // the row's values, one virtual slice per lane of wave 0, in one round trip
    float* rowv = reinterpret_cast<float*>(s.H0 + 1024);  // [0] m1, [2..3] p_slice (f64)
    uint32_t* rowu = s.H0 + 1032;                        // [0] ncand, [1] bad, [2] candidate base
    if (t < 64u) {
      const bool in = lane < Gv;
      const float mi = in ? ws.part_max[lane] : kNegInf;
      const double ei = in ? ws.part_e[lane] : 0.0;
      const uint32_t ci = in ? ws.part_cn[lane] : 0u;
      const float m1w = wave_reduce(mi, kNegInf, op_maxl);
      const double term = (lane < vs && mi != kNegInf) ? ei * exp((double)mi - (double)m1w) : 0.0;
      const double ps = wave_reduce(term, 0.0, [](double l, double r) { return l + r; });
      const uint32_t cin = wave_scan_incl(ci, 0u, op_add_u32);
      const uint32_t nc = wave_read(cin, 63);
      const bool nan = __ballot(in && !(ei == ei)) != 0ull;
      // an earlier slice holding the maximum has added exp(0) = 1
      const bool one = __ballot(lane < vs && mi == m1w) != 0ull;
      if (lane == vs) rowu[2] = cin - ci;
      if (lane == 0) {
        rowv[0] = m1w;
        rowv[1] = one ? 1.f : 0.f;
        *reinterpret_cast<double*>(rowv + 2) = ps;
        rowu[0] = nc;
        rowu[1] = (nan || !is_finite(m1w) || nc > (uint32_t)kCandCap) ? 1u : 0u;
      }
    }
    __syncthreads();
    m1 = rowv[0];
    const double p_slice = *reinterpret_cast<const double*>(rowv + 2);
    const float lb_slice = rowv[1];
    const uint32_t cbase = rowu[2];
    bad = !ok || rowu[1] != 0u;
    __syncthreads();
    if (bad) break;
    float* hg = a.hist + ((uint64_t)b * kMaxSlices + vs) * kMassBins;
    // Candidates in index order at the slice's block: (logit bits << 32) |
    // id, and exp(v - m1) in the second half of the buffer; their exp-mass
    // binned by the bits of exp(v - m1) into this slice's histogram (bin 0
    // holds the largest values). The LDS copy of the slice is indexed by
    // the bits of cmask: first the logits, then the summands.
    float* L = res_buf(s);
    float* hl = reinterpret_cast<float*>(s.H0 + 1536);  // [kBins]
    float* Lt = L + t * kResPitch;
    uint32_t* cande = reinterpret_cast<uint32_t*>(cand + kCandCap);
    {
      uint32_t m = cmask;
      uint32_t o = cbase + coff;
      while (m) {
        const uint32_t k = (uint32_t)(__ffs(m) - 1);
        m &= m - 1u;
        if (o < (uint32_t)kCandCap) cand[o] = ((uint64_t)__float_as_uint(Lt[k]) << 32) | (sc.lo + t * kResK + k);
        ++o;
      }
    }
    for (uint32_t i = t; i < kBins; i += kThreads) hl[i] = 0.f;
    // the exact summands exp(v - m1), into this thread's LDS row
#pragma unroll
    for (int qq = 0; qq < (int)kResK / 4; ++qq) {
      const float e0 = expf_glibc_nonpos(__fsub_rn(x[4 * qq], m1));
      const float e1 = expf_glibc_nonpos(__fsub_rn(x[4 * qq + 1], m1));
      const float e2 = expf_glibc_nonpos(__fsub_rn(x[4 * qq + 2], m1));
      const float e3 = expf_glibc_nonpos(__fsub_rn(x[4 * qq + 3], m1));
      *reinterpret_cast<float4*>(Lt + 4 * qq) = make_float4(e0, e1, e2, e3);
    }
    LUMEN_TICK("rb_exps", b);
    const uint32_t bsh = res_bin_shift(tau ? expf_glibc_nonpos(__fsub_rn(tv, m1)) : 0.f);
    __syncthreads();  // the histogram is cleared
    {
      uint32_t m = cmask;
      uint32_t o = cbase + coff;
      while (m) {
        const uint32_t k = (uint32_t)(__ffs(m) - 1);
        m &= m - 1u;
        const float ek = Lt[k];
        if (o < (uint32_t)kCandCap) cande[o] = __float_as_uint(ek);
        ++o;
        atomicAdd(&hl[res_bin(ek, bsh)], ek);
      }
    }
    __syncthreads();
    for (uint32_t i = t; i < kBins; i += kThreads) hg[i] = hl[i];
    LUMEN_TICK("rb_hist", b);
    const uint32_t nthr = (sc.hi - sc.lo + kResK - 1u) / kResK;
    const RecCount rc = res_record(Lt, p_slice, sc.lo, nthr, res_rec(a, b, vs), s, 0.f, lb_slice);
    if (t == 0) {
      ws.part_nrec[vs] = rc.ok ? rc.items : 0xffffffffu;
      ws.part_nraw[vs] = rc.raws;
    }
    __syncthreads();
  }
  const uint32_t ncand = s.H0[1032];
  if (bad && t == 0) __hip_atomic_fetch_or(&ws.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  LUMEN_TICK("r_phaseB", b);
  const uint32_t arr = wg_arrive(&ws.arrive, G - 1u, s);
  if (arr == G - 2u) {
    res_s1_walker(a, b, G, Gv, s);
    return;
  }
  if (arr != G - 1u) return;
  LUMEN_TICK("r_finisher", b);
  const uint32_t Gr = G;
  G = Gv;  // from here on, slices are the virtual slices

  // ---- finisher ----
  // The walker (res_s1_walker) computes the exact S1 meanwhile. Until it
  // arrives, the window is planned with an upper bound of S1 and sorted by
  // e = exp(v - m1), which orders the candidates as p = e / S1 does except
  // among equal p (repaired below).
  bad = bad || __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
  constexpr uint32_t kPer = (uint32_t)kCandCap / (uint32_t)kThreads;
  // gather, every load issued before any store: the summed mass histogram
  // into s.H, the candidates (logit bits << 32) | id into list A, and the
  // upper bound of S1 from the slices' estimates
  uint32_t ej[kPer];  // exp(v - m1) of candidates kPer*t .. kPer*t + kPer-1
  {
    uint64_t cv[kPer];
    const uint32_t* cande = reinterpret_cast<const uint32_t*>(cand + kCandCap);
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q) {
      const uint32_t f = t + (uint32_t)q * kThreads;
      cv[q] = f < ncand ? cand[f] : 0ull;
    }
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q) {
      const uint32_t f = kPer * t + (uint32_t)q;
      ej[q] = f < ncand ? cande[f] : 0u;
    }
    float hs = 0.f;
    if (t < kBins) {
      const float* hp = a.hist + (uint64_t)b * kMaxSlices * kMassBins + t;
      float hv[kMaxSlices];
#pragma unroll
      for (uint32_t i = 0; i < (uint32_t)kMaxSlices; ++i) hv[i] = i < G ? hp[(uint64_t)i * kMassBins] : 0.f;
#pragma unroll
      for (uint32_t i = 0; i < (uint32_t)kMaxSlices; ++i) hs += hv[i];
    }
    if (t < 64u) {
      const bool in = lane < G;
      const float mi = in ? ws.part_max[lane] : kNegInf;
      const double ei = in ? ws.part_e[lane] : 0.0;
      const double term = (in && mi != kNegInf) ? ei * exp((double)mi - (double)m1) : 0.0;
      const double est = wave_reduce(term, 0.0, [](double l, double r) { return l + r; });
      // the sequential f32 sum is within ~1e-3 of the estimate; the window's
      // margin covers that, and the checks after the walk make it exact
      if (lane == 0) s.red_f[2] = (float)est;
    }
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q) {
      const uint32_t f = t + (uint32_t)q * kThreads;
      if (f < ncand) s.A[f] = cv[q];
    }
    if (t < kBins) reinterpret_cast<float*>(s.H)[t] = hs;
    __syncthreads();
  }
  LUMEN_TICK("r_gathered", b);
  const float S1_hi = s.red_f[2];
  // Window: the lowest mass bin (from the top) whose running mass reaches
  // top_p * S1 with a margin, plus one spare bin, bounds the window from
  // below at e_edge. Every logit >= tv is a candidate, so every token with
  // e > e(tv) is one: the window keeps only e > e(tv).
  const float e_tv = tau ? expf_glibc_nonpos(__fsub_rn(tv, m1)) : 0.f;
  const uint32_t bsh = res_bin_shift(e_tv);
  if (t < 64u) {
    const float* hm = reinterpret_cast<const float*>(s.H);
    const float target = fminf(__fmul_rn(__fmul_rn(P.top_p, S1_hi), 1.004f), S1_hi);
    float run = 0.f;
    uint32_t hit = kBins;
    for (uint32_t base = 0; base < kBins && hit == kBins; base += 64u) {
      const float m = wave_scan_incl(hm[base + t], 0.f, [](float l, float r) { return l + r; });
      const unsigned long long hmsk = __ballot(run + m >= target);
      if (hmsk) hit = base + (uint32_t)(__ffsll((long long)hmsk) - 1);
      run += wave_read(m, 63);
    }
    if (t == 0) s.misc_u[2] = hit;
  }
  __syncthreads();
  float e_lo;
  {
    const uint32_t hit = s.misc_u[2];
    e_lo = fmaxf(hit + 1u < kBins ? res_bin_lo(hit + 1u, bsh) : 0.f, e_tv);
  }
  // the window's sort keys (~e << 32) | f in list B (f, the candidate's
  // position, orders like its id); candidates 8t .. 8t+7 per thread
  // (contiguous, so one block scan keeps index order)
  uint32_t wmask = 0;
  {
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q) {
      const float e = __uint_as_float(ej[q]);
      wmask |= (e > e_tv && e >= e_lo && e > 0.f ? 1u : 0u) << q;
    }
  }
  uint32_t nw;
  uint32_t wo = block_excl_scan_u32((uint32_t)__popc(wmask), s, &nw);
#pragma unroll
  for (int q = 0; q < (int)kPer; ++q)
    if ((wmask >> q) & 1u) s.Bk[wo++] = ((uint64_t)(~ej[q]) << 32) | (kPer * t + (uint32_t)q);
  __syncthreads();
  LUMEN_TICK("r_window", b);
  // a window over half of list B sorts through list A (the candidates are
  // then read again from the row's buffer)
  const bool cand_lds = nw <= kResWindowCap;
  uint64_t* const wtmp = cand_lds ? s.Bk + kResWindowCap : s.A;
  if (!bad && nw > 0u) {
    const uint32_t khi = ~__float_as_uint(1.0f), klo = ~__float_as_uint(e_lo);
    const uint64_t hint = ((uint64_t)(khi ^ klo) << 32) | span_mask(kCandCap);
    sort_u64_asc(s.Bk, nw, wtmp, s, hint);
  }
  LUMEN_TICK("r_sorted", b);
  // S1 from the walker (always released, also on failure)
  const bool got = wg_wait_geq(a, &ws.bar, 2u * Gr, s);
  if (t == 0) {
    if (got) {
      s.misc_u[2] = __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s.red_f[0] = __uint_as_float(ws.unused0);
    } else {
      // giving up on the walker: whichever of the two touches the row's
      // block last restores it. A walker that has not released yet finds
      // the mark and resets; otherwise this workgroup does, as usual. After
      // the mark this workgroup no longer reads or writes the block.
      const uint32_t old =
          __hip_atomic_fetch_add(&ws.bar, kAbandoned, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if (old < 2u * Gr) s.finisher = 0u;
      s.misc_u[2] = 1u;
    }
  }
  __syncthreads();
  const float S1 = s.red_f[0];
  bad = bad || !got || s.misc_u[2] != 0u;
  __syncthreads();
  LUMEN_TICK("r_S1", b);
  if (bad || nw == 0u) {
    row_single<false>(a, b, s);
    return;
  }
  // the keys as p = e / S1 (monotone in e, so the order holds), then the
  // order among equal p repaired: (p desc, id asc) is the reference's
  // stable sort (sampling.rs:952)
  {
    uint32_t swap = 0;
    for (uint32_t j = t; j < nw; j += kThreads) {
      const uint64_t k = s.Bk[j];
      const float p = __fdiv_rn(__uint_as_float(~(uint32_t)(k >> 32)), S1);
      s.Bk[j] = ((uint64_t)(~__float_as_uint(p)) << 32) | (uint32_t)k;
    }
    __syncthreads();
    LUMEN_TICK("x_p", b);
    for (uint32_t j = t; j + 1u < nw; j += kThreads) swap |= s.Bk[j] > s.Bk[j + 1u] ? 1u : 0u;
    swap = block_or_u32(swap, s);
    if (swap) sort_u64_asc(s.Bk, nw, wtmp, s);
    LUMEN_TICK(swap ? "x_resorted" : "x_inorder", b);
  }
  const float p_x = __fdiv_rn(e_lo, S1);  // every token outside the window has p <= p_x
  const EcssResult wk = list_ecss_block(
      nw, [&](uint32_t j) { return __uint_as_float(~(uint32_t)(s.Bk[j] >> 32)); }, kEcssFindGe, P.top_p, 0.f, s);
  LUMEN_TICK("r_crossing", b);
  // the crossing's p must exceed every p outside the window, so no token
  // outside it ties with (or precedes) the kept set
  if (!wk.found || !(__uint_as_float(~(uint32_t)(s.Bk[wk.pos] >> 32)) > p_x)) {
    row_single<false>(a, b, s);
    return;
  }
  // the nucleus: the sorted window's first wk.pos + 1 entries, marked in a
  // bitmap by candidate position, then compacted in index order into list A
  // as (idx << 32) | key
  uint32_t* kbits = s.H;  // [kCandCap / 32]
  for (uint32_t i = t; i < (uint32_t)kCandCap / 32u; i += kThreads) kbits[i] = 0u;
  __syncthreads();
  for (uint32_t j = t; j <= (uint32_t)wk.pos; j += kThreads) {
    const uint32_t f = (uint32_t)s.Bk[j];
    atomicOr(&kbits[f >> 5], 1u << (f & 31u));
  }
  __syncthreads();
  // at T = 1 without min-p the final softmax sums the kept values' own
  // exp(v - m1): they travel in the list in place of the keys
  const bool pre_exp = P.inv_temp == 1.0f && !(P.flags & kMinP);
  uint32_t nk;
  {
    const uint32_t kmask = (kbits[t >> 2] >> (8u * (t & 3u))) & 0xffu;  // candidates 8t .. 8t+7
    uint64_t cv[kPer];
    uint32_t ev[kPer];
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q) {
      const bool in = (kmask >> q) & 1u;
      cv[q] = in ? (cand_lds ? s.A[kPer * t + (uint32_t)q] : cand[kPer * t + (uint32_t)q]) : 0ull;
      ev[q] = in && pre_exp ? ej[q] : 0u;
    }
    uint32_t ko = block_excl_scan_u32((uint32_t)__popc(kmask), s, &nk);
#pragma unroll
    for (int q = 0; q < (int)kPer; ++q)
      if ((kmask >> q) & 1u)
        s.A[ko++] = ((uint64_t)(uint32_t)cv[q] << 32) |
                    (pre_exp ? ev[q] : tkey(__uint_as_float((uint32_t)(cv[q] >> 32))));
    __syncthreads();
  }
  RowTrace tr;
  init_trace(tr, V);
  tr.path = 4u | 2u;
  tr.passes = 1;
  tr.windows = 1;
  tr.topp_sum = S1;
  tr.topp_kept = (uint32_t)wk.pos + 1u;
  tr.topp_cum = wk.c;
  tr.pad[0] = 0;
  tr.pad[1] = ncand | (nw << 16);
  LUMEN_TICK("r_kept", b);
  // the nucleus holds the row maximum m1 (the largest p)
  const uint32_t tok = final_on_list(a, P, nk, rdraw, s, tr, m1, pre_exp);
  LUMEN_TICK("r_final", b);
  write_result(a, b, tok, tr);
}

}  // namespace lumen
