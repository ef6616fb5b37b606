// Exact sequential f32 sums over a whole row by one workgroup (included by
// sampler_kernels.hip after resident.h; used by the row_single of
// lumen_sample_rows_single).
//
// The reference sums in index order one element at a time: the softmax sum
// (crates/lumen-runtime/src/sampling.rs:216-221) and the inverse-CDF walk
// (:1003-1014). row_rec_sum reproduces that sum, or finds the walk's first
// element whose running sum exceeds a draw, with the record method of the
// register-resident paths:
//  - the row is cut into blocks of kResSlice elements; in each block thread t
//    holds the 32 contiguous summands 32t .. 32t+31 in registers;
//  - each block writes its record (runs of threads whose binade the f64
//    estimate fixes, as parity maps, and the raw summands of the others) to
//    the row's own record area (KernelArgs::rsum), one area per block;
//  - one walk on wave 0 over all records gives the exact result.
// Its LDS needs are the record walk's (s.H), the class codes (s.H0) and the
// scan scratch, so it runs beside the bf16 value counts held in lists A and
// B. A walk that fails, or records that do not fit, return ok = false and
// the caller takes the chunked method.
#pragma once

namespace lumen {

// Block blk's record area of row b.
__device__ __forceinline__ uint32_t* rs_rec(const KernelArgs& a, int b, uint32_t blk) {
  return a.rsum + ((uint64_t)b * kMaxSlices + blk) * kRsBlockWords;
}

// res_record for summands held in registers, into an area of kRsBlockWords
// words (at most kRsItemCap items, kRsRawCap raws); also returns the
// block's f64 total (the estimate of the next block's start). Three
// barriers: the f64 prefix, the neighbours' class codes at wave edges, and
// the wave totals of the segmented run scan and of the item / raw counts
// (each wave combines the totals of the waves before it itself). Its LDS
// scratch (s.H0[0 .. 191]) is rewritten only after the next two barriers,
// so consecutive calls need none in between.
template <bool FIND>
__device__ __forceinline__ RecCount res_record_regs(const float (&e)[kResK], double p_slice,
                                                    uint32_t pos0, uint32_t nthr, uint32_t* rec,
                                                    Smem& s, float probe, double* tot_out) {
  const uint32_t t = threadIdx.x, lane = t & 63u, w = t >> 6;
  const bool live = t < nthr;
  // the thread's total, pairwise in f32: relative error below 3e-7, far
  // inside the margins below
  float q8[kResK / 8];
#pragma unroll
  for (int m = 0; m < (int)kResK / 8; ++m)
    q8[m] = ((e[8 * m] + e[8 * m + 1]) + (e[8 * m + 2] + e[8 * m + 3])) +
            ((e[8 * m + 4] + e[8 * m + 5]) + (e[8 * m + 6] + e[8 * m + 7]));
  const double d = (double)((q8[0] + q8[1]) + (q8[2] + q8[3]));
  // 1. f64 prefix of the thread totals: the estimated running sum at the
  // thread's start
  double* wt = reinterpret_cast<double*>(s.H0);  // [kWaves]
  const double dinc = wave_scan_incl(d, 0.0, [](double l, double r) { return l + r; });
  if (lane == 63u) wt[w] = dinc;
  __syncthreads();
  double pre = 0.0, tot = 0.0;
#pragma unroll
  for (uint32_t i = 0; i < (uint32_t)kWaves; ++i) {
    const double x = wt[i];
    if (i < w) pre += x;
    tot += x;
  }
  *tot_out = tot;
  const double P = p_slice + pre + (dinc - d);
  const double rel = 5e-5 + 4e-9 * (double)(pos0 + t * kResK + kResK);
  const uint32_t blo = est_binade(P * (1.0 - rel));
  const uint32_t bhi = est_binade((P + d) * (1.0 + rel));
  // a search: a thread whose running sum surely starts above the probe
  // cannot hold the hit and records nothing (a walk that then finds no hit
  // fails, and the caller takes the chunked method)
  const bool past = FIND && live && P * (1.0 - 1e-4) > (double)probe;
  const bool act = live && !past;
  bool unc = act && blo != bhi;
  // the probe's margin is the drift of a probability sum from its estimate
  // (the exact softmax sum divided out): observed up to ~3e-5 of it
  constexpr double kProbeRel = 1e-4;
  if (FIND)
    unc = unc || (act && P * (1.0 - kProbeRel) <= (double)probe && (double)probe <= (P + d) * (1.0 + kProbeRel));
  const uint32_t bin = unc ? est_binade(P + 0.5 * d) : blo;
  float y0 = __uint_as_float(bin), y1 = __uint_as_float(bin | 1u);
#pragma unroll
  for (int k = 0; k < (int)kResK; ++k) {
    y0 = __fadd_rn(y0, e[k]);
    y1 = __fadd_rn(y1, e[k]);
  }
  const uint32_t n0 = __float_as_uint(y0) - bin, n1 = __float_as_uint(y1) - (bin | 1u);
  const PMap own{n0 > kSat ? kSat : n0, n1 > kSat ? kSat : n1};
  // 2. class codes of the neighbours (runs are maximal spans of certain
  // threads in one binade)
  constexpr uint32_t kUnc = 1u, kDead = 2u;
  const uint32_t code = !act ? kDead : unc ? kUnc : bin;
  uint32_t* bc = s.H0 + 64;  // [kWaves][2]: first and last code of each wave
  if (lane == 0u) bc[2u * w] = code;
  if (lane == 63u) bc[2u * w + 1u] = code;
  __syncthreads();
  uint32_t prv = wave_shr1(code, kDead);
  if (lane == 0u) prv = w > 0u ? bc[2u * w - 1u] : kDead;
  uint32_t nxt = (uint32_t)__shfl_down((int)code, 1);
  if (lane == 63u) nxt = w + 1u < (uint32_t)kWaves ? bc[2u * w + 2u] : kDead;
  const bool head = act && (unc || prv != code);
  const bool last = act && !unc && nxt != code;
  const uint32_t packed = ((unc || last) ? 1u : 0u) | ((unc ? 1u : 0u) << 16);
  // 3. the segmented scan of the run maps and the scan of the item / raw
  // counts, wave by wave, then across the waves
  const SegVal id{0u, PMap{0u, 0u}};
  const SegVal sinc = wave_scan_incl(SegVal{head ? 1u : 0u, (act && !unc) ? own : PMap{0u, 0u}}, id,
                                     seg_combine);
  const uint32_t pinc = wave_scan_incl(packed, 0u, op_add_u32);
  uint32_t* st = s.H0 + 128;  // [kWaves][4]: head, a0, a1, count total
  if (lane == 63u) {
    st[4u * w] = sinc.head;
    st[4u * w + 1u] = sinc.m.a0;
    st[4u * w + 2u] = sinc.m.a1;
    st[4u * w + 3u] = pinc;
  }
  __syncthreads();
  SegVal spre = id;
  uint32_t ppre = 0, ptot = 0;
#pragma unroll
  for (uint32_t i = 0; i < (uint32_t)kWaves; ++i) {
    const SegVal x{st[4u * i], PMap{st[4u * i + 1u], st[4u * i + 2u]}};
    const uint32_t c = st[4u * i + 3u];
    if (i < w) {
      spre = seg_combine(spre, x);
      ppre += c;
    }
    ptot += c;
  }
  const SegVal inc = seg_combine(spre, sinc);
  const uint32_t pos = ppre + pinc - packed;
  RecCount rc{ptot & 0xffffu, ptot >> 16, true};
  if (rc.items > kRsItemCap || rc.raws > kRsRawCap) {
    rc.ok = false;
    return rc;
  }
  const uint32_t ip = pos & 0xffffu, rp = pos >> 16;
  if (unc) {
    gst(reinterpret_cast<u32x4*>(rec + 4u * ip), u32x4{bin, own.a0, own.a1, FIND ? rp | (t << 16) : rp});
    u32x4* raw = reinterpret_cast<u32x4*>(rec + kRsRawOff + kResK * rp);
#pragma unroll
    for (int m = 0; m < (int)kResK / 4; ++m)
      gst(raw + m, u32x4{__float_as_uint(e[4 * m]), __float_as_uint(e[4 * m + 1]),
                         __float_as_uint(e[4 * m + 2]), __float_as_uint(e[4 * m + 3])});
  } else if (last) {
    gst(reinterpret_cast<u32x4*>(rec + 4u * ip), u32x4{bin, inc.m.a0, inc.m.a1, kNoRaw});
  }
  return rc;
}

// Logits i0 .. i0+31 of the row (i0 a multiple of 32); past the row's end
// they read as -inf.
__device__ __forceinline__ void row_load32(const Row& row, uint32_t i0, float (&v)[kResK]) {
  if (i0 + kResK <= row.V && row.vec) {
    if (row.f) {
      const f32x4* p = reinterpret_cast<const f32x4*>(row.f + i0);
      f32x4 q[kResK / 4];
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) q[m] = gld(p + m);
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) {
        v[4 * m] = q[m].x;
        v[4 * m + 1] = q[m].y;
        v[4 * m + 2] = q[m].z;
        v[4 * m + 3] = q[m].w;
      }
    } else {
      const u16x4* p = reinterpret_cast<const u16x4*>(row.h + i0);
      u16x4 q[kResK / 4];
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) q[m] = gld(p + m);
#pragma unroll
      for (int m = 0; m < (int)kResK / 4; ++m) {
        v[4 * m] = __uint_as_float((uint32_t)q[m].x << 16);
        v[4 * m + 1] = __uint_as_float((uint32_t)q[m].y << 16);
        v[4 * m + 2] = __uint_as_float((uint32_t)q[m].z << 16);
        v[4 * m + 3] = __uint_as_float((uint32_t)q[m].w << 16);
      }
    }
  } else {
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k)
      v[k] = i0 + (uint32_t)k < row.V ? row.at(i0 + (uint32_t)k) : kNegInf;
  }
}

// The records of the G blocks gathered into s.H (at most 4096 words; ib, rb
// in s.H0 + [0, 64)); false when they do not fit.
__device__ __forceinline__ bool rec_gather_small(const KernelArgs& a, int b, uint32_t G,
                                                 const uint32_t* nrec, const uint32_t* nraw,
                                                 Smem& s, uint32_t* nit_out, uint32_t* rawbase_out) {
  const uint32_t t = threadIdx.x, lane = t & 63u;
  uint32_t* ib = s.H0;
  uint32_t* rb = s.H0 + 32;
  if (t < 64u) {
    const bool in = lane < G;
    const uint32_t ni = in ? nrec[lane] : 0u;
    const uint32_t nr = in ? nraw[lane] : 0u;
    const uint32_t ei = wave_scan_incl(ni, 0u, op_add_u32);
    const uint32_t er = wave_scan_incl(nr, 0u, op_add_u32);
    const uint32_t pi = wave_shr1(ei, 0u), pr = wave_shr1(er, 0u);
    if (lane <= G) {
      ib[lane] = pi;
      rb[lane] = pr;
    }
  }
  __syncthreads();
  const uint32_t nit = ib[G], nrw = rb[G];
  const uint32_t rawbase = 4u * nit;
  const uint32_t nw = rawbase + kResK * nrw;
  __syncthreads();
  if (nw > 4096u) return false;
  uint32_t* words = s.H;
  for (uint32_t f = t; f < nw; f += kThreads) {
    uint32_t i = 0;
    const uint32_t* src;
    if (f < rawbase) {
      const uint32_t it = f >> 2;
      while (i + 1u < G && ib[i + 1] <= it) ++i;
      src = rs_rec(a, b, i) + 4u * (it - ib[i]) + (f & 3u);
    } else {
      const uint32_t r = (f - rawbase) / kResK;
      while (i + 1u < G && rb[i + 1] <= r) ++i;
      src = rs_rec(a, b, i) + kRsRawOff + kResK * (r - rb[i]) + (f - rawbase) % kResK;
    }
    words[f] = gld(src);
  }
  __syncthreads();
  *nit_out = nit;
  *rawbase_out = rawbase;
  return true;
}

// The exact sequential sum of xf(i, v) over the row in index order (FIND
// false), or the first element whose running sum exceeds probe (FIND true:
// found, pos, the sums before and at it). The summands must be finite and
// >= 0. ok = false: the method could not finish (nothing is wrong), or the
// launch has no record area.
template <bool FIND, class XF>
__device__ __forceinline__ EcssResult row_rec_sum(const KernelArgs& a, int b, const Row& row,
                                                  XF&& xf, float probe, Smem& s, bool& ok) {
  const uint32_t V = row.V, t = threadIdx.x;
  const uint32_t nblk = (V + kResSlice - 1u) / kResSlice;
  EcssResult r{0.f, 0, -1, 0.f};
  ok = false;
  if (!a.rsum || nblk == 0u || nblk > (uint32_t)kMaxSlices) return r;
  uint32_t* nrec = s.H0 + 1040;  // [kMaxSlices]
  uint32_t* nraw = s.H0 + 1056;  // [kMaxSlices]
  double P = 0.0;
  bool fit = true;
  uint32_t nb = nblk;  // blocks recorded
  for (uint32_t blk = 0; blk < nblk; ++blk) {
    const uint32_t lo = blk * kResSlice;
    const uint32_t n = min(kResSlice, V - lo);
    float e[kResK];
    row_load32(row, lo + t * kResK, e);
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k) {
      const uint32_t i = lo + t * kResK + (uint32_t)k;
      e[k] = i < V ? xf(i, e[k]) : 0.f;
    }
    LUMEN_TICK("rr_x", b);
    double tot;
    const RecCount rc = res_record_regs<FIND>(e, P, lo, (n + kResK - 1u) / kResK, rs_rec(a, b, blk),
                                              s, probe, &tot);
    P += tot;
    LUMEN_TICK("rr_rec", b);
    if (t == 0) {
      nrec[blk] = rc.items;
      nraw[blk] = rc.raws;
    }
    fit = fit && rc.ok;
    // searching: once the running sum is surely above the probe where the
    // next block starts, the hit lies in the blocks recorded so far
    if (FIND && blk + 1u < nblk &&
        (double)probe < P * (1.0 - (5e-5 + 4e-9 * (double)(lo + n)))) {
      nb = blk + 1u;
      break;
    }
  }
  __syncthreads();
  uint32_t nit = 0, rawbase = 0;
  if (!fit || !rec_gather_small(a, b, nb, nrec, nraw, s, &nit, &rawbase)) return r;
  LUMEN_TICK("rr_gather", b);
  if (t < 64u) res_walk_at<FIND>(nb, nit, rawbase, probe, s.H, s);
  __syncthreads();
  LUMEN_TICK("rr_walk", b);
  const bool found = s.misc_u[1] != 0u;
  // a search must have found its hit (its records skip threads surely
  // past the probe, and it may have stopped early)
  ok = s.misc_u[0] != 0u && (found || !FIND);
  const uint32_t hk = s.misc_u[2], hj = s.misc_u[3];
  r.c = s.red_f[0];
  r.before = s.red_f[1];
  r.found = found ? 1 : 0;
  if (found) {
    const uint32_t* ib = s.H0;
    uint32_t i = 0;
    while (i + 1u < nb && ib[i + 1] <= hk) ++i;
    const uint32_t th = (s.H[4u * hk + 3u] >> 16) & 0x3ffu;
    r.pos = (int)(i * kResSlice + th * kResK + hj);
  }
  __syncthreads();
  return r;
}

}  // namespace lumen
