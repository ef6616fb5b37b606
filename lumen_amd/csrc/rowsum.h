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
//    row's records in LDS (s.H: items from the bottom, raws from the top);
//  - one walk on wave 0 over all records gives the exact result.
// Its LDS needs are the record walk's (s.H), the class codes (s.H0) and the
// scan scratch, so it runs beside the bf16 value counts held in lists A and
// B. A walk that fails, or records that do not fit, return ok = false and
// the caller takes the chunked method.
#pragma once

namespace lumen {

// LDS words of a row's records (all of s.H).
constexpr uint32_t kRsLdsWords = 4096;

// res_record for summands held in registers, into the row's records in s.H
// (at most kRsItemCap items and kRsRawCap raws per block, kRsLdsWords words
// per row; ibase / rbase: the items and raws before this block); also returns the
// block's f64 total (the estimate of the next block's start). Three
// barriers: the f64 prefix, the neighbours' class codes at wave edges, and
// the wave totals of the segmented run scan and of the item / raw counts
// (each wave combines the totals of the waves before it itself). Its LDS
// scratch (s.H0[0 .. 191]) is rewritten only after the next two barriers,
// so consecutive calls need none in between.
template <bool FIND>
__device__ __forceinline__ RecCount res_record_regs(const float (&e)[kResK], double p_slice,
                                                    uint32_t pos0, uint32_t nthr, uint32_t ibase,
                                                    uint32_t rbase,
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
  if (rc.items > kRsItemCap || rc.raws > kRsRawCap ||
      4u * (ibase + rc.items) + kResK * (rbase + rc.raws) > kRsLdsWords) {
    rc.ok = false;
    return rc;
  }
  // items from the bottom of s.H, raw slot r at the top (kResK words ending
  // kResK * r below it)
  const uint32_t ip = ibase + (pos & 0xffffu), rg = rbase + (pos >> 16);
  u32x4* items = reinterpret_cast<u32x4*>(s.H);
  if (unc) {
    items[ip] = u32x4{bin, own.a0, own.a1, FIND ? rg | (t << 16) : rg};
    u32x4* raw = reinterpret_cast<u32x4*>(s.H + kRsLdsWords - kResK * (rg + 1u));
#pragma unroll
    for (int m = 0; m < (int)kResK / 4; ++m)
      raw[m] = u32x4{__float_as_uint(e[4 * m]), __float_as_uint(e[4 * m + 1]),
                     __float_as_uint(e[4 * m + 2]), __float_as_uint(e[4 * m + 3])};
  } else if (last) {
    items[ip] = u32x4{bin, inc.m.a0, inc.m.a1, kNoRaw};
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

// The exact sequential sum of xf(i, v) over the row in index order (FIND
// false), or the first element whose running sum exceeds probe (FIND true:
// found, pos, the sums before and at it). The summands must be finite and
// >= 0. ok = false: the method could not finish (nothing is wrong). The
// records live in s.H (at most kRsLdsWords words for the whole row).
template <bool FIND, class XF>
__device__ __forceinline__ EcssResult row_rec_sum(const KernelArgs& a, int b, const Row& row,
                                                  XF&& xf, float probe, Smem& s, bool& ok) {
  const uint32_t V = row.V, t = threadIdx.x;
  const uint32_t nblk = (V + kResSlice - 1u) / kResSlice;
  EcssResult r{0.f, 0, -1, 0.f};
  ok = false;
  if (nblk == 0u || nblk > (uint32_t)kMaxSlices) return r;
  uint32_t* ioff = s.H0 + 1040;  // [kMaxSlices] each block's first item
  double P = 0.0;
  bool fit = true;
  uint32_t nb = nblk;  // blocks recorded
  uint32_t ibase = 0, rbase = 0;  // items and raws recorded so far
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
    const RecCount rc = res_record_regs<FIND>(e, P, lo, (n + kResK - 1u) / kResK, ibase, rbase, s,
                                              probe, &tot);
    P += tot;
    LUMEN_TICK("rr_rec", b);
    if (t == 0) ioff[blk] = ibase;
    fit = fit && rc.ok;
    if (!fit) break;
    ibase += rc.items;
    rbase += rc.raws;
    // searching: once the running sum is surely above the probe where the
    // next block starts, the hit lies in the blocks recorded so far
    if (FIND && blk + 1u < nblk &&
        (double)probe < P * (1.0 - (5e-5 + 4e-9 * (double)(lo + n)))) {
      nb = blk + 1u;
      break;
    }
  }
  __syncthreads();
  if (!fit) return r;
  // the raws, moved to follow the items in slot order (the walk's layout),
  // and the blocks' item offsets (raw slots are numbered across the row)
  const uint32_t nit = ibase, rawbase = 4u * nit, rw = kResK * rbase;
  uint32_t mv[kRsLdsWords / kThreads];
#pragma unroll
  for (uint32_t k = 0; k < kRsLdsWords / kThreads; ++k) {
    const uint32_t f = t + k * kThreads;
    mv[k] = f < rw ? s.H[kRsLdsWords - kResK * (f / kResK + 1u) + f % kResK] : 0u;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t k = 0; k < kRsLdsWords / kThreads; ++k) {
    const uint32_t f = t + k * kThreads;
    if (f < rw) s.H[rawbase + f] = mv[k];
  }
  if (t < 32u) {
    s.H0[t] = t < nb ? ioff[t] : nit;
    s.H0[32u + t] = 0u;
  }
  __syncthreads();
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
