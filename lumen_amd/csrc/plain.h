// Register-resident split path for rows without top-k, top-p or min-p
// (included by sampler_kernels.hip after resident.h).
//
// Reference semantics: sample_logits (crates/lumen-runtime/src/sampling.rs:
// 452-527) with only the penalties (:850-900), the temperature (:516-520),
// softmax_inplace (:207-231) and sample_categorical (:1003-1014) active. This
// is the chain of SamplingParams::default() (T 1.0, :313-325) and of a server
// request that leaves top_p unset (T 0.7 with the default repetition penalty).
//
// Each of the G workgroups of a row owns a slice of at most kResSlice logits,
// read from HBM once and kept in registers (32 contiguous elements per
// thread, through the LDS transpose of resident.h):
//
//  phase A  penalties, the slice maximum, a NaN flag and an estimate of the
//           slice's sum of exp(v * inv_temp - max);
//  barrier  the row maximum m1, so m3 = m1 * inv_temp (rounding is monotone);
//  phase B  the exact summands e = exp(v * inv_temp - m3), kept in registers,
//           and the slice's record of the exact sequential softmax sum;
//  S        the last workgroup to arrive walks the G records: the exact sum S
//           and the exact running sum at each slice start, published to the
//           row's block; the other workgroups wait for them;
//  phase C  p = e / S and the slice's record of the sequential CDF sum, where
//           every thread whose CDF range may hold the draw r keeps its raw
//           probabilities;
//  draw     the last workgroup to arrive walks the CDF records to the first
//           cumulative sum above r, which lies in a raw: the token.
//
// Estimates only decide speed. Any check that fails (a record the exact sum
// does not fit, a crossing outside a raw, NaN, a non-finite maximum, a wait
// that times out) hands the row to the exact single-workgroup path.
#pragma once

namespace lumen {

// Plain temperature sampling over register-resident slices; see the header
// comment. Workgroup sl owns the q virtual slices sl*q .. sl*q+q-1 of the
// row's G*q (res_chunks); with q > 1 each is read again (from cache) in the
// later phases.
template <bool BF16, bool MULTI>
__device__ __forceinline__ void temp_res(const KernelArgs& a, int b, uint32_t sl, uint32_t G,
                                         uint32_t q_rt, Smem& s) {
  ROW_CONTEXT(a, b);
  const uint32_t q = MULTI ? q_rt : 1u;  // one chunk: straight-line code
  const uint32_t V = a.vocab, t = threadIdx.x, lane = t & 63u;
  const uint32_t Gv = G * q;
  const bool pen = (P.flags & kPen) && hist_hi(a, b) > a.hist_off[b];
  const float invT = P.inv_temp;

  // ---- phase A ----
  float v[8][4];
  float x[kResK];
  for (uint32_t j = 0; j < q; ++j) {
    const uint32_t vs = sl * q + j;
    const Slice sc = slice_bounds(V, Gv, vs);
    res_issue<BF16>(row, sc, v);
    res_load<BF16>(a, b, P, row, sc, pen, v, x, s);
    if (a.pen_out) {
      float* po = a.pen_out + (uint64_t)b * V + sc.lo + t * kResK;
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k)
        if (sc.lo + t * kResK + (uint32_t)k < sc.hi) po[k] = x[k];
    }
    float mt = kNegInf;
    uint32_t nan = 0;
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k) {
      mt = op_maxl(mt, x[k]);  // f32::max folds skip NaN (sampling.rs:209)
      nan |= is_nan(x[k]) ? 1u : 0u;
    }
    const float ms = block_maxl(mt, s);
    nan = block_or_u32(nan, s);
    float et = 0.f;
    if (ms != kNegInf) {
      const float mts = __fmul_rn(ms, invT);
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k) et += __expf(__fmul_rn(x[k], invT) - mts);
    }
    const double es = block_sum_f64((double)et, s);
    if (t == 0) {
      ws.part_max[vs] = ms;
      ws.part_nan[vs] = nan;
      ws.part_e[vs] = es;
    }
  }
  wg_arrive(&ws.bar, 0xffffffffu, s);
  bool ok = wg_wait_geq(a, &ws.bar, G, s);

  // ---- phase B: the last chunk first (its logits are in registers) ----
  float m3 = 0.f;
  bool bad = !ok;
  float* Lt = res_buf(s) + t * kResPitch;
  for (uint32_t jj = 0; jj < q && !bad; ++jj) {
    const uint32_t vs = sl * q + (q - 1u - jj);
    const Slice sc = slice_bounds(V, Gv, vs);
    if (jj > 0) {
      res_issue<BF16>(row, sc, v);
      res_load<BF16>(a, b, P, row, sc, pen, v, x, s);
    }
    float* rowv = reinterpret_cast<float*>(s.H0 + 1024);  // [0] m1, [2..3] p_slice (f64)
    uint32_t* rowu = s.H0 + 1032;                        // [1] bad
    if (t < 64u) {
      const bool in = lane < Gv;
      const float mi = in ? ws.part_max[lane] : kNegInf;
      const double ei = in ? ws.part_e[lane] : 0.0;
      const bool ni = in && ws.part_nan[lane] != 0u;
      const float m1w = wave_reduce(mi, kNegInf, op_maxl);
      const float m3w = __fmul_rn(m1w, invT);
      const double term = (lane < vs && mi != kNegInf)
                              ? ei * exp((double)__fmul_rn(mi, invT) - (double)m3w) : 0.0;
      const double ps = wave_reduce(term, 0.0, [](double l, double r) { return l + r; });
      const bool anynan = __ballot(ni || (in && !(ei == ei))) != 0ull;
      // an earlier slice holding the maximum has added exp(0) = 1
      const bool one = __ballot(lane < vs && mi == m1w) != 0ull;
      if (lane == 0) {
        rowv[0] = m1w;
        rowv[1] = one ? 1.f : 0.f;
        *reinterpret_cast<double*>(rowv + 2) = ps;
        rowu[1] = (anynan || !is_finite(m1w) || !is_finite(m3w)) ? 1u : 0u;
      }
    }
    __syncthreads();
    m3 = __fmul_rn(rowv[0], invT);
    const double p_slice = *reinterpret_cast<const double*>(rowv + 2);
    const float lb_slice = rowv[1];
    bad = rowu[1] != 0u;
    __syncthreads();
    if (bad) break;
    // the exact summands, in registers (they outlive the LDS copy)
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k) x[k] = expf_glibc_nonpos(__fsub_rn(__fmul_rn(x[k], invT), m3));
#pragma unroll
    for (int qq = 0; qq < (int)kResK / 4; ++qq)
      *reinterpret_cast<float4*>(Lt + 4 * qq) =
          make_float4(x[4 * qq], x[4 * qq + 1], x[4 * qq + 2], x[4 * qq + 3]);
    __syncthreads();
    const uint32_t nthr = (sc.hi - sc.lo + kResK - 1u) / kResK;
    const RecCount rc = res_record(Lt, p_slice, sc.lo, nthr, res_rec(a, b, vs), s, 0.f, lb_slice);
    if (t == 0) {
      ws.part_nrec[vs] = rc.ok ? rc.items : 0xffffffffu;
      ws.part_nraw[vs] = rc.raws;
    }
    __syncthreads();
  }
  if (bad && t == 0) __hip_atomic_fetch_or(&ws.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // ---- S: the exact softmax sum, by the last workgroup to arrive ----
  if (wg_arrive(&ws.arrive, G - 1u, s) == G - 1u) {
    // this workgroup finishes the draw only if it also arrives last below
    if (t == 0) s.finisher = 0u;
    float* starts = reinterpret_cast<float*>(s.H0 + 64);  // [Gv]
    uint32_t nit = 0, rawbase = 0;
    bool good = __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u &&
                res_gather(a, b, Gv, s, &nit, &rawbase);
    if (good) {
      if (t < 64u) res_walk<false>(Gv, nit, rawbase, 0.f, starts, s);
      __syncthreads();
      good = s.misc_u[0] != 0u;
    }
    if (t == 0) {
      if (good) {
        ws.unused0 = __float_as_uint(s.red_f[0]);
        for (uint32_t i = 0; i < Gv; ++i) ws.part_max[i] = starts[i];
      } else {
        __hip_atomic_fetch_or(&ws.status, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_fetch_add(&ws.bar, G, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
  } else {
    ok = wg_wait_geq(a, &ws.bar, 2u * G, s);
    if (!ok && t == 0) __hip_atomic_fetch_or(&ws.status, 8u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- phase C: the CDF records; chunk sl*q first (its summands are in
  // registers), the others read and exponentiated again ----
  if (t == 0) {
    s.misc_u[0] = __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s.red_f[0] = __uint_as_float(ws.unused0);
  }
  __syncthreads();
  bad = s.misc_u[0] != 0u;
  const float S = s.red_f[0];
  __syncthreads();
  for (uint32_t j = 0; j < q && !bad; ++j) {
    const uint32_t vs = sl * q + j;
    const Slice sc = slice_bounds(V, Gv, vs);
    if (j > 0) {
      res_issue<BF16>(row, sc, v);
      res_load<BF16>(a, b, P, row, sc, pen, v, x, s);
#pragma unroll
      for (int k = 0; k < (int)kResK; ++k) x[k] = expf_glibc_nonpos(__fsub_rn(__fmul_rn(x[k], invT), m3));
    }
    const float start = ws.part_max[vs];
#pragma unroll
    for (int k = 0; k < (int)kResK; ++k) x[k] = __fdiv_rn(x[k], S);
#pragma unroll
    for (int qq = 0; qq < (int)kResK / 4; ++qq)
      *reinterpret_cast<float4*>(Lt + 4 * qq) =
          make_float4(x[4 * qq], x[4 * qq + 1], x[4 * qq + 2], x[4 * qq + 3]);
    __syncthreads();
    const uint32_t nthr = (sc.hi - sc.lo + kResK - 1u) / kResK;
    const RecCount rc =
        res_record<true>(Lt, (double)start / (double)S, sc.lo, nthr, res_rec(a, b, vs), s, rdraw);
    if (t == 0) {
      ws.part_nrec[vs] = rc.ok ? rc.items : 0xffffffffu;
      ws.part_nraw[vs] = rc.raws;
    }
    __syncthreads();
  }
  if (wg_arrive(&ws.arrive, 2u * G - 1u, s) != 2u * G - 1u) return;

  // ---- the draw, by the last workgroup to arrive ----
  uint32_t nit = 0, rawbase = 0;
  bool good = __hip_atomic_load(&ws.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u &&
              res_gather(a, b, Gv, s, &nit, &rawbase);
  if (good) {
    if (t < 64u) res_walk<true>(Gv, nit, rawbase, rdraw, nullptr, s);
    __syncthreads();
    // the records skip threads surely past the draw: no hit means the
    // chunked method decides
    good = s.misc_u[0] != 0u && s.misc_u[1] != 0u;
  }
  if (!good) {
    row_single<false>(a, b, s);
    return;
  }
  const bool found = s.misc_u[1] != 0u;
  const uint32_t hk = s.misc_u[2], hj = s.misc_u[3];
  const float c_at = s.red_f[0], c_before = s.red_f[1];
  uint32_t tok = V - 1u;  // fall-through (sampling.rs:1013)
  if (found) {
    const uint32_t* ib = s.H0;
    const uint4* items = reinterpret_cast<const uint4*>(s.Bk);
    uint32_t i = 0;
    while (i + 1u < Gv && ib[i + 1] <= hk) ++i;
    const uint32_t th = (items[hk].w >> 16) & 0x3ffu;
    tok = slice_bounds(V, Gv, i).lo + th * kResK + hj;
  }
  RowTrace tr;
  init_trace(tr, V);
  tr.path = 4u;
  tr.passes = q > 1u ? 3u : 1u;
  tr.final_max = m3;
  tr.final_sum = S;
  tr.cdf_before = found ? c_before : c_at;
  tr.cdf_at = c_at;
  write_result(a, b, tok, tr);
}

}  // namespace lumen
