// Wave64 scans and reductions on the DPP lane network of gfx950.
//
// A cross-lane step through ds_bpermute (what __shfl_* compiles to) costs
// an LDS round trip; DPP row shifts and row broadcasts move data between
// lanes inside the VALU. An inclusive scan of a wave is six DPP steps:
// row_shr 1, 2, 4, 8 build the prefixes of each 16-lane row, row_bcast15
// folds row r's last lane into row r + 1, row_bcast31 folds lane 31 into
// rows 2 and 3. Lanes that receive nothing keep `ident`, so `op` only needs
// an identity and associativity (not commutativity): the operand from
// lower lanes is always on the left.
//
// Every function here must be called with all 64 lanes of the wave active.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lumen {

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_word(uint32_t ident, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, CTRL, ROW_MASK, 0xf, false);
}

// One DPP move applied to every 32-bit word of a trivially copyable T.
template <int CTRL, int ROW_MASK, class T>
__device__ __forceinline__ T dpp_move(T ident, T v) {
  static_assert(sizeof(T) % 4 == 0, "DPP moves 32-bit words");
  constexpr int kW = (int)(sizeof(T) / 4);
  uint32_t wi[kW], wv[kW];
  __builtin_memcpy(wi, &ident, sizeof(T));
  __builtin_memcpy(wv, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < kW; ++k) wv[k] = dpp_word<CTRL, ROW_MASK>(wi[k], wv[k]);
  T o;
  __builtin_memcpy(&o, wv, sizeof(T));
  return o;
}

// Inclusive scan in lane order: lane i gets op(x_0, ..., x_i).
template <class T, class Op>
__device__ __forceinline__ T wave_scan_incl(T v, T ident, Op op) {
  v = op(dpp_move<0x111, 0xf>(ident, v), v);  // row_shr:1
  v = op(dpp_move<0x112, 0xf>(ident, v), v);  // row_shr:2
  v = op(dpp_move<0x114, 0xf>(ident, v), v);  // row_shr:4
  v = op(dpp_move<0x118, 0xf>(ident, v), v);  // row_shr:8
  v = op(dpp_move<0x142, 0xa>(ident, v), v);  // row_bcast:15 into rows 1, 3
  v = op(dpp_move<0x143, 0xc>(ident, v), v);  // row_bcast:31 into rows 2, 3
  return v;
}

// Value of the next lower lane (lane 0 gets ident).
template <class T>
__device__ __forceinline__ T wave_shr1(T v, T ident) {
  return dpp_move<0x138, 0xf>(ident, v);  // wave_shr:1
}

// Lane `lane`'s value, uniform across the wave (lane must be uniform).
template <class T>
__device__ __forceinline__ T wave_read(T v, int lane) {
  constexpr int kW = (int)(sizeof(T) / 4);
  uint32_t w[kW];
  __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
  for (int k = 0; k < kW; ++k) w[k] = (uint32_t)__builtin_amdgcn_readlane((int)w[k], lane);
  T o;
  __builtin_memcpy(&o, w, sizeof(T));
  return o;
}

// op over all 64 lanes, uniform result.
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, T ident, Op op) {
  return wave_read(wave_scan_incl(v, ident, op), 63);
}

}  // namespace lumen
