// Development-only phase timing, included by sampler_kernels.hip only in
// code objects built with -DLUMEN_TIMING (never in the shipped one): thread 0
// of each workgroup of row LUMEN_TIMING_ROW records wall-clock ticks (100 MHz)
// at phase ends, and the row's finisher prints them when it writes the row.
#pragma once
#include <cstdio>
#ifndef LUMEN_TIMING_ROW
#define LUMEN_TIMING_ROW 0
#endif
// one log per slice of the traced row in device memory; the workgroup's log
// index (or -1) sits in LDS
__device__ unsigned long long g_tick_t[16][64];
__device__ const char* g_tick_l[16][64];
__device__ int g_tick_n[16];
__shared__ int g_tick_slot;
__shared__ unsigned int g_wg_t0;  // this workgroup's start (low 32 bits of the wall clock)
__shared__ int g_nticks;
#define LUMEN_TICK(label, b)                                                   \
  do {                                                                        \
    if (threadIdx.x == 0 && (b) == LUMEN_TIMING_ROW && g_tick_slot >= 0 && g_nticks < 64) {  \
      g_tick_t[g_tick_slot][g_nticks] = wall_clock64();                       \
      g_tick_l[g_tick_slot][g_nticks++] = label;                              \
      g_tick_n[g_tick_slot] = g_nticks;                                       \
    }                                                                         \
  } while (0)
#define LUMEN_TICK_INIT() \
  do {                    \
    if (threadIdx.x == 0) { g_nticks = 0; g_tick_slot = -1; g_wg_t0 = (unsigned int)wall_clock64(); } \
  } while (0)
// every row: the finishing workgroup's start and end times in the trace's
// pad words (the host prints each row's end relative to the earliest start)
#define LUMEN_ROW_TIMES(tr)                                 \
  do {                                                      \
    tr.pad[0] = g_wg_t0;                                    \
    tr.pad[1] = (unsigned int)wall_clock64();               \
  } while (0)
#define LUMEN_TICK_SLOT(row, sl) \
  do {                           \
    if (threadIdx.x == 0) g_tick_slot = ((row) == LUMEN_TIMING_ROW && (sl) < 16) ? (int)(sl) : -1; \
  } while (0)
#define LUMEN_TICK_RESET(b) \
  do {                      \
    if (threadIdx.x == 0 && (b) == LUMEN_TIMING_ROW) g_nticks = 0; \
  } while (0)
// times from the earliest first tick of any slice of the row
#define LUMEN_TICK_DUMP(b)                                                       \
  do {                                                                          \
    if (threadIdx.x == 0 && (b) == LUMEN_TIMING_ROW && g_tick_slot >= 0) {      \
      unsigned long long t0_ = ~0ull;                                           \
      for (int k_ = 0; k_ < 16; ++k_)                                           \
        if (g_tick_n[k_] > 0 && g_tick_t[k_][0] < t0_) t0_ = g_tick_t[k_][0];   \
      for (int k_ = 0; k_ < 16; ++k_)                                           \
        if (k_ != g_tick_slot && g_tick_n[k_] > 0)                              \
          for (int i_ = (g_tick_n[k_] > 12 ? g_tick_n[k_] - 12 : 0); i_ < g_tick_n[k_]; ++i_) \
          printf("tick[%d] %s %f us\n", k_, g_tick_l[k_][i_], \
                 (double)(g_tick_t[k_][i_] - t0_) / 100.0);       \
      for (int i_ = 0; i_ < g_nticks; ++i_)                                     \
        printf("tick[%d] %s %f us\n", g_tick_slot, g_tick_l[g_tick_slot][i_],  \
               (double)(g_tick_t[g_tick_slot][i_] - t0_) / 100.0);              \
      for (int k_ = 0; k_ < 16; ++k_) g_tick_n[k_] = 0;                         \
    }                                                                           \
  } while (0)
