// Structures shared by the host library (sampler_host.cpp) and the gfx950
// code object (sampler_kernels.hip). Plain C layout, no HIP types.
#pragma once
#include <stdint.h>

namespace lumen {

// Per-row parameters resolved on the host exactly as the reference decides
// which stages run (crates/lumen-runtime/src/sampling.rs:452-527).
struct RowParams {
  float temperature;  // <= 0 selects greedy (sampling.rs:468)
  float inv_temp;     // 1.0f / temperature, computed once in f32 (sampling.rs:517)
  float top_p;        // used iff kTopP
  float log_min_p;    // logf(min_p) (sampling.rs:989), used iff kMinP
  float rep;          // repetition penalty
  float presence;     // presence penalty
  float freq;         // frequency penalty
  uint32_t top_k;     // used iff kTopK; 1 <= top_k < V
  uint32_t flags;
  uint32_t window;    // repeat_last_n clipped to 32 bits; 0 = the whole history (sampling.rs:864)
  uint32_t pad[2];
};

enum RowFlags : uint32_t {
  kGreedy = 1u,   // temperature <= 0
  kPen = 2u,      // penalties_active() and a non-empty window (sampling.rs:332-337, 858)
  kRep = 4u,      // |rep - 1| >= f32::EPSILON (sampling.rs:887)
  kTopK = 8u,     // 0 < k < V (sampling.rs:493)
  kTopP = 16u,    // 0 < p < 1 (sampling.rs:503)
  kMinP = 32u,    // min_p > 0 (sampling.rs:511)
  kAnti = 64u,    // greedy with the anti-restate guard (sampling.rs:472-474): candidates out
};

// Per-row diagnostics (optional output), mirrors the oracle's trace.
struct RowTrace {
  uint32_t status;          // 0 ok, else a RowStatus code
  uint32_t path;            // bit0 greedy, bit1 small path, bit2 large path, bit3 uniform top-p,
                            // bit4 uniform final, bit5 NaN final
  uint32_t topk_cutoff_key; // total_cmp key of the k-th largest logit
  uint32_t topk_survivors;
  float topp_sum;           // softmax sum inside top-p
  uint32_t topp_kept;       // reference `kept` (V when the loop never broke)
  float topp_cum;           // cum value at the crossing
  uint32_t windows;         // top-p windows walked
  float final_max;
  float final_sum;
  float cdf_before;
  float cdf_at;
  uint32_t token;
  uint32_t passes;          // full-row passes made over the logits
  uint32_t pad[2];
};

enum RowStatus : uint32_t {
  kStatusOk = 0,
  kStatusTieOverflow = 1,   // > list capacity of exactly-equal keys in one top-p window
  kStatusListOverflow = 2,  // internal: window larger than planned
  kStatusHistOverflow = 3,  // device history: the penalty window is longer than the ring
};

// Device history rings hold at most this many tokens per row (the window
// counts are built in an LDS hash table of twice as many slots).
constexpr uint32_t kRingMaxCap = 8192;
constexpr uint32_t kHistBad = 0xffffffffu;     // hist_off value of a row whose window overflowed
constexpr uint32_t kTokenError = 0xffffffffu;  // LUMEN_TOKEN_ERROR

constexpr int kInlineRows = 8;
constexpr int kMaxSlices = 16;      // workgroups cooperating on one row
constexpr uint32_t kIdleBlock = 0xffffffffu;
constexpr int kCandCap = 8192;      // per-row candidate buffer (entries)
// Row stride of the candidate buffers: kCandCap entries, then (register-
// resident top-p rows) each candidate's exp(v - m1) as a u32 array.
constexpr int kCandStride = 2 * kCandCap;
// Split top-k rows take k up to kTopKSplitMax; their candidates may fill the
// whole row stride of the candidate buffer.
constexpr uint32_t kTopKSplitMax = 4096;
constexpr uint32_t kTopKCandCap = (uint32_t)kCandStride;
constexpr int kMassBins = 512;      // top-p window planning bins
constexpr int kChainMaxQ = 2;       // sub-chunks per slice in the softmax-sum chain
constexpr int kRowRecs = kMaxSlices * kChainMaxQ * 16;  // run records per row (one per wave segment)
constexpr int kRecWords = 1152;     // words per run record slot
// Records of the exact row sums of lumen_sample_rows_single (row_rec_sum),
// kept in LDS: per block of kResSlice logits at most
constexpr uint32_t kRsItemCap = 512;   // items (4 words each)
constexpr uint32_t kRsRawCap = 64;     // raws (32 words each)


// Per-row coordination block in device memory. Zero at allocation; the last
// workgroup of a row to finish restores the counters to zero, so every
// launch starts from a clean block.
struct RowWs {
  uint32_t arrive;       // last-arriver counter
  uint32_t bar;          // spin barrier counter
  uint32_t unused0;
  uint32_t cand_n;       // candidates appended
  uint32_t status;       // row failure bits
  uint32_t pad[3];
  float part_max[kMaxSlices];
  uint32_t part_nan[kMaxSlices];
  uint64_t part_arg[kMaxSlices];
  double part_e[kMaxSlices];
  uint64_t part_top[kMaxSlices][8];  // anti-restate rows: each slice's 8 largest finite keys
  // register-resident top-p rows: each slice's candidate block (start, count)
  // in the row's candidate buffer and its exact-sum record (items, raw slots)
  uint32_t part_cb[kMaxSlices];
  uint32_t part_cn[kMaxSlices];
  uint32_t part_nrec[kMaxSlices];
  uint32_t part_nraw[kMaxSlices];
};

// Anti-restate candidates per row: [0] the raw argmax (total_cmp over every
// value, lowest index on ties), [1..8] the 8 largest finite values' ids in
// (value desc, id asc) order, kGuardNone where fewer exist.
constexpr int kGuardWords = 9;
constexpr uint32_t kGuardNone = 0xffffffffu;

// Arguments of lumen_zero_tokens (an empty vocabulary).
struct ZeroArgs {
  uint32_t* tokens;
  uint32_t* ring;      // form C history ring, or NULL
  uint32_t* ring_len;
  uint32_t n;
  uint32_t ring_cap;
};

struct KernelArgs {
  const void* logits;        // [B][row_stride] f32 or bf16, device
  uint64_t row_stride;       // elements
  uint32_t vocab;
  uint32_t batch;
  int32_t dtype;             // 0 = f32, 1 = bf16
  uint32_t pad0;
  const RowParams* params;   // [B] device
  const uint32_t* hist_off;  // [B+1] offsets into hist_ids / hist_cnt (row b ends at
                             // hist_off[b + 1], or at hist_end[b] when hist_end is set)
  const uint32_t* hist_ids;  // unique token ids of the penalty window, per row
  const uint32_t* hist_cnt;  // occurrence counts
  const float* uniforms;     // [B] draw per row (ignored by greedy rows)
  uint32_t* tokens;          // [B] output
  RowTrace* trace;           // [B] optional
  float* pen_scratch;        // [B][pen_stride] penalized rows (f32)
  uint64_t pen_stride;
  float* pen_out;            // optional [B][vocab] copy of penalized logits
  // Small batches pass their parameters and draws inside the kernel
  // arguments (no staging copy): used when inline_rows > 0.
  RowWs* ws;                 // [B] coordination blocks
  uint32_t* est;             // [B][kRowRecs][kRecWords] run records of wave segments
  uint64_t* cand;            // [B][kCandCap] candidate buffers
  float* hist;               // [B][kMaxSlices][kMassBins] candidate exp-mass per logit bin
  uint32_t slices;           // workgroups per row (G) when blk_map is NULL
  uint32_t xcd_rows;         // 1: place all slices of a row on one XCD (blk_map NULL)
  // Per-block placement: (row << 10) | (G << 5) | slice, or kIdleBlock. Rows
  // get slice counts weighted by their path's cost, and a row's slices sit on
  // one XCD. NULL: every row has `slices` workgroups, mapped as above.
  const uint32_t* blk_map;
  uint32_t inline_rows;      // > 0: params come from inline_params
  uint32_t inline_draws;     // != 0: draws come from inline_uniforms
  uint32_t count_cap;        // form C: count entries per row (ring_cap, or vocab for long windows)
  // Bound of every cross-workgroup wait, in ticks of the 100 MHz wall clock;
  // 0 makes every such wait give up at once. A wait that gives up adds 1 to
  // *timeouts (device memory of the context) and its row takes the exact
  // single-workgroup path.
  uint32_t wait_ticks;
  uint32_t* timeouts;
  // Synchronous calls: the token is also written to pinned host memory
  // mapped into the device, and *done_mapped (host memory) counts the rows
  // written, so the host waits on that count instead of a copy and a stream
  // synchronization. NULL otherwise.
  uint32_t* tokens_mapped;
  uint32_t* done_mapped;
  // Device RNG: when non-NULL the draw of a sampled row is next_f32 of
  // rng_dev[b] (Xorshift64, sampling.rs:74-104), and the row's finisher
  // stores the advanced state.
  uint64_t* rng_dev;
  // Device history: a ring of the last ring_cap tokens of each row
  // ([B][ring_cap], token k of row b at k % ring_cap) and the count of tokens
  // recorded (ring_len[b]). lumen_hist_window builds the penalty window's
  // counts from it into hist_off / hist_ids / hist_cnt (a region of
  // count_cap entries per row) and hist_end; the finisher of each row records its token.
  uint32_t* ring;
  uint32_t* ring_len;
  uint32_t* hist_end;        // [B] end of row b's counts (hist_off[b] = kHistBad on overflow)
  uint32_t ring_cap;
  uint32_t ring_epoch;       // lumen_batch.hist_epoch
  // [B][8] what row b's counts reflect: ring_len, window, ring address (lo,
  // hi), ring_cap, ring_epoch, count_cap. When the next call finds exactly one more token recorded
  // in the same ring with the same window, lumen_hist_window updates the
  // counts by that token (and the one leaving the window) instead of counting
  // the window again. ring_len 0xffffffff: nothing valid.
  uint32_t* hist_state;
  // Anti-restate rows: candidates to guard[B][kGuardWords] (device) and, in
  // synchronous calls, to guard_mapped (mapped pinned host memory) before
  // the row is counted in done_mapped.
  uint32_t* guard;
  uint32_t* guard_mapped;
  float inline_uniforms[kInlineRows];
  RowParams inline_params[kInlineRows];
};

// Stamp of the layouts the host library and the code object share. The
// code object exports it (lumen_kernel_abi) and the library refuses a code
// object whose stamp differs from its own: kernel arguments read with
// another layout would be garbage pointers. kAbiVersion changes with any
// change of meaning that keeps the sizes.
constexpr uint32_t kAbiVersion = 8;
constexpr uint32_t kAbiStamp =
    (kAbiVersion * 0x9E3779B1u) ^ ((uint32_t)sizeof(KernelArgs) * 0x85EBCA77u) ^
    ((uint32_t)sizeof(RowWs) * 0xC2B2AE3Du) ^ ((uint32_t)sizeof(RowParams) * 0x27D4EB2Fu) ^
    ((uint32_t)sizeof(RowTrace) * 0x165667B1u) ^ (kRsItemCap * 0xD3A2646Cu) ^
    ((uint32_t)kCandStride * 0xFD7046C5u) ^ ((uint32_t)kRowRecs * 0xB55A4F09u);

}  // namespace lumen
