// Host side of the gfx950 sampling engine: the C ABI of include/lumen_sampler.h.
//
// Responsibilities:
//  * load the gfx950 code object (embedded with .incbin, or a file named by
//    LUMEN_SAMPLER_CODE_OBJECT) through hipModuleLoadData;
//  * resolve each row's SamplingParams into the stage flags exactly as the
//    reference decides them (crates/lumen-runtime/src/sampling.rs:452-527);
//  * build the penalty window counts from raw histories (form A,
//    sampling.rs:850-879) or take caller-resident counts (form B);
//  * stage small host inputs (inline kernel arguments for up to 8 rows, a
//    pinned staging buffer otherwise) and launch one workgroup per row.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "../../include/lumen_sampler.h"
#include "kernel_abi.h"
#include "noalloc.h"

extern "C" const unsigned char lumen_gfx950_code_object[];
extern "C" const unsigned char lumen_gfx950_code_object_end[];

using lumen::KernelArgs;
using lumen::RowParams;

namespace {

// Path a row takes in the kernel when it has G > 1 workgroups (mirrors the
// dispatch in lumen_sample_rows).
enum RowPath { kPathGreedy, kPathTopK, kPathTopP, kPathSingle };
constexpr uint32_t kWgThreads = 1024;  // lumen_sample_rows workgroup size
constexpr uint32_t kResSlice = 32u * kWgThreads;  // logits per register-resident slice

// Chunks per workgroup of a register-resident row with G workgroups (the
// kernel's res_chunks): the fewest q <= 4 with G * q <= kMaxSlices whose
// G * q slices each hold at most kResSlice logits; 0 when none does.
uint32_t res_chunks(uint32_t V, uint32_t G) {
  for (uint32_t q = 1; q <= 4u && G * q <= (uint32_t)lumen::kMaxSlices; ++q)
    if ((((V + G * q - 1u) / (G * q) + 15u) & ~15u) <= kResSlice) return q;
  return 0u;
}

RowPath row_path(const RowParams& r, uint32_t V, uint32_t G) {
  if (r.flags & lumen::kGreedy) return kPathGreedy;
  if ((r.flags & lumen::kTopK) && r.top_k <= lumen::kTopKSplitMax) return kPathTopK;
  const uint32_t per = G ? ((V + G - 1u) / G + 15u) & ~15u : V;
  // register-resident rows: top-p (any penalties, min-p, temperature), and
  // plain temperature rows (no top-k, top-p or min-p)
  if (!(r.flags & lumen::kTopK) && ((r.flags & lumen::kTopP) || !(r.flags & lumen::kMinP)) &&
      V >= 64u && G > 1u && res_chunks(V, G) != 0u)
    return kPathTopP;
  if ((r.flags & lumen::kTopP) && !(r.flags & (lumen::kTopK | lumen::kPen)) &&
      per <= 32u * kWgThreads * (uint32_t)lumen::kChainMaxQ)
    return kPathTopP;
  return kPathSingle;
}

// Workgroups per row, weighted by the cost of the row's path (a top-p row
// reads its row twice and has the longest finisher; a greedy row reads it
// once and finishes in a few microseconds), and their placement: with
// blocks dispatched to the 8 XCDs round-robin, block ids x, x + 8, ... land
// on XCD x, so each row's slices are packed into one XCD's list. The total
// never exceeds the resident capacity, so every row's workgroups are
// co-resident. Returns the grid size; map[block] = (row << 10) | (G << 5) |
// slice, or kIdleBlock.
uint32_t plan_blocks(const std::vector<RowParams>& rows, uint32_t V, uint32_t cap,
                     uint32_t g_uniform, std::vector<uint32_t>& map) {
  const uint32_t B = (uint32_t)rows.size();
  const uint32_t kX = 8;
  const uint32_t bin_cap = cap / kX;
  std::vector<uint32_t> G(B, 1), w(B, 0);
  // slice weights of the greedy, top-k and top-p paths (timed on the mixed
  // config-3 batch and the defaults batch: 2,3,8 best)
  struct Weights {
    uint32_t g = 2, k = 3, p = 8;
  };
  constexpr Weights wt{};
  uint64_t wsum = 0;
  uint32_t fixed = 0;
  for (uint32_t b = 0; b < B; ++b) {
    switch (row_path(rows[b], V, lumen::kMaxSlices)) {
      case kPathGreedy: w[b] = wt.g; break;
      case kPathTopK: w[b] = wt.k; break;
      case kPathTopP: w[b] = wt.p; break;
      default: w[b] = 0; ++fixed; break;  // exact single-workgroup row
    }
    wsum += w[b];
  }
  const uint32_t spare = cap > fixed ? cap - fixed : 0;
  // fewest slices that keep a register-resident row at one chunk per
  // workgroup; with up to 4 chunks per workgroup it may go down to a quarter
  uint32_t g_res = 1;
  while (g_res < lumen::kMaxSlices && ((V + g_res - 1u) / g_res + 15u) / 16u * 16u > kResSlice) ++g_res;
  uint32_t g_min = std::max<uint32_t>(2u, (g_res + 3u) / 4u);
  while (g_min < g_res && res_chunks(V, g_min) == 0u) ++g_min;
  std::vector<uint8_t> res(B, 0);
  uint64_t used = 0;
  for (uint32_t b = 0; b < B; ++b) {
    if (!w[b]) continue;
    uint64_t g = wsum ? ((uint64_t)spare * w[b] + wsum / 2) / wsum : 1;
    G[b] = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(g, lumen::kMaxSlices));
    const RowParams& r = rows[b];
    res[b] = !(r.flags & (lumen::kTopK | lumen::kGreedy)) &&
                     ((r.flags & lumen::kTopP) || !(r.flags & lumen::kMinP)) ? 1 : 0;
    if (res[b] && G[b] < g_res) G[b] = g_res;
    if (row_path(rows[b], V, G[b]) == kPathSingle) G[b] = 1;
    used += G[b];
  }
  // raising resident rows to g_res may overrun the spare workgroups: take
  // them back from the rows with the most slices, resident rows down to g_min
  while (used > spare) {
    uint32_t pick = B;
    for (uint32_t b = 0; b < B; ++b) {
      const uint32_t floor = res[b] ? g_min : 1u;
      if (G[b] > floor && (pick == B || G[b] > G[pick])) pick = b;
    }
    if (pick == B) break;  // every row at its floor: the XCD packing below trims
    uint32_t g = G[pick] - 1u;
    if (row_path(rows[pick], V, g) == kPathSingle) g = 1;
    used -= G[pick] - g;
    G[pick] = g;
  }
  // every row at g_uniform: the kernel's arithmetic mapping places the same
  // grid without a map (one dependent load less per workgroup)
  bool uniform = true;
  for (uint32_t b = 0; b < B; ++b) uniform = uniform && w[b] && G[b] == g_uniform;
  if (uniform) {
    map.clear();
    return 0;
  }
  // pack rows (largest first) into the XCD lists
  std::vector<uint32_t> order(B);
  for (uint32_t b = 0; b < B; ++b) order[b] = b;
  std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) { return G[x] > G[y]; });
  std::vector<std::vector<uint32_t>> bins(kX);
  for (uint32_t b : order) {
    uint32_t best = 0;
    for (uint32_t x = 1; x < kX; ++x)
      if (bins[x].size() < bins[best].size()) best = x;
    uint32_t free_slots = bin_cap > bins[best].size() ? bin_cap - (uint32_t)bins[best].size() : 0;
    uint32_t g = std::min(G[b], std::max<uint32_t>(free_slots, 1u));
    if (g > 1 && row_path(rows[b], V, g) == kPathSingle) g = 1;
    for (uint32_t sl = 0; sl < g; ++sl) bins[best].push_back((b << 10) | (g << 5) | sl);
  }
  size_t depth = 0;
  for (const auto& v : bins) depth = std::max(depth, v.size());
  const uint32_t nblocks = (uint32_t)depth * kX;
  map.assign(nblocks, lumen::kIdleBlock);
  for (uint32_t x = 0; x < kX; ++x)
    for (size_t k = 0; k < bins[x].size(); ++k) map[x + kX * k] = bins[x][k];
  return nblocks;
}

constexpr float kF32Eps = 1.1920929e-7f;  // f32::EPSILON

struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
};

}  // namespace

struct lumen_sampler {
  int device = 0;
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  hipFunction_t fn_hist = nullptr;  // lumen_hist_window
  hipFunction_t fn_zero = nullptr;  // lumen_zero_tokens (no-allocation entry, empty vocabulary)
  hipFunction_t fn_single = nullptr;  // lumen_sample_rows_single (one workgroup per row)
  // staging: one pinned host block and one device block, same layout
  void* pin = nullptr;
  size_t pin_cap = 0;
  DevBuf stage;
  DevBuf pen_scratch;
  DevBuf ws;    // [B] RowWs, zeroed at allocation, self-resetting afterwards
  DevBuf cand;  // [B][kCandStride] candidate buffers
  DevBuf est;   // [B][kRowRecs][kRecWords] run records of the split top-p path
  DevBuf hist;  // [B][kMaxSlices][kMassBins] candidate mass histograms
  DevBuf guard;  // [B][kGuardWords] anti-restate candidates when the caller passes none
  uint32_t* guard_dev = nullptr;  // where the last call's candidates went
  bool any_anti = false;          // the last call had anti-restate rows
  DevBuf wcnt;  // device history: [B] offsets, [B] ends, [B][ccap] ids, [B][ccap] counts, [B][8] state
  uint32_t wcnt_rows = 0, wcnt_ccap = 0;  // layout of the last call (rows, count capacity)
  int cu_count = 0;
  int max_resident = 0;  // workgroups of lumen_sample_rows resident at once
  hipEvent_t staged = nullptr;  // recorded after the last staging copy
  bool staged_pending = false;
  std::vector<uint32_t> ids, cnts, offs;
  std::vector<uint32_t> tmp;
  std::vector<uint32_t> blk_map;  // per-block placement of the current call
  std::vector<char> img, last_img;  // static staging block: current / on the device
  // synchronous calls: tokens and a written-row count in pinned host memory
  // that the kernel writes through its mapping
  uint32_t* map_host = nullptr;  // [0] count, [1..] tokens
  uint32_t* map_dev = nullptr;
  uint32_t map_cap = 0;
  // bound of each cross-workgroup wait (lumen_sampler_set_wait_limit) and
  // the device count of waits that gave up
  uint32_t wait_us = 2000;
  uint32_t* timeouts_dev = nullptr;
};

namespace {

thread_local char g_last_error[256] = "";

int fail(int code, const char* why) {
  std::snprintf(g_last_error, sizeof g_last_error, "%s", why);
  return code;
}

int hip_fail(hipError_t e) {
  if (e == hipSuccess) return LUMEN_OK;
  std::snprintf(g_last_error, sizeof g_last_error, "HIP error: %s", hipGetErrorString(e));
  return LUMEN_ERR_HIP;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// True while `st` is being captured into a graph. A call that would allocate,
// clear or stage memory then refuses: those steps would be recorded into the
// graph (and replayed) or are illegal under capture.
bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) return false;
  return cs != hipStreamCaptureStatusNone;
}

constexpr const char* kCaptureMsg =
    "this call needs device set-up (a first call, a larger shape or a new history layout) "
    "and cannot run under stream capture: make one eager call with the same shapes first";

int ensure_dev(DevBuf& b, size_t bytes, hipStream_t st) {
  if (b.cap >= bytes) return LUMEN_OK;
  if (capturing(st)) return fail(LUMEN_ERR_INVALID, kCaptureMsg);
  if (b.p) {
    if (hipDeviceSynchronize() != hipSuccess) return LUMEN_ERR_HIP;
    (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
  }
  size_t cap = std::max<size_t>(bytes, 4096);
  if (hipMalloc(&b.p, cap) != hipSuccess) return LUMEN_ERR_HIP;
  b.cap = cap;
  return LUMEN_OK;
}

// Window counts of the device history (form C), in s->wcnt: [B] offsets,
// [B] ends, [B][ccap] ids, [B][ccap] counts, [B][8] state. ccap is the ring
// capacity, or the vocabulary when a penalized row counts its whole history
// (repeat_last_n 0) or a window longer than the ring: such counts are kept up
// to date token by token and can hold every distinct id.
struct RingLayout {
  uint32_t *off, *end, *ids, *cnt, *state;
};

int ring_layout(lumen_sampler* s, uint32_t B, uint32_t cap, uint32_t ccap, hipStream_t st,
                RingLayout& L) {
  const size_t state_off = 2 * (size_t)B + 2 * (size_t)ccap * B;
  const size_t need = sizeof(uint32_t) * (state_off + 8 * (size_t)B);
  const void* before = s->wcnt.p;
  int rc = ensure_dev(s->wcnt, need, st);
  if (rc != LUMEN_OK) return rc;
  uint32_t* w = static_cast<uint32_t*>(s->wcnt.p);
  if (s->wcnt.p != before || s->wcnt_rows != B || s->wcnt_ccap != ccap) {
    if (capturing(st)) return fail(LUMEN_ERR_INVALID, kCaptureMsg);
    // a new layout: nothing counted yet
    if (hipMemsetAsync(w + state_off, 0xff, sizeof(uint32_t) * 8 * (size_t)B, st) != hipSuccess)
      return fail(LUMEN_ERR_HIP, "window-count state init");
    s->wcnt_rows = B;
    s->wcnt_ccap = ccap;
  }
  (void)cap;
  L.off = w;
  L.end = w + B;
  L.ids = w + 2 * (size_t)B;
  L.cnt = w + 2 * (size_t)B + (size_t)ccap * B;
  L.state = w + state_off;
  return LUMEN_OK;
}

// Resolves one row (sampling.rs:452-527). Returns LUMEN_OK or an error.
void resolve_row(const lumen_sampling_params& p, uint32_t V, bool has_window, RowParams& r) {
  std::memset(&r, 0, sizeof(r));
  r.temperature = p.temperature;
  const float rep = p.repetition_penalty, pres = p.presence_penalty, freq = p.frequency_penalty;
  // penalties_active (sampling.rs:332-337); apply_penalties returns early on
  // an empty history (:858)
  const bool pen = std::fabs(rep - 1.0f) >= kF32Eps || pres != 0.0f || freq != 0.0f;
  r.window = p.repeat_last_n > 0xffffffffull ? 0xffffffffu : (uint32_t)p.repeat_last_n;
  r.rep = rep;
  r.presence = pres;
  r.freq = freq;
  if (pen && has_window) r.flags |= lumen::kPen;
  if (std::fabs(rep - 1.0f) >= kF32Eps) r.flags |= lumen::kRep;
  if (p.temperature <= 0.0f) {  // greedy branch (sampling.rs:468-476)
    r.flags |= lumen::kGreedy;
    if (p.anti_restate) r.flags |= lumen::kAnti;
    return;
  }
  if (p.top_k > 0 && p.top_k < (uint64_t)V) {  // sampling.rs:492-496
    r.flags |= lumen::kTopK;
    r.top_k = (uint32_t)p.top_k;
  }
  if (p.top_p > 0.0f && p.top_p < 1.0f) {  // sampling.rs:502-506
    r.flags |= lumen::kTopP;
    r.top_p = p.top_p;
  }
  if (p.min_p > 0.0f) {  // sampling.rs:510-514; ln() as in :989
    r.flags |= lumen::kMinP;
    r.log_min_p = logf(p.min_p);
  }
  r.inv_temp = 1.0f / p.temperature;  // sampling.rs:517
  return;
}

// Form A: counts over the last repeat_last_n ids of the history
// (sampling.rs:860-878), appended as (id, count) with ascending ids.
void count_window(lumen_sampler* s, const uint32_t* h, uint64_t len, uint64_t window) {
  uint64_t start = 0;
  if (window > 0 && window < len) start = len - window;
  s->tmp.assign(h + start, h + len);
  std::sort(s->tmp.begin(), s->tmp.end());
  for (size_t i = 0; i < s->tmp.size();) {
    size_t j = i;
    while (j < s->tmp.size() && s->tmp[j] == s->tmp[i]) ++j;
    s->ids.push_back(s->tmp[i]);
    s->cnts.push_back((uint32_t)(j - i));
    i = j;
  }
}

// ---- anti-restate rules (sampling.rs:552-836) ----
constexpr int kAntiMaxSkip = 8;          // ANTI_RESTATE_MAX_SKIP
constexpr size_t kLoopWindow = 28;       // ANTI_RESTATE_LOOP_WINDOW
constexpr size_t kLoopThresh = 5;        // ANTI_RESTATE_LOOP_THRESH
constexpr size_t kMinSuffix = 4;         // ANTI_RESTATE_MIN_SUFFIX
constexpr size_t kMinSpan = 3, kMaxSpan = 8;  // ANTI_RESTATE_{MIN,MAX}_SPAN

struct AntiRules {
  bool subword, ngram, loop;
};

// A rule is on unless its variable reads 0 / false / no / off (sampling.rs:631-636).
bool rule_on(const char* name) {
  const char* e = std::getenv(name);
  if (!e) return true;
  return std::strcmp(e, "0") != 0 && std::strcmp(e, "false") != 0 && std::strcmp(e, "no") != 0 &&
         std::strcmp(e, "off") != 0;
}

// Resolved once per process (sampling.rs:638-651).
const AntiRules& anti_rules() {
  static const AntiRules r{rule_on("LUMEN_ANTI_RESTATE_SUBWORD"), rule_on("LUMEN_ANTI_RESTATE_NGRAM"),
                           rule_on("LUMEN_ANTI_RESTATE_LOOP")};
  return r;
}

// u8::is_ascii_whitespace: space, \t, \n, \x0C, \r (not \x0B)
bool ascii_ws(uint8_t c) { return c == ' ' || c == '\t' || c == '\n' || c == 0x0C || c == '\r'; }

struct Bytes {
  const uint8_t* p;
  size_t n;
};

Bytes token_bytes(const lumen_token_bytes* d, uint32_t id) {
  if (!d || !d->offsets || id >= d->count) return {nullptr, 0};
  const uint64_t lo = d->offsets[id], hi = d->offsets[id + 1];
  if (hi <= lo || !d->data) return {nullptr, 0};
  return {d->data + lo, (size_t)(hi - lo)};
}

// sampling.rs:732-780
bool restates_subword(uint32_t cand, const uint32_t* h, size_t hl, const lumen_token_bytes* d) {
  if (!d || hl == 0) return false;
  const Bytes c = token_bytes(d, cand);
  if (c.n == 0) return false;
  for (size_t i = 0; i < c.n; ++i)
    if (ascii_ws(c.p[i])) return false;
  const Bytes prev = token_bytes(d, h[hl - 1]);
  if (prev.n == 0) return false;
  size_t tail = 0;
  for (size_t i = prev.n; i > 0; --i)
    if (ascii_ws(prev.p[i - 1])) {
      tail = i;
      break;
    }
  const uint8_t* word = prev.p + tail;
  const size_t wl = prev.n - tail;
  if (wl < kMinSuffix) return false;
  for (size_t sl = wl; sl >= kMinSuffix; --sl)
    if (c.n >= sl && std::memcmp(c.p, word + (wl - sl), sl) == 0) return true;
  return false;
}

// sampling.rs:819-836
bool restates_ngram(uint32_t cand, const uint32_t* h, size_t hl) {
  for (size_t k = kMinSpan; k <= kMaxSpan; ++k) {
    if (hl + 1 < 2 * k) continue;
    const size_t w0 = hl - (k - 1), p0 = hl - (2 * k - 1);
    if (std::equal(h + w0, h + hl, h + p0) && cand == h[p0 + k - 1]) return true;
  }
  return false;
}

// sampling.rs:693-701
bool runaway_loop(uint32_t cand, const uint32_t* h, size_t hl) {
  if (hl < kLoopThresh) return false;
  const size_t start = hl > kLoopWindow ? hl - kLoopWindow : 0;
  return (size_t)std::count(h + start, h + hl, cand) >= kLoopThresh;
}

// sampling.rs:657-662
bool degenerate(uint32_t cand, const uint32_t* h, size_t hl, const lumen_token_bytes* d) {
  const AntiRules& r = anti_rules();
  return (r.subword && restates_subword(cand, h, hl, d)) || (r.ngram && restates_ngram(cand, h, hl)) ||
         (r.loop && runaway_loop(cand, h, hl));
}

}  // namespace

extern "C" {

uint32_t lumen_anti_restate_select(const uint32_t* cands, const uint32_t* history,
                                   uint64_t history_len, const lumen_token_bytes* decoder) {
  if (!cands) return LUMEN_TOKEN_ERROR;
  const uint32_t raw = cands[0];
  if (history_len == 0 || !history) return raw;  // sampling.rs:566-568
  uint32_t cand = raw;
  int j = 1;
  for (int probe = 0; probe < kAntiMaxSkip; ++probe) {  // sampling.rs:571-583
    if (!degenerate(cand, history, (size_t)history_len, decoder)) return cand;
    // argmax_excluding: the next finite candidate not yet probed
    while (j < lumen::kGuardWords && cands[j] == raw) ++j;
    if (j >= lumen::kGuardWords || cands[j] == lumen::kGuardNone) break;
    cand = cands[j++];
  }
  return raw;
}

uint64_t lumen_xorshift64_new(uint64_t seed) {
  // sampling.rs:64-83
  uint64_t base = seed == 0 ? 0xDEADBEEFCAFEBABEull : seed;
  uint64_t x = base + 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  x ^= x >> 31;
  return x == 0 ? 0xDEADBEEFCAFEBABEull : x;
}

uint64_t lumen_xorshift64_next_u64(uint64_t* state) {
  // sampling.rs:86-93
  uint64_t x = *state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *state = x;
  return x;
}

float lumen_xorshift64_next_f32(uint64_t* state) {
  // sampling.rs:96-99
  const float scale = 1.0f / (float)(1ull << 24);
  return (float)(lumen_xorshift64_next_u64(state) >> 40) * scale;
}

const char* lumen_sampler_version(void) { return "lumen_sampler 0.1.0 gfx950"; }

const char* lumen_sampler_last_error(void) { return g_last_error; }

int lumen_sampling_params_validate(const lumen_sampling_params* p) {
  if (!p) return fail(LUMEN_ERR_INVALID, "null params");
  const float t = p->temperature, q = p->top_p;
  // crates/lumen-server/src/wire/openai.rs:361-378: NaN and infinities fail the range test too
  if (!std::isfinite(t) || !(t >= 0.0f && t <= 2.0f))
    return fail(LUMEN_ERR_INVALID, "temperature must be between 0 and 2");
  if (!std::isfinite(q) || !(q >= 0.0f && q <= 1.0f))
    return fail(LUMEN_ERR_INVALID, "top_p must be between 0 and 1");
  return LUMEN_OK;
}

int lumen_sampler_create(lumen_sampler** out, int device) {
  if (!out) return LUMEN_ERR_INVALID;
  *out = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return LUMEN_ERR_NO_DEVICE;
  if (device < 0 || device >= ndev) return LUMEN_ERR_INVALID;
  DeviceGuard g(device);
  lumen_sampler* s = new (std::nothrow) lumen_sampler();
  if (!s) return LUMEN_ERR_INVALID;
  s->device = device;
  std::vector<char> file;
  const void* image = lumen_gfx950_code_object;
  if (const char* path = std::getenv("LUMEN_SAMPLER_CODE_OBJECT")) {
    FILE* f = std::fopen(path, "rb");
    if (!f) {
      delete s;
      return LUMEN_ERR_CODE_OBJECT;
    }
    char buf[65536];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) file.insert(file.end(), buf, buf + n);
    std::fclose(f);
    if (file.empty()) {
      delete s;
      return LUMEN_ERR_CODE_OBJECT;
    }
    image = file.data();
  } else if (lumen_gfx950_code_object_end == lumen_gfx950_code_object) {
    delete s;
    return LUMEN_ERR_CODE_OBJECT;
  }
  if (hipModuleLoadData(&s->module, image) != hipSuccess) {
    (void)hipGetLastError();
    delete s;
    return LUMEN_ERR_CODE_OBJECT;
  }
  if (hipModuleGetFunction(&s->fn, s->module, "lumen_sample_rows") != hipSuccess ||
      hipModuleGetFunction(&s->fn_hist, s->module, "lumen_hist_window") != hipSuccess ||
      hipModuleGetFunction(&s->fn_zero, s->module, "lumen_zero_tokens") != hipSuccess ||
      hipModuleGetFunction(&s->fn_single, s->module, "lumen_sample_rows_single") != hipSuccess) {
    (void)hipGetLastError();
    (void)hipModuleUnload(s->module);
    delete s;
    return LUMEN_ERR_CODE_OBJECT;
  }
  {
    // a code object built from another layout of kernel_abi.h would read
    // its arguments at the wrong offsets: refuse it
    hipDeviceptr_t gp = nullptr;
    size_t gsz = 0;
    uint32_t stamp = 0;
    const bool got = hipModuleGetGlobal(&gp, &gsz, s->module, "lumen_kernel_abi") == hipSuccess &&
                     gsz == sizeof(uint32_t) && hipMemcpyDtoH(&stamp, gp, sizeof(stamp)) == hipSuccess;
    if (!got || stamp != lumen::kAbiStamp) {
      (void)hipGetLastError();
      (void)hipModuleUnload(s->module);
      delete s;
      return fail(LUMEN_ERR_CODE_OBJECT, "code object built for another kernel ABI (rebuild it)");
    }
  }
  if (hipDeviceGetAttribute(&s->cu_count, hipDeviceAttributeMultiprocessorCount, device) !=
      hipSuccess)
    s->cu_count = 0;
  {
    int per_cu = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, s->fn, 1024, 0) != hipSuccess)
      per_cu = 0;
    s->max_resident = per_cu * s->cu_count;
  }
  {
    // the no-allocation entry point's scratch array on this device
    void* na = nullptr;
    if (lumen::noalloc_scratch(&na) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipModuleUnload(s->module);
      delete s;
      return LUMEN_ERR_HIP;
    }
  }
  if (hipEventCreateWithFlags(&s->staged, hipEventDisableTiming) != hipSuccess) {
    (void)hipModuleUnload(s->module);
    delete s;
    return LUMEN_ERR_HIP;
  }
  if (hipMalloc(reinterpret_cast<void**>(&s->timeouts_dev), 256) != hipSuccess ||
      hipMemset(s->timeouts_dev, 0, 256) != hipSuccess) {
    (void)hipGetLastError();
    if (s->timeouts_dev) (void)hipFree(s->timeouts_dev);
    (void)hipEventDestroy(s->staged);
    (void)hipModuleUnload(s->module);
    delete s;
    return LUMEN_ERR_HIP;
  }
  *out = s;
  return LUMEN_OK;
}

int lumen_sampler_set_wait_limit(lumen_sampler* s, uint32_t microseconds) {
  if (!s) return fail(LUMEN_ERR_INVALID, "null context");
  s->wait_us = microseconds;
  return LUMEN_OK;
}

int lumen_sampler_wait_timeouts(lumen_sampler* s, uint64_t* count) {
  if (!s || !count) return fail(LUMEN_ERR_INVALID, "null context or count");
  DeviceGuard g(s->device);
  uint32_t n = 0;
  const hipError_t e = hipMemcpy(&n, s->timeouts_dev, sizeof n, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e);
  *count = n;
  return LUMEN_OK;
}

namespace {
// The no-allocation array of each GPU belongs to one context at a time: the
// first context that makes a no-allocation call on the GPU, until it is
// destroyed. Calls from any other context are refused, so two contexts
// cannot overlap on the array; a context itself is used on one stream at a
// time (the header's convention), which serializes its own calls.
std::mutex g_na_mu;
lumen_sampler* g_na_owner[64] = {};

bool noalloc_claim(lumen_sampler* s) {
  if (s->device < 0 || s->device >= 64) return false;
  std::lock_guard<std::mutex> lk(g_na_mu);
  if (!g_na_owner[s->device]) g_na_owner[s->device] = s;
  return g_na_owner[s->device] == s;
}

void noalloc_release(lumen_sampler* s) {
  if (s->device < 0 || s->device >= 64) return;
  std::lock_guard<std::mutex> lk(g_na_mu);
  if (g_na_owner[s->device] == s) g_na_owner[s->device] = nullptr;
}
}  // namespace

void lumen_sampler_destroy(lumen_sampler* s) {
  if (!s) return;
  DeviceGuard g(s->device);
  (void)hipDeviceSynchronize();
  noalloc_release(s);
  if (s->pin) (void)hipHostFree(s->pin);
  if (s->stage.p) (void)hipFree(s->stage.p);
  if (s->pen_scratch.p) (void)hipFree(s->pen_scratch.p);
  if (s->ws.p) (void)hipFree(s->ws.p);
  if (s->cand.p) (void)hipFree(s->cand.p);
  if (s->est.p) (void)hipFree(s->est.p);
  if (s->hist.p) (void)hipFree(s->hist.p);
  if (s->guard.p) (void)hipFree(s->guard.p);
  if (s->wcnt.p) (void)hipFree(s->wcnt.p);
  if (s->staged) (void)hipEventDestroy(s->staged);
  if (s->module) (void)hipModuleUnload(s->module);
  if (s->map_host) (void)hipHostFree(s->map_host);
  if (s->timeouts_dev) (void)hipFree(s->timeouts_dev);
  delete s;
}

namespace {
int launch_batch(lumen_sampler* s, const lumen_batch* bt, lumen_stream stream, uint32_t* tok_map,
                 uint32_t* done_map, uint32_t* guard_map, bool sync, bool noalloc = false);

}  // namespace

int lumen_sampler_sample_batch(lumen_sampler* s, const lumen_batch* bt, lumen_stream stream) {
  return launch_batch(s, bt, stream, nullptr, nullptr, nullptr, false);
}

int lumen_sampler_sample_batch_noalloc(lumen_sampler* s, const lumen_batch* bt, lumen_stream stream) {
  return launch_batch(s, bt, stream, nullptr, nullptr, nullptr, false, true);
}

namespace {
// Device buffers of the no-allocation entry point, carved in order from the
// scratch array (256-byte aligned pieces).
struct Arena {
  char* base = nullptr;
  size_t used = 0;
  void* take(size_t bytes) {
    const size_t at = (used + 255) & ~size_t(255);
    if (at + bytes > lumen::kNoAllocBytes) return nullptr;
    used = at + bytes;
    return base + at;
  }
};

int launch_batch(lumen_sampler* s, const lumen_batch* bt, lumen_stream stream, uint32_t* tok_map,
                 uint32_t* done_map, uint32_t* guard_map, bool sync, bool noalloc) {
  if (!s || !bt) return fail(LUMEN_ERR_INVALID, "null context or batch");
  const uint32_t B = bt->batch, V = bt->vocab;
  if (noalloc) {
    if (!noalloc_claim(s))
      return fail(LUMEN_ERR_INVALID,
                  "noalloc: this GPU's no-allocation array belongs to another context (one context "
                  "per GPU may use it, until that context is destroyed)");
    if (B > lumen::kNoAllocMaxRows) return fail(LUMEN_ERR_INVALID, "noalloc: batch must be at most 8 rows");
    if (V > lumen::kNoAllocMaxVocab) return fail(LUMEN_ERR_INVALID, "noalloc: vocab must be at most 262144");
    if (bt->hist_ring_dev) return fail(LUMEN_ERR_INVALID, "noalloc: hist_ring_dev is not supported");
  }
  if (B == 0) return LUMEN_OK;
  if (!bt->params || !bt->tokens) return fail(LUMEN_ERR_INVALID, "params and tokens are required");
  if (bt->dtype != LUMEN_DTYPE_F32 && bt->dtype != LUMEN_DTYPE_BF16)
    return fail(LUMEN_ERR_INVALID, "dtype must be LUMEN_DTYPE_F32 or LUMEN_DTYPE_BF16");
  if (V > 0 && (!bt->logits || bt->row_stride < V))
    return fail(LUMEN_ERR_INVALID, "logits missing or row_stride < vocab");
  // draws made on the device: caller-resident uniforms, or the device RNG
  const bool dev_draws = bt->uniforms_dev || bt->rng_states_dev;
  if (!bt->uniforms && !bt->rng_states && !dev_draws) {
    for (uint32_t b = 0; b < B; ++b)
      if (bt->params[b].temperature > 0.0f)
        return fail(LUMEN_ERR_INVALID, "sampled rows need uniforms or rng_states");
  }
  if (bt->pen_offsets && (!bt->pen_ids || !bt->pen_counts))
    return fail(LUMEN_ERR_INVALID, "pen_offsets needs pen_ids and pen_counts");
  if (bt->history_offsets && !bt->history && bt->history_offsets[B] > 0)
    return fail(LUMEN_ERR_INVALID, "history_offsets without history");
  const bool ring = bt->hist_ring_dev != nullptr;
  if (ring) {
    if (!bt->hist_len_dev) return fail(LUMEN_ERR_INVALID, "hist_ring_dev needs hist_len_dev");
    if (bt->hist_cap == 0 || bt->hist_cap > lumen::kRingMaxCap)
      return fail(LUMEN_ERR_INVALID, "hist_cap must be between 1 and 8192");
    if (bt->pen_offsets || bt->history_offsets)
      return fail(LUMEN_ERR_INVALID, "hist_ring_dev excludes history_offsets and pen_offsets");
  }
  DeviceGuard g(s->device);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  Arena arena;
  lumen::RowWs* na_ws = nullptr;
  if (noalloc) {
    void* p = nullptr;
    if (lumen::noalloc_scratch(&p) != hipSuccess) return fail(LUMEN_ERR_HIP, "noalloc: scratch address");
    arena.base = static_cast<char*>(p);
    // The row coordination blocks sit first, at the same place in every
    // call: zero when the code object is loaded, and every launch leaves
    // them zero (each row's last workgroup restores its block), so nothing
    // is cleared per call.
    na_ws = static_cast<lumen::RowWs*>(arena.take(sizeof(lumen::RowWs) * lumen::kNoAllocMaxRows));
  }

  // rows, draws, penalty windows (host side)
  std::vector<RowParams> rows(B);
  std::vector<float> draws(B, 0.0f);
  s->ids.clear();
  s->cnts.clear();
  s->offs.assign(B + 1, 0);
  bool any_pen = false;
  bool any_anti = false;
  for (uint32_t b = 0; b < B; ++b) {
    const lumen_sampling_params& p = bt->params[b];
    bool has_window = false;
    uint64_t h0 = 0, h1 = 0;
    if (ring) {
      has_window = true;  // counted on the device; an empty window applies nothing
    } else if (!bt->pen_offsets && bt->history_offsets) {
      h0 = bt->history_offsets[b];
      h1 = bt->history_offsets[b + 1];
      if (h1 < h0) return fail(LUMEN_ERR_INVALID, "history_offsets must be non-decreasing");
      has_window = h1 > h0;
    } else if (bt->pen_offsets) {
      has_window = true;  // an empty count range applies nothing either way
    }
    resolve_row(p, V, has_window, rows[b]);
    if (rows[b].flags & lumen::kAnti) {
      any_anti = true;
      if (sync && (bt->pen_offsets || ring))
        return fail(LUMEN_ERR_UNSUPPORTED,
                    "anti_restate rows need the token history (history_offsets) in a synchronous call");
      if (!sync && !bt->guard_out)
        return fail(LUMEN_ERR_INVALID, "anti_restate rows need guard_out in an asynchronous call");
    }
    if (!bt->pen_offsets && !ring && (rows[b].flags & lumen::kPen))
      count_window(s, bt->history + h0, h1 - h0, p.repeat_last_n);
    s->offs[b + 1] = (uint32_t)s->ids.size();
    any_pen |= (rows[b].flags & lumen::kPen) != 0;
    if (V > 0 && !dev_draws && !(rows[b].flags & lumen::kGreedy)) {
      // exactly one draw per sampled row (sampling.rs:1004)
      draws[b] = bt->rng_states ? lumen_xorshift64_next_f32(&bt->rng_states[b]) : bt->uniforms[b];
    }
  }
  if (V == 0) {
    // sampling.rs:458-460: empty logits sample token 0 and draw nothing;
    // Sampler::sample records it (sampling.rs:429-433), so in form C the
    // kernel also appends 0 to each row's ring. A kernel (no staging copy,
    // no memset node) keeps the call capturable and allocation-free.
    s->any_anti = false;
    lumen::ZeroArgs za{};
    za.tokens = bt->tokens;
    za.n = B;
    za.ring = bt->hist_ring_dev;
    za.ring_len = bt->hist_len_dev;
    za.ring_cap = bt->hist_cap;
    size_t zs = sizeof(za);
    void* zc[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &za, HIP_LAUNCH_PARAM_BUFFER_SIZE, &zs, HIP_LAUNCH_PARAM_END};
    return hip_fail(hipModuleLaunchKernel(s->fn_zero, (B + 255) / 256, 1, 1, 256, 1, 1, 0,
                                          reinterpret_cast<hipStream_t>(stream), nullptr, zc));
  }

  KernelArgs ka;
  std::memset(&ka, 0, sizeof(ka));
  ka.logits = bt->logits;
  ka.row_stride = bt->row_stride;
  ka.vocab = V;
  ka.batch = B;
  ka.dtype = bt->dtype;
  ka.tokens = bt->tokens;
  ka.trace = reinterpret_cast<lumen::RowTrace*>(bt->trace);
  ka.pen_out = bt->penalized_out;
  ka.wait_ticks = (uint32_t)std::min<uint64_t>(100ull * s->wait_us, 0xffffffffull);
  ka.timeouts = s->timeouts_dev;

  // Workgroups per row: enough to occupy every CU once (all co-resident),
  // at most kMaxSlices. With 8+ rows, a row's slices share one XCD.
  uint32_t G = 1;
  const uint32_t padded = B >= 8 ? ((B + 7u) / 8u) * 8u : B;
  if (s->max_resident > 0 && std::getenv("LUMEN_SAMPLER_SINGLE") == nullptr)
    G = std::max<uint32_t>(1u, std::min<uint32_t>(lumen::kMaxSlices,
                                                  (uint32_t)s->max_resident / padded));
  ka.slices = G;
  ka.xcd_rows = (B >= 8 && G > 1) ? 1u : 0u;
  uint32_t nblocks = G == 1 ? B : (ka.xcd_rows ? padded * G : B * G);
  if (G > 1 && B >= 8 && !noalloc) {
    const uint32_t nb = plan_blocks(rows, V, (uint32_t)s->max_resident, G, s->blk_map);
    if (nb) {
      nblocks = nb;
      ka.slices = lumen::kMaxSlices;  // buffers are sized for the largest G
    }
  } else {
    s->blk_map.clear();
  }
  // Staging. Two blocks share one pinned host buffer and one device buffer:
  //   static block [params][offs][ids][cnts]: copied only when its bytes
  //                differ from what the device buffer already holds;
  //   draw block   [uniforms]: copied every call unless the draws are inline
  //                kernel arguments or already in device memory.
  const bool inl = B <= (uint32_t)lumen::kInlineRows;
  const bool host_csr = !bt->pen_offsets && !ring;
  auto a16 = [](size_t x) { return (x + 15) & ~size_t(15); };
  const size_t off_offs = inl ? 0 : a16(sizeof(RowParams) * B);
  const size_t off_ids = off_offs + (host_csr ? sizeof(uint32_t) * (B + 1) : 0);
  const size_t off_cnts = off_ids + (host_csr ? sizeof(uint32_t) * s->ids.size() : 0);
  const size_t off_map = a16(off_cnts + (host_csr ? sizeof(uint32_t) * s->cnts.size() : 0));
  const size_t static_sz = a16(off_map + sizeof(uint32_t) * s->blk_map.size());
  const bool draw_block = !dev_draws && !inl;
  const size_t total = static_sz + (draw_block ? sizeof(float) * B : 0);
  if (inl) {
    ka.inline_rows = B;
    for (uint32_t b = 0; b < B; ++b) ka.inline_params[b] = rows[b];
  }
  if (bt->uniforms_dev) {
    ka.uniforms = bt->uniforms_dev;
  } else if (bt->rng_states_dev) {
    ka.rng_dev = bt->rng_states_dev;
  } else if (inl) {
    ka.inline_draws = 1;
    for (uint32_t b = 0; b < B; ++b) ka.inline_uniforms[b] = draws[b];
  }
  if (total > 0 && noalloc) {
    // the penalty counts of form A into the scratch array (inline rows and
    // draws need nothing else); the copy reads pageable host memory, which
    // HIP stages before hipMemcpyAsync returns
    if (s->ids.size() > lumen::kNoAllocMaxCsr)
      return fail(LUMEN_ERR_INVALID, "noalloc: more than 65536 form-A penalty entries");
    // a captured copy would read this host buffer at every replay, after
    // later calls have refilled (or moved) it
    if (capturing(st))
      return fail(LUMEN_ERR_INVALID,
                  "noalloc under stream capture: form-A histories (history_offsets) need a host "
                  "copy; pass device penalty counts (pen_offsets) instead");
    s->img.assign(static_sz, 0);
    std::memcpy(s->img.data() + off_offs, s->offs.data(), sizeof(uint32_t) * (B + 1));
    if (!s->ids.empty()) {
      std::memcpy(s->img.data() + off_ids, s->ids.data(), sizeof(uint32_t) * s->ids.size());
      std::memcpy(s->img.data() + off_cnts, s->cnts.data(), sizeof(uint32_t) * s->cnts.size());
    }
    char* dp = static_cast<char*>(arena.take(static_sz));
    if (!dp) return fail(LUMEN_ERR_INVALID, "noalloc: scratch too small");
    if (hipMemcpyAsync(dp, s->img.data(), static_sz, hipMemcpyHostToDevice, st) != hipSuccess)
      return fail(LUMEN_ERR_HIP, "staging copy");
    ka.hist_off = reinterpret_cast<const uint32_t*>(dp + off_offs);
    ka.hist_ids = reinterpret_cast<const uint32_t*>(dp + off_ids);
    ka.hist_cnt = reinterpret_cast<const uint32_t*>(dp + off_cnts);
  } else if (total > 0) {
    s->img.assign(static_sz, 0);
    if (!inl) std::memcpy(s->img.data(), rows.data(), sizeof(RowParams) * B);
    if (!s->blk_map.empty())
      std::memcpy(s->img.data() + off_map, s->blk_map.data(), sizeof(uint32_t) * s->blk_map.size());
    if (host_csr) {
      std::memcpy(s->img.data() + off_offs, s->offs.data(), sizeof(uint32_t) * (B + 1));
      if (!s->ids.empty()) {
        std::memcpy(s->img.data() + off_ids, s->ids.data(), sizeof(uint32_t) * s->ids.size());
        std::memcpy(s->img.data() + off_cnts, s->cnts.data(), sizeof(uint32_t) * s->cnts.size());
      }
    }
    const size_t dev_cap_before = s->stage.cap;
    int rc = ensure_dev(s->stage, total, st);
    if (rc != LUMEN_OK) return rc;
    if (s->stage.cap != dev_cap_before) s->last_img.clear();  // new device buffer
    const bool copy_static = static_sz > 0 && s->img != s->last_img;
    if (copy_static || draw_block) {
      if (capturing(st)) return fail(LUMEN_ERR_INVALID, kCaptureMsg);
      if (s->staged_pending) {
        if (hipEventSynchronize(s->staged) != hipSuccess) return fail(LUMEN_ERR_HIP, "staging wait");
        s->staged_pending = false;
      }
      if (s->pin_cap < total) {
        if (s->pin) (void)hipHostFree(s->pin);
        s->pin = nullptr;
        s->pin_cap = 0;
        size_t cap = std::max<size_t>(total, 65536);
        if (hipHostMalloc(&s->pin, cap, hipHostMallocDefault) != hipSuccess)
          return fail(LUMEN_ERR_HIP, "pinned staging allocation");
        s->pin_cap = cap;
      }
      char* hp = static_cast<char*>(s->pin);
      char* dp = static_cast<char*>(s->stage.p);
      size_t lo = copy_static ? 0 : static_sz;
      if (copy_static) std::memcpy(hp, s->img.data(), static_sz);
      if (draw_block) std::memcpy(hp + static_sz, draws.data(), sizeof(float) * B);
      if (hipMemcpyAsync(dp + lo, hp + lo, total - lo, hipMemcpyHostToDevice, st) != hipSuccess)
        return fail(LUMEN_ERR_HIP, "staging copy");
      if (hipEventRecord(s->staged, st) != hipSuccess) return fail(LUMEN_ERR_HIP, "event record");
      s->staged_pending = true;
      if (copy_static) s->last_img = s->img;
    }
    char* dp = static_cast<char*>(s->stage.p);
    if (!inl) ka.params = reinterpret_cast<const RowParams*>(dp);
    if (!s->blk_map.empty()) ka.blk_map = reinterpret_cast<const uint32_t*>(dp + off_map);
    if (draw_block) ka.uniforms = reinterpret_cast<const float*>(dp + static_sz);
    if (host_csr) {
      ka.hist_off = reinterpret_cast<const uint32_t*>(dp + off_offs);
      ka.hist_ids = reinterpret_cast<const uint32_t*>(dp + off_ids);
      ka.hist_cnt = reinterpret_cast<const uint32_t*>(dp + off_cnts);
    }
  }
  if (ring) {
    uint32_t ccap = bt->hist_cap;
    for (uint32_t b = 0; b < B; ++b)
      if ((rows[b].flags & lumen::kPen) && (rows[b].window == 0u || rows[b].window > bt->hist_cap))
        ccap = std::max<uint32_t>(ccap, V);
    RingLayout L;
    int rc = ring_layout(s, B, bt->hist_cap, ccap, st, L);
    if (rc != LUMEN_OK) return rc;
    ka.hist_state = L.state;
    ka.hist_off = L.off;
    ka.hist_end = L.end;
    ka.hist_ids = L.ids;
    ka.hist_cnt = L.cnt;
    ka.count_cap = ccap;
    ka.ring = bt->hist_ring_dev;
    ka.ring_len = bt->hist_len_dev;
    ka.ring_cap = bt->hist_cap;
    ka.ring_epoch = bt->hist_epoch;
  } else if (!host_csr) {
    ka.hist_off = bt->pen_offsets;
    ka.hist_ids = bt->pen_ids;
    ka.hist_cnt = bt->pen_counts;
  }
  if (any_pen) {
    const uint64_t stride = ((uint64_t)V + 63) & ~uint64_t(63);
    if (noalloc) {
      ka.pen_scratch = static_cast<float*>(arena.take(sizeof(float) * stride * B));
      if (!ka.pen_scratch) return fail(LUMEN_ERR_INVALID, "noalloc: scratch too small");
    } else {
      int rc = ensure_dev(s->pen_scratch, sizeof(float) * stride * B, st);
      if (rc != LUMEN_OK) return rc;
      ka.pen_scratch = static_cast<float*>(s->pen_scratch.p);
    }
    ka.pen_stride = stride;
  }
  ka.tokens_mapped = tok_map;
  ka.done_mapped = done_map;
  if (any_anti) {
    if (bt->guard_out) {
      ka.guard = bt->guard_out;
    } else if (noalloc) {
      return fail(LUMEN_ERR_INVALID, "noalloc: anti_restate rows need guard_out");
    } else {
      int rc = ensure_dev(s->guard, sizeof(uint32_t) * lumen::kGuardWords * B, st);
      if (rc != LUMEN_OK) return rc;
      ka.guard = static_cast<uint32_t*>(s->guard.p);
    }
    ka.guard_mapped = guard_map;
    s->guard_dev = ka.guard;
  }
  s->any_anti = any_anti;
  if (ring) {
    // the window counts of every row, ahead of the sampler on the same stream
    size_t hsz = sizeof(ka);
    void* hcfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &ka, HIP_LAUNCH_PARAM_BUFFER_SIZE, &hsz,
                    HIP_LAUNCH_PARAM_END};
    hipError_t e = hipModuleLaunchKernel(s->fn_hist, B, 1, 1, 1024, 1, 1, 0, st, nullptr, hcfg);
    if (e != hipSuccess) return hip_fail(e);
  }
  if (G > 1 && noalloc) {
    ka.ws = na_ws;
    ka.cand = static_cast<uint64_t*>(arena.take(sizeof(uint64_t) * lumen::kCandStride * B));
    ka.est = static_cast<uint32_t*>(arena.take(sizeof(uint32_t) * lumen::kRecWords * lumen::kRowRecs * B));
    ka.hist = static_cast<float*>(arena.take(sizeof(float) * lumen::kMaxSlices * lumen::kMassBins * B));
    if (!ka.ws || !ka.cand || !ka.est || !ka.hist) return fail(LUMEN_ERR_INVALID, "noalloc: scratch too small");
  } else if (G > 1) {
    const size_t ws_bytes = sizeof(lumen::RowWs) * B;
    if (s->ws.cap < ws_bytes) {
      int rc = ensure_dev(s->ws, ws_bytes, st);
      if (rc != LUMEN_OK) return rc;
      // zero once at allocation; afterwards each launch leaves it zeroed
      if (hipMemset(s->ws.p, 0, s->ws.cap) != hipSuccess) return fail(LUMEN_ERR_HIP, "workspace init");
    }
    int rc = ensure_dev(s->cand, sizeof(uint64_t) * lumen::kCandStride * B, st);
    if (rc != LUMEN_OK) return rc;
    rc = ensure_dev(s->est, sizeof(uint32_t) * lumen::kRecWords * lumen::kRowRecs * B, st);
    if (rc != LUMEN_OK) return rc;
    ka.ws = static_cast<lumen::RowWs*>(s->ws.p);
    ka.cand = static_cast<uint64_t*>(s->cand.p);
    ka.est = static_cast<uint32_t*>(s->est.p);
    rc = ensure_dev(s->hist, sizeof(float) * lumen::kMaxSlices * lumen::kMassBins * B, st);
    if (rc != LUMEN_OK) return rc;
    ka.hist = static_cast<float*>(s->hist.p);
    // Every wait inside the kernel is bounded and reports a row failure on
    // timeout, so an ordinary launch is safe; a cooperative launch (which
    // guarantees co-residency of the grid) costs ~18 us more per call and is
    // opt-in through LUMEN_SAMPLER_COOP.
    if (std::getenv("LUMEN_SAMPLER_COOP") != nullptr) {
      void* params[] = {&ka};
      hipError_t e =
          hipModuleLaunchCooperativeKernel(s->fn, nblocks, 1, 1, 1024, 1, 1, 0, st, params);
      return hip_fail(e);
    }
  }
  size_t argsz = sizeof(ka);
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &ka, HIP_LAUNCH_PARAM_BUFFER_SIZE, &argsz,
                 HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(G == 1 ? s->fn_single : s->fn, nblocks, 1, 1, 1024, 1, 1, 0,
                                       st, nullptr, cfg);
  return hip_fail(e);
}
}  // namespace

int lumen_sampler_decode_seed(lumen_sampler* s, const lumen_decode_seed* d, lumen_stream stream) {
  if (!s || !d) return fail(LUMEN_ERR_INVALID, "null context or seed");
  const uint32_t B = d->batch, cap = d->hist_cap;
  if (B == 0) return LUMEN_OK;
  if (!d->hist_ring_dev || !d->hist_len_dev) return fail(LUMEN_ERR_INVALID, "hist_ring_dev and hist_len_dev are required");
  if (cap == 0 || cap > lumen::kRingMaxCap) return fail(LUMEN_ERR_INVALID, "hist_cap must be between 1 and 8192");
  if (d->rng_states_dev && !d->rng_seed_states) return fail(LUMEN_ERR_INVALID, "rng_states_dev needs rng_seed_states");
  if (d->prompt_offsets && !d->prompt_ids && d->prompt_offsets[B] > d->prompt_offsets[0])
    return fail(LUMEN_ERR_INVALID, "prompt_offsets without prompt_ids");
  DeviceGuard g(s->device);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (capturing(st)) return fail(LUMEN_ERR_INVALID, "lumen_sampler_decode_seed cannot run under stream capture");
  auto prompt = [&](uint32_t b, const uint32_t** p, uint64_t* n) {
    *p = nullptr;
    *n = 0;
    if (!d->prompt_offsets) return true;
    const uint64_t h0 = d->prompt_offsets[b], h1 = d->prompt_offsets[b + 1];
    if (h1 < h0 || h1 - h0 > 0xfffffffeull) return false;
    *p = d->prompt_ids + h0;
    *n = h1 - h0;
    return true;
  };
  // host image: [B] u64 states | [B] lens | [B][cap] ring | window counts
  std::vector<uint32_t> lens(B), ring((size_t)B * cap, 0u);
  for (uint32_t b = 0; b < B; ++b) {
    const uint32_t* p;
    uint64_t n;
    if (!prompt(b, &p, &n)) return fail(LUMEN_ERR_INVALID, "prompt_offsets must be non-decreasing");
    lens[b] = (uint32_t)n;
    for (uint64_t k = n > cap ? n - cap : 0; k < n; ++k) ring[(size_t)b * cap + k % cap] = p[k];
  }
  // window counts (form A's counting, sampling.rs:860-878), with the state
  // words lumen_hist_window keeps: counts made at ring_len = prompt length
  RingLayout L{};
  uint32_t ccap = cap;
  std::vector<RowParams> rows(B);
  std::vector<uint32_t> head;  // [B] offsets, [B] ends, [B][8] state
  std::vector<uint32_t> rstart(B + 1, 0);
  s->ids.clear();
  s->cnts.clear();
  if (d->params) {
    for (uint32_t b = 0; b < B; ++b) {
      resolve_row(d->params[b], d->vocab, true, rows[b]);
      if ((rows[b].flags & lumen::kPen) && (rows[b].window == 0u || rows[b].window > cap))
        ccap = std::max<uint32_t>(ccap, d->vocab);
    }
    head.assign(2 * (size_t)B + 8 * (size_t)B, 0xffffffffu);
    const uint64_t rid = (uint64_t)(uintptr_t)d->hist_ring_dev;
    for (uint32_t b = 0; b < B; ++b) {
      const uint32_t base = b * ccap;
      head[b] = base;
      head[B + b] = base;
      if (rows[b].flags & lumen::kPen) {
        const uint32_t* p;
        uint64_t n;
        (void)prompt(b, &p, &n);
        const size_t k0 = s->ids.size();
        if (n > 0) count_window(s, p, n, rows[b].window);
        const size_t k = s->ids.size() - k0;
        if (k > ccap) return fail(LUMEN_ERR_INVALID, "prompt ids outside the vocabulary");
        head[B + b] = base + (uint32_t)k;
        uint32_t* sw = &head[2 * (size_t)B + 8 * (size_t)b];
        sw[0] = (uint32_t)n;
        sw[1] = rows[b].window;
        sw[2] = (uint32_t)rid;
        sw[3] = (uint32_t)(rid >> 32);
        sw[4] = cap;
        sw[5] = d->hist_epoch;
        sw[6] = ccap;
        sw[7] = 0;
      }
      rstart[b + 1] = (uint32_t)s->ids.size();
    }
    int rc = ring_layout(s, B, cap, ccap, st, L);
    if (rc != LUMEN_OK) return rc;
  }
  const size_t n_ids = s->ids.size();
  const size_t bytes = sizeof(uint64_t) * B + sizeof(uint32_t) * (B + ring.size() + head.size() + 2 * n_ids);
  if (s->staged_pending) {
    if (hipEventSynchronize(s->staged) != hipSuccess) return fail(LUMEN_ERR_HIP, "staging wait");
    s->staged_pending = false;
  }
  if (s->pin_cap < bytes) {
    if (s->pin) (void)hipHostFree(s->pin);
    s->pin = nullptr;
    s->pin_cap = 0;
    const size_t c = std::max<size_t>(bytes, 65536);
    if (hipHostMalloc(&s->pin, c, hipHostMallocDefault) != hipSuccess)
      return fail(LUMEN_ERR_HIP, "pinned staging allocation");
    s->pin_cap = c;
  }
  char* hp = static_cast<char*>(s->pin);
  auto put = [&](void* dst, const void* src, size_t n) -> bool {
    if (n == 0) return true;
    std::memcpy(hp, src, n);
    const bool ok = hipMemcpyAsync(dst, hp, n, hipMemcpyHostToDevice, st) == hipSuccess;
    hp += n;
    return ok;
  };
  bool ok = true;
  if (d->rng_states_dev) ok &= put(d->rng_states_dev, d->rng_seed_states, sizeof(uint64_t) * B);
  ok &= put(d->hist_len_dev, lens.data(), sizeof(uint32_t) * B);
  ok &= put(d->hist_ring_dev, ring.data(), sizeof(uint32_t) * ring.size());
  if (d->params) {
    ok &= put(L.off, head.data(), sizeof(uint32_t) * 2 * B);
    ok &= put(L.state, head.data() + 2 * B, sizeof(uint32_t) * 8 * B);
    for (uint32_t b = 0; b < B; ++b) {
      const size_t k0 = rstart[b], k = rstart[b + 1] - k0;
      ok &= put(L.ids + (size_t)b * ccap, s->ids.data() + k0, sizeof(uint32_t) * k);
      ok &= put(L.cnt + (size_t)b * ccap, s->cnts.data() + k0, sizeof(uint32_t) * k);
    }
  }
  if (!ok) return fail(LUMEN_ERR_HIP, "seed copy");
  if (hipEventRecord(s->staged, st) != hipSuccess) return fail(LUMEN_ERR_HIP, "event record");
  s->staged_pending = true;
  return LUMEN_OK;
}

int lumen_sampler_sample_batch_sync(lumen_sampler* s, const lumen_batch* bt, uint32_t* tokens_host,
                                    lumen_stream stream) {
  if (!tokens_host) return fail(LUMEN_ERR_INVALID, "tokens_host is required");
  if (!s || !bt) return fail(LUMEN_ERR_INVALID, "null context or batch");
  const uint32_t B = bt->batch;
  DeviceGuard g(s->device);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // The kernel writes each row's token through the mapping of a pinned host
  // buffer and counts the rows with a system-scope release, so the host waits
  // on that count (about a microsecond after the last row) instead of a copy
  // and a stream synchronization (about 15 us). A wait that outlasts its
  // bound, or a launch error, takes the copy-and-synchronize route, which
  // also reports device errors.
  if (B > s->map_cap) {
    if (s->map_host) (void)hipHostFree(s->map_host);
    s->map_host = nullptr;
    s->map_dev = nullptr;
    s->map_cap = 0;
    void* h = nullptr;
    // [0] rows written, [1 .. B] tokens, then [B][kGuardWords] guard candidates
    if (hipHostMalloc(&h, sizeof(uint32_t) * (1 + B + (size_t)lumen::kGuardWords * B),
                      hipHostMallocMapped | hipHostMallocCoherent) ==
        hipSuccess) {
      void* d = nullptr;
      if (hipHostGetDevicePointer(&d, h, 0) == hipSuccess) {
        s->map_host = static_cast<uint32_t*>(h);
        s->map_dev = static_cast<uint32_t*>(d);
        s->map_cap = B;
      } else {
        (void)hipHostFree(h);
      }
    }
  }
  const bool mapped = s->map_host != nullptr && B > 0 && bt->vocab > 0;  // V = 0 launches nothing
  if (mapped) __atomic_store_n(&s->map_host[0], 0u, __ATOMIC_RELEASE);
  int rc = mapped ? launch_batch(s, bt, stream, s->map_dev + 1, s->map_dev, s->map_dev + 1 + B, true)
                  : launch_batch(s, bt, stream, nullptr, nullptr, nullptr, true);
  if (rc != LUMEN_OK) return rc;
  bool done = false;
  if (mapped) {
    const auto t0 = std::chrono::steady_clock::now();
    for (uint32_t spin = 0;; ++spin) {
      if (__atomic_load_n(&s->map_host[0], __ATOMIC_ACQUIRE) >= B) {
        done = true;
        break;
      }
      if ((spin & 1023u) == 1023u &&
          std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(200))
        break;
    }
    if (done) std::memcpy(tokens_host, s->map_host + 1, sizeof(uint32_t) * B);
  }
  if (!done) {
    if (hipMemcpyAsync(tokens_host, bt->tokens, sizeof(uint32_t) * B, hipMemcpyDeviceToHost, st) !=
        hipSuccess)
      return LUMEN_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return LUMEN_ERR_HIP;
  }
  if (s->any_anti) {
    // the guard's rules on the host (guarded_argmax, sampling.rs:563-603)
    const uint32_t* cand = nullptr;
    std::vector<uint32_t> cbuf;
    if (done) {
      cand = s->map_host + 1 + B;
    } else {
      cbuf.resize((size_t)lumen::kGuardWords * B);
      if (hipMemcpyAsync(cbuf.data(), s->guard_dev, sizeof(uint32_t) * cbuf.size(),
                         hipMemcpyDeviceToHost, st) != hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return fail(LUMEN_ERR_HIP, "guard candidates copy");
      cand = cbuf.data();
    }
    bool changed = false;
    for (uint32_t b = 0; b < B; ++b) {
      const lumen_sampling_params& p = bt->params[b];
      if (!(p.temperature <= 0.0f && p.anti_restate) || tokens_host[b] == LUMEN_TOKEN_ERROR) continue;
      const uint32_t* h = nullptr;
      uint64_t hl = 0;
      if (bt->history_offsets) {
        h = bt->history + bt->history_offsets[b];
        hl = bt->history_offsets[b + 1] - bt->history_offsets[b];
      }
      const uint32_t tok =
          lumen_anti_restate_select(cand + (size_t)lumen::kGuardWords * b, h, hl, bt->decoder);
      if (tok != tokens_host[b]) {
        tokens_host[b] = tok;
        changed = true;
      }
    }
    if (changed) {
      // the device copy of the tokens gets the guarded choices too
      if (hipMemcpyAsync(bt->tokens, tokens_host, sizeof(uint32_t) * B, hipMemcpyHostToDevice, st) !=
              hipSuccess ||
          hipStreamSynchronize(st) != hipSuccess)
        return fail(LUMEN_ERR_HIP, "guarded token copy");
    }
  }
  for (uint32_t b = 0; b < bt->batch; ++b)
    if (tokens_host[b] == LUMEN_TOKEN_ERROR) return fail(LUMEN_ERR_ROW, "a row reported a failure (see its trace status)");
  return LUMEN_OK;
}

}  // extern "C"
