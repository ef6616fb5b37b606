/*
 * CPU oracle: C restatement of Lumen `crates/lumen-runtime/src/sampling.rs`
 * (x86_64 code path). TEST INFRASTRUCTURE ONLY -- see sampling_ref.h.
 *
 * Every function cites the reference lines it restates. f32 arithmetic is
 * done one IEEE operation at a time (built with -ffp-contract=off), and the
 * transcendental calls go to the same glibc `expf` / `logf` that Rust's
 * `f32::exp` / `f32::ln` lower to on x86_64-unknown-linux-gnu.
 */
#define _GNU_SOURCE
#include "sampling_ref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f32::total_cmp as an unsigned key (core::f32::total_cmp: flip the
 * magnitude bits of negatives, then compare as signed; equivalently flip all
 * bits of negatives and only the sign bit of non-negatives, compare as u32). */
static inline uint32_t tkey(float f) {
    uint32_t u = f2u(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* f32::max: if one operand is NaN the other is returned. */
static inline float rust_fmax(float a, float b) {
    if (isnan(a)) return b;
    if (isnan(b)) return a;
    return a > b ? a : b;
}

/* ---- Xorshift64 (sampling.rs:45-106) ---------------------------------- */

uint64_t ref_xorshift64_new(uint64_t seed) {
    /* sampling.rs:64-83: seed 0 -> fallback, then the SplitMix64 finalizer,
     * and a 0 result is mapped to the same fallback. */
    uint64_t base = seed == 0 ? 0xDEADBEEFCAFEBABEull : seed;
    uint64_t x = base + 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    x ^= x >> 31;
    return x == 0 ? 0xDEADBEEFCAFEBABEull : x;
}

uint64_t ref_xorshift64_next_u64(uint64_t *state) {
    /* sampling.rs:86-93: Marsaglia xorshift64 with shifts 13/7/17. */
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

float ref_xorshift64_next_f32(uint64_t *state) {
    /* sampling.rs:96-99: top 24 bits scaled by 2^-24. */
    const float scale = 1.0f / (float)(1ull << 24);
    return (float)(ref_xorshift64_next_u64(state) >> 40) * scale;
}

/* ---- softmax (sampling.rs:207-231, non-aarch64 path) ------------------- */

void ref_softmax_inplace(float *v, size_t n) {
    if (n == 0) return;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = rust_fmax(mx, v[i]);
    if (!isfinite(mx)) {
        float u = 1.0f / (float)n;
        for (size_t i = 0; i < n; i++) v[i] = u;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    if (sum <= 1.1920929e-7f /* f32::EPSILON */) {
        float u = 1.0f / (float)n;
        for (size_t i = 0; i < n; i++) v[i] = u;
        return;
    }
    for (size_t i = 0; i < n; i++) v[i] /= sum;
}

/* ---- argmax (sampling.rs:538-547): lowest index of the total_cmp max --- */

size_t ref_argmax(const float *v, size_t n) {
    if (n == 0) return 0;
    size_t best = 0;
    uint32_t bk = tkey(v[0]);
    for (size_t i = 1; i < n; i++) {
        uint32_t k = tkey(v[i]);
        if (k > bk) { bk = k; best = i; }
    }
    return best;
}

/* ---- sorting helpers --------------------------------------------------- */

/* Bottom-up merge sort of u64 keys, ascending. Keys used here are unique
 * (value key in the high half, index in the low half) or compared by value
 * only, so any correct sort yields the same sequence. */
static void msort_u64(uint64_t *a, size_t n) {
    if (n < 2) return;
    uint64_t *tmp = (uint64_t *)malloc(n * sizeof(uint64_t));
    uint64_t *src = a, *dst = tmp;
    /* insertion-sort runs of 16 */
    const size_t RUN = 16;
    for (size_t s = 0; s < n; s += RUN) {
        size_t e = s + RUN < n ? s + RUN : n;
        for (size_t i = s + 1; i < e; i++) {
            uint64_t x = a[i];
            size_t j = i;
            while (j > s && a[j - 1] > x) { a[j] = a[j - 1]; j--; }
            a[j] = x;
        }
    }
    for (size_t w = RUN; w < n; w *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * w) {
            size_t mid = lo + w < n ? lo + w : n;
            size_t hi = lo + 2 * w < n ? lo + 2 * w : n;
            size_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) dst[k++] = (src[j] < src[i]) ? src[j++] : src[i++];
            while (i < mid) dst[k++] = src[i++];
            while (j < hi) dst[k++] = src[j++];
        }
        uint64_t *t = src; src = dst; dst = t;
    }
    if (src != a) memcpy(a, src, n * sizeof(uint64_t));
    free(tmp);
}

/* ---- penalties (sampling.rs:332-337, 850-900) ------------------------- */

int ref_penalties_active(const ref_params *p) {
    /* sampling.rs:332-337 */
    return fabsf(p->repetition_penalty - 1.0f) >= 1.1920929e-7f ||
           p->presence_penalty != 0.0f || p->frequency_penalty != 0.0f;
}

static void apply_penalty_one(float *logits, size_t n, uint32_t tok, uint32_t count,
                              float rep, float presence, float freq) {
    /* sampling.rs:881-900 */
    size_t idx = tok;
    if (idx >= n) return;
    float v = logits[idx];
    float nv;
    if (fabsf(rep - 1.0f) >= 1.1920929e-7f) {
        nv = v > 0.0f ? v / rep : v * rep;
    } else {
        nv = v;
    }
    nv -= presence;
    float fc = freq * (float)count;
    nv -= fc;
    logits[idx] = nv;
}

void ref_apply_penalties(float *logits, size_t n, const ref_params *p,
                         const uint32_t *history, size_t hist_len) {
    /* sampling.rs:850-879. The reference iterates a HashMap of
     * (token -> count); each token is touched exactly once, so the iteration
     * order does not affect the result. Counts are taken over the last
     * `repeat_last_n` ids when it is > 0, else over the whole history. */
    float rep = p->repetition_penalty, presence = p->presence_penalty, freq = p->frequency_penalty;
    if (fabsf(rep - 1.0f) < 1.1920929e-7f && presence == 0.0f && freq == 0.0f) return;
    if (hist_len == 0) return;
    size_t start = 0;
    if (p->repeat_last_n > 0 && p->repeat_last_n < hist_len) start = hist_len - p->repeat_last_n;
    size_t m = hist_len - start;
    uint64_t *ids = (uint64_t *)malloc(m * sizeof(uint64_t));
    for (size_t i = 0; i < m; i++) ids[i] = history[start + i];
    msort_u64(ids, m);
    for (size_t i = 0; i < m;) {
        size_t j = i;
        while (j < m && ids[j] == ids[i]) j++;
        apply_penalty_one(logits, n, (uint32_t)ids[i], (uint32_t)(j - i), rep, presence, freq);
        i = j;
    }
    free(ids);
}

/* ---- top-k (sampling.rs:904-933) --------------------------------------- */

static __thread uint32_t g_topk_cutoff, g_topk_count;

void ref_apply_top_k(float *logits, size_t n, size_t k) {
    if (k == 1) {
        size_t keep = ref_argmax(logits, n);
        g_topk_cutoff = tkey(logits[keep]);
        g_topk_count = 1;
        for (size_t i = 0; i < n; i++)
            if (i != keep) logits[i] = -INFINITY;
        return;
    }
    /* Full descending sort of a copy by total_cmp; cutoff = sorted[k-1];
     * mask only values strictly below the cutoff (ties survive). */
    uint64_t *keys = (uint64_t *)malloc(n * sizeof(uint64_t));
    for (size_t i = 0; i < n; i++) keys[i] = (uint64_t)(~tkey(logits[i]));
    msort_u64(keys, n);
    uint32_t cutoff = ~(uint32_t)keys[k - 1];
    free(keys);
    uint32_t cnt = 0;
    for (size_t i = 0; i < n; i++) {
        if (tkey(logits[i]) < cutoff) logits[i] = -INFINITY;
        else cnt++;
    }
    g_topk_cutoff = cutoff;
    g_topk_count = cnt;
}

/* ---- top-p (sampling.rs:942-967) ---------------------------------------- */

static __thread uint32_t g_last_topp_kept;
static __thread float g_last_topp_sum, g_last_topp_cum, g_last_topp_cum_before;

void ref_apply_top_p_on_logits(float *logits, size_t n, float p) {
    if (n == 0) return;
    float *probs = (float *)malloc(n * sizeof(float));
    memcpy(probs, logits, n * sizeof(float));
    ref_softmax_inplace(probs, n);
    /* for the trace: the sum the softmax divided by */
    {
        float mx = -INFINITY;
        for (size_t i = 0; i < n; i++) mx = rust_fmax(mx, logits[i]);
        float s = 0.0f;
        if (isfinite(mx))
            for (size_t i = 0; i < n; i++) s += expf(logits[i] - mx);
        g_last_topp_sum = s;
    }
    /* idx.sort_by(|&a,&b| probs[b].total_cmp(&probs[a])): stable, descending
     * by prob, so equal probs keep ascending index. Key: (~probkey, idx). */
    uint64_t *keys = (uint64_t *)malloc(n * sizeof(uint64_t));
    for (size_t i = 0; i < n; i++)
        keys[i] = ((uint64_t)(~tkey(probs[i])) << 32) | (uint64_t)i;
    msort_u64(keys, n);
    float cum = 0.0f, before = 0.0f;
    size_t kept = 0;
    for (size_t rank = 0; rank < n; rank++) {
        size_t i = (size_t)(uint32_t)keys[rank];
        before = cum;
        cum += probs[i];
        kept = rank + 1;
        if (cum >= p) break;
    }
    g_last_topp_kept = (uint32_t)kept;
    g_last_topp_cum = cum;
    g_last_topp_cum_before = before;
    for (size_t rank = kept; rank < n; rank++) logits[(uint32_t)keys[rank]] = -INFINITY;
    free(keys);
    free(probs);
}

/* ---- min-p (sampling.rs:976-994) --------------------------------------- */

void ref_apply_min_p_on_logits(float *logits, size_t n, float min_p) {
    if (n == 0) return;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = rust_fmax(mx, logits[i]);
    if (!isfinite(mx)) return;
    float bound = mx + logf(min_p);
    for (size_t i = 0; i < n; i++)
        if (logits[i] < bound) logits[i] = -INFINITY;
}

/* ---- categorical draw (sampling.rs:1003-1014) -------------------------- */

static __thread float g_last_cdf_before, g_last_cdf_at;

uint32_t ref_sample_categorical(const float *probs, size_t n, float r) {
    float cumsum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float before = cumsum;
        cumsum += probs[i];
        if (r < cumsum) {
            g_last_cdf_before = before;
            g_last_cdf_at = cumsum;
            return (uint32_t)i;
        }
    }
    g_last_cdf_before = cumsum;
    g_last_cdf_at = cumsum;
    return (uint32_t)(n - 1);
}

/* ---- anti-restate guard (sampling.rs:563-836) -------------------------- */

#define ANTI_RESTATE_MAX_SKIP 8   /* sampling.rs:553 */
#define ANTI_RESTATE_LOOP_WINDOW 28 /* sampling.rs:677 */
#define ANTI_RESTATE_LOOP_THRESH 5  /* sampling.rs:689 */
#define ANTI_RESTATE_MIN_SUFFIX 4   /* sampling.rs:708 */
#define ANTI_RESTATE_MIN_SPAN 3     /* sampling.rs:790 */
#define ANTI_RESTATE_MAX_SPAN 8     /* sampling.rs:802 */

static int rule_enabled(const char *name) {
    /* sampling.rs:625-630 */
    const char *v = getenv(name);
    if (!v) return 1;
    return !(strcmp(v, "0") == 0 || strcmp(v, "false") == 0 || strcmp(v, "no") == 0 ||
             strcmp(v, "off") == 0);
}

static int is_ws(uint8_t b) { return b == ' ' || b == '\t' || b == '\n' || b == '\r' || b == 0x0c; }

static int restates_subword(uint32_t cand, const uint32_t *h, size_t hl, const ref_decoder *dec) {
    /* sampling.rs:732-780 */
    if (!dec || dec->vocab == 0) return 0;
    if (hl == 0) return 0;
    uint32_t last = h[hl - 1];
    if (cand >= dec->vocab || last >= dec->vocab) return 0;
    const uint8_t *c = dec->bytes + dec->offsets[cand];
    size_t cl = (size_t)(dec->offsets[cand + 1] - dec->offsets[cand]);
    if (cl == 0) return 0;
    for (size_t i = 0; i < cl; i++)
        if (is_ws(c[i])) return 0;
    const uint8_t *prev = dec->bytes + dec->offsets[last];
    size_t pl = (size_t)(dec->offsets[last + 1] - dec->offsets[last]);
    if (pl == 0) return 0;
    size_t tail = 0;
    for (size_t i = pl; i > 0; i--)
        if (is_ws(prev[i - 1])) { tail = i; break; }
    const uint8_t *word = prev + tail;
    size_t wl = pl - tail;
    if (wl < ANTI_RESTATE_MIN_SUFFIX) return 0;
    for (size_t s = wl; s >= ANTI_RESTATE_MIN_SUFFIX; s--) {
        if (cl >= s && memcmp(c, word + wl - s, s) == 0) return 1;
    }
    return 0;
}

static int restates_ngram(uint32_t cand, const uint32_t *h, size_t hl) {
    /* sampling.rs:819-836 */
    for (size_t k = ANTI_RESTATE_MIN_SPAN; k <= ANTI_RESTATE_MAX_SPAN; k++) {
        if (hl + 1 < 2 * k) continue;
        size_t w = hl - (k - 1), ps = hl - (2 * k - 1);
        int eq = 1;
        for (size_t i = 0; i < k - 1; i++)
            if (h[w + i] != h[ps + i]) { eq = 0; break; }
        if (eq && cand == h[ps + k - 1]) return 1;
    }
    return 0;
}

static int runaway_loop(uint32_t cand, const uint32_t *h, size_t hl) {
    /* sampling.rs:693-701 */
    if (hl < ANTI_RESTATE_LOOP_THRESH) return 0;
    size_t start = hl > ANTI_RESTATE_LOOP_WINDOW ? hl - ANTI_RESTATE_LOOP_WINDOW : 0;
    size_t cnt = 0;
    for (size_t i = start; i < hl; i++) cnt += h[i] == cand;
    return cnt >= ANTI_RESTATE_LOOP_THRESH;
}

static int is_degenerate(uint32_t cand, const uint32_t *h, size_t hl, const ref_decoder *dec) {
    /* sampling.rs:656-662; the env gates are re-read per call here (the
     * reference caches them once per process). */
    return (rule_enabled("LUMEN_ANTI_RESTATE_SUBWORD") && restates_subword(cand, h, hl, dec)) ||
           (rule_enabled("LUMEN_ANTI_RESTATE_NGRAM") && restates_ngram(cand, h, hl)) ||
           (rule_enabled("LUMEN_ANTI_RESTATE_LOOP") && runaway_loop(cand, h, hl));
}

static long argmax_excluding(const float *v, size_t n, const size_t *ex, size_t nex) {
    /* sampling.rs:592-604 */
    long best = -1;
    uint32_t bk = 0;
    for (size_t i = 0; i < n; i++) {
        if (!isfinite(v[i])) continue;
        int skip = 0;
        for (size_t j = 0; j < nex; j++)
            if (ex[j] == i) { skip = 1; break; }
        if (skip) continue;
        uint32_t k = tkey(v[i]);
        if (best < 0 || k > bk) { best = (long)i; bk = k; }
    }
    return best;
}

uint32_t ref_guarded_argmax(const float *logits, size_t n, const uint32_t *history,
                            size_t hist_len, const ref_decoder *dec) {
    /* sampling.rs:563-585 */
    size_t raw = ref_argmax(logits, n);
    if (hist_len == 0) return (uint32_t)raw;
    size_t excluded[ANTI_RESTATE_MAX_SKIP];
    size_t nex = 0;
    size_t cand = raw;
    for (int it = 0; it < ANTI_RESTATE_MAX_SKIP; it++) {
        if (!is_degenerate((uint32_t)cand, history, hist_len, dec)) return (uint32_t)cand;
        excluded[nex++] = cand;
        long nx = argmax_excluding(logits, n, excluded, nex);
        if (nx < 0) break;
        cand = (size_t)nx;
    }
    return (uint32_t)raw;
}

/* ---- sample_logits (sampling.rs:452-527) ------------------------------- */

static uint32_t sample_core(float *logits, size_t n, const ref_params *p,
                            const uint32_t *history, size_t hist_len,
                            const ref_decoder *dec, uint64_t *rng, float r_given,
                            ref_trace *tr) {
    if (tr) memset(tr, 0, sizeof(*tr));
    if (n == 0) return 0;
    if (p->temperature <= 0.0f) {
        /* sampling.rs:468-476 */
        if (tr) tr->greedy = 1;
        if (ref_penalties_active(p)) ref_apply_penalties(logits, n, p, history, hist_len);
        uint32_t t = p->anti_restate ? ref_guarded_argmax(logits, n, history, hist_len, dec)
                                     : (uint32_t)ref_argmax(logits, n);
        if (tr) tr->token = t;
        return t;
    }
    ref_apply_penalties(logits, n, p, history, hist_len);  /* sampling.rs:489 */
    if (p->top_k > 0 && p->top_k < n) {                   /* sampling.rs:492-496 */
        ref_apply_top_k(logits, n, (size_t)p->top_k);
        if (tr) {
            tr->topk_applied = 1;
            tr->topk_survivors = g_topk_count;
            tr->topk_cutoff_key = g_topk_cutoff;
        }
    }
    if (p->top_p > 0.0f && p->top_p < 1.0f) {            /* sampling.rs:502-506 */
        ref_apply_top_p_on_logits(logits, n, p->top_p);
        if (tr) {
            tr->topp_applied = 1;
            tr->topp_sum = g_last_topp_sum;
            tr->topp_kept = g_last_topp_kept;
            tr->topp_cum_at_cross = g_last_topp_cum;
            tr->topp_cum_before = g_last_topp_cum_before;
        }
    }
    if (p->min_p > 0.0f) {                                /* sampling.rs:510-514 */
        ref_apply_min_p_on_logits(logits, n, p->min_p);
        if (tr) tr->minp_applied = 1;
    }
    float inv_temp = 1.0f / p->temperature;               /* sampling.rs:517-520 */
    for (size_t i = 0; i < n; i++) logits[i] *= inv_temp;
    if (tr) {
        float mx = -INFINITY;
        for (size_t i = 0; i < n; i++) mx = rust_fmax(mx, logits[i]);
        tr->final_max = mx;
        tr->final_uniform = !isfinite(mx);
        float s = 0.0f;
        if (isfinite(mx))
            for (size_t i = 0; i < n; i++) s += expf(logits[i] - mx);
        tr->final_sum = s;
    }
    ref_softmax_inplace(logits, n);                       /* sampling.rs:523 */
    float r = rng ? ref_xorshift64_next_f32(rng) : r_given;
    uint32_t t = ref_sample_categorical(logits, n, r);    /* sampling.rs:526 */
    if (tr) {
        tr->draw_r = r;
        tr->cdf_before = g_last_cdf_before;
        tr->cdf_at = g_last_cdf_at;
        tr->token = t;
    }
    return t;
}

uint32_t ref_sample_logits(float *logits, size_t n, const ref_params *p,
                           const uint32_t *history, size_t hist_len,
                           const ref_decoder *dec, uint64_t *rng_state) {
    return sample_core(logits, n, p, history, hist_len, dec, rng_state, 0.0f, NULL);
}

uint32_t ref_sample_logits_r(float *logits, size_t n, const ref_params *p,
                             const uint32_t *history, size_t hist_len,
                             float r, ref_trace *trace) {
    return sample_core(logits, n, p, history, hist_len, NULL, NULL, r, trace);
}

void ref_bf16_to_f32(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = u2f((uint32_t)src[i] << 16);
}

/* ---- batch driver (rows are independent; statically partitioned) ------ */

typedef struct {
    const float *logits;
    size_t B, V, b0, b1;
    const ref_params *params;
    const uint64_t *hist_off;
    const uint32_t *hist;
    const float *uniforms;
    uint32_t *out;
} batch_job;

static void *batch_worker(void *arg) {
    batch_job *j = (batch_job *)arg;
    float *row = (float *)malloc(j->V * sizeof(float));
    for (size_t b = j->b0; b < j->b1; b++) {
        memcpy(row, j->logits + b * j->V, j->V * sizeof(float));
        const uint32_t *h = j->hist + j->hist_off[b];
        size_t hl = (size_t)(j->hist_off[b + 1] - j->hist_off[b]);
        j->out[b] = sample_core(row, j->V, &j->params[b], h, hl, NULL, NULL, j->uniforms[b], NULL);
    }
    free(row);
    return NULL;
}

void ref_sample_batch(const float *logits, size_t B, size_t V, const ref_params *params,
                      const uint64_t *hist_off, const uint32_t *hist, const float *uniforms,
                      uint32_t *tokens_out, int threads) {
    if (threads < 1) threads = 1;
    if ((size_t)threads > B) threads = (int)(B ? B : 1);
    pthread_t tid[256];
    batch_job jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (batch_job){logits, B, V, B * (size_t)t / threads, B * (size_t)(t + 1) / threads,
                              params, hist_off, hist, uniforms, tokens_out};
    }
    if (threads == 1) { batch_worker(&jobs[0]); return; }
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, batch_worker, &jobs[t]);
    for (int t = 0; t < threads; t++) pthread_join(tid[t], NULL);
}
