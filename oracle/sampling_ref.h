/*
 * CPU oracle for the token-sampling path: a C restatement of the x86_64 code
 * path of Lumen's `crates/lumen-runtime/src/sampling.rs` (reference workspace
 * version 0.11.0).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (lumen_amd/, include/) may
 * link, load or call this code. It is used by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -march=native,
 * no -ffast-math) so every f32 operation is a single IEEE-754 binary32
 * operation, as in the Rust reference compiled for x86_64.
 *
 * Parameter encoding: the Rust `Option<_>` fields are encoded by the neutral
 * value that the reference treats identically to `None`:
 *   top_k None == 0            (sampling.rs:492-496 acts only for 0 < k < len)
 *   top_p None == 1.0          (sampling.rs:502-506 acts only for 0 < p < 1)
 *   min_p None == 0.0          (sampling.rs:510-514 acts only for m > 0)
 *   repetition_penalty None == 1.0, presence/frequency None == 0.0
 *                              (sampling.rs:851-853 unwrap_or defaults)
 *   repeat_last_n None == 0    (sampling.rs:863 filter(n > 0))
 */
#ifndef LUMEN_ORACLE_SAMPLING_REF_H
#define LUMEN_ORACLE_SAMPLING_REF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float temperature;
    uint64_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    uint64_t repeat_last_n;
    int32_t anti_restate;
} ref_params;

/* Xorshift64 (sampling.rs:45-106). */
uint64_t ref_xorshift64_new(uint64_t seed);
uint64_t ref_xorshift64_next_u64(uint64_t *state);
float ref_xorshift64_next_f32(uint64_t *state);

/* Primitives (sampling.rs:207-231, 538-547, 850-1014). */
void ref_softmax_inplace(float *v, size_t n);
size_t ref_argmax(const float *v, size_t n);
int ref_penalties_active(const ref_params *p);
void ref_apply_penalties(float *logits, size_t n, const ref_params *p,
                         const uint32_t *history, size_t hist_len);
void ref_apply_top_k(float *logits, size_t n, size_t k);
void ref_apply_top_p_on_logits(float *logits, size_t n, float p);
void ref_apply_min_p_on_logits(float *logits, size_t n, float min_p);
uint32_t ref_sample_categorical(const float *probs, size_t n, float r);

/* Optional byte decoder for the anti-restate guard: token t decodes to
 * bytes[offsets[t] .. offsets[t+1]). vocab == 0 means "no decoder". */
typedef struct {
    const uint8_t *bytes;
    const uint64_t *offsets;
    size_t vocab;
} ref_decoder;

/* Full per-row sampler (sampling.rs:452-527). `logits` is overwritten, as in
 * the reference. `history` is SamplerState::history. `rng_state` advances
 * exactly once iff temperature > 0 and n > 0. */
uint32_t ref_sample_logits(float *logits, size_t n, const ref_params *p,
                           const uint32_t *history, size_t hist_len,
                           const ref_decoder *dec, uint64_t *rng_state);

/* Same algorithm with a caller-supplied uniform `r` in place of the RNG
 * draw (the GPU engine takes host-generated uniforms), plus a trace of the
 * intermediate quantities used by the parity harness. Any trace pointer may
 * be NULL. */
typedef struct {
    int32_t greedy;          /* 1 if the T <= 0 branch ran */
    int32_t topk_applied;
    uint32_t topk_survivors; /* finite-or-not count of tokens not masked by top-k */
    uint32_t topk_cutoff_key; /* total_cmp key of the k-th largest */
    int32_t topp_applied;
    float topp_sum;          /* softmax sum inside top-p (T = 1) */
    uint32_t topp_kept;      /* `kept` in sampling.rs:956-963 */
    float topp_cum_at_cross; /* cum value at which the loop stopped */
    float topp_cum_before;   /* cum value one step before */
    int32_t minp_applied;
    float final_max;
    float final_sum;         /* final softmax sum (sampling.rs:218-222) */
    int32_t final_uniform;   /* final softmax took the uniform branch */
    float draw_r;
    float cdf_before;        /* cumsum before the selected token */
    float cdf_at;            /* cumsum including the selected token */
    uint32_t token;
} ref_trace;

uint32_t ref_sample_logits_r(float *logits, size_t n, const ref_params *p,
                             const uint32_t *history, size_t hist_len,
                             float r, ref_trace *trace);

/* Greedy anti-degeneration guard (sampling.rs:563-836). */
uint32_t ref_guarded_argmax(const float *logits, size_t n,
                            const uint32_t *history, size_t hist_len,
                            const ref_decoder *dec);

/* Batched convenience: rows sampled independently, rows split statically
 * over `threads` POSIX threads (threads <= 1 runs inline). hist_off has
 * B+1 entries into `hist`. uniforms[b] is used for non-greedy rows. */
void ref_sample_batch(const float *logits, size_t B, size_t V,
                      const ref_params *params, const uint64_t *hist_off,
                      const uint32_t *hist, const float *uniforms,
                      uint32_t *tokens_out, int threads);

/* bf16 -> f32 widening (exact). */
void ref_bf16_to_f32(const uint16_t *src, float *dst, size_t n);

#ifdef __cplusplus
}
#endif
#endif
