/*
 * lumen_sampler -- MI355X (gfx950) token-sampling engine, C ABI.
 *
 * Drop-in for the sampler of Lumen's lumen-runtime
 * (crates/lumen-runtime/src/sampling.rs). Same parameter surface, same
 * pipeline order, same results:
 *   penalties -> top-k -> top-p (T = 1) -> min-p -> temperature -> softmax
 *   -> inverse-CDF draw; temperature <= 0 is (penalized) greedy argmax.
 *
 * Conventions
 *   - Every call returns 0 (LUMEN_OK) or a negative lumen_status; nothing
 *     aborts the process.
 *   - Logits are read from device memory and never modified (stricter than
 *     the reference, which mutates its slice: sampling.rs:426-428).
 *   - Host arrays (params, histories, uniforms) are staged by the library;
 *     the caller may reuse them as soon as the call returns.
 *   - One lumen_sampler per stream/thread. Calls on one context are
 *     serialized on the stream they are issued on.
 *   - A token value of LUMEN_TOKEN_ERROR (0xFFFFFFFF) in the output marks a
 *     row the engine could not resolve (its trace status says why).
 */
#ifndef LUMEN_SAMPLER_H
#define LUMEN_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lumen_sampler lumen_sampler;
typedef struct ihipStream_t *lumen_stream;  /* hipStream_t */

typedef enum {
    LUMEN_OK = 0,
    LUMEN_ERR_INVALID = -1,      /* bad argument (null pointer, shape, dtype) */
    LUMEN_ERR_HIP = -2,          /* a HIP runtime call failed */
    LUMEN_ERR_CODE_OBJECT = -3,  /* the gfx950 code object is missing/corrupt */
    LUMEN_ERR_NO_DEVICE = -4,
    LUMEN_ERR_UNSUPPORTED = -5,  /* a row needs a feature this build lacks */
    LUMEN_ERR_ROW = -6,          /* at least one row reported a failure */
} lumen_status;

#define LUMEN_TOKEN_ERROR 0xFFFFFFFFu

typedef enum { LUMEN_DTYPE_F32 = 0, LUMEN_DTYPE_BF16 = 1 } lumen_dtype;

/*
 * Sampling parameters, one per row. Mirrors SamplingParams
 * (sampling.rs:239-325). Each `Option<_>` field is encoded by the value the
 * reference treats exactly like `None`:
 *   top_k 0, top_p 1.0, min_p 0.0, repetition_penalty 1.0,
 *   presence_penalty 0.0, frequency_penalty 0.0, repeat_last_n 0.
 * `seed` is not part of a per-call row: callers hold the RNG
 * (lumen_xorshift64_*) or pass uniforms directly.
 */
typedef struct {
    float temperature;          /* <= 0: greedy */
    float top_p;
    float min_p;
    float repetition_penalty;
    float presence_penalty;
    float frequency_penalty;
    uint64_t top_k;
    uint64_t repeat_last_n;
    int32_t anti_restate;       /* greedy anti-degeneration guard (sampling.rs:
                                   472-474, 563-836); see lumen_batch.guard_out */
    int32_t reserved;
} lumen_sampling_params;

/* Token bytes for the anti-restate guard's sub-word rule -- the embedder's
 * per-id byte decoder (SamplerState::decoder, sampling.rs:343-378) as a
 * table: the bytes of id i are data[offsets[i] .. offsets[i + 1]); ids at or
 * above `count` decode to no bytes. */
typedef struct {
    const uint8_t *data;
    const uint64_t *offsets;            /* [count + 1] */
    uint64_t count;
} lumen_token_bytes;

/* Per-row diagnostics (optional). */
typedef struct {
    uint32_t status;           /* 0 ok; 1 tie overflow; 2 internal list overflow;
                                  3 device history window longer than the ring */
    uint32_t path;             /* bit0 greedy, bit1 LDS path, bit2 streaming path,
                                  bit3 uniform top-p, bit4 uniform final, bit5 NaN */
    uint32_t topk_cutoff_key;  /* f32::total_cmp key of the k-th largest logit */
    uint32_t topk_survivors;
    float topp_sum;            /* softmax sum inside top-p */
    uint32_t topp_kept;        /* `kept` of sampling.rs:956-963 (V if never broke) */
    float topp_cum;
    uint32_t windows;
    float final_max;
    float final_sum;
    float cdf_before;
    float cdf_at;
    uint32_t token;
    uint32_t passes;           /* streaming passes over the row */
    uint32_t pad[2];
} lumen_row_trace;

/*
 * One batch. Row b of the logits starts at logits + b * row_stride
 * elements. Histories are the SamplerState::history of each row
 * (sampling.rs:352-393), flattened: row b uses
 * history[history_offsets[b] .. history_offsets[b+1]). The library applies
 * the repeat_last_n window and counts occurrences exactly as
 * apply_penalties (sampling.rs:850-879). history_offsets may be NULL (no
 * history for any row).
 *
 * The draw of row b is uniforms[b] in [0, 1). When rng_states is non-NULL
 * the library instead draws Xorshift64::next_f32 from rng_states[b]
 * (advancing it in place) for every row with temperature > 0, matching
 * `sample_logits(.., rng)` (sampling.rs:1004). Greedy rows consume no draw.
 * uniforms_dev keeps the draws in device memory (no staging copy).
 *
 * Staging: per-row parameters and host-built penalty counts are copied to
 * the device only when they differ from the previous call on the context;
 * up to 8 rows travel inside the kernel arguments.
 */
typedef struct {
    const void *logits;                 /* device */
    int32_t dtype;                      /* lumen_dtype */
    uint32_t batch;
    uint32_t vocab;
    uint64_t row_stride;                /* elements between row starts */
    const lumen_sampling_params *params;/* host, [batch] */
    /* Penalty window, form A (host): raw SamplerState::history per row; the
     * library applies repeat_last_n and counts occurrences. */
    const uint64_t *history_offsets;    /* host, [batch + 1] or NULL */
    const uint32_t *history;            /* host */
    /* Penalty window, form B (device, pre-counted): the distinct token ids of
     * each row's window and their counts -- the SamplerState::freq map
     * (sampling.rs:356) kept resident by the caller. Row b uses entries
     * [pen_offsets[b], pen_offsets[b+1]). Used instead of form A when
     * pen_offsets is non-NULL; the caller has already applied the window. */
    const uint32_t *pen_offsets;        /* device, [batch + 1] or NULL */
    const uint32_t *pen_ids;            /* device */
    const uint32_t *pen_counts;         /* device */
    const float *uniforms;              /* host, [batch]; may be NULL if rng_states */
    uint64_t *rng_states;               /* host, [batch] in/out; may be NULL */
    const float *uniforms_dev;          /* device, [batch]; when non-NULL it is used
                                           instead of uniforms / rng_states */
    uint32_t *tokens;                   /* device, [batch] output */
    lumen_row_trace *trace;             /* device, [batch] or NULL */
    float *penalized_out;               /* device, [batch][vocab] or NULL (debug) */
    /* Device-resident RNG (the decode-loop form of `rng`, sampling.rs:1004):
     * the Xorshift64 state of each row in device memory. When non-NULL (and
     * uniforms_dev is NULL) the kernel draws next_f32 from rng_states_dev[b]
     * for every row with temperature > 0 and vocab > 0, and stores the
     * advanced state back; greedy rows leave their state untouched. No host
     * draw and no staging copy per call. */
    uint64_t *rng_states_dev;           /* device, [batch] in/out; may be NULL */
    /* Penalty window, form C (device-resident history, the decode-loop form
     * of SamplerState, sampling.rs:353-389): hist_ring_dev holds the last
     * hist_cap tokens of each row ([batch][hist_cap], the k-th recorded token
     * of row b at k % hist_cap) and hist_len_dev[b] counts the tokens
     * recorded. The library counts each row's window on the device
     * (repeat_last_n, or the whole history when it is 0) and, after
     * sampling, records the row's token (SamplerState::record) -- every row
     * with vocab > 0 and a token other than LUMEN_TOKEN_ERROR. A window
     * longer than hist_cap cannot be counted: that row's token is
     * LUMEN_TOKEN_ERROR with trace status 3. 1 <= hist_cap <= 8192. Excludes
     * forms A and B. */
    uint32_t *hist_ring_dev;            /* device, [batch][hist_cap] in/out; may be NULL */
    uint32_t *hist_len_dev;             /* device, [batch] in/out */
    uint32_t hist_cap;
    /* Form C: a number the caller changes whenever it writes the ring or
     * hist_len_dev itself (a new sequence, a new prompt). While it stays the
     * same and each call finds exactly the one token the library recorded
     * since the last call, the window counts are updated by that token
     * instead of counted again. */
    uint32_t hist_epoch;
    /* Greedy rows with anti_restate (sampling.rs:472-474). The device picks
     * the guard's candidates: guard_out[b][0] = the raw argmax,
     * guard_out[b][1..8] = the ids of the 8 largest finite penalized logits
     * in (value desc, id asc) order (LUMEN_TOKEN_ERROR where fewer exist) --
     * everything guarded_argmax (sampling.rs:563-603) can probe.
     *   - sample_batch_sync applies the guard's rules itself
     *     (lumen_anti_restate_select) with form-A histories and `decoder`,
     *     and returns the guarded token on the host and in `tokens`;
     *     guard_out may be NULL. Forms B and C are rejected for such rows
     *     (LUMEN_ERR_UNSUPPORTED): the rules need the token sequence.
     *   - sample_batch leaves the raw argmax in `tokens`; guard_out is then
     *     required and the caller applies lumen_anti_restate_select. */
    uint32_t *guard_out;                /* device, [batch][9] or NULL */
    const lumen_token_bytes *decoder;   /* host, or NULL (sub-word rule off) */
} lumen_batch;

/* Fresh-run initialisation of the device decode state: what
 * decode_token_sampled does once per generation from GpuSamplerRunCfg
 * (compute/mod.rs:202-227; engine.rs:340-371), the device form of
 * `Xorshift64::new(seed)` plus the prompt recorded into SamplerState
 * (sampling.rs:395-403, 381-384). */
typedef struct lumen_decode_seed {
    uint32_t batch;
    /* The logits' vocabulary of the run's sample calls: whole-history
     * windows keep counts for up to `vocab` distinct ids. */
    uint32_t vocab;
    /* [batch] the run's parameters, or NULL. When given, the penalty window
     * of each penalized row is counted here from the prompt, so the first
     * sample call finds its counts made (a prompt longer than hist_cap
     * then works for a whole-history window, repeat_last_n 0). The sample
     * calls must pass the same parameters, vocab, hist_cap and hist_epoch. */
    const lumen_sampling_params *params;
    const uint64_t *rng_seed_states;    /* host [batch]: Xorshift64::new(seed).state() */
    /* host: row b's prompt is prompt_ids[prompt_offsets[b] .. prompt_offsets[b+1]]
     * (GpuSamplerRunCfg.prompt_history); prompt_offsets NULL: empty prompts */
    const uint64_t *prompt_offsets;
    const uint32_t *prompt_ids;
    uint64_t *rng_states_dev;           /* device [batch] out (lumen_batch.rng_states_dev), or NULL */
    uint32_t *hist_ring_dev;            /* device [batch][hist_cap] out: the last hist_cap prompt ids */
    uint32_t *hist_len_dev;             /* device [batch] out: prompt lengths */
    uint32_t hist_cap;
    uint32_t hist_epoch;
} lumen_decode_seed;

/* Writes the device decode state of lumen_decode_seed on `stream`
 * (asynchronous; host inputs are staged before return). Not capturable:
 * run it before capturing the decode step. */
int lumen_sampler_decode_seed(lumen_sampler *s, const lumen_decode_seed *seed, lumen_stream stream);

/* Context: loads the gfx950 code object on `device`. The code object is
 * embedded in the library; LUMEN_SAMPLER_CODE_OBJECT=<path> overrides it. */
int lumen_sampler_create(lumen_sampler **out, int device);
void lumen_sampler_destroy(lumen_sampler *s);

/* Batched sampler. Asynchronous on `stream` (host inputs are staged before
 * return). Replaces sample_logits (sampling.rs:452-527) applied to every
 * row, and the GPU hook ComputeBackend::decode_token_sampled
 * (compute/mod.rs:424-438). */
int lumen_sampler_sample_batch(lumen_sampler *s, const lumen_batch *batch, lumen_stream stream);

/* The same as lumen_sampler_sample_batch, allocating nothing: no device or
 * pinned memory is allocated, by the library or by a library it calls. No
 * counterpart in the reference; it is for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Its device buffers are carved from one 32 MiB array per GPU in
 * the library itself, so a call takes at most 8 rows of at most 262144
 * logits, no device history (hist_ring_dev), at most 65536 form-A penalty
 * entries, and anti_restate rows need guard_out; anything beyond returns
 * LUMEN_ERR_INVALID with lumen_sampler_last_error() naming the limit. The
 * array of a GPU belongs to the first context that makes a no-allocation
 * call there, until that context is destroyed; calls from other contexts
 * return LUMEN_ERR_INVALID. Calls of the owning context share the array, so
 * they must not overlap: issue them on one stream (the convention for every
 * context). Under stream capture, form-A histories are refused (their counts
 * would be copied from host memory at every replay): pass pen_offsets. */
int lumen_sampler_sample_batch_noalloc(lumen_sampler *s, const lumen_batch *batch,
                                       lumen_stream stream);

/* Synchronous convenience: same as above, then waits and copies the tokens
 * to host memory. Returns LUMEN_ERR_ROW if a row reported a failure.
 * Mirrors Sampler::sample / sample_token_with_state (sampling.rs:429-433,
 * engine.rs:80-88) for a batch. */
int lumen_sampler_sample_batch_sync(lumen_sampler *s, const lumen_batch *batch,
                                    uint32_t *tokens_host, lumen_stream stream);

/* Bound of every cross-workgroup wait inside a launch, in microseconds of
 * the device wall clock (default 2000). A row's workgroups wait for each
 * other at a few points; they are co-resident when the call has the GPU to
 * itself, but kernels of other streams can hold CUs. A wait that reaches the
 * bound gives up, is counted (lumen_sampler_wait_timeouts) and its row is
 * resolved by the exact single-workgroup path: the token is the same, the
 * call slower. 0 makes every such wait give up at once. Applies to the
 * following calls on the context. No counterpart in the reference, whose
 * CPU sampler has no cross-workgroup waits; it plays the part of its GPU
 * path's visible fallback (cuda/backend_impl.rs:1276-1293). */
int lumen_sampler_set_wait_limit(lumen_sampler *s, uint32_t microseconds);

/* Number of cross-workgroup waits that gave up since the context was
 * created (see lumen_sampler_set_wait_limit). Reads device memory: call it
 * once the calls to count have completed. */
int lumen_sampler_wait_timeouts(lumen_sampler *s, uint64_t *count);

/* Range checks of the server's wire layer
 * (crates/lumen-server/src/wire/openai.rs:357-381): temperature must be
 * finite and in [0, 2], top_p finite and in [0, 1]. Returns LUMEN_OK or LUMEN_ERR_INVALID, and
 * lumen_sampler_last_error() names the field. The sampler itself does not
 * call it: like sample_logits, it accepts any value and skips a stage whose
 * parameter is out of its active range (sampling.rs:493, 503, 511). */
int lumen_sampling_params_validate(const lumen_sampling_params *p);

/* The anti-restate guard's choice (guarded_argmax, sampling.rs:563-603)
 * from the 9 candidates of lumen_batch.guard_out, the row's history
 * (SamplerState::history, oldest first) and an optional decoder: probes the
 * raw argmax, then the finite candidates in order, vetoing each that
 * restates a sub-word (sampling.rs:732-780), closes a back-to-back repeat of
 * a 3..8-token span (:819-836) or occurs 5+ times in the last 28 tokens
 * (:693-701); at most 8 probes, else the raw argmax. The rules read
 * LUMEN_ANTI_RESTATE_{SUBWORD,NGRAM,LOOP} once (0/false/no/off disables a
 * rule, :625-662). */
uint32_t lumen_anti_restate_select(const uint32_t *candidates, const uint32_t *history,
                                   uint64_t history_len, const lumen_token_bytes *decoder);

/* Reference RNG (sampling.rs:45-106): Xorshift64 seeded through the
 * SplitMix64 finalizer. */
uint64_t lumen_xorshift64_new(uint64_t seed);
uint64_t lumen_xorshift64_next_u64(uint64_t *state);
float lumen_xorshift64_next_f32(uint64_t *state);

/* Library / code-object version string. */
const char *lumen_sampler_version(void);

/* Human-readable reason for the last failing call on this thread. The
 * reference's backend hooks return RuntimeError strings
 * (compute/mod.rs:424-438); this is their C-ABI counterpart. */
const char *lumen_sampler_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* LUMEN_SAMPLER_H */
