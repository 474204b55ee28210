/*
 * tachyon_sampler.h - C ABI of the MI355X batched token-sampling path.
 *
 * One call samples the next token of every row of a [rows x row_stride] f32
 * logits matrix that already sits in device memory (HBM).  Per row it runs
 * the pipeline of Tachyon's CPU sampler (src/sampler.rs) plus the extension
 * fields this path adds:
 *
 *   repetition / presence / frequency penalties from the row's history
 *   -> window of best candidates (top_n, or the 30*T cutoff when there is no
 *      top-k) -> packed-mask filter with the reference's window/fallback rule
 *   -> truncate to top-k -> probabilities exp((l - l0) / T) -> min-p
 *   -> top-p -> inverse-CDF draw with the caller's uniform
 *   -> optional logprob of the pick and the top-n alternatives (raw logits).
 *
 * Every array argument is a DEVICE pointer.  Work is queued on the caller's
 * HIP stream and is asynchronous; results are valid once the stream reaches
 * the call.  The context is not re-entrant: one context per stream, one call
 * at a time (as with the reference's GpuBackend, src/gpu/mod.rs:440-442).
 *
 * Errors follow the reference's FFI convention (src/gpu/shim.m:130,
 * src/gpu/mod.rs:467-480): a NULL handle or a nonzero int status, and a
 * NUL-terminated message written into the caller's (err, errlen) buffer.
 * "Nothing allowed" is not an error: such a row returns the argmax of its raw
 * logits, as the reference does (src/sampler.rs:139-141).  Neither are NaN or
 * infinite logits: such rows get the reference's result (top_n's insertion
 * order, src/sampler.rs:267-285; argmax's first index, :314-322), with NaN
 * probabilities and logprobs where the reference's are NaN.
 */
#ifndef TACHYON_SAMPLER_H
#define TACHYON_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Most alternatives a row may ask logprobs for (src/server.rs:625-634 caps
 * `top_logprobs` at 20). */
#define TSM_MAX_LOGPROBS 20u
/* Longest history a row may carry (token counts are kept in 16 bits). */
#define TSM_MAX_HISTORY 65535u
/* Largest vocabulary (usable ids per row) a context accepts. */
#define TSM_MAX_VOCAB (1u << 22)

/* tsm_row_params.flags */
#define TSM_ROW_CONSTRAINED 1u /* sample_with(): the row's mask bits apply   */
#define TSM_ROW_LOGPROBS    2u /* report logprob of the pick + n_logprobs   */

/*
 * Per-row sampling settings.  The first five fields are Tachyon's
 * SamplerConfig (src/sampler.rs:6-17) minus the seed: the RNG stays with the
 * host-side Sampler, which passes one uniform per row instead.  The three
 * penalty/min-p fields are extensions; their zero values reproduce the
 * reference exactly.  Layout is fixed: 40 bytes, 4-byte aligned.
 */
typedef struct tsm_row_params {
    float    temperature;        /* <= 0: greedy (sampler.rs:8, :161)            */
    uint32_t top_k;              /* 0: no limit (sampler.rs:10, :179)            */
    float    top_p;              /* >= 1: off (sampler.rs:235)                   */
    float    repetition_penalty; /* 1: off (sampler.rs:165-175)                 */
    float    presence_penalty;   /* extension, 0: off                            */
    float    frequency_penalty;  /* extension, 0: off                            */
    float    min_p;              /* extension, <= 0: off                         */
    uint32_t flags;              /* TSM_ROW_* bits                               */
    uint32_t n_logprobs;         /* alternatives when TSM_ROW_LOGPROBS, <= 20    */
    uint32_t reserved;           /* must be 0                                    */
} tsm_row_params;

/*
 * One step's inputs.  Row r's logits are logits[r*row_stride .. +usable]
 * (src/scheduler.rs:625-626,652: usable = min(tokenizer.len(), vocab)).
 * History is CSR: row r's ids are hist_ids[hist_offsets[r] ..
 * hist_offsets[r+1]) (the `recent` slice of src/scheduler.rs:653); ids >=
 * usable are ignored, as the reference's `buf.get_mut(id)` ignores them.
 * The mask is packed LSB-first: bit b of word w of row r allows token 32w+b;
 * bits at or above `usable` must be 0.
 */
typedef struct tsm_batch {
    const float*          logits;       /* [rows][row_stride]                   */
    uint32_t              rows;
    uint32_t              row_stride;   /* elements; >= usable                  */
    uint32_t              usable;       /* ids considered per row; >= 1         */
    uint32_t              mask_stride;  /* u32 words per mask row               */
    const tsm_row_params* params;       /* [rows]                               */
    const uint32_t*       hist_ids;     /* CSR values, NULL if every row empty  */
    const uint32_t*       hist_offsets; /* [rows+1], NULL if every row empty    */
    const uint32_t*       mask;         /* [rows][mask_stride], NULL if no row
                                           sets TSM_ROW_CONSTRAINED             */
    const float*          uniforms;     /* [rows], each in [0, 1)               */
    uint32_t              row_kinds;    /* OR of tsm_row_kind() over the rows
                                           (host-side configs), or 0 when not
                                           known: then every kernel is queued */
    uint32_t              reserved;     /* must be 0                            */
} tsm_batch;

/*
 * Row kinds.  In a batch of up to 16 rows a step queues one kernel per kind
 * present: the split-row kernel (a row cut over many workgroups) for rows
 * with a top-k window (sampler.rs:192-194) and a short penalizing history,
 * the whole-row kernel for the others (no top-k: the 30*T cutoff set,
 * sampler.rs:195-208; long histories).  Larger batches take the whole-row
 * kernel for every row.  A batch that names its kinds skips the kernels it
 * does not need (about 2 us each); in a small batch, a row of a kind the
 * batch did not name is not sampled and sets TSM_STATUS_ROW_KIND.
 * tsm_row_kind() gives a row's kind from the same fields the device reads:
 * its parameters, the batch's `usable`, the row's history length and whether
 * the batch has a mask.  In a batch of up to 16 rows, a row whose kind holds
 * TSM_ROWKIND_SPLIT need add only that bit to the batch's row_kinds (its
 * other bit names the whole-row kernel that takes it in a larger batch).
 */
#define TSM_ROWKIND_SPLIT 1u /* the split-row kernel (batches of up to 16 rows)      */
#define TSM_ROWKIND_WHOLE 2u /* the general whole-row kernel                         */
#define TSM_ROWKIND_LEAN  4u /* the lean whole-row kernel: top-k rows with at most
                                64 kept ids and penalties that only lower values
                                (a split row of a larger batch takes it too)       */

/* One step's outputs.  `token` is required; every other pointer may be NULL. */
typedef struct tsm_outputs {
    uint32_t* token;        /* [rows] picked id                                  */
    float*    logprob;      /* [rows] raw log-softmax of the pick
                               (sampler::logprobs, src/sampler.rs:297-312)     */
    uint32_t* top_ids;      /* [rows][top_stride] best raw ids, ties -> lower id */
    float*    top_logprobs; /* [rows][top_stride] their log-softmax values       */
    uint32_t  top_stride;   /* >= every row's n_logprobs when top_* are given    */
    uint32_t  reserved;
    float*    prob;         /* [rows] probability of the pick under the final,
                               normalised distribution (p_tok / mass)           */
    uint32_t* keep;         /* [rows] size of the kept set the draw used         */
} tsm_outputs;

typedef struct tsm_ctx tsm_ctx;

/*
 * Creates a sampling context on HIP device `device` for calls with up to
 * `max_rows` rows of up to `max_vocab` usable ids; all device scratch is
 * allocated here, none per call.  Returns NULL and fills `err` on failure.
 * Replaces: the per-sequence scratch of Sampler::new (src/sampler.rs:63-73);
 * FFI shape follows tm_create (src/gpu/mod.rs:117-123).
 */
tsm_ctx* tsm_create(int device, uint32_t max_rows, uint32_t max_vocab,
                    char* err, size_t errlen);

/* Frees a context (NULL is a no-op).  Replaces tm_destroy (src/gpu/mod.rs:124). */
void tsm_destroy(tsm_ctx* ctx);

/*
 * Samples one token per row.  `stream` is a hipStream_t (NULL: the null
 * stream).  Returns 0, or nonzero with a message in `err` when an argument is
 * invalid (checked on the host before anything is queued).
 * Replaces: the per-row loop of src/scheduler.rs:638-675, i.e. for each row
 * Sampler::sample / Sampler::sample_with (src/sampler.rs:77-97) followed by
 * sampler::logprobs (src/sampler.rs:297-312).
 */
int tsm_sample(tsm_ctx* ctx, void* stream, const tsm_batch* batch,
               const tsm_outputs* out, char* err, size_t errlen);

/*
 * Writes each row's final distribution, best first, as normalised (id, p)
 * pairs: row r gets min(keep, dist_stride) pairs in dist_ids/dist_probs
 * [r*dist_stride ..] and its full kept count in keep[r].  No draw is made;
 * `batch->uniforms` may be NULL and TSM_ROW_CONSTRAINED is ignored, as
 * Sampler::distribution takes no constraint.
 * Replaces: Sampler::distribution (src/sampler.rs:102-116), used by
 * speculative decoding (src/speculative.rs:96-97, :306).
 */
int tsm_distribution(tsm_ctx* ctx, void* stream, const tsm_batch* batch,
                     uint32_t* dist_ids, float* dist_probs,
                     uint32_t dist_stride, uint32_t* keep,
                     char* err, size_t errlen);

/*
 * Waits for the context's last call (an event on that call's stream; other
 * streams are not waited for) and returns the device-side status:
 * 0 when every row was sampled by the specified rule, otherwise TSM_STATUS_*
 * bits (e.g. a history row longer than TSM_MAX_HISTORY, whose counts are
 * then capped, or a row whose n_logprobs exceeds top_stride, whose list is
 * then cut to top_stride).  Clears the status.  A call queued on the context
 * while tsm_status() runs races with the clearing (a context serves one
 * caller at a time).
 */
#define TSM_STATUS_HISTORY_TOO_LONG 1u
#define TSM_STATUS_BAD_PARAMS       2u
#define TSM_STATUS_DIST_TRUNCATED   4u
#define TSM_STATUS_INTERNAL         8u /* a row the device could not sample
                                          exactly; token 0 and keep 0
                                          written.  Rows holding NaN or
                                          infinite logits are sampled as the
                                          reference does.  Known case: a row
                                          without top-k whose candidates hold
                                          more than three dense clusters, each
                                          narrower than 1/2048 of the row's
                                          value span and with more distinct
                                          values near one fold event than the
                                          exact folds' census takes (2048).
                                          Fallback: sample that row with the
                                          reference's CPU Sampler */
#define TSM_STATUS_ROW_KIND        16u /* a row of a kind the batch's row_kinds
                                          left out: token 0 written           */
int tsm_status(tsm_ctx* ctx, uint32_t* status, char* err, size_t errlen);

/*
 * tsm_sample() without a context and without allocating anything: for
 * callers that cannot call hipMalloc (code under HIP graph capture, serving
 * loops and harnesses that forbid it).  It has no counterpart in the
 * reference.  Its scratch is a fixed array in the library's device memory,
 * one per GPU (about 25 MB, held until the process ends), which takes batches
 * of up to 16 rows of up to 2^18 ids on the split-row kernel; other batches
 * (up to 65535 rows of up to TSM_MAX_VOCAB ids) take the whole-row kernel,
 * which needs no scratch.  Larger batches are rejected.  Works on the current
 * HIP device.  `status` (a device word, may be NULL) is cleared and then
 * receives this call's TSM_STATUS_* bits.  Calls on one GPU share its scratch:
 * calls that overlap on one GPU (other streams, other threads) race.
 */
int tsm_sample_static(void* stream, const tsm_batch* batch, const tsm_outputs* out,
                      uint32_t* status, char* err, size_t errlen);

/* The kinds (TSM_ROWKIND_* bits) of a row: `p` is the row's parameters (host
 * memory), `usable` the batch's, `hist_len` the row's history length,
 * `has_mask` whether the batch passes a mask.  TSM_ROWKIND_SPLIT when the
 * split-row kernel takes the row in a small batch, and TSM_ROWKIND_LEAN or
 * TSM_ROWKIND_WHOLE for the whole-row kernel that takes it otherwise. */
uint32_t tsm_row_kind(const tsm_row_params* p, uint32_t usable, uint32_t hist_len, int has_mask);

/*
 * ---- The mask producer: a JSON-object constraint -> packed allow-bits -------
 *
 * Tachyon checks `c.allows(tok, id)` (src/constrain.rs:286-290) for each id the
 * sampler probes (src/scheduler.rs:653-656).  These entry points produce a
 * whole row of those answers at once on the GPU, in the mask layout
 * tsm_batch.mask consumes, for rows whose constraint is a JsonObject
 * (OutputFormat::JsonObject, src/constrain.rs:14-33: `response_format:
 * json_object`).  The automaton's state lives with the host-side sequence, as
 * the reference's Box<dyn Constraint> does; each step the host passes every
 * constrained row's state (12 bytes) and gets its mask row.
 */

/* JsonObject's state (src/constrain.rs:88-93): the automaton state, the
 * stack of open containers (bit i of `stack`: level i is an object; at most
 * 32 levels) and the whitespace run.  Built by tsm_json_init and advanced by
 * tsm_json_advance only; the fields are not an interface. */
typedef struct tsm_json_state {
    uint32_t stack;
    uint8_t  depth;
    uint8_t  state;
    uint8_t  aux;
    uint8_t  len;
    uint8_t  whitespace;
    uint8_t  pad[3];
} tsm_json_state;

/* The tokenizer's token bytes (src/tokenizer.rs:189-195), in device memory:
 * token t's bytes are bytes[offsets[t] .. offsets[t+1]).  Ids at or above
 * n_tokens have no bytes (never allowed).  `special` (may be NULL) holds one
 * bit per token, LSB-first: set = a special token, never allowed. */
typedef struct tsm_vocab {
    const uint8_t*  bytes;
    const uint32_t* offsets;   /* [n_tokens + 1] */
    const uint32_t* special;   /* [ceil(n_tokens / 32)] or NULL */
    uint32_t        n_tokens;
    uint32_t        reserved;  /* must be 0 */
} tsm_vocab;

/* JsonObject::default() (src/constrain.rs:95-103).  Host function. */
void tsm_json_init(tsm_json_state* s);
/* Constraint::advance with the chosen token's bytes (src/constrain.rs:292-296,
 * called at src/scheduler.rs:698).  Host function. */
void tsm_json_advance(tsm_json_state* s, const uint8_t* bytes, size_t n);
/* JsonObject::accepts_bytes (src/constrain.rs:280-283): 1 if every byte steps
 * a copy of the automaton.  Host function. */
int tsm_json_accepts(const tsm_json_state* s, const uint8_t* bytes, size_t n);
/* Constraint::is_complete (src/constrain.rs:298-300).  Host function. */
int tsm_json_is_complete(const tsm_json_state* s);

/*
 * Writes the allow-bits of `rows` rows: bit b of word w of row r (mask +
 * r*mask_stride) is set exactly when JsonObject::allows holds for token 32w+b
 * in state states[r] (not special, has bytes, and accepts_bytes); ids at or
 * above `usable` get 0 bits.  `states` and `mask` are device pointers;
 * mask_stride >= ceil(usable / 32).  Queued on `stream`; allocates nothing.
 * Replaces: the `&|t| c.allows(tok, t)` closure of src/scheduler.rs:653-656
 * for JsonObject constraints, evaluated for the whole vocabulary.
 */
int tsm_json_mask(void* stream, const tsm_vocab* vocab, const tsm_json_state* states, uint32_t rows,
                  uint32_t usable, uint32_t* mask, uint32_t mask_stride, char* err, size_t errlen);

/*
 * A mask set: tsm_json_mask for a serving loop, where many rows share a state
 * (every row writing string text at one depth, say) and states recur from step
 * to step.  Each call evaluates every distinct state of its rows once, keeps
 * the masks of up to `capacity` states in device memory (least recently used
 * out first), and fills each row's mask by a copy from its state's mask.  The
 * masks written are the ones tsm_json_mask writes for the same states.
 * Replaces: the same closure as tsm_json_mask (src/scheduler.rs:653-656),
 * with the per-state reuse the reference's probing has no need of.
 *
 * tsm_json_masks_create allocates the set on `device` (GPU memory:
 * capacity * ceil(ceil(usable / 32) / 64) * 256 bytes, plus about 2 * 44
 * bytes per row of staging in pinned host memory, which the kernels read over
 * the bus); `capacity` 0 keeps no
 * masks between calls (rows sharing a state within a call still share one
 * evaluation).  NULL on failure, with the reason in err.
 *
 * tsm_json_masks_fill: `states` is a HOST array of `rows` (<= max_rows)
 * states, as tsm_json_advance keeps them; `mask` (device) gets one row per
 * state, words [0, ceil(usable / 32)) of each written.  `stats` (may be NULL)
 * receives the call's counts.  Queued on `stream`: at most one evaluation
 * launch and one copy launch.  The call waits on the host only for the
 * launches of the call before the last one (the staging alternates between
 * two halves).  The slots are tied to the
 * vocabulary's device pointers and n_tokens: a call with other ones empties
 * the set first; after changing a vocabulary's bytes in place, call
 * tsm_json_masks_reset.  Calls on one set must come from one host thread at a
 * time and be queued on one stream (or ordered by the caller): a later call
 * may overwrite a slot an earlier call's copies still read.
 */
typedef struct tsm_json_masks tsm_json_masks;
typedef struct tsm_json_fill_stats {
    uint32_t rows;       /* rows filled */
    uint32_t distinct;   /* distinct states among them */
    uint32_t hits;       /* distinct states whose mask the set already held */
    uint32_t evaluated;  /* states evaluated by this call (distinct - hits) */
} tsm_json_fill_stats;

tsm_json_masks* tsm_json_masks_create(int device, uint32_t max_rows, uint32_t capacity, uint32_t usable, char* err,
                                      size_t errlen);
void tsm_json_masks_destroy(tsm_json_masks* set);
void tsm_json_masks_reset(tsm_json_masks* set);
int tsm_json_masks_fill(tsm_json_masks* set, void* stream, const tsm_vocab* vocab, const tsm_json_state* states,
                        uint32_t rows, uint32_t* mask, uint32_t mask_stride, tsm_json_fill_stats* stats, char* err,
                        size_t errlen);

/* ---- the logits producer ------------------------------------------------
 * Tachyon's output layer for the rows that get logits: xb = rmsnorm(x[r])
 * in f32 (src/model.rs:702-709 over src/kernels.rs:522-528), then
 * logits[r][v] = dot(W[v], xb) over a bf16 lm_head matrix W [vocab, dim]
 * (src/model.rs:711-715, the Bf16 arm of src/weights.rs:230-239,
 * src/kernels.rs:1411-1413), on the MFMA matrix cores.
 * Replaces: the rmsnorm + lm_head.matmul pair of src/model.rs:700-716 (CPU)
 * and src/gpu/mod.rs:1044-1047 (Metal), for a Bf16 lm_head.
 *
 * With TSM_LM_SPLIT each activation is carried as two bf16 values (hi =
 * bf16(xb), lo = bf16(xb - hi), within 2^-17 of xb) and both are multiplied
 * with W: twice the matrix work, activations about as exact as the
 * reference's f32.  Without it the activations are rounded to bf16 once
 * (relative error up to 2^-9 each).
 */
#define TSM_LM_SPLIT    1u
#define TSM_LM_MAX_ROWS 65536u
#define TSM_LM_MAX_DIM  32768u

/* Device bytes tsm_lm_head needs as workspace for `rows` rows of `dim`
 * (the bf16 operands, rows padded to the workgroup tile: 16, 32, 64, 128 or 256). */
size_t tsm_lm_head_workspace(uint32_t rows, uint32_t dim, uint32_t flags);

/*
 * Queues the logits of `rows` rows on `stream`: row r of x (f32, x + r *
 * x_stride, dim values) is normalized with norm_w (f32 [dim]) and eps, and
 * logits + r * ld receives its dot product with each of the vocab rows of w
 * (bf16 [vocab][dim], 16-byte aligned).  dim is a multiple of 64 (at most
 * TSM_LM_MAX_DIM); workspace (16-byte aligned, at least
 * tsm_lm_head_workspace bytes) is overwritten.  All pointers are device
 * pointers.  Allocates nothing; returns nonzero with a message on a bad
 * argument, before anything is queued.
 */
int tsm_lm_head(void* stream, const float* x, uint32_t x_stride, const float* norm_w, float eps,
                const uint16_t* w, uint32_t rows, uint32_t dim, uint32_t vocab, uint32_t flags, void* workspace,
                size_t workspace_bytes, float* logits, uint32_t ld, char* err, size_t errlen);

/*
 * The same output layer over a Q8 lm_head (weights.rs:64-70, llama.cpp's
 * Q8_0): wq (int8 [vocab][dim], 16-byte aligned) and wscale (f16 bits
 * [vocab][dim / 32]: one scale per block of 32 weights, 2-byte aligned;
 * read fastest when dim is a multiple of 256 and wscale 16-byte aligned).
 * The logits are bit-identical to the reference's scalar path.  Each row of x is
 * normalized (the sum of squares as the reference's left fold) and quantized
 * per 32-value block (quantize_input, weights.rs:652-664, over
 * kernels.rs:84-100); logits + r * ld receives, per vocab row, the blocks'
 * exact integer dots, each times the weight block's scale and the row
 * block's scale, summed in f32 in block order (the scalar dot_q8_with,
 * kernels.rs:1420-1430).  dim is a multiple of 32 (at most TSM_LM_MAX_DIM);
 * workspace (16-byte aligned, at least tsm_lm_head_q8_workspace bytes) is
 * overwritten.  Replaces: lm_head.matmul for a Q8 matrix (model.rs:711-715,
 * the Q8 arm of weights.rs:213-260).  Allocates nothing; two kernel launches.
 */
size_t tsm_lm_head_q8_workspace(uint32_t rows, uint32_t dim);
int tsm_lm_head_q8(void* stream, const float* x, uint32_t x_stride, const float* norm_w, float eps, const int8_t* wq,
                   const uint16_t* wscale, uint32_t rows, uint32_t dim, uint32_t vocab, void* workspace,
                   size_t workspace_bytes, float* logits, uint32_t ld, char* err, size_t errlen);

/* Library version string, e.g. "tachyon-sampler 0.1 gfx950". */
const char* tsm_version(void);

#ifdef __cplusplus
}
#endif

#endif /* TACHYON_SAMPLER_H */
