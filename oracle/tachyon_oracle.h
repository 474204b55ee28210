/*
 * tachyon_oracle.h - CPU restatement of Tachyon's sampler (src/sampler.rs),
 * used ONLY as test infrastructure: the parity checker of tests/, smoke() and
 * bench.py's cpu_baseline leg.  Nothing in the product links it.
 *
 * Built with gcc -O2 -ffp-contract=off (no fast-math) and calling glibc
 * expf/exp/log, which is what Rust's f32::exp, f64::exp and f64::ln call on
 * linux-gnu, so it reproduces the Rust sampler's arithmetic bit for bit.
 */
#ifndef TACHYON_ORACLE_H
#define TACHYON_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/tachyon_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* SamplerConfig (src/sampler.rs:6-17) plus the extension fields. */
typedef struct or_config {
    float    temperature;
    uint32_t top_k;
    float    top_p;
    float    repetition_penalty;
    uint64_t seed;
    float    presence_penalty;
    float    frequency_penalty;
    float    min_p;
} or_config;

typedef struct or_sampler or_sampler;

/* Which branch of the reference produced the ranked list. */
enum {
    OR_PATH_ARGMAX_FAST = 0, /* sample()'s greedy shortcut, sampler.rs:79-82  */
    OR_PATH_TOP_N = 1,       /* window <= 1024, sampler.rs:193-194            */
    OR_PATH_CUTOFF = 2,      /* window > 1024, sampler.rs:195-208             */
    OR_PATH_FALLBACK = 3,    /* nothing allowed in window, sampler.rs:211-221 */
    OR_PATH_NONE_ALLOWED = 4 /* keep == 0 -> argmax, sampler.rs:139-141       */
};

/* Per-row diagnostics for parity checks (not part of the reference). */
typedef struct or_row_diag {
    uint32_t path;       /* OR_PATH_*                                        */
    uint32_t ranked;     /* |ranked| after truncation to want (A6)           */
    uint32_t survivors;  /* after min-p (== ranked when min-p is off)        */
    uint32_t keep;       /* kept by top-p (sequential f32, the reference)    */
    uint32_t pick;       /* index of the pick in ranked order                */
    uint32_t consumed_u; /* 1 if the row used its uniform                    */
    float    mass;       /* the reference's f32 mass                          */
    float    best;       /* ranked[0] penalized logit (l0)                   */
} or_row_diag;

/* ---- building blocks, each a restatement of one reference function ---- */

/* xorshift64*: state of Sampler::new (sampler.rs:64) and next_f32 (:255-261). */
uint64_t or_rng_seed(uint64_t seed);
float    or_rng_next(uint64_t* state);

/* top_n (sampler.rs:267-285): writes min(n, len) pairs, best first. */
size_t or_top_n(const float* x, size_t len, size_t n, float* vals, uint32_t* ids);

/* argmax (sampler.rs:314-322): first maximum. */
uint32_t or_argmax(const float* x, size_t len);

/* logprobs (sampler.rs:297-312).  top_ids/top_lp get min(n, len) entries. */
float or_logprobs(const float* x, size_t len, uint32_t token, size_t n,
                  uint32_t* top_ids, float* top_lp, float* lse_out);

/* Penalties (sampler.rs:165-175 + extension B.1) applied in place to buf. */
void or_penalize(float* buf, size_t n, const uint32_t* recent, size_t nrecent,
                 float repetition, float presence, float frequency);

/* glibc expf over an array (for checking the device restatement). */
void or_expf_array(const float* x, float* y, size_t n);

/* ---- Sampler object API (sampler.rs:53-262) ---- */
or_sampler* or_sampler_new(const or_config* cfg);
void        or_sampler_free(or_sampler* s);
/* sample(): `vocab` caps the ids (sampler.rs:77-84). */
uint32_t or_sample(or_sampler* s, const float* logits, size_t len, size_t vocab,
                   const uint32_t* recent, size_t nrecent);
/* sample_with(): `mask` is the packed allow-mask of the row (B.4). */
uint32_t or_sample_with(or_sampler* s, const float* logits, size_t len,
                        size_t vocab, const uint32_t* recent, size_t nrecent,
                        const uint32_t* mask);
/* distribution(): returns the kept count; writes min(keep, cap) pairs. */
size_t or_distribution(or_sampler* s, const float* logits, size_t len,
                       size_t vocab, const uint32_t* recent, size_t nrecent,
                       uint32_t* ids, float* probs, size_t cap);
/* draw() (sampler.rs:120-130) and uniform() (:250-252). */
uint32_t or_draw(or_sampler* s, const uint32_t* ids, const float* w, size_t n);
float    or_uniform(or_sampler* s);
uint64_t or_sampler_state(const or_sampler* s);

/* speculative::verify (src/speculative.rs:167-189) on (id, p) lists.
 * Returns 1 for Accept; 0 for Resample with the residual written to
 * (res_ids, res_p, *res_n) (capacity np). */
int or_verify(const uint32_t* p_ids, const float* p_p, size_t np,
              const uint32_t* q_ids, const float* q_p, size_t nq,
              uint32_t x, float u, uint32_t* res_ids, float* res_p,
              size_t* res_n);

/*
 * The batched call of tsm_sample() on HOST arrays, row by row with the
 * reference's arithmetic, using the caller's uniform per row (B.3).
 * `nthreads` >= 1 spreads rows over that many threads (one row per task).
 * Any output pointer may be NULL.  Returns 0.
 */
int or_sample_batch(const float* logits, uint32_t rows, uint32_t row_stride,
                    uint32_t usable, const tsm_row_params* params,
                    const uint32_t* hist_ids, const uint32_t* hist_offsets,
                    const uint32_t* mask, uint32_t mask_stride,
                    const float* uniforms, uint32_t* token, float* logprob,
                    uint32_t* top_ids, float* top_lp, uint32_t top_stride,
                    float* prob, uint32_t* keep, or_row_diag* diag,
                    int nthreads);

/*
 * Parity diagnostics for one row (not a reference function): the distance
 * *du that the row's uniform u, and *dp that its top_p, must move for the
 * reference's arithmetic to pick `token` with kept count `keep` (0 when the
 * pair is already the reference's).  `mask` is the row's packed mask or NULL.
 * Returns 1 when no move of u and top_p gives the pair (the token is not
 * among the first `keep` ranked ids, or `keep` is not a possible count).
 */
int or_reconcile(const float* logits, uint32_t usable, const tsm_row_params* p,
                 const uint32_t* recent, size_t nrecent, const uint32_t* mask,
                 float u, uint32_t token, uint32_t keep, double* du, double* dp);

/* tsm_distribution() on host arrays.  Returns 0. */
int or_distribution_batch(const float* logits, uint32_t rows,
                          uint32_t row_stride, uint32_t usable,
                          const tsm_row_params* params,
                          const uint32_t* hist_ids,
                          const uint32_t* hist_offsets, uint32_t* dist_ids,
                          float* dist_probs, uint32_t dist_stride,
                          uint32_t* keep, int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* TACHYON_ORACLE_H */
