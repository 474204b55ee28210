// tachyon_oracle.cpp - CPU restatement of Tachyon's sampler, TEST
// INFRASTRUCTURE ONLY.
//
// This file is the parity checker: tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py load it through ctypes.  The product library
// (tachyon_amd/csrc) never links, loads or calls it.
//
// It restates /root/reference/src/sampler.rs function by function (each
// function cites the lines it follows) plus the extension rules this path
// adds (presence/frequency penalties, min-p, packed mask, caller-supplied
// uniform).  Build: g++ -O2 -ffp-contract=off, no fast-math, so float and
// double operations round exactly as Rust's do, and expf/exp/log are glibc's,
// which is what Rust's f32::exp / f64::exp / f64::ln call on linux-gnu.
//
// Pinning (what checks this file, see tests/test_oracle.py):
//   * the reference's own known-answer tests (sampler.rs:328-395,
//     speculative.rs:349-375), ported;
//   * closed forms: xorshift64* golden sequence, log-softmax, penalties;
//   * brute force against oracle/naive.py (a full-sort restatement written
//     independently in numpy) on small and tie-heavy inputs.

#include "tachyon_oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint32_t f2u(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

// f32::total_cmp as an unsigned key: a larger key is later in the total
// order (-NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN).
inline uint32_t total_key(float f) {
    uint32_t u = f2u(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Composite key sorting ascending as "value descending by total_cmp, then
// id ascending".  sort_unstable_by (sampler.rs:207, :220) leaves the order of
// equal values unspecified; this build defines it as lower id first.
inline uint64_t desc_key(float v, uint32_t id) {
    return (static_cast<uint64_t>(~total_key(v)) << 32) | id;
}

struct Scratch {
    std::vector<float> buf;
    std::vector<float> rv;     // ranked values
    std::vector<uint32_t> ri;  // ranked ids
    std::vector<float> probs;
    std::vector<uint64_t> keys;
    std::vector<uint32_t> seen;
};

}  // namespace

struct or_sampler {
    or_config cfg;
    uint64_t rng;
    Scratch s;
};

extern "C" {

// Sampler::new (sampler.rs:63-64).
uint64_t or_rng_seed(uint64_t seed) { return (seed * 0x2545F4914F6CDD1DULL) | 1ULL; }

// Sampler::next_f32 (sampler.rs:255-261).
float or_rng_next(uint64_t* state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    uint64_t m = x * 0x2545F4914F6CDD1DULL;
    return static_cast<float>(m >> 40) / static_cast<float>(1ULL << 24);
}

// top_n (sampler.rs:267-285): one pass, a value is inserted only when the list
// is not full or it beats the current n-th best; equal values go after the
// ones already kept (partition_point(w >= v)), so ties keep the lower id.
size_t or_top_n(const float* x, size_t len, size_t n, float* vals, uint32_t* ids) {
    size_t k = 0;
    if (n == 0) return 0;
    float floor = -INFINITY;
    for (size_t i = 0; i < len; i++) {
        float v = x[i];
        if (k < n || v > floor) {
            // partition_point(|&(w, _)| w >= v), probing as the reference's
            // toolchain does (Rust 1.87.0, pinned by .github/workflows/ci.yml:16-17,
            // :64-65): partition_point is binary_search_by with `w >= v` as
            // Less, whose loop runs while size > 1 { half = size / 2; mid =
            // base + half; pred(mid) moves base to mid; size -= half } and
            // returns base + pred(base).  With a NaN in the list the
            // predicate is not monotone and only this probe order gives the
            // reference's position.
            size_t at = 0;
            if (k > 0) {
                size_t size = k, base = 0;
                while (size > 1) {
                    const size_t half = size / 2, mid = base + half;
                    if (vals[mid] >= v) base = mid;
                    size -= half;
                }
                at = base + (vals[base] >= v ? 1 : 0);
            }
            if (k == n) k--;  // out.pop()
            std::memmove(vals + at + 1, vals + at, (k - at) * sizeof(float));
            std::memmove(ids + at + 1, ids + at, (k - at) * sizeof(uint32_t));
            vals[at] = v;
            ids[at] = static_cast<uint32_t>(i);
            k++;
            if (k == n) floor = vals[n - 1];
        }
    }
    return k;
}

// argmax (sampler.rs:314-322): strict '>' keeps the first maximum.
uint32_t or_argmax(const float* x, size_t len) {
    size_t best = 0;
    for (size_t i = 0; i < len; i++)
        if (x[i] > x[best]) best = i;
    return static_cast<uint32_t>(best);
}

// logprobs (sampler.rs:297-312): max by f32::max fold, f64 sum of
// exp((l - max) as f64) in order, ln, cast to f32, added to max in f32.
float or_logprobs(const float* x, size_t len, uint32_t token, size_t n,
                  uint32_t* top_ids, float* top_lp, float* lse_out) {
    float mx = -INFINITY;
    for (size_t i = 0; i < len; i++) mx = std::fmax(mx, x[i]);
    double sum = 0.0;
    for (size_t i = 0; i < len; i++) sum += std::exp(static_cast<double>(x[i] - mx));
    float lse = mx + static_cast<float>(std::log(sum));
    if (lse_out) *lse_out = lse;
    if (n > 0 && top_ids && top_lp) {
        std::vector<float> v(n);
        std::vector<uint32_t> id(n);
        size_t k = or_top_n(x, len, n, v.data(), id.data());
        for (size_t j = 0; j < k; j++) {
            top_ids[j] = id[j];
            top_lp[j] = v[j] - lse;
        }
    }
    return x[token] - lse;
}

static void penalize_impl(float* buf, size_t n, const uint32_t* recent, size_t nrecent,
                          float rep, float pres, float freq, std::vector<uint32_t>& seen) {
    if (nrecent == 0) return;
    seen.assign(recent, recent + nrecent);
    std::sort(seen.begin(), seen.end());  // seen.sort_unstable() (sampler.rs:167)
    // sampler.rs:165-175: each DISTINCT id once, l>0 ? l/R : l*R.
    if (rep != 1.0f) {
        for (size_t i = 0; i < seen.size(); i++) {
            if (i > 0 && seen[i] == seen[i - 1]) continue;  // dedup
            uint32_t id = seen[i];
            if (id < n) {
                float l = buf[id];
                buf[id] = l > 0.0f ? l / rep : l * rep;
            }
        }
    }
    // Extension B.1 (OpenAI/vLLM presence and frequency penalties), after the
    // repetition penalty, in this exact order with no fused multiply-add:
    // l = (l - freq * (f32)count) - pres.
    if (pres != 0.0f || freq != 0.0f) {
        size_t i = 0;
        while (i < seen.size()) {
            size_t j = i;
            while (j < seen.size() && seen[j] == seen[i]) j++;
            uint32_t id = seen[i];
            if (id < n) {
                float c = static_cast<float>(j - i);
                float fc = freq * c;
                float l = buf[id] - fc;
                buf[id] = l - pres;
            }
            i = j;
        }
    }
}

void or_penalize(float* buf, size_t n, const uint32_t* recent, size_t nrecent,
                 float repetition, float presence, float frequency) {
    std::vector<uint32_t> seen;
    penalize_impl(buf, n, recent, nrecent, repetition, presence, frequency, seen);
}

void or_expf_array(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = std::exp(x[i]);  // float overload = expf
}

}  // extern "C"

namespace {

inline bool mask_allows(const uint32_t* mask, uint32_t id) {
    return (mask[id >> 5] >> (id & 31)) & 1u;
}

// Sampler::candidates (sampler.rs:155-247) plus min-p (B.2).  Fills s.ri with
// candidate ids best first and s.probs with their unnormalised
// probabilities; returns how many survive top-p.  `mask` NULL means
// unconstrained.  The ranked count after min-p is returned in *survivors.
size_t candidates(const or_config& cfg, Scratch& s, const float* logits, size_t n,
                  const uint32_t* recent, size_t nrecent, const uint32_t* mask,
                  or_row_diag* d) {
    const bool greedy = cfg.temperature <= 0.0f;
    const float t = greedy ? 1.0f : cfg.temperature;
    s.buf.assign(logits, logits + n);  // sampler.rs:163-164
    penalize_impl(s.buf.data(), n, recent, nrecent, cfg.repetition_penalty,
                  cfg.presence_penalty, cfg.frequency_penalty, s.seen);
    // sampler.rs:176-190
    size_t want = greedy ? 1 : (cfg.top_k == 0 ? n : std::min<size_t>(cfg.top_k, n));
    size_t window = mask ? std::min(std::max<size_t>(want, 256), n) : want;

    uint32_t path;
    s.rv.resize(std::max<size_t>(window, 1));
    s.ri.resize(std::max<size_t>(window, 1));
    size_t len;
    if (window <= 1024) {  // sampler.rs:193-194
        len = or_top_n(s.buf.data(), n, window, s.rv.data(), s.ri.data());
        path = OR_PATH_TOP_N;
    } else {  // sampler.rs:195-208
        float mx = -INFINITY;
        for (size_t i = 0; i < n; i++) mx = std::fmax(mx, s.buf[i]);
        const float cutoff = mx - 30.0f * t;
        s.keys.clear();
        for (size_t i = 0; i < n; i++)
            if (s.buf[i] >= cutoff) s.keys.push_back(desc_key(s.buf[i], static_cast<uint32_t>(i)));
        std::sort(s.keys.begin(), s.keys.end());
        len = s.keys.size();
        s.rv.resize(len);
        s.ri.resize(len);
        for (size_t j = 0; j < len; j++) {
            s.ri[j] = static_cast<uint32_t>(s.keys[j]);
            s.rv[j] = s.buf[s.ri[j]];
        }
        path = OR_PATH_CUTOFF;
    }
    if (mask) {  // sampler.rs:209-222
        size_t w = 0;
        for (size_t j = 0; j < len; j++)
            if (mask_allows(mask, s.ri[j])) {
                s.rv[w] = s.rv[j];
                s.ri[w] = s.ri[j];
                w++;
            }
        len = w;
        if (len == 0) {
            s.keys.clear();
            for (size_t i = 0; i < n; i++)
                if (mask_allows(mask, static_cast<uint32_t>(i)))
                    s.keys.push_back(desc_key(s.buf[i], static_cast<uint32_t>(i)));
            std::sort(s.keys.begin(), s.keys.end());
            len = s.keys.size();
            s.rv.resize(len);
            s.ri.resize(len);
            for (size_t j = 0; j < len; j++) {
                s.ri[j] = static_cast<uint32_t>(s.keys[j]);
                s.rv[j] = s.buf[s.ri[j]];
            }
            path = OR_PATH_FALLBACK;
        }
    }
    len = std::min(len, want);  // ranked.truncate(want) (sampler.rs:223)
    if (d) {
        d->path = path;
        d->ranked = static_cast<uint32_t>(len);
    }
    if (len == 0) {  // sampler.rs:226-229
        s.probs.clear();
        if (d) {
            d->path = OR_PATH_NONE_ALLOWED;
            d->survivors = 0;
        }
        return 0;
    }
    const float best = s.rv[0];  // sampler.rs:231-234
    s.probs.resize(len);
    for (size_t j = 0; j < len; j++) s.probs[j] = std::exp((s.rv[j] - best) / t);
    // Extension B.2 (min-p, as vLLM applies it before top-p): keep the
    // best-first prefix whose p_j = exp((l_j - l_0)/t) >= min_p, never fewer
    // than the best candidate.
    if (!greedy && cfg.min_p > 0.0f) {
        size_t m = 0;
        while (m < len && s.probs[m] >= cfg.min_p) m++;
        len = std::max<size_t>(m, 1);
        s.probs.resize(len);
    }
    if (d) {
        d->survivors = static_cast<uint32_t>(len);
        d->best = best;
    }
    if (greedy || cfg.top_p >= 1.0f) return len;  // sampler.rs:235-237
    float total = 0.0f;                            // sampler.rs:238-246
    for (size_t j = 0; j < len; j++) total += s.probs[j];
    float acc = 0.0f;
    for (size_t j = 0; j < len; j++) {
        acc += s.probs[j] / total;
        if (acc >= cfg.top_p) return j + 1;
    }
    return len;
}

// Sampler::pick (sampler.rs:132-151) with the uniform supplied (B.3).
// Returns the token; *keep_out = keep; prob = p_pick / mass.
uint32_t pick_impl(const or_config& cfg, Scratch& s, const float* logits, size_t n,
                   const uint32_t* recent, size_t nrecent, const uint32_t* mask,
                   float u, uint32_t* keep_out, float* prob_out, or_row_diag* d) {
    size_t keep = candidates(cfg, s, logits, n, recent, nrecent, mask, d);
    if (keep_out) *keep_out = static_cast<uint32_t>(keep);
    if (keep == 0) {  // nothing allowed: argmax of the raw row, no draw
        if (prob_out) *prob_out = 1.0f;
        if (d) {
            d->keep = 0;
            d->pick = 0;
            d->consumed_u = 0;
        }
        return or_argmax(logits, n);
    }
    float mass = 0.0f;
    for (size_t j = 0; j < keep; j++) mass += s.probs[j];
    float r = u * mass;
    size_t pick = keep - 1;
    for (size_t j = 0; j < keep; j++) {
        r -= s.probs[j];
        if (r <= 0.0f) {
            pick = j;
            break;
        }
    }
    if (prob_out) *prob_out = s.probs[pick] / mass;
    if (d) {
        d->keep = static_cast<uint32_t>(keep);
        d->pick = static_cast<uint32_t>(pick);
        d->consumed_u = 1;
        d->mass = mass;
    }
    return s.ri[pick];
}

bool fast_path(const or_config& cfg, size_t nrecent) {
    // sampler.rs:79-82, with the condition widened to the extension
    // penalties (B.1): greedy and nothing to penalize -> plain argmax.
    bool penalize = nrecent > 0 && (cfg.repetition_penalty != 1.0f ||
                                    cfg.presence_penalty != 0.0f ||
                                    cfg.frequency_penalty != 0.0f);
    return cfg.temperature <= 0.0f && !penalize;
}

or_config cfg_from_params(const tsm_row_params& p) {
    or_config c;
    c.temperature = p.temperature;
    c.top_k = p.top_k;
    c.top_p = p.top_p;
    c.repetition_penalty = p.repetition_penalty;
    c.seed = 0;
    c.presence_penalty = p.presence_penalty;
    c.frequency_penalty = p.frequency_penalty;
    c.min_p = p.min_p;
    return c;
}

template <class F>
void parallel_rows(uint32_t rows, int nthreads, F&& f) {
    if (nthreads <= 1 || rows <= 1) {
        Scratch s;
        for (uint32_t r = 0; r < rows; r++) f(r, s);
        return;
    }
    std::atomic<uint32_t> next{0};
    std::vector<std::thread> th;
    int nt = std::min<int>(nthreads, static_cast<int>(rows));
    for (int t = 0; t < nt; t++)
        th.emplace_back([&] {
            Scratch s;
            for (;;) {
                uint32_t r = next.fetch_add(1);
                if (r >= rows) break;
                f(r, s);
            }
        });
    for (auto& x : th) x.join();
}

}  // namespace

extern "C" {

or_sampler* or_sampler_new(const or_config* cfg) {
    or_sampler* s = new or_sampler();
    s->cfg = *cfg;
    s->rng = or_rng_seed(cfg->seed);
    return s;
}

void or_sampler_free(or_sampler* s) { delete s; }

uint64_t or_sampler_state(const or_sampler* s) { return s->rng; }

float or_uniform(or_sampler* s) { return or_rng_next(&s->rng); }

// Sampler::sample (sampler.rs:77-84).
uint32_t or_sample(or_sampler* s, const float* logits, size_t len, size_t vocab,
                   const uint32_t* recent, size_t nrecent) {
    size_t n = std::min(vocab, len);
    if (fast_path(s->cfg, nrecent)) return or_argmax(logits, n);
    size_t keep = candidates(s->cfg, s->s, logits, n, recent, nrecent, nullptr, nullptr);
    if (keep == 0) return or_argmax(logits, n);
    float mass = 0.0f;
    for (size_t j = 0; j < keep; j++) mass += s->s.probs[j];
    float r = or_rng_next(&s->rng) * mass;
    for (size_t j = 0; j < keep; j++) {
        r -= s->s.probs[j];
        if (r <= 0.0f) return s->s.ri[j];
    }
    return s->s.ri[keep - 1];
}

// Sampler::sample_with (sampler.rs:88-97): always picks.
uint32_t or_sample_with(or_sampler* s, const float* logits, size_t len, size_t vocab,
                        const uint32_t* recent, size_t nrecent, const uint32_t* mask) {
    size_t n = std::min(vocab, len);
    size_t keep = candidates(s->cfg, s->s, logits, n, recent, nrecent, mask, nullptr);
    if (keep == 0) return or_argmax(logits, n);
    float mass = 0.0f;
    for (size_t j = 0; j < keep; j++) mass += s->s.probs[j];
    float r = or_rng_next(&s->rng) * mass;
    for (size_t j = 0; j < keep; j++) {
        r -= s->s.probs[j];
        if (r <= 0.0f) return s->s.ri[j];
    }
    return s->s.ri[keep - 1];
}

// Sampler::distribution (sampler.rs:102-116).
size_t or_distribution(or_sampler* s, const float* logits, size_t len, size_t vocab,
                       const uint32_t* recent, size_t nrecent, uint32_t* ids,
                       float* probs, size_t cap) {
    size_t n = std::min(vocab, len);
    size_t keep = candidates(s->cfg, s->s, logits, n, recent, nrecent, nullptr, nullptr);
    float mass = 0.0f;
    for (size_t j = 0; j < keep; j++) mass += s->s.probs[j];
    for (size_t j = 0; j < keep && j < cap; j++) {
        ids[j] = s->s.ri[j];
        probs[j] = s->s.probs[j] / mass;
    }
    return keep;
}

// Sampler::draw (sampler.rs:120-130).
uint32_t or_draw(or_sampler* s, const uint32_t* ids, const float* w, size_t n) {
    float total = 0.0f;
    for (size_t j = 0; j < n; j++) total += w[j];
    float r = or_rng_next(&s->rng) * total;
    for (size_t j = 0; j < n; j++) {
        r -= w[j];
        if (r <= 0.0f) return ids[j];
    }
    return n ? ids[n - 1] : 0;
}

// speculative::verify (speculative.rs:160-189).
int or_verify(const uint32_t* p_ids, const float* p_p, size_t np, const uint32_t* q_ids,
              const float* q_p, size_t nq, uint32_t x, float u, uint32_t* res_ids,
              float* res_p, size_t* res_n) {
    auto prob = [](const uint32_t* ids, const float* p, size_t n, uint32_t t) -> float {
        for (size_t i = 0; i < n; i++)
            if (ids[i] == t) return p[i];
        return 0.0f;
    };
    auto q_of = [&](uint32_t t) -> float {
        if (nq == 0) return t == x ? 1.0f : 0.0f;
        return prob(q_ids, q_p, nq, t);
    };
    float qx = q_of(x);
    if (qx > 0.0f && u < std::fmin(prob(p_ids, p_p, np, x) / qx, 1.0f)) return 1;
    size_t k = 0;
    for (size_t i = 0; i < np; i++) {
        float r = std::fmax(p_p[i] - q_of(p_ids[i]), 0.0f);
        if (r > 0.0f) {
            res_ids[k] = p_ids[i];
            res_p[k] = r;
            k++;
        }
    }
    if (k == 0) {
        for (size_t i = 0; i < np; i++) {
            res_ids[i] = p_ids[i];
            res_p[i] = p_p[i];
        }
        k = np;
    }
    *res_n = k;
    return 0;
}

// The batched step: for each row, what src/scheduler.rs:651-663 does, with
// the row's uniform in place of Sampler::next_f32 (B.3).
int or_sample_batch(const float* logits, uint32_t rows, uint32_t row_stride, uint32_t usable,
                    const tsm_row_params* params, const uint32_t* hist_ids,
                    const uint32_t* hist_offsets, const uint32_t* mask, uint32_t mask_stride,
                    const float* uniforms, uint32_t* token, float* logprob, uint32_t* top_ids,
                    float* top_lp, uint32_t top_stride, float* prob, uint32_t* keep,
                    or_row_diag* diag, int nthreads) {
    parallel_rows(rows, nthreads, [&](uint32_t r, Scratch& s) {
        const float* x = logits + static_cast<size_t>(r) * row_stride;
        const size_t n = usable;
        const tsm_row_params& p = params[r];
        const or_config cfg = cfg_from_params(p);
        const uint32_t* recent = nullptr;
        size_t nrecent = 0;
        if (hist_offsets) {
            recent = hist_ids + hist_offsets[r];
            nrecent = hist_offsets[r + 1] - hist_offsets[r];
        }
        const bool constrained = (p.flags & TSM_ROW_CONSTRAINED) != 0;
        const uint32_t* mrow = constrained ? mask + static_cast<size_t>(r) * mask_stride : nullptr;
        or_row_diag dl;
        std::memset(&dl, 0, sizeof(dl));
        uint32_t tok, kp;
        float pr;
        if (!constrained && fast_path(cfg, nrecent)) {  // sampler.rs:79-82
            tok = or_argmax(x, n);
            kp = 1;
            pr = 1.0f;
            dl.path = OR_PATH_ARGMAX_FAST;
            dl.ranked = dl.survivors = dl.keep = 1;
        } else {
            tok = pick_impl(cfg, s, x, n, recent, nrecent, mrow, uniforms[r], &kp, &pr, &dl);
        }
        token[r] = tok;
        if (keep) keep[r] = kp;
        if (prob) prob[r] = pr;
        if (p.flags & TSM_ROW_LOGPROBS) {  // scheduler.rs:660-663
            uint32_t* ti = top_ids ? top_ids + static_cast<size_t>(r) * top_stride : nullptr;
            float* tl = top_lp ? top_lp + static_cast<size_t>(r) * top_stride : nullptr;
            float lp = or_logprobs(x, n, tok, std::min<uint32_t>(p.n_logprobs, TSM_MAX_LOGPROBS),
                                   ti, tl, nullptr);
            if (logprob) logprob[r] = lp;
        }
        if (diag) diag[r] = dl;
    });
    return 0;
}

// Parity diagnostics (not a reference function): how far u and top_p must
// move for the reference's own arithmetic to return `token` with kept count
// `keep`.  The kept count is a step function of top_p: keep = k exactly when
// acc_{k-1} < top_p <= acc_k (sampler.rs:238-245, the f32 fold).  Given keep,
// the pick depends on u only through r0 = u * mass (sampler.rs:142-149), and
// is nondecreasing in r0, so the r0 values that pick position j form one
// interval of floats, found by bisection over their bit patterns.
int or_reconcile(const float* logits, uint32_t usable, const tsm_row_params* prm,
                 const uint32_t* recent, size_t nrecent, const uint32_t* mask, float u,
                 uint32_t token, uint32_t keep, double* du, double* dp) {
    Scratch s;
    or_config cfg = cfg_from_params(*prm);
    const float top_p = cfg.top_p;
    const bool greedy = cfg.temperature <= 0.0f;
    cfg.top_p = 1.0f;  // every survivor, with its probability
    const size_t len = candidates(cfg, s, logits, usable, recent, nrecent, mask, nullptr);
    *du = 0.0;
    *dp = 0.0;
    if (keep == 0 || keep > len) return 1;
    if (greedy || top_p >= 1.0f) {
        if (keep != len) return 1;
    } else {
        float total = 0.0f;
        for (size_t j = 0; j < len; j++) total += s.probs[j];
        float acc = 0.0f, lo = -INFINITY, hi = INFINITY;
        for (size_t j = 0; j < len; j++) {
            acc += s.probs[j] / total;
            if (j + 1 == keep - 1) lo = acc;
            if (j + 1 == keep) {
                hi = keep == len ? INFINITY : acc;
                break;
            }
        }
        if (keep == 1) lo = -INFINITY;
        // keep = k for top_p in (acc_{k-1}, acc_k]; for k = len, above acc_{len-1}
        const double P = top_p;
        if (P <= lo) *dp = static_cast<double>(lo) - P;
        else if (P > hi) *dp = P - static_cast<double>(hi);
    }
    size_t j = 0;
    while (j < keep && s.ri[j] != token) j++;
    if (j == keep) return 1;
    float mass = 0.0f;
    for (size_t i = 0; i < keep; i++) mass += s.probs[i];
    auto pick_at = [&](uint32_t bits) -> size_t {
        float r;
        std::memcpy(&r, &bits, 4);
        for (size_t i = 0; i < keep; i++) {
            r -= s.probs[i];
            if (r <= 0.0f) return i;
        }
        return keep - 1;
    };
    const uint32_t top = 0x7F800000u;  // +inf: every finite r0 >= 0 lies below
    // smallest r0 picking >= j, largest picking <= j
    uint32_t a = 0, b = top;
    while (a < b) {
        const uint32_t m = a + (b - a) / 2;
        if (pick_at(m) >= j) b = m;
        else a = m + 1;
    }
    const uint32_t rlo = a;
    a = 0;
    b = top;
    while (a < b) {
        const uint32_t m = a + (b - a + 1) / 2;
        if (pick_at(m) <= j) a = m;
        else b = m - 1;
    }
    const uint32_t rhi = a;
    if (pick_at(rlo) != j || pick_at(rhi) != j || rlo > rhi) return 1;
    float flo, fhi;
    std::memcpy(&flo, &rlo, 4);
    std::memcpy(&fhi, &rhi, 4);
    const double ulo = static_cast<double>(flo) / mass, uhi = static_cast<double>(fhi) / mass;
    const double U = u;
    if (U < ulo) *du = ulo - U;
    else if (U > uhi) *du = U - uhi;
    return 0;
}

int or_distribution_batch(const float* logits, uint32_t rows, uint32_t row_stride,
                          uint32_t usable, const tsm_row_params* params,
                          const uint32_t* hist_ids, const uint32_t* hist_offsets,
                          uint32_t* dist_ids, float* dist_probs, uint32_t dist_stride,
                          uint32_t* keep, int nthreads) {
    parallel_rows(rows, nthreads, [&](uint32_t r, Scratch& s) {
        const float* x = logits + static_cast<size_t>(r) * row_stride;
        const tsm_row_params& p = params[r];
        const or_config cfg = cfg_from_params(p);
        const uint32_t* recent = nullptr;
        size_t nrecent = 0;
        if (hist_offsets) {
            recent = hist_ids + hist_offsets[r];
            nrecent = hist_offsets[r + 1] - hist_offsets[r];
        }
        size_t k = candidates(cfg, s, x, usable, recent, nrecent, nullptr, nullptr);
        float mass = 0.0f;
        for (size_t j = 0; j < k; j++) mass += s.probs[j];
        for (size_t j = 0; j < k && j < dist_stride; j++) {
            dist_ids[static_cast<size_t>(r) * dist_stride + j] = s.ri[j];
            dist_probs[static_cast<size_t>(r) * dist_stride + j] = s.probs[j] / mass;
        }
        keep[r] = static_cast<uint32_t>(k);
    });
    return 0;
}

}  // extern "C"
