// sampler.hpp - the host side of the MI355X sampling path in C++: Tachyon's
// Sampler API (src/sampler.rs) over the C ABI of include/tachyon_sampler.h.
//
// The reference's Sampler is a per-sequence object that owns the settings and
// an xorshift64* RNG and samples one row at a time on the CPU
// (src/sampler.rs:53-262); the scheduler loops over the rows of a step
// (src/scheduler.rs:638-675).  Here the same per-sequence object keeps the
// settings and the RNG, and BatchSampler samples every row of a step in one
// call on the GPU.  The RNG of each sequence advances exactly as the
// reference's would: no draw on sample()'s greedy shortcut
// (sampler.rs:79-82), no draw when nothing is kept (sampler.rs:139-141), one
// draw otherwise (sampler.rs:143).
//
// Errors are thrown as tachyon::Error carrying the C ABI's message (the
// reference's crate error is Error(String), src/lib.rs:42-71).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "tachyon_sampler.h"

namespace tachyon {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// SamplerConfig (sampler.rs:6-42), plus the extension fields of the batched
// path, whose zero values are the reference's behaviour.
struct SamplerConfig {
    float temperature = 0.7f;         // <= 0: greedy (sampler.rs:8)
    size_t top_k = 20;                // 0: no limit (sampler.rs:10)
    float top_p = 0.8f;               // (sampler.rs:12)
    float repetition_penalty = 1.05f; // (sampler.rs:14)
    uint64_t seed = clock_seed();     // (sampler.rs:15, :45-52)
    float presence_penalty = 0.0f;    // extension
    float frequency_penalty = 0.0f;   // extension
    float min_p = 0.0f;               // extension

    // SamplerConfig::greedy (sampler.rs:33-41).
    static SamplerConfig greedy();
    static uint64_t clock_seed();
};

// A uniform in [0, 1) on the 2^-24 grid, and the state after it: xorshift64*
// as Sampler::next_f32 (sampler.rs:255-261).
float xorshift_next(uint64_t* state);

// One sequence's sampler: its settings and RNG (sampler.rs:53-73).
class Sampler {
  public:
    explicit Sampler(SamplerConfig cfg);
    const SamplerConfig& config() const { return cfg_; }
    // Sampler::uniform (sampler.rs:249-252).
    float uniform() { return xorshift_next(&rng_); }
    // The RNG state, and setting it back (BatchSampler undoes a draw the
    // reference would not have made).
    uint64_t rng_state() const { return rng_; }
    void set_rng_state(uint64_t s) { rng_ = s; }

  private:
    SamplerConfig cfg_;
    uint64_t rng_;
};

// Sampler::draw (sampler.rs:119-130): a draw from weights that need not sum to
// one; the sequential f32 sums of the reference.
uint32_t draw(Sampler& s, const std::vector<std::pair<uint32_t, float>>& weighted);

// A distribution as (token, p) pairs (speculative.rs: `Dist`).
using Dist = std::vector<std::pair<uint32_t, float>>;

// The speculative sampling rule (speculative.rs:306-318) for one draft x
// drawn from q (an empty q: the draft was chosen deterministically), given the
// target's p, e.g. from BatchSampler::distribution, and a uniform u in [0, 1):
// accept when q(x) > 0 and u < min(p(x) / q(x), 1); otherwise the replacement
// is drawn from the residual max(p - q, 0) (p itself when that is empty).
struct Verdict {
    bool accept = false;
    Dist resample;  // when rejected: the distribution to draw the replacement from
};
Verdict verify(const Dist& p, const Dist& q, uint32_t x, float u);

// TokenLogprob (sampler.rs:287-295): the pick's log-probability under the raw
// logits and the best alternatives, best first.
struct TokenLogprob {
    uint32_t token = 0;
    float logprob = 0.0f;
    std::vector<std::pair<uint32_t, float>> top;
};

// One row of a step.
struct RowRequest {
    Sampler* sampler = nullptr;         // the sequence (its RNG advances)
    const uint32_t* recent = nullptr;   // host ids: the `recent` slice (scheduler.rs:653)
    size_t n_recent = 0;
    bool constrained = false;           // sample_with(): the mask row applies (sampler.rs:88-97)
    size_t logprobs = 0;                // with want_logprobs: alternatives, <= 20 (server.rs:633)
    bool want_logprobs = false;
};

// The batched sampler of one HIP stream (not re-entrant, as the reference's
// GpuBackend, src/gpu/mod.rs:440-442).  Device buffers and pinned staging are
// allocated once, here; a call allocates nothing.
class BatchSampler {
  public:
    BatchSampler(int device, uint32_t max_rows, uint32_t max_vocab, uint32_t max_recent_per_row = 1024,
                 uint32_t max_dist_pairs = 1024);
    ~BatchSampler();
    BatchSampler(const BatchSampler&) = delete;
    BatchSampler& operator=(const BatchSampler&) = delete;

    // Samples one token per row: logits is a DEVICE [rows][row_stride] f32
    // matrix, vocab caps the ids (scheduler.rs:625-626), mask (DEVICE,
    // [rows][mask_stride] packed words) is read by constrained rows only.
    // Waits for the call to finish.  With `logprobs`, rows that ask get
    // their TokenLogprob (others an empty one).
    std::vector<uint32_t> sample(const float* logits, uint32_t rows, uint32_t row_stride, size_t vocab,
                                 const std::vector<RowRequest>& req, const uint32_t* mask = nullptr,
                                 uint32_t mask_stride = 0, void* stream = nullptr,
                                 std::vector<TokenLogprob>* logprobs = nullptr);

    // Sampler::distribution (sampler.rs:102-116) of every row: normalised
    // (token, p) pairs, best first, at most max_pairs (<= max_dist_pairs) per
    // row (`kept` gets each row's full count).  No draw; constraints do not
    // apply.
    std::vector<std::vector<std::pair<uint32_t, float>>> distribution(
        const float* logits, uint32_t rows, uint32_t row_stride, size_t vocab, const std::vector<RowRequest>& req,
        uint32_t max_pairs, void* stream = nullptr, std::vector<uint32_t>* kept = nullptr);

    // The device status of the last call (TSM_STATUS_* bits of tsm_status).
    uint32_t last_status() const { return last_status_; }

  private:
    struct Staging;
    void stage_inputs(uint32_t rows, const std::vector<RowRequest>& req, bool for_distribution,
                      std::vector<uint64_t>* saved_rng, std::vector<char>* drew);
    int device_;
    uint32_t max_rows_, max_recent_, max_dist_;
    uint32_t last_status_ = 0;
    tsm_ctx* ctx_ = nullptr;
    Staging* st_ = nullptr;
};

// ---- constrained decoding: JsonObject (src/constrain.rs) -----------------------

// A tokenizer's token bytes and special flags on the host (tokenizer.rs:
// 189-195: token_bytes, is_special).
struct Vocab {
    std::vector<std::vector<uint8_t>> tokens;
    std::vector<bool> special;  // empty or one flag per token
};

// The Constraint for `response_format: json_object` (constrain.rs:14-42,
// 88-302), on the packed state the GPU mask producer reads.
class JsonObjectConstraint {
  public:
    JsonObjectConstraint();                       // JsonObject::default()
    // Constraint::allows (constrain.rs:286-290) for one token, on the host.
    bool allows(const Vocab& v, uint32_t token) const;
    bool accepts(const uint8_t* bytes, size_t n) const;  // accepts_bytes
    void advance(const uint8_t* bytes, size_t n);        // Constraint::advance
    bool is_complete() const;                            // Constraint::is_complete
    const tsm_json_state& state() const { return s_; }

  private:
    tsm_json_state s_;
};

// The vocabulary in device memory for the mask producer, uploaded once, with
// room for the states of up to max_rows constrained rows (a step allocates
// nothing).
class DeviceVocab {
  public:
    DeviceVocab(int device, const Vocab& v, uint32_t max_rows = 1024);
    ~DeviceVocab();
    DeviceVocab(const DeviceVocab&) = delete;
    DeviceVocab& operator=(const DeviceVocab&) = delete;
    const tsm_vocab& abi() const { return abi_; }
    uint32_t size() const { return abi_.n_tokens; }

    // The allow-bits of a step's constrained rows, every token at once on the
    // GPU (tsm_json_mask): row r of `mask` (DEVICE, [rows][mask_stride]
    // words) gets rows[r]'s allows() for ids [0, usable), the layout
    // BatchSampler::sample takes.  Waits for the masks.
    void json_masks(const std::vector<const JsonObjectConstraint*>& rows, uint32_t usable, uint32_t* mask,
                    uint32_t mask_stride, void* stream = nullptr);

  private:
    int device_;
    uint32_t max_rows_;
    tsm_vocab abi_{};
    void* mem_ = nullptr;
    tsm_json_state* states_ = nullptr;  // device, [max_rows]
};

}  // namespace tachyon
