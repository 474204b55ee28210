// sampler.cpp - Tachyon's Sampler API on the batched GPU path (see sampler.hpp).
#include "sampler.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <type_traits>

namespace tachyon {

namespace {

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

// The reference decides per row whether pick() runs and so whether the RNG
// advances: sample() takes no draw on its greedy shortcut (sampler.rs:79-82;
// the condition widened to the extension penalties), sample_with() always
// picks (sampler.rs:96).
bool greedy_shortcut(const SamplerConfig& c, const RowRequest& r) {
    const bool penalize = r.n_recent > 0 && (c.repetition_penalty != 1.0f || c.presence_penalty != 0.0f ||
                                             c.frequency_penalty != 0.0f);
    return !r.constrained && c.temperature <= 0.0f && !penalize;
}

}  // namespace

SamplerConfig SamplerConfig::greedy() {
    SamplerConfig c;
    c.temperature = 0.0f;
    c.top_k = 1;
    c.top_p = 1.0f;
    c.repetition_penalty = 1.0f;
    c.seed = 0;
    return c;
}

uint64_t SamplerConfig::clock_seed() {
    const auto ns = std::chrono::duration_cast<std::chrono::nanoseconds>(
                        std::chrono::system_clock::now().time_since_epoch())
                        .count();
    return ns > 0 ? static_cast<uint64_t>(ns) : 0x9E3779B9ull;  // sampler.rs:45-52
}

float xorshift_next(uint64_t* state) {
    uint64_t s = *state;
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    *state = s;
    const uint64_t x = s * 0x2545F4914F6CDD1Dull;
    return static_cast<float>(x >> 40) / static_cast<float>(1ull << 24);
}

Sampler::Sampler(SamplerConfig cfg) : cfg_(cfg), rng_(cfg.seed * 0x2545F4914F6CDD1Dull | 1ull) {}

uint32_t draw(Sampler& s, const std::vector<std::pair<uint32_t, float>>& weighted) {
    float total = 0.0f;
    for (const auto& w : weighted) total += w.second;
    float r = s.uniform() * total;
    for (const auto& w : weighted) {
        r -= w.second;
        if (r <= 0.0f) return w.first;
    }
    return weighted.empty() ? 0u : weighted.back().first;
}

namespace {
float prob_of(const Dist& d, uint32_t t) {
    for (const auto& e : d)
        if (e.first == t) return e.second;
    return 0.0f;
}
}  // namespace

Verdict verify(const Dist& p, const Dist& q, uint32_t x, float u) {
    auto q_of = [&](uint32_t t) { return q.empty() ? (t == x ? 1.0f : 0.0f) : prob_of(q, t); };
    Verdict v;
    const float qx = q_of(x);
    if (qx > 0.0f && u < std::min(prob_of(p, x) / qx, 1.0f)) {
        v.accept = true;
        return v;
    }
    for (const auto& e : p) {
        const float r = std::max(e.second - q_of(e.first), 0.0f);
        if (r > 0.0f) v.resample.emplace_back(e.first, r);
    }
    if (v.resample.empty()) v.resample = p;
    return v;
}

// Device inputs/outputs and their pinned host mirrors, sized at creation.
struct BatchSampler::Staging {
    tsm_row_params* h_params = nullptr;
    uint32_t* h_hist_off = nullptr;
    uint32_t* h_hist_ids = nullptr;
    float* h_u = nullptr;
    uint32_t* h_token = nullptr;
    float* h_logprob = nullptr;
    uint32_t* h_top_ids = nullptr;
    float* h_top_lp = nullptr;
    uint32_t* h_keep = nullptr;
    tsm_row_params* d_params = nullptr;
    uint32_t* d_hist_off = nullptr;
    uint32_t* d_hist_ids = nullptr;
    float* d_u = nullptr;
    uint32_t* d_token = nullptr;
    float* d_logprob = nullptr;
    uint32_t* d_top_ids = nullptr;
    float* d_top_lp = nullptr;
    uint32_t* d_keep = nullptr;
    uint32_t* d_dist_ids = nullptr;
    float* d_dist_p = nullptr;
    uint32_t hist_total = 0;
};

BatchSampler::BatchSampler(int device, uint32_t max_rows, uint32_t max_vocab, uint32_t max_recent_per_row,
                           uint32_t max_dist_pairs)
    : device_(device),
      max_rows_(max_rows),
      max_recent_(max_recent_per_row),
      max_dist_(max_dist_pairs) {
    char err[256] = {0};
    ctx_ = tsm_create(device, max_rows, max_vocab, err, sizeof err);
    if (!ctx_) throw Error(err);
    check(hipSetDevice(device), "hipSetDevice");
    st_ = new Staging();
    const size_t hist = static_cast<size_t>(max_rows) * max_recent_per_row;
    const size_t tops = static_cast<size_t>(max_rows) * TSM_MAX_LOGPROBS;
    auto both = [&](auto** h, auto** d, size_t n) {
        using T = std::remove_pointer_t<std::remove_pointer_t<decltype(h)>>;
        check(hipHostMalloc(reinterpret_cast<void**>(h), n * sizeof(T), hipHostMallocDefault), "hipHostMalloc");
        check(hipMalloc(reinterpret_cast<void**>(d), n * sizeof(T)), "hipMalloc");
    };
    both(&st_->h_params, &st_->d_params, max_rows);
    both(&st_->h_hist_off, &st_->d_hist_off, max_rows + 1u);
    both(&st_->h_hist_ids, &st_->d_hist_ids, hist ? hist : 1);
    both(&st_->h_u, &st_->d_u, max_rows);
    both(&st_->h_token, &st_->d_token, max_rows);
    both(&st_->h_logprob, &st_->d_logprob, max_rows);
    both(&st_->h_top_ids, &st_->d_top_ids, tops);
    both(&st_->h_top_lp, &st_->d_top_lp, tops);
    both(&st_->h_keep, &st_->d_keep, max_rows);
    const size_t dist = static_cast<size_t>(max_rows) * (max_dist_pairs ? max_dist_pairs : 1u);
    check(hipMalloc(reinterpret_cast<void**>(&st_->d_dist_ids), dist * sizeof(uint32_t)), "hipMalloc");
    check(hipMalloc(reinterpret_cast<void**>(&st_->d_dist_p), dist * sizeof(float)), "hipMalloc");
}

BatchSampler::~BatchSampler() {
    if (st_) {
        for (void* p : {static_cast<void*>(st_->h_params), static_cast<void*>(st_->h_hist_off),
                        static_cast<void*>(st_->h_hist_ids), static_cast<void*>(st_->h_u),
                        static_cast<void*>(st_->h_token), static_cast<void*>(st_->h_logprob),
                        static_cast<void*>(st_->h_top_ids), static_cast<void*>(st_->h_top_lp),
                        static_cast<void*>(st_->h_keep)})
            if (p) (void)hipHostFree(p);
        for (void* p : {static_cast<void*>(st_->d_params), static_cast<void*>(st_->d_hist_off),
                        static_cast<void*>(st_->d_hist_ids), static_cast<void*>(st_->d_u),
                        static_cast<void*>(st_->d_token), static_cast<void*>(st_->d_logprob),
                        static_cast<void*>(st_->d_top_ids), static_cast<void*>(st_->d_top_lp),
                        static_cast<void*>(st_->d_keep), static_cast<void*>(st_->d_dist_ids),
                        static_cast<void*>(st_->d_dist_p)})
            if (p) (void)hipFree(p);
        delete st_;
    }
    tsm_destroy(ctx_);
}

// Fills the pinned staging from the requests; for sample(), draws each row's
// uniform where the reference's pick() would, remembering the state before.
void BatchSampler::stage_inputs(uint32_t rows, const std::vector<RowRequest>& req, bool for_distribution,
                                std::vector<uint64_t>* saved_rng, std::vector<char>* drew) {
    if (rows > max_rows_) throw Error("rows " + std::to_string(rows) + " exceed max_rows " + std::to_string(max_rows_));
    if (req.size() != rows) throw Error("one RowRequest per row is required");
    // every row is checked before any RNG advances
    for (uint32_t r = 0; r < rows; r++) {
        const RowRequest& q = req[r];
        if (!q.sampler) throw Error("row " + std::to_string(r) + " has no sampler");
        if (q.sampler->config().top_k > 0xFFFFFFFFull) throw Error("top_k does not fit 32 bits");
        if (!for_distribution && q.want_logprobs && q.logprobs > TSM_MAX_LOGPROBS)
            throw Error("logprobs " + std::to_string(q.logprobs) + " above " + std::to_string(TSM_MAX_LOGPROBS));
        if (q.n_recent > max_recent_)
            throw Error("row " + std::to_string(r) + ": recent longer than max_recent_per_row");
    }
    uint32_t off = 0;
    for (uint32_t r = 0; r < rows; r++) {
        const RowRequest& q = req[r];
        const SamplerConfig& c = q.sampler->config();
        tsm_row_params& p = st_->h_params[r];
        std::memset(&p, 0, sizeof p);
        p.temperature = c.temperature;
        p.top_k = static_cast<uint32_t>(c.top_k);
        p.top_p = c.top_p;
        p.repetition_penalty = c.repetition_penalty;
        p.presence_penalty = c.presence_penalty;
        p.frequency_penalty = c.frequency_penalty;
        p.min_p = c.min_p;
        if (!for_distribution) {
            p.flags = (q.constrained ? TSM_ROW_CONSTRAINED : 0u) | (q.want_logprobs ? TSM_ROW_LOGPROBS : 0u);
            p.n_logprobs = q.want_logprobs ? static_cast<uint32_t>(q.logprobs) : 0u;
        }
        st_->h_hist_off[r] = off;
        if (q.n_recent) std::memcpy(st_->h_hist_ids + off, q.recent, q.n_recent * sizeof(uint32_t));
        off += static_cast<uint32_t>(q.n_recent);
        float u = 0.0f;
        if (!for_distribution) {
            (*saved_rng)[r] = q.sampler->rng_state();
            (*drew)[r] = !greedy_shortcut(c, q);
            if ((*drew)[r]) u = q.sampler->uniform();
        }
        st_->h_u[r] = u;
    }
    st_->h_hist_off[rows] = off;
    st_->hist_total = off;
}

std::vector<uint32_t> BatchSampler::sample(const float* logits, uint32_t rows, uint32_t row_stride, size_t vocab,
                                           const std::vector<RowRequest>& req, const uint32_t* mask,
                                           uint32_t mask_stride, void* stream, std::vector<TokenLogprob>* logprobs) {
    std::vector<uint64_t> saved(rows);
    std::vector<char> drew(rows);
    stage_inputs(rows, req, false, &saved, &drew);
    const uint32_t usable = static_cast<uint32_t>(vocab < row_stride ? vocab : row_stride);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    check(hipSetDevice(device_), "hipSetDevice");
    check(hipMemcpyAsync(st_->d_params, st_->h_params, rows * sizeof(tsm_row_params), hipMemcpyHostToDevice, s),
          "copy params");
    check(hipMemcpyAsync(st_->d_hist_off, st_->h_hist_off, (rows + 1u) * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy history offsets");
    if (st_->hist_total)
        check(hipMemcpyAsync(st_->d_hist_ids, st_->h_hist_ids, st_->hist_total * sizeof(uint32_t),
                             hipMemcpyHostToDevice, s),
              "copy history");
    check(hipMemcpyAsync(st_->d_u, st_->h_u, rows * sizeof(float), hipMemcpyHostToDevice, s), "copy uniforms");
    tsm_batch b{};
    b.logits = logits;
    b.rows = rows;
    b.row_stride = row_stride;
    b.usable = usable;
    b.mask_stride = mask_stride;
    b.params = st_->d_params;
    b.hist_ids = st_->hist_total ? st_->d_hist_ids : nullptr;
    b.hist_offsets = st_->hist_total ? st_->d_hist_off : nullptr;
    b.mask = mask;
    b.uniforms = st_->d_u;
    tsm_outputs o{};
    o.token = st_->d_token;
    o.keep = st_->d_keep;
    const bool lp = logprobs != nullptr;
    if (lp) {
        o.logprob = st_->d_logprob;
        o.top_ids = st_->d_top_ids;
        o.top_logprobs = st_->d_top_lp;
        o.top_stride = TSM_MAX_LOGPROBS;
    }
    char err[256] = {0};
    if (tsm_sample(ctx_, stream, &b, &o, err, sizeof err) != 0) {
        for (uint32_t r = 0; r < rows; r++) req[r].sampler->set_rng_state(saved[r]);  // nothing was sampled
        throw Error(err);
    }
    check(hipMemcpyAsync(st_->h_token, st_->d_token, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, s),
          "copy tokens");
    check(hipMemcpyAsync(st_->h_keep, st_->d_keep, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, s), "copy keep");
    if (lp) {
        check(hipMemcpyAsync(st_->h_logprob, st_->d_logprob, rows * sizeof(float), hipMemcpyDeviceToHost, s),
              "copy logprobs");
        check(hipMemcpyAsync(st_->h_top_ids, st_->d_top_ids, rows * TSM_MAX_LOGPROBS * sizeof(uint32_t),
                             hipMemcpyDeviceToHost, s),
              "copy top ids");
        check(hipMemcpyAsync(st_->h_top_lp, st_->d_top_lp, rows * TSM_MAX_LOGPROBS * sizeof(float),
                             hipMemcpyDeviceToHost, s),
              "copy top logprobs");
    }
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    std::vector<uint32_t> tokens(st_->h_token, st_->h_token + rows);
    for (uint32_t r = 0; r < rows; r++)
        if (drew[r] && st_->h_keep[r] == 0) req[r].sampler->set_rng_state(saved[r]);  // sampler.rs:139-141: no draw
    if (lp) {
        logprobs->assign(rows, TokenLogprob{});
        for (uint32_t r = 0; r < rows; r++) {
            if (!req[r].want_logprobs) continue;
            TokenLogprob& t = (*logprobs)[r];
            t.token = tokens[r];
            t.logprob = st_->h_logprob[r];
            for (size_t j = 0; j < req[r].logprobs; j++)
                t.top.emplace_back(st_->h_top_ids[r * TSM_MAX_LOGPROBS + j], st_->h_top_lp[r * TSM_MAX_LOGPROBS + j]);
        }
    }
    if (tsm_status(ctx_, &last_status_, err, sizeof err) != 0) throw Error(err);
    return tokens;
}

std::vector<std::vector<std::pair<uint32_t, float>>> BatchSampler::distribution(
    const float* logits, uint32_t rows, uint32_t row_stride, size_t vocab, const std::vector<RowRequest>& req,
    uint32_t max_pairs, void* stream, std::vector<uint32_t>* kept) {
    if (max_pairs == 0 || max_pairs > max_dist_)
        throw Error("max_pairs must be in [1, " + std::to_string(max_dist_) + "]");
    stage_inputs(rows, req, true, nullptr, nullptr);
    const uint32_t usable = static_cast<uint32_t>(vocab < row_stride ? vocab : row_stride);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    check(hipSetDevice(device_), "hipSetDevice");
    const size_t n = static_cast<size_t>(rows) * max_pairs;
    std::vector<uint32_t> ids(n), keep(rows);
    std::vector<float> p(n);
    check(hipMemcpyAsync(st_->d_params, st_->h_params, rows * sizeof(tsm_row_params), hipMemcpyHostToDevice, s),
          "copy params");
    check(hipMemcpyAsync(st_->d_hist_off, st_->h_hist_off, (rows + 1u) * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy history offsets");
    if (st_->hist_total)
        check(hipMemcpyAsync(st_->d_hist_ids, st_->h_hist_ids, st_->hist_total * sizeof(uint32_t),
                             hipMemcpyHostToDevice, s),
              "copy history");
    tsm_batch b{};
    b.logits = logits;
    b.rows = rows;
    b.row_stride = row_stride;
    b.usable = usable;
    b.params = st_->d_params;
    b.hist_ids = st_->hist_total ? st_->d_hist_ids : nullptr;
    b.hist_offsets = st_->hist_total ? st_->d_hist_off : nullptr;
    char err[256] = {0};
    if (tsm_distribution(ctx_, stream, &b, st_->d_dist_ids, st_->d_dist_p, max_pairs, st_->d_keep, err, sizeof err))
        throw Error(err);
    check(hipMemcpyAsync(ids.data(), st_->d_dist_ids, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s), "copy ids");
    check(hipMemcpyAsync(p.data(), st_->d_dist_p, n * sizeof(float), hipMemcpyDeviceToHost, s), "copy probs");
    check(hipMemcpyAsync(keep.data(), st_->d_keep, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, s), "copy keep");
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (tsm_status(ctx_, &last_status_, err, sizeof err) != 0) throw Error(err);
    std::vector<std::vector<std::pair<uint32_t, float>>> out(rows);
    for (uint32_t r = 0; r < rows; r++) {
        const uint32_t m = keep[r] < max_pairs ? keep[r] : max_pairs;
        for (uint32_t j = 0; j < m; j++)
            out[r].emplace_back(ids[static_cast<size_t>(r) * max_pairs + j], p[static_cast<size_t>(r) * max_pairs + j]);
    }
    if (kept) *kept = keep;
    return out;
}

// ---- constrained decoding: JsonObject ---------------------------------------------

JsonObjectConstraint::JsonObjectConstraint() { tsm_json_init(&s_); }

bool JsonObjectConstraint::allows(const Vocab& v, uint32_t token) const {
    if (token >= v.tokens.size()) return false;  // token_bytes: empty past the table
    if (token < v.special.size() && v.special[token]) return false;
    const auto& b = v.tokens[token];
    return !b.empty() && tsm_json_accepts(&s_, b.data(), b.size()) != 0;
}

bool JsonObjectConstraint::accepts(const uint8_t* bytes, size_t n) const { return tsm_json_accepts(&s_, bytes, n) != 0; }

void JsonObjectConstraint::advance(const uint8_t* bytes, size_t n) { tsm_json_advance(&s_, bytes, n); }

bool JsonObjectConstraint::is_complete() const { return tsm_json_is_complete(&s_) != 0; }

DeviceVocab::DeviceVocab(int device, const Vocab& v, uint32_t max_rows) : device_(device), max_rows_(max_rows) {
    const size_t n = v.tokens.size();
    std::vector<uint32_t> offsets(n + 1, 0);
    for (size_t i = 0; i < n; i++) offsets[i + 1] = offsets[i] + static_cast<uint32_t>(v.tokens[i].size());
    std::vector<uint8_t> bytes(offsets[n] ? offsets[n] : 1u, 0);
    for (size_t i = 0; i < n; i++)
        if (!v.tokens[i].empty()) std::memcpy(bytes.data() + offsets[i], v.tokens[i].data(), v.tokens[i].size());
    std::vector<uint32_t> special((n + 31) / 32 + 1, 0u);
    for (size_t i = 0; i < n && i < v.special.size(); i++)
        if (v.special[i]) special[i >> 5] |= 1u << (i & 31u);
    const size_t ob = offsets.size() * 4, sb = special.size() * 4, bb = bytes.size();
    const size_t stb = (static_cast<size_t>(max_rows_) * sizeof(tsm_json_state) + 255) / 256 * 256;
    int prev = 0;
    check(hipGetDevice(&prev), "hipGetDevice");
    check(hipSetDevice(device_), "hipSetDevice");
    hipError_t e = hipMalloc(&mem_, stb + ob + sb + bb);
    states_ = static_cast<tsm_json_state*>(mem_);
    char* p = static_cast<char*>(mem_) + stb;
    if (e == hipSuccess) e = hipMemcpy(p, offsets.data(), ob, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p + ob, special.data(), sb, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p + ob + sb, bytes.data(), bb, hipMemcpyHostToDevice);
    (void)hipSetDevice(prev);
    check(e, "DeviceVocab upload");
    abi_.offsets = reinterpret_cast<const uint32_t*>(p);
    abi_.special = reinterpret_cast<const uint32_t*>(p + ob);
    abi_.bytes = reinterpret_cast<const uint8_t*>(p + ob + sb);
    abi_.n_tokens = static_cast<uint32_t>(n);
    abi_.reserved = 0;
}

DeviceVocab::~DeviceVocab() {
    if (mem_) (void)hipFree(mem_);
}

void DeviceVocab::json_masks(const std::vector<const JsonObjectConstraint*>& rows, uint32_t usable, uint32_t* mask,
                             uint32_t mask_stride, void* stream) {
    if (rows.empty()) return;
    if (rows.size() > max_rows_)
        throw Error("json_masks: " + std::to_string(rows.size()) + " rows exceed the vocabulary's max_rows " +
                    std::to_string(max_rows_));
    std::vector<tsm_json_state> states(rows.size());
    for (size_t r = 0; r < rows.size(); r++) {
        if (!rows[r]) throw Error("json_masks: a row has no constraint");
        states[r] = rows[r]->state();
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    check(hipMemcpyAsync(states_, states.data(), states.size() * sizeof(tsm_json_state), hipMemcpyHostToDevice, s),
          "json_masks upload");
    char err[256] = {0};
    const int rc = tsm_json_mask(stream, &abi_, states_, static_cast<uint32_t>(rows.size()), usable, mask,
                                 mask_stride, err, sizeof(err));
    check(hipStreamSynchronize(s), "json_masks");  // `states` is read by the copy until then
    if (rc != 0) throw Error(err);
}

}  // namespace tachyon
