// test_sampler_host.cpp - the C++ Sampler API (tachyon_amd/host/sampler.hpp)
// tested the way the reference tests its sampler (src/sampler.rs:324-395),
// plus a sequence-level check against the CPU oracle: tokens and RNG states of
// several sequences over many steps.
//
//   test_sampler_host --cpu   host-only tests (RNG, draw, settings)
//   test_sampler_host         host-only tests and the GPU tests
//
// Prints one line per test and exits nonzero if any fails.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "../../oracle/tachyon_oracle.h"
#include "../../tachyon_amd/host/sampler.hpp"

using namespace tachyon;

namespace {

int g_failed = 0;

#define EXPECT(cond, ...)                                                \
    do {                                                                 \
        if (!(cond)) {                                                   \
            char m_[512];                                                \
            std::snprintf(m_, sizeof m_, __VA_ARGS__);                   \
            throw std::runtime_error(std::string(#cond) + ": " + m_);    \
        }                                                                \
    } while (0)

void run(const char* name, const std::function<void()>& f) {
    try {
        f();
        std::printf("PASS %s\n", name);
    } catch (const std::exception& e) {
        std::printf("FAIL %s: %s\n", name, e.what());
        g_failed++;
    }
    std::fflush(stdout);
}

SamplerConfig cfg(float t, size_t k, float p, float r, uint64_t seed) {
    SamplerConfig c;
    c.temperature = t;
    c.top_k = k;
    c.top_p = p;
    c.repetition_penalty = r;
    c.seed = seed;
    return c;
}

or_config ocfg(const SamplerConfig& c) {
    or_config o{};
    o.temperature = c.temperature;
    o.top_k = static_cast<uint32_t>(c.top_k);
    o.top_p = c.top_p;
    o.repetition_penalty = c.repetition_penalty;
    o.seed = c.seed;
    o.presence_penalty = c.presence_penalty;
    o.frequency_penalty = c.frequency_penalty;
    o.min_p = c.min_p;
    return o;
}

// Device copy of host rows (freed by the caller).
template <class T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), std::max<size_t>(h.size(), 1) * sizeof(T)) != hipSuccess)
        throw std::runtime_error("hipMalloc");
    if (!h.empty() && hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("hipMemcpy");
    return d;
}

std::vector<uint32_t> pack(const std::vector<bool>& allowed) {
    std::vector<uint32_t> w((allowed.size() + 31) / 32, 0u);
    for (size_t i = 0; i < allowed.size(); i++)
        if (allowed[i]) w[i / 32] |= 1u << (i % 32);
    return w;
}

// One row sampled through the batched API (B = 1), as Sampler::sample /
// sample_with.
uint32_t sample1(BatchSampler& bs, Sampler& s, const std::vector<float>& logits, const std::vector<uint32_t>& recent,
                 const std::vector<bool>* allowed = nullptr, std::vector<TokenLogprob>* lp = nullptr,
                 size_t n_lp = 0) {
    float* d = to_device(logits);
    uint32_t* dm = nullptr;
    std::vector<uint32_t> words;
    if (allowed) {
        words = pack(*allowed);
        dm = to_device(words);
    }
    RowRequest q;
    q.sampler = &s;
    q.recent = recent.data();
    q.n_recent = recent.size();
    q.constrained = allowed != nullptr;
    q.want_logprobs = lp != nullptr;
    q.logprobs = n_lp;
    std::vector<uint32_t> t;
    try {
        t = bs.sample(d, 1, static_cast<uint32_t>(logits.size()), logits.size(), {q}, dm,
                      static_cast<uint32_t>(words.size()), nullptr, lp);
    } catch (...) {
        (void)hipFree(d);
        if (dm) (void)hipFree(dm);
        throw;
    }
    (void)hipFree(d);
    if (dm) (void)hipFree(dm);
    return t[0];
}

// ---- host-only ----

void rng_matches_the_oracle() {
    for (uint64_t seed : {0ull, 1ull, 3ull, 42ull, 0x5EED0004ull, 0xFFFFFFFFFFFFFFFFull}) {
        Sampler s(cfg(1.0f, 0, 1.0f, 1.0f, seed));
        or_config oc = ocfg(s.config());
        or_sampler* o = or_sampler_new(&oc);
        for (int i = 0; i < 1000; i++) {
            const float a = s.uniform(), b = or_uniform(o);
            EXPECT(a == b && s.rng_state() == or_sampler_state(o), "seed %llu draw %d: %.9g vs %.9g",
                   static_cast<unsigned long long>(seed), i, a, b);
            EXPECT(a >= 0.0f && a < 1.0f && std::ldexp(a, 24) == std::floor(std::ldexp(a, 24)), "u %.9g off grid", a);
        }
        or_sampler_free(o);
    }
}

void draw_matches_the_oracle() {
    std::mt19937 g(7);
    for (int t = 0; t < 200; t++) {
        const uint64_t seed = g();
        Sampler s(cfg(1.0f, 0, 1.0f, 1.0f, seed));
        or_config oc = ocfg(s.config());
        or_sampler* o = or_sampler_new(&oc);
        std::vector<std::pair<uint32_t, float>> w(1 + g() % 50);
        std::vector<uint32_t> ids;
        std::vector<float> ps;
        for (auto& x : w) {
            x = {static_cast<uint32_t>(g() % 1000), std::uniform_real_distribution<float>(0.0f, 1.0f)(g)};
            ids.push_back(x.first);
            ps.push_back(x.second);
        }
        const uint32_t a = draw(s, w), b = or_draw(o, ids.data(), ps.data(), ids.size());
        EXPECT(a == b, "case %d: %u vs %u", t, a, b);
        or_sampler_free(o);
    }
}

void greedy_settings() {
    const SamplerConfig c = SamplerConfig::greedy();  // sampler.rs:33-41
    EXPECT(c.temperature == 0.0f && c.top_k == 1 && c.top_p == 1.0f && c.repetition_penalty == 1.0f && c.seed == 0,
           "greedy()");
    const SamplerConfig d;  // sampler.rs:19-30
    EXPECT(d.temperature == 0.7f && d.top_k == 20 && d.top_p == 0.8f && d.repetition_penalty == 1.05f, "default()");
}

// ---- speculative sampling (the reference's tests, speculative.rs:349-385) ----

void speculative_sampling_preserves_the_target_distribution() {
    const Dist p = {{0, 0.5f}, {1, 0.3f}, {2, 0.2f}};
    const Dist q = {{0, 0.2f}, {1, 0.6f}, {2, 0.2f}};
    Sampler rng(cfg(1.0f, 0, 1.0f, 1.0f, 7));
    const int trials = 200000;
    int counts[3] = {0, 0, 0};
    for (int i = 0; i < trials; i++) {
        const uint32_t x = draw(rng, q);
        const float u = rng.uniform();
        const Verdict v = verify(p, q, x, u);
        const uint32_t t = v.accept ? x : draw(rng, v.resample);
        counts[t]++;
    }
    for (int i = 0; i < 3; i++) {
        const float got = static_cast<float>(counts[i]) / trials;
        EXPECT(std::fabs(got - p[i].second) < 0.01f, "token %d: %.4f vs %.4f", i, got, p[i].second);
    }
}

void deterministic_drafts_reduce_to_greedy() {
    const Dist p = {{4, 1.0f}};
    EXPECT(verify(p, {}, 4, 0.99f).accept, "accept");
    const Verdict v = verify(p, {}, 5, 0.0f);
    EXPECT(!v.accept && v.resample.size() == 1 && v.resample[0].first == 4 && v.resample[0].second == 1.0f,
           "resample");
}

// ---- GPU (the reference's tests, sampler.rs:328-395, through the batched path) ----

void greedy_and_top_k(BatchSampler& bs) {
    const std::vector<float> logits = {0.1f, 3.0f, 2.9f, -1.0f};
    Sampler g(SamplerConfig::greedy());
    EXPECT(sample1(bs, g, logits, {}) == 1, "greedy pick");
    Sampler s(cfg(1.0f, 2, 1.0f, 1.0f, 3));
    for (int i = 0; i < 200; i++) {
        const uint32_t t = sample1(bs, s, logits, {});
        EXPECT(t == 1 || t == 2, "draw %d gave %u", i, t);
    }
}

void constraint_and_distribution(BatchSampler& bs) {
    const std::vector<float> logits = {0.1f, 3.0f, 2.9f, -1.0f};
    Sampler g(SamplerConfig::greedy());
    const std::vector<bool> not1 = {true, false, true, true};
    EXPECT(sample1(bs, g, logits, {}, &not1) == 2, "sample_with");
    Sampler s(cfg(1.0f, 0, 1.0f, 1.0f, 1));
    float* d = to_device(logits);
    RowRequest q;
    q.sampler = &s;
    const auto dist = bs.distribution(d, 1, 4, 4, {q}, 16);
    (void)hipFree(d);
    EXPECT(!dist[0].empty() && dist[0][0].first == 1, "best first");
    float sum = 0.0f;
    for (const auto& x : dist[0]) sum += x.second;
    EXPECT(std::fabs(sum - 1.0f) < 1e-5f, "sum %.9g", sum);
}

void top_n_matches_a_full_sort(BatchSampler& bs) {
    // the reference's values (sampler.rs:361-364); the batched path reports at
    // most 20 alternatives (server.rs:633), so 20 of the 37
    std::vector<float> x(5000);
    for (uint32_t i = 0; i < 5000; i++) x[i] = static_cast<float>((i * 2654435761u) % 10007u);
    std::vector<float> sorted = x;
    std::sort(sorted.begin(), sorted.end(), std::greater<float>());
    Sampler g(SamplerConfig::greedy());
    std::vector<TokenLogprob> lp;
    sample1(bs, g, x, {}, nullptr, &lp, 20);
    EXPECT(lp[0].top.size() == 20, "%zu alternatives", lp[0].top.size());
    for (size_t j = 0; j < 20; j++) {
        const uint32_t id = lp[0].top[j].first;
        EXPECT(x[id] == sorted[j], "rank %zu: id %u value %.1f, sorted %.1f", j, id, x[id], sorted[j]);
    }
}

void logprobs_are_log_softmax(BatchSampler& bs) {
    // logprobs(&[1.0, 2.0, 3.0], 1, 2) (sampler.rs:379-384): token 1 is made
    // the pick by a mask that allows only it
    const std::vector<float> logits = {1.0f, 2.0f, 3.0f};
    const std::vector<bool> only1 = {false, true, false};
    Sampler g(SamplerConfig::greedy());
    std::vector<TokenLogprob> lp;
    EXPECT(sample1(bs, g, logits, {}, &only1, &lp, 2) == 1, "pick");
    const float z = std::log(std::exp(1.0f) + std::exp(2.0f) + std::exp(3.0f));
    EXPECT(std::fabs(lp[0].logprob - (2.0f - z)) < 1e-5f, "logprob %.9g vs %.9g", lp[0].logprob, 2.0f - z);
    EXPECT(lp[0].top.size() == 2 && lp[0].top[0].first == 2 && lp[0].top[1].first == 1, "top ids");
}

void penalty_can_flip_the_choice(BatchSampler& bs) {
    SamplerConfig c = SamplerConfig::greedy();
    c.repetition_penalty = 2.0f;
    Sampler s(c);
    EXPECT(sample1(bs, s, {0.0f, 3.0f, 2.0f}, {1}) == 2, "penalized pick");
}

// Several sequences over many steps, batched: every step's tokens and every
// sequence's RNG state equal the oracle's per-sequence Sampler.
void sequences_match_the_oracle(BatchSampler& bs) {
    const uint32_t rows = 13, vocab = 3000;
    std::mt19937 g(11);
    std::vector<SamplerConfig> cs;
    for (uint32_t r = 0; r < rows; r++) {
        SamplerConfig c = cfg(0.8f, 40, 0.9f, 1.1f, 1000 + r);
        if (r % 6 == 0) c = SamplerConfig::greedy();              // sample(): no draw
        if (r % 6 == 1) c.temperature = 0.0f;                     // greedy with penalty: one draw
        if (r % 6 == 2) c.top_k = 500, c.top_p = 0.98f;           // a wide window
        if (r % 6 == 3) c.min_p = 0.05f, c.presence_penalty = 0.3f;
        if (r == 12) c = SamplerConfig::greedy();                 // constrained below: sample_with() draws
        cs.push_back(c);
    }
    std::vector<Sampler> ss;
    std::vector<or_sampler*> os;
    for (const auto& c : cs) {
        ss.emplace_back(c);
        or_config oc = ocfg(c);
        os.push_back(or_sampler_new(&oc));
    }
    std::vector<std::vector<uint32_t>> recent(rows);
    const uint32_t words = (vocab + 31) / 32;
    for (int step = 0; step < 25; step++) {
        std::vector<float> logits(static_cast<size_t>(rows) * vocab);
        std::normal_distribution<float> nd(0.0f, 3.0f);
        for (auto& v : logits) v = nd(g);
        std::vector<uint32_t> mask(static_cast<size_t>(rows) * words, 0u);
        std::vector<RowRequest> req(rows);
        for (uint32_t r = 0; r < rows; r++) {
            req[r].sampler = &ss[r];
            req[r].recent = recent[r].data();
            req[r].n_recent = recent[r].size();
            req[r].constrained = (r % 4 == 3) || r == 12;
            if (req[r].constrained) {
                // a third of the rows' masks allow nothing at some steps: no draw
                const bool none = (r % 3 == 0) && (step % 5 == 4);
                for (uint32_t i = 0; i < vocab; i++)
                    if (!none && g() % 10 < 3) mask[r * words + i / 32] |= 1u << (i % 32);
            }
        }
        float* dl = to_device(logits);
        uint32_t* dm = to_device(mask);
        const auto tok = bs.sample(dl, rows, vocab, vocab, req, dm, words);
        (void)hipFree(dl);
        (void)hipFree(dm);
        for (uint32_t r = 0; r < rows; r++) {
            const float* x = logits.data() + static_cast<size_t>(r) * vocab;
            const uint32_t want = req[r].constrained
                                      ? or_sample_with(os[r], x, vocab, vocab, recent[r].data(), recent[r].size(),
                                                       mask.data() + static_cast<size_t>(r) * words)
                                      : or_sample(os[r], x, vocab, vocab, recent[r].data(), recent[r].size());
            EXPECT(tok[r] == want, "step %d row %u: token %u, oracle %u", step, r, tok[r], want);
            EXPECT(ss[r].rng_state() == or_sampler_state(os[r]), "step %d row %u: RNG state differs", step, r);
            recent[r].push_back(tok[r]);
            if (recent[r].size() > 64) recent[r].erase(recent[r].begin());  // the last 64 (scheduler.rs:653)
        }
    }
    for (auto* o : os) or_sampler_free(o);
}

void errors_are_reported(BatchSampler& bs) {
    Sampler s(SamplerConfig::greedy());
    RowRequest q;
    q.sampler = &s;
    q.want_logprobs = true;
    q.logprobs = 21;
    float* d = to_device(std::vector<float>{1.0f, 2.0f});
    bool threw = false;
    try {
        bs.sample(d, 1, 2, 2, {q});
    } catch (const Error&) {
        threw = true;
    }
    (void)hipFree(d);
    EXPECT(threw, "21 logprobs accepted");
    threw = false;
    try {
        BatchSampler too_big(0, 1, TSM_MAX_VOCAB + 1u);
    } catch (const Error&) {
        threw = true;
    }
    EXPECT(threw, "a vocabulary above TSM_MAX_VOCAB accepted");
}

}  // namespace

// ---- JsonObject constraint (constrain.rs) ------------------------------------

static std::vector<uint8_t> bytes_of(const std::string& t) { return std::vector<uint8_t>(t.begin(), t.end()); }

static std::pair<bool, bool> json_check(const std::string& t) {
    JsonObjectConstraint c;
    const auto b = bytes_of(t);
    const bool ok = c.accepts(b.data(), b.size());
    c.advance(b.data(), b.size());
    return {ok, c.is_complete()};
}

// The reference's constraint tests (constrain.rs:313-362) on the C++ API.
static void json_reference_tests() {
    for (const char* t : {"{}", "{\"a\": 1}",
                          "{\"name\": \"Ada\", \"age\": 36, \"langs\": [\"en\", \"fr\"], \"ok\": true, \"x\": null}",
                          "{\"n\": -0.5e+10, \"z\": 0, \"e\": \"\xc3\xa9\\n\\\"q\\\"\"}",
                          "{\n  \"nested\": {\"deep\": [[1, 2], {\"k\": false}]}\n}"}) {
        const auto r = json_check(t);
        EXPECT(r.first && r.second, "valid: %s", t);
    }
    for (const char* t : {"{\"a\": \"unfinished", "{\"a\": [1, 2", "{\"a\": tr", "{\"a\": 12"}) {
        const auto r = json_check(t);
        EXPECT(r.first && !r.second, "prefix: %s", t);
    }
    for (const char* t : {"[1]", "\"top\"", "{a: 1}", "{\"a\" 1}", "{\"a\": 01}", "{\"a\": 1,}", "{\"a\": tru}",
                          "{\"a\": \"\\x\"}", "{\"a\": [1}", "{\"a\": 1}}", "{\"a\": \"line\nbreak\"}",
                          "{\"a\": .5}"}) {
        EXPECT(!json_check(t).first, "invalid accepted: %s", t);
    }
    EXPECT(!json_check("{" + std::string(40, ' ')).first, "whitespace is bounded");
}

// Constrained generation through the batched path: each step the masks of
// four JSON-object sequences come from the GPU producer and must equal the
// host automaton's allows() bit for bit; every pick is allowed, is the
// oracle's sample_with() under the same mask, and advances its constraint.
static void json_constrained_generation(BatchSampler& bs) {
    Vocab v;
    for (int b = 0; b < 256; b++) v.tokens.push_back({static_cast<uint8_t>(b)});
    for (const char* t : {"{", "}", "{\"", "\":", "\": ", "\", \"", "\"}", "[", "]", "true", "false", "null",
                          "12", "-0.5", "e+3", " ", "\n  ", "\"name", "\"a\"", ": [", "],", "\\n", "\\u00e9", "ab"})
        v.tokens.push_back(bytes_of(t));
    v.tokens.push_back({});               // an empty token: never allowed
    v.tokens.push_back(bytes_of("<|x|>")); // a special token: never allowed
    v.special.assign(v.tokens.size(), false);
    v.special.back() = true;
    const uint32_t V = static_cast<uint32_t>(v.tokens.size()), words = (V + 31) / 32, rows = 4;
    DeviceVocab dv(0, v, rows);
    std::vector<JsonObjectConstraint> cs(rows);
    std::vector<Sampler> ss;
    std::vector<or_sampler*> os;
    for (uint32_t r = 0; r < rows; r++) {
        SamplerConfig c = cfg(1.0f, r % 2 ? 0 : 8, 0.95f, 1.0f, 77 + r);
        ss.emplace_back(c);
        or_config oc = ocfg(c);
        os.push_back(or_sampler_new(&oc));
    }
    uint32_t* dmask = nullptr;
    EXPECT(hipMalloc(&dmask, rows * words * 4) == hipSuccess, "hipMalloc");
    std::mt19937 g(5);
    std::normal_distribution<float> nd(0.0f, 2.0f);
    int done = 0;
    for (int step = 0; step < 40; step++) {
        std::vector<const JsonObjectConstraint*> cp;
        for (auto& c : cs) cp.push_back(&c);
        dv.json_masks(cp, V, dmask, words);
        std::vector<uint32_t> mask(rows * words);
        EXPECT(hipMemcpy(mask.data(), dmask, mask.size() * 4, hipMemcpyDeviceToHost) == hipSuccess, "copy");
        for (uint32_t r = 0; r < rows; r++)
            for (uint32_t t = 0; t < V; t++)
                EXPECT(((mask[r * words + t / 32] >> (t % 32)) & 1u) == (cs[r].allows(v, t) ? 1u : 0u),
                       "step %d row %u token %u: mask bit differs from allows()", step, r, t);
        std::vector<float> logits(static_cast<size_t>(rows) * V);
        for (auto& x : logits) x = nd(g);
        std::vector<RowRequest> req(rows);
        for (uint32_t r = 0; r < rows; r++) {
            req[r].sampler = &ss[r];
            req[r].constrained = true;
        }
        float* dl = to_device(logits);
        const auto tok = bs.sample(dl, rows, V, V, req, dmask, words);
        (void)hipFree(dl);
        for (uint32_t r = 0; r < rows; r++) {
            const uint32_t want = or_sample_with(os[r], logits.data() + static_cast<size_t>(r) * V, V, V, nullptr, 0,
                                                 mask.data() + r * words);
            EXPECT(tok[r] == want, "step %d row %u: token %u, oracle %u", step, r, tok[r], want);
            if (cs[r].is_complete()) continue;  // the object closed: nothing is allowed any more
            EXPECT(cs[r].allows(v, tok[r]), "step %d row %u: token %u not allowed", step, r, tok[r]);
            cs[r].advance(v.tokens[tok[r]].data(), v.tokens[tok[r]].size());
            if (cs[r].is_complete()) done++;
        }
    }
    (void)hipFree(dmask);
    for (auto* o : os) or_sampler_free(o);
    std::printf("  %d of %u sequences closed their object\n", done, rows);
}

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    run("rng_matches_the_oracle", rng_matches_the_oracle);
    run("draw_matches_the_oracle", draw_matches_the_oracle);
    run("greedy_settings", greedy_settings);
    run("speculative_sampling_preserves_the_target_distribution",
        speculative_sampling_preserves_the_target_distribution);
    run("deterministic_drafts_reduce_to_greedy", deterministic_drafts_reduce_to_greedy);
    run("json_reference_tests", json_reference_tests);
    if (!cpu_only) {
        BatchSampler bs(0, 16, 8192, 128);
        run("greedy_and_top_k", [&] { greedy_and_top_k(bs); });
        run("constraint_and_distribution", [&] { constraint_and_distribution(bs); });
        run("top_n_matches_a_full_sort", [&] { top_n_matches_a_full_sort(bs); });
        run("logprobs_are_log_softmax", [&] { logprobs_are_log_softmax(bs); });
        run("penalty_can_flip_the_choice", [&] { penalty_can_flip_the_choice(bs); });
        run("sequences_match_the_oracle", [&] { sequences_match_the_oracle(bs); });
        run("errors_are_reported", [&] { errors_are_reported(bs); });
        run("json_constrained_generation", [&] { json_constrained_generation(bs); });
    }
    std::printf("%s: %d failed\n", g_failed ? "FAILED" : "OK", g_failed);
    return g_failed ? 1 : 0;
}
