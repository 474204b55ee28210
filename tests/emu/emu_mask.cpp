// The mask producer's sources on the CPU emulation (test infrastructure):
// tsm_json_masks_fill (a mask set: distinct states once, recent states kept,
// rows filled by copies) against tsm_json_mask on the same states, and both
// against the host stepping of tsm_json_accepts, over calls that hit, miss
// and overflow the kept masks, a set keeping nothing and a new vocabulary.
// Prints "ok" and exits 0 when every word and count agrees.
#include "../../tachyon_amd/csrc/tsm_mask.hip"

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

static int fails = 0;
#define CHECK(c, ...)                          \
    do {                                       \
        if (!(c)) {                            \
            std::fprintf(stderr, __VA_ARGS__); \
            std::fprintf(stderr, "\n");        \
            fails++;                           \
        }                                      \
    } while (0)

struct Vocab {
    std::vector<uint8_t> bytes;
    std::vector<uint32_t> offsets, special;
    uint32_t n = 0;
};

static Vocab make_vocab() {
    std::vector<std::string> toks;
    for (int b = 0; b < 256; b++) toks.push_back(std::string(1, static_cast<char>(b)));
    const char* frags[] = {"{", "}", "[", "]", "\"", ":", ",", " ", "\n", "{\"", "\":", "\",", "\"}", "true", "false",
                           "null", "tru", "nul", "1", "12", "-3", "0.5", "1e9", "abc", "hello world", "\\n", "\\u00",
                           "\xc3\xa9", "\":\"", "\"a\"", "}]", "],", " {", "  ", "x\"", "\\\"", "1,", "2}", "", "ab\"c"};
    for (const char* f : frags) toks.push_back(f);
    Vocab v;
    v.n = static_cast<uint32_t>(toks.size());
    v.offsets.push_back(0);
    for (const auto& t : toks) {
        v.bytes.insert(v.bytes.end(), t.begin(), t.end());
        v.offsets.push_back(static_cast<uint32_t>(v.bytes.size()));
    }
    v.special.assign((v.n + 31) / 32, 0u);
    v.special[(256 + 5) / 32] |= 1u << ((256 + 5) % 32);  // one special token
    return v;
}

static tsm_json_state state_of(const char* prefix) {
    tsm_json_state s;
    tsm_json_init(&s);
    tsm_json_advance(&s, reinterpret_cast<const uint8_t*>(prefix), std::strlen(prefix));
    return s;
}

static bool same_state(const tsm_json_state& a, const tsm_json_state& b) {
    return a.stack == b.stack && a.depth == b.depth && a.state == b.state && a.aux == b.aux && a.len == b.len &&
           a.whitespace == b.whitespace;
}

static uint32_t distinct(const std::vector<tsm_json_state>& rows) {
    uint32_t d = 0;
    for (size_t i = 0; i < rows.size(); i++) {
        bool seen = false;
        for (size_t j = 0; j < i && !seen; j++) seen = same_state(rows[i], rows[j]);
        d += seen ? 0u : 1u;
    }
    return d;
}

int main() {
    const Vocab v = make_vocab();
    const uint32_t usable = v.n + 3;  // ids past the tokenizer: never allowed
    const uint32_t nw = (usable + 31) / 32, stride = nw + 2;
    tsm_vocab tv{v.bytes.data(), v.offsets.data(), v.special.data(), v.n, 0};
    const std::vector<uint8_t> bytes2 = v.bytes;  // the same vocabulary at other addresses
    const std::vector<uint32_t> offsets2 = v.offsets, special2 = v.special;
    tsm_vocab tv2{bytes2.data(), offsets2.data(), special2.data(), v.n, 0};

    const char* prefixes[] = {"", "{", "{\"a\"", "{\"a\":", "{\"a\": \"x", "[1,", "{\"k\": [true, ", "\"str", "{\"a\":1}",
                              "{\"a\": \"b\", \"c\": 12", "[[[", "{\"x\": nu", "  {", "{\"a\": \"\\u00", "[1e",
                              "{\"q\": \"\xc3", "{\"z\": [1, 2], \"w\""};
    const uint32_t np = sizeof(prefixes) / sizeof(prefixes[0]);
    std::vector<tsm_json_state> pool;
    for (uint32_t i = 0; i < np; i++) pool.push_back(state_of(prefixes[i]));
    char err[256];

    // host reference: allows() token by token
    auto host_mask = [&](const tsm_json_state& s, std::vector<uint32_t>& w) {
        w.assign(nw, 0u);
        for (uint32_t t = 0; t < usable && t < v.n; t++) {
            const bool sp = (v.special[t >> 5] >> (t & 31u)) & 1u;
            const uint32_t b0 = v.offsets[t], b1 = v.offsets[t + 1];
            if (sp || b1 == b0) continue;
            if (tsm_json_accepts(&s, v.bytes.data() + b0, b1 - b0)) w[t >> 5] |= 1u << (t & 31u);
        }
    };
    auto direct = [&](const std::vector<tsm_json_state>& rows, std::vector<uint32_t>& out) {
        out.assign(rows.size() * stride, 0x5A5A5A5Au);
        const int rc = tsm_json_mask(nullptr, &tv, rows.data(), static_cast<uint32_t>(rows.size()), usable, out.data(),
                                     stride, err, sizeof(err));
        CHECK(rc == 0, "tsm_json_mask: %s", err);
    };
    auto check_rows = [&](const char* label, const std::vector<tsm_json_state>& rows, const std::vector<uint32_t>& got) {
        std::vector<uint32_t> ref, hw;
        direct(rows, ref);
        for (size_t r = 0; r < rows.size(); r++) {
            host_mask(rows[r], hw);
            for (uint32_t w = 0; w < nw; w++) {
                CHECK(got[r * stride + w] == ref[r * stride + w], "%s row %zu word %u: set %08x direct %08x", label, r,
                      w, got[r * stride + w], ref[r * stride + w]);
                CHECK(ref[r * stride + w] == hw[w], "%s row %zu word %u: direct %08x host %08x", label, r, w,
                      ref[r * stride + w], hw[w]);
            }
            for (uint32_t w = nw; w < stride; w++)
                CHECK(got[r * stride + w] == 0x5A5A5A5Au, "%s row %zu: word %u past the row written", label, r, w);
        }
    };
    auto fill = [&](tsm_json_masks* m, const tsm_vocab* voc, const std::vector<tsm_json_state>& rows,
                    std::vector<uint32_t>& out, tsm_json_fill_stats& st) {
        out.assign(rows.size() * stride, 0x5A5A5A5Au);
        const int rc = tsm_json_masks_fill(m, nullptr, voc, rows.data(), static_cast<uint32_t>(rows.size()), out.data(),
                                           stride, &st, err, sizeof(err));
        CHECK(rc == 0, "tsm_json_masks_fill: %s", err);
    };

    // call 1: 40 rows over the pool (repeats), a set keeping 4 states
    std::vector<tsm_json_state> rows1;
    for (uint32_t i = 0; i < 40; i++) rows1.push_back(pool[(i * 7 + i / 3) % 10u]);  // 10 of the pool
    rows1[39].pad[0] = 0xAB;  // stray padding: the same state
    tsm_json_masks* m = tsm_json_masks_create(0, 64, 4, usable, err, sizeof(err));
    CHECK(m != nullptr, "create: %s", err);
    std::vector<uint32_t> got;
    tsm_json_fill_stats st;
    fill(m, &tv, rows1, got, st);
    check_rows("call 1", rows1, got);
    const uint32_t d1 = distinct(rows1);
    CHECK(st.rows == 40 && st.distinct == d1 && st.hits == 0 && st.evaluated == d1, "call 1 stats %u %u %u %u (distinct %u)",
          st.rows, st.distinct, st.hits, st.evaluated, d1);
    // call 2: the first two distinct states of call 1 (kept) and three others
    std::vector<tsm_json_state> firsts;
    for (const auto& s : rows1) {
        bool seen = false;
        for (const auto& f : firsts) seen = seen || same_state(f, s);
        if (!seen) firsts.push_back(s);
    }
    std::vector<tsm_json_state> fresh;
    for (const auto& s : pool) {
        bool seen = false;
        for (const auto& f : firsts) seen = seen || same_state(f, s);
        for (const auto& f : fresh) seen = seen || same_state(f, s);
        if (!seen) fresh.push_back(s);
    }
    CHECK(fresh.size() >= 3, "only %zu states outside call 1", fresh.size());
    if (fresh.size() >= 3) {
        std::vector<tsm_json_state> rows2 = {firsts[0], firsts[1], fresh[0], firsts[0], fresh[1], fresh[2], fresh[0]};
        fill(m, &tv, rows2, got, st);
        check_rows("call 2", rows2, got);
        CHECK(st.rows == 7 && st.distinct == 5 && st.hits == 2 && st.evaluated == 3, "call 2 stats %u %u %u %u",
              st.rows, st.distinct, st.hits, st.evaluated);
        // call 3: the same rows, 4 of their 5 states kept
        fill(m, &tv, rows2, got, st);
        check_rows("call 3", rows2, got);
        CHECK(st.distinct == 5 && st.hits == 4 && st.evaluated == 1, "call 3 stats %u %u %u", st.distinct, st.hits,
              st.evaluated);
        // another vocabulary: nothing kept is used
        fill(m, &tv2, rows2, got, st);
        check_rows("call 4", rows2, got);
        CHECK(st.hits == 0 && st.evaluated == 5, "call 4 stats %u %u", st.hits, st.evaluated);
    }
    // bad arguments
    CHECK(tsm_json_masks_fill(m, nullptr, &tv, rows1.data(), 65, got.data(), stride, nullptr, err, sizeof(err)) != 0,
          "rows past max_rows accepted");
    CHECK(tsm_json_masks_fill(m, nullptr, &tv, rows1.data(), 1, got.data(), nw - 1, nullptr, err, sizeof(err)) != 0,
          "a short stride accepted");
    tsm_json_masks_destroy(m);
    // a set keeping nothing: each distinct state of a call evaluated once
    tsm_json_masks* m0 = tsm_json_masks_create(0, 64, 0, usable, err, sizeof(err));
    CHECK(m0 != nullptr, "create (capacity 0): %s", err);
    fill(m0, &tv, rows1, got, st);
    check_rows("capacity 0", rows1, got);
    CHECK(st.distinct == d1 && st.hits == 0 && st.evaluated == d1, "capacity 0 stats %u %u %u", st.distinct, st.hits,
          st.evaluated);
    fill(m0, &tv, rows1, got, st);
    CHECK(st.hits == 0 && st.evaluated == d1, "capacity 0, again: %u %u", st.hits, st.evaluated);
    tsm_json_masks_destroy(m0);
    if (fails) {
        std::fprintf(stderr, "%d checks failed\n", fails);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
