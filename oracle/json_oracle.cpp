// json_oracle.cpp - CPU restatement of Tachyon's JsonObject constraint, TEST
// INFRASTRUCTURE ONLY.
//
// The parity checker of the mask producer (tsm_json_mask): tests/ load it
// through ctypes, inside libtachyon_oracle.so.  The product library never
// links, loads or calls it.
//
// It restates /root/reference/src/constrain.rs:42-302 in the reference's own
// shape: an enum state with its fields, a growable stack of booleans, the
// match arms in their order.  (The product's automaton, tachyon_amd/csrc/
// tsm_json.h, packs the same state into 12 bytes for the GPU; the two are
// written separately.)
//
// Pinning (tests/test_oracle.py): the reference's own tests
// (constrain.rs:304-362: valid objects, prefixes that are not complete,
// invalid JSON, bounded whitespace), plus hand-derived cases for the
// number limit, escapes and the depth limit.
#include <cstdint>
#include <cstring>
#include <vector>

namespace {

enum class Num { Minus, Zero, Int, Dot, Frac, Exp, ExpSign, ExpDigits };
enum class Kind { Value, ArrayStart, ObjectStart, Key, Colon, After, Str, Number, Literal, Done };

const char* const kTrue = "true";
const char* const kFalse = "false";
const char* const kNull = "null";

struct State {
    Kind kind = Kind::Value;
    bool key = false, escape = false;  // Str
    uint8_t hex = 0;                   // Str
    Num num = Num::Minus;              // Number
    uint8_t len = 0;                   // Number
    const char* word = nullptr;        // Literal
    uint8_t at = 0;                    // Literal
};

// JsonObject (constrain.rs:88-93)
struct Json {
    std::vector<bool> stack;  // true = object, false = array
    State state;
    uint8_t whitespace = 0;

    void value_done() {  // constrain.rs:106-112
        state = State();
        state.kind = stack.empty() ? Kind::Done : Kind::After;
    }
    bool open(bool object) {  // constrain.rs:114-124
        if (stack.size() >= 32) return false;
        stack.push_back(object);
        state = State();
        state.kind = object ? Kind::ObjectStart : Kind::ArrayStart;
        return true;
    }
    bool close(bool object) {  // constrain.rs:126-133
        if (stack.empty() || stack.back() != object) return false;
        stack.pop_back();
        value_done();
        return true;
    }
    bool start_value(uint8_t b) {  // constrain.rs:135-157
        if (stack.empty()) return b == '{' && open(true);
        State s;
        switch (b) {
            case '{': return open(true);
            case '[': return open(false);
            case '"': s.kind = Kind::Str; break;
            case '-': s.kind = Kind::Number; s.num = Num::Minus; s.len = 1; break;
            case '0': s.kind = Kind::Number; s.num = Num::Zero; s.len = 1; break;
            case 't': s.kind = Kind::Literal; s.word = kTrue; s.at = 1; break;
            case 'f': s.kind = Kind::Literal; s.word = kFalse; s.at = 1; break;
            case 'n': s.kind = Kind::Literal; s.word = kNull; s.at = 1; break;
            default:
                if (b >= '1' && b <= '9') {
                    s.kind = Kind::Number;
                    s.num = Num::Int;
                    s.len = 1;
                    break;
                }
                return false;
        }
        state = s;
        return true;
    }
    static bool hexdigit(uint8_t b) {
        return (b >= '0' && b <= '9') || (b >= 'a' && b <= 'f') || (b >= 'A' && b <= 'F');
    }
    bool step(uint8_t b) {  // constrain.rs:160-277
        const bool ws = b == ' ' || b == '\t' || b == '\n' || b == '\r';
        switch (state.kind) {
            case Kind::Str: {
                const bool key = state.key;
                if (state.hex > 0) {
                    const bool ok = hexdigit(b);
                    state.escape = false;
                    state.hex = static_cast<uint8_t>(state.hex - 1);
                    (void)key;
                    return ok;
                }
                if (state.escape) {
                    state.escape = false;
                    state.hex = b == 'u' ? 4 : 0;
                    return b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' || b == 'r' ||
                           b == 't' || b == 'u';
                }
                if (b == '"') {
                    if (key) {
                        state = State();
                        state.kind = Kind::Colon;
                    } else {
                        value_done();
                    }
                    return true;
                }
                if (b == '\\') {
                    state.escape = true;
                    state.hex = 0;
                    return true;
                }
                return b >= 0x20;
            }
            case Kind::Number: {
                const bool digit = b >= '0' && b <= '9';
                const Num n = state.num;
                bool has = true;
                Num next = n;
                if (n == Num::Minus && b == '0') next = Num::Zero;
                else if (n == Num::Minus && digit) next = Num::Int;
                else if ((n == Num::Zero || n == Num::Int) && b == '.') next = Num::Dot;
                else if (n == Num::Int && digit) next = Num::Int;
                else if ((n == Num::Dot || n == Num::Frac) && digit) next = Num::Frac;
                else if ((n == Num::Zero || n == Num::Int || n == Num::Frac) && (b == 'e' || b == 'E')) next = Num::Exp;
                else if (n == Num::Exp && (b == '+' || b == '-')) next = Num::ExpSign;
                else if ((n == Num::Exp || n == Num::ExpSign || n == Num::ExpDigits) && digit) next = Num::ExpDigits;
                else has = false;
                if (has) {
                    const uint8_t len = state.len;
                    state.num = next;
                    state.len = static_cast<uint8_t>(len + 1);  // u8 arithmetic of a release build
                    return len < 40;
                }
                if (!(n == Num::Zero || n == Num::Int || n == Num::Frac || n == Num::ExpDigits)) return false;
                value_done();
                break;
            }
            case Kind::Literal: {
                if (static_cast<uint8_t>(state.word[state.at]) != b) return false;
                if (static_cast<size_t>(state.at) + 1 == std::strlen(state.word)) value_done();
                else state.at++;
                return true;
            }
            default: break;
        }
        if (ws) {
            whitespace = static_cast<uint8_t>(whitespace + 1);
            return whitespace <= 16 && state.kind != Kind::Done;
        }
        whitespace = 0;
        switch (state.kind) {
            case Kind::Value: return start_value(b);
            case Kind::ArrayStart: return b == ']' ? close(false) : start_value(b);
            case Kind::ObjectStart:
                if (b == '}') return close(true);
                [[fallthrough]];
            case Kind::Key:
                if (b == '"') {
                    state = State();
                    state.kind = Kind::Str;
                    state.key = true;
                    return true;
                }
                return false;
            case Kind::Colon:
                if (b == ':') {
                    state = State();
                    state.kind = Kind::Value;
                    return true;
                }
                return false;
            case Kind::After:
                if (b == ',' && !stack.empty() && stack.back()) {
                    state = State();
                    state.kind = Kind::Key;
                    return true;
                }
                if (b == ',' && !stack.empty() && !stack.back()) {
                    state = State();
                    state.kind = Kind::Value;
                    return true;
                }
                if (b == '}') return close(true);
                if (b == ']') return close(false);
                return false;
            default: return false;
        }
    }
    bool accepts_bytes(const uint8_t* p, size_t n) const {  // constrain.rs:280-283
        Json probe = *this;
        for (size_t i = 0; i < n; i++)
            if (!probe.step(p[i])) return false;
        return true;
    }
};

}  // namespace

extern "C" {

void* or_json_new() { return new Json(); }
void or_json_free(void* j) { delete static_cast<Json*>(j); }
void* or_json_clone(const void* j) { return new Json(*static_cast<const Json*>(j)); }
// Constraint::advance (constrain.rs:292-296)
void or_json_advance(void* j, const uint8_t* bytes, size_t n) {
    Json* s = static_cast<Json*>(j);
    for (size_t i = 0; i < n; i++) (void)s->step(bytes[i]);
}
int or_json_accepts(const void* j, const uint8_t* bytes, size_t n) {
    return static_cast<const Json*>(j)->accepts_bytes(bytes, n) ? 1 : 0;
}
int or_json_is_complete(const void* j) { return static_cast<const Json*>(j)->state.kind == Kind::Done ? 1 : 0; }
// The constrain.rs tests' check(): (accepts_bytes, is_complete after advance)
void or_json_check(const uint8_t* text, size_t n, int* ok, int* complete) {
    Json j;
    *ok = j.accepts_bytes(text, n) ? 1 : 0;
    for (size_t i = 0; i < n; i++) (void)j.step(text[i]);
    *complete = j.state.kind == Kind::Done ? 1 : 0;
}
// allows() (constrain.rs:286-290) for ids [0, usable) as packed LSB-first
// words: ids at or above n_tokens have no bytes; special[] may be NULL.
void or_json_mask(const void* j, const uint8_t* bytes, const uint32_t* offsets, const uint32_t* special,
                  uint32_t n_tokens, uint32_t usable, uint32_t* words) {
    const Json* s = static_cast<const Json*>(j);
    for (uint32_t w = 0; w < (usable + 31) / 32; w++) words[w] = 0;
    for (uint32_t id = 0; id < usable && id < n_tokens; id++) {
        if (special && ((special[id >> 5] >> (id & 31)) & 1u)) continue;
        const uint32_t b0 = offsets[id], b1 = offsets[id + 1];
        if (b1 <= b0) continue;
        if (s->accepts_bytes(bytes + b0, b1 - b0)) words[id >> 5] |= 1u << (id & 31);
    }
}

}  // extern "C"
