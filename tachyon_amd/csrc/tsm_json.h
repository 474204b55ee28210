// tsm_json.h - the JSON-object constraint's byte automaton on a packed
// 12-byte state, for the host and the device alike.
//
// Tachyon's JsonObject (src/constrain.rs:88-302) is a byte-level pushdown
// automaton for one JSON object (RFC 8259): a state, a stack of open
// containers (at most 32 deep) and a count of consecutive whitespace bytes
// (at most 16).  A token is allowed when its bytes all step a copy of the
// automaton successfully (accepts_bytes, constrain.rs:280-283), it is not a
// special token and it has bytes (constrain.rs:286-290).  Here the stack is a
// 32-bit word (bit i: level i is an object), so a row's whole state fits in
// tsm_json_state and every token of the vocabulary can be probed by its own
// GPU thread from a register copy.
//
// The step below follows constrain.rs:160-277 byte for byte, including what
// Constraint::advance (constrain.rs:292-296) leaves behind after a byte the
// automaton rejects: a number's length still grows past its limit, a string
// escape still resets, and the u8 counters wrap as Rust's release build does.
#pragma once

#include <hip/hip_runtime.h>

#include "tachyon_sampler.h"

namespace tsm {
namespace json {

// tsm_json_state.state
enum : uint8_t {
    JS_VALUE = 0,        // a value must start here (the top level takes only '{')
    JS_ARRAY_START = 1,  // just after '[': a value or ']'
    JS_OBJECT_START = 2, // just after '{': a key or '}'
    JS_KEY = 3,          // after ',' in an object: a key
    JS_COLON = 4,        // after a key: ':'
    JS_AFTER = 5,        // after a value inside a container: ',' or the closing bracket
    JS_STR = 6,          // inside a string; aux = key | escape << 1 | hex << 2
    JS_NUMBER = 7,       // aux = the number's part (N_*), len = its length so far
    JS_LITERAL = 8,      // aux = the word (0 true, 1 false, 2 null), len = bytes matched
    JS_DONE = 9,         // the object is closed
};
// number parts (constrain.rs:44-54)
enum : uint8_t { N_MINUS = 0, N_ZERO, N_INT, N_DOT, N_FRAC, N_EXP, N_EXPSIGN, N_EXPDIGITS };

constexpr uint8_t kMaxWhitespace = 16;  // constrain.rs:84
constexpr uint8_t kMaxNumber = 40;      // constrain.rs:85
constexpr uint8_t kMaxDepth = 32;       // constrain.rs:86

__host__ __device__ inline void init(tsm_json_state* s) {
    s->stack = 0;
    s->depth = 0;
    s->state = JS_VALUE;
    s->aux = 0;
    s->len = 0;
    s->whitespace = 0;
    s->pad[0] = s->pad[1] = s->pad[2] = 0;
}

__host__ __device__ inline bool is_digit(uint8_t b) { return b >= '0' && b <= '9'; }
__host__ __device__ inline bool is_hex(uint8_t b) {
    return is_digit(b) || (b >= 'a' && b <= 'f') || (b >= 'A' && b <= 'F');
}
// The top container: 1 object, 0 array (depth in [1, 32]).
__host__ __device__ inline uint32_t top(const tsm_json_state& s) { return (s.stack >> ((s.depth - 1u) & 31u)) & 1u; }

__host__ __device__ inline void value_done(tsm_json_state& s) { s.state = s.depth == 0 ? JS_DONE : JS_AFTER; }

__host__ __device__ inline bool open(tsm_json_state& s, uint32_t object) {
    if (s.depth >= kMaxDepth) return false;
    s.stack = (s.stack & ((1u << s.depth) - 1u)) | (object << s.depth);
    s.depth++;
    s.state = object ? JS_OBJECT_START : JS_ARRAY_START;
    return true;
}

__host__ __device__ inline bool close(tsm_json_state& s, uint32_t object) {
    if (s.depth == 0 || top(s) != object) return false;
    s.depth--;
    value_done(s);
    return true;
}

__host__ __device__ inline bool start_value(tsm_json_state& s, uint8_t b) {
    if (s.depth == 0) return b == '{' && open(s, 1u);
    switch (b) {
        case '{': return open(s, 1u);
        case '[': return open(s, 0u);
        case '"': s.state = JS_STR; s.aux = 0; return true;
        case '-': s.state = JS_NUMBER; s.aux = N_MINUS; s.len = 1; return true;
        case '0': s.state = JS_NUMBER; s.aux = N_ZERO; s.len = 1; return true;
        case 't': s.state = JS_LITERAL; s.aux = 0; s.len = 1; return true;
        case 'f': s.state = JS_LITERAL; s.aux = 1; s.len = 1; return true;
        case 'n': s.state = JS_LITERAL; s.aux = 2; s.len = 1; return true;
        default:
            if (b >= '1' && b <= '9') {
                s.state = JS_NUMBER;
                s.aux = N_INT;
                s.len = 1;
                return true;
            }
            return false;
    }
}

// The next number part after byte b, or 0xFF when b does not continue the
// number (constrain.rs:202-213).
__host__ __device__ inline uint8_t number_next(uint8_t n, uint8_t b) {
    const bool d = is_digit(b);
    switch (n) {
        case N_MINUS: return b == '0' ? N_ZERO : (d ? N_INT : 0xFF);
        case N_ZERO: return b == '.' ? N_DOT : (b == 'e' || b == 'E') ? N_EXP : 0xFF;
        case N_INT: return b == '.' ? N_DOT : d ? N_INT : (b == 'e' || b == 'E') ? N_EXP : 0xFF;
        case N_DOT: return d ? N_FRAC : 0xFF;
        case N_FRAC: return d ? N_FRAC : (b == 'e' || b == 'E') ? N_EXP : 0xFF;
        case N_EXP: return (b == '+' || b == '-') ? N_EXPSIGN : d ? N_EXPDIGITS : 0xFF;
        case N_EXPSIGN: return d ? N_EXPDIGITS : 0xFF;
        default: return d ? N_EXPDIGITS : 0xFF;  // N_EXPDIGITS
    }
}

// Feeds one byte; false if it cannot appear here (JsonObject::step).
__host__ __device__ inline bool step(tsm_json_state& s, uint8_t b) {
    const bool ws = b == ' ' || b == '\t' || b == '\n' || b == '\r';
    if (s.state == JS_STR) {
        const uint8_t key = s.aux & 1u, esc = (s.aux >> 1) & 1u, hex = s.aux >> 2;
        if (hex > 0) {
            s.aux = static_cast<uint8_t>(key | ((hex - 1u) << 2));
            return is_hex(b);
        }
        if (esc) {
            s.aux = static_cast<uint8_t>(key | ((b == 'u' ? 4u : 0u) << 2));
            return b == '"' || b == '\\' || b == '/' || b == 'b' || b == 'f' || b == 'n' || b == 'r' || b == 't' ||
                   b == 'u';
        }
        if (b == '"') {
            if (key) s.state = JS_COLON;
            else value_done(s);
            return true;
        }
        if (b == '\\') {
            s.aux = static_cast<uint8_t>(key | 2u);
            return true;
        }
        return b >= 0x20;
    }
    if (s.state == JS_NUMBER) {
        const uint8_t next = number_next(s.aux, b);
        if (next != 0xFF) {
            const uint8_t len = s.len;
            s.aux = next;
            s.len = static_cast<uint8_t>(len + 1u);
            return len < kMaxNumber;
        }
        // the number ends here if it can; the byte then belongs to what follows
        if (!(s.aux == N_ZERO || s.aux == N_INT || s.aux == N_FRAC || s.aux == N_EXPDIGITS)) return false;
        value_done(s);
    } else if (s.state == JS_LITERAL) {
        const char* word = s.aux == 0 ? "true" : s.aux == 1 ? "false" : "null";
        const uint8_t wlen = s.aux == 1 ? 5 : 4;
        if (s.len >= wlen) return false;  // not a state step() makes: the word's end is not read past
        if (static_cast<uint8_t>(word[s.len]) != b) return false;
        if (s.len + 1u == wlen) value_done(s);
        else s.len++;
        return true;
    }
    if (ws) {
        s.whitespace = static_cast<uint8_t>(s.whitespace + 1u);
        return s.whitespace <= kMaxWhitespace && s.state != JS_DONE;
    }
    s.whitespace = 0;
    switch (s.state) {
        case JS_VALUE: return start_value(s, b);
        case JS_ARRAY_START: return b == ']' ? close(s, 0u) : start_value(s, b);
        case JS_OBJECT_START:
            if (b == '}') return close(s, 1u);
            if (b == '"') {
                s.state = JS_STR;
                s.aux = 1;  // a key
                return true;
            }
            return false;
        case JS_KEY:
            if (b == '"') {
                s.state = JS_STR;
                s.aux = 1;
                return true;
            }
            return false;
        case JS_COLON:
            if (b == ':') {
                s.state = JS_VALUE;
                return true;
            }
            return false;
        case JS_AFTER:
            if (s.depth == 0) return false;  // not reached from init(): a value inside nothing is DONE
            if (b == ',') {
                s.state = top(s) ? JS_KEY : JS_VALUE;
                return true;
            }
            if (b == '}') return close(s, 1u);
            if (b == ']') return close(s, 0u);
            return false;
        default: return false;
    }
}

// Whether these bytes may come next (JsonObject::accepts_bytes): a copy steps
// until the first byte it rejects.  Inside a string with no escape pending, a
// byte other than '"', '\\' and the control bytes only passes (step's last
// case), which is taken without the full step: a GPU wave walks its tokens in
// lockstep, and most of a string's bytes are such bytes.
__host__ __device__ inline bool accepts(tsm_json_state s, const uint8_t* bytes, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        const uint8_t b = bytes[i];
        if (s.state == JS_STR && s.aux <= 1u && b >= 0x20 && b != '"' && b != '\\') continue;
        if (!step(s, b)) return false;
    }
    return true;
}

}  // namespace json
}  // namespace tsm
