// tsm_mask.hip - the mask producer: JsonObject's allows() for every token of
// the vocabulary, on the GPU, written as the packed allow-bits that
// sample_kernel and split_kernel consume (tsm_batch.mask).
//
// One thread per token and a group of rows: the workgroup stages its 256
// tokens' bytes in LDS, then per row each thread copies the row's 12-byte
// automaton state into registers and steps it through its token's bytes until
// the first rejected byte (tsm_json.h).  A wave's 64 answers become two mask
// words by one ballot, so every word of a row's mask is written exactly once,
// coalesced, with no atomics.  Most tokens are rejected at their first byte
// outside strings (only a few bytes can follow a value, a key or a colon), so
// the work is about one load of the token's offsets and a few bytes per
// token; inside a string most tokens are walked to their end.
#include <cstdarg>
#include <cstdio>

#include "tsm_device.h"
#include "tsm_json.h"

namespace tsm {
namespace mask {

constexpr int kMB = 256;             // threads per workgroup: 256 consecutive tokens
constexpr uint32_t kRowsPer = 32;    // rows per workgroup: the staged bytes serve each
constexpr uint32_t kStage = 16384;   // LDS bytes for the workgroup's tokens

struct JsonMaskArgs {
    const uint8_t* bytes;
    const uint32_t* offsets;
    const uint32_t* special;
    const tsm_json_state* states;
    uint32_t* mask;
    uint32_t n_tokens, usable, mask_stride, nwords, rows;
};

// Workgroup (token block, row group): the block's token bytes are one
// contiguous range of the vocabulary's bytes, staged into LDS with coalesced
// loads once and then stepped through for each of the group's rows (a block
// whose bytes exceed the stage reads them from global memory instead).
__global__ __launch_bounds__(kMB) void json_mask_kernel(JsonMaskArgs a) {
    __shared__ uint8_t stage[kStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t t0 = blockIdx.x * kMB;
    const uint32_t id = t0 + tid;
    const uint32_t lim = a.usable < a.n_tokens ? a.usable : a.n_tokens;  // ids with bytes that count
    const uint32_t tend = t0 + kMB < lim ? t0 + kMB : lim;
    bool has = false;
    uint32_t b0 = 0, b1 = 0;
    if (id < lim) {
        b0 = a.offsets[id];
        b1 = a.offsets[id + 1u];
        const bool special = a.special != nullptr && ((a.special[id >> 5] >> (id & 31u)) & 1u);
        has = !special && b1 > b0;
    }
    uint32_t lo = 0, hi = 0;
    if (t0 < tend) {
        lo = a.offsets[t0];
        hi = a.offsets[tend];
    }
    const bool staged = hi >= lo && hi - lo <= kStage;
    if (staged) {
        for (uint32_t k = tid; k < hi - lo; k += kMB) stage[k] = a.bytes[lo + k];
        __syncthreads();
    }
    // a token's bytes lie inside [lo, hi) when the offsets are ordered; a
    // token outside it is read from global memory
    const bool mine_staged = staged && b0 >= lo && b1 <= hi;
    const uint8_t* src = mine_staged ? stage + (b0 - lo) : a.bytes + b0;
    const uint32_t len = b1 - b0;
    // a token of string text only (no '"', no '\\', no control byte) is
    // accepted whole inside a string with no escape pending: found once here
    // for all the group's rows
    bool plain = has;
    for (uint32_t k = 0; plain && k < len; k++) {
        const uint8_t c = src[k];
        plain = c >= 0x20 && c != '"' && c != '\\';
    }
    const uint32_t lane = lane_id();
    const uint32_t w = (t0 + (tid & ~(kWave - 1u))) / 32u + lane;  // lanes 0, 1: the wave's words
    const uint32_t r0 = blockIdx.y * kRowsPer;
    for (uint32_t r = r0; r < r0 + kRowsPer && r < a.rows; r++) {
        const tsm_json_state st = a.states[r];
        const bool in_text = st.state == json::JS_STR && st.aux <= 1u;
        const bool ok = has && ((in_text && plain) || json::accepts(st, src, len));
        const uint64_t b = wave_ballot(ok);
        if (lane < 2u && w < a.nwords)
            a.mask[static_cast<size_t>(r) * a.mask_stride + w] = static_cast<uint32_t>(lane ? (b >> 32) : b);
    }
}

void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

}  // namespace mask
}  // namespace tsm

extern "C" {

void tsm_json_init(tsm_json_state* s) {
    if (s) tsm::json::init(s);
}

void tsm_json_advance(tsm_json_state* s, const uint8_t* bytes, size_t n) {
    if (!s || (!bytes && n)) return;
    for (size_t i = 0; i < n; i++) (void)tsm::json::step(*s, bytes[i]);  // advance ignores rejections
}

int tsm_json_accepts(const tsm_json_state* s, const uint8_t* bytes, size_t n) {
    if (!s || (!bytes && n)) return 0;
    tsm_json_state c = *s;
    for (size_t i = 0; i < n; i++)
        if (!tsm::json::step(c, bytes[i])) return 0;
    return 1;
}

int tsm_json_is_complete(const tsm_json_state* s) { return s && s->state == tsm::json::JS_DONE ? 1 : 0; }

int tsm_json_mask(void* stream, const tsm_vocab* vocab, const tsm_json_state* states, uint32_t rows,
                  uint32_t usable, uint32_t* mask, uint32_t mask_stride, char* err, size_t errlen) {
    using tsm::mask::set_err;
    if (!vocab) return set_err(err, errlen, "vocab is NULL"), 1;
    if (vocab->reserved != 0) return set_err(err, errlen, "vocab->reserved must be 0"), 1;
    if (vocab->n_tokens > 0 && (!vocab->bytes || !vocab->offsets))
        return set_err(err, errlen, "vocab->bytes and vocab->offsets must be set when n_tokens > 0"), 1;
    if (!states) return set_err(err, errlen, "states is NULL"), 1;
    if (!mask) return set_err(err, errlen, "mask is NULL"), 1;
    if (rows == 0 || rows > 65535u) return set_err(err, errlen, "rows %u is outside [1, 65535]", rows), 1;
    if (usable == 0 || usable > TSM_MAX_VOCAB)
        return set_err(err, errlen, "usable %u is outside [1, %u]", usable, TSM_MAX_VOCAB), 1;
    const uint32_t nwords = (usable + 31u) / 32u;
    if (mask_stride < nwords)
        return set_err(err, errlen, "mask_stride %u is below ceil(usable / 32) = %u", mask_stride, nwords), 1;
    tsm::mask::JsonMaskArgs a;
    a.bytes = vocab->bytes;
    a.offsets = vocab->offsets;
    a.special = vocab->special;
    a.states = states;
    a.mask = mask;
    a.n_tokens = vocab->n_tokens;
    a.usable = usable;
    a.mask_stride = mask_stride;
    a.nwords = nwords;
    a.rows = rows;
    const dim3 grid((usable + tsm::mask::kMB - 1) / tsm::mask::kMB,
                    (rows + tsm::mask::kRowsPer - 1) / tsm::mask::kRowsPer);
    hipLaunchKernelGGL(tsm::mask::json_mask_kernel, grid, dim3(tsm::mask::kMB), 0,
                       static_cast<hipStream_t>(stream), a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

}  // extern "C"
