// tsm_split.h - the split-row sampling kernel: records it keeps in the
// context's device scratch, its argument record and its host-side launcher
// (defined in tsm_split.hip).
#pragma once

#include "tsm_sample.h"

namespace tsm {
namespace split {

constexpr int kSB = 256;                         // threads per workgroup (4 waves)
constexpr int kSW = kSB / kWave;                 // waves per workgroup
constexpr int kSlots = 19;                       // float4 slots per thread: a segment lives in registers
constexpr uint32_t kSegQuant = 4u * kSB;         // segment lengths are multiples of 1024 ids
constexpr uint32_t kSegMax = kSlots * kSegQuant; // 19456 ids per segment at most
constexpr uint32_t kSegMin = 4096;               // shortest segment the host picks
constexpr uint32_t kCandCap = 3072;              // candidate entries per segment at most
constexpr uint32_t kSplitHist = 1024;            // longest penalizing history a row may have on this path
constexpr uint32_t kSplitNeed = 1536;            // window + penalizing history at most (candidate area bound)
constexpr uint32_t kMaxSegs = 1023;              // segments per row at most
constexpr uint32_t kSplitRowsMax = 16;           // batches of more rows take the whole-row kernel

// Per (row, segment) summary, written by the segment's workgroup before it
// arrives at the row's counter; read by the row's last workgroup.
struct SegSum {
    float xmax;              // raw maximum over the segment's ids (NaN ignored; -inf when every id is -inf or NaN)
    uint32_t nallow;         // allowed ids in the segment (constrained rows)
    double lsum;             // sum over the segment of exp(x - xmax)
    float tall, tal;         // emission thresholds: every id with x >= tall (any) or x >= tal (allowed) was emitted
    uint32_t flags;          // SEG_* bits
    uint32_t pad[5];
};
static_assert(sizeof(SegSum) == 48, "SegSum layout");
constexpr uint32_t SEG_NAN = 1u;        // the segment holds a NaN logit
constexpr uint32_t SEG_EXACT = 2u;      // thresholds were refined exactly (tie-heavy segment)

// Candidate entry: raw logit bits and id | flags (ids < 2^22).
constexpr uint32_t kEntAllowed = 0x80000000u;
constexpr uint32_t kEntPen = 0x40000000u;
constexpr uint32_t kEntSkip = 0x3FFFFFFFu;  // id field of an entry the finish ignores (a penalized id)
constexpr uint32_t kIdMask = 0x003FFFFFu;

// Device scratch of the split path, owned by the context (sized at create).
struct SplitScratch {
    SegSum* sums;          // [rows * nseg]
    uint2* cand;           // [rows][nseg * kCandCap]: a row's candidates, each segment's in one run
    uint2* pen;            // [rows][kSplitHist]: the row's history ids with their repeats: x bits, id | allowed
    uint64_t* row_ctr;     // [rows] bits 0-23: candidate entries reserved, 24-35: history
                           // entries reserved, 36-47: segments arrived (0 between calls)
};

struct SplitArgs {
    SampleArgs s;
    SplitScratch w;
    uint32_t seg_len, nseg;
    uint32_t general;      // 1: rows this kernel does not take are sampled by sample_kernel
};

constexpr uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }
constexpr uint64_t align256(uint64_t b) { return (b + 255) & ~static_cast<uint64_t>(255); }
// The most segments a call of up to `rows` rows of up to `vocab` ids asks for.
// With L = pick_seg_len(r, u) >= kSegMin, a call has r * ceil(u / L) <= rows *
// ceil(vocab / kSegMin) segments; and L = kSegMax gives rows * ceil(vocab /
// kSegMax), while L between kSegMin and kSegMax (rounded up from r * u / 2048)
// or L = kSegMin (only when r * u <= 2048 * kSegMin) give at most 2048 + r.
constexpr uint64_t max_segments(uint32_t rows, uint32_t vocab) {
    const uint64_t big = static_cast<uint64_t>(rows) * ceil_div(vocab, kSegMax);
    const uint64_t mid = 2048u + 2ull * rows;
    const uint64_t lim = static_cast<uint64_t>(rows) * ceil_div(vocab, kSegMin);
    const uint64_t b = big > mid ? big : mid;
    return b < lim ? b : lim;
}
// Device scratch bytes for `rows` rows of `vocab` ids (the layout of scratch_carve).
constexpr uint64_t scratch_bytes(uint32_t rows, uint32_t vocab) {
    return align256(max_segments(rows, vocab) * sizeof(SegSum)) +
           align256(max_segments(rows, vocab) * kCandCap * sizeof(uint2)) +
           align256(static_cast<uint64_t>(rows) * kSplitHist * sizeof(uint2)) + align256(rows * 8ull);
}
// Carves `base` (scratch_bytes(rows, vocab) bytes) into the scratch record.
SplitScratch scratch_carve(void* base, uint32_t rows, uint32_t vocab);
// Segment length the host picks for a batch (a multiple of kSegQuant).
uint32_t pick_seg_len(uint32_t rows, uint32_t usable);
// Whether a row of this mode and history length is sampled by the split
// kernel: a top-k window, and few enough penalized ids that a segment's exact
// candidate set (window + penalized ids, plus as many allowed ids) fits its
// candidate area.  A history that penalizes nothing does not count.
__host__ __device__ inline bool takes_row(const RowMode& m, uint32_t hist_len) {
    const uint32_t h = m.penal ? hist_len : 0u;
    return m.topk && h <= kSplitHist && m.window + h <= kSplitNeed;
}
// Queues one step of the split kernel on `stream`.
void launch(const SplitArgs& a, uint32_t rows, bool vec_loads, hipStream_t stream);

}  // namespace split
}  // namespace tsm
