// tsm_sample.hip - the sampling kernel: one 1024-thread workgroup per row,
// one launch per step, no device memory besides the caller's inputs and
// outputs and one status word.
//
// Streaming pass (every row): the workgroup reads its row once, in tiles of
// float4 loads with the next tile prefetched into registers, and in the same
// pass
//   * applies the repetition penalty (sampler.rs:165-175) and the presence /
//     frequency penalties in registers: the row's history is turned once into
//     an LDS bitmap of its ids plus a table of their counts;
//   * reads the tile's packed allow-mask words and counts allowed ids;
//   * accumulates max and sum exp(x - max) of the raw logits (sampler.rs:
//     298-304) per thread;
//   * appends to an LDS candidate buffer every element at or above one of
//     three running thresholds: the row's window (top-W by penalized value,
//     sampler.rs:186-194), the best non-penalized values (the raw top-n of
//     logprobs) and the best allowed values (the whole-vocabulary fallback
//     of sampler.rs:211-221).  Penalized ids also go to a list with their
//     raw values.  A threshold starts from a lower bound read off the first
//     tile's group maxima.  After that the waves never wait for each other:
//     each wave reserves buffer slots with one LDS atomic, every kept
//     element is also counted in a small per-threshold histogram of its key,
//     and one wave per tile raises the thresholds (LDS atomicMax) to the
//     highest histogram edge with enough counted elements above it.  The
//     buffer ends holding a small superset of every element the finish can
//     need.
// Finish: exact radix selects over the buffer give the window, the allowed
// ids inside it (or the fallback set) and the raw top-n; the ranked list is
// sorted and finished with the reference's own sequential f32 arithmetic
// (tsm_select.h: exact_finalize), so tokens are bit-exact.
//
// Rows without top-k (window > 1024), rows whose candidates cannot be
// bounded (pathological ties) and rows whose history does not fit the LDS
// table are finished by re-reading the row (tsm_select.h), which is exact
// and slower.
#include "tsm_sample.h"
#include "tsm_nucleus.h"
#include "tsm_serial.h"
#include "tsm_split.h"

namespace tsm {

enum : uint32_t {
    ROWF_BUF_OVERFLOW = 1u,  // the buffer could not hold the candidates: re-read the row
    ROWF_SLOW_HISTORY = 2u,  // history beyond the LDS table: penalties only on re-read
};
constexpr uint32_t kKeyNegInf = 0x007FFFFFu;     // canon_key(-inf): a threshold every non-NaN value passes
constexpr uint32_t kKeyUntracked = 0xFFFFFFFFu;  // threshold of a target not tracked: reads as NaN, keeps nothing
constexpr uint32_t kBigEmit = 64;                // a wave's candidate groups in one tile (of 128) past which it tightens first
constexpr uint32_t kEntPen = 0x80000000u;    // buffer entry flags (ids < 2^22)
constexpr uint32_t kEntAllowed = 0x40000000u;
constexpr uint32_t kEntId = 0x003FFFFFu;
static_assert(kVec == 2, "one group of 8 ids per thread and tile (tile_bounds)");
static_assert(kSBins == 8 * kWave, "raise_thresholds reads 8 bins per lane");

// Selection kinds over the buffer (and the penalized list).
enum : uint32_t {
    SK_ALL = 0,      // every buffer entry, canon(y)
    SK_RAW = 1,      // non-penalized entries, canon(y) == canon(x); plus the penalized list, canon(x)
    SK_ALLOWED = 2,  // allowed entries, total(y) (f32::total_cmp)
};

// Elements each target (SK_*) must keep: 0 = not tracked.
struct Targets {
    uint32_t need[3];
};

struct Sel3 {
    uint64_t T[3];
};

__device__ __forceinline__ uint2* lds_buf() { return reinterpret_cast<uint2*>(lds_base() + kOffBuf); }
__device__ __forceinline__ uint2* lds_pen() { return reinterpret_cast<uint2*>(lds_base() + kOffPen); }
__device__ __forceinline__ uint32_t* lds_hist3() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHist); }
__device__ __forceinline__ uint32_t* lds_misc() { return reinterpret_cast<uint32_t*>(lds_base() + kOffMisc); }
__device__ __forceinline__ double* lds_miscd() { return reinterpret_cast<double*>(lds_base() + kOffMiscD); }
__device__ __forceinline__ uint32_t* lds_tmp() { return reinterpret_cast<uint32_t*>(lds_base() + kOffTmp); }
__device__ __forceinline__ uint32_t* lds_bitmap() { return reinterpret_cast<uint32_t*>(lds_base() + kOffBitmap); }
__device__ __forceinline__ uint32_t* lds_hkey() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHashKey); }
__device__ __forceinline__ uint32_t* lds_hcnt() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHashCnt); }
__device__ __forceinline__ uint32_t* lds_shist() { return reinterpret_cast<uint32_t*>(lds_base() + kOffSHist); }
// One word per wave, written only by that wave: no other wave's write can
// race its initialisation, so the stream needs no barrier for it.
__device__ __forceinline__ uint32_t* lds_nan_wave() { return reinterpret_cast<uint32_t*>(lds_base() + kOffNanW); }
// Some wave's word set: the row holds a NaN logit (a wave-wide read; after a
// barrier that follows the stream).
__device__ __forceinline__ bool row_has_nan() {
    const uint32_t lane = lane_id();
    return wave_ballot(lane < kBlock / kWave && lds_nan_wave()[lane] != 0u) != 0u;
}

// The running thresholds are canon keys in LDS (misc[M_THR + g]), raised
// only by atomicMax.  As a float, y >= key_to_float(k) holds exactly when
// canon_key(y) >= k for every non-NaN y; kKeyUntracked reads as NaN.
__device__ __forceinline__ float thr_float(uint32_t k) { return key_to_float(k); }

// ---- history lookup -----------------------------------------------------------
__device__ __forceinline__ uint32_t hash_slot(uint32_t id) { return (id * 2654435761u) >> 20; }  // 12 bits
static_assert(kHashSlots == 4096, "hash_slot yields 12 bits");

// The row's history ids this thread adds to the lookup (ids tid and
// tid + kBlock of the row's history; ~0 past its end), loaded at the start
// of the kernel so their latency overlaps the first tiles'.
constexpr uint32_t kHistPerThread = kHistFast / kBlock;

// Words read in place of an absent optional input (history offsets, uniforms),
// so that the loads at the start of the kernel need no branch: a branch
// would end the block there and force a wait on every load issued so far.
__device__ uint32_t kZeroWords[4];
static_assert(kHistPerThread * kBlock == kHistFast, "history ids per thread");

// Builds the bitmap of the row's history ids (< n) and their counts.  Needs
// hlen <= kHistFast (the table then stays at most half full) and n <=
// 32 * kBitmapWords.  Starts and ends with a barrier.
__device__ __forceinline__ void history_build(const uint32_t (&hid)[kHistPerThread], uint32_t n) {
    const uint32_t tid = threadIdx.x;
    uint32_t* bm = lds_bitmap();
    uint32_t* hk = lds_hkey();
    uint32_t* hc = lds_hcnt();
    TSM_LDS_SYNC();
    const uint32_t words = (n + 31) / 32;
    for (uint32_t i = tid; i < words; i += kBlock) bm[i] = 0;
    for (uint32_t i = tid; i < kHashSlots; i += kBlock) {
        hk[i] = 0;
        hc[i] = 0;
    }
    TSM_LDS_SYNC();
#pragma unroll
    for (uint32_t k = 0; k < kHistPerThread; k++) {
        const uint32_t id = hid[k];
        if (id >= n) continue;  // past the history, or past the vocabulary cap (sampler.rs:171)
        atomicOr(&bm[id >> 5], 1u << (id & 31u));
        uint32_t s = hash_slot(id);
        for (uint32_t probe = 0; probe < kHashSlots; probe++) {
            const uint32_t old = atomicCAS(&hk[s], 0u, id + 1u);
            if (old == 0u || old == id + 1u) {
                atomicAdd(&hc[s], 1u);
                break;
            }
            s = (s + 1) & (kHashSlots - 1);
        }
    }
    TSM_LDS_SYNC();
}

// Count of `id` in the history (its bitmap bit is set).
__device__ __forceinline__ uint32_t history_count(uint32_t id) {
    const uint32_t* hk = lds_hkey();
    uint32_t s = hash_slot(id);
    for (uint32_t probe = 0; probe < kHashSlots; probe++) {
        const uint32_t k = hk[s];
        if (k == id + 1u) return lds_hcnt()[s];
        if (k == 0u) return 0u;
        s = (s + 1) & (kHashSlots - 1);
    }
    return 0u;
}

// ---- buffer selections -----------------------------------------------------------
__device__ __forceinline__ uint64_t entry_comp(uint32_t kind, uint2 e) {
    const float y = __uint_as_float(e.x);
    const uint32_t key = kind == SK_ALLOWED ? total_key(y) : canon_key(y);
    return composite(key, e.y & kEntId);
}

__device__ __forceinline__ bool entry_in(uint32_t kind, uint2 e) {
    return kind == SK_ALL || (kind == SK_RAW ? !(e.y & kEntPen) : (e.y & kEntAllowed) != 0);
}

// Three block-wide exclusive scans at once (two barriers).
__device__ __forceinline__ void block_excl_scan3(const uint32_t v[3], uint32_t before[3], uint32_t total[3]) {
    constexpr int NW = kBlock / kWave;
    uint32_t* tmp = lds_tmp();
    const uint32_t lane = lane_id(), wid = threadIdx.x / kWave;
    uint32_t inc[3];
#pragma unroll
    for (int g = 0; g < 3; g++) {
        inc[g] = wave_incl_scan(v[g]);
        if (lane == kWave - 1) tmp[g * NW + wid] = inc[g];
    }
    TSM_LDS_SYNC();
    uint32_t t[3];
#pragma unroll
    for (int g = 0; g < 3; g++) t[g] = lane < NW ? tmp[g * NW + lane] : 0u;  // one round trip
#pragma unroll
    for (int g = 0; g < 3; g++) {
        before[g] = row_sum16(lane < wid ? t[g] : 0u) + inc[g] - v[g];
        total[g] = row_sum16(t[g]);
    }
    TSM_LDS_SYNC();
}

// For up to three histograms (kBins bins each, ascending digit = best
// first), finds the digit where the inclusive count reaches need[g] (> 0).
// misc[M_SEL + 2g] = digit or ~0 (fewer than need), misc[M_SEL + 2g + 1] =
// count before it.
__device__ void hist_find3(const uint32_t need[3]) {
    const uint32_t t = threadIdx.x;
    const uint32_t* h = lds_hist3();
    uint32_t* res = lds_misc() + M_SEL;
    static_assert(kBins == 2 * kBlock, "two bins per thread");
    uint32_t c0[3], c1[3], s[3];
#pragma unroll
    for (int g = 0; g < 3; g++) {
        c0[g] = need[g] ? h[g * kBins + 2 * t] : 0u;
        c1[g] = need[g] ? h[g * kBins + 2 * t + 1] : 0u;
        s[g] = c0[g] + c1[g];
    }
    if (t < 6) res[t] = (t & 1) ? 0u : 0xFFFFFFFFu;
    uint32_t before[3], total[3];
    block_excl_scan3(s, before, total);  // its barriers also order the res[] reset
#pragma unroll
    for (int g = 0; g < 3; g++) {
        const uint32_t nd = need[g];
        if (nd && before[g] < nd && before[g] + s[g] >= nd) {
            const bool first = before[g] + c0[g] >= nd;
            res[2 * g] = first ? 2 * t : 2 * t + 1;
            res[2 * g + 1] = first ? before[g] : before[g] + c0[g];
        }
    }
    TSM_LDS_SYNC();
}

// Block-wide min and max of up to three u64 values per thread (one barrier
// pair).  Empty inputs are min = ~0, max = 0.
__device__ __forceinline__ void block_minmax3(unsigned long long mn[3], unsigned long long mx[3]) {
    constexpr int NW = kBlock / kWave;
    unsigned long long* t = reinterpret_cast<unsigned long long*>(lds_base() + kOffHist);  // 96 u64
    const uint32_t lane = lane_id(), wid = threadIdx.x / kWave;
#pragma unroll
    for (int g = 0; g < 3; g++) {
        mn[g] = wave_min_u64_dpp(mn[g]);
        mx[g] = wave_max_u64_dpp(mx[g]);
        if (lane == 0) {
            t[(2 * g) * NW + wid] = mn[g];
            t[(2 * g + 1) * NW + wid] = mx[g];
        }
    }
    TSM_LDS_SYNC();
    unsigned long long a[3], b[3];
#pragma unroll
    for (int g = 0; g < 3; g++) {  // lanes 0..NW-1 read the waves' values in one round trip
        a[g] = lane < NW ? t[(2 * g) * NW + lane] : ~0ull;
        b[g] = lane < NW ? t[(2 * g + 1) * NW + lane] : 0ull;
    }
#pragma unroll
    for (int g = 0; g < 3; g++) {
        mn[g] = row_min16_u64(a[g]);
        mx[g] = row_max16_u64(b[g]);
    }
    TSM_LDS_SYNC();
}

__device__ __forceinline__ int high_bit64(unsigned long long v) { return v ? 63 - __builtin_clzll(v) : -1; }

// Exact selection over the buffer (and, for SK_RAW with `with_pen`, the
// penalized list): for each target g with need[g] > 0, the composite T[g]
// such that exactly need[g] of its entries have composite <= T[g] (low bits
// past the deciding digit are ones), or ~0 when it has fewer entries.
// Radix rounds of up to 11 bits over the composite (~key << 32 | id) start,
// per target, at the highest bit where its entries differ (so the digits
// spread over the bins instead of piling into a few) and skip bits 22..31,
// which are zero in every composite; a target stops as soon as its digit's
// bin holds exactly what is left.
__device__ __forceinline__ Sel3 buf_select(uint32_t bufn, uint32_t penn, bool with_pen, Targets tg) {
    const uint32_t tid = threadIdx.x;
    const uint2* buf = lds_buf();
    const uint2* pen = lds_pen();
    uint32_t* h3 = lds_hist3();
    const uint32_t* misc = lds_misc();
    Sel3 out;
    uint32_t need[3];
    unsigned long long known[3];
    int top[3];  // bits >= top are fixed (known); the next digit ends there
    bool active[3];
    {
        unsigned long long mn[3] = {~0ull, ~0ull, ~0ull}, mx[3] = {0ull, 0ull, 0ull};
        for (uint32_t i = tid; i < bufn; i += kBlock) {
            const uint2 e = buf[i];
#pragma unroll
            for (uint32_t g = 0; g < 3; g++) {
                if (!tg.need[g] || !entry_in(g, e)) continue;
                const unsigned long long c = entry_comp(g, e);
                mn[g] = c < mn[g] ? c : mn[g];
                mx[g] = c > mx[g] ? c : mx[g];
            }
        }
        if (with_pen && tg.need[SK_RAW]) {
            for (uint32_t i = tid; i < penn; i += kBlock) {
                const uint2 e = pen[i];
                const unsigned long long c = composite(canon_key(__uint_as_float(e.x)), e.y & kEntId);
                mn[SK_RAW] = c < mn[SK_RAW] ? c : mn[SK_RAW];
                mx[SK_RAW] = c > mx[SK_RAW] ? c : mx[SK_RAW];
            }
        }
        block_minmax3(mn, mx);
#pragma unroll
        for (int g = 0; g < 3; g++) {
            need[g] = tg.need[g];
            out.T[g] = ~0ull;
            active[g] = need[g] > 0 && mn[g] <= mx[g];  // something to select from
            const int hb = high_bit64(mn[g] ^ mx[g]);
            top[g] = hb + 1;  // 0: every entry has the same composite (one entry)
            known[g] = hb < 0 ? mn[g] : hb >= 63 ? 0ull : (mn[g] & ~((2ull << hb) - 1ull));
            if (active[g] && top[g] == 0) {  // a single entry
                if (need[g] == 1) out.T[g] = mn[g];
                active[g] = false;
            }
        }
    }
    for (int r = 0; r < 6; r++) {
        if (!(active[0] || active[1] || active[2])) break;
        int lo[3];
#pragma unroll
        for (int g = 0; g < 3; g++) lo[g] = top[g] > 11 ? top[g] - 11 : 0;
        for (uint32_t i = tid; i < 3 * kBins; i += kBlock) h3[i] = 0;
        TSM_LDS_SYNC();
        for (uint32_t i = tid; i < bufn; i += kBlock) {
            const uint2 e = buf[i];
#pragma unroll
            for (uint32_t g = 0; g < 3; g++) {
                if (!active[g] || !entry_in(g, e)) continue;
                const unsigned long long c = entry_comp(g, e);
                if (top[g] < 64 && (c >> top[g]) != (known[g] >> top[g])) continue;
                atomicAdd(&h3[g * kBins + static_cast<uint32_t>((c >> lo[g]) & ((1ull << (top[g] - lo[g])) - 1ull))],
                          1u);
            }
        }
        if (with_pen && active[SK_RAW]) {
            const int t1 = top[SK_RAW], l1 = lo[SK_RAW];
            for (uint32_t i = tid; i < penn; i += kBlock) {
                const uint2 e = pen[i];
                const unsigned long long c = composite(canon_key(__uint_as_float(e.x)), e.y & kEntId);
                if (t1 < 64 && (c >> t1) != (known[SK_RAW] >> t1)) continue;
                atomicAdd(&h3[SK_RAW * kBins + static_cast<uint32_t>((c >> l1) & ((1ull << (t1 - l1)) - 1ull))], 1u);
            }
        }
        TSM_LDS_SYNC();
        uint32_t nd[3];
#pragma unroll
        for (int g = 0; g < 3; g++) nd[g] = active[g] ? need[g] : 0u;
        hist_find3(nd);
        uint32_t d[3], before[3], inbin[3];
#pragma unroll
        for (int g = 0; g < 3; g++) {
            d[g] = misc[M_SEL + 2 * g];
            before[g] = misc[M_SEL + 2 * g + 1];
            inbin[g] = (active[g] && d[g] != 0xFFFFFFFFu) ? h3[g * kBins + d[g]] : 0u;
        }
        TSM_LDS_SYNC();  // before the next round clears the histograms / rewrites M_SEL
#pragma unroll
        for (int g = 0; g < 3; g++) {
            if (!active[g]) continue;
            if (d[g] == 0xFFFFFFFFu) {  // fewer entries than need
                active[g] = false;
                continue;
            }
            known[g] |= static_cast<unsigned long long>(d[g]) << lo[g];
            need[g] -= before[g];
            if (inbin[g] == need[g] || lo[g] == 0) {
                out.T[g] = lo[g] == 0 ? known[g] : (known[g] | ((1ull << lo[g]) - 1ull));
                active[g] = false;
            }
            top[g] = lo[g];
            if (top[g] > 22 && top[g] <= 32) top[g] = 22;  // bits 22..31 of a composite are zero
        }
    }
    return out;
}

// Stream emission rule: an element that is not penalized is kept when it is
// at or above the all / raw threshold (tAR, the lower of the two), or when it
// is allowed and at or above the allowed threshold.  Branch-free; an
// untracked threshold is NaN and keeps nothing.  Penalized ids never go to
// the buffer during the stream: they are listed with their raw values and
// join the buffer at the end if their penalized value passes.
__device__ __forceinline__ bool keep2(float y, bool al, float tAR, float tL) {
    return static_cast<bool>((y >= tAR) | (al & (y >= tL)));
}

// Two stream histograms of the keys of emitted (non-penalized) elements:
// H[0] counts every one (it raises the all and raw thresholds), H[1] the
// allowed ones (the allowed threshold).  bin = (key - base) >> shift, clamped
// to the last bin; keys below base are not counted.  A bin's count is a
// number of distinct elements of the row whose keys are at or above the bin's
// lower edge, which is all a raise needs.
struct SHist {
    uint32_t base[2], shift[2];
};

__device__ __forceinline__ void count_kept(float y, bool al, const SHist& h) {
    uint32_t* sh = lds_shist();
    const uint32_t key = canon_key(y);
    if (key >= h.base[0]) atomicAdd(&sh[min((key - h.base[0]) >> h.shift[0], kSBins - 1)], 1u);
    if (al && key >= h.base[1]) atomicAdd(&sh[kSBins + min((key - h.base[1]) >> h.shift[1], kSBins - 1)], 1u);
}

// One wave raises the tracked thresholds: for each, the lower edge of the
// highest histogram bin at which the counts, summed from the top bin down,
// reach need[g].  Other waves keep adding to the counts meanwhile; counts
// only grow, so whatever mix of old and new counts is read is still a valid
// lower bound.  A bin that holds an element has its edge at or below that
// element's key, so the edge never wraps.
__device__ __forceinline__ void raise_from(uint32_t hh, uint32_t need0, uint32_t g0, uint32_t need1, uint32_t g1,
                                           const SHist& h) {
    const uint32_t lane = lane_id();
    uint32_t* misc = lds_misc();
    const uint32_t lo = kSBins - 8u * (lane + 1u);  // lane 0 holds the 8 top bins
    uint32_t* bins = lds_shist() + hh * kSBins + lo;
    uint32_t c[8], sum = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        c[i] = lds_load_relaxed(bins + i);
        sum += c[i];
    }
    const uint32_t incl = wave_incl_scan(sum);  // counts in this lane's bins and every bin above
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t need = k == 0 ? need0 : need1;
        if (!need) continue;
        const uint64_t hit = wave_ballot(incl >= need);
        if (hit == 0) continue;
        if (lane == static_cast<uint32_t>(__builtin_ctzll(hit))) {
            uint32_t acc = incl - sum;  // < need: the lanes above fall short
            uint32_t found = 0;
            bool done = false;
#pragma unroll
            for (int i = 7; i >= 0; i--) {
                acc += c[i];
                if (!done && acc >= need) {
                    found = static_cast<uint32_t>(i);
                    done = true;
                }
            }
            const uint32_t bin = lo + found;
            if (bin > 0) atomicMax(&misc[M_THR + (k == 0 ? g0 : g1)], h.base[hh] + (bin << h.shift[hh]));
        }
    }
}

// ---- candidate groups of the stream ----------------------------------------------
// From the first tile on, the stream keeps its candidates as groups: the four
// values of one float4 load (an aligned group of ids) whenever any of them is
// at or above a threshold, with a tag: the group's first id | its allowed
// nibble << 24.  One compare of the group's maximum decides a group, so the
// stream spends about one instruction per element on candidates; which of a
// group's ids are candidates, and which of them are penalized, is sorted out
// only where groups are counted for a raise and where the stream is closed
// up.  A group is kept on its raw values: a penalized id may pass on its raw
// value and is filtered later.  The group area lies past the first tile's
// distance histograms and ends before the penalized list.
//
// Waves take room for a tile's groups from one bump counter (an LDS atomic
// per wave and tile) and then publish the range in a log slot of its own, so
// the room goes to whichever waves need it.  A raise counts the log's
// published ranges in log order, up to the first slot not yet published.
constexpr uint32_t kG4Base = kOffHist + 4096;               // float4[kG4Cap] values, u32[kG4Cap] tags, u32[kG4Log] log
constexpr uint32_t kG4Cap = 3264;
constexpr uint32_t kG4Log = 1024;                           // reservations per row (16 waves x 64 tiles)
constexpr uint32_t kG4Tag = kG4Base + kG4Cap * 16;
constexpr uint32_t kG4LogOff = kG4Tag + kG4Cap * 4;
static_assert(kG4Base % 16 == 0 && kG4LogOff + kG4Log * 4 <= kOffPen,
              "group area between the histograms and the penalized list");
constexpr uint32_t kG4Nib = 24;                             // tag: allowed nibble's shift
constexpr uint32_t kG4Raise = 128;                          // groups between two raises on demand
constexpr uint32_t kG4Held = (kG4Cap + kBlock - 1) / kBlock;  // groups per thread at the close-up
__device__ __forceinline__ float4* lds_g4val() { return reinterpret_cast<float4*>(lds_base() + kG4Base); }
__device__ __forceinline__ uint32_t* lds_g4tag() { return reinterpret_cast<uint32_t*>(lds_base() + kG4Tag); }
// log slot: the range's first group | its group count << 16 (0: not published)
__device__ __forceinline__ uint32_t* lds_g4log() { return reinterpret_cast<uint32_t*>(lds_base() + kG4LogOff); }
// counters, in the stream's scalar words: G_FILL holds the groups reserved
// (bits 0-15) and the log slots reserved (bits 16-31), so that one atomicAdd
// reserves a slot and its range and the slots' ranges follow each other in
// slot order; G_LOGDONE is the first slot not yet counted by a raise
enum : uint32_t { G_FILL = 0, G_LOGDONE = 2 };
constexpr uint32_t kG4SlotOne = 1u << 16;
__device__ __forceinline__ uint32_t* lds_gctr() { return reinterpret_cast<uint32_t*>(lds_base() + kOffSeg); }
__device__ __forceinline__ float g4_at(const float4& x, uint32_t c) {
    return c == 0u ? x.x : (c == 1u ? x.y : (c == 2u ? x.z : x.w));
}

// Counts the groups published since the last count (one wave): the log slots
// from the counted mark up to the first one not yet published (at most 64)
// are claimed with atomicMax on the mark, so two raising waves never count a
// slot twice.  Their ranges follow each other in the area, so the wave's
// lanes take the claimed groups in turn; each group's ids inside the row that
// are not penalized (the row's history bitmap, when it has one) are counted
// by their values.
__device__ __forceinline__ void count_published_g(const SHist& h, uint32_t n, bool pen_lookup) {
    const uint32_t lane = lane_id();
    uint32_t* ctr = lds_gctr();
    const uint32_t d = lds_load_relaxed(&ctr[G_LOGDONE]);
    const uint32_t nlog = min(lds_load_relaxed(&ctr[G_FILL]) >> 16, kG4Log);
    const uint32_t i = d + lane;
    const uint32_t ent = i < nlog ? lds_load_acquire(&lds_g4log()[i]) : 0u;
    const uint64_t open = wave_ballot(ent == 0u);
    const uint32_t k = open ? static_cast<uint32_t>(__builtin_ctzll(open)) : kWave;  // published slots d .. d+k-1
    if (k == 0u) return;
    uint32_t from = 0;
    if (lane == 0) from = atomicMax(&ctr[G_LOGDONE], d + k);
    from = wave_read(from, 0);
    if (from >= d + k) return;  // another raise counted them
    const uint32_t e0 = wave_read(ent, from - d), e1 = wave_read(ent, k - 1u);
    const uint32_t g_from = e0 & 0xFFFFu, g_to = (e1 & 0xFFFFu) + (e1 >> 16);
    const float4* gv = lds_g4val();
    const uint32_t* gt = lds_g4tag();
    for (uint32_t g = g_from + lane; g < g_to; g += kWave) {
        const float4 x = gv[g];
        const uint32_t tag = gt[g];
        const uint32_t id0 = tag & kEntId;
        const uint32_t pb = pen_lookup ? lds_bitmap()[id0 >> 5] >> (id0 & 31u) : 0u;
#pragma unroll
        for (uint32_t c = 0; c < 4u; c++)
            if (id0 + c < n && !((pb >> c) & 1u)) count_kept(g4_at(x, c), (tag >> (kG4Nib + c)) & 1u, h);
    }
}

__device__ __forceinline__ void raise_thresholds(const Targets& tg, const SHist& h) {
    if (tg.need[SK_ALL] | tg.need[SK_RAW]) raise_from(0, tg.need[SK_ALL], SK_ALL, tg.need[SK_RAW], SK_RAW, h);
    if (tg.need[SK_ALLOWED]) raise_from(1, tg.need[SK_ALLOWED], SK_ALLOWED, 0u, 0u, h);
}

// Wave-local lower bound for a threshold: with lm this lane's largest key
// among its relevant elements (0: none), the need-th largest lane maximum
// (need <= 64) has at least `need` elements of the row at or above it.
// Bitwise search with one ballot per bit; returns 0 when fewer than `need`
// lanes have a relevant element.
__device__ __forceinline__ uint32_t wave_lane_bound(uint32_t lm, uint32_t need) {
    uint32_t k = 0;
#pragma nounroll
    for (int b = 31; b >= 0; b--) {
        const uint32_t c = k | (1u << b);
        if (static_cast<uint32_t>(__popcll(wave_ballot(lm >= c))) >= need) k = c;
    }
    return k;
}

// Key distances below the first tile's largest key, in bins of 1/8 octave:
// distances 0..7 exactly, then for d in [2^e, 2^(e+1)) the bin (e-2)*8 + the
// three bits after the leading one (240 bins up to d < 2^32).
constexpr uint32_t kDistBins = 240;
__device__ __forceinline__ uint32_t dist_bin(uint32_t d) {
    if (d < 8u) return d;
    const uint32_t e = 31u - static_cast<uint32_t>(__builtin_clz(d));
    return ((e - 2u) << 3) | ((d >> (e - 3u)) & 7u);
}
// The largest distance that falls in bin b.
__device__ __forceinline__ uint64_t dist_hi(uint32_t b) {
    if (b < 8u) return b;
    const uint32_t e = (b >> 3) + 2u;
    return ((static_cast<uint64_t>(9u + (b & 7u))) << (e - 3u)) - 1u;
}

// Lower bounds for the thresholds from the first tile: k[g] is this thread's
// largest key among its 8 ids relevant to target g (0: none), so the k[g] are
// distinct elements of the row.  For each target the block's largest k[g]
// (kmax) is found, the distances kmax - k[g] are histogrammed (dist_bin),
// and the bin where the count from the top reaches need[g] gives a key with
// at least need[g] of these elements at or above it.  key[g] gets the target's
// threshold (a canon key, the larger of that bound and the target's start),
// top[g] the largest canon key among the tile's elements relevant to target g
// (0: none), *low a canon key at or below every group maximum of target 0
// (the bottom of the tile's range, for histogram geometry; 0: none); thread 0
// stores the thresholds in misc[M_THR + g], visible after
// the caller's next barrier.  Block-wide, two barriers; every wave finds the
// bins itself, so no third barrier hands the result over.
__device__ __forceinline__ void tile_bounds(Targets tg, uint32_t k0, uint32_t k1, uint32_t k2, uint32_t key[3],
                                            uint32_t top[3], uint32_t* low) {
    constexpr uint32_t NW = kBlock / kWave;
    static_assert(3 * kDistBins <= kBlock && 4 * kWave >= kDistBins, "bin layout");
    const uint32_t tid = threadIdx.x, lane = lane_id(), wid = tid / kWave;
    uint32_t* h = lds_hist3();
    uint32_t* tmp = lds_tmp();
    const uint32_t k[3] = {k0, k1, k2};
    if (tid < 3 * kDistBins) h[tid] = 0;
#pragma unroll
    for (int g = 0; g < 3; g++) {
        const uint32_t wm = wave_max_u32(tg.need[g] ? k[g] : 0u);
        if (lane == 0) tmp[g * NW + wid] = wm;
    }
    TSM_LDS_SYNC();
    uint32_t kmax[3];
#pragma unroll
    for (int g = 0; g < 3; g++) kmax[g] = row_max16(lane < NW ? tmp[g * NW + lane] : 0u);
#pragma unroll
    for (int g = 0; g < 3; g++)
        if (tg.need[g] && k[g] != 0u) atomicAdd(&h[g * kDistBins + dist_bin(kmax[g] - k[g])], 1u);
    TSM_LDS_SYNC();
    *low = 0u;
#pragma unroll
    for (int g = 0; g < 3; g++) {
        key[g] = tg.need[g] ? kKeyNegInf : kKeyUntracked;
        top[g] = kmax[g] ? canon_key(key_to_float(kmax[g])) : 0u;
        if (!tg.need[g] || kmax[g] == 0u) continue;
        // lane l holds bins 4l .. 4l+3, smallest distance first
        uint32_t c[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t bi = 4u * lane + i;
            c[i] = bi < kDistBins ? h[g * kDistBins + bi] : 0u;
            sum += c[i];
        }
        const uint32_t incl = wave_incl_scan(sum);
        if (g == 0) {
            // the largest distance any group maximum has: the bottom of the range
            uint32_t hb = 0;
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (c[i]) hb = 4u * lane + i;
            hb = wave_max_u32(hb);
            const uint64_t hhi = dist_hi(hb);
            const uint32_t kl = hhi >= kmax[0] ? 0u : kmax[0] - static_cast<uint32_t>(hhi);
            *low = kl <= 0x007FFFFFu ? kKeyNegInf : canon_key(key_to_float(kl));
        }
        const uint64_t hit = wave_ballot(incl >= tg.need[g]);
        if (hit == 0) continue;  // fewer relevant elements than need: no bound
        uint32_t run = incl - sum, bin = 0;
        bool done = false;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (!done && run + c[i] >= tg.need[g]) {
                bin = 4u * lane + i;
                done = true;
            }
            run += c[i];
        }
        bin = wave_read(bin, static_cast<uint32_t>(__builtin_ctzll(hit)));
        const uint64_t hi = dist_hi(bin);
        if (hi >= kmax[g]) continue;
        const uint32_t kb = kmax[g] - static_cast<uint32_t>(hi);
        const float b = kb <= 0x007FFFFFu ? -INFINITY : key_to_float(kb);
        key[g] = max(key[g], canon_key(b));
    }
    if (tid == 0) {
#pragma unroll
        for (int g = 0; g < 3; g++) lds_misc()[M_THR + g] = key[g];
    }
}

// Loads one tile into registers.  With vector loads (row_stride a multiple of
// 4, 16-byte aligned rows) every tile takes the same code path: ids past the
// row are clamped to the row's last aligned float4, which lies inside the
// row's allocation, and the consumer masks them (mask_tail).  A single path
// matters: where two paths merge, the compiler copies the loaded registers,
// and a copy waits for the load, which would stall the prefetch.  mp is the
// row's mask, or any readable row of words when there is none (then unused).
template <bool kVecLoads>
__device__ __forceinline__ void load_tile(const float* rowp, const uint32_t* mp, uint32_t tb, uint32_t n,
                                          float (&v)[kVec][4], uint32_t (&mw)[kVec]) {
    const uint32_t tid = threadIdx.x;
    if (kVecLoads) {
        const uint32_t last = (n - 1u) & ~3u;
#pragma unroll
        for (int j = 0; j < kVec; j++) {
            const uint32_t id = min(tb + 4u * (j * kBlock + tid), last);
            const float4 f4 = *reinterpret_cast<const float4*>(rowp + id);
            v[j][0] = f4.x;
            v[j][1] = f4.y;
            v[j][2] = f4.z;
            v[j][3] = f4.w;
            mw[j] = mp[id >> 5];
        }
    } else {
#pragma unroll
        for (int j = 0; j < kVec; j++) {
            const uint32_t id = tb + 4u * (j * kBlock + tid);
#pragma unroll
            for (int q = 0; q < 4; q++) v[j][q] = (id + q < n) ? rowp[id + q] : -INFINITY;
            mw[j] = mp[min(id, n - 1u) >> 5];
        }
    }
}

// The logits half of load_tile (the first tiles' logits are requested before
// anything else is known about the row).
template <bool kVecLoads>
__device__ __forceinline__ void load_logits(const float* rowp, uint32_t tb, uint32_t n, float (&v)[kVec][4]) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < kVec; j++) {
        if (kVecLoads) {
            const uint32_t id = min(tb + 4u * (j * kBlock + tid), (n - 1u) & ~3u);
            const float4 f4 = *reinterpret_cast<const float4*>(rowp + id);
            v[j][0] = f4.x;
            v[j][1] = f4.y;
            v[j][2] = f4.z;
            v[j][3] = f4.w;
        } else {
            const uint32_t id = tb + 4u * (j * kBlock + tid);
#pragma unroll
            for (int q = 0; q < 4; q++) v[j][q] = (id + q < n) ? rowp[id + q] : -INFINITY;
        }
    }
}
// The mask-word half of load_tile.
__device__ __forceinline__ void load_mask(const uint32_t* mp, uint32_t tb, uint32_t n, uint32_t (&mw)[kVec]) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < kVec; j++) mw[j] = mp[min(tb + 4u * (j * kBlock + tid), n - 1u) >> 5];
}

// The row's last tile: ids past the row read -inf (the clamped loads above
// hold other ids' values there).
// Marks a tile's registers as used here, on every path.  A loaded register
// that some path never reads (the mask words of an unconstrained row, the
// logits of a row that tracks nothing) stays a pending load in the
// compiler's wait analysis until it is overwritten; the loop then waits for
// it where the next prefetch reuses the register, which drains the prefetch
// pipeline.  Taking them here puts that wait where the tile is consumed
// anyway.
__device__ __forceinline__ void tile_arrived(const float (&v)[kVec][4], const uint32_t (&mw)[kVec]) {
#pragma unroll
    for (int j = 0; j < kVec; j++) {
        asm volatile("" ::"v"(v[j][0]), "v"(v[j][1]), "v"(v[j][2]), "v"(v[j][3]), "v"(mw[j]));
    }
}

__device__ __forceinline__ void mask_tail(float (&v)[kVec][4], uint32_t tb, uint32_t n) {
    if (tb + kTile <= n) return;  // uniform
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int e = 0; e < kVec * 4; e++)
        if (tb + 4u * ((e >> 2) * kBlock + tid) + (e & 3) >= n) v[e >> 2][e & 3] = -INFINITY;
}

// Emission mask of this thread's tile elements under the thresholds; elig
// marks the elements that may be emitted (in the row, not penalized).
__device__ __forceinline__ uint32_t emit_mask(float tAR, float tL, const float (&v)[kVec][4], uint32_t elig,
                                              uint32_t al_bits) {
    uint32_t emit = 0;
#pragma unroll
    for (int e = 0; e < kVec * 4; e++)
        emit |= static_cast<uint32_t>(keep2(v[e >> 2][e & 3], (al_bits >> e) & 1u, tAR, tL)) << e;
    return emit & elig;
}

// Per-tile work of every thread before the candidates: logsumexp partials of
// the raw logits and the flags.  Ids past the row hold -inf and add 0; a
// tile whose terms grow past 2^100 moves the reference to its own maximum.  Penalized ids are not
// candidates during the stream; with track_pen they are listed with their raw
// values (the list holds every penalized id of the row: at most one entry per
// distinct history id).
constexpr float kL2E = 1.44269504088896341f;  // log2(e) in f32

// Per-thread logsumexp accumulator: sum = sum of exp(x - ref) over this
// thread's ids.  A term is exp2(fma(x, kL2E, nl)) with nl = -ref * kL2E
// rounded; the rounding error eps = fma(ref, kL2E, nl) (exact) shifts every
// exponent by the same amount, which corr = 2^-eps takes back out.
struct LseAcc {
    float ref = 0.0f, nl = 0.0f, corr = 1.0f;
    double sum = 0.0;
    __device__ __forceinline__ void set_ref(float r) {
        ref = r;
        nl = -r * kL2E;
        corr = __builtin_amdgcn_exp2f(-__builtin_fmaf(r, kL2E, nl));
    }
};

struct TileFlags {
    uint32_t elig;  // in the row and not penalized
    uint32_t valid; // in the row
    uint32_t pen;   // penalized (in the row)
    uint32_t al;    // allowed (in the row)
};

__device__ __forceinline__ TileFlags tile_prep(const float (&v)[kVec][4], const uint32_t (&mw)[kVec], uint32_t tb,
                                               uint32_t n, bool logprobs, bool pen_lookup, bool constrained,
                                               LseAcc& L, uint32_t& nallow) {
    const uint32_t tid = threadIdx.x;
    uint32_t valid = (1u << (kVec * 4)) - 1u;
    if (tb + kTile > n) {  // the row's last, partial tile
        valid = 0;
#pragma unroll
        for (int e = 0; e < kVec * 4; e++)
            if (tb + 4u * ((e >> 2) * kBlock + tid) + (e & 3) < n) valid |= 1u << e;
    }
    // NaN logits: a logprobs row finds them in its logsumexp sum (tested
    // after the stream); other rows compare, and a wave that meets one marks
    // its own LDS word (no register carries it through the stream)
    if (!logprobs) {
        bool nan = false;
#pragma unroll
        for (int e = 0; e < kVec * 4; e++) nan |= ((valid >> e) & 1u) && v[e >> 2][e & 3] != v[e >> 2][e & 3];
        if (wave_ballot(nan) && lane_id() == 0) lds_nan_wave()[tid / kWave] = 1u;
    }
    // bitmap words first: their LDS latency overlaps the exponentials (words
    // past the row are read, in bounds, and masked off below)
    uint32_t bw[kVec];
#pragma unroll
    for (int j = 0; j < kVec; j++) bw[j] = pen_lookup ? lds_bitmap()[(tb + 4u * (j * kBlock + tid)) >> 5] : 0u;
    if (logprobs) {
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < kVec * 4; e++)
            sum += __builtin_amdgcn_exp2f(__builtin_fmaf(v[e >> 2][e & 3], kL2E, L.nl));
        if (!(sum < 0x1p100f)) {
            float tmax = L.ref;
#pragma unroll
            for (int e = 0; e < kVec * 4; e++) tmax = fmaxf(tmax, v[e >> 2][e & 3]);
            L.sum *= exp2(static_cast<double>(L.ref - tmax) * 1.4426950408889634);
            L.set_ref(tmax);
            sum = 0.0f;
#pragma unroll
            for (int e = 0; e < kVec * 4; e++)
                sum += __builtin_amdgcn_exp2f(__builtin_fmaf(v[e >> 2][e & 3], kL2E, L.nl));
        }
        L.sum += static_cast<double>(sum * L.corr);
    }
    uint32_t pen = 0, al = 0;
#pragma unroll
    for (int j = 0; j < kVec; j++) {
        const uint32_t sh = (tb + 4u * (j * kBlock + tid)) & 31u;
        pen |= ((bw[j] >> sh) & 0xFu) << (j * 4);
        if (constrained) al |= ((mw[j] >> sh) & 0xFu) << (j * 4);
    }
    pen &= valid;
    al &= valid;
    nallow += __popc(al);
    TileFlags fl;
    fl.elig = valid & ~pen;
    fl.valid = valid;
    fl.pen = pen;
    fl.al = al;
    return fl;
}

// Histogram shift that puts a span of keys into at most 256 bins.
__device__ __forceinline__ uint32_t geo_shift(uint32_t base, uint32_t top) {
    const uint32_t span = top > base ? top - base : 0u;
    const int bits = 32 - __clz(static_cast<int>(span));
    return bits > 8 ? static_cast<uint32_t>(bits - 8) : 0u;
}

// After the streaming pass: logsumexp and allowed count, then the pick (or
// the distribution) and the logprobs of the row.
__device__ __forceinline__ serial::Row serial_row(const Fin& f) {
    serial::Row r;
    r.x = f.rowp;
    r.n = f.n;
    r.hist = f.hist;
    r.hlen = f.hist ? f.hlen : 0u;
    r.mrow = f.mrow;
    r.m = f.m;
    r.P = f.P;
    r.u = f.u;
    return r;
}

// The serial path's LDS areas in the whole-row kernel: region A (the history
// table and the finish's lists), which the stream no longer needs.
__device__ __forceinline__ serial::Lds serial_lds(const Fin& f) {
    serial::Lds s;
    s.cnt = f.cnt();
    s.val = f.ry();
    s.id = f.rid();
    s.comp = f.gcomp();
    s.p = f.rp();
    s.tile = kReTile;
    return s;
}

// The raw top-n of a row holding a NaN (sampler.rs:305-311 through top_n):
// ids in top_n's order, logprobs NaN (the row's logsumexp is NaN).  Wave 0.
// Inlined, as finish_nan: the serial functions it calls take its local copies
// (a reference into the kernel's argument block passed to a function that is
// not inlined would turn the kernel's global loads into flat loads).
__device__ __forceinline__ void nan_top_list(uint32_t* top_ids, float* top_lp, uint32_t top_stride, const Fin& f,
                                             uint32_t nlp) {
    const serial::Row r = serial_row(f);
    const serial::Lds s = serial_lds(f);
    const uint32_t k = serial::top_n_ref(r, s, nlp, false);
    const uint32_t lane = lane_id();
    if (lane < k) {
        const size_t o = static_cast<size_t>(blockIdx.x) * top_stride + lane;
        top_ids[o] = s.id[lane];
        if (top_lp) top_lp[o] = __uint_as_float(0x7FC00000u);
    }
}

__device__ __forceinline__ void finish_row(const SampleArgs& a, const Fin& f_in, const Targets tg0,
                                           const uint32_t nlp, const float lref, const double lsum, uint32_t nallow,
                                           uint32_t bufn) {
    // the re-read functions take the row by reference, which puts it in
    // scratch memory: the copy made here keeps those stores on this path
    Fin f = f_in;
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t n = f.n;
    const RowMode m = f.m;
    uint32_t* misc = lds_misc();
    uint32_t* tmp = lds_tmp();
    const uint2* buf = lds_buf();
    const uint2* pen = lds_pen();

    // ---------------- row statistics ----------------
    TSM_LDS_SYNC();
    {
        const uint32_t wal = wave_sum(nallow);
        if (lane_id() == 0) tmp[tid / kWave] = wal;
        TSM_LDS_SYNC();
        uint32_t al = 0;
        for (int w = 0; w < kBlock / kWave; w++) al += tmp[w];
        nallow = al;
        TSM_LDS_SYNC();
    }
    const uint32_t flags = misc[M_FLAGS];
    const uint32_t penn = misc[M_PENN];
    const bool buf_ok = !(flags & (ROWF_BUF_OVERFLOW | ROWF_SLOW_HISTORY));
    const bool raw_ok = buf_ok && penn <= kPenCap && tg0.need[SK_RAW] > 0;
    TSM_LDS_SYNC();
    // the best raw logit (value desc, id asc): the raw argmax and the max of
    // the logsumexp, from the buffer's non-penalized entries and the
    // penalized list, or by re-reading the row
    uint64_t raw_best = ~0ull;
    const bool none_allowed = m.constrained && nallow == 0;
    if (m.logprobs || none_allowed) {
        if (raw_ok) {
            unsigned long long best = ~0ull;
            for (uint32_t i = tid; i < bufn; i += kBlock) {
                const uint2 e = buf[i];
                if (!(e.y & kEntPen)) {
                    const uint64_t c = entry_comp(SK_ALL, e);
                    best = c < best ? c : best;
                }
            }
            for (uint32_t i = tid; i < min(penn, kPenCap); i += kBlock) {
                const uint2 e = pen[i];
                const uint64_t c = composite(canon_key(__uint_as_float(e.x)), e.y & kEntId);
                best = c < best ? c : best;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const unsigned long long w = __shfl_xor(best, o, kWave);
                best = w < best ? w : best;
            }
            unsigned long long* wb = reinterpret_cast<unsigned long long*>(lds_miscd() + 8);
            if (lane_id() == 0) wb[tid / kWave] = best;
            TSM_LDS_SYNC();
            unsigned long long all = ~0ull;
            for (int w = 0; w < kBlock / kWave; w++) all = wb[w] < all ? wb[w] : all;
            TSM_LDS_SYNC();
            raw_best = all;
        } else {
            Filt q;
            q.order = ORD_CANON_X;
            raw_best = exact_at(f, q, select_kth(f, q, 1));
        }
    }
    float lse = 0.0f;
    if (m.logprobs) {
        // sampler.rs:298-304: lse = max + (f32) ln(sum exp((f64)(l - max)))
        const float rmax = key_to_float(~static_cast<uint32_t>(raw_best >> 32));
        double part = lsum * exp(static_cast<double>(lref) - static_cast<double>(rmax));
        part = wave_sum(part);
        double* wsum = lds_miscd() + 16;  // 16 doubles
        if (lane_id() == 0) wsum[tid / kWave] = part;
        TSM_LDS_SYNC();
        double rs = 0.0;
        for (int w = 0; w < kBlock / kWave; w++) rs += wsum[w];
        lse = rmax + static_cast<float>(log(rs));
        TSM_LDS_SYNC();
    }

    // ---------------- finish ----------------
    const float u = f.u;
    DistOut dist;
    const DistOut* dptr = nullptr;
    if (a.distribution) {
        dist.ids = a.dist_ids + static_cast<size_t>(row) * a.dist_stride;
        dist.probs = a.dist_probs + static_cast<size_t>(row) * a.dist_stride;
        dist.stride = a.dist_stride;
        dist.status = a.status;
        dptr = &dist;
    }
    // exact selections over the buffer: the window, the fallback set, the raw top-n
    Sel3 sel;
    sel.T[0] = sel.T[1] = sel.T[2] = ~0ull;
    if (buf_ok) {
        Targets fin = tg0;
        if (!raw_ok) fin.need[SK_RAW] = 0;
        sel = buf_select(bufn, min(penn, kPenCap), true, fin);
    }
    // raw top-n (sampler.rs:305-311), before the finish reuses the buffer's
    // LDS: from the buffer's non-penalized entries and the penalized list, or
    // by re-reading the row; thread i keeps the i-th composite
    uint64_t raw_mine = ~0ull;
    uint32_t nraw = 0;
    if (nlp > 0) {
        uint64_t* gcomp = f.gcomp();
        if (raw_ok && sel.T[SK_RAW] != ~0ull) {
            if (tid == 0) misc[M_CNT] = 0;
            TSM_LDS_SYNC();
            for (uint32_t i = tid; i < bufn; i += kBlock) {
                const uint2 e = buf[i];
                if (e.y & kEntPen) continue;
                const uint64_t c = entry_comp(SK_ALL, e);
                if (c <= sel.T[SK_RAW]) {
                    const uint32_t pos = atomicAdd(&misc[M_CNT], 1u);
                    if (pos < kExactCap) gcomp[pos] = c;
                }
            }
            for (uint32_t i = tid; i < min(penn, kPenCap); i += kBlock) {
                const uint2 e = pen[i];
                const uint64_t c = composite(canon_key(__uint_as_float(e.x)), e.y & kEntId);
                if (c <= sel.T[SK_RAW]) {
                    const uint32_t pos = atomicAdd(&misc[M_CNT], 1u);
                    if (pos < kExactCap) gcomp[pos] = c;
                }
            }
            TSM_LDS_SYNC();
            const uint32_t g = min(misc[M_CNT], kExactCap);
            TSM_LDS_SYNC();
            sort_u64(gcomp, g);
            nraw = min(g, nlp);
        } else {
            nraw = reread_raw_top(f, nlp);
        }
        if (tid < nraw) raw_mine = gcomp[tid];
        TSM_LDS_SYNC();
    }
    Pick pk;
    pk.token = 0;
    pk.keep = 0;
    pk.prob = 1.0f;
    pk.mass = 0.0f;
    if (none_allowed) {
        // nothing allowed: argmax of the raw row, no draw (sampler.rs:139-141)
        pk.token = static_cast<uint32_t>(raw_best);
    } else if (!m.topk) {
        pk = reread_nucleus(f, nallow, u, dptr);
    } else if (!buf_ok) {
        const uint32_t len = reread_topk_list(f, nallow);
        pk = finish_list(f, len, u, dptr);
    } else {
        // the ranked list from the buffer
        uint64_t* gcomp = f.gcomp();
        if (tid == 0) misc[M_CNT] = 0;
        TSM_LDS_SYNC();
        const bool constrained = m.constrained;
        for (uint32_t i = tid; i < bufn; i += kBlock) {
            const uint2 e = buf[i];
            const uint64_t c = entry_comp(SK_ALL, e);
            if (c <= sel.T[SK_ALL] && (!constrained || (e.y & kEntAllowed))) {
                const uint32_t pos = atomicAdd(&misc[M_CNT], 1u);
                if (pos < kExactCap) gcomp[pos] = c;
            }
        }
        TSM_LDS_SYNC();
        uint32_t g = min(misc[M_CNT], kExactCap);
        TSM_LDS_SYNC();
        uint32_t len = 0;
        if (g > 0) {
            sort_gathered(f, g);
            len = min(g, m.want);
        } else if (constrained) {
            // no allowed id in the window: the whole-vocabulary fallback
            // (sampler.rs:211-221), ordered by f32::total_cmp
            if (tid == 0) misc[M_CNT] = 0;
            TSM_LDS_SYNC();
            for (uint32_t i = tid; i < bufn; i += kBlock) {
                const uint2 e = buf[i];
                if (!(e.y & kEntAllowed)) continue;
                const uint64_t c = entry_comp(SK_ALLOWED, e);
                if (c <= sel.T[SK_ALLOWED]) {
                    const uint32_t pos = atomicAdd(&misc[M_CNT], 1u);
                    if (pos < kExactCap) gcomp[pos] = c;
                }
            }
            TSM_LDS_SYNC();
            g = min(misc[M_CNT], kExactCap);
            TSM_LDS_SYNC();
            sort_gathered(f, g);
            len = min(g, m.want);
        }
        pk = finish_list(f, len, u, dptr);
    }

    // ---------------- outputs ----------------
    if (pk.token >= n) {  // a selection came back empty (e.g. NaN logits)
        if (tid == 0) atomicOr(a.status, TSM_STATUS_INTERNAL);
        pk.token = 0;
    }
    if (a.distribution) {
        if (tid == 0) a.out_keep[row] = pk.keep;
        return;
    }
    if (tid == 0) {
        a.out_token[row] = pk.token;
        if (a.out_prob) a.out_prob[row] = pk.prob;
        if (a.out_keep) a.out_keep[row] = pk.keep;
        if (m.logprobs && a.out_logprob) a.out_logprob[row] = f.rowp[pk.token] - lse;
    }
    if (row_has_nan()) {  // a nucleus row holding a NaN: its raw top-n in top_n's own order
        TSM_LDS_SYNC();
        if (tid < kWave && nlp > 0) nan_top_list(a.out_top_ids, a.out_top_lp, a.top_stride, f, nlp);
        return;
    }
    if (tid < nraw) {
        const uint32_t id = static_cast<uint32_t>(raw_mine);
        const float x = key_to_float(~static_cast<uint32_t>(raw_mine >> 32));
        const size_t o = static_cast<size_t>(row) * a.top_stride + tid;
        a.out_top_ids[o] = id;
        if (a.out_top_lp) a.out_top_lp[o] = x - lse;
    }
}

// ---- single-wave finish ------------------------------------------------------------
// The common rows (top-k, a valid candidate buffer, a ranked list of at most
// 64, not distribution mode) are finished by one wave without a block
// barrier: the block first filters the buffer against the final thresholds
// into two lists (two barriers), then waves 1-15 leave and wave 0 selects,
// sorts and applies the reference's arithmetic.  Within the wave, lanes talk
// through LDS between wave barriers (the wave runs in lockstep; the barrier
// keeps the compiler from reordering across it).
constexpr uint32_t kListCap = 1024;                 // entries of each filtered list (the wave finish takes no more)
__device__ __forceinline__ uint2* lds_swin() { return reinterpret_cast<uint2*>(lds_base()); }  // region A
__device__ __forceinline__ uint64_t* lds_sraw() { return reinterpret_cast<uint64_t*>(lds_base() + kListCap * 8); }
__device__ __forceinline__ uint32_t* lds_whist() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHist); }
__device__ __forceinline__ uint64_t* lds_wlist() { return reinterpret_cast<uint64_t*>(lds_base() + kOffHist + 1024); }
static_assert(kListCap * 16 <= kRegionA, "both filtered lists fit region A");
static_assert(1024 + kWaveList * 8 <= kBins * 12, "wave scratch fits the histogram region");

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long w = __shfl_xor(v, o, kWave);
        v = w < v ? w : v;
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long w = __shfl_xor(v, o, kWave);
        v = w > v ? w : v;
    }
    return v;
}

// The k-th smallest (1-based) of the keys key_of(i, &c) gives for i < n
// (false: not in the set); ~0 when the set has fewer than k keys.  Keys are
// distinct (an id in the low bits).  Radix rounds of 8 bits over a 256-bin
// LDS histogram, from the highest bit where the keys differ; bits 22..31 of a
// composite are zero and skipped; a round whose bin holds one key ends early.
template <class KeyOf>
__device__ uint64_t wave_kth(uint32_t n, uint32_t k, KeyOf key_of) {
    const uint32_t lane = lane_id();
    uint32_t* hist = lds_whist();
    unsigned long long mn = ~0ull, mx = 0;
    uint32_t cnt = 0;
    for (uint32_t i = lane; i < n; i += kWave) {
        uint64_t c;
        if (key_of(i, &c)) {
            mn = c < mn ? c : mn;
            mx = c > mx ? c : mx;
            cnt++;
        }
    }
    mn = wave_min_u64(mn);
    mx = wave_max_u64(mx);
    cnt = wave_sum(cnt);
    if (k == 0 || cnt < k) return ~0ull;
    if (cnt == 1) return mn;
    int top = high_bit64(mn ^ mx) + 1;  // bits >= top are common to every key
    uint64_t prefix = top >= 64 ? 0ull : (mn >> top) << top;
    uint32_t need = k;
    while (top > 0) {
        if (top > 22 && top <= 32) top = 22;  // the zero bits of a composite
        const int lo = top > 8 ? top - 8 : 0;
        const uint32_t width_mask = (1u << (top - lo)) - 1u;
#pragma unroll
        for (int b = 0; b < 4; b++) hist[lane * 4 + b] = 0;
        __builtin_amdgcn_wave_barrier();
        for (uint32_t i = lane; i < n; i += kWave) {
            uint64_t c;
            if (key_of(i, &c) && (top >= 64 || (c >> top) == (prefix >> top)))
                atomicAdd(&hist[static_cast<uint32_t>(c >> lo) & width_mask], 1u);
        }
        __builtin_amdgcn_wave_barrier();
        uint32_t h[4], sum = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            h[b] = hist[lane * 4 + b];
            sum += h[b];
        }
        const uint32_t incl = wave_incl_scan(sum);
        const uint64_t hit = wave_ballot(incl >= need);
        const uint32_t L = static_cast<uint32_t>(__builtin_ctzll(hit));  // the set holds >= need keys here
        uint32_t run = incl - sum, d = 0, before = 0, inbin = 0;
        bool done = false;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (!done && run + h[b] >= need) {
                d = lane * 4 + b;
                before = run;
                inbin = h[b];
                done = true;
            }
            run += h[b];
        }
        d = wave_read(d, L);
        before = wave_read(before, L);
        inbin = wave_read(inbin, L);
        __builtin_amdgcn_wave_barrier();  // every lane has read the bins before the next round clears them
        prefix |= static_cast<uint64_t>(d) << lo;
        need -= before;
        top = lo;
        if (inbin == 1 && top > 0) {
            // the only key with this prefix
            unsigned long long f = ~0ull;
            for (uint32_t i = lane; i < n; i += kWave) {
                uint64_t c;
                if (key_of(i, &c) && (c >> top) == (prefix >> top)) f = c;
            }
            return wave_min_u64(f);
        }
    }
    return prefix;
}

// Register-resident lists for the wave finish: entry i of a list of n sits
// in slot r = i / 64 of lane i % 64 (kWaveRegs slots per lane).
constexpr uint32_t kWaveRegs = 16;
constexpr uint32_t kWaveRegCap = kWaveRegs * kWave;
static_assert(kWaveRegCap <= kListCap, "a list that fits the wave's registers fits its LDS list");

// wave_kth over a register list: key_of(r, &c) gives the key of this lane's
// slot r (false: not in the set); slots at or past n are never asked.
template <class KeyOf>
__device__ __forceinline__ uint64_t wave_kth_reg(uint32_t n, uint32_t k, KeyOf key_of) {
    const uint32_t lane = lane_id();
    uint32_t* hist = lds_whist();
    unsigned long long mn = ~0ull, mx = 0;
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t r = 0; r < kWaveRegs; r++) {
        if (r * kWave >= n) break;
        uint64_t c;
        if (r * kWave + lane < n && key_of(r, &c)) {
            mn = c < mn ? c : mn;
            mx = c > mx ? c : mx;
            cnt++;
        }
    }
    mn = wave_min_u64_dpp(mn);
    mx = wave_max_u64_dpp(mx);
    cnt = wave_sum_dpp(cnt);
    if (k == 0 || cnt < k) return ~0ull;
    if (cnt == 1) return mn;
    int top = high_bit64(mn ^ mx) + 1;
    uint64_t prefix = top >= 64 ? 0ull : (mn >> top) << top;
    uint32_t need = k;
    while (top > 0) {
        if (top > 22 && top <= 32) top = 22;  // the zero bits of a composite
        const int lo = top > 8 ? top - 8 : 0;
        const uint32_t width_mask = (1u << (top - lo)) - 1u;
#pragma unroll
        for (int b = 0; b < 4; b++) hist[lane * 4 + b] = 0;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (uint32_t r = 0; r < kWaveRegs; r++) {
            if (r * kWave >= n) break;
            uint64_t c;
            if (r * kWave + lane < n && key_of(r, &c) && (top >= 64 || (c >> top) == (prefix >> top)))
                atomicAdd(&hist[static_cast<uint32_t>(c >> lo) & width_mask], 1u);
        }
        __builtin_amdgcn_wave_barrier();
        uint32_t h[4], sum = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            h[b] = hist[lane * 4 + b];
            sum += h[b];
        }
        const uint32_t incl = wave_incl_scan(sum);
        const uint32_t L = static_cast<uint32_t>(__builtin_ctzll(wave_ballot(incl >= need)));
        uint32_t run = incl - sum, d = 0, before = 0, inbin = 0;
        bool done = false;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (!done && run + h[b] >= need) {
                d = lane * 4 + b;
                before = run;
                inbin = h[b];
                done = true;
            }
            run += h[b];
        }
        d = wave_read(d, L);
        before = wave_read(before, L);
        inbin = wave_read(inbin, L);
        __builtin_amdgcn_wave_barrier();
        prefix |= static_cast<uint64_t>(d) << lo;
        need -= before;
        top = lo;
        if (inbin == 1 && top > 0) {
            unsigned long long f = ~0ull;
#pragma unroll
            for (uint32_t r = 0; r < kWaveRegs; r++) {
                if (r * kWave >= n) break;
                uint64_t c;
                if (r * kWave + lane < n && key_of(r, &c) && (c >> top) == (prefix >> top)) f = c;
            }
            return wave_min_u64_dpp(f);
        }
    }
    return prefix;
}

// Writes the register list's keys key_of gives (true) into lds_wlist(), in
// any order; returns how many.
template <class KeyOf>
__device__ __forceinline__ uint32_t wave_gather_reg(uint32_t n, KeyOf key_of) {
    const uint32_t lane = lane_id();
    uint64_t* out = lds_wlist();
    uint32_t cnt = 0;
#pragma unroll
    for (uint32_t r = 0; r < kWaveRegs; r++) {
        if (r * kWave >= n) break;
        uint64_t c = 0;
        const bool in = r * kWave + lane < n && key_of(r, &c);
        const uint64_t b = wave_ballot(in);
        if (in) out[cnt + lanes_below(b)] = c;
        cnt += static_cast<uint32_t>(__popcll(b));
    }
    __builtin_amdgcn_wave_barrier();
    return cnt;
}

// Sorts one u64 per lane ascending across the wave (bitonic; lanes past the
// list hold ~0).
__device__ __forceinline__ uint64_t wave_sort64(uint64_t v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (uint32_t k = 2; k <= static_cast<uint32_t>(kWave); k <<= 1)
#pragma unroll
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            const unsigned long long o = __shfl_xor(static_cast<unsigned long long>(v), static_cast<int>(j), kWave);
            const bool keep_min = ((lane & j) == 0) == ((lane & k) == 0);
            v = keep_min ? (o < v ? o : v) : (o > v ? o : v);
        }
    return v;
}

__device__ __forceinline__ uint64_t* lds_wsort() { return reinterpret_cast<uint64_t*>(lds_base() + kOffHist + 1024 + kWaveList * 8); }
static_assert(1024 + 2 * kWaveList * 8 <= kBins * 12, "wave sort scratch fits the histogram region");

// Sorts the keys of lanes < n (n <= 64, distinct) ascending: the keys go to
// LDS, each lane counts the keys below its own with loads every lane makes
// at the same address (one LDS access each, no readlane round trips), then
// the keys trade places through LDS.  Lanes >= n get ~0.
__device__ __forceinline__ uint64_t wave_sort_rank(uint64_t v, uint32_t n) {
    const uint32_t lane = lane_id();
    uint64_t* t = lds_wsort();
    t[lane] = lane < n ? v : ~0ull;  // a key past the list (~0) is never below a listed one
    __builtin_amdgcn_wave_barrier();
    uint32_t rank = 0;
    for (uint32_t j0 = 0; j0 < n; j0 += 8) {
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) rank += t[j0 + i] < v ? 1u : 0u;
    }
    // the wave's reads above complete before its writes below (LDS operations
    // of one wave run in order)
    __builtin_amdgcn_wave_barrier();
    if (lane < n) t[rank] = v;
    __builtin_amdgcn_wave_barrier();
    const uint64_t r = lane < n ? t[lane] : ~0ull;
    __builtin_amdgcn_wave_barrier();
    return r;
}

// Rank sort of up to kRankMax distinct keys by one wave: the keys in
// lds_rkeys()[0..n), padded with ~0 keys to a multiple of 8; each lane takes
// K = ceil(n / 64) of them, counts for each the keys below it, eight keys per
// step with loads every lane makes at the same address, and writes it at its
// rank in lds_rsorted().  n / 8 steps of 8K compares per lane.
constexpr uint32_t kRankMax = 256;
constexpr uint32_t kRankCut = 96;  // more allowed keys than this: only those at or below a cut are sorted
__device__ __forceinline__ uint64_t* lds_rkeys() { return reinterpret_cast<uint64_t*>(lds_base() + kOffHist + 4096); }
__device__ __forceinline__ uint64_t* lds_rsorted() { return lds_rkeys() + kRankMax + 8; }
static_assert(4096 + (2 * kRankMax + 8) * 8 <= kBins * 12, "rank sort scratch fits the histogram region");
template <uint32_t K>
__device__ __forceinline__ void wave_rank_sort_k(uint32_t n) {
    const uint32_t lane = lane_id();
    const uint64_t* t = lds_rkeys();
    uint64_t v[K];
    uint32_t rk[K];
#pragma unroll
    for (uint32_t k = 0; k < K; k++) {
        const uint32_t i = k * kWave + lane;
        v[k] = i < n ? t[i] : ~0ull;
        rk[k] = 0;
    }
    for (uint32_t j = 0; j < n; j += 8) {
        uint64_t a[8];
#pragma unroll
        for (uint32_t q = 0; q < 8; q++) a[q] = t[j + q];
#pragma unroll
        for (uint32_t q = 0; q < 8; q++)
#pragma unroll
            for (uint32_t k = 0; k < K; k++) rk[k] += a[q] < v[k] ? 1u : 0u;
    }
    // the wave's reads above complete before its writes below (LDS operations
    // of one wave run in order)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (uint32_t k = 0; k < K; k++)
        if (k * kWave + lane < n) lds_rsorted()[rk[k]] = v[k];
    __builtin_amdgcn_wave_barrier();
}
__device__ __forceinline__ void wave_rank_sort(uint32_t n) {
    if (n <= kWave) wave_rank_sort_k<1>(n);
    else if (n <= 2 * kWave) wave_rank_sort_k<2>(n);
    else wave_rank_sort_k<4>(n);
}

// The reference's arithmetic on a ranked list held one entry per lane (lane
// j: value y, best first, j < len <= 64), as exact_finalize does it:
// p_j = expf((y_j - y_0) / t) (sampler.rs:231-234), min-p, top-p
// (sampler.rs:235-246) and the draw (sampler.rs:142-150), every fold in list
// order so the roundings are the CPU sampler's.
__device__ __forceinline__ Pick wave_finalize(float y, uint32_t id, uint32_t len, float u, const RowMode& m,
                                              const tsm_row_params& P) {
    const uint32_t lane = lane_id();
    const float y0 = readlane_f(y, 0);
    const float p = lane < len ? glibc_expf((y - y0) / m.t) : 0.0f;
    if (!m.greedy && P.min_p > 0.0f) {
        const uint64_t below = wave_ballot(lane < len && !(p >= P.min_p));
        if (below) len = max(static_cast<uint32_t>(__builtin_ctzll(below)), 1u);
    }
    // The three folds run over the list in steps of eight elements, without a
    // branch per element: every lane adds the same terms in list order (read
    // from LDS at one address for all lanes), records the running value in
    // the lane of the element just added, and the first lane that meets a
    // condition is found by ballot afterwards.  Past the list p is 0, which
    // leaves a running sum as it is (sums of non-negative terms start from
    // +0).  The list's keys are in registers by now, so the sort's LDS words
    // hold the terms.
    const float pl = lane < len ? p : 0.0f;
    float* tp = reinterpret_cast<float*>(lds_wsort());  // [64] p, then [64] q
    tp[lane] = pl;
    __builtin_amdgcn_wave_barrier();
    // prefix sums (left fold) of p over the list
    float total = 0.0f, pre = 0.0f;
    for (uint32_t j0 = 0; j0 < len; j0 += 8) {
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            total += tp[j0 + i];
            pre = lane == j0 + i ? total : pre;
        }
    }
    uint32_t keep = len;
    if (!(m.greedy || P.top_p >= 1.0f)) {
        // the first j with q_0 + ... + q_j >= top_p (sampler.rs:240-246)
        const float q = lane < len ? pl / total : 0.0f;
        tp[kWave + lane] = q;
        __builtin_amdgcn_wave_barrier();
        float acc = 0.0f, accl = 0.0f;
        for (uint32_t j0 = 0; j0 < len; j0 += 8) {
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                acc += tp[kWave + j0 + i];
                accl = lane == j0 + i ? acc : accl;
            }
        }
        const uint64_t hit = wave_ballot(lane < len && accl >= P.top_p);
        if (hit) keep = static_cast<uint32_t>(__builtin_ctzll(hit)) + 1u;
    }
    const float mass = readlane_f(pre, keep - 1);
    // the draw: the first j < keep where u * mass - p_0 - ... - p_j <= 0
    // (sampler.rs:142-150), else the last kept
    uint32_t pick = keep - 1;
    float r = u * mass, rl = 0.0f;
    for (uint32_t j0 = 0; j0 < keep; j0 += 8) {
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            r -= tp[j0 + i];
            rl = lane == j0 + i ? r : rl;
        }
    }
    __builtin_amdgcn_wave_barrier();  // the terms are read before the next sort reuses the words
    const uint64_t hit = wave_ballot(lane < keep && rl <= 0.0f);
    if (hit) pick = static_cast<uint32_t>(__builtin_ctzll(hit));
    Pick out;
    out.token = wave_read(id, pick);
    out.keep = keep;
    out.prob = readlane_f(p, pick) / mass;
    out.mass = mass;
    return out;
}

// Writes into lds_wlist() the keys key_of gives (true) for i < n, in any
// order; returns how many.
template <class KeyOf>
__device__ __forceinline__ uint32_t wave_gather(uint32_t n, KeyOf key_of) {
    const uint32_t lane = lane_id();
    uint64_t* out = lds_wlist();
    uint32_t cnt = 0;
    for (uint32_t i0 = 0; i0 < n; i0 += kWave) {
        const uint32_t i = i0 + lane;
        uint64_t c = 0;
        const bool in = i < n && key_of(i, &c);
        const uint64_t b = wave_ballot(in);
        if (in) out[cnt + lanes_below(b)] = c;
        cnt += static_cast<uint32_t>(__popcll(b));
    }
    __builtin_amdgcn_wave_barrier();
    return cnt;
}

// The finish of a row by one wave (see above).  The whole block takes part
// in the filtering; returns false, before any wave leaves, when a list does
// not fit (the caller then runs the block finish), true once the row is done.
// Inlined: were the kernel's argument block passed by reference to a function
// that is not inlined, it would escape, every pointer read from it would lose
// its global address space, and the stream's loads would become flat loads
// (which every LDS wait then also waits for).
__device__ __forceinline__ bool finish_wave(const SampleArgs& a, const Fin& f, const Targets tg0, const uint32_t nlp, const float lref,
                            const double lsum, const uint32_t nallow, const uint32_t bufn) {
    constexpr uint32_t NW = kBlock / kWave;
    constexpr uint32_t kB = kBufCap / NW / kWave;  // buffer entries per lane in a wave's slice
    constexpr uint32_t kP = kPenCap / NW / kWave;  // penalized-list entries per lane
    const uint32_t row = blockIdx.x, tid = threadIdx.x, lane = lane_id(), wid = tid / kWave;
    const RowMode m = f.m;
    uint32_t* misc = lds_misc();
    uint32_t* tmp = lds_tmp();
    double* md = lds_miscd();
    unsigned long long* mbest = reinterpret_cast<unsigned long long*>(md + NW);
    const uint2* buf = lds_buf();
    const uint2* pen = lds_pen();
    const float tA = thr_float(misc[M_THR + static_cast<uint32_t>(SK_ALL)]);
    const float tR = thr_float(misc[M_THR + static_cast<uint32_t>(SK_RAW)]);
    const float tL = thr_float(misc[M_THR + static_cast<uint32_t>(SK_ALLOWED)]);
    const uint32_t penn = min(misc[M_PENN], kPenCap);
    const bool need_raw = tg0.need[SK_RAW] > 0;

    // ---- the block: each wave filters its slice of the buffer (window and
    // fallback candidates at or above the final thresholds; raw candidates)
    // and of the penalized list (raw candidates, by raw value) ----
    const uint32_t bseg = (bufn + NW - 1) / NW, pseg = (penn + NW - 1) / NW;
    uint2 we[kB];
    bool win[kB], rawk[kB], prk[kP];
    uint64_t pc[kP];
    unsigned long long best = ~0ull;  // the best raw (value desc, id asc)
    uint32_t cw = 0, cr = 0;
#pragma unroll
    for (uint32_t k = 0; k < kB; k++) {
        const uint32_t j = lane + k * kWave, i = wid * bseg + j;
        win[k] = rawk[k] = false;
        we[k] = make_uint2(0u, 0u);
        if (j < bseg && i < bufn) {
            const uint2 e = buf[i];
            const float y = __uint_as_float(e.x);
            win[k] = keep2(y, (e.y & kEntAllowed) != 0u, tA, tL);
            if (!(e.y & kEntPen)) {
                const unsigned long long c = composite(canon_key(y), e.y & kEntId);
                best = c < best ? c : best;
                rawk[k] = need_raw && y >= tR;
            }
            we[k] = e;
        }
        cw += static_cast<uint32_t>(__popcll(wave_ballot(win[k])));
        cr += static_cast<uint32_t>(__popcll(wave_ballot(rawk[k])));
    }
#pragma unroll
    for (uint32_t k = 0; k < kP; k++) {
        const uint32_t j = lane + k * kWave, i = wid * pseg + j;
        prk[k] = false;
        pc[k] = 0;
        if (j < pseg && i < penn) {
            const uint2 e = pen[i];
            const float x = __uint_as_float(e.x);
            const unsigned long long c = composite(canon_key(x), e.y & kEntId);
            best = c < best ? c : best;
            prk[k] = need_raw && x >= tR;
            pc[k] = c;
        }
        cr += static_cast<uint32_t>(__popcll(wave_ballot(prk[k])));
    }
    // the wave's shares of the allowed count and of the logsumexp (its own
    // reference: the largest of its threads')
    const uint32_t nallow_w = wave_sum_dpp(nallow);
    const float mref = wave_max_dpp(lsum > 0.0 ? lref : -INFINITY);
    // (the rescale factors are f32 exponentials: a term's relative error is
    // about |exponent| * 2^-24 while its size is 2^exponent, far inside the
    // logprob tolerance; an f64 exp costs each of the 16 waves ~100 VALU)
    double sw = lsum > 0.0 ? lsum * static_cast<double>(__builtin_amdgcn_exp2f((lref - mref) * kL2E)) : 0.0;
    sw = wave_sum_f64_dpp(sw);
    best = wave_min_u64_dpp(best);
    if (lane == 0) {
        tmp[wid] = cw;
        tmp[NW + wid] = cr;
        tmp[2 * NW + wid] = nallow_w;
        tmp[3 * NW + wid] = __float_as_uint(mref);
        md[wid] = sw;
        mbest[wid] = best;
    }
    TSM_LDS_SYNC();
    const uint32_t c1 = lane < NW ? tmp[lane] : 0u, c2 = lane < NW ? tmp[NW + lane] : 0u;  // one round trip
    uint32_t bw = row_sum16(lane < wid ? c1 : 0u), br = row_sum16(lane < wid ? c2 : 0u);
    const uint32_t nwin = row_sum16(c1), nraw_all = row_sum16(c2);
    const bool fits = nwin <= kWaveRegCap && nraw_all <= kWaveRegCap;  // wave 0 holds both in registers
    if (fits) {
        uint2* swin = lds_swin();
        uint64_t* sraw = lds_sraw();
#pragma unroll
        for (uint32_t k = 0; k < kB; k++) {
            const uint64_t b = wave_ballot(win[k]);
            if (win[k]) swin[bw + lanes_below(b)] = we[k];
            bw += static_cast<uint32_t>(__popcll(b));
            const uint64_t b2 = wave_ballot(rawk[k]);
            if (rawk[k]) sraw[br + lanes_below(b2)] = composite(canon_key(__uint_as_float(we[k].x)), we[k].y & kEntId);
            br += static_cast<uint32_t>(__popcll(b2));
        }
#pragma unroll
        for (uint32_t k = 0; k < kP; k++) {
            const uint64_t b = wave_ballot(prk[k]);
            if (prk[k]) sraw[br + lanes_below(b)] = pc[k];
            br += static_cast<uint32_t>(__popcll(b));
        }
    }
    TSM_LDS_SYNC();
    if (!fits) return false;
    if (wid != 0) return true;

    // ---- wave 0 ----
    const uint32_t nallow_all = wave_sum_dpp(lane < NW ? tmp[2 * NW + lane] : 0u);
    const unsigned long long raw_best = wave_min_u64_dpp(lane < NW ? mbest[lane] : ~0ull);
    float lse = 0.0f;
    if (m.logprobs) {
        // sampler.rs:298-304: lse = max + (f32) ln(sum exp((f64)(l - max)))
        const float rmax = key_to_float(~static_cast<uint32_t>(raw_best >> 32));
        double term = 0.0;
        if (lane < NW) {
            const float mw = __uint_as_float(tmp[3 * NW + lane]);
            if (mw != -INFINITY) term = md[lane] * static_cast<double>(__builtin_amdgcn_exp2f((mw - rmax) * kL2E));
        }
        lse = rmax + static_cast<float>(log(wave_sum_f64_dpp(term)));
    }
    const float u = f.u;
    Pick pk;
    pk.token = 0;
    pk.keep = 0;
    pk.prob = 1.0f;
    pk.mass = 0.0f;
    if (m.constrained && nallow_all == 0) {
        pk.token = static_cast<uint32_t>(raw_best);  // nothing allowed: the raw argmax (sampler.rs:139-141)
    } else {
        // the window list, in registers
        uint2 wl[kWaveRegs];
        {
            const uint2* swin = lds_swin();
#pragma unroll
            for (uint32_t r = 0; r < kWaveRegs; r++) {
                const uint32_t i = r * kWave + lane;
                wl[r] = i < nwin ? swin[i] : make_uint2(0u, 0u);
            }
        }
        auto canon_all = [&](uint32_t r, uint64_t* c) {
            *c = composite(canon_key(__uint_as_float(wl[r].x)), wl[r].y & kEntId);
            return true;
        };
        auto allowed_c = [&](uint32_t r, uint64_t* c) {
            if (!(wl[r].y & kEntAllowed)) return false;
            return canon_all(r, c);
        };
        // A constrained row keeps the `want` best allowed ids of the window
        // when the window holds at least that many (sampler.rs:209-210,
        // :223).  Those are then the `want` best allowed ids of the row: the
        // want-th of them, ta, decides it alone when at most W listed
        // entries rank at or above it (every element at or above the window
        // threshold is listed, so the count is the rank of ta in the row
        // whenever it is <= W), and the window boundary is not needed.
        uint64_t ta = ~0ull;
        bool fast = false, sorted = false;
        uint32_t nal_sorted = 0;  // keys in lds_rsorted() when sorted
        uint64_t cut = ~0ull;     // the allowed keys above it are not in lds_rsorted()
        if (m.constrained) {
            // the window list's allowed keys, ranked against each other when
            // at most kRankMax: the want-th is then read off, and the kept list
            // is the sorted prefix
            uint32_t nal = 0;
            uint64_t* rk = lds_rkeys();
            // Of many allowed keys only the best want + 1 matter (the kept
            // list, ta, and the first key after the kept ones).  Each lane's
            // best is a distinct key, so at least ci + 1 keys lie at or below
            // the (ci+1)-th best of the lanes' bests (ci = want, or 63 when
            // want is 64), and the keys above that cut are left out of the
            // sort.  (A row that is not fast has fewer than want allowed keys
            // inside the window, so its window boundary lies below the cut
            // too.)
            const uint32_t ci = min(m.want, static_cast<uint32_t>(kWave) - 1u);
            {
                uint64_t lb = ~0ull;
                uint32_t cnt = 0;
#pragma unroll
                for (uint32_t r = 0; r < kWaveRegs; r++) {
                    if (r * kWave >= nwin) break;
                    uint64_t c = 0;
                    if (r * kWave + lane < nwin && allowed_c(r, &c)) {
                        lb = c < lb ? c : lb;
                        cnt++;
                    }
                }
                const uint32_t lanes = static_cast<uint32_t>(__popcll(wave_ballot(lb != ~0ull)));
                if (wave_sum_dpp(cnt) > kRankCut && lanes > ci) {
                    // lanes without an allowed key hold ~0 and sort last
                    const uint64_t srt = wave_sort_rank(lb, kWave);
                    cut = (static_cast<uint64_t>(wave_read(static_cast<uint32_t>(srt >> 32), ci)) << 32) |
                          wave_read(static_cast<uint32_t>(srt), ci);
                }
            }
#pragma unroll
            for (uint32_t r = 0; r < kWaveRegs; r++) {
                if (r * kWave >= nwin) break;
                uint64_t c = 0;
                const bool in = r * kWave + lane < nwin && allowed_c(r, &c) && c <= cut;
                const uint64_t b = wave_ballot(in);
                const uint32_t at = nal + lanes_below(b);
                if (in && at < kRankMax) rk[at] = c;
                nal += static_cast<uint32_t>(__popcll(b));
            }
            if (nal <= kRankMax && nal > 0u) {
                if (lane < 8u) rk[nal + lane] = ~0ull;  // the pad to a multiple of 8
                __builtin_amdgcn_wave_barrier();
                wave_rank_sort(nal);
                // fewer than `want` allowed keys listed: no want-th (not fast)
                ta = nal >= m.want ? lds_rsorted()[m.want - 1u] : ~0ull;
                sorted = true;
                nal_sorted = nal;
            } else if (nal > kRankMax) {
                __builtin_amdgcn_wave_barrier();
                ta = wave_kth_reg(nwin, m.want, allowed_c);
            }
            if (ta != ~0ull) {
                uint32_t rank = 0;
#pragma unroll
                for (uint32_t r = 0; r < kWaveRegs; r++) {
                    if (r * kWave >= nwin) break;
                    uint64_t c;
                    rank += (r * kWave + lane < nwin && canon_all(r, &c) && c <= ta) ? 1u : 0u;
                }
                fast = wave_sum_dpp(rank) <= m.window;
            }
        }
        uint32_t g;
        bool prefix = false;  // the kept list is lds_rsorted()[0..g)
        if (fast && sorted) {
            g = m.want;  // lds_rsorted()[0..want): the kept list, in order
            prefix = true;
        } else if (m.constrained && sorted) {
            // fewer than `want` allowed ids rank inside the window: the kept
            // list is every allowed id inside it (sampler.rs:209-210), which
            // is the prefix of the sorted allowed keys at or below the window
            // boundary
            const uint64_t tw = wave_kth_reg(nwin, m.window, canon_all);
            uint32_t inw = 0;
            for (uint32_t i = lane; i < nal_sorted; i += kWave) inw += lds_rsorted()[i] <= tw ? 1u : 0u;
            inw = wave_sum_dpp(inw);
            // with no value +-0 among them, the best allowed ids by
            // f32::total_cmp (the fallback below) are the sorted prefix too:
            // the two orders differ only between -0 and +0
            const uint32_t lf = min(nal_sorted, m.want);
            auto is_zero = [&](uint32_t i) {
                return static_cast<uint32_t>(lds_rsorted()[i] >> 32) == ~canon_key(0.0f);
            };
            // the kept ones and the first one after them (when the cut left
            // that one out, the check cannot be made: the general path)
            const bool zero = (lane < lf && is_zero(lane)) || (lane == 0 && lf < nal_sorted && is_zero(lf)) ||
                              (lane == 0 && lf == nal_sorted && cut != ~0ull);
            if (inw > 0) {
                g = min(inw, m.want);
                prefix = true;
            } else if (!wave_ballot(zero)) {
                g = lf;  // none in the window: the row's best allowed ids (sampler.rs:211-221)
                prefix = true;
            } else {
                // none in the window: the best allowed ids of the whole row by
                // f32::total_cmp (sampler.rs:211-221)
                auto allowed_total = [&](uint32_t r, uint64_t* c) {
                    if (!(wl[r].y & kEntAllowed)) return false;
                    *c = composite(total_key(__uint_as_float(wl[r].x)), wl[r].y & kEntId);
                    return true;
                };
                const uint64_t tf = wave_kth_reg(nwin, m.want, allowed_total);
                g = wave_gather_reg(nwin, [&](uint32_t r, uint64_t* c) { return allowed_total(r, c) && *c <= tf; });
            }
        } else if (fast) {
            g = wave_gather_reg(nwin, [&](uint32_t r, uint64_t* c) { return allowed_c(r, c) && *c <= ta; });
        } else if (!m.constrained) {
            // the window boundary: the W-th best by IEEE order (top_n, sampler.rs:192-194)
            const uint64_t tw = wave_kth_reg(nwin, m.window, canon_all);
            g = wave_gather_reg(nwin, [&](uint32_t r, uint64_t* c) { return canon_all(r, c) && *c <= tw; });
        } else {
            const uint64_t tw = wave_kth_reg(nwin, m.window, canon_all);
            // allowed ids inside the window (sampler.rs:209-210)
            auto in_window = [&](uint32_t r, uint64_t* c) {
                if (!(wl[r].y & kEntAllowed)) return false;
                return canon_all(r, c) && *c <= tw;
            };
            uint32_t inw = 0;
#pragma unroll
            for (uint32_t r = 0; r < kWaveRegs; r++) {
                if (r * kWave >= nwin) break;
                uint64_t c;
                inw += (r * kWave + lane < nwin && in_window(r, &c)) ? 1u : 0u;
            }
            inw = wave_sum_dpp(inw);
            if (inw > 0) {
                const uint64_t tin = inw > m.want ? wave_kth_reg(nwin, m.want, in_window) : ~0ull;
                g = wave_gather_reg(nwin, [&](uint32_t r, uint64_t* c) { return in_window(r, c) && *c <= tin; });
            } else {
                // none in the window: the best allowed ids of the whole row by
                // f32::total_cmp (sampler.rs:211-221)
                auto allowed_total = [&](uint32_t r, uint64_t* c) {
                    if (!(wl[r].y & kEntAllowed)) return false;
                    *c = composite(total_key(__uint_as_float(wl[r].x)), wl[r].y & kEntId);
                    return true;
                };
                const uint64_t tf = wave_kth_reg(nwin, m.want, allowed_total);
                g = wave_gather_reg(nwin, [&](uint32_t r, uint64_t* c) { return allowed_total(r, c) && *c <= tf; });
            }
        }
        const uint32_t len = min(g, m.want);
        const uint64_t mine = prefix ? (lane < len ? lds_rsorted()[lane] : ~0ull)
                                     : wave_sort_rank(lane < g ? lds_wlist()[lane] : ~0ull, g);
        if (len == 0) {
            pk.token = 0xFFFFFFFFu;  // nothing to rank (e.g. NaN logits): flagged below
        } else {
            const float y = key_to_float(~static_cast<uint32_t>(mine >> 32));
            pk = wave_finalize(y, static_cast<uint32_t>(mine), len, u, m, f.P);
        }
    }

    // ---- outputs ----
    if (pk.token >= f.n) {
        if (lane == 0) atomicOr(a.status, TSM_STATUS_INTERNAL);
        pk.token = 0;
    }
    // the token's raw logit is requested now and used last, after the raw top-n
    const float x_tok = (m.logprobs && a.out_logprob) ? f.rowp[pk.token] : 0.0f;
    if (nlp > 0) {
        // raw top-n (sampler.rs:305-311), ties -> lower id
        uint64_t rl[kWaveRegs];
        {
            const uint64_t* sraw = lds_sraw();
#pragma unroll
            for (uint32_t r = 0; r < kWaveRegs; r++) {
                const uint32_t i = r * kWave + lane;
                rl[r] = i < nraw_all ? sraw[i] : ~0ull;
            }
        }
        auto raw_key = [&](uint32_t r, uint64_t* c) {
            *c = rl[r];
            return true;
        };
        uint64_t mine;
        uint32_t g;
        if (nraw_all <= static_cast<uint32_t>(kWave)) {  // one entry per lane: rank them all
            g = nraw_all;
            mine = wave_sort_rank(rl[0], g);
        } else {
            const uint64_t tr = wave_kth_reg(nraw_all, nlp, raw_key);
            g = wave_gather_reg(nraw_all, [&](uint32_t r, uint64_t* c) { return raw_key(r, c) && *c <= tr; });
            mine = wave_sort_rank(lane < g ? lds_wlist()[lane] : ~0ull, g);
        }
        const uint32_t nraw = min(g, nlp);
        if (lane < nraw) {
            const size_t o = static_cast<size_t>(row) * a.top_stride + lane;
            a.out_top_ids[o] = static_cast<uint32_t>(mine);
            if (a.out_top_lp) a.out_top_lp[o] = key_to_float(~static_cast<uint32_t>(mine >> 32)) - lse;
        }
    }
    if (lane == 0) {
        a.out_token[row] = pk.token;
        if (a.out_prob) a.out_prob[row] = pk.prob;
        if (a.out_keep) a.out_keep[row] = pk.keep;
        if (m.logprobs && a.out_logprob) a.out_logprob[row] = x_tok - lse;
    }
    return true;
}

// Top_n-path rows (and sample()'s greedy shortcut) whose logits hold a NaN
// (tsm_serial.h): wave 0 samples the row step by step.  The logprobs are
// NaN, as the reference's logsumexp is then (sampler.rs:298-304).  A nucleus
// row keeps the cutoff path, which a NaN never enters (it fails `l >=
// cutoff`, sampler.rs:203); only its raw top-n is redone (nan_top_list).
__device__ __forceinline__ void finish_nan(const SampleArgs& a, const Fin& f, uint32_t nlp) {
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const RowMode m = f.m;
    const serial::Row r = serial_row(f);
    const serial::Lds s = serial_lds(f);
    constexpr float kNaN = __builtin_nanf("");
    TSM_LDS_SYNC();
    serial::Result res;
    res.token = res.keep = res.len = 0;
    res.prob = res.mass = 0.0f;
    uint32_t* misc = lds_misc();
    if (tid < kWave) {
        res = serial::run(r, s, !a.distribution);
        if (tid == 0) {
            misc[M_TOKEN] = res.token;
            misc[M_KEEP] = res.keep;
            misc[M_PROB] = __float_as_uint(res.prob);
            misc[M_MASS] = __float_as_uint(res.mass);
        }
    }
    TSM_LDS_SYNC();
    res.token = misc[M_TOKEN];
    res.keep = misc[M_KEEP];
    res.prob = __uint_as_float(misc[M_PROB]);
    res.mass = __uint_as_float(misc[M_MASS]);
    if (a.distribution) {
        const uint32_t k = min(res.keep, a.dist_stride);
        uint32_t* ids = a.dist_ids + static_cast<size_t>(row) * a.dist_stride;
        float* probs = a.dist_probs + static_cast<size_t>(row) * a.dist_stride;
        for (uint32_t j = tid; j < k; j += kBlock) {
            ids[j] = s.id[j];
            probs[j] = s.p[j] / res.mass;
        }
        if (res.keep > a.dist_stride && tid == 0) atomicOr(a.status, TSM_STATUS_DIST_TRUNCATED);
        if (tid == 0) a.out_keep[row] = res.keep;
        return;
    }
    if (tid == 0) {
        a.out_token[row] = res.token;
        if (a.out_prob) a.out_prob[row] = res.prob;
        if (a.out_keep) a.out_keep[row] = res.keep;
        if (m.logprobs && a.out_logprob) a.out_logprob[row] = kNaN;
    }
    if (nlp > 0) {
        TSM_LDS_SYNC();  // the list areas are taken again
        if (tid < kWave) nan_top_list(a.out_top_ids, a.out_top_lp, a.top_stride, f, nlp);
    }
}

// finish_nan's arguments, handed over in LDS (the histogram area, unused
// once the stream is done): the call then passes nothing in registers, so
// the rare NaN branch adds no register pressure to the kernel's stream.
struct NanCall {
    SampleArgs a;
    Fin f;
    uint32_t nlp;
};
static_assert(sizeof(NanCall) <= kBins * 12, "NanCall fits the histogram area");
__device__ __forceinline__ NanCall* nan_call() { return reinterpret_cast<NanCall*>(lds_base() + kOffHist); }

__device__ __noinline__ void finish_nan_call() {
    const SampleArgs a = nan_call()->a;
    const Fin f = nan_call()->f;
    const uint32_t nlp = nan_call()->nlp;
    finish_nan(a, f, nlp);
}

// A penalty that can only lower a value: repetition penalty >= 1 (finite),
// presence and frequency penalties >= 0 (finite) (sampler.rs:165-175 and the
// extension).
__device__ __forceinline__ bool lowers_only(const tsm_row_params& P) {
    return P.repetition_penalty >= 1.0f && P.repetition_penalty <= 3.4e38f && P.frequency_penalty >= 0.0f &&
           P.frequency_penalty <= 3.4e38f && P.presence_penalty >= 0.0f && P.presence_penalty <= 3.4e38f;
}

// The general finish of a row the lean kernel could not finish on one wave
// (candidates past its buffers): its arguments come through LDS, so the call
// passes only the per-thread partials in registers and adds nothing to the
// lean kernel's register use.
struct RowCall {
    SampleArgs a;
    Fin f;
    Targets tg0;
    uint32_t nlp, bufn;
};
static_assert(sizeof(RowCall) <= kBins * 12, "RowCall fits the histogram area");
__device__ __forceinline__ RowCall* row_call() { return reinterpret_cast<RowCall*>(lds_base() + kOffHist); }
__device__ __noinline__ void finish_row_call(float lref, double lsum, uint32_t nallow) {
    const SampleArgs a = row_call()->a;
    const Fin f = row_call()->f;
    const Targets tg0 = row_call()->tg0;
    const uint32_t nlp = row_call()->nlp, bufn = row_call()->bufn;
    TSM_LDS_SYNC();  // read by every thread before the finish reuses the area
    finish_row(a, f, tg0, nlp, lref, lsum, nallow, bufn);
}

// One row of a sampling step.  kLean: the lean kernel, which takes only the
// rows of lean_takes (and finishes a row it cannot finish on one wave, a NaN
// logit or candidates past its buffers, through out-of-line calls);
// otherwise the general kernel, which leaves those rows to the lean kernel
// when it runs (a.skip_lean).
template <bool kVecLoads, bool kLean>
__device__ __forceinline__ void sample_row(const SampleArgs& a) {
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t n = a.usable;
    // first the loads that depend on nothing: the row's history offsets,
    // parameters and uniform, then the first two tiles' logits.  Loads
    // complete in order, so the small ones go first: the history ids and mask
    // words that depend on them can then be requested while the tiles are
    // still in flight.
    // The mask words are read whenever the batch has a mask (used only for
    // constrained rows), else from the logits, in place.
    float v[kVec][4], vB[kVec][4], vC[kVec][4];
    uint32_t mw[kVec], mwB[kVec], mwC[kVec];
    const float* rowp0 = a.logits + static_cast<size_t>(row) * a.row_stride;
    const uint32_t* hop = a.hist_off ? a.hist_off + row : kZeroWords;
    const uint32_t h0 = const_as(hop)[0], h1 = const_as(hop)[1];
    tsm_row_params P;
    {
        static_assert(sizeof(tsm_row_params) % 4 == 0, "row parameters are whole words");
        constexpr int kW = sizeof(tsm_row_params) / 4;
        const TSM_CONST_AS uint32_t* pw = const_as(reinterpret_cast<const uint32_t*>(a.params + row));
        uint32_t w[kW];
#pragma unroll
        for (int i = 0; i < kW; i++) w[i] = pw[i];
        __builtin_memcpy(&P, w, sizeof(P));
    }
    const float u_load =
        __uint_as_float(const_as(a.uniforms ? reinterpret_cast<const uint32_t*>(a.uniforms) + row : kZeroWords)[0]);
    const uint32_t* mp = a.mask ? a.mask + static_cast<size_t>(row) * a.mask_stride
                                : reinterpret_cast<const uint32_t*>(rowp0);
    // which kernel takes the row, decided before any tile is requested
    if (kLean || a.skip_lean) {
        const uint32_t hl = h1 > h0 ? h1 - h0 : 0u;
        const RowMode m0 = row_mode(P, n, hl, a.mask != nullptr && !a.distribution);
        if (a.skip_split && split::takes_row(m0, hl)) return;  // sampled by split_kernel
        const bool lean = lean_takes(m0, P, hl, n, a.distribution != 0u);
        if (!kLean && lean) return;  // sampled by the lean kernel
        if (kLean && !lean) {
            // sampled by the general kernel; without it (the batch said it
            // holds no such row) the row is reported instead
            if (!a.general && tid == 0) {
                a.out_token[row] = 0;
                atomicOr(a.status, TSM_STATUS_ROW_KIND);
            }
            return;
        }
    }
    load_logits<kVecLoads>(rowp0, 0, n, v);
    load_mask(mp, 0, n, mw);
    load_logits<kVecLoads>(rowp0, kTile, n, vB);
    load_mask(mp, kTile, n, mwB);
    const float u_row = a.distribution ? 0.0f : u_load;
    const uint32_t hlen = h1 > h0 ? h1 - h0 : 0u;
    uint32_t hid[kHistPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kHistPerThread; k++) {
        const uint32_t h = tid + k * kBlock;
        hid[k] = (a.hist_ids && h < hlen && hlen <= kHistFast) ? a.hist_ids[h0 + h] : 0xFFFFFFFFu;
    }
    Fin f;
    f.rowp = rowp0;
    f.hist = a.hist_ids ? a.hist_ids + h0 : nullptr;
    f.hlen = hlen;
    f.n = n;
    f.u = u_row;
    // distribution() takes no constraint (sampler.rs:102-116)
    f.m = row_mode(P, n, hlen, a.mask != nullptr && !a.distribution);
    f.mrow = f.m.constrained ? a.mask + static_cast<size_t>(row) * a.mask_stride : nullptr;
    f.P = P;
    const RowMode m = f.m;  // register copies: f escapes to the re-read functions
    if (a.skip_split && split::takes_row(m, hlen)) return;  // sampled by split_kernel
    const float* rowp = f.rowp;
    uint32_t* misc = lds_misc();
    uint2* buf = lds_buf();
    uint2* pen = lds_pen();

    uint32_t nlp = (m.logprobs && a.out_top_ids != nullptr) ? m.nlp : 0u;
    if (nlp > a.top_stride) {  // the list must fit the row's slots
        if (tid == 0) atomicOr(a.status, TSM_STATUS_BAD_PARAMS);
        nlp = a.top_stride;
    }
    // penalties need the history lookup; without it the stream keeps no candidates
    const bool fast_hist = kLean || !m.penal || (hlen <= kHistFast && n <= 32 * kBitmapWords);
    Targets tg;
    tg.need[SK_ALL] = (m.topk && fast_hist) ? m.window : 0u;
    // the raw top-n, and the raw best for the logsumexp / the argmax when nothing is allowed
    tg.need[SK_RAW] = fast_hist ? max(nlp, (m.constrained || m.logprobs) ? 1u : 0u) : 0u;
    tg.need[SK_ALLOWED] = (m.topk && m.constrained && fast_hist) ? m.want : 0u;
    Targets tg0 = tg;
    if (!fast_hist) tg0.need[SK_RAW] = 0u;
    const bool tracking = kLean || (tg.need[SK_ALL] | tg.need[SK_RAW] | tg.need[SK_ALLOWED]) != 0;
    const bool pen_lookup = m.penal && fast_hist;  // the row's history bitmap and counts are built
    // A penalty that can only lower a value (repetition penalty >= 1, finite;
    // presence and frequency penalties >= 0, finite: sampler.rs:165-175 and
    // the extension) leaves every penalized value at or below its raw value,
    // so the stream's groups, kept on raw values, hold every penalized id the
    // finish can need, and the penalized list is filed from them when the
    // stream is closed up.  Otherwise the penalized list is gathered up front
    // from the history table (a penalized value may rise above its raw value).
    const bool lower_only = kLean || lowers_only(P);
    const bool track_pen = pen_lookup && tracking && !lower_only;  // the list gathered up front
    const bool file_pen = pen_lookup && tracking && lower_only;     // the list filed at the close-up
    if (tid == 0) {
        misc[M_BUFN] = 0;
        misc[M_PENN] = 0;
        misc[M_OVF] = 0;
        misc[M_FLAGS] = fast_hist ? 0u : ROWF_SLOW_HISTORY;
        for (int g = 0; g < 3; g++) misc[M_THR + g] = tg.need[g] ? kKeyNegInf : kKeyUntracked;
    }
    if (tracking) {  // first used after the first tile's barriers
        for (uint32_t i = tid; i < 2 * kSBins; i += kBlock) lds_shist()[i] = 0;
        if (tid < 4) lds_gctr()[tid] = 0;  // group, log and count counters
        for (uint32_t i = tid; i < kG4Log; i += kBlock) lds_g4log()[i] = 0u;
    }
    // three register sets take the tiles in turn (tile t in set t mod 3):
    // tiles t+1 and t+2 are in flight while tile t is processed, and no set is
    // ever copied to another (a copy would wait for its loads).  Loads past
    // the row's last tile read in bounds and go unused: an unconditional load
    // keeps one code path.
    if (pen_lookup) history_build(hid, n);  // barriers inside
    // The penalized list (raw logit, id, allowed bit) is gathered once, from
    // the history table's distinct ids: each thread loads the logits and mask
    // words of its table slots now and files them after the first tile, when
    // the loads have long arrived; the stream itself only skips penalized ids.
    constexpr uint32_t kSlotsPerThread = kHashSlots / kBlock;
    static_assert(kSlotsPerThread * kBlock == kHashSlots, "table slots per thread");
    float pen_x[kSlotsPerThread];
    uint32_t pen_w[kSlotsPerThread], pen_id[kSlotsPerThread];
#pragma unroll
    for (uint32_t k = 0; k < kSlotsPerThread; k++) {
        pen_x[k] = 0.0f;
        pen_w[k] = 0u;
        pen_id[k] = 0xFFFFFFFFu;
    }
    if (track_pen) {
#pragma unroll
        for (uint32_t k = 0; k < kSlotsPerThread; k++) {
            const uint32_t key = lds_hkey()[tid + k * kBlock];  // id + 1, 0 = empty
            pen_id[k] = key - 1u;
            const uint32_t id = key ? key - 1u : 0u;
            pen_x[k] = rowp[id];
            pen_w[k] = mp[id >> 5];
        }
    }

    SHist sh;
    sh.base[0] = sh.base[1] = kKeyUntracked;
    sh.shift[0] = sh.shift[1] = 0;
    bool wave_track = tracking;  // uniform per wave; cleared once the buffer overflows
    const uint32_t wid = tid / kWave, lane = lane_id();

    // ---------------- streaming pass ----------------
    if (lane == 0) lds_nan_wave()[wid] = 0u;
    LseAcc lse;
    mask_tail(v, 0, n);
    if (m.logprobs) {
        float t0 = -INFINITY;
#pragma unroll
        for (int e = 0; e < kVec * 4; e++) t0 = fmaxf(t0, v[e >> 2][e & 3]);
        lse.set_ref(t0 == -INFINITY ? 0.0f : t0);
    }
    uint32_t nallow = 0;
    // the stream's results (candidates, allowed count, logsumexp) serve
    // top-k rows, constrained rows and logprob rows; any other row (a nucleus
    // over the whole vocabulary) is finished by re-reading and stops after
    // the first tile
    const bool stream_all = tracking || m.logprobs || m.constrained;
    const uint32_t ntiles = stream_all ? (n + kTile - 1) / kTile : 1u;
    load_tile<kVecLoads>(rowp, mp, 2 * kTile, n, vC, mwC);  // prefetch
    {
        // first tile: block-wide, so the thresholds can start from the tile's
        // own group-max bounds; its groups fill [0, seg0) of the group area
        const TileFlags fl = tile_prep(v, mw, 0, n, m.logprobs, pen_lookup, m.constrained, lse, nallow);
        if (tracking) {
            uint32_t k[3] = {0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < kVec * 4; e++) {
                if (!((fl.elig >> e) & 1u)) continue;
                const float y = v[e >> 2][e & 3];
                k[SK_ALL] = max(k[SK_ALL], canon_key(y));
                if ((fl.al >> e) & 1u) k[SK_ALLOWED] = max(k[SK_ALLOWED], total_key(y));
            }
            k[SK_RAW] = k[SK_ALL];  // bounds from the non-penalized ids
            uint32_t top[3], key[3], low;
            tile_bounds(tg, k[0], k[1], k[2], key, top, &low);
            float th[3];
#pragma unroll
            for (int g = 0; g < 3; g++) th[g] = thr_float(key[g]);
            // histogram geometry: H[0] from the all / raw bounds; H[1] from
            // the allowed bound, or H[0]'s when the first tile gave none
            uint32_t b0 = kKeyUntracked, t0 = 0;
#pragma unroll
            for (int g = 0; g < 2; g++)
                if (tg.need[g]) {
                    b0 = min(b0, key[g]);
                    t0 = max(t0, top[g]);
                }
            sh.base[0] = b0;
            sh.shift[0] = geo_shift(b0, t0);
            if (tg.need[SK_ALLOWED] && key[SK_ALLOWED] > kKeyNegInf) {
                sh.base[1] = key[SK_ALLOWED];
                sh.shift[1] = geo_shift(key[SK_ALLOWED], top[SK_ALLOWED]);
            } else if (tg.need[SK_ALLOWED] && b0 > low && t0 > b0) {
                // too few allowed ids in the first tile to bound them: the
                // allowed histogram reaches three spans of the window
                // histogram further down (not below the tile's lowest
                // group maximum), so allowed candidates below the other
                // thresholds are still counted
                const uint64_t ext = min(3ull * (t0 - b0), static_cast<uint64_t>(b0 - low));
                sh.base[1] = b0 - static_cast<uint32_t>(ext);
                sh.shift[1] = geo_shift(sh.base[1], t0);
            } else {
                sh.base[1] = sh.base[0];
                sh.shift[1] = sh.shift[0];
            }
            // a group is kept when any of its ids in the row passes on its raw
            // value (penalized ids too); the non-penalized ones that pass are
            // counted for the raises
            const float tAR = fminf(th[SK_ALL], th[SK_RAW]), tL = th[SK_ALLOWED];
            const uint32_t pass = emit_mask(tAR, tL, v, fl.valid, fl.al);
            uint32_t gpass = 0;
#pragma unroll
            for (int j = 0; j < kVec; j++) gpass |= ((pass >> (4 * j)) & 0xFu) ? (1u << j) : 0u;
            uint32_t total;
            uint32_t pos = block_excl_scan<kBlock>(__popc(gpass), lds_tmp(), &total);
            float4* gv = lds_g4val();
            uint32_t* gt = lds_g4tag();
#pragma unroll
            for (int j = 0; j < kVec; j++) {
                if (!((gpass >> j) & 1u)) continue;
                gv[pos] = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
                gt[pos] = (4u * (j * kBlock + tid)) | (((fl.al >> (4 * j)) & 0xFu) << kG4Nib);
                pos++;
            }
            const uint32_t cnt = pass & fl.elig;
#pragma unroll
            for (int e = 0; e < kVec * 4; e++)
                if ((cnt >> e) & 1u) count_kept(v[e >> 2][e & 3], (fl.al >> e) & 1u, sh);
            if (track_pen) {
                // one LDS atomic per wave reserves the wave's places
                uint64_t b[kSlotsPerThread];
                uint32_t cntp = 0;
#pragma unroll
                for (uint32_t q = 0; q < kSlotsPerThread; q++) {
                    b[q] = wave_ballot(pen_id[q] != 0xFFFFFFFFu);
                    cntp += static_cast<uint32_t>(__popcll(b[q]));
                }
                uint32_t at = 0;
                if (cntp && lane == 0) at = atomicAdd(&misc[M_PENN], cntp);
                at = wave_uniform(wave_read(at, 0));
#pragma unroll
                for (uint32_t q = 0; q < kSlotsPerThread; q++) {
                    const uint32_t id = pen_id[q];
                    if (id != 0xFFFFFFFFu) {
                        const bool al = m.constrained && ((pen_w[q] >> (id & 31u)) & 1u);
                        pen[at + lanes_below(b[q])] = make_uint2(__float_as_uint(pen_x[q]), id | (al ? kEntAllowed : 0u));
                    }
                    at += static_cast<uint32_t>(__popcll(b[q]));
                }
            }
            if (tid == 0) lds_gctr()[G_FILL] = total;  // <= kVec * kBlock groups
            TSM_LDS_SYNC();
        }
    }
    // tile t (>= 1) in register set v, the prefetch of tile t+2 into set pf
    auto step = [&](const uint32_t t, float (&v)[kVec][4], const uint32_t (&mw)[kVec], float (&pf)[kVec][4],
                    uint32_t (&mpf)[kVec]) __attribute__((always_inline)) {
        const uint32_t tb = t * kTile;
        load_tile<kVecLoads>(rowp, mp, tb + 2 * kTile, n, pf, mpf);
        tile_arrived(v, mw);
        mask_tail(v, tb, n);
        // the thresholds as they are now (they only rise, so any value read is
        // valid), loaded before the tile's arithmetic so it hides their latency
        uint32_t ovf = 0, kA = 0, kR = 0, kL = 0;
        if (wave_track) {
            ovf = lds_load_relaxed(&misc[M_OVF]);
            kA = lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_ALL)]);
            kR = lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_RAW)]);
            kL = lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_ALLOWED)]);
        }
        const TileFlags fl = tile_prep(v, mw, tb, n, m.logprobs, false, m.constrained, lse, nallow);
        if (wave_track && wave_uniform(ovf) != 0u) wave_track = false;  // the finish re-reads the row
        if (wave_track) {
            // no barriers: each wave appends its groups to its own segment and
            // publishes the segment's fill
            const bool tail = tb + kTile > n;
            float tAR = fminf(thr_float(wave_uniform(kA)), thr_float(wave_uniform(kR)));
            float tL = thr_float(wave_uniform(kL));
            bool use_l = !(tL >= tAR) && tL == tL;  // allowed ids need a compare of their own
            // group maxima, over every id and over the allowed ids
            float gm[kVec], ga[kVec];
#pragma unroll
            for (int j = 0; j < kVec; j++) {
                gm[j] = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
                ga[j] = -INFINITY;
            }
            auto group_pass = [&](int j) __attribute__((always_inline)) {
                bool k = gm[j] >= tAR;
                // (ga is -inf for a group without allowed ids, which a -inf
                // allowed threshold would pass: the nibble decides that)
                if (use_l) k = static_cast<bool>(k | (((fl.al >> (4 * j)) & 0xFu) != 0u && ga[j] >= tL));
                if (tail) k = static_cast<bool>(k & static_cast<bool>((fl.valid >> (4 * j)) & 0xFu));
                return k;
            };
            auto allowed_max = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < kVec; j++) {
                    float a = -INFINITY;
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        if ((fl.al >> (4 * j + c)) & 1u) a = fmaxf(a, v[j][c]);
                    ga[j] = a;
                }
            };
            if (use_l) allowed_max();
            uint64_t gb[kVec];
            uint32_t tot = 0;
#pragma unroll
            for (int j = 0; j < kVec; j++) {
                gb[j] = wave_ballot(group_pass(j));
                tot += static_cast<uint32_t>(__popcll(gb[j]));
            }
            auto reload = [&]() __attribute__((always_inline)) {
                tAR = fminf(thr_float(wave_uniform(lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_ALL)]))),
                            thr_float(wave_uniform(lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_RAW)]))));
                tL = thr_float(wave_uniform(lds_load_relaxed(&misc[M_THR + static_cast<uint32_t>(SK_ALLOWED)])));
                const bool was_l = use_l;
                use_l = !(tL >= tAR) && tL == tL;
                if (use_l && !was_l) allowed_max();
                tot = 0;
#pragma unroll
                for (int j = 0; j < kVec; j++) {
                    gb[j] = wave_ballot(group_pass(j));
                    tot += static_cast<uint32_t>(__popcll(gb[j]));
                }
            };
            if (tot > kBigEmit) {
                // far more groups than a tile should bring (a target the first
                // tile could not bound, or a dense stretch of the row): raise
                // the thresholds from this wave's own lane maxima over its ids
                // that are not penalized, then keep what still passes
                uint32_t pb = 0;
                if (pen_lookup) {
#pragma unroll
                    for (int j = 0; j < kVec; j++) {
                        const uint32_t id0 = tb + 4u * (j * kBlock + tid);
                        pb |= ((lds_bitmap()[min(id0, n - 1u) >> 5] >> (id0 & 31u)) & 0xFu) << (4 * j);
                    }
                }
                uint32_t lmA = 0, lmL = 0;
#pragma unroll
                for (int e = 0; e < kVec * 4; e++)
                    if (((fl.valid & ~pb) >> e) & 1u) {
                        const uint32_t ck = canon_key(v[e >> 2][e & 3]);
                        lmA = max(lmA, ck);
                        if ((fl.al >> e) & 1u) lmL = max(lmL, ck);
                    }
#pragma unroll
                for (int g = 0; g < 3; g++) {
                    const uint32_t need = tg.need[g];
                    if (need == 0 || need > static_cast<uint32_t>(kWave)) continue;
                    const uint32_t kb = wave_lane_bound(g == SK_ALLOWED ? lmL : lmA, need);
                    if (kb != 0u && lane == 0) atomicMax(&misc[M_THR + g], kb);
                }
                reload();
            }
            if (tot) {
                uint32_t* ctr = lds_gctr();
                if ((wave_uniform(lds_load_relaxed(&ctr[G_FILL])) & 0xFFFFu) + tot > kG4Cap) {
                    // the area cannot take the tile's groups: raise the
                    // thresholds from everything published so far (any wave
                    // may raise), then count again before giving up
                    count_published_g(sh, n, pen_lookup);
                    raise_thresholds(tg, sh);
                    reload();
                }
                uint32_t r = 0;
                if (tot && lane == 0) r = atomicAdd(&ctr[G_FILL], tot | kG4SlotOne);
                r = wave_read(r, 0);
                const uint32_t at0 = r & 0xFFFFu, slot = r >> 16;
                if (!tot) {
                } else if (at0 + tot <= kG4Cap && slot < kG4Log) {
                    uint32_t pos = at0;
                    float4* gv = lds_g4val();
                    uint32_t* gt = lds_g4tag();
#pragma unroll
                    for (int j = 0; j < kVec; j++) {
                        if (gb[j] == 0) continue;
                        if ((gb[j] >> lane) & 1u) {
                            const uint32_t at = pos + lanes_below(gb[j]);
                            gv[at] = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
                            gt[at] = (tb + 4u * (j * kBlock + tid)) | (((fl.al >> (4 * j)) & 0xFu) << kG4Nib);
                        }
                        pos += static_cast<uint32_t>(__popcll(gb[j]));
                    }
                    // every lane releases its own writes with the publish
                    // (read-modify-writes of one value: one release sequence)
                    __builtin_amdgcn_wave_barrier();
                    lds_publish_max(&lds_g4log()[slot], at0 | (tot << 16));
                    // the wave whose groups cross a multiple of kG4Raise in
                    // the area raises the thresholds at once: the raises keep
                    // up with the groups however fast they come
                    if ((at0 + tot) / kG4Raise != at0 / kG4Raise) {
                        count_published_g(sh, n, pen_lookup);
                        raise_thresholds(tg, sh);
                    }
                } else {
                    // no room left (the row is re-read by the finish)
                    if (lane == 0) atomicOr(&misc[M_OVF], 1u);
                    wave_track = false;
                }
            }
            // one wave counts what was published and raises the thresholds
            // on every tile
            if (wave_track && wid == (t & (kBlock / kWave - 1))) {
                count_published_g(sh, n, pen_lookup);
                raise_thresholds(tg, sh);
            }
        }
    };
    // whole rounds of three tiles, then the one or two left: a break inside
    // the round would let the compiler's wait analysis see a path from a
    // round's first tile back to the loop head, and the head would then wait
    // for that tile's prefetch on every round
    uint32_t t = 1;
    for (; t + 2 < ntiles; t += 3) {
        step(t, vB, mwB, v, mw);
        step(t + 1, vC, mwC, vB, mwB);
        step(t + 2, v, mw, vC, mwC);
    }
    if (t < ntiles) step(t, vB, mwB, v, mw);
    if (t + 1 < ntiles) step(t + 1, vC, mwC, vB, mwB);
    TSM_LDS_SYNC();
    uint32_t bufn = 0;
    if (tracking) {
        // the stream's final state, read by every thread before anything below
        // changes it (the decisions taken from it must be uniform)
        const uint32_t ovf0 = misc[M_OVF], penn0 = file_pen ? 0u : misc[M_PENN];
        const float tA = thr_float(misc[M_THR + static_cast<uint32_t>(SK_ALL)]);
        const float tR = thr_float(misc[M_THR + static_cast<uint32_t>(SK_RAW)]);
        const float tL = thr_float(misc[M_THR + static_cast<uint32_t>(SK_ALLOWED)]);
        const bool need_raw = tg.need[SK_RAW] > 0;
        const float tAR = fminf(tA, tR);  // a non-penalized entry serves the window and the raw top-n
        // close-up: every thread takes its share of the groups into
        // registers, then, after a barrier (the candidate buffer overlaps the group area), writes the
        // ids that pass the final thresholds as buffer entries: not
        // penalized on their values; penalized ones, when the penalized list
        // is filed here, on their penalized values (and into the list on
        // their raw values, when they can be among the raw top-n).
        const uint32_t ng = ovf0 ? 0u : min(lds_gctr()[G_FILL] & 0xFFFFu, kG4Cap);  // every reserved group is written
        constexpr uint32_t kHeld = kG4Held;
        float4 hv[kHeld];
        uint32_t ht[kHeld];
#pragma unroll
        for (uint32_t q = 0; q < kHeld; q++) {
            const uint32_t i = tid + q * kBlock;
            ht[q] = 0xFFFFFFFFu;
            hv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (i < ng) {
                hv[q] = lds_g4val()[i];
                ht[q] = lds_g4tag()[i];
            }
        }
        if (tid == 0) misc[M_BUFN] = 0u;
        TSM_LDS_SYNC();
        // this thread's entries, counted, then written at the wave's places
        auto pen_bits = [&](uint32_t id0) -> uint32_t {
            return pen_lookup ? (lds_bitmap()[id0 >> 5] >> (id0 & 31u)) & 0xFu : 0u;
        };
        uint32_t nb_mine = 0, np_mine = 0;
#pragma unroll
        for (uint32_t q = 0; q < kHeld; q++) {
            if (ht[q] == 0xFFFFFFFFu) continue;
            const uint32_t id0 = ht[q] & kEntId, pb = pen_bits(id0);
#pragma unroll
            for (uint32_t c = 0; c < 4u; c++) {
                const uint32_t id = id0 + c;
                if (id >= n) continue;
                const float y = g4_at(hv[q], c);
                const bool al = (ht[q] >> (kG4Nib + c)) & 1u;
                if (!((pb >> c) & 1u)) {
                    nb_mine += keep2(y, al, tAR, tL) ? 1u : 0u;
                } else if (file_pen) {
                    np_mine += (need_raw && y >= tR) ? 1u : 0u;
                    nb_mine += keep2(penalize(y, history_count(id), m, P), al, tA, tL) ? 1u : 0u;
                }
            }
        }
        const uint32_t wb = wave_incl_scan(nb_mine), wp = wave_incl_scan(np_mine);
        uint32_t bat = 0, pat = 0;
        if (lane == kWave - 1) {
            if (wb) bat = atomicAdd(&misc[M_BUFN], wb);
            if (wp) pat = atomicAdd(&misc[M_PENN], wp);
        }
        bat = wave_read(bat, kWave - 1) + wb - nb_mine;
        pat = wave_read(pat, kWave - 1) + wp - np_mine;
        if (nb_mine | np_mine) {
#pragma unroll
            for (uint32_t q = 0; q < kHeld; q++) {
                if (ht[q] == 0xFFFFFFFFu) continue;
                const uint32_t id0 = ht[q] & kEntId, pb = pen_bits(id0);
#pragma unroll
                for (uint32_t c = 0; c < 4u; c++) {
                    const uint32_t id = id0 + c;
                    if (id >= n) continue;
                    const float y = g4_at(hv[q], c);
                    const bool al = (ht[q] >> (kG4Nib + c)) & 1u;
                    const uint32_t alf = al ? kEntAllowed : 0u;
                    if (!((pb >> c) & 1u)) {
                        if (keep2(y, al, tAR, tL)) {
                            if (bat < kBufCap) buf[bat] = make_uint2(__float_as_uint(y), id | alf);
                            bat++;
                        }
                    } else if (file_pen) {
                        if (need_raw && y >= tR) {
                            if (pat < kPenCap) pen[pat] = make_uint2(__float_as_uint(y), id | alf);
                            pat++;
                        }
                        const float yp = penalize(y, history_count(id), m, P);
                        if (keep2(yp, al, tA, tL)) {
                            if (bat < kBufCap) buf[bat] = make_uint2(__float_as_uint(yp), id | kEntPen | alf);
                            bat++;
                        }
                    }
                }
            }
        }
        TSM_LDS_SYNC();
        // a gathered penalized list: its ids join the candidates when their
        // penalized value passes the final thresholds (every element at or
        // above them is then in the buffer)
        if (track_pen && ovf0 == 0u && misc[M_BUFN] <= kBufCap) {
            const uint32_t penn = min(penn0, kPenCap);
            for (uint32_t i = tid; i < penn; i += kBlock) {
                const uint2 e = pen[i];
                const uint32_t id = e.y & kEntId;
                const float y = penalize(__uint_as_float(e.x), history_count(id), m, P);
                const bool al = (e.y & kEntAllowed) != 0u;
                if (keep2(y, al, tA, tL)) {
                    const uint32_t pos = atomicAdd(&misc[M_BUFN], 1u);
                    if (pos < kBufCap) buf[pos] = make_uint2(__float_as_uint(y), id | kEntPen | (al ? kEntAllowed : 0u));
                }
            }
            TSM_LDS_SYNC();
        }
        const uint32_t fill = misc[M_BUFN];
        if (tid == 0 && (fill > kBufCap || misc[M_OVF] != 0u || misc[M_PENN] > kPenCap)) misc[M_FLAGS] |= ROWF_BUF_OVERFLOW;
        bufn = min(fill, kBufCap);
    }
    // a NaN logit (or +inf, whose steps make the sum NaN as well; the serial
    // path is exact for those rows too) leaves a logprobs row's sum NaN
    if (wave_ballot(m.logprobs && !(lse.sum == lse.sum)) && lane == 0) lds_nan_wave()[wid] = 1u;
    // the finish: one wave for the common rows, the whole block otherwise
    TSM_LDS_SYNC();
    const uint32_t flags = misc[M_FLAGS];
    if constexpr (kLean) {
        // the single-wave finish; the rare rows it cannot take go through the
        // out-of-line general finishes (their arguments through LDS)
        // (a lean row writes no distribution: its pointers are not passed,
        // so they need not stay live through the row)
        if (row_has_nan()) {
            if (tid == 0) {
                nan_call()->a = a;
                nan_call()->a.dist_ids = nullptr;
                nan_call()->a.dist_probs = nullptr;
                nan_call()->f = f;
                nan_call()->nlp = nlp;
            }
            TSM_LDS_SYNC();
            finish_nan_call();
            return;
        }
        if (!(flags & (ROWF_BUF_OVERFLOW | ROWF_SLOW_HISTORY)) &&
            finish_wave(a, f, tg0, nlp, lse.ref, lse.sum, nallow, bufn))
            return;
        if (tid == 0) {
            row_call()->a = a;
            row_call()->a.dist_ids = nullptr;
            row_call()->a.dist_probs = nullptr;
            row_call()->f = f;
            row_call()->tg0 = tg0;
            row_call()->nlp = nlp;
            row_call()->bufn = bufn;
        }
        TSM_LDS_SYNC();
        finish_row_call(lse.ref, lse.sum, nallow);
    } else {
    if (m.topk && row_has_nan()) {
        if (tid == 0) {
            nan_call()->a = a;
            nan_call()->f = f;
            nan_call()->nlp = nlp;
        }
        TSM_LDS_SYNC();
        finish_nan_call();
        return;
    }
    if (tracking && !(flags & (ROWF_BUF_OVERFLOW | ROWF_SLOW_HISTORY)) && m.topk && !a.distribution &&
        m.want <= kWaveList && nlp <= kWaveList) {
        if (finish_wave(a, f, tg0, nlp, lse.ref, lse.sum, nallow, bufn)) return;
    }
    finish_row(a, f, tg0, nlp, lse.ref, lse.sum, nallow, bufn);
    }
}

// The general kernel: every row kind (re-reads, exact nucleus folds, NaN
// rows, the block finish).
template <bool kVecLoads>
__global__ __launch_bounds__(kBlock) void sample_kernel(SampleArgs a) {
    sample_row<kVecLoads, false>(a);
}
// The lean kernel: the common top-k rows only (lean_takes).  Without the
// general path inlined, the stream and the single-wave finish keep their
// state in registers (no scratch).
template <bool kVecLoads>
__global__ __launch_bounds__(kBlock) void topk_kernel(SampleArgs a) {
    sample_row<kVecLoads, true>(a);
}

template __global__ void sample_kernel<true>(SampleArgs);
template __global__ void sample_kernel<false>(SampleArgs);
template __global__ void topk_kernel<true>(SampleArgs);
template __global__ void topk_kernel<false>(SampleArgs);

void launch_sample(const SampleArgs& a_in, uint32_t rows, bool vec_loads, bool lean, bool general,
                   hipStream_t stream) {
    SampleArgs a = a_in;
    a.skip_lean = lean ? 1u : 0u;
    a.general = general ? 1u : 0u;
    if (lean) {
        if (vec_loads)
            hipLaunchKernelGGL(topk_kernel<true>, dim3(rows), dim3(kBlock), kSmem, stream, a);
        else
            hipLaunchKernelGGL(topk_kernel<false>, dim3(rows), dim3(kBlock), kSmem, stream, a);
    }
    if (general) {
        if (vec_loads)
            hipLaunchKernelGGL(sample_kernel<true>, dim3(rows), dim3(kBlock), kSmem, stream, a);
        else
            hipLaunchKernelGGL(sample_kernel<false>, dim3(rows), dim3(kBlock), kSmem, stream, a);
    }
}

hipError_t sample_set_smem_attr() {
    const void* ks[4] = {reinterpret_cast<const void*>(&sample_kernel<true>),
                         reinterpret_cast<const void*>(&sample_kernel<false>),
                         reinterpret_cast<const void*>(&topk_kernel<true>),
                         reinterpret_cast<const void*>(&topk_kernel<false>)};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 4 && e == hipSuccess; i++)
        e = hipFuncSetAttribute(ks[i], hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kSmem));
    return e;
}

}  // namespace tsm
