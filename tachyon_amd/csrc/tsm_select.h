// tsm_select.h - order statistics over one row for a 1024-thread workgroup:
// the row re-read machinery (radix select in LDS over the row held in HBM /
// L2 / MALL, mass selection for big nucleus sets) and the exact finish of a
// ranked candidate list (the reference's sequential f32 arithmetic).
//
// A re-read streams the row in 16384-id tiles and answers order-statistic
// questions with 11-bit LDS histograms:
//   * select_kth: the k-th element in (value desc, id asc) order (radix);
//   * mass selection: the first element whose cumulative probability reaches
//     a target, with f64 partial sums, used when more than 1024 candidates
//     remain.  Value bins (counts and masses per bin of (y0 - y) / t) find
//     the bin that holds the target and one gather resolves it; radix rounds
//     (mass_select) decide where a bin holds too many equal values.
// When at most 1024 candidates remain they are gathered, sorted and finished
// by exact_finalize, which reproduces the CPU sampler's roundings.
#pragma once

#include "tsm_device.h"

namespace tsm {

// ---- LDS layout of the sampling workgroup (bytes) -----------------------------
// Region A holds the streaming pass's history lookup (a bitmap of the ids in
// the row's history and an open-addressing table of their counts) and, once
// the stream is done, the finish's ranked lists and the re-read's per-tile
// history counts.  The histograms, the candidate buffer, the penalized list
// and the scalars have their own regions.
constexpr uint32_t kReTile = 16384;        // ids per tile of a re-read pass
constexpr uint32_t kBitmapWords = 8192;    // history bitmap: rows of up to 262144 ids
constexpr uint32_t kHashSlots = 4096;      // history count table (histories up to kHistFast ids)
constexpr uint32_t kHistFast = kHashSlots / 2;
constexpr uint32_t kBufCap = 6144;         // candidate buffer entries (y bits, id | flags)
constexpr uint32_t kPenCap = 2048;         // penalized-id list entries (raw x bits, id)
constexpr uint32_t kOffBitmap = 0;                              // u32[kBitmapWords]
constexpr uint32_t kOffHashKey = kOffBitmap + kBitmapWords * 4;  // u32[kHashSlots]: id + 1, 0 = empty
constexpr uint32_t kOffHashCnt = kOffHashKey + kHashSlots * 4;   // u32[kHashSlots]
constexpr uint32_t kOffCnt = 0;                                  // u16 history counts of one re-read tile
constexpr uint32_t kOffRank = kOffCnt + kReTile * 2;             // ry, rid, rp [kExactCap]
constexpr uint32_t kOffGather = kOffRank + kExactCap * 12;       // rP, rq [kExactCap] | gcomp u64[kExactCap]
constexpr uint32_t kRegionA = 65536;
static_assert(kOffHashCnt + kHashSlots * 4 <= kRegionA && kOffGather + kExactCap * 8 <= kRegionA, "region A");
constexpr uint32_t kOffHist = kRegionA;                          // 3 x u32[kBins] | hcnt u32[kBins] + hmass f64[kBins]
constexpr uint32_t kOffBuf = kOffHist + kBins * 12;              // uint2[kBufCap]
constexpr uint32_t kOffPen = kOffBuf + kBufCap * 8;              // uint2[kPenCap]
constexpr uint32_t kOffMisc = kOffPen + kPenCap * 8;             // u32[64]
constexpr uint32_t kOffMiscD = kOffMisc + 64 * 4;                // f64[32]
constexpr uint32_t kOffTmp = kOffMiscD + 32 * 8;                 // u32[64] scan scratch
constexpr uint32_t kSBins = 512;                                 // stream histogram bins per threshold
constexpr uint32_t kOffSHist = kOffTmp + 64 * 4;                 // 2 x u32[kSBins]
constexpr uint32_t kOffSeg = kOffSHist + 2 * kSBins * 4;         // per wave: published fill, counted fill
constexpr uint32_t kSmem = kOffSeg + 2 * (kBlock / kWave) * 4;
static_assert(kOffGather % 8 == 0 && (kOffHist + kBins * 4) % 8 == 0 && kOffBuf % 8 == 0 && kOffPen % 8 == 0 &&
                  kOffMiscD % 8 == 0,
              "u64 / f64 LDS records are 8-byte aligned");
static_assert(kSmem <= 160 * 1024, "LDS budget");

enum : uint32_t {  // misc word indices
    M_FIND = 0,     // 2 words
    M_FIND2 = 2,    // 2 words
    M_CNT = 4,
    M_FIRST = 5,
    M_TOTAL = 6,
    M_TOKEN = 7,
    M_KEEP = 8,
    M_PROB = 9,
    M_MASS = 10,
    M_BUFN = 11,    // candidate buffer fill
    M_PENN = 12,    // penalized list fill (may exceed kPenCap: overflow)
    M_FLAGS = 13,   // ROWF_* bits
    M_VBAD = 14,    // a value-bin pass met a NaN
    M_THR = 16,     // 3 stream thresholds (canon keys): all, raw, allowed
    M_OVF = 19,     // nonzero once a reservation ran past the candidate buffer
    M_SEL = 20,     // 3 x 2 hist_find3 results
    M_RED = 32,     // 32 words of reduction results
};

enum : uint8_t { ORD_CANON_Y = 0, ORD_TOTAL_Y = 1, ORD_CANON_X = 2 };

struct Filt {
    uint8_t order = ORD_CANON_Y;
    bool need_allowed = false;
    bool use_cut = false;
    bool use_max = false;
    bool use_minp = false;
    float cut = 0.0f;
    uint64_t max_comp = ~0ull;
    float y0 = 0.0f;
    float minp = 0.0f;
    // min-p band: y >= minp_hi is kept and y < minp_lo dropped without the
    // exponential; only values in between evaluate it
    float minp_lo = 0.0f, minp_hi = 0.0f;
};

// One row being finished: its global inputs and settings.  LDS structures are
// reached through accessors at fixed offsets from lds_base().
struct Fin {
    const float* rowp;
    const uint32_t* mrow;
    const uint32_t* hist;
    uint32_t hlen, n;
    float u;  // the row's uniform draw (0 for distribution())
    RowMode m;
    tsm_row_params P;
    __device__ __forceinline__ uint32_t* cnt() const { return reinterpret_cast<uint32_t*>(lds_base() + kOffCnt); }
    __device__ __forceinline__ float* ry() const { return reinterpret_cast<float*>(lds_base() + kOffRank); }
    __device__ __forceinline__ uint32_t* rid() const {
        return reinterpret_cast<uint32_t*>(lds_base() + kOffRank + kExactCap * 4);
    }
    __device__ __forceinline__ float* rp() const {
        return reinterpret_cast<float*>(lds_base() + kOffRank + kExactCap * 8);
    }
    __device__ __forceinline__ float* rP() const { return reinterpret_cast<float*>(lds_base() + kOffGather); }
    __device__ __forceinline__ float* rq() const {
        return reinterpret_cast<float*>(lds_base() + kOffGather + kExactCap * 4);
    }
    __device__ __forceinline__ uint64_t* gcomp() const {
        return reinterpret_cast<uint64_t*>(lds_base() + kOffGather);
    }
    __device__ __forceinline__ uint32_t* hcnt() const { return reinterpret_cast<uint32_t*>(lds_base() + kOffHist); }
    __device__ __forceinline__ double* hmass() const {
        return reinterpret_cast<double*>(lds_base() + kOffHist + kBins * 4);
    }
    __device__ __forceinline__ uint32_t* misc() const { return reinterpret_cast<uint32_t*>(lds_base() + kOffMisc); }
    __device__ __forceinline__ double* miscd() const { return reinterpret_cast<double*>(lds_base() + kOffMiscD); }
    __device__ __forceinline__ uint32_t* tmp() const { return reinterpret_cast<uint32_t*>(lds_base() + kOffTmp); }
};

__device__ __forceinline__ bool allowed_bit(const Fin& f, uint32_t id) {
    return (f.mrow[id >> 5] >> (id & 31u)) & 1u;
}

__device__ __forceinline__ uint64_t comp_of(uint8_t order, uint32_t id, float x, float y) {
    const uint32_t k = order == ORD_CANON_Y ? canon_key(y) : order == ORD_TOTAL_Y ? total_key(y) : canon_key(x);
    return composite(k, id);
}

__device__ __forceinline__ bool keep_el(const Fin& f, const Filt& q, uint32_t id, float y, uint64_t c) {
    if (q.need_allowed && !allowed_bit(f, id)) return false;
    if (q.use_cut && !(y >= q.cut)) return false;
    if (q.use_max && c > q.max_comp) return false;
    if (q.use_minp) {
        if (y < q.minp_lo) return false;
        if (!(y >= q.minp_hi) && !(glibc_expf((y - q.y0) / f.m.t) >= q.minp)) return false;
    }
    return true;
}

// One re-read of the row in tiles; fn(id, raw, penalized) for every id.  Each
// thread loads G elements before it processes them, so G loads are in flight
// per thread (G > 1 for the passes that dominate a long re-read path).
template <int G = 1, class F>
__device__ void row_pass(Fin& f, F&& fn) {
    const uint32_t tid = threadIdx.x;
    const uint32_t n = f.n;
    const bool penal = f.m.penal;
    const TSM_GLOBAL_AS float* rowp = global_as(f.rowp);
    const TSM_GLOBAL_AS uint32_t* hist = global_as(f.hist);
    const uint32_t hc = min(f.hlen, TSM_MAX_HISTORY);
    for (uint32_t tb = 0; tb < n; tb += kReTile) {
        const uint32_t tl = min(kReTile, n - tb);
        if (penal) {
            TSM_LDS_SYNC();
            for (uint32_t i = tid; i < kReTile / 2; i += kBlock) f.cnt()[i] = 0;
            TSM_LDS_SYNC();
            for (uint32_t h = tid; h < hc; h += kBlock) {
                const uint32_t li = hist[h] - tb;
                if (li < tl) atomicAdd(&f.cnt()[li >> 1], 1u << ((li & 1u) << 4));
            }
            TSM_LDS_SYNC();
        }
        for (uint32_t i0 = tid; i0 < tl; i0 += G * kBlock) {
            float xs[G];
#pragma unroll
            for (int k = 0; k < G; k++) {
                const uint32_t i = i0 + static_cast<uint32_t>(k) * kBlock;
                xs[k] = i < tl ? rowp[tb + i] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < G; k++) {
                const uint32_t i = i0 + static_cast<uint32_t>(k) * kBlock;
                if (i < tl) {
                    const uint32_t id = tb + i;
                    const float x = xs[k];
                    float y = x;
                    if (penal) {
                        const uint32_t c = (f.cnt()[i >> 1] >> ((i & 1u) << 4)) & 0xFFFFu;
                        if (c) y = penalize(x, c, f.m, f.P);
                    }
                    fn(id, x, y);
                }
            }
        }
    }
    TSM_LDS_SYNC();
}

// Block-wide bitonic sort, ascending, of n u64 (n a power of two <= 4096).
__device__ void bitonic_sort(uint64_t* a, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += kBlock) {
                const uint32_t ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t x = a[i], y = a[ixj];
                    const bool up = (i & k) == 0;
                    if ((x > y) == up) {
                        a[i] = y;
                        a[ixj] = x;
                    }
                }
            }
            TSM_LDS_SYNC();
        }
}

__device__ __forceinline__ uint32_t pow2_ceil(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Counts filtered elements (one pass).
template <int G = 1>
__device__ __forceinline__ uint32_t count_pass(Fin& f, const Filt& q) {
    uint32_t local = 0;
    row_pass<G>(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) local++;
    });
    return block_sum<kBlock>(local, f.tmp());
}

// Radix rounds over the 64-bit composite (~key << 32 | id, ids < 2^22): bits
// [lo, lo + width) per round; bits 22..31 are always zero and are skipped.
__constant__ int kRoundLo[5] = {53, 42, 32, 11, 0};
__constant__ int kRoundW[5] = {11, 11, 10, 11, 11};

// Count-based select starting at round r0 with the bits at and above
// position `known_lo` fixed to those of `known`.  Returns T such that exactly
// `need` filtered elements sharing those bits have composite <= T, or ~0 if
// fewer than `need` exist.
__device__ __forceinline__ uint64_t select_from(Fin& f, const Filt& q, uint32_t need, int r0, uint64_t known,
                                int known_lo) {
    const uint32_t tid = threadIdx.x;
    for (int r = r0; r < 5; r++) {
        const int lo = kRoundLo[r], w = kRoundW[r];
        for (uint32_t i = tid; i < kBins; i += kBlock) f.hcnt()[i] = 0;
        if (tid < 2) f.misc()[M_FIND + tid] = 0xFFFFFFFFu;
        TSM_LDS_SYNC();
        const uint64_t kn = known;
        const int kl = known_lo;
        row_pass(f, [&](uint32_t id, float x, float y) {
            const uint64_t c = comp_of(q.order, id, x, y);
            if ((kl >= 64 || (c >> kl) == (kn >> kl)) && keep_el(f, q, id, y, c))
                atomicAdd(&f.hcnt()[(c >> lo) & ((1u << w) - 1u)], 1u);
        });
        hist_find<kBlock>(f.hcnt(), need, f.tmp(), f.misc() + M_FIND);
        const uint32_t d = f.misc()[M_FIND];
        if (d == 0xFFFFFFFFu) return ~0ull;
        const uint32_t before = f.misc()[M_FIND + 1];
        const uint32_t binc = f.hcnt()[d];
        TSM_LDS_SYNC();
        known |= static_cast<uint64_t>(d) << lo;
        known_lo = lo;
        need -= before;
        if (binc == need) return lo == 0 ? known : (known | ((1ull << lo) - 1ull));
    }
    return known;
}

__device__ __forceinline__ uint64_t select_kth(Fin& f, const Filt& q, uint32_t k) {
    return select_from(f, q, k, 0, 0, 64);
}

// The filtered element with the largest composite <= T, or ~0 when there is
// none.  select_kth / mass_select return a threshold whose low bits may be
// padding; this resolves it to the element itself (its id is the low word).
__device__ __forceinline__ uint64_t exact_at(Fin& f, const Filt& q, uint64_t T) {
    unsigned long long best = 0;
    uint32_t any = 0;
    row_pass(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (c <= T && keep_el(f, q, id, y, c) && (!any || c > best)) {
            best = c;
            any = 1;
        }
    });
    best = any ? best + 1ull : 0ull;  // 0 = nothing; composites fit below ~0
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long w = __shfl_xor(best, o, kWave);
        best = w > best ? w : best;
    }
    unsigned long long* wtmp = reinterpret_cast<unsigned long long*>(f.miscd() + 8);
    if ((threadIdx.x & (kWave - 1)) == 0) wtmp[threadIdx.x / kWave] = best;
    TSM_LDS_SYNC();
    unsigned long long all = 0;
    for (int w = 0; w < kBlock / kWave; w++) all = wtmp[w] > all ? wtmp[w] : all;
    TSM_LDS_SYNC();
    return all == 0 ? ~0ull : all - 1ull;
}

// Block-wide exclusive f64 scan (1024 threads).
__device__ double block_excl_scan_f64(double v, double* tmp, double* total) {
    constexpr int NW = kBlock / kWave;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    double inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const double w = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += w;
    }
    if (lane == kWave - 1) tmp[wid] = inc;
    TSM_LDS_SYNC();
    double before = 0.0, all = 0.0;
    for (int w = 0; w < NW; w++) {
        const double t = tmp[w];
        if (w < wid) before += t;
        all += t;
    }
    TSM_LDS_SYNC();
    *total = all;
    return before + inc - v;
}

struct MassSel {
    uint64_t T;
    double cum;     // cumulative probability through T
    uint32_t rank;  // elements through T
};

// First filtered element, in (value desc, id asc) order, whose inclusive
// cumulative p = exp((y - y0) / t) reaches `target`.
__device__ __noinline__ MassSel mass_select(Fin& f_in, const Filt& q_in, float y0, double target) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const uint32_t tid = threadIdx.x;
    uint64_t known = 0;
    int known_lo = 64;
    double cum_before = 0.0;
    uint32_t cnt_before = 0;
    double* dtmp = f.miscd() + 8;
    for (int r = 0; r < 3; r++) {
        const int lo = kRoundLo[r], w = kRoundW[r];
        for (uint32_t i = tid; i < kBins; i += kBlock) {
            f.hcnt()[i] = 0;
            f.hmass()[i] = 0.0;
        }
        if (tid == 0) {
            f.misc()[M_FIND] = 0xFFFFFFFFu;
            f.misc()[M_FIND2] = 0;
        }
        TSM_LDS_SYNC();
        const uint64_t kn = known;
        const int kl = known_lo;
        row_pass(f, [&](uint32_t id, float x, float y) {
            const uint64_t c = comp_of(q.order, id, x, y);
            if ((kl >= 64 || (c >> kl) == (kn >> kl)) && keep_el(f, q, id, y, c)) {
                const uint32_t d = (c >> lo) & ((1u << w) - 1u);
                atomicAdd(&f.hcnt()[d], 1u);
                atomicAdd(&f.hmass()[d], static_cast<double>(glibc_expf((y - y0) / f.m.t)));
            }
        });
        // thread t owns bins 2t, 2t+1
        const uint32_t b0 = 2 * tid;
        const uint32_t c0 = f.hcnt()[b0], c1 = f.hcnt()[b0 + 1];
        const double m0 = f.hmass()[b0], m1 = f.hmass()[b0 + 1];
        double mtot;
        const double mb = block_excl_scan_f64(m0 + m1, dtmp, &mtot);
        uint32_t ctot;
        const uint32_t cb = block_excl_scan<kBlock>(c0 + c1, f.tmp(), &ctot);
        const double base = cum_before + mb;
        uint32_t cand = 0xFFFFFFFFu;
        if (c0 > 0 && base + m0 >= target) cand = b0;
        else if (c1 > 0 && base + m0 + m1 >= target) cand = b0 + 1;
        if (cand != 0xFFFFFFFFu) atomicMin(&f.misc()[M_FIND], cand);
        if (c0 + c1 > 0) atomicMax(&f.misc()[M_FIND2], (c1 > 0 ? b0 + 1 : b0) + 1);  // last nonempty + 1
        TSM_LDS_SYNC();
        uint32_t d = f.misc()[M_FIND];
        const bool overshoot = d == 0xFFFFFFFFu;  // read now: select_from below rewrites M_FIND
        if (overshoot) d = f.misc()[M_FIND2] - 1;   // target beyond the total: last element
        if ((d >> 1) == tid) {
            const bool second = d & 1u;
            f.miscd()[0] = base + (second ? m0 : 0.0);
            f.misc()[M_CNT] = cb + (second ? c0 : 0u);
            f.misc()[M_TOTAL] = second ? c1 : c0;
        }
        TSM_LDS_SYNC();
        cum_before = f.miscd()[0];
        cnt_before += f.misc()[M_CNT];
        const uint32_t ties = f.misc()[M_TOTAL];
        known |= static_cast<uint64_t>(d) << lo;
        known_lo = lo;
        TSM_LDS_SYNC();
        if (r == 2) {
            // key resolved: all `ties` elements share one value and one p
            const uint32_t key = ~static_cast<uint32_t>(known >> 32);
            const float yk = key_to_float(key);
            const double pk = static_cast<double>(glibc_expf((yk - y0) / f.m.t));
            double need_d = pk > 0.0 ? ceil((target - cum_before) / pk) : 1.0;
            uint32_t need = need_d < 1.0 ? 1u : (need_d > static_cast<double>(ties) ? ties : static_cast<uint32_t>(need_d));
            if (overshoot) need = ties;  // take the last
            MassSel s;
            s.T = (need == ties) ? (known | 0xFFFFFFFFull) : select_from(f, q, need, 3, known, 32);
            s.cum = cum_before + static_cast<double>(need) * pk;
            s.rank = cnt_before + need;
            return s;
        }
    }
    return MassSel{};  // not reached
}

// Sum of p over the filtered elements (f64) and their count.
__device__ __forceinline__ double mass_total(Fin& f, const Filt& q, float y0) {
    double local = 0.0;
    row_pass(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) local += static_cast<double>(glibc_expf((y - y0) / f.m.t));
    });
    double tot;
    block_excl_scan_f64(local, f.miscd() + 8, &tot);
    return tot;
}

// Gathers filtered elements' composites into gcomp (caller guarantees <= cap).
template <int G = 1>
__device__ __forceinline__ uint32_t gather_pass(Fin& f, const Filt& q, uint32_t cap) {
    if (threadIdx.x == 0) f.misc()[M_CNT] = 0;
    TSM_LDS_SYNC();
    row_pass<G>(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) {
            const uint32_t pos = atomicAdd(&f.misc()[M_CNT], 1u);
            if (pos < cap) f.gcomp()[pos] = c;
        }
    });
    const uint32_t n = min(f.misc()[M_CNT], cap);
    TSM_LDS_SYNC();
    return n;
}

// Sorts a[0..n) ascending; n <= 1024 and a has room for pow2_ceil(n)
// entries.  Up to 64 entries are sorted by wave 0 in registers (no block
// barrier inside); longer lists by the whole block in LDS.
__device__ void sort_u64(uint64_t* a, uint32_t n) {
    const uint32_t tid = threadIdx.x;
    if (n <= static_cast<uint32_t>(kWave)) {
        if (tid < kWave) {
            unsigned long long v = tid < n ? a[tid] : ~0ull;
#pragma unroll
            for (uint32_t k = 2; k <= static_cast<uint32_t>(kWave); k <<= 1)
#pragma unroll
                for (uint32_t j = k >> 1; j > 0; j >>= 1) {
                    const unsigned long long o = __shfl_xor(v, static_cast<int>(j), kWave);
                    const bool keep_min = ((tid & j) == 0) == ((tid & k) == 0);
                    v = keep_min ? (o < v ? o : v) : (o > v ? o : v);
                }
            if (tid < n) a[tid] = v;
        }
        TSM_LDS_SYNC();
        return;
    }
    const uint32_t n2 = pow2_ceil(n);
    for (uint32_t i = n + tid; i < n2; i += kBlock) a[i] = ~0ull;
    TSM_LDS_SYNC();
    bitonic_sort(a, n2);
}

// Sorts gcomp[0..n) and unpacks it into the ranked arrays (ids in the low word).
__device__ void sort_gathered(Fin& f, uint32_t n) {
    sort_u64(f.gcomp(), n);
    for (uint32_t j = threadIdx.x; j < n; j += kBlock) {
        const uint64_t c = f.gcomp()[j];
        f.ry()[j] = key_to_float(~static_cast<uint32_t>(c >> 32));
        f.rid()[j] = static_cast<uint32_t>(c);
    }
    TSM_LDS_SYNC();
}

// Sorts a[0..n) ascending, n <= kBlock distinct values: each thread ranks
// its value by counting the smaller ones (broadcast LDS reads, no barrier per
// stage as in a bitonic sort) and stores it at its rank.
__device__ __forceinline__ void rank_sort_u64(uint64_t* a, uint32_t n) {
    const uint32_t tid = threadIdx.x;
    uint64_t v = 0;
    uint32_t r = 0;
    if (tid < n) {
        v = a[tid];
        for (uint32_t j = 0; j < n; j++) r += a[j] < v ? 1u : 0u;
    }
    TSM_LDS_SYNC();
    if (tid < n) a[r] = v;
    TSM_LDS_SYNC();
}

constexpr int kNucGroup = 4;  // loads in flight per thread in the nucleus passes

// ---- value-binned mass selection -------------------------------------------------
// The nucleus of a row without top-k holds up to the whole vocabulary.  Its
// mass selections (top-p, then the draw among the kept) bin the filtered
// elements by value: bin(y) = floor((y0 - y) * mul), clamped to [0, kBins).
// (y0 - y) * mul is monotone in y, so ascending bins visit the elements in
// (value desc) order and equal values share a bin.  One pass builds the
// counts and f64 masses p = exp((y - y0) / t) per bin; the bin where the
// cumulative mass reaches the target is then gathered (at most kExactCap
// elements), sorted, and resolved with an f64 prefix sum.  A bin with more
// elements is split once more into kBins sub-bins by the fraction of
// (y0 - y) * mul, which is exact for a non-clamped bin; a sub-bin that is
// still too big (many equal values) is left to the radix selections.
struct VBins {
    float y0, mul;
    __device__ __forceinline__ float pos(float y) const { return (y0 - y) * mul; }
    __device__ __forceinline__ uint32_t bin(float y) const {
        const float d = pos(y);
        return d >= static_cast<float>(kBins - 1) ? kBins - 1u : (d > 0.0f ? static_cast<uint32_t>(d) : 0u);
    }
    // level-2 index of y inside bin b < kBins - 1, where pos(y) - b in [0, 1) is exact
    __device__ __forceinline__ uint32_t sub(float y, uint32_t b) const {
        const float fr = (pos(y) - static_cast<float>(b)) * static_cast<float>(kBins);
        return fr >= static_cast<float>(kBins - 1) ? kBins - 1u : (fr > 0.0f ? static_cast<uint32_t>(fr) : 0u);
    }
};
static_assert(kBins == 2 * kBlock, "two bins per thread");

// Counts and f64 masses of the filtered elements per bin (level 1), or per
// sub-bin of bin b1 (level 2).  Returns false when a filtered value is NaN.
__device__ __noinline__ bool vbin_hist(Fin& f_in, const Filt& q_in, const VBins& vb_in, bool level2, uint32_t b1) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const VBins vb = vb_in;
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < kBins; i += kBlock) {
        f.hcnt()[i] = 0;
        f.hmass()[i] = 0.0;
    }
    if (tid == 0) f.misc()[M_VBAD] = 0;
    TSM_LDS_SYNC();
    // bin masses locate a target's bin and give the mass before it; they use
    // the hardware exp2 (relative error of a term below 3e-6, largest for the
    // smallest terms), while the elements of the bin that is resolved are
    // summed from exact glibc_expf terms
    const float l2t = 1.4426950408889634f / f.m.t;
    uint32_t bad = 0;
    row_pass<kNucGroup>(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (!keep_el(f, q, id, y, c)) return;
        uint32_t b = vb.bin(y);
        if (level2) {
            if (b != b1) return;
            b = vb.sub(y, b1);
        }
        bad |= y != y;
        atomicAdd(&f.hcnt()[b], 1u);
        atomicAdd(&f.hmass()[b], static_cast<double>(__builtin_amdgcn_exp2f((y - vb.y0) * l2t)));
    });
    if (bad) f.misc()[M_VBAD] = 1u;
    TSM_LDS_SYNC();
    const bool ok = f.misc()[M_VBAD] == 0;
    TSM_LDS_SYNC();
    return ok;
}

// Element count and f64 mass of the histogram.
__device__ __forceinline__ uint32_t vbin_totals(Fin& f, double* mass) {
    const uint32_t b0 = 2 * threadIdx.x;
    block_excl_scan_f64(f.hmass()[b0] + f.hmass()[b0 + 1], f.miscd() + 8, mass);
    return block_sum<kBlock>(f.hcnt()[b0] + f.hcnt()[b0 + 1], f.tmp());
}

struct BinHit {
    uint32_t bin;       // kBins: the histogram is empty
    uint32_t cnt;       // elements in the bin
    uint32_t before_n;  // elements in earlier bins
    double before;      // base + the mass of earlier bins
};

// The first non-empty bin whose cumulative mass (from base) reaches target,
// or the last non-empty bin when none does.
__device__ __forceinline__ BinHit vbin_find(Fin& f, double base, double target) {
    const uint32_t tid = threadIdx.x;
    const uint32_t b0 = 2 * tid;
    const uint32_t c0 = f.hcnt()[b0], c1 = f.hcnt()[b0 + 1];
    const double m0 = f.hmass()[b0], m1 = f.hmass()[b0 + 1];
    if (tid == 0) {
        f.misc()[M_FIND] = 0xFFFFFFFFu;
        f.misc()[M_FIND2] = 0;
    }
    double mtot;
    const double mb = block_excl_scan_f64(m0 + m1, f.miscd() + 8, &mtot);  // barriers order the init above
    uint32_t ctot;
    const uint32_t cb = block_excl_scan<kBlock>(c0 + c1, f.tmp(), &ctot);
    const double bs = base + mb;
    uint32_t cand = 0xFFFFFFFFu;
    if (c0 > 0 && bs + m0 >= target) cand = b0;
    else if (c1 > 0 && bs + m0 + m1 >= target) cand = b0 + 1;
    if (cand != 0xFFFFFFFFu) atomicMin(&f.misc()[M_FIND], cand);
    if (c0 + c1 > 0) atomicMax(&f.misc()[M_FIND2], (c1 > 0 ? b0 + 1 : b0) + 1);
    TSM_LDS_SYNC();
    uint32_t d = f.misc()[M_FIND];
    if (d == 0xFFFFFFFFu) d = f.misc()[M_FIND2] == 0 ? kBins : f.misc()[M_FIND2] - 1;
    if (d < kBins && (d >> 1) == tid) {
        const bool second = d & 1u;
        f.miscd()[0] = bs + (second ? m0 : 0.0);
        f.misc()[M_CNT] = cb + (second ? c0 : 0u);
        f.misc()[M_TOTAL] = second ? c1 : c0;
    }
    TSM_LDS_SYNC();
    BinHit h;
    h.bin = d;
    h.cnt = d < kBins ? f.misc()[M_TOTAL] : 0u;
    h.before_n = d < kBins ? f.misc()[M_CNT] : ctot;
    h.before = d < kBins ? f.miscd()[0] : base + mtot;
    TSM_LDS_SYNC();
    return h;
}

// vbin_find for two targets (from base 0) with one scan of the bins.
__device__ __forceinline__ void vbin_find2(Fin& f, double ta, double tb, BinHit* ha, BinHit* hb) {
    const uint32_t tid = threadIdx.x;
    const uint32_t b0 = 2 * tid;
    const uint32_t c0 = f.hcnt()[b0], c1 = f.hcnt()[b0 + 1];
    const double m0 = f.hmass()[b0], m1 = f.hmass()[b0 + 1];
    uint32_t* fs = f.misc() + M_RED;  // first hits [0..1], last non-empty + 1 [2], per target: before_n, cnt
    if (tid == 0) {
        fs[0] = fs[1] = 0xFFFFFFFFu;
        fs[2] = 0;
    }
    double mtot;
    const double bs = block_excl_scan_f64(m0 + m1, f.miscd() + 8, &mtot);  // barriers order the init above
    uint32_t ctot;
    const uint32_t cb = block_excl_scan<kBlock>(c0 + c1, f.tmp(), &ctot);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const double target = k == 0 ? ta : tb;
        uint32_t cand = 0xFFFFFFFFu;
        if (c0 > 0 && bs + m0 >= target) cand = b0;
        else if (c1 > 0 && bs + m0 + m1 >= target) cand = b0 + 1;
        if (cand != 0xFFFFFFFFu) atomicMin(&fs[k], cand);
    }
    if (c0 + c1 > 0) atomicMax(&fs[2], (c1 > 0 ? b0 + 1 : b0) + 1);
    TSM_LDS_SYNC();
    uint32_t d[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        d[k] = fs[k];
        if (d[k] == 0xFFFFFFFFu) d[k] = fs[2] == 0 ? kBins : fs[2] - 1;
        if (d[k] < kBins && (d[k] >> 1) == tid) {
            const bool second = d[k] & 1u;
            f.miscd()[k] = bs + (second ? m0 : 0.0);
            fs[3 + k] = cb + (second ? c0 : 0u);
            fs[5 + k] = second ? c1 : c0;
        }
    }
    TSM_LDS_SYNC();
#pragma unroll
    for (int k = 0; k < 2; k++) {
        BinHit* h = k == 0 ? ha : hb;
        h->bin = d[k];
        h->cnt = d[k] < kBins ? fs[5 + k] : 0u;
        h->before_n = d[k] < kBins ? fs[3 + k] : ctot;
        h->before = d[k] < kBins ? f.miscd()[k] : mtot;
    }
    TSM_LDS_SYNC();
}

// Gathers the filtered elements of bin b1 (level 1) or of its sub-bin b2
// (level 2), sorts them, and returns the first whose cumulative mass (from
// h.before) reaches target, or the last.  False when the bin holds more than
// kExactCap elements.
__device__ __forceinline__ bool vbin_resolve(Fin& f, const Filt& q, const VBins& vb, bool level2, uint32_t b1, const BinHit& h,
                             uint32_t before_n, double target, MassSel* out) {
    const uint32_t tid = threadIdx.x;
    if (h.bin >= kBins || h.cnt == 0 || h.cnt > kExactCap) return false;
    const uint32_t b2 = h.bin;
    if (tid == 0) f.misc()[M_CNT] = 0;
    TSM_LDS_SYNC();
    row_pass<kNucGroup>(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (!keep_el(f, q, id, y, c)) return;
        const uint32_t b = vb.bin(y);
        if (b != b1 || (level2 && vb.sub(y, b1) != b2)) return;
        const uint32_t pos = atomicAdd(&f.misc()[M_CNT], 1u);
        if (pos < kExactCap) f.gcomp()[pos] = c;
    });
    const uint32_t n = min(f.misc()[M_CNT], kExactCap);
    TSM_LDS_SYNC();
    if (n == 0) return false;
    rank_sort_u64(f.gcomp(), n);
    TSM_LDS_SYNC();
    double p = 0.0;
    uint64_t c = 0;
    if (tid < n) {
        c = f.gcomp()[tid];
        const float y = key_to_float(~static_cast<uint32_t>(c >> 32));
        p = static_cast<double>(glibc_expf((y - vb.y0) / f.m.t));
    }
    if (tid == 0) f.misc()[M_FIND] = 0xFFFFFFFFu;
    double tot;
    const double incl = h.before + (block_excl_scan_f64(p, f.miscd() + 8, &tot) + p);
    if (tid < n && incl >= target) atomicMin(&f.misc()[M_FIND], tid);
    TSM_LDS_SYNC();
    uint32_t j = f.misc()[M_FIND];
    if (j == 0xFFFFFFFFu) j = n - 1;
    if (tid == j) {
        f.miscd()[0] = incl;
        f.gcomp()[kExactCap - 1] = c;  // sorted list no longer needed
    }
    TSM_LDS_SYNC();
    out->T = f.gcomp()[kExactCap - 1];
    out->cum = f.miscd()[0];
    out->rank = before_n + j + 1;
    TSM_LDS_SYNC();
    return true;
}

// mass selection over the histogram in LDS (level 1 bins of q): the element
// of q whose cumulative mass reaches target.  *l1 is cleared when the level-1
// histogram was overwritten.  False when the radix selection must decide.
__device__ __noinline__ bool vbin_select(Fin& f_in, const Filt& q_in, const VBins& vb_in, double target, MassSel* out,
                                         BinHit* hit, bool* l1) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const VBins vb = vb_in;
    const BinHit h = vbin_find(f, 0.0, target);
    *hit = h;
    if (h.bin >= kBins) return false;
    if (h.cnt <= kExactCap) return vbin_resolve(f, q, vb, false, h.bin, h, h.before_n, target, out);
    if (h.bin >= kBins - 1) return false;  // clamped bin: no exact split
    *l1 = false;
    if (!vbin_hist(f, q, vb, true, h.bin)) return false;
    const BinHit h2 = vbin_find(f, h.before, target);
    return vbin_resolve(f, q, vb, true, h.bin, h2, h.before_n + h2.before_n, target, out);
}

struct Pick {
    uint32_t token, keep;
    float prob;
    float mass;
};

__device__ __forceinline__ float readlane_f(float v, uint32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), static_cast<int>(lane)));
}

// The reference's arithmetic on the ranked list ry/rid[0..len) (1 <= len <=
// 1024, best first): p_j = expf((l_j - l_0) / t) (sampler.rs:231-234), min-p
// (extension: the best-first prefix with p_j >= min_p), top-p
// (sampler.rs:235-246) and the inverse-CDF draw (sampler.rs:142-150).
// Every p_j is computed in parallel; the order-dependent f32 folds (total,
// acc, mass, r) run in wave 0 over 64-wide slices, each value broadcast in
// list order with readlane, so every rounding matches the CPU sampler's.
__device__ Pick exact_finalize(Fin& f, uint32_t len, float u, bool draw) {
    const uint32_t tid = threadIdx.x;
    const float y0 = f.ry()[0];
    for (uint32_t j = tid; j < len; j += kBlock) f.rp()[j] = glibc_expf((f.ry()[j] - y0) / f.m.t);
    if (tid == 0) f.misc()[M_FIRST] = len;
    TSM_LDS_SYNC();
    if (!f.m.greedy && f.P.min_p > 0.0f) {
        for (uint32_t j = tid; j < len; j += kBlock)
            if (!(f.rp()[j] >= f.P.min_p)) atomicMin(&f.misc()[M_FIRST], j);
        TSM_LDS_SYNC();
        len = max(f.misc()[M_FIRST], 1u);
    }
    const bool topp = !(f.m.greedy || f.P.top_p >= 1.0f);
    if (tid < kWave) {  // total = sum p_j (left fold), and every prefix sum
        const uint32_t lane = tid;
        float total = 0.0f;
        for (uint32_t b = 0; b < len; b += kWave) {
            const uint32_t cnt = min(static_cast<uint32_t>(kWave), len - b);
            const float v = lane < cnt ? f.rp()[b + lane] : 0.0f;
            float mine = 0.0f;
            for (uint32_t j = 0; j < cnt; j++) {
                total += readlane_f(v, j);
                mine = lane == j ? total : mine;
            }
            if (lane < cnt) f.rP()[b + lane] = mine;
        }
    }
    TSM_LDS_SYNC();
    if (tid < kWave) {
        const uint32_t lane = tid;
        const float total = f.rP()[len - 1];
        // top-p: acc += p_j / total until acc >= p
        uint32_t keep = len;
        if (topp) {
            float acc = 0.0f;
            bool hit = false;
            for (uint32_t b = 0; b < len && !hit; b += kWave) {
                const uint32_t cnt = min(static_cast<uint32_t>(kWave), len - b);
                const float q = lane < cnt ? f.rp()[b + lane] / total : 0.0f;
                for (uint32_t j = 0; j < cnt; j++) {
                    acc += readlane_f(q, j);
                    if (acc >= f.P.top_p) {
                        keep = b + j + 1;
                        hit = true;
                        break;
                    }
                }
            }
        }
        const float mass = f.rP()[keep - 1];  // sum of p_j over the kept prefix
        uint32_t pick = keep - 1;
        if (draw) {
            float r = u * mass;
            bool hit = false;
            for (uint32_t b = 0; b < keep && !hit; b += kWave) {
                const uint32_t cnt = min(static_cast<uint32_t>(kWave), keep - b);
                const float v = lane < cnt ? f.rp()[b + lane] : 0.0f;
                for (uint32_t j = 0; j < cnt; j++) {
                    r -= readlane_f(v, j);
                    if (r <= 0.0f) {
                        pick = b + j;
                        hit = true;
                        break;
                    }
                }
            }
        }
        if (lane == 0) {
            f.misc()[M_TOKEN] = f.rid()[pick];
            f.misc()[M_KEEP] = keep;
            f.misc()[M_PROB] = __float_as_uint(f.rp()[pick] / mass);
            f.misc()[M_MASS] = __float_as_uint(mass);
        }
    }
    TSM_LDS_SYNC();
    Pick p;
    p.token = f.misc()[M_TOKEN];
    p.keep = f.misc()[M_KEEP];
    p.prob = __uint_as_float(f.misc()[M_PROB]);
    p.mass = __uint_as_float(f.misc()[M_MASS]);
    TSM_LDS_SYNC();
    return p;
}

// Writes the first min(keep, dist_stride) entries of the kept distribution,
// normalised by the kept mass (Sampler::distribution, sampler.rs:102-116).
__device__ void write_dist_exact(const Fin& f, uint32_t* ids, float* probs, uint32_t stride, uint32_t* status,
                                 const Pick& p) {
    const uint32_t k = min(p.keep, stride);
    for (uint32_t j = threadIdx.x; j < k; j += kBlock) {
        ids[j] = f.rid()[j];
        probs[j] = f.rp()[j] / p.mass;
    }
    if (p.keep > stride && threadIdx.x == 0) atomicOr(status, TSM_STATUS_DIST_TRUNCATED);
}

// Top-W by IEEE order, then the window rule.  Returns false when the mask
// leaves nothing in the window (the caller runs the whole-vocabulary
// fallback).  The ranked list is left in ry/rid; *len gets its length.
__device__ bool slow_topk_window(Fin& f, uint32_t* len) {
    Filt q;
    q.order = ORD_CANON_Y;
    const uint64_t T = select_kth(f, q, f.m.window);
    q.use_max = true;
    q.max_comp = T;
    const uint32_t g = gather_pass(f, q, kExactCap);
    sort_gathered(f, g);
    if (!f.m.constrained) {
        *len = min(g, f.m.want);
        return true;
    }
    // stable compaction of allowed ids
    const uint32_t tid = threadIdx.x;
    const bool ok = tid < g && allowed_bit(f, f.rid()[tid]);
    const float yv = tid < g ? f.ry()[tid] : 0.0f;
    const uint32_t idv = tid < g ? f.rid()[tid] : 0u;
    uint32_t total;
    const uint32_t pos = block_excl_scan<kBlock>(ok ? 1u : 0u, f.tmp(), &total);
    if (ok) {
        f.ry()[pos] = yv;
        f.rid()[pos] = idv;
    }
    TSM_LDS_SYNC();
    *len = min(total, f.m.want);
    return total > 0;
}

// Whole-vocabulary fallback (sampler.rs:211-221): top-want allowed ids by
// total_cmp order, gathered by re-reading the row.
__device__ uint32_t slow_fallback(Fin& f, uint32_t n_allowed) {
    Filt q;
    q.order = ORD_TOTAL_Y;
    q.need_allowed = true;
    const uint32_t k = min(f.m.want, n_allowed);
    const uint64_t T = select_kth(f, q, k);
    q.use_max = true;
    q.max_comp = T;
    const uint32_t g = gather_pass(f, q, kExactCap);
    sort_gathered(f, g);
    return min(g, f.m.want);
}



// Outputs of a distribution() call for one row (row-offset pointers).
struct DistOut {
    uint32_t* ids;
    float* probs;
    uint32_t stride;
    uint32_t* status;
};

// Finishes a ranked list of `len` candidates in ry/rid: the exact arithmetic,
// and in distribution mode the kept distribution.
__device__ Pick finish_list(Fin& f, uint32_t len, float u, const DistOut* dist) {
    if (len == 0) {  // nothing to rank (e.g. NaN logits): the caller flags it
        Pick e;
        e.token = 0xFFFFFFFFu;
        e.keep = 0;
        e.prob = 0.0f;
        e.mass = 0.0f;
        return e;
    }
    const Pick p = exact_finalize(f, len, u, dist == nullptr);
    if (dist && p.keep > 0) write_dist_exact(f, dist->ids, dist->probs, dist->stride, dist->status, p);
    return p;
}

// Top-k rows whose candidates could not be bounded in LDS (pathological
// ties): the top-W by re-reading the row, then the window rule and the
// whole-vocabulary fallback (sampler.rs:192-222).  Leaves the ranked list in
// ry/rid and returns its length.
__device__ uint32_t reread_topk_list(Fin& f, uint32_t nallow) {
    uint32_t len = 0;
    if (!slow_topk_window(f, &len)) len = slow_fallback(f, nallow);
    return len;
}

// Top-p and the draw from one gather.  The kept mass M lies in (before,
// before + mass] of the top-p bin hp, so the draw target u * M can only fall
// in the bins that cover [u * before, u * (before + mass)]: hp and those bins
// are gathered together, sorted, and both picks are resolved from the list
// with f64 prefix sums.  False (nothing decided, the histogram intact) when
// they hold more than kExactCap elements; the caller then selects in passes
// of their own.
__device__ __noinline__ bool vbin_topp_draw(Fin& f_in, const Filt& q_in, const VBins& vb_in, double target_p,
                                            float u, MassSel* sp, uint64_t* drawn) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const VBins vb = vb_in;
    const uint32_t tid = threadIdx.x;
    const BinHit hp = vbin_find(f, 0.0, target_p);
    if (hp.bin >= kBins || hp.cnt == 0 || hp.cnt > kExactCap) return false;
    const double hmass_p = f.hmass()[hp.bin];
    const double du = static_cast<double>(u);
    BinHit hlo, hhi;
    vbin_find2(f, du * hp.before, du * (hp.before + hmass_p), &hlo, &hhi);
    const uint32_t jlo = min(hlo.bin, hp.bin), jhi = min(hhi.bin, hp.bin);
    // bins jlo..jhi (contiguous) and hp.bin; hp's elements sort last
    const uint32_t n_low = jhi < hp.bin ? (hhi.before_n + hhi.cnt) - hlo.before_n : hp.before_n - hlo.before_n;
    const uint32_t want_n = n_low + hp.cnt;
    if (want_n > kExactCap) return false;
    if (tid == 0) f.misc()[M_CNT] = 0;
    TSM_LDS_SYNC();
    const uint32_t bstar = hp.bin;
    row_pass<kNucGroup>(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (!keep_el(f, q, id, y, c)) return;
        const uint32_t b = vb.bin(y);
        if (b != bstar && (b < jlo || b > jhi)) return;
        const uint32_t pos = atomicAdd(&f.misc()[M_CNT], 1u);
        if (pos < kExactCap) f.gcomp()[pos] = c;
    });
    const uint32_t n = f.misc()[M_CNT];
    TSM_LDS_SYNC();
    if (n != want_n) return false;  // not reached: the histogram counted the same elements
    rank_sort_u64(f.gcomp(), n);
    TSM_LDS_SYNC();
    const uint32_t s0 = n - hp.cnt;  // list index of hp's first element
    double p = 0.0;
    uint64_t c = 0;
    if (tid < n) {
        c = f.gcomp()[tid];
        const float y = key_to_float(~static_cast<uint32_t>(c >> 32));
        p = static_cast<double>(glibc_expf((y - vb.y0) / f.m.t));
    }
    // top-p inside hp
    if (tid == 0) {
        f.misc()[M_FIND] = 0xFFFFFFFFu;
        f.misc()[M_FIND2] = 0xFFFFFFFFu;
    }
    double tot;
    const double pin = tid >= s0 ? p : 0.0;
    const double cum_p = hp.before + (block_excl_scan_f64(pin, f.miscd() + 8, &tot) + pin);
    if (tid >= s0 && tid < n && cum_p >= target_p) atomicMin(&f.misc()[M_FIND], tid);
    TSM_LDS_SYNC();
    uint32_t jp = f.misc()[M_FIND];
    if (jp == 0xFFFFFFFFu) jp = n - 1;
    if (tid == jp) f.miscd()[0] = cum_p;
    TSM_LDS_SYNC();
    const double M = f.miscd()[0];
    const double td = du * M;
    // the draw: inside hp (through the top-p pick) or in bins jlo..jhi; with
    // no bin gathered below hp, hp holds the row's first elements
    const bool in_hp = td > hp.before || s0 == 0;
    const double plo = (!in_hp && tid < s0) ? p : 0.0;
    const double cum_d = in_hp ? cum_p : hlo.before + (block_excl_scan_f64(plo, f.miscd() + 8, &tot) + plo);
    const uint32_t lo_j = in_hp ? s0 : 0u, hi_j = in_hp ? jp + 1 : s0;
    if (tid >= lo_j && tid < hi_j && cum_d >= td) atomicMin(&f.misc()[M_FIND2], tid);
    TSM_LDS_SYNC();
    uint32_t jd = f.misc()[M_FIND2];
    bool ok = true;
    if (jd == 0xFFFFFFFFu) {
        if (in_hp) jd = jp;  // u * M reaches past the pick only by rounding: the last kept
        else ok = false;     // rounding put the target outside the gathered bins
    }
    TSM_LDS_SYNC();
    if (!ok) return false;
    sp->T = f.gcomp()[jp];
    sp->cum = M;
    sp->rank = hp.before_n + (jp - s0) + 1;
    *drawn = f.gcomp()[jd];
    TSM_LDS_SYNC();
    return true;
}

// Restricts the level-1 histogram to the elements through the top-p pick,
// which lies in bin hb: later bins are emptied and bin hb keeps its kept part.
__device__ __forceinline__ void vbin_cut(Fin& f, const BinHit& hb, uint32_t keep, double mass) {
    for (uint32_t i = threadIdx.x; i < kBins; i += kBlock) {
        if (i > hb.bin) {
            f.hcnt()[i] = 0;
            f.hmass()[i] = 0.0;
        } else if (i == hb.bin) {
            f.hcnt()[i] = keep - hb.before_n;
            f.hmass()[i] = mass - hb.before;
        }
    }
    TSM_LDS_SYNC();
}

// Up to kExactCap survivors: gathered, sorted and finished exactly.
__device__ __noinline__ Pick nucleus_exact(Fin& f_in, const Filt& q_in, float u, const DistOut* dist) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const uint32_t g = gather_pass<kNucGroup>(f, q, kExactCap);
    sort_gathered(f, g);
    return finish_list(f, g, u, dist);
}

// Rows without top-k (window > 1024): the cutoff set (sampler.rs:195-208),
// the window rule, truncation to want, min-p, then top-p and the draw, all
// by re-reading the row.  Up to 1024 survivors are finished exactly
// (finish_list); larger sets use f64 mass selections, through value bins
// where they resolve and through radix rounds otherwise.
__device__ __noinline__ Pick reread_nucleus(Fin& f, uint32_t nallow, float u, const DistOut* dist) {
    const uint32_t tid = threadIdx.x;
    const RowMode& m = f.m;
    float mall = -INFINITY, mal = -INFINITY, mlo = INFINITY;
    {
        float la = -INFINITY, lb = -INFINITY, lc = INFINITY;
        row_pass<2 * kNucGroup>(f, [&](uint32_t id, float x, float y) {
            la = fmaxf(la, y);
            lc = fminf(lc, y);
            if (m.constrained && allowed_bit(f, id)) lb = fmaxf(lb, y);
        });
        la = wave_max(la);
        lb = wave_max(lb);
        lc = -wave_max(-lc);
        float* ftmp = reinterpret_cast<float*>(f.miscd() + 8);
        if ((tid & 63) == 0) {
            ftmp[tid / 64] = la;
            ftmp[16 + tid / 64] = lb;
            ftmp[32 + tid / 64] = lc;
        }
        TSM_LDS_SYNC();
        for (int w = 0; w < kBlock / kWave; w++) {
            mall = fmaxf(mall, ftmp[w]);
            mal = fmaxf(mal, ftmp[16 + w]);
            mlo = fminf(mlo, ftmp[32 + w]);
        }
        TSM_LDS_SYNC();
    }
    const float cut = mall - 30.0f * m.t;  // sampler.rs:198-199
    const float y0 = m.constrained ? mal : mall;
    // value bins over [y0 - 30.5 t, y0], or the row's narrower range
    VBins vb;
    vb.y0 = y0;
    {
        float span = fminf(30.5f, (y0 - mlo) / m.t);
        if (!(span > 0.0f)) span = 1.0f;
        vb.mul = (static_cast<float>(kBins) / span) / m.t;
    }
    bool use_vb = m.t > 0.0f && __builtin_isfinite(y0) && __builtin_isfinite(vb.mul) && vb.mul > 0.0f;
    bool hist_ok = false;  // the level-1 histogram in LDS is that of q2
    Filt q0;
    q0.order = ORD_TOTAL_Y;
    q0.use_cut = true;
    q0.cut = cut;
    q0.need_allowed = m.constrained;
    uint32_t n0;
    if (f.P.min_p > 0.0f && !m.constrained && m.want >= f.n) {
        // the cutoff set's size decides nothing here (no truncation, no
        // fallback): min-p's count below is the first one needed
        n0 = m.want;
    } else if (use_vb) {
        use_vb = vbin_hist(f, q0, vb, false, 0);
        double mass0;
        n0 = vbin_totals(f, &mass0);
        hist_ok = use_vb;
    } else {
        n0 = count_pass<kNucGroup>(f, q0);
    }
    if (m.constrained && n0 == 0) {  // sampler.rs:211-221
        q0.use_cut = false;
        n0 = nallow;
        hist_ok = false;
    }
    Filt q1 = q0;
    uint32_t n1 = n0;
    if (n0 > m.want) {  // ranked.truncate(want)
        q1.use_max = true;
        q1.max_comp = select_kth(f, q0, m.want);
        n1 = m.want;
        hist_ok = false;
    }
    Filt q2 = q1;
    uint32_t n2c = n1;
    if (f.P.min_p > 0.0f) {  // extension: min-p prefix
        q2.use_minp = true;
        q2.y0 = y0;
        q2.minp = f.P.min_p;
        // p >= min_p  <=>  y >= y0 + t ln(min_p), up to the roundings of the
        // subtraction, the division and expf (below 1e-6 relative): a band of
        // 1e-3 (|y0| + |t ln min_p| + t) on either side holds every value
        // those roundings could put on the other side
        const float a = m.t * logf(f.P.min_p);
        const float band = 1e-3f * (fabsf(y0) + fabsf(a) + m.t);
        q2.minp_lo = (y0 + a) - band;
        q2.minp_hi = (y0 + a) + band;
        n2c = count_pass<kNucGroup>(f, q2);
        if (n2c == 0) {
            q2 = q1;
            q2.use_max = true;
            q2.max_comp = select_kth(f, q1, 1);
            n2c = 1;
        }
        hist_ok = false;
    }
    if (n2c <= kExactCap) return nucleus_exact(f, q2, u, dist);
    // more than 1024 candidates: exact-arithmetic (f64) cumulative sums
    double total;
    if (use_vb && !hist_ok) {
        use_vb = vbin_hist(f, q2, vb, false, 0);
        hist_ok = use_vb;
    }
    if (hist_ok) vbin_totals(f, &total);
    else total = mass_total(f, q2, y0);
    Filt q3 = q2;
    double mass = total;
    uint32_t keep = n2c;
    BinHit hp;
    hp.bin = kBins;
    if (!(f.P.top_p >= 1.0f) && !dist && hist_ok) {
        // top-p and the draw from one gather
        const double target = static_cast<double>(f.P.top_p) * total;
        MassSel sp;
        uint64_t ce;
        if (vbin_topp_draw(f, q2, vb, target, u, &sp, &ce)) {
            Pick pk;
            pk.keep = sp.rank;
            pk.mass = static_cast<float>(sp.cum);
            const float yk = key_to_float(~static_cast<uint32_t>(ce >> 32));
            pk.token = static_cast<uint32_t>(ce);
            pk.prob = static_cast<float>(static_cast<double>(glibc_expf((yk - y0) / m.t)) / sp.cum);
            return pk;
        }
    }
    if (!(f.P.top_p >= 1.0f)) {
        const double target = static_cast<double>(f.P.top_p) * total;
        MassSel sp;
        if (!(hist_ok && vbin_select(f, q2, vb, target, &sp, &hp, &hist_ok))) {
            hist_ok = false;
            sp = mass_select(f, q2, y0, target);
        }
        q3.use_max = true;
        q3.max_comp = sp.T;
        mass = sp.cum;
        keep = sp.rank;
    }
    Pick pk;
    pk.keep = keep;
    pk.mass = static_cast<float>(mass);
    if (dist) {
        Filt qd = q3;
        const uint32_t k = min(min(keep, dist->stride), kExactCap);
        if (k < keep) {
            qd.use_max = true;
            qd.max_comp = select_kth(f, q3, k);
        }
        const uint32_t g = gather_pass(f, qd, kExactCap);
        sort_gathered(f, g);
        for (uint32_t j = tid; j < g; j += kBlock) {
            dist->ids[j] = f.rid()[j];
            dist->probs[j] = static_cast<float>(static_cast<double>(glibc_expf((f.ry()[j] - y0) / m.t)) / mass);
        }
        if (keep > g && tid == 0) atomicOr(dist->status, TSM_STATUS_DIST_TRUNCATED);
        pk.token = g > 0 ? f.rid()[0] : 0u;
        pk.prob = 0.0f;
        TSM_LDS_SYNC();
        return pk;
    }
    // the draw among the kept (sampler.rs:142-150)
    const double dtarget = static_cast<double>(u) * mass;
    uint64_t ce;
    bool drawn = false;
    if (use_vb) {
        if (hist_ok && hp.bin < kBins) vbin_cut(f, hp, keep, mass);
        if (!hist_ok) hist_ok = vbin_hist(f, q3, vb, false, 0);
        MassSel sd;
        BinHit hd;
        bool l1 = true;
        if (hist_ok && vbin_select(f, q3, vb, dtarget, &sd, &hd, &l1)) {
            ce = sd.T;
            drawn = true;
        }
    }
    if (!drawn) {
        const MassSel sr = mass_select(f, q3, y0, dtarget);
        ce = exact_at(f, q3, sr.T);
    }
    const float yk = key_to_float(~static_cast<uint32_t>(ce >> 32));
    pk.token = static_cast<uint32_t>(ce);
    pk.prob = static_cast<float>(static_cast<double>(glibc_expf((yk - y0) / m.t)) / mass);
    return pk;
}

// Raw top-n (value desc, id asc) by re-reading the row: composites of the
// n best raw logits, sorted, in gcomp[0..return).
__device__ uint32_t reread_raw_top(Fin& f, uint32_t nlp) {
    Filt q;
    q.order = ORD_CANON_X;
    const uint64_t T = select_kth(f, q, nlp);
    q.use_max = true;
    q.max_comp = T;
    const uint32_t g = gather_pass(f, q, kExactCap);
    sort_u64(f.gcomp(), g);
    return min(g, nlp);
}

}  // namespace tsm
