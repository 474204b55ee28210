// tsm_select.h - order statistics over one row for a 1024-thread workgroup:
// the row re-read machinery (radix select in LDS over the row held in HBM /
// L2 / MALL) and the exact finish of a ranked candidate list (the reference's
// sequential f32 arithmetic).
//
// A re-read streams the row in 8192-id tiles and answers order-statistic
// questions with 11-bit LDS histograms: select_kth gives the k-th element in
// (value desc, id asc) order (radix).  When at most 1024 candidates remain
// they are gathered, sorted and finished by exact_finalize, which reproduces
// the CPU sampler's roundings; larger nucleus sets are finished by the value-
// bin folds of tsm_nucleus.h.
#pragma once

#include "tsm_device.h"

namespace tsm {

// ---- LDS layout of the sampling workgroup (bytes) -----------------------------
// Region A holds the streaming pass's history lookup (a bitmap of the ids in
// the row's history and an open-addressing table of their counts) and, once
// the stream is done, the finish's ranked lists and the re-read's per-tile
// history counts.  The histograms, the candidate buffer, the penalized list
// and the scalars have their own regions.
constexpr uint32_t kReTile = 8192;         // ids per tile of a re-read pass
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
constexpr uint32_t kOffSeg = kOffSHist + 2 * kSBins * 4;         // stream counters (candidate groups)
constexpr uint32_t kOffNanW = kOffSeg + 2 * (kBlock / kWave) * 4;  // per wave: met a NaN logit
constexpr uint32_t kSmem = kOffNanW + (kBlock / kWave) * 4;
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
    bool use_min = false;  // composites above min_comp only (a chunk after the ones before it)
    bool use_minp = false;
    float cut = 0.0f;
    uint64_t max_comp = ~0ull;
    uint64_t min_comp = 0ull;
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
    if (q.use_min && c <= q.min_comp) return false;
    if (q.use_minp) {
        if (y < q.minp_lo) return false;
        if (!(y >= q.minp_hi) && !(glibc_expf((y - q.y0) / f.m.t) >= q.minp)) return false;
    }
    return true;
}

// One re-read of the row in tiles of kReTile ids; fn(id, raw, penalized) for
// every id.  The row is read as 16-byte blocks from the aligned address at or
// below its start (ids outside the row are skipped; a block that reaches
// before the row's first id or past its last is read element by element), two
// blocks per thread per tile, with the next tile's blocks in flight while one
// is processed.  Penalized rows count the history ids of each tile in LDS.
template <int G = 1, class F>
__device__ void row_pass(Fin& f, F&& fn) {
    (void)G;
    const uint32_t tid = threadIdx.x;
    const uint32_t n = f.n;
    const bool penal = f.m.penal;
    const TSM_GLOBAL_AS float* rowp = global_as(f.rowp);
    const uint32_t head = static_cast<uint32_t>((reinterpret_cast<uintptr_t>(f.rowp) >> 2) & 3u);
    const TSM_GLOBAL_AS float* base = rowp - head;  // 16-byte aligned
    const uint32_t span = head + n;         // aligned-base-relative end
    const uint32_t nblk = (span + 3u) / 4u;  // blocks that hold row ids
    const uint32_t full = span / 4u;         // blocks wholly before the row's end
    constexpr uint32_t kTB = kReTile / 4u;  // blocks per tile
    constexpr uint32_t kPer = kTB / kBlock;
    static_assert(kPer * kBlock == kTB, "blocks per thread per tile");
    const TSM_GLOBAL_AS uint32_t* hist = global_as(f.hist);
    const uint32_t hc = min(f.hlen, TSM_MAX_HISTORY);
    auto load_blk = [&](uint32_t j) -> float4 {
        if (j < full && (j > 0u || head == 0u)) return load4(base + 4u * j);
        float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (j < nblk) {
            const uint32_t i0 = 4u * j;
            if (i0 >= head && i0 < span) r.x = rowp[i0 - head];
            if (i0 + 1u >= head && i0 + 1u < span) r.y = rowp[i0 + 1u - head];
            if (i0 + 2u >= head && i0 + 2u < span) r.z = rowp[i0 + 2u - head];
            if (i0 + 3u >= head && i0 + 3u < span) r.w = rowp[i0 + 3u - head];
        }
        return r;
    };
    float4 cur[kPer], nxt[kPer];
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) cur[k] = load_blk(tid + k * kBlock);
    const uint32_t ntiles = (nblk + kTB - 1u) / kTB;
    for (uint32_t t = 0; t < ntiles; t++) {
        if (t + 1u < ntiles) {
#pragma unroll
            for (uint32_t k = 0; k < kPer; k++) nxt[k] = load_blk((t + 1u) * kTB + tid + k * kBlock);
        }
        const uint32_t tb = t * kReTile;  // aligned-base-relative first id of the tile
        if (penal) {
            TSM_LDS_SYNC();
            for (uint32_t i = tid; i < kReTile / 2; i += kBlock) f.cnt()[i] = 0;
            TSM_LDS_SYNC();
            for (uint32_t h = tid; h < hc; h += kBlock) {
                const uint32_t li = hist[h] + head - tb;
                if (li < kReTile && hist[h] < n) atomicAdd(&f.cnt()[li >> 1], 1u << ((li & 1u) << 4));
            }
            TSM_LDS_SYNC();
        }
#pragma unroll
        for (uint32_t k = 0; k < kPer; k++) {
            const uint32_t j = t * kTB + tid + k * kBlock;
            if (j >= nblk) continue;
            const float xv[4] = {cur[k].x, cur[k].y, cur[k].z, cur[k].w};
#pragma unroll
            for (uint32_t q = 0; q < 4u; q++) {
                const uint32_t i = 4u * j + q;
                if (i < head || i >= span) continue;
                const float x = xv[q];
                float y = x;
                if (penal) {
                    const uint32_t li = i - tb;
                    const uint32_t c = (f.cnt()[li >> 1] >> ((li & 1u) << 4)) & 0xFFFFu;
                    if (c) y = penalize(x, c, f.m, f.P);
                }
                fn(i - head, x, y);
            }
        }
        if (t + 1u < ntiles) {
#pragma unroll
            for (uint32_t k = 0; k < kPer; k++) cur[k] = nxt[k];
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
// none.  select_kth returns a threshold whose low bits may be padding; this
// resolves it to the element itself (its id is the low word).
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

constexpr int kNucGroup = 4;  // loads in flight per thread in the nucleus passes

// ---- value bins ------------------------------------------------------------------
// bin(y) = floor((y0 - y) * mul), clamped to [0, kBins): (y0 - y) * mul is
// monotone in y, so ascending bins visit the elements in (value desc) order
// and equal values share a bin.
struct VBins {
    float y0, mul;
    __device__ __forceinline__ float pos(float y) const { return (y0 - y) * mul; }
    __device__ __forceinline__ uint32_t bin(float y) const {
        const float d = pos(y);
        return d >= static_cast<float>(kBins - 1) ? kBins - 1u : (d > 0.0f ? static_cast<uint32_t>(d) : 0u);
    }
};
static_assert(kBins == 2 * kBlock, "two bins per thread");

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

// Up to kExactCap survivors: gathered, sorted and finished exactly.
__device__ __noinline__ Pick nucleus_exact(Fin& f_in, const Filt& q_in, float u, const DistOut* dist) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const uint32_t g = gather_pass<kNucGroup>(f, q, kExactCap);
    sort_gathered(f, g);
    return finish_list(f, g, u, dist);
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
