// tsm_split.hip - the split-row sampling kernel: rows with a top-k window
// (window <= 1024, sampler.rs:192-194) and short histories.
//
// A row is cut into segments of up to 19456 ids; one 256-thread workgroup
// per (segment, row).  The grid is rows x segments, so even small batches
// fill the chip, and a segment lives in registers: it is read from HBM once,
// with every load issued before any is used.
//
// Segment workgroup:
//   * group maxima: each thread folds its 19 float4 slots into 8 group
//     maxima of the raw logits (and, for constrained rows, of the allowed
//     ones).  Group maxima are distinct elements, so if `need` of the
//     workgroup's 2048 group maxima are >= T, at least `need` elements are.
//     A 256-bin histogram of the group maxima gives such a T (the smallest
//     group maximum in the bins counted from the top until `need`);
//   * `need` is the row's window (and the logprob count) plus the number of
//     distinct penalized ids in the segment: then at least `window`
//     non-penalized elements are >= T, so every element of the row's window
//     that is not penalized and lies in this segment is >= T (a penalized id
//     can outrank at most one element each);
//   * every element >= T (or allowed and >= the allowed threshold) is written
//     to the segment's candidate area; penalized ids are written as skipped
//     entries and listed separately with their raw and penalized values;
//   * logsumexp partials of the raw logits (sampler.rs:298-304);
//   * the workgroup arrives at the row's counter; the last one finishes.
// Finish (the row's last workgroup): the candidates of every segment (a
// superset of the row's window, of its best allowed ids and of its raw
// top-n) plus the penalized list go to registers; exact radix selections
// give the window, the allowed ids in it or the whole-vocabulary fallback
// (sampler.rs:209-222) and the raw top-n; the ranked list is sorted and
// finished with the reference's own f32 arithmetic (sampler.rs:142-150,
// 223-246).
//
// Segments that hold too many candidates for their area (ties) redo their
// thresholds exactly by radix selection over the segment (re-read from L2).
#include "tsm_split.h"
#include "tsm_serial.h"

namespace tsm {
namespace split {

// ---- LDS layout (bytes) ---------------------------------------------------------
constexpr uint32_t kHSlots = 2 * kSplitHist;                  // history table slots
constexpr uint32_t kOffHKey = 0;                               // u32[kHSlots]: id + 1, 0 = empty | finish: region starts
constexpr uint32_t kOffHCnt = kOffHKey + kHSlots * 4;         // u32[kHSlots] counts
constexpr uint32_t kOffGH = kOffHCnt + kHSlots * 4;           // u32[3][256] histograms
constexpr uint32_t kOffMisc = kOffGH + 3 * 256 * 4;           // u32[64]
constexpr uint32_t kOffTmp = kOffMisc + 64 * 4;               // u32[64] reduction scratch
constexpr uint32_t kOffTmpD = kOffTmp + 64 * 4;               // f64[16]
constexpr uint32_t kRedW = 16;                                // words per wave in a reduction area
constexpr uint32_t kOffRed = kOffTmpD + 16 * 8;               // u32[2][kSW][kRedW] reduction areas
constexpr uint32_t kListMax = kMaxWindow;                     // ranked list entries
constexpr uint32_t kOffLY = kOffRed + 2 * kSW * kRedW * 4;    // u32[kListMax] y bits (sorted list)
constexpr uint32_t kOffLI = kOffLY + kListMax * 4;            // u32[kListMax] ids
constexpr uint32_t kOffLP = kOffLI + kListMax * 4;            // f32[kListMax] p_j
constexpr uint32_t kOffLQ = kOffLP + kListMax * 4;            // u64[kListMax] unsorted composites
constexpr uint32_t kOffFilt = kOffLQ + kListMax * 8;             // u32[128]: filter of the finish's table ids
constexpr uint32_t kSmemSplit = kOffFilt + 128 * 4;
static_assert(kSmemSplit <= 64 * 1024, "split kernel LDS");
static_assert(4 * kMaxSegs + 2 <= 2 * kHSlots, "region starts fit the history table region");

__device__ __forceinline__ uint32_t* s_hkey() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHKey); }
__device__ __forceinline__ uint32_t* s_hcnt() { return reinterpret_cast<uint32_t*>(lds_base() + kOffHCnt); }
__device__ __forceinline__ uint32_t* s_gh() { return reinterpret_cast<uint32_t*>(lds_base() + kOffGH); }
__device__ __forceinline__ uint32_t* s_misc() { return reinterpret_cast<uint32_t*>(lds_base() + kOffMisc); }
__device__ __forceinline__ uint32_t* s_tmp() { return reinterpret_cast<uint32_t*>(lds_base() + kOffTmp); }
__device__ __forceinline__ double* s_tmpd() { return reinterpret_cast<double*>(lds_base() + kOffTmpD); }
__device__ __forceinline__ uint32_t* s_ly() { return reinterpret_cast<uint32_t*>(lds_base() + kOffLY); }
__device__ __forceinline__ uint32_t* s_li() { return reinterpret_cast<uint32_t*>(lds_base() + kOffLI); }
__device__ __forceinline__ float* s_lp() { return reinterpret_cast<float*>(lds_base() + kOffLP); }
__device__ __forceinline__ uint64_t* s_lq() { return reinterpret_cast<uint64_t*>(lds_base() + kOffLQ); }
__device__ __forceinline__ uint32_t* s_filt() { return reinterpret_cast<uint32_t*>(lds_base() + kOffFilt); }
// slot staging of the scan, over the list region: per wave kFStage float4
// slots (plus one dummy) and their first id | allowed nibble << 24
constexpr uint32_t kFStage = (kSmemSplit - kOffLY) / 20 / kSW - 1;
__device__ __forceinline__ float4* s_fstage() { return reinterpret_cast<float4*>(lds_base() + kOffLY); }
__device__ __forceinline__ uint32_t* s_fid() {
    return reinterpret_cast<uint32_t*>(lds_base() + kOffLY + kSW * (kFStage + 1) * 16);
}
static_assert(kOffLY % 16 == 0, "float4 staging alignment");

// Per-wave partial results meet in LDS at a few barriers only: each wave
// reduces its values with DPP and lane 0 files them in s_red (kRedW words per
// wave); after the barrier every thread reads the waves' words.  The two
// areas have LDS of their own: a wave that has read them may go on to write
// the scratch words and the staging slots while another still reads.
__device__ __forceinline__ uint32_t* s_red(int k) {  // k = 0 or 1 (two areas)
    return reinterpret_cast<uint32_t*>(lds_base() + kOffRed) + k * kSW * kRedW;
}

// misc[] slots
enum : uint32_t {
    MS_LAST = 0,     // this workgroup arrived last at its row
    MS_PBASE = 1,    // first slot of this segment's penalized entries in the row's list
    MS_CBASE = 3,    // first slot of this segment's candidates in the row's area
    MS_NSTREAM = 6,  // the row's candidate entries (the last arrival)
    MS_NPEN = 7,     // the row's history entries (the last arrival)
    MS_BSTAR = 4,    // histogram bin reached (2 targets)
    MS_SEL = 8,      // selection results: 3 x {digit or bin, count before it, its count}
    MS_CNT = 20,     // counters (3)
    MS_PICK = 24,    // token, keep, prob, mass | 3 selected composites (2 words each)
};

constexpr float kNaNf = __builtin_nanf("");
constexpr float kLog2E = 1.44269504088896341f;  // log2(e) in f32

__device__ __forceinline__ float lane_f(float v, uint32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), static_cast<int>(lane)));
}

// ---- memory shared between the workgroups of a row -------------------------------
// Every word one workgroup writes and another reads (candidates, penalized
// entries, segment summaries, counters) goes through device-scope atomic
// loads and stores, each coherent across the chip's L2 caches on its own
// (global_load/store ... sc1).  The order between a workgroup's stores and
// the last arrival's loads comes from the arrival itself: workgroup-scope
// release and acquire around a barrier, and an agent-scope acquire-release
// read-modify-write of the row's counter (split_kernel).
__device__ __forceinline__ void dev_st32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void dev_st64(void* p, uint64_t v) {
    __hip_atomic_store(static_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t dev_ld32(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t dev_ld64(const void* p) {
    return __hip_atomic_load(static_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t dev_add32(uint32_t* p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t dev_add64(uint64_t* p, uint64_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The row's counter word: candidates and history entries reserved, segments
// arrived.  Reservations come before a segment's arrival, so the last arrival
// reads the row's totals off the counter's previous value.
constexpr uint32_t kCtrPenShift = 24, kCtrArrShift = 36;
__device__ __forceinline__ uint32_t ctr_cand(uint64_t c) { return static_cast<uint32_t>(c) & 0xFFFFFFu; }
__device__ __forceinline__ uint32_t ctr_pen(uint64_t c) { return static_cast<uint32_t>(c >> kCtrPenShift) & 0xFFFu; }
__device__ __forceinline__ uint32_t ctr_arr(uint64_t c) { return static_cast<uint32_t>(c >> kCtrArrShift) & 0xFFFu; }
static_assert(kMaxSegs * kCandCap < (1u << kCtrPenShift) && kSplitHist < 4096u && kMaxSegs < 4096u,
              "counter fields");
__device__ __forceinline__ uint64_t pack2(uint32_t lo, uint32_t hi) {
    return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}
__device__ __forceinline__ void st_entry(uint2* p, uint32_t xb, uint32_t idf) { dev_st64(p, pack2(xb, idf)); }
__device__ __forceinline__ uint2 ld_entry(const uint2* p) {
    const uint64_t v = dev_ld64(p);
    return make_uint2(static_cast<uint32_t>(v), static_cast<uint32_t>(v >> 32));
}
__device__ __forceinline__ void st_sum(SegSum* p, const SegSum& s) {
    uint64_t w[sizeof(SegSum) / 8];
    __builtin_memcpy(w, &s, sizeof(SegSum));
#pragma unroll
    for (uint32_t i = 0; i < sizeof(SegSum) / 8; i++) dev_st64(reinterpret_cast<uint64_t*>(p) + i, w[i]);
}
__device__ __forceinline__ SegSum ld_sum(const SegSum* p) {
    uint64_t w[sizeof(SegSum) / 8];
#pragma unroll
    for (uint32_t i = 0; i < sizeof(SegSum) / 8; i++) w[i] = dev_ld64(reinterpret_cast<const uint64_t*>(p) + i);
    SegSum s;
    __builtin_memcpy(&s, w, sizeof(SegSum));
    return s;
}

// ---- small block helpers (256 threads) ---------------------------------------------
__device__ __forceinline__ float block_max_f(float v) {
    const uint32_t k = wave_max_u32(canon_key(v));  // NaN-free inputs
    uint32_t* tmp = s_tmp();
    if (lane_id() == 0) tmp[threadIdx.x / kWave] = k;
    TSM_LDS_SYNC();
    uint32_t all = tmp[0];
#pragma unroll
    for (int w = 1; w < kSW; w++) all = tmp[w] > all ? tmp[w] : all;
    TSM_LDS_SYNC();
    return key_to_float(all);
}

__device__ __forceinline__ double block_sum_d(double v) {
    v = wave_sum_f64_dpp(v);
    double* tmp = s_tmpd();
    if (lane_id() == 0) tmp[threadIdx.x / kWave] = v;
    TSM_LDS_SYNC();
    double all = 0.0;
#pragma unroll
    for (int w = 0; w < kSW; w++) all += tmp[w];
    TSM_LDS_SYNC();
    return all;
}

// u32 block reductions of four values at once (one barrier pair).
struct Red4 {
    uint32_t v[4];
};
template <class Op>
__device__ __forceinline__ Red4 block_red4(Red4 r, uint32_t idty, Op op) {
    uint32_t* tmp = s_tmp();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t w = dpp_reduce32(r.v[i], idty, op);
        if (lane_id() == 0) tmp[i * kSW + threadIdx.x / kWave] = w;
    }
    TSM_LDS_SYNC();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t a = tmp[i * kSW];
#pragma unroll
        for (int w = 1; w < kSW; w++) a = op(a, tmp[i * kSW + w]);
        r.v[i] = a;
    }
    TSM_LDS_SYNC();
    return r;
}

// Number of the n composites in LDS at q[0..n) that are below c: eight reads
// in flight at a time (a loop of single reads waits out the LDS latency on
// every element).
__device__ __forceinline__ uint32_t rank_below(const uint64_t* q, uint32_t n, uint64_t c) {
    uint32_t rank = 0, j = 0;
    for (; j + 8 <= n; j += 8) {
        uint64_t t[8];
#pragma unroll
        for (int k = 0; k < 8; k++) t[k] = q[j + k];
#pragma unroll
        for (int k = 0; k < 8; k++) rank += t[k] < c ? 1u : 0u;
    }
    for (; j < n; j++) rank += q[j] < c ? 1u : 0u;
    return rank;
}

// ---- history ------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hslot(uint32_t id) { return (id * 2654435761u) >> 21; }  // 11 bits
static_assert(kHSlots == 2048, "hslot yields 11 bits");

// A 4096-bit filter of the table's ids (kept beside the table by the finish):
// an id whose bit is clear is not in the table, with no probe.
__device__ __forceinline__ uint32_t hfilt_bit(uint32_t id) { return (id * 0x9E3779B1u) >> 20; }  // 12 bits
__device__ __forceinline__ bool pen_listed(uint32_t id);
// Count of `id` in the segment's history table (0 when absent).
__device__ __forceinline__ uint32_t hist_lookup(uint32_t id) {
    const uint32_t* key = s_hkey();
    uint32_t s = hslot(id);
    for (uint32_t probe = 0; probe < kHSlots; probe++) {
        const uint32_t k = key[s];
        if (k == 0) return 0;
        if (k == id + 1) return s_hcnt()[s];
        s = (s + 1) & (kHSlots - 1);
    }
    return 0;
}

// Whether `id` is one of the finish's table ids (the filter first).
__device__ __forceinline__ bool pen_listed(uint32_t id) {
    const uint32_t b = hfilt_bit(id);
    if (!((s_filt()[b >> 5] >> (b & 31)) & 1u)) return false;
    return hist_lookup(id) != 0u;
}

// ---- exact composite selection over the segment, re-read from global memory ---------
// Rare path (segments whose candidates overflow their area): the k-th smallest
// composite (~canon_key(x) << 22 | id) among the segment's ids [lo, hi)
// (allowed ones only when `allowed_only`), by 8-bit radix rounds over 54 bits.
// Returns ~0 when fewer than k ids qualify.
__device__ __noinline__ uint64_t seg_select_exact(const float* rowp, const uint32_t* mrow, uint32_t lo, uint32_t hi,
                                                   uint32_t k, bool allowed_only) {
    const uint32_t tid = threadIdx.x;
    uint32_t* hist = s_gh();
    uint32_t* misc = s_misc();
    uint64_t prefix = 0;
    int shift = 54;  // bits above `shift` are fixed by prefix
    uint32_t need = k;
    {
        uint32_t c = 0;
        for (uint32_t e = lo + tid; e < hi; e += kSB) {
            const float x = rowp[e];
            const bool al = !allowed_only || ((mrow[e >> 5] >> (e & 31)) & 1u);
            c += (al && x == x) ? 1u : 0u;
        }
        if (block_sum<kSB>(c, s_tmp()) < k) return ~0ull;
    }
    while (shift > 0) {
        const int sh = shift >= 8 ? shift - 8 : 0;
        const int width = shift - sh;
        hist[tid] = 0;
        TSM_LDS_SYNC();
        for (uint32_t e = lo + tid; e < hi; e += kSB) {
            const float x = rowp[e];
            if (x != x) continue;
            if (allowed_only && !((mrow[e >> 5] >> (e & 31)) & 1u)) continue;
            const uint64_t c = (static_cast<uint64_t>(~canon_key(x)) << 22) | e;
            if ((c >> shift) != prefix) continue;
            atomicAdd(&hist[(c >> sh) & ((1u << width) - 1u)], 1u);
        }
        TSM_LDS_SYNC();
        if (tid < kWave) {  // wave 0 finds the digit where the count reaches `need`
            const uint32_t lane = tid;
            uint32_t c4[4], s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                c4[i] = hist[lane * 4 + i];
                s += c4[i];
            }
            const uint32_t incl = wave_incl_scan(s), excl = incl - s;
            if (excl < need && incl >= need) {
                uint32_t run = excl;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (run + c4[i] >= need) {
                        misc[MS_SEL] = lane * 4 + i;
                        misc[MS_SEL + 1] = run;
                        misc[MS_SEL + 2] = c4[i];
                        break;
                    }
                    run += c4[i];
                }
            }
        }
        TSM_LDS_SYNC();
        const uint32_t digit = misc[MS_SEL], before = misc[MS_SEL + 1], cnt = misc[MS_SEL + 2];
        TSM_LDS_SYNC();
        need -= before;
        prefix = (prefix << width) | digit;
        shift = sh;
        if (cnt == need) break;  // every composite with this prefix is taken
    }
    return (prefix << shift) | ((1ull << shift) - 1ull);
}

// ---- finish: multi-target radix selection ---------------------------------------------
constexpr int kFinRegs = 16;                          // stream entries per thread held in registers
constexpr uint32_t kFinCap = kFinRegs * kSB;          // 4096: rows with more read them from memory
constexpr int kPenRegs = kSplitHist / kSB;            // penalized entries per thread (always registers)

// Entries held by the finish: y and x bits, id | flags.  Invalid: id field kEntSkip.
struct FinEnt {
    uint32_t yb[kFinRegs], xb[kFinRegs], idf[kFinRegs];
    uint32_t pyb[kPenRegs], pxb[kPenRegs], pidf[kPenRegs];
};

// Where the row's stream entries live: the row's candidate area (nstream
// entries, each segment's in one run).  Entries below the row's bounds
// (t_star for any id, tal_star for allowed ids) are dropped: every segment
// holds at least `window` non-penalized ids at or above its own tall, so the
// row's window, raw top-n and best allowed ids all lie at or above them.
// Penalized ids are dropped too (when `penal`): their values come from the
// penalized entries, with the history table in LDS (s_hkey) telling them.
struct FinSrc {
    const uint2* cbase;
    uint32_t nstream;
    float t_star, tal_star;
    bool penal;
};

enum : uint32_t {
    TG_WIN = 0,    // canon(y), every valid entry
    TG_AL = 1,     // canon(y), allowed entries
    TG_RAW = 2,    // canon(x), every valid entry
    TG_FALL = 3,   // total(y) (f32::total_cmp), allowed entries
};

__device__ __forceinline__ bool ent_valid(uint32_t idf) { return idf != kEntSkip; }

// Stream entry j of the row.
__device__ __forceinline__ void fin_decode(const FinSrc& S, uint32_t j, uint32_t& yb, uint32_t& xb, uint32_t& idf) {
    yb = xb = 0u;
    idf = kEntSkip;
    if (j < S.nstream) {
        const uint2 e = ld_entry(S.cbase + j);
        const float x = __uint_as_float(e.x);
        const bool al = (e.y & kEntAllowed) != 0u;
        if ((x >= S.t_star || (al && x >= S.tal_star)) && !(S.penal && pen_listed(e.y & kIdMask))) {
            yb = xb = e.x;
            idf = e.y;
        }
    }
}

// Calls f(yb, xb, idf) for every entry this thread holds: stream entries from
// registers, or (kG) straight from memory for rows of more than kFinCap of
// them; then the penalized entries.
template <bool kG, class F>
__device__ __forceinline__ void fin_for_each(const FinEnt& E, const FinSrc& S, F&& f) {
    if (!kG) {
#pragma unroll
        for (int r = 0; r < kFinRegs; r++) f(E.yb[r], E.xb[r], E.idf[r]);
    } else {
        for (uint32_t j = threadIdx.x; j < S.nstream; j += kSB) {
            uint32_t yb, xb, idf;
            fin_decode(S, j, yb, xb, idf);
            f(yb, xb, idf);
        }
    }
#pragma unroll
    for (int r = 0; r < kPenRegs; r++) f(E.pyb[r], E.pxb[r], E.pidf[r]);
}

// 54-bit composite: ascending = best first (key descending, id ascending).
__device__ __forceinline__ uint64_t comp54(uint32_t key, uint32_t idf) {
    return (static_cast<uint64_t>(~key) << 22) | (idf & kIdMask);
}
__device__ __forceinline__ bool tg_admits(uint32_t tg, uint32_t idf) {
    if (!ent_valid(idf)) return false;
    return (tg == TG_AL || tg == TG_FALL) ? (idf & kEntAllowed) != 0u : true;
}
__device__ __forceinline__ uint64_t tg_comp(uint32_t tg, uint32_t yb, uint32_t xb, uint32_t idf) {
    if (tg == TG_RAW) return comp54(canon_key(__uint_as_float(xb)), idf);
    if (tg == TG_FALL) return comp54(total_key(__uint_as_float(yb)), idf);
    return comp54(canon_key(__uint_as_float(yb)), idf);
}

// Up to three selections at once: for slot i (kind tg[i], need[i] > 0), the
// need[i]-th smallest composite among the entries it admits, or ~0 when
// fewer qualify.  need[i] == 0: the slot is unused.  8-bit radix rounds from
// the top of the 54-bit composite; a slot stops once its digit's bin holds
// exactly what is left.
struct Sel3s {
    uint64_t T[3];
};
template <bool kG>
__device__ __forceinline__ Sel3s fin_select(const FinEnt& E, const FinSrc& S, const uint32_t tg[3],
                                            const uint32_t need_in[3]) {
    const uint32_t tid = threadIdx.x;
    uint32_t* gh = s_gh();
    uint32_t* misc = s_misc();
    Sel3s out;
    uint32_t need[3];
    uint64_t prefix[3];
    int shift[3];
    bool live[3];
    Red4 c;
    c.v[0] = c.v[1] = c.v[2] = c.v[3] = 0;
    fin_for_each<kG>(E, S, [&](uint32_t, uint32_t, uint32_t idf) {
#pragma unroll
        for (int i = 0; i < 3; i++) c.v[i] += (need_in[i] && tg_admits(tg[i], idf)) ? 1u : 0u;
    });
    c = block_red4(c, 0u, [](uint32_t a, uint32_t b) { return a + b; });
#pragma unroll
    for (int i = 0; i < 3; i++) {
        need[i] = need_in[i];
        prefix[i] = 0;
        shift[i] = 54;
        live[i] = need[i] > 0 && c.v[i] >= need[i];
        out.T[i] = ~0ull;
    }
    while (live[0] || live[1] || live[2]) {
        int sh[3];
#pragma unroll
        for (int i = 0; i < 3; i++) sh[i] = shift[i] >= 8 ? shift[i] - 8 : 0;
        gh[tid] = 0;
        gh[256 + tid] = 0;
        gh[512 + tid] = 0;
        TSM_LDS_SYNC();
        fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
#pragma unroll
            for (int i = 0; i < 3; i++) {
                if (!live[i] || !tg_admits(tg[i], idf)) continue;
                const uint64_t cp = tg_comp(tg[i], yb, xb, idf);
                if ((cp >> shift[i]) != prefix[i]) continue;
                const uint32_t width = static_cast<uint32_t>(shift[i] - sh[i]);
                atomicAdd(&gh[i * 256 + static_cast<uint32_t>((cp >> sh[i]) & ((1ull << width) - 1ull))], 1u);
            }
        });
        TSM_LDS_SYNC();
        const uint32_t wid = tid / kWave, lane = lane_id();
        if (wid < 3 && live[wid]) {  // wave i scans slot i's histogram
            uint32_t c4[4], s = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                c4[j] = gh[wid * 256 + lane * 4 + j];
                s += c4[j];
            }
            const uint32_t incl = wave_incl_scan(s), excl = incl - s;
            if (excl < need[wid] && incl >= need[wid]) {
                uint32_t run = excl;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (run + c4[j] >= need[wid]) {
                        misc[MS_SEL + 3 * wid] = lane * 4 + j;
                        misc[MS_SEL + 3 * wid + 1] = run;
                        misc[MS_SEL + 3 * wid + 2] = c4[j];
                        break;
                    }
                    run += c4[j];
                }
            }
        }
        TSM_LDS_SYNC();
#pragma unroll
        for (int i = 0; i < 3; i++) {
            if (!live[i]) continue;
            const uint32_t digit = misc[MS_SEL + 3 * i], before = misc[MS_SEL + 3 * i + 1],
                           cnt = misc[MS_SEL + 3 * i + 2];
            const int width = shift[i] - sh[i];
            need[i] -= before;
            prefix[i] = (prefix[i] << width) | digit;
            shift[i] = sh[i];
            if (cnt == need[i] || shift[i] == 0) {
                live[i] = false;
                out.T[i] = (prefix[i] << shift[i]) | ((1ull << shift[i]) - 1ull);
            }
        }
        TSM_LDS_SYNC();
    }
    return out;
}

// The same selections by value bins, for the common case: per target the
// admitted values' range is cut into 256 equal bins, the bin holding the
// need-th best entry is found from the counts, and only that bin's entries
// are sorted exactly (by composite) to pick it.  A bin of more than kBinCap
// entries, or a range with an infinity, takes the radix rounds of fin_select.
constexpr uint32_t kBinCap = 256;
template <bool kG>
__device__ __forceinline__ Sel3s fin_select_bins(const FinEnt& E, const FinSrc& S, const uint32_t tg[3],
                                                 const uint32_t need[3]) {
    const uint32_t tid = threadIdx.x;
    uint32_t* gh = s_gh();
    uint32_t* misc = s_misc();
    uint64_t* lq = s_lq();
    auto val_of = [&](uint32_t t, uint32_t yb, uint32_t xb) { return __uint_as_float(t == TG_RAW ? xb : yb); };
    // counts and value ranges (canon keys: +-0 one value)
    Red4 cnt, mn, mx;
    cnt.v[3] = 0;
    mn.v[3] = 0xFFFFFFFFu;
    mx.v[3] = 0u;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        cnt.v[i] = 0;
        mn.v[i] = 0xFFFFFFFFu;
        mx.v[i] = 0u;
    }
    fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
#pragma unroll
        for (int i = 0; i < 3; i++) {
            if (!need[i] || !tg_admits(tg[i], idf)) continue;
            const uint32_t k = canon_key(val_of(tg[i], yb, xb));
            cnt.v[i]++;
            mn.v[i] = k < mn.v[i] ? k : mn.v[i];
            mx.v[i] = k > mx.v[i] ? k : mx.v[i];
        }
    });
    {  // one exchange: per target the count, the lowest and the highest key
        uint32_t* r = s_red(1) + (threadIdx.x / kWave) * kRedW;
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const uint32_t c = wave_sum_dpp(cnt.v[i]);
            const uint32_t lo_k = dpp_reduce32(mn.v[i], 0xFFFFFFFFu, [](uint32_t x, uint32_t y) { return x < y ? x : y; });
            const uint32_t hi_k = dpp_reduce32(mx.v[i], 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            if (lane_id() == 0) r[3 * i] = c, r[3 * i + 1] = lo_k, r[3 * i + 2] = hi_k;
        }
        TSM_LDS_SYNC();
#pragma unroll
        for (int i = 0; i < 3; i++) {
            cnt.v[i] = 0, mn.v[i] = 0xFFFFFFFFu, mx.v[i] = 0u;
#pragma unroll
            for (int w = 0; w < kSW; w++) {
                const uint32_t* q = s_red(1) + w * kRedW;
                cnt.v[i] += q[3 * i];
                mn.v[i] = q[3 * i + 1] < mn.v[i] ? q[3 * i + 1] : mn.v[i];
                mx.v[i] = q[3 * i + 2] > mx.v[i] ? q[3 * i + 2] : mx.v[i];
            }
        }
    }
    Sel3s out;
    float lo[3], scale[3];
    bool live[3], flat[3];
    bool fallback = false;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        out.T[i] = ~0ull;
        live[i] = need[i] > 0 && cnt.v[i] >= need[i];
        lo[i] = key_to_float(mn.v[i]);
        const float hi = key_to_float(mx.v[i]);
        flat[i] = mn.v[i] == mx.v[i];
        scale[i] = flat[i] ? 0.0f : 256.0f / (hi - lo[i]);
        if (live[i] && !flat[i] && !(scale[i] > 0.0f && scale[i] < 1e30f)) fallback = true;  // infinities, tiny spans
    }
    if (fallback) return fin_select<kG>(E, S, tg, need);
    auto bin_of = [&](int i, float v) -> uint32_t {
        if (flat[i]) return 0u;
        const float b = (v - lo[i]) * scale[i];
        return b < 255.0f ? static_cast<uint32_t>(b) : 255u;
    };
    gh[tid] = 0;
    gh[256 + tid] = 0;
    gh[512 + tid] = 0;
    TSM_LDS_SYNC();
    fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
#pragma unroll
        for (int i = 0; i < 3; i++)
            if (live[i] && tg_admits(tg[i], idf)) atomicAdd(&gh[i * 256 + bin_of(i, val_of(tg[i], yb, xb))], 1u);
    });
    TSM_LDS_SYNC();
    {  // wave i finds target i's bin, counting from the top bin down
        const uint32_t wid = tid / kWave, lane = lane_id();
        if (wid < 3 && live[wid]) {
            uint32_t c4[4], sm = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                c4[j] = gh[wid * 256 + 255 - (lane * 4 + j)];
                sm += c4[j];
            }
            const uint32_t incl = wave_incl_scan(sm), excl = incl - sm;
            if (excl < need[wid] && incl >= need[wid]) {
                uint32_t run = excl;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (run + c4[j] >= need[wid]) {
                        misc[MS_SEL + 3 * wid] = 255 - (lane * 4 + j);
                        misc[MS_SEL + 3 * wid + 1] = run;
                        misc[MS_SEL + 3 * wid + 2] = c4[j];
                        break;
                    }
                    run += c4[j];
                }
            }
        }
        if (tid < 3) misc[MS_CNT + tid] = 0;
    }
    TSM_LDS_SYNC();
    uint32_t bsel[3], before[3], bcnt[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        bsel[i] = misc[MS_SEL + 3 * i];
        before[i] = misc[MS_SEL + 3 * i + 1];
        bcnt[i] = misc[MS_SEL + 3 * i + 2];
        if (live[i] && bcnt[i] > kBinCap) fallback = true;
    }
    if (fallback) {
        TSM_LDS_SYNC();
        return fin_select<kG>(E, S, tg, need);
    }
    // the bins' entries, then each sorted exactly
    fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
#pragma unroll
        for (int i = 0; i < 3; i++) {
            if (!live[i] || !tg_admits(tg[i], idf) || bin_of(i, val_of(tg[i], yb, xb)) != bsel[i]) continue;
            const uint32_t pos = atomicAdd(&misc[MS_CNT + i], 1u);
            lq[i * kBinCap + pos] = tg_comp(tg[i], yb, xb, idf);
        }
    });
    TSM_LDS_SYNC();
    {  // wave i ranks target i's bin
        const uint32_t wid = tid / kWave, lane = lane_id();
#pragma unroll
        for (int i = 0; i < 3; i++) {
            if (static_cast<uint32_t>(i) != wid || !live[i]) continue;
            const uint32_t want = need[i] - before[i];  // 1-based rank inside the bin
            for (uint32_t q = lane; q < bcnt[i]; q += kWave) {
                const uint64_t ci = lq[i * kBinCap + q];
                uint32_t rank = 0;
                rank += rank_below(lq + i * kBinCap, bcnt[i], ci);
                if (rank + 1 == want) {
                    misc[MS_PICK + 2 * i] = static_cast<uint32_t>(ci);
                    misc[MS_PICK + 2 * i + 1] = static_cast<uint32_t>(ci >> 32);
                }
            }
        }
    }
    TSM_LDS_SYNC();
#pragma unroll
    for (int i = 0; i < 3; i++)
        if (live[i]) out.T[i] = static_cast<uint64_t>(misc[MS_PICK + 2 * i]) | (static_cast<uint64_t>(misc[MS_PICK + 2 * i + 1]) << 32);
    TSM_LDS_SYNC();
    return out;
}

// Number of entries target `tg` admits with composite <= T.
template <bool kG>
__device__ __forceinline__ uint32_t fin_count(const FinEnt& E, const FinSrc& S, uint32_t tg, uint64_t T) {
    uint32_t mine = 0;
    fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
        mine += (tg_admits(tg, idf) && tg_comp(tg, yb, xb, idf) <= T) ? 1u : 0u;
    });
    return block_sum<kSB>(mine, s_tmp());
}

// The entries target `tg` admits with composite <= T (at most kListMax),
// sorted by composite (rank counting): ids to s_li, values to s_ly.
// Returns how many.
template <bool kG>
__device__ __forceinline__ uint32_t fin_gather_sorted(const FinEnt& E, const FinSrc& S, uint32_t tg, uint64_t T) {
    const uint32_t tid = threadIdx.x;
    uint64_t* lq = s_lq();
    uint32_t* misc = s_misc();
    if (tid == 0) misc[MS_CNT] = 0;
    TSM_LDS_SYNC();
    fin_for_each<kG>(E, S, [&](uint32_t yb, uint32_t xb, uint32_t idf) {
        if (!tg_admits(tg, idf)) return;
        const uint64_t cp = tg_comp(tg, yb, xb, idf);
        if (cp <= T) {
            const uint32_t pos = atomicAdd(&misc[MS_CNT], 1u);
            if (pos < kListMax) lq[pos] = cp;
        }
    });
    TSM_LDS_SYNC();
    const uint32_t total = misc[MS_CNT];
    const uint32_t n = total < kListMax ? total : kListMax;
    // composites are distinct (ids are): each one's rank is its place
    for (uint32_t i = tid; i < n; i += kSB) {
        const uint64_t ci = lq[i];
        uint32_t rank = 0;
        rank += rank_below(lq, n, ci);
        s_li()[rank] = static_cast<uint32_t>(ci & kIdMask);
        // the key gives the value back (canon: +-0 read as +0; total: exact)
        const uint32_t key = ~static_cast<uint32_t>(ci >> 22);
        s_ly()[rank] = tg == TG_FALL ? ((key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key)
                                     : __float_as_uint(key_to_float(key));
    }
    TSM_LDS_SYNC();
    return n;
}

// The reference's arithmetic on the sorted list s_ly/s_li[0..len), 1 <= len <=
// kListMax, by wave 0 (as exact_finalize): p_j = expf((y_j - y_0) / t)
// (sampler.rs:231-234), min-p (extension: the best-first prefix with p_j >=
// min_p), top-p (sampler.rs:235-246), the inverse-CDF draw (sampler.rs:
// 142-150).  The folds run in list order, one element at a time, so every
// rounding is the CPU sampler's.  Result in misc[MS_PICK..].
__device__ __forceinline__ void fin_finalize(uint32_t len, float u, const RowMode& m, const tsm_row_params& P,
                                             bool draw) {
    const uint32_t tid = threadIdx.x;
    float* lp = s_lp();
    const float y0 = __uint_as_float(s_ly()[0]);
    for (uint32_t j = tid; j < len; j += kSB) lp[j] = glibc_expf((__uint_as_float(s_ly()[j]) - y0) / m.t);
    if (tid == 0) s_misc()[MS_CNT] = len;
    TSM_LDS_SYNC();
    if (!m.greedy && P.min_p > 0.0f) {
        for (uint32_t j = tid; j < len; j += kSB)
            if (!(lp[j] >= P.min_p)) atomicMin(&s_misc()[MS_CNT], j);
        TSM_LDS_SYNC();
        const uint32_t first = s_misc()[MS_CNT];
        len = first > 1u ? first : 1u;
    }
    if (tid < kWave) {
        const uint32_t lane = tid;
        // total and the prefix sums (left fold)
        float total = 0.0f;
        for (uint32_t b = 0; b < len; b += kWave) {
            const uint32_t cnt = len - b < static_cast<uint32_t>(kWave) ? len - b : static_cast<uint32_t>(kWave);
            const float v = lane < cnt ? lp[b + lane] : 0.0f;
            float mine = 0.0f;
            for (uint32_t j = 0; j < cnt; j++) {
                total += lane_f(v, j);
                mine = lane == j ? total : mine;
            }
            if (lane < cnt) reinterpret_cast<float*>(s_lq())[b + lane] = mine;  // prefix sums
        }
        uint32_t keep = len;
        if (!(m.greedy || P.top_p >= 1.0f)) {
            float acc = 0.0f;
            bool hit = false;
            for (uint32_t b = 0; b < len && !hit; b += kWave) {
                const uint32_t cnt = len - b < static_cast<uint32_t>(kWave) ? len - b : static_cast<uint32_t>(kWave);
                const float q = lane < cnt ? lp[b + lane] / total : 0.0f;
                for (uint32_t j = 0; j < cnt; j++) {
                    acc += lane_f(q, j);
                    if (acc >= P.top_p) {
                        keep = b + j + 1;
                        hit = true;
                        break;
                    }
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
        const float mass = reinterpret_cast<float*>(s_lq())[keep - 1];
        uint32_t pick = keep - 1;
        if (draw) {
            float r = u * mass;
            bool hit = false;
            for (uint32_t b = 0; b < keep && !hit; b += kWave) {
                const uint32_t cnt = keep - b < static_cast<uint32_t>(kWave) ? keep - b : static_cast<uint32_t>(kWave);
                const float v = lane < cnt ? lp[b + lane] : 0.0f;
                for (uint32_t j = 0; j < cnt; j++) {
                    r -= lane_f(v, j);
                    if (r <= 0.0f) {
                        pick = b + j;
                        hit = true;
                        break;
                    }
                }
            }
        }
        if (lane == 0) {
            s_misc()[MS_PICK] = s_li()[pick];
            s_misc()[MS_PICK + 1] = keep;
            s_misc()[MS_PICK + 2] = __float_as_uint(lp[pick] / mass);
            s_misc()[MS_PICK + 3] = __float_as_uint(mass);
        }
    }
    TSM_LDS_SYNC();
}

// ---- the row's finish ------------------------------------------------------------
// Window (sampler.rs:192-194), the constraint filter and its fallback
// (sampler.rs:209-222), truncation, the reference's arithmetic, the raw top-n
// and the outputs; the row's counters are reset for the next call.
template <bool kG>
__device__ __forceinline__ void fin_row(const SplitArgs& a, const FinSrc& S, const RowMode& m,
                                        const tsm_row_params& P, uint32_t row, uint32_t nlp, float lse,
                                        uint32_t flags_row, FinEnt& E) {
    const uint32_t tid = threadIdx.x;
    const uint32_t n = a.s.usable;
    // penalized entries: the segments listed their history ids with every
    // repeat; the first to claim an id's slot in the LDS table keeps the entry
    // and applies the penalties with the id's count (sampler.rs:165-175 +
    // presence / frequency)
    {
        uint32_t slot[kPenRegs];
        if (S.penal) {
            for (uint32_t q = tid; q < kHSlots; q += kSB) {
                s_hkey()[q] = 0;
                if (q < 128) s_filt()[q] = 0;
                s_hcnt()[q] = 0;
            }
            TSM_LDS_SYNC();
#pragma unroll
            for (int r = 0; r < kPenRegs; r++) {
                slot[r] = kHSlots;
                if (E.pidf[r] == kEntSkip) continue;
                const uint32_t id = E.pidf[r] & kIdMask;
                uint32_t q = hslot(id);
                while (true) {
                    const uint32_t prev = atomicCAS(&s_hkey()[q], 0u, id + 1u);
                    if (prev == 0u || prev == id + 1u) {
                        atomicAdd(&s_hcnt()[q], 1u);
                        if (prev == 0u) atomicOr(&s_filt()[hfilt_bit(id) >> 5], 1u << (hfilt_bit(id) & 31));
                        if (prev != 0u) E.pidf[r] = kEntSkip;  // a repeat: the slot's first entry stands for it
                        slot[r] = q;
                        break;
                    }
                    q = (q + 1) & (kHSlots - 1);
                }
            }
            TSM_LDS_SYNC();
        }
#pragma unroll
        for (int r = 0; r < kPenRegs; r++) {
            E.pyb[r] = 0u;
            if (E.pidf[r] == kEntSkip) continue;
            const float y = penalize(__uint_as_float(E.pxb[r]), s_hcnt()[slot[r]], m, P);
            if (y == y) {
                E.pyb[r] = __float_as_uint(y);
                E.pidf[r] |= kEntPen;
            } else {
                E.pidf[r] = kEntSkip;  // a NaN penalized value: the row's NaN flag reports it
            }
        }
        if (!kG) {  // the stream entries held since the start: the row's bounds, penalized ids out
#pragma unroll
            for (int r = 0; r < kFinRegs; r++) {
                const float x = __uint_as_float(E.yb[r]);
                const bool al = (E.idf[r] & kEntAllowed) != 0u;
                if (!ent_valid(E.idf[r]) || !(x >= S.t_star || (al && x >= S.tal_star)) ||
                    (S.penal && pen_listed(E.idf[r] & kIdMask)))
                    E.idf[r] = kEntSkip;
                E.xb[r] = E.yb[r];
            }
        }
    }
    // selections: the window, the want-th best allowed id, the raw top-n
    // (and the raw best: the argmax when nothing is allowed, sampler.rs:139-141)
    const uint32_t nlp_raw = m.constrained ? (nlp > 1u ? nlp : 1u) : nlp;
    const uint32_t tg[3] = {TG_WIN, TG_AL, TG_RAW};
    const uint32_t nd[3] = {m.window, m.constrained ? m.want : 0u, nlp_raw};
    const Sel3s S1 = fin_select_bins<kG>(E, S, tg, nd);
    const uint64_t Tw = S1.T[0], Ta = S1.T[1], Tr = S1.T[2];
    uint64_t Tlist = Tw;
    uint32_t tglist = TG_WIN;
    if (m.constrained) {
        if (Ta <= Tw) {
            Tlist = Ta;  // the want-th best allowed id ranks inside the window
            tglist = TG_AL;
        } else if (fin_count<kG>(E, S, TG_AL, Tw) > 0) {
            Tlist = Tw;  // fewer than `want` allowed ids in the window: all of them
            tglist = TG_AL;
        } else {
            // none in the window: the best allowed ids of the whole row by
            // f32::total_cmp (sampler.rs:211-221)
            const uint32_t tg2[3] = {TG_FALL, TG_FALL, TG_FALL};
            const uint32_t nd2[3] = {m.want, 0u, 0u};
            Tlist = fin_select<kG>(E, S, tg2, nd2).T[0];
            tglist = TG_FALL;
        }
    }
    uint32_t len = fin_gather_sorted<kG>(E, S, tglist, Tlist);
    if (len > m.want) len = m.want;

    // ---- the pick ----
    uint32_t token = 0xFFFFFFFFu, keep = 0;
    float prob = 0.0f;
    const float u = a.s.distribution ? 0.0f : a.s.uniforms[row];
    if (len > 0) {
        fin_finalize(len, u, m, P, !a.s.distribution);
        token = s_misc()[MS_PICK];
        keep = s_misc()[MS_PICK + 1];
        prob = __uint_as_float(s_misc()[MS_PICK + 2]);
        const float mass = __uint_as_float(s_misc()[MS_PICK + 3]);
        if (a.s.distribution) {
            const uint32_t k = keep < a.s.dist_stride ? keep : a.s.dist_stride;
            for (uint32_t j = tid; j < k; j += kSB) {
                a.s.dist_ids[static_cast<size_t>(row) * a.s.dist_stride + j] = s_li()[j];
                a.s.dist_probs[static_cast<size_t>(row) * a.s.dist_stride + j] = s_lp()[j] / mass;
            }
            if (keep > a.s.dist_stride && tid == 0) atomicOr(a.s.status, TSM_STATUS_DIST_TRUNCATED);
        }
        TSM_LDS_SYNC();
    }
    // raw top-n (sampler.rs:305-311) and the raw argmax when nothing is kept
    uint32_t nraw = 0;
    if (nlp_raw > 0) nraw = fin_gather_sorted<kG>(E, S, TG_RAW, Tr);
    if (len == 0) {  // nothing kept: the raw argmax, with probability 1
        token = nraw > 0 ? s_li()[0] : 0xFFFFFFFFu;
        prob = 1.0f;
    }
    // the token's raw logit, from the entry that holds it (sampler.rs:307)
    if (m.logprobs && a.s.out_logprob) {
        if (tid == 0) s_misc()[MS_CNT] = 0x7FC00000u;
        TSM_LDS_SYNC();
        fin_for_each<kG>(E, S, [&](uint32_t, uint32_t xb, uint32_t idf) {
            if (ent_valid(idf) && (idf & kIdMask) == token) s_misc()[MS_CNT] = xb;
        });
        TSM_LDS_SYNC();
    }

    // ---- outputs ----
    const bool bad = token >= n;
    if (bad && tid == 0) atomicOr(a.s.status, TSM_STATUS_INTERNAL);
    if (token >= n) token = 0;
    if (a.s.distribution) {
        if (tid == 0) a.s.out_keep[row] = keep;
    } else {
        if (tid == 0) {
            a.s.out_token[row] = token;
            if (a.s.out_prob) a.s.out_prob[row] = prob;
            if (a.s.out_keep) a.s.out_keep[row] = keep;
            if (m.logprobs && a.s.out_logprob) a.s.out_logprob[row] = __uint_as_float(s_misc()[MS_CNT]) - lse;
        }
        if (tid < nlp && tid < nraw) {
            const size_t o = static_cast<size_t>(row) * a.s.top_stride + tid;
            a.s.out_top_ids[o] = s_li()[tid];
            if (a.s.out_top_lp) a.s.out_top_lp[o] = __uint_as_float(s_ly()[tid]) - lse;
        }
    }
    if (m.logprobs && a.s.out_top_ids && m.nlp > a.s.top_stride && tid == 0)
        atomicOr(a.s.status, TSM_STATUS_BAD_PARAMS);
    // counters back to 0 for the next call (every segment has arrived)
    if (tid == 0) dev_st64(&a.w.row_ctr[row], 0ull);
}

// ---- threshold from group maxima (the allowed ids' pass) ----------------------------
// A value T such that at least `need` of the block's group maxima are >= T
// (group maxima are distinct elements, so at least `need` elements are): -inf
// when fewer than `need` are finite, the lowest when all are equal or their
// span is too narrow to bin, else the lowest group maximum in the bins of a
// 256-bin histogram counted from the top until `need`.  Uses s_gh()[256..512).
__device__ __forceinline__ float group_threshold(const float (&gm)[8], uint32_t need) {
    const uint32_t tid = threadIdx.x;
    uint32_t* h = s_gh() + 256;
    Red4 r;
    uint32_t kmin = 0xFFFFFFFFu, kmax = 0u, c = 0u;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        if (gm[g] > -INFINITY) {
            const uint32_t k = canon_key(gm[g]);
            kmin = k < kmin ? k : kmin;
            kmax = k > kmax ? k : kmax;
            c++;
        }
    }
    h[tid] = 0;
    r.v[0] = ~kmin, r.v[1] = kmax, r.v[2] = 0u, r.v[3] = 0u;
    r = block_red4(r, 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
    kmin = ~r.v[0];
    kmax = r.v[1];
    c = block_sum<kSB>(c, s_tmp());
    if (c < need) return -INFINITY;
    const float lo = key_to_float(kmin);
    if (kmin == kmax) return lo;
    const float scale = 256.0f / (key_to_float(kmax) - lo);
    if (!(scale < 1e30f)) return lo;
    auto bin_of = [&](float vv) -> uint32_t {
        const float bb = (vv - lo) * scale;
        return bb < 255.0f ? static_cast<uint32_t>(bb) : 255u;
    };
#pragma unroll
    for (int g = 0; g < 8; g++)
        if (gm[g] > -INFINITY) atomicAdd(&h[bin_of(gm[g])], 1u);
    TSM_LDS_SYNC();
    if (tid < kWave) {
        const uint32_t lane = tid;
        uint32_t c4[4], sm = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            c4[j] = h[255 - (lane * 4 + j)];
            sm += c4[j];
        }
        const uint32_t incl = wave_incl_scan(sm), excl = incl - sm;
        if (excl < need && incl >= need) {
            uint32_t run = excl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (run + c4[j] >= need) {
                    s_misc()[MS_BSTAR + 1] = 255 - (lane * 4 + j);
                    break;
                }
                run += c4[j];
            }
        }
    }
    TSM_LDS_SYNC();
    const uint32_t bstar = s_misc()[MS_BSTAR + 1];
    uint32_t tk = 0xFFFFFFFFu;
#pragma unroll
    for (int g = 0; g < 8; g++) {
        if (gm[g] > -INFINITY && bin_of(gm[g]) >= bstar) {
            const uint32_t k = canon_key(gm[g]);
            tk = k < tk ? k : tk;
        }
    }
    return key_to_float(block_min<kSB>(tk, s_tmp()));
}

// ---- the kernel ----------------------------------------------------------------------

// A row whose logits hold a NaN (tsm_serial.h): wave 0 of the row's last
// workgroup samples it step by step from the row in memory; the LDS of the
// history table and of the finish's lists holds the serial path's areas.
// The logprobs are NaN, as the reference's logsumexp is (sampler.rs:298-304).
__device__ __noinline__ void fin_nan(const SplitArgs& a, const serial::Row& r, uint32_t row, uint32_t nlp) {
    const uint32_t tid = threadIdx.x;
    constexpr float kNaN = __builtin_nanf("");
    serial::Lds s;
    s.tile = 4096;
    s.cnt = s_hkey();                                                       // 8 KB
    s.val = reinterpret_cast<float*>(lds_base() + kOffHKey + 8192);         // 4 KB
    s.id = reinterpret_cast<uint32_t*>(lds_base() + kOffHKey + 12288);      // 4 KB
    s.comp = s_lq();
    s.p = s_lp();
    static_assert(kHSlots * 8 >= 16384 && kListMax >= kMaxWindow, "serial areas");
    TSM_LDS_SYNC();
    serial::Result res;
    res.token = res.keep = res.len = 0;
    res.prob = res.mass = 0.0f;
    if (tid < kWave) {
        res = serial::run(r, s, !a.s.distribution);
        if (tid == 0) {
            s_misc()[MS_PICK] = res.token;
            s_misc()[MS_PICK + 1] = res.keep;
            s_misc()[MS_PICK + 2] = __float_as_uint(res.prob);
            s_misc()[MS_PICK + 3] = __float_as_uint(res.mass);
        }
    }
    TSM_LDS_SYNC();
    res.token = s_misc()[MS_PICK];
    res.keep = s_misc()[MS_PICK + 1];
    res.prob = __uint_as_float(s_misc()[MS_PICK + 2]);
    res.mass = __uint_as_float(s_misc()[MS_PICK + 3]);
    if (a.s.distribution) {
        const uint32_t k = min(res.keep, a.s.dist_stride);
        uint32_t* ids = a.s.dist_ids + static_cast<size_t>(row) * a.s.dist_stride;
        float* probs = a.s.dist_probs + static_cast<size_t>(row) * a.s.dist_stride;
        for (uint32_t j = tid; j < k; j += kSB) {
            ids[j] = s.id[j];
            probs[j] = s.p[j] / res.mass;
        }
        if (res.keep > a.s.dist_stride && tid == 0) atomicOr(a.s.status, TSM_STATUS_DIST_TRUNCATED);
        if (tid == 0) a.s.out_keep[row] = res.keep;
    } else {
        if (tid == 0) {
            a.s.out_token[row] = res.token;
            if (a.s.out_prob) a.s.out_prob[row] = res.prob;
            if (a.s.out_keep) a.s.out_keep[row] = res.keep;
            if (r.m.logprobs && a.s.out_logprob) a.s.out_logprob[row] = kNaN;
        }
        if (nlp > 0) {
            TSM_LDS_SYNC();  // the list areas are taken again
            if (tid < kWave) {
                const uint32_t k = serial::top_n_ref(r, s, nlp, false);
                if (tid < k) {
                    const size_t o = static_cast<size_t>(row) * a.s.top_stride + tid;
                    a.s.out_top_ids[o] = s.id[tid];
                    if (a.s.out_top_lp) a.s.out_top_lp[o] = kNaN;
                }
            }
        }
    }
    if (r.m.logprobs && a.s.out_top_ids && r.m.nlp > a.s.top_stride && tid == 0)
        atomicOr(a.s.status, TSM_STATUS_BAD_PARAMS);
    // counters back to 0 for the next call (every segment has arrived)
    if (tid == 0) dev_st64(&a.w.row_ctr[row], 0ull);
}

template <bool kVecLoads>
__global__ __launch_bounds__(kSB) void split_kernel(SplitArgs a) {
    const uint32_t tid = threadIdx.x, seg = blockIdx.x, row = blockIdx.y;
    const uint32_t wid = tid / kWave, lane = lane_id();
    const uint32_t n = a.s.usable;
    const uint32_t lo = seg * a.seg_len;
    const uint32_t hi = lo + a.seg_len < n ? lo + a.seg_len : n;
    const uint32_t nslot = (hi - lo + kSegQuant - 1) / kSegQuant;
    const bool full = hi - lo == nslot * kSegQuant;
    const float* rowp = a.s.logits + static_cast<size_t>(row) * a.s.row_stride;
    // every slot of the segment, requested first (its addresses depend on
    // nothing the row's parameters say) when every row of the batch is one
    // of this kernel's; otherwise after the row's kind is known, so that a
    // row this kernel does not take costs no reads
    float4 v[kSlots];
    auto load_slots = [&]() {
#pragma unroll
        for (int i = 0; i < kSlots; i++) {
            v[i] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);  // slots past the segment
            if (static_cast<uint32_t>(i) < nslot) {
                const uint32_t e0 = lo + 4u * (static_cast<uint32_t>(i) * kSB + tid);
                const uint32_t ec = e0 < hi ? e0 : lo;  // in bounds; ids past the segment are masked below
                if (kVecLoads) {
                    v[i] = *reinterpret_cast<const float4*>(rowp + ec);
                } else {
                    v[i].x = rowp[ec];
                    v[i].y = rowp[ec + 1 < hi ? ec + 1 : lo];
                    v[i].z = rowp[ec + 2 < hi ? ec + 2 : lo];
                    v[i].w = rowp[ec + 3 < hi ? ec + 3 : lo];
                }
            }
        }
    };
    if (!a.general) load_slots();
    const uint32_t* hop = a.s.hist_off ? a.s.hist_off + row : nullptr;
    const uint32_t h0 = hop ? const_as(hop)[0] : 0u, h1 = hop ? const_as(hop)[1] : 0u;
    const uint32_t hlen = h1 > h0 ? h1 - h0 : 0u;
    tsm_row_params P;
    {
        constexpr int kW = sizeof(tsm_row_params) / 4;
        const TSM_CONST_AS uint32_t* pw = const_as(reinterpret_cast<const uint32_t*>(a.s.params + row));
        uint32_t w[kW];
#pragma unroll
        for (int i = 0; i < kW; i++) w[i] = pw[i];
        __builtin_memcpy(&P, w, sizeof(P));
    }
    const RowMode m = row_mode(P, n, hlen, a.s.mask != nullptr && !a.s.distribution);
    if (!takes_row(m, hlen)) {
        // sampled by sample_kernel; without it (the batch said it holds no
        // such row) the row is reported instead
        if (!a.general && seg == 0 && tid == 0) {
            if (a.s.distribution) {
                a.s.out_keep[row] = 0;
            } else {
                a.s.out_token[row] = 0;
            }
            atomicOr(a.s.status, TSM_STATUS_ROW_KIND);
        }
        return;
    }
    if (a.general) load_slots();
    const uint32_t* mrow = m.constrained ? a.s.mask + static_cast<size_t>(row) * a.s.mask_stride : nullptr;

    // ---- the segment's mask words, then the row's history ids (only their
    // count in this segment is needed before the thresholds) ----
    uint32_t mw[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; i++) mw[i] = 0;
    if (mrow) {
#pragma unroll
        for (int i = 0; i < kSlots; i++) {
            if (static_cast<uint32_t>(i) < nslot) {
                const uint32_t e0 = lo + 4u * (static_cast<uint32_t>(i) * kSB + tid);
                mw[i] = mrow[(e0 < hi ? e0 : lo) >> 5];
            }
        }
    }
    constexpr uint32_t kHPer = kSplitHist / kSB;
    uint32_t hid[kHPer];
#pragma unroll
    for (uint32_t k = 0; k < kHPer; k++) {
        const uint32_t j = tid + k * kSB;
        hid[k] = (m.penal && j < hlen) ? a.s.hist_ids[h0 + j] : 0xFFFFFFFFu;
    }
    const uint32_t msh = 4u * (tid & 7u);  // bit of this thread's first id in its mask word
    s_gh()[tid] = 0;  // the threshold histogram (first used after a barrier)

    // ---- pass 1 over the slots: group maxima, logsumexp partials, allowed
    // ids and their 4-bit masks (packed 8 slots to a word), NaN ----
    if (!full) {  // ids past the segment: -inf, not allowed
#pragma unroll
        for (int i = 0; i < kSlots; i++) {
            if (static_cast<uint32_t>(i) >= nslot) continue;
            const uint32_t e0 = lo + 4u * (static_cast<uint32_t>(i) * kSB + tid);
            if (e0 + 0 >= hi) v[i].x = -INFINITY;
            if (e0 + 1 >= hi) v[i].y = -INFINITY;
            if (e0 + 2 >= hi) v[i].z = -INFINITY;
            if (e0 + 3 >= hi) v[i].w = -INFINITY;
            const uint32_t nv = e0 >= hi ? 0u : (hi - e0 >= 4u ? 4u : hi - e0);
            mw[i] &= ((1u << nv) - 1u) << msh;
        }
    }
    float gm[8];
#pragma unroll
    for (int g = 0; g < 8; g++) gm[g] = -INFINITY;
    uint32_t nib[(kSlots + 7) / 8] = {};
    uint32_t nallow = 0;
    bool has_nan = false;
#pragma unroll
    for (int i = 0; i < kSlots; i++) {
        if (static_cast<uint32_t>(i) >= nslot) continue;
        const float4 x = v[i];
        gm[i & 7] = fmaxf(gm[i & 7], fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w)));
        has_nan |= (x.x != x.x) | (x.y != x.y) | (x.z != x.z) | (x.w != x.w);
        if (mrow) {
            const uint32_t w4 = (mw[i] >> msh) & 0xFu;
            nib[i >> 3] |= w4 << (4 * (i & 7));
            nallow += __popc(w4);
        }
    }
    auto nib_of = [&](int i) -> uint32_t { return (nib[i >> 3] >> (4 * (i & 7))) & 0xFu; };

    // ---- logsumexp partials (sampler.rs:298-304) ----
    float tmax = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; g++) tmax = fmaxf(tmax, gm[g]);
    double lsum_t = 0.0;
    if (m.logprobs && tmax > -INFINITY) {
        // term = exp2(fma(x, log2e, nl)), nl = -tmax * log2e rounded; the
        // rounding error eps shifts every exponent alike and corr = 2^-eps
        // takes it back out
        const float nl = -tmax * kLog2E;
        const float corr = __builtin_amdgcn_exp2f(-__builtin_fmaf(tmax, kLog2E, nl));
#pragma unroll
        for (int i = 0; i < kSlots; i++) {
            if (static_cast<uint32_t>(i) >= nslot) continue;
            const float4 x = v[i];
            const float sm = __builtin_amdgcn_exp2f(__builtin_fmaf(x.x, kLog2E, nl)) +
                             __builtin_amdgcn_exp2f(__builtin_fmaf(x.y, kLog2E, nl)) +
                             __builtin_amdgcn_exp2f(__builtin_fmaf(x.z, kLog2E, nl)) +
                             __builtin_amdgcn_exp2f(__builtin_fmaf(x.w, kLog2E, nl));
            lsum_t += static_cast<double>(sm);
        }
        lsum_t *= static_cast<double>(corr);
    }

    // ---- history ids in this segment: counted now, their logits gathered ----
    uint32_t nh = 0, nh_al = 0;
    float hx[kHPer];
    uint32_t hw[kHPer];
#pragma unroll
    for (uint32_t k = 0; k < kHPer; k++) {
        const bool in = hid[k] >= lo && hid[k] < hi;
        nh += in ? 1u : 0u;
        hx[k] = in ? rowp[hid[k]] : 0.0f;
        hw[k] = (in && mrow) ? mrow[hid[k] >> 5] : 0u;
        nh_al += ((hw[k] >> (hid[k] & 31)) & 1u) && in ? 1u : 0u;
    }

    // ---- statistics: one exchange for the whole block ----
    uint32_t gmin, gmax, gcnt;
    {
        uint32_t kmin = 0xFFFFFFFFu, kmax = 0u, c = 0u;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            if (gm[g] > -INFINITY) {
                const uint32_t k = canon_key(gm[g]);
                kmin = k < kmin ? k : kmin;
                kmax = k > kmax ? k : kmax;
                c++;
            }
        }
        kmin = dpp_reduce32(kmin, 0xFFFFFFFFu, [](uint32_t x, uint32_t y) { return x < y ? x : y; });
        kmax = dpp_reduce32(kmax, 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        c = wave_sum_dpp(c);
        const uint32_t w_allow = wave_sum_dpp(nallow), w_nan = wave_sum_dpp(has_nan ? 1u : 0u), w_nh = wave_sum_dpp(nh);
        const uint32_t w_nhal = wave_sum_dpp(nh_al);
        uint32_t* r = s_red(0) + wid * kRedW;
        if (lane == 0) r[0] = kmin, r[1] = kmax, r[2] = c, r[3] = w_allow, r[4] = w_nan, r[5] = w_nh, r[6] = w_nhal;
    }
    TSM_LDS_SYNC();
    uint32_t nallow_seg = 0, nan_seg = 0, nh_seg = 0, nhal_seg = 0;
    gmin = 0xFFFFFFFFu, gmax = 0u, gcnt = 0u;
#pragma unroll
    for (int w = 0; w < kSW; w++) {
        const uint32_t* r = s_red(0) + w * kRedW;
        gmin = r[0] < gmin ? r[0] : gmin;
        gmax = r[1] > gmax ? r[1] : gmax;
        gcnt += r[2];
        nallow_seg += r[3];
        nan_seg += r[4];
        nh_seg += r[5];
        nhal_seg += r[6];
    }
    const float xmax_seg = gcnt ? key_to_float(gmax) : -INFINITY;

    // ---- the threshold for any id from the group maxima ----
    // `need` adds the history ids in the segment, with their repeats: at
    // least the distinct penalized ids among the elements (for the allowed
    // threshold, the allowed ones)
    const uint32_t nlp = (m.logprobs && a.s.out_top_ids != nullptr)
                             ? (m.nlp < a.s.top_stride ? m.nlp : a.s.top_stride)
                             : 0u;
    uint32_t need[2];
    {
        uint32_t base = m.window;
        base = nlp > base ? nlp : base;
        base = base > 1u ? base : 1u;
        need[0] = base + nh_seg;
        need[1] = m.constrained ? m.want + nhal_seg : 0u;
    }
    float tall;
    double lsum_seg = 0.0;
    {
        // -inf when fewer than `need` group maxima are finite (every element
        // counts), the lowest group maximum when all are equal or the span is
        // too narrow to bin, else from a 256-bin histogram
        float lo_v = 0.0f, scale = 0.0f;
        bool binned = false;
        if (gcnt < need[0]) {
            tall = -INFINITY;
        } else {
            lo_v = key_to_float(gmin);
            tall = lo_v;
            if (gmin != gmax) {
                scale = 256.0f / (key_to_float(gmax) - lo_v);
                binned = scale < 1e30f;
            }
        }
        auto bin_of = [&](float vv) -> uint32_t {
            const float bb = (vv - lo_v) * scale;
            return bb < 255.0f ? static_cast<uint32_t>(bb) : 255u;
        };
        if (binned) {
#pragma unroll
            for (int g = 0; g < 8; g++)
                if (gm[g] > -INFINITY) atomicAdd(&s_gh()[bin_of(gm[g])], 1u);
            TSM_LDS_SYNC();
            if (wid == 0) {  // the bin reached counting from the top bin down
                uint32_t c4[4], sm = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    c4[j] = s_gh()[255 - (lane * 4 + j)];
                    sm += c4[j];
                }
                const uint32_t incl = wave_incl_scan(sm), excl = incl - sm;
                if (excl < need[0] && incl >= need[0]) {
                    uint32_t run = excl;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (run + c4[j] >= need[0]) {
                            s_misc()[MS_BSTAR] = 255 - (lane * 4 + j);
                            break;
                        }
                        run += c4[j];
                    }
                }
            }
            TSM_LDS_SYNC();
        }
        // the lowest group maximum in the bins from the one reached up, with
        // the block's logsumexp partial (it needs the segment maximum)
        uint32_t kmin = 0xFFFFFFFFu;
        if (binned) {
            const uint32_t bstar = s_misc()[MS_BSTAR];
#pragma unroll
            for (int g = 0; g < 8; g++) {
                if (gm[g] > -INFINITY && bin_of(gm[g]) >= bstar) {
                    const uint32_t k = canon_key(gm[g]);
                    kmin = k < kmin ? k : kmin;
                }
            }
        }
        kmin = dpp_reduce32(kmin, 0xFFFFFFFFu, [](uint32_t x, uint32_t y) { return x < y ? x : y; });
        double lw = 0.0;
        if (m.logprobs && tmax > -INFINITY && xmax_seg > -INFINITY)
            lw = lsum_t * exp(static_cast<double>(tmax) - static_cast<double>(xmax_seg));
        lw = wave_sum_f64_dpp(lw);
        uint32_t* r = s_red(1) + wid * kRedW;
        if (lane == 0) {
            r[0] = kmin;
            r[1] = static_cast<uint32_t>(__double_as_longlong(lw));
            r[2] = static_cast<uint32_t>(static_cast<uint64_t>(__double_as_longlong(lw)) >> 32);
        }
        TSM_LDS_SYNC();
        uint32_t tk = 0xFFFFFFFFu;
#pragma unroll
        for (int w = 0; w < kSW; w++) {
            const uint32_t* rr = s_red(1) + w * kRedW;
            tk = rr[0] < tk ? rr[0] : tk;
            lsum_seg += __longlong_as_double(static_cast<long long>(static_cast<uint64_t>(rr[1]) |
                                                                    (static_cast<uint64_t>(rr[2]) << 32)));
        }
        if (binned) tall = key_to_float(tk);
    }

    // ---- pass 2: the slots holding an element >= tall, staged per wave
    // (ballot-placed; a lane with nothing to stage writes the dummy slot) ----
    float4* fst = s_fstage() + wid * (kFStage + 1);
    uint32_t* fid = s_fid() + wid * (kFStage + 1);
    uint32_t fpos = 0;
    const bool all_in = !(tall > -INFINITY);  // a -inf threshold: check the range
#pragma unroll
    for (int i = 0; i < kSlots; i++) {
        if (static_cast<uint32_t>(i) >= nslot) continue;
        const uint32_t e0 = lo + 4u * (static_cast<uint32_t>(i) * kSB + tid);
        const float m4 = fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w));
        bool ok = m4 >= tall;
        if (all_in) ok = e0 < hi;
        const uint64_t b = wave_ballot(ok);
        const uint32_t at = fpos + lanes_below(b);
        const uint32_t sl = ok && at < kFStage ? at : kFStage;
        fst[sl] = v[i];
        fid[sl] = e0 | (nib_of(i) << 24);
        fpos += static_cast<uint32_t>(__popcll(b));
    }
    // the allowed ids at or above tall, in the staged slots
    uint32_t al_above = 0;
    if (mrow && fpos <= kFStage) {
        for (uint32_t j = lane; j < fpos; j += kWave) {
            const float4 x = fst[j];
            const uint32_t nb = fid[j] >> 24;
            al_above += ((nb & 1u) && x.x >= tall) + ((nb & 2u) && x.y >= tall) + ((nb & 4u) && x.z >= tall) +
                        ((nb & 8u) && x.w >= tall);
        }
        al_above = wave_sum_dpp(al_above);
    }
    if (lane == 0) {
        s_tmp()[48 + wid] = fpos;
        s_tmp()[52 + wid] = al_above;
    }
    TSM_LDS_SYNC();
    bool ovf = false;
    uint32_t al_seg = 0;
#pragma unroll
    for (int w = 0; w < kSW; w++) {
        ovf |= s_tmp()[48 + w] > kFStage;
        al_seg += s_tmp()[52 + w];
    }
    // ---- pass 3 (constrained rows with too few allowed ids >= tall): the
    // allowed threshold from the allowed ids' group maxima, and the slots
    // holding an allowed id above it ----
    float tal = kNaNf;
    if (mrow && !ovf) {
        if (al_seg >= need[1]) {
            tal = tall;  // every allowed id >= tall is staged, and they are enough
        } else {
            float agm[8];
#pragma unroll
            for (int g = 0; g < 8; g++) agm[g] = -INFINITY;
#pragma unroll
            for (int i = 0; i < kSlots; i++) {
                if (static_cast<uint32_t>(i) >= nslot) continue;
                const float4 x = v[i];
                const uint32_t nb = nib_of(i);
                const float a0 = (nb & 1u) ? x.x : -INFINITY, a1 = (nb & 2u) ? x.y : -INFINITY;
                const float a2 = (nb & 4u) ? x.z : -INFINITY, a3 = (nb & 8u) ? x.w : -INFINITY;
                agm[i & 7] = fmaxf(agm[i & 7], fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)));
            }
            tal = group_threshold(agm, need[1]);  // barriers inside
            const bool al_all = !(tal > -INFINITY);
#pragma unroll
            for (int i = 0; i < kSlots; i++) {
                if (static_cast<uint32_t>(i) >= nslot) continue;
                const uint32_t e0 = lo + 4u * (static_cast<uint32_t>(i) * kSB + tid);
                const float4 x = v[i];
                const uint32_t nb = nib_of(i);
                const float a0 = (nb & 1u) ? x.x : -INFINITY, a1 = (nb & 2u) ? x.y : -INFINITY;
                const float a2 = (nb & 4u) ? x.z : -INFINITY, a3 = (nb & 8u) ? x.w : -INFINITY;
                const float am = fmaxf(fmaxf(a0, a1), fmaxf(a2, a3));
                const float m4 = fmaxf(fmaxf(x.x, x.y), fmaxf(x.z, x.w));
                const bool before = all_in ? e0 < hi : m4 >= tall;  // staged in pass 2
                bool ok = !before && (al_all ? (nb != 0u && e0 < hi) : am >= tal);
                const uint64_t b = wave_ballot(ok);
                const uint32_t at = fpos + lanes_below(b);
                const uint32_t sl = ok && at < kFStage ? at : kFStage;
                fst[sl] = x;
                fid[sl] = e0 | (nb << 24);
                fpos += static_cast<uint32_t>(__popcll(b));
            }
            if (lane == 0) s_tmp()[48 + wid] = fpos;
            TSM_LDS_SYNC();
#pragma unroll
            for (int w = 0; w < kSW; w++) ovf |= s_tmp()[48 + w] > kFStage;
        }
    }
    float tall_out = tall, tal_out = tal;
    uint32_t seg_flags = nan_seg ? SEG_NAN : 0u;
    uint32_t pen_off = 0;
    uint2* const rcand = a.w.cand + static_cast<size_t>(row) * a.nseg * kCandCap;  // the row's area
    // ---- the staged slots' elements that pass, counted: a segment writes
    // at most kCandCap entries (the row's area holds kCandCap per segment),
    // so a segment whose count exceeds it takes the exact thresholds below.
    // The count can: the staging holds up to kSW * kFStage * 4 elements, and
    // with fewer finite group maxima than `need` every element passes ----
    const bool two = tal == tal && tal < tall;
    const bool tal_all = two && !(tal > -INFINITY);
    auto pass = [&](float x, uint32_t nb, int c, uint32_t e) {
        const bool al = (nb >> c) & 1u;
        if (e >= hi) return false;
        return x >= tall || (two && al && (tal_all || x >= tal));
    };
    uint32_t mine = 0;
    if (!ovf) {
        for (uint32_t j = lane; j < fpos; j += kWave) {
            const float4 x = fst[j];
            const uint32_t f = fid[j], e0 = f & kIdMask, nb = f >> 24;
            mine += pass(x.x, nb, 0, e0) + pass(x.y, nb, 1, e0 + 1) + pass(x.z, nb, 2, e0 + 2) + pass(x.w, nb, 3, e0 + 3);
        }
        const uint32_t wn = wave_sum_dpp(mine);
        if (lane == 0) s_tmp()[56 + wid] = wn;
        TSM_LDS_SYNC();  // ovf is the same in every thread: a uniform barrier
        uint32_t seg_total = 0;
#pragma unroll
        for (int w = 0; w < kSW; w++) seg_total += s_tmp()[56 + w];
        ovf = seg_total > kCandCap;
    }
    if (!ovf) {
        // one reservation per wave for its candidates and its history entries
        const uint32_t wn = wave_sum_dpp(mine), wh = m.penal ? wave_sum_dpp(nh) : 0u;
        uint64_t prev = 0;
        if (lane == 0 && (wn | wh))
            prev = dev_add64(&a.w.row_ctr[row], static_cast<uint64_t>(wn) | (static_cast<uint64_t>(wh) << kCtrPenShift));
        prev = (static_cast<uint64_t>(wave_read(static_cast<uint32_t>(prev >> 32), 0)) << 32) |
               wave_read(static_cast<uint32_t>(prev), 0);
        pen_off = ctr_pen(prev);
        uint32_t off = ctr_cand(prev) + wave_incl_scan(mine) - mine;
        for (uint32_t j = lane; j < fpos; j += kWave) {
            const float4 x = fst[j];
            const uint32_t f = fid[j], e0 = f & kIdMask, nb = f >> 24;
            const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (pass(xs[c], nb, c, e0 + c)) {
                    st_entry(rcand + off, __float_as_uint(xs[c]), (e0 + c) | (((nb >> c) & 1u) << 31));
                    off++;
                }
            }
        }
        if (!two) tal_out = mrow ? tall : kNaNf;
    } else {
        // too many for the staging area or for the segment's candidate area
        // (ties, or too few group maxima to bound it): exact thresholds by
        // radix selection, and the entries written straight from the row in
        // memory into a reservation of kCandCap (unused slots skipped).  At
        // most need[0] + need[1] <= 2 * kSplitNeed entries pass them.
        static_assert(2 * kSplitNeed <= kCandCap, "the exact thresholds' entries fit a segment's area");
        seg_flags |= SEG_EXACT;
        const uint64_t ca = seg_select_exact(rowp, mrow, lo, hi, need[0], false);
        const uint64_t cl = mrow ? seg_select_exact(rowp, mrow, lo, hi, need[1], true) : 0ull;
        if (tid == 0) s_misc()[MS_CBASE] = ctr_cand(dev_add64(&a.w.row_ctr[row], kCandCap));
        TSM_LDS_SYNC();
        uint2* sout = rcand + s_misc()[MS_CBASE];
        uint32_t total = 0;
        for (uint32_t bb = lo; bb < hi; bb += kSB) {
            const uint32_t e = bb + tid;
            bool ok = false;
            float x = 0.0f;
            bool al = false;
            if (e < hi) {
                x = rowp[e];
                al = mrow && ((mrow[e >> 5] >> (e & 31)) & 1u);
                if (x == x) {
                    const uint64_t cp = (static_cast<uint64_t>(~canon_key(x)) << 22) | e;
                    ok = cp <= ca || (al && cp <= cl);
                }
            }
            uint32_t t;
            const uint32_t pos = block_excl_scan<kSB>(ok ? 1u : 0u, s_tmp(), &t);
            if (ok && total + pos < kCandCap) st_entry(sout + total + pos, __float_as_uint(x), e | (al ? kEntAllowed : 0u));
            total += t;
        }
        for (uint32_t j = total + tid; j < kCandCap; j += kSB) st_entry(sout + j, 0u, kEntSkip);
        tall_out = ca == ~0ull ? -INFINITY : key_to_float(~static_cast<uint32_t>(ca >> 22));
        tal_out = !mrow ? kNaNf : (cl == ~0ull ? -INFINITY : key_to_float(~static_cast<uint32_t>(cl >> 22)));
        const uint32_t wh = m.penal ? wave_sum_dpp(nh) : 0u;
        uint32_t p = 0;
        if (lane == 0 && wh) p = ctr_pen(dev_add64(&a.w.row_ctr[row], static_cast<uint64_t>(wh) << kCtrPenShift));
        pen_off = wave_read(p, 0);
    }
    // this segment's history ids (with their repeats): raw logit and allowed
    // bit, into the row's list, at the wave's reservation
    if (m.penal) {
        uint32_t off = pen_off + wave_incl_scan(nh) - nh;
        uint2* pl = a.w.pen + static_cast<size_t>(row) * kSplitHist;
#pragma unroll
        for (uint32_t k = 0; k < kHPer; k++) {
            if (!(hid[k] >= lo && hid[k] < hi)) continue;
            const bool al = (hw[k] >> (hid[k] & 31)) & 1u;
            st_entry(pl + off, __float_as_uint(hx[k]), hid[k] | (al ? kEntAllowed : 0u));
            off++;
        }
    }

    // ---- summary, arrival ----
    if (tid == 0) {
        SegSum S;
        S.xmax = xmax_seg;
        S.nallow = nallow_seg;
        S.lsum = lsum_seg;
        S.tall = tall_out;
        S.tal = tal_out;
        S.flags = seg_flags;
        for (int q = 0; q < 5; q++) S.pad[q] = 0;
        st_sum(a.w.sums + static_cast<size_t>(row) * a.nseg + seg, S);
    }
    // The handoff to the row's last workgroup, in the memory model's terms:
    // every thread's stores are released at workgroup scope and meet at the
    // barrier; thread 0's arrival is an agent-scope acquire-release
    // read-modify-write, so the stores of every workgroup that arrived before
    // happen before whatever the last arrival reads after its own arrival
    // (each of its threads acquires at workgroup scope behind the barrier).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (tid == 0) {
        const uint64_t prev = __hip_atomic_fetch_add(&a.w.row_ctr[row], uint64_t{1} << kCtrArrShift, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_misc()[MS_LAST] = ctr_arr(prev) == a.nseg - 1u ? 1u : 0u;
        s_misc()[MS_NSTREAM] = ctr_cand(prev);
        s_misc()[MS_NPEN] = ctr_pen(prev);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (!s_misc()[MS_LAST]) return;

    // ================= finish: the row's last workgroup =================
    const uint32_t nseg = a.nseg;
    const uint32_t nstream = s_misc()[MS_NSTREAM], npen = m.penal ? s_misc()[MS_NPEN] : 0u;
    const SegSum* sums = a.w.sums + static_cast<size_t>(row) * nseg;
    // every load of the finish at once: the segments' summaries, the
    // candidate entries (held in registers when they fit) and the history
    // entries
    FinEnt E;
    SegSum mysum;
    if (tid < nseg) mysum = ld_sum(sums + tid);
    if (nstream <= kFinCap) {
#pragma unroll
        for (int r = 0; r < kFinRegs; r++) {
            const uint32_t j = tid + static_cast<uint32_t>(r) * kSB;
            const uint2 e = j < nstream ? ld_entry(rcand + j) : make_uint2(0u, kEntSkip);
            E.yb[r] = e.x;
            E.idf[r] = e.y;
        }
    }
    {
        const uint2* pl = a.w.pen + static_cast<size_t>(row) * kSplitHist;
#pragma unroll
        for (int r = 0; r < kPenRegs; r++) {
            const uint32_t j = tid + static_cast<uint32_t>(r) * kSB;
            const uint2 e = j < npen ? ld_entry(pl + j) : make_uint2(0u, kEntSkip);
            E.pxb[r] = e.x;
            E.pidf[r] = e.y;
        }
    }
    // row statistics: the raw maximum, the bounds, flags, and the
    // logsumexp (sampler.rs:298-304)
    float xmax_row = -INFINITY, t_star = -INFINITY, tal_star = -INFINITY;
    uint32_t flags_row = 0;
    for (uint32_t sg = tid; sg < nseg; sg += kSB) {
        const SegSum S = sg == tid ? mysum : ld_sum(sums + sg);
        xmax_row = fmaxf(xmax_row, S.xmax);
        t_star = fmaxf(t_star, S.tall);
        if (S.tal == S.tal) tal_star = fmaxf(tal_star, S.tal);
        flags_row |= S.flags;
    }
    {
        uint32_t k0 = dpp_reduce32(canon_key(xmax_row), 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        uint32_t k1 = dpp_reduce32(canon_key(t_star), 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        uint32_t k2 = dpp_reduce32(canon_key(tal_star), 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        uint32_t f = dpp_reduce32(flags_row, 0u, [](uint32_t x, uint32_t y) { return x | y; });
        uint32_t* r = s_red(0) + wid * kRedW;
        if (lane == 0) r[0] = k0, r[1] = k1, r[2] = k2, r[3] = f;
        TSM_LDS_SYNC();
        k0 = k1 = k2 = f = 0u;
#pragma unroll
        for (int w = 0; w < kSW; w++) {
            const uint32_t* q = s_red(0) + w * kRedW;
            k0 = q[0] > k0 ? q[0] : k0;
            k1 = q[1] > k1 ? q[1] : k1;
            k2 = q[2] > k2 ? q[2] : k2;
            f |= q[3];
        }
        xmax_row = key_to_float(k0);
        t_star = key_to_float(k1);
        tal_star = key_to_float(k2);
        flags_row = f;
    }
    float lse = 0.0f;
    if (m.logprobs) {
        double ls = 0.0;
        for (uint32_t sg = tid; sg < nseg; sg += kSB) {
            const SegSum S = sg == tid ? mysum : ld_sum(sums + sg);
            if (S.xmax > -INFINITY) ls += S.lsum * exp(static_cast<double>(S.xmax) - static_cast<double>(xmax_row));
        }
        ls = block_sum_d(ls);
        lse = xmax_row + static_cast<float>(log(ls));
        if (flags_row & SEG_NAN) lse = kNaNf;  // a NaN logit makes the reference's sum NaN
    }
    if (flags_row & SEG_NAN) {
        serial::Row r;
        r.x = rowp;
        r.n = n;
        r.hist = (a.s.hist_ids && hlen) ? a.s.hist_ids + h0 : nullptr;
        r.hlen = r.hist ? hlen : 0u;
        r.mrow = mrow;
        r.m = m;
        r.P = P;
        r.u = a.s.distribution ? 0.0f : a.s.uniforms[row];
        fin_nan(a, r, row, nlp);
        return;
    }
    FinSrc S;
    S.cbase = rcand;
    S.nstream = nstream;
    S.t_star = t_star;
    S.tal_star = tal_star;
    S.penal = m.penal;
    if (nstream <= kFinCap)
        fin_row<false>(a, S, m, P, row, nlp, lse, flags_row, E);
    else
        fin_row<true>(a, S, m, P, row, nlp, lse, flags_row, E);
}

template __global__ void split_kernel<true>(SplitArgs);
template __global__ void split_kernel<false>(SplitArgs);

// ---- host side ---------------------------------------------------------------------

uint32_t pick_seg_len(uint32_t rows, uint32_t usable) {
    // about 2048 workgroups per step (8 per CU), each segment between kSegMin
    // and kSegMax ids, at most kMaxSegs segments per row
    const uint64_t ids = static_cast<uint64_t>(rows) * usable;
    uint64_t len = (ids + 2047) / 2048;
    if (len < kSegMin) len = kSegMin;
    if (len > kSegMax) len = kSegMax;
    const uint64_t min_len = (static_cast<uint64_t>(usable) + kMaxSegs - 1) / kMaxSegs;
    if (len < min_len) len = min_len;
    len = (len + kSegQuant - 1) / kSegQuant * kSegQuant;
    if (len > kSegMax) len = kSegMax;
    return static_cast<uint32_t>(len);
}

SplitScratch scratch_carve(void* base, uint32_t rows, uint32_t vocab) {
    const uint64_t segs = max_segments(rows, vocab);
    char* p = static_cast<char*>(base);
    SplitScratch w;
    w.sums = reinterpret_cast<SegSum*>(p);
    p += align256(segs * sizeof(SegSum));
    w.cand = reinterpret_cast<uint2*>(p);
    p += align256(segs * kCandCap * sizeof(uint2));
    w.pen = reinterpret_cast<uint2*>(p);
    p += align256(static_cast<size_t>(rows) * kSplitHist * sizeof(uint2));
    w.row_ctr = reinterpret_cast<uint64_t*>(p);
    return w;
}

void launch(const SplitArgs& a, uint32_t rows, bool vec_loads, hipStream_t stream) {
    const dim3 grid(a.nseg, rows);
    if (vec_loads)
        hipLaunchKernelGGL(split_kernel<true>, grid, dim3(kSB), kSmemSplit, stream, a);
    else
        hipLaunchKernelGGL(split_kernel<false>, grid, dim3(kSB), kSmemSplit, stream, a);
}

}  // namespace split
}  // namespace tsm
