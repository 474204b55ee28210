// tsm_nucleus.h - rows without top-k whose nucleus holds more than 1024
// candidates (the cutoff set, sampler.rs:195-208): the reference's sequential
// f32 folds reproduced exactly, over value bins.
//
// The reference folds best first, in f32: total = sum of p_j; acc += p_j /
// total until acc >= top_p (sampler.rs:238-245); mass = the kept prefix's sum
// (sampler.rs:142); r = u * mass, r -= p_j until r <= 0 (sampler.rs:143-149).
// While a fold's value x stays in one binade [2^e, 2^(e+1)), the step x + tau
// rounds tau to the grid 2^(e-23): it adds RN_e(tau) grid units whatever the
// order of the terms, unless tau lies exactly halfway between two grid points
// (then the result's parity decides).  A subtraction rounds on the grid of its
// result, the binade below when x is a power of two.  So over a value bin (a
// range of values: a contiguous stretch of the sorted list) a fold advances by
// the bin's sum of RN_e terms, as long as it neither leaves the binade nor
// meets such a tie nor reaches its decision inside the bin.
//
// A re-read pass computes, per bin, the sums for the one or two grids the bin
// can see (planned from approximate cumulative masses), and a census of the
// bins where the fold steps element by element (binade crossings, ties,
// decisions): their distinct values with multiplicities and smallest ids, in
// list order.  Wave 0 then walks the bins, 64 per step, with a prefix sum of
// their grid sums, up to the first bin that leaves the binade, holds a tie,
// decides, or was planned for another grid; that bin is stepped through its
// distinct values (64 per step the same way, runs of equal values in closed
// form, single exact f32 steps where needed).  A bin the census lacks is
// censused by one more re-read, and the walk resumes where it stopped.
//
// Passes over the row: the maximum, the bin counts and approximate masses,
// the grid sums of total and of the draw (with the census), the grid sums of
// acc once total is known (with a census), and a census round where a walk
// meets a bin the census lacks.
#pragma once

#include "tsm_select.h"

namespace tsm {
namespace nuc {

constexpr uint32_t kNB = kBins;     // value bins
constexpr uint32_t kHS = 2048;      // census capacity: distinct values
constexpr uint32_t kReqMax = 512;   // bins per census
constexpr uint32_t kReqCnt = kHS / 2;      // candidates per census (distinct values at most that many)
constexpr uint32_t kNoBin = 0xFFFFFFFFu;
constexpr uint32_t kBL = 4;         // bins per lane in a walk step

// ---- LDS layout (above the re-read pass's per-tile history counts) ----------
constexpr uint32_t kOffE = kOffRank;
constexpr uint32_t kOffECnt = kOffE;                     // u32[kNB] candidates per bin
constexpr uint32_t kOffEMass = kOffECnt + kNB * 4;       // f64[kNB] approximate masses; after planning:
constexpr uint32_t kOffESStart = kOffEMass;              //   f32[kNB] total's fold value at each bin start
constexpr uint32_t kOffEPStart = kOffEMass + kNB * 4;    //   u32[kNB] candidates before each bin
constexpr uint32_t kOffELay = kOffEMass + kNB * 8;       // u32[kNB] candidates before each coarse bin
constexpr uint32_t kOffEPlan = kOffELay + kNB * 4;       // u32[kNB] grid plans
constexpr uint32_t kOffESum = kOffEPlan + kNB * 4;       // u32[4][kNB] grid sums
constexpr uint32_t kOffETie = kOffESum + 4 * kNB * 4;    // u32[4 * kNB / 32] sums with a tie or invalid
constexpr uint32_t kOffETieB = kOffETie + kNB * 4 / 8;   // u32[4 * kNB / 32] sums invalid (or two ties)
constexpr uint32_t kOffEReq = kOffETieB + kNB * 4 / 8;   // u32[kNB / 32] census requests
constexpr uint32_t kOffECpl = kOffEReq + kNB / 8;        // u32[kNB / 32] censused completely
constexpr uint32_t kOffEWpre = kOffECpl + kNB / 8;       // u32[kNB / 32] requests before each word
constexpr uint32_t kOffEBcnt = kOffEWpre + kNB / 8;      // u32[kReqMax] census buckets
constexpr uint32_t kOffEXreq = kOffEBcnt + kReqMax * 4;  // u32[3][kNB / 32] bins each fold expects to step through
constexpr uint32_t kOffETmpB = kOffEXreq + 3 * kNB / 8;  // u32[kNB / 32] request staging
constexpr uint32_t kOffESc = kOffETmpB + kNB / 8;        // u32[32] scalars
constexpr uint32_t kOffEScd = kOffESc + 32 * 4;          // f64[8]
constexpr uint32_t kOffEHKey = kOffEScd + 8 * 8;         // u32[kHS] census keys; runs after census_finish
constexpr uint32_t kOffEHCnt = kOffEHKey + kHS * 4;      // u32[kHS] multiplicities
constexpr uint32_t kOffEHMin = kOffEHCnt + kHS * 4;      // u32[kHS] smallest ids
constexpr uint32_t kOffESort = kOffEHMin + kHS * 4;      // u64[kHS] bucket sort; then u32 run bins
constexpr uint32_t kOffERunP = kOffESort + kHS * 8;      // f32[kHS] run probabilities
constexpr uint32_t kOffEExp = kOffERunP + kHS * 4;       // u64[32] the expf table
constexpr uint32_t kOffESHi = kOffEExp + 32 * 8;         // f32[kNB] total's value at bin starts, ties up
// crowded coarse bins (see FBins): a count, kCrowd coarse bin ids, then each
// one's cumulative-count table at its kSub + 1 sub-bin edges
constexpr uint32_t kCrowd = 3;
constexpr uint32_t kSub = 256;
constexpr uint32_t kOffECrowd = kOffESHi + kNB * 4;      // u32[4]: slots used, coarse bins
constexpr uint32_t kOffECdf = kOffECrowd + 16;           // u16[kCrowd][kSub + 1] sub-bin edges' CDF (of 65535)
constexpr uint32_t kOffEEnd = kOffECdf + ((kCrowd * (kSub + 1) * 2 + 7) & ~7u);
static_assert(kOffEMass % 8 == 0 && kOffEScd % 8 == 0 && kOffESort % 8 == 0 && kOffEExp % 8 == 0,
              "8-byte LDS records");
static_assert(kOffEEnd <= kOffMisc, "engine LDS overlaps the row's scalars");

__device__ __forceinline__ uint32_t* e_u32(uint32_t off) { return reinterpret_cast<uint32_t*>(lds_base() + off); }
__device__ __forceinline__ uint32_t* e_cnt() { return e_u32(kOffECnt); }
__device__ __forceinline__ double* e_mass() { return reinterpret_cast<double*>(lds_base() + kOffEMass); }
__device__ __forceinline__ float* e_sstart() { return reinterpret_cast<float*>(lds_base() + kOffESStart); }
__device__ __forceinline__ uint32_t* e_pstart() { return e_u32(kOffEPStart); }
__device__ __forceinline__ uint32_t* e_lay() { return e_u32(kOffELay); }
__device__ __forceinline__ uint32_t* e_plan() { return e_u32(kOffEPlan); }
__device__ __forceinline__ uint32_t* e_sum(uint32_t slot) { return e_u32(kOffESum + slot * kNB * 4); }
__device__ __forceinline__ uint32_t* e_tie() { return e_u32(kOffETie); }
__device__ __forceinline__ uint32_t* e_tieb() { return e_u32(kOffETieB); }
__device__ __forceinline__ float* e_shi() { return reinterpret_cast<float*>(lds_base() + kOffESHi); }
__device__ __forceinline__ uint32_t* e_req() { return e_u32(kOffEReq); }
__device__ __forceinline__ uint32_t* e_cpl() { return e_u32(kOffECpl); }
__device__ __forceinline__ uint32_t* e_wpre() { return e_u32(kOffEWpre); }
__device__ __forceinline__ uint32_t* e_bcnt() { return e_u32(kOffEBcnt); }
__device__ __forceinline__ uint32_t* e_xreq(int k) { return e_u32(kOffEXreq + static_cast<uint32_t>(k) * kNB / 8); }
__device__ __forceinline__ uint32_t* e_tmpb() { return e_u32(kOffETmpB); }
__device__ __forceinline__ uint32_t* e_sc() { return e_u32(kOffESc); }
__device__ __forceinline__ double* e_scd() { return reinterpret_cast<double*>(lds_base() + kOffEScd); }
__device__ __forceinline__ uint32_t* e_hkey() { return e_u32(kOffEHKey); }
__device__ __forceinline__ uint32_t* e_hcnt() { return e_u32(kOffEHCnt); }
__device__ __forceinline__ uint32_t* e_hmin() { return e_u32(kOffEHMin); }
__device__ __forceinline__ uint64_t* e_sort() { return reinterpret_cast<uint64_t*>(lds_base() + kOffESort); }
__device__ __forceinline__ uint32_t* e_rbin() { return e_u32(kOffESort); }
__device__ __forceinline__ float* e_runp() { return reinterpret_cast<float*>(lds_base() + kOffERunP); }
__device__ __forceinline__ uint64_t* e_exptab() { return reinterpret_cast<uint64_t*>(lds_base() + kOffEExp); }
__device__ __forceinline__ uint32_t* e_crowd() { return e_u32(kOffECrowd); }
__device__ __forceinline__ uint16_t* e_cdf(uint32_t slot) {
    return reinterpret_cast<uint16_t*>(lds_base() + kOffECdf) + slot * (kSub + 1u);
}

enum : uint32_t {  // e_sc() words
    SC_FIRST = 0,   // first nonempty bin
    SC_LAST = 1,    // last nonempty bin
    SC_NAN = 2,     // a candidate is NaN
    SC_KLO = 3,     // predicted top-p bins: first, last
    SC_KHI = 4,
    SC_NRUNS = 5,   // runs of the current census
    SC_RES = 6,     // walk: result, next bin, position, run, index within run, x bits
    SC_B = 7,
    SC_POS = 8,
    SC_RUN = 9,
    SC_WITHIN = 10,
    SC_X = 11,
    SC_OVF = 12,    // census table full
    SC_CMIN = 13,   // smallest candidate value's total key
    SC_TIED = 14,   // walk: a bin sum it added holds a tie
};

// Grid plan of a bin, one byte per fold for the lower grid's binade (+128)
// and one of flags.
enum : uint32_t {
    PF_TWO_S = 1u << 24, PF_TWO_R = 1u << 25, PF_TWO_A = 1u << 26,
    PF_MUST_S = 1u << 27, PF_MUST_R = 1u << 28, PF_MUST_A = 1u << 29,
    PF_R = 1u << 30,  // the draw may reach this bin
};
enum : int { FK_S = 0, FK_A = 1, FK_R = 2 };  // total (and the kept mass), acc, the draw
enum : uint32_t { SL_S0 = 0, SL_S1 = 1, SL_R0 = 2, SL_R1 = 3 };  // acc reuses slots 0 and 1
enum : uint32_t { W_DONE = 0, W_NEED = 1, W_DECIDED = 2 };

__device__ __forceinline__ uint32_t plan_shift(int k) { return k == FK_S ? 0u : k == FK_R ? 8u : 16u; }
__device__ __forceinline__ uint32_t plan_two(int k) { return k == FK_S ? PF_TWO_S : k == FK_R ? PF_TWO_R : PF_TWO_A; }
__device__ __forceinline__ uint32_t plan_must(int k) {
    return k == FK_S ? PF_MUST_S : k == FK_R ? PF_MUST_R : PF_MUST_A;
}
__device__ __forceinline__ uint32_t slot0(int k) { return k == FK_R ? SL_R0 : SL_S0; }

__device__ __forceinline__ bool tie_bit(uint32_t slot, uint32_t b) {
    const uint32_t i = slot * kNB + b;
    return (e_tie()[i >> 5] >> (i & 31u)) & 1u;
}
// The sum cannot bound the bin's steps (a term too large, a possible wrap, or
// more than one tie).
__device__ __forceinline__ bool bad_bit(uint32_t slot, uint32_t b) {
    const uint32_t i = slot * kNB + b;
    return (e_tieb()[i >> 5] >> (i & 31u)) & 1u;
}
__device__ __forceinline__ bool bit_of(const uint32_t* w, uint32_t b) { return (w[b >> 5] >> (b & 31u)) & 1u; }

// ---- grids -------------------------------------------------------------------
// floor(log2 x) for x > 0 (subnormals: -127, whose grid is that of -126).
__device__ __forceinline__ int binade_of(float x) {
    const int ex = static_cast<int>((__float_as_uint(x) >> 23) & 0xFFu);
    return ex == 0 ? -127 : ex - 127;
}
// log2 of the spacing of floats in binade e.
__device__ __forceinline__ int grid_of(int e) { return (e < -126 ? -126 : e) - 23; }
// The binade whose grid a step from x > 0 rounds on: x's own, or for a
// subtraction from an exact power of two the one below.
__device__ __forceinline__ int step_binade(float x, bool sub) {
    int e = binade_of(x);
    if (sub && (__float_as_uint(x) & 0x7FFFFFu) == 0u && e > -126) e -= 1;
    return e;
}

constexpr uint32_t kTieTerm = 0xFFFFFFFFu;  // tau halfway between grid points
constexpr uint32_t kBigTerm = 0xFFFFFFFEu;  // tau >= 2^(e+1): no grid sum holds its step
// RN_e(tau) in grid units of binade e, or kTieTerm (tau exactly halfway
// between grid points; *fl gets the lower one) or kBigTerm.
__device__ __forceinline__ uint32_t grid_term(float tau, int e, uint32_t* fl = nullptr) {
    if (!(tau < ldexpf(1.0f, e + 1))) return kBigTerm;
    const float v = ldexpf(tau, -grid_of(e));  // < 2^24: exact
    const float k = floorf(v);
    const float fr = v - k;
    if (fl) *fl = static_cast<uint32_t>(k);
    if (fr == 0.5f) return kTieTerm;
    return static_cast<uint32_t>(k) + (fr > 0.5f ? 1u : 0u);
}

__device__ __forceinline__ uint64_t wave_incl_scan64(uint64_t v, uint32_t lane) {
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint64_t w = __shfl_up(v, static_cast<unsigned>(o), kWave);
        if (lane >= static_cast<uint32_t>(o)) v += w;
    }
    return v;
}
__device__ __forceinline__ uint32_t first_lane(uint64_t mask) {
    return mask ? static_cast<uint32_t>(__builtin_ctzll(mask)) : 64u;
}
__device__ __forceinline__ uint64_t wave_read64(uint64_t v, uint32_t lane) {
    const uint32_t lo = wave_read(static_cast<uint32_t>(v), lane);
    const uint32_t hi = wave_read(static_cast<uint32_t>(v >> 32), lane);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ---- bins -----------------------------------------------------------------------
// Fine bins of about equal counts: with C(c) the candidates in coarse bins
// (VBins) before c and n(c) those in c, a value at fraction fr of coarse bin
// c goes to fine bin floor((C(c) + fr * n(c)) * kNB / len).  Monotone in y
// (fine bins keep the list order), equal values share a bin, and a value
// spread that is even inside each coarse bin gives each fine bin about len /
// kNB candidates.  e_lay()[c] = C(c); scale = kNB / len (0: fine = coarse).
//
// A coarse bin whose values are far from even inside it (a dense cluster
// narrower than the bin) can leave one fine bin more candidates than a census
// round takes.  Such a bin (crowded: up to kCrowd of them, cr[]) is laid out
// from a histogram of its own: fr is replaced by the bin's cumulative count
// at fr, interpolated linearly between its kSub sub-bin edges, so its fine
// bins hold about equal counts at the sub-bin's resolution.  The map stays
// monotone in y (the edges' counts never fall) and a function of y alone.
__device__ __forceinline__ float crowd_frac(const uint16_t* F, float fr) {
    const float x = fr * static_cast<float>(kSub);
    const uint32_t j = x < static_cast<float>(kSub - 1u) ? static_cast<uint32_t>(x) : kSub - 1u;
    const float w = x - static_cast<float>(j);  // in [0, 1]
    const float a = static_cast<float>(F[j]), b = static_cast<float>(F[j + 1u]);
    const float v = (a + w * (b - a)) * (1.0f / 65535.0f);
    return v < 1.0f ? v : 1.0f;
}
struct FBins {
    VBins vb;
    float scale;
    uint32_t cr[kCrowd];  // crowded coarse bins laid out from their own sub-histogram (kNoBin: none)
    __device__ __forceinline__ float frac(float y, uint32_t c) const {
        const float fr = vb.pos(y) - static_cast<float>(c);
        return fr > 0.0f ? (fr < 1.0f ? fr : 1.0f) : 0.0f;
    }
    __device__ __forceinline__ uint32_t bin(float y) const {
        const uint32_t c = vb.bin(y);
        if (scale == 0.0f) return c;
        const uint32_t c0 = e_lay()[c], c1 = c + 1u < kNB ? e_lay()[c + 1u] : c0 + (kNB - 1u);
        float fr = frac(y, c);
#pragma unroll
        for (uint32_t s = 0; s < kCrowd; s++)
            if (c == cr[s]) fr = crowd_frac(e_cdf(s), fr);
        const float v = (static_cast<float>(c0) + fr * static_cast<float>(c1 - c0)) * scale;
        return v >= static_cast<float>(kNB - 1u) ? kNB - 1u : static_cast<uint32_t>(v);
    }
};

// ---- census -------------------------------------------------------------------
// Requested bins in bin order get bucket numbers.
__device__ __forceinline__ uint32_t req_rank(uint32_t b) {
    return e_wpre()[b >> 5] + static_cast<uint32_t>(__popc(e_req()[b >> 5] & ((1u << (b & 31u)) - 1u)));
}

// Empties the census table for the requested bins (at most kReqMax bins and
// kReqCnt candidates, as request_bins leaves them).
__device__ void census_clear() {
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < kHS; i += kBlock) {
        e_hkey()[i] = 0u;
        e_hcnt()[i] = 0u;
        e_hmin()[i] = 0xFFFFFFFFu;
    }
    if (tid < kWave) {  // one request word per lane
        const uint32_t w = e_req()[tid];
        const uint32_t c = static_cast<uint32_t>(__popc(w));
        e_wpre()[tid] = wave_incl_scan(c) - c;
        e_cpl()[tid] = w;
        if (tid == 0) e_sc()[SC_OVF] = 0u;
    }
    TSM_LDS_SYNC();
}

__device__ __forceinline__ void census_insert(uint32_t key, uint32_t id, uint32_t b) {
    const uint32_t h = (key * 0x9E3779B1u) >> 21;
    for (uint32_t i = 0; i < 64u; i++) {
        const uint32_t s = (h + i) & (kHS - 1u);
        const uint32_t k = atomicCAS(&e_hkey()[s], 0u, key);
        if (k == 0u || k == key) {
            atomicAdd(&e_hcnt()[s], 1u);
            atomicMin(&e_hmin()[s], id);
            return;
        }
    }
    atomicAnd(&e_cpl()[b >> 5], ~(1u << (b & 31u)));  // no free slot near: the bin stays incomplete
    e_sc()[SC_OVF] = 1u;
}

// Turns the census into runs in list order (value descending): key,
// multiplicity, smallest id, bin and p = exp((y - y0) / t), each bucket (one
// bin) ranked by comparing keys.  Returns the number of runs.
__device__ uint32_t census_finish(const FBins& vb, float t) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < kReqMax; i += kBlock) e_bcnt()[i] = 0u;
    TSM_LDS_SYNC();
    for (uint32_t s = tid; s < kHS; s += kBlock) {
        const uint32_t key = e_hkey()[s];
        if (key) atomicAdd(&e_bcnt()[req_rank(vb.bin(key_to_float(key)))], 1u);
    }
    TSM_LDS_SYNC();
    uint32_t total;
    const uint32_t v = tid < kReqMax ? e_bcnt()[tid] : 0u;
    const uint32_t ex = block_excl_scan<kBlock>(v, reinterpret_cast<uint32_t*>(lds_base() + kOffTmp), &total);
    if (tid < kReqMax) e_bcnt()[tid] = ex;
    TSM_LDS_SYNC();
    for (uint32_t s = tid; s < kHS; s += kBlock) {
        const uint32_t key = e_hkey()[s];
        if (key) {
            const uint32_t pos = atomicAdd(&e_bcnt()[req_rank(vb.bin(key_to_float(key)))], 1u);
            e_sort()[pos] = (static_cast<uint64_t>(~key) << 32) | s;
        }
    }
    TSM_LDS_SYNC();
    // e_bcnt()[i] is now the end of bucket i
    constexpr uint32_t kPer = kHS / kBlock;
    uint32_t fin[kPer], fk[kPer], fc[kPer], fm[kPer], fb[kPer];
    float fp[kPer];
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
        const uint32_t pos = tid + k * kBlock;
        fin[k] = 0xFFFFFFFFu;
        if (pos < total) {
            const uint64_t me = e_sort()[pos];
            const uint32_t key = ~static_cast<uint32_t>(me >> 32), slot = static_cast<uint32_t>(me);
            const float y = key_to_float(key);
            const uint32_t b = vb.bin(y);
            const uint32_t ci = req_rank(b);
            const uint32_t bs = ci ? e_bcnt()[ci - 1] : 0u, be = e_bcnt()[ci];
            uint32_t rank = 0;
            for (uint32_t j = bs; j < be; j++) rank += e_sort()[j] < me ? 1u : 0u;
            fin[k] = bs + rank;
            fk[k] = key;
            fc[k] = e_hcnt()[slot];
            fm[k] = e_hmin()[slot];
            fb[k] = b;
            fp[k] = glibc_expf_lds((y - vb.vb.y0) / t, e_exptab());
        }
    }
    TSM_LDS_SYNC();
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++)
        if (fin[k] != 0xFFFFFFFFu) {
            e_hkey()[fin[k]] = fk[k];
            e_hcnt()[fin[k]] = fc[k];
            e_hmin()[fin[k]] = fm[k];
            e_rbin()[fin[k]] = fb[k];
            e_runp()[fin[k]] = fp[k];
        }
    if (tid == 0) e_sc()[SC_NRUNS] = total;
    TSM_LDS_SYNC();
    return total;
}

// The first run whose bin is >= b (or > b with `after`): a 64-way search in
// two steps (each lane tests one position).  Wave-uniform; every lane of the
// wave takes part.
__device__ __forceinline__ uint32_t runs_bound(uint32_t b, uint32_t nruns, bool after) {
    const uint32_t lane = lane_id();
    auto below = [&](uint32_t pos) { return pos < nruns && (after ? e_rbin()[pos] <= b : e_rbin()[pos] < b); };
    static_assert(kHS <= 64u * 64u, "two 64-way steps cover the runs");
    // step 1: blocks of 64 runs; lane l tests the last run of block l
    const uint32_t nb1 = static_cast<uint32_t>(__popcll(wave_ballot(below(lane * 64u + 63u))));
    const uint32_t base = nb1 * 64u;  // runs before base are all below
    const uint32_t nb2 = static_cast<uint32_t>(__popcll(wave_ballot(below(base + lane))));
    const uint32_t r = base + nb2;
    return r < nruns ? r : nruns;
}
// First run of bin b and the end of its runs.
__device__ __forceinline__ void runs_of(uint32_t b, uint32_t nruns, uint32_t* r0, uint32_t* r1) {
    *r0 = runs_bound(b, nruns, false);
    *r1 = runs_bound(b, nruns, true);
}

// ---- stepping one run of equal terms ----------------------------------------
// m steps of x <- x + tau (S, A) or x <- x - tau (R) in f32, exactly as the
// reference's loop computes them, stopping at the decision (A: x >= thr;
// R: x <= 0).  Steps that stay in one binade without a tie repeat the same
// grid increment and are taken together.  Returns the steps taken (with the
// deciding one).  Wave-uniform scalar code.
template <int K>
__device__ uint32_t run_steps(float& x, float tau, uint32_t m, float thr, bool* decided) {
    constexpr bool sub = K == FK_R;
    uint32_t done = 0;
    *decided = false;
    while (done < m) {
        const float nx = sub ? x - tau : x + tau;
        const bool dec = K == FK_A ? (nx >= thr) : (K == FK_R ? (nx <= 0.0f) : false);
        if (dec) {
            x = nx;
            *decided = true;
            return done + 1;
        }
        if (x > 0.0f) {
            const int e = step_binade(x, sub);
            const int g = grid_of(e);
            const uint32_t c = grid_term(tau, e);
            if (c < kBigTerm) {
                const uint64_t M = static_cast<uint64_t>(ldexpf(x, -g));
                const uint32_t left = m - done;
                if (c == 0u) return m;  // every remaining step rounds back to x, and none decides
                uint64_t n;
                if (sub) {
                    n = M > (1ull << 23) ? (M - (1ull << 23) - 1u) / c : 0u;  // stays above 2^e
                } else {
                    n = ((1ull << 24) - M) / c;  // stays at or below 2^(e+1)
                    if (K == FK_A) {
                        const uint64_t mt = static_cast<uint64_t>(ceilf(ldexpf(thr, -g)));
                        const uint64_t nd = mt > M ? (mt - M - 1u) / c : 0u;  // stays below thr
                        n = n < nd ? n : nd;
                    }
                }
                if (n > left) n = left;
                if (n > 0u) {
                    const uint64_t M2 = sub ? M - n * c : M + n * c;
                    x = ldexpf(static_cast<float>(M2), g);
                    done += static_cast<uint32_t>(n);
                    continue;
                }
            }
        }
        x = nx;
        done++;
    }
    return done;
}

struct Walk {
    float x;          // the fold's value
    uint32_t b;       // next bin
    uint32_t pos;     // candidates folded so far
    uint32_t run;     // W_DECIDED: the deciding run and the index within it
    uint32_t within;
    uint32_t tied;    // a bound walk added a bin sum holding a tie (else its result is exact)
};

// The runs [r0, r1) of one bin, in order, folding at most up to candidate
// `lim` (the kept count; ~0 for no limit).  Wave 0.
template <int K>
__device__ uint32_t walk_runs(Walk& w, uint32_t r0, uint32_t r1, float T, float thr, uint32_t lim) {
    constexpr bool sub = K == FK_R;
    const uint32_t lane = lane_id();
    uint32_t i = r0;
    while (i < r1) {
        if (w.x > 0.0f) {
            const int e = step_binade(w.x, sub);
            const int g = grid_of(e);
            const uint64_t M = static_cast<uint64_t>(ldexpf(w.x, -g));
            const uint32_t j = i + lane;
            uint32_t mraw = j < r1 ? e_hcnt()[j] : 0u;
            const uint32_t mpre = wave_incl_scan(mraw) - mraw;
            const uint32_t room = lim - w.pos;  // lim >= w.pos
            uint32_t m = mpre >= room ? 0u : (mraw < room - mpre ? mraw : room - mpre);
            bool ok = j < r1 && m > 0u;
            uint64_t c = 0;
            if (ok) {
                const float p = e_runp()[j];
                const float tau = K == FK_A ? p / T : p;
                const uint32_t t = grid_term(tau, e);
                if (t >= kBigTerm) ok = false;
                else c = static_cast<uint64_t>(m) * t;
            }
            // past 2^25 units a lane leaves the binade anyway: the clamp keeps
            // the prefix sums in 32 bits
            const uint32_t c32 = c > (1ull << 25) ? (1u << 25) : static_cast<uint32_t>(c);
            const uint64_t incl = wave_incl_scan(c32);
            const uint64_t excl = incl - c32;
            bool bad = !ok;
            bool restart = false;
            if (sub) {
                const int64_t end = static_cast<int64_t>(M) - static_cast<int64_t>(incl);
                bad |= end <= static_cast<int64_t>(1ull << 23);
            } else {
                const uint64_t start = M + excl, end = M + incl;
                restart = start >= (1ull << 24);
                bad |= restart || end > (1ull << 24);
                if (K == FK_A) bad |= end >= static_cast<uint64_t>(ceilf(ldexpf(thr, -g)));
            }
            const uint32_t f = first_lane(wave_ballot(bad));
            const uint32_t fl = f < 64u ? f : 63u;
            const uint64_t applied = f < 64u ? wave_read64(excl, fl) : wave_read64(incl, 63u);
            const uint32_t mapplied = f < 64u ? wave_read(mpre, fl) : wave_read(mpre + m, 63u);
            const uint64_t M2 = sub ? M - applied : M + applied;
            w.x = ldexpf(static_cast<float>(M2), g);
            w.pos += mapplied;
            i += f < 64u ? f : 64u;
            if (f == 64u) continue;
            if (i >= r1 || w.pos >= lim) return W_DONE;
            if (wave_read(restart ? 1u : 0u, fl)) continue;
        }
        // one run exactly
        const uint32_t mraw = e_hcnt()[i];
        const uint32_t room = lim - w.pos;
        const uint32_t m = mraw < room ? mraw : room;
        if (m == 0u) return W_DONE;
        const float p = e_runp()[i];
        const float tau = K == FK_A ? p / T : p;
        bool dec;
        const uint32_t steps = run_steps<K>(w.x, tau, m, thr, &dec);
        w.pos += steps;
        if (dec) {
            w.run = i;
            w.within = steps - 1u;
            return W_DECIDED;
        }
        i++;
    }
    return W_DONE;
}

// The bins from w.b up to bend, in order (wave 0).  A bin is added as its grid
// sum when its plan holds the fold's grid, no step in it ties or runs past
// its sum's range, and the fold stays in its binade and undecided through it;
// otherwise it is stepped through its census runs (W_NEED when the census
// lacks it).  `force` is a bin always stepped through (the kept count's bin,
// whose sums also count candidates past it).  Total's walk records the fold
// value and position at every bin start.
template <int K, int kB = 0>
__device__ uint32_t walk_bins(Walk& w, uint32_t bend, uint32_t nruns, float T, float thr, uint32_t force,
                              uint32_t lim) {
    constexpr bool sub = K == FK_R;
    const uint32_t lane = lane_id();
    while (w.b < bend) {
        bool expand = false;
        if (w.x == 0.0f) {
            // the first step starts from zero: the first nonempty bin is stepped through
            const uint32_t b = w.b + lane;
            const uint32_t n = b < bend ? e_cnt()[b] : 0u;
            const uint32_t f = first_lane(wave_ballot(n > 0u || b >= bend));
            if (K == FK_S && b < bend && lane <= f) {
                if (kB != 2) e_sstart()[b] = 0.0f;
                if (kB != 1) e_shi()[b] = 0.0f;
                if (kB != 2) e_pstart()[b] = w.pos;  // the ties-up walk runs beside the ties-down one
            }
            if (f == 64u) {
                w.b += 64u;
                continue;
            }
            w.b += f;
            if (w.b >= bend) break;
            expand = true;
        } else {
            // kBL bins per lane: lane l takes bins w.b + kBL*l .. + kBL-1
            const int e = step_binade(w.x, sub);
            const int g = grid_of(e);
            const uint64_t M = static_cast<uint64_t>(ldexpf(w.x, -g));
            const uint64_t mthr = K == FK_A ? static_cast<uint64_t>(ceilf(ldexpf(thr, -g))) : 0u;
            const uint32_t bl = w.b + kBL * lane;
            uint32_t nj[kBL], cj[kBL];
            bool okj[kBL];
            uint32_t ln = 0, lc = 0, tmask = 0;  // tmask: the lane's summable bins holding a tie
#pragma unroll
            for (uint32_t j = 0; j < kBL; j++) {
                const uint32_t b = bl + j;
                uint32_t n = 0;
                bool ok = b < bend;  // past bend: the end marker
                uint64_t c = 0;
                if (ok) {
                    n = e_cnt()[b];
                    if (n) {
                        const uint32_t pw = e_plan()[b];
                        const int g0 = static_cast<int>((pw >> plan_shift(K)) & 0xFFu) - 128;
                        uint32_t slot = 0xFFFFFFFFu;
                        if (!(pw & plan_must(K)) && (K != FK_R || (pw & PF_R))) {
                            if (e == g0) slot = slot0(K);
                            else if (e == g0 + 1 && (pw & plan_two(K))) slot = slot0(K) + 1u;
                        }
                        // exact walks step through a bin with a tie; bound walks
                        // take its lower (kB 1) or upper (kB 2) end
                        ok = slot != 0xFFFFFFFFu && b != force &&
                             (kB == 0 ? !tie_bit(slot, b) : !bad_bit(slot, b));
                        if (ok) {
                            const bool tie = kB != 0 && tie_bit(slot, b);
                            c = static_cast<uint64_t>(e_sum(slot)[b]) + (kB == 2 && tie ? 1u : 0u);
                            if (tie) tmask |= 1u << j;
                        }
                    }
                }
                // past 2^25 units a bin leaves the binade anyway: the clamps keep
                // the prefix sums in 32 bits
                cj[j] = c > (1ull << 25) ? (1u << 25) : static_cast<uint32_t>(c);
                nj[j] = n;
                okj[j] = ok;
                ln += n;
                lc = min(lc + cj[j], 1u << 25);
            }
            const uint32_t npre = wave_incl_scan(ln) - ln;
            const uint32_t cpre = wave_incl_scan(lc) - lc;
            uint32_t jb = kBL;  // the lane's first bin the sums cannot take
            bool restart = false;
            uint64_t pre = cpre;
            uint32_t np = npre;
            uint64_t pre_at = 0;
            uint32_t np_at = 0;
#pragma unroll
            for (uint32_t j = 0; j < kBL; j++) {
                const uint64_t start = sub ? M - pre : M + pre;
                bool bad = !okj[j];
                bool rs = false;
                if (sub) {
                    const int64_t end = static_cast<int64_t>(M) - static_cast<int64_t>(pre + cj[j]);
                    bad |= nj[j] > 0u && end <= static_cast<int64_t>(1ull << 23);
                } else {
                    const uint64_t end = M + pre + cj[j];
                    rs = start >= (1ull << 24);
                    bad |= rs || end > (1ull << 24);
                    if (K == FK_A) bad |= nj[j] > 0u && end >= mthr;
                }
                if (jb == kBL) {
                    if (K == FK_S && bl + j < bend) {
                        const float sv = ldexpf(static_cast<float>(start), g);
                        if (kB != 2) e_sstart()[bl + j] = sv;
                        if (kB != 1) e_shi()[bl + j] = sv;
                        if (kB != 2) e_pstart()[bl + j] = w.pos + np;
                    }
                    if (bad) {
                        jb = j;
                        restart = rs;
                        pre_at = pre;
                        np_at = np;
                    }
                }
                pre += cj[j];
                np += nj[j];
            }
            const uint32_t f = first_lane(wave_ballot(jb < kBL));
            if (kB != 0) {  // the bins added below: every bin of the lanes before f, lane f's before jb
                const uint32_t applied = lane < f ? tmask : (lane == f ? tmask & ((1u << jb) - 1u) : 0u);
                if (wave_ballot(applied != 0u)) w.tied = 1u;
            }
            // lanes after f recorded bin starts past the stop; the next step
            // writes them again from the right value
            if (f == 64u) {
                const uint64_t applied = wave_read64(pre, 63u);  // cpre + lc of the last lane
                w.x = ldexpf(static_cast<float>(sub ? M - applied : M + applied), g);
                w.pos += wave_read(np, 63u);
                w.b += kBL * 64u;
                continue;
            }
            const uint64_t applied = wave_read64(pre_at, f);
            w.x = ldexpf(static_cast<float>(sub ? M - applied : M + applied), g);
            w.pos += wave_read(np_at, f);
            w.b = wave_read(bl + jb, f);
            if (w.b >= bend) break;
            if (wave_read(restart ? 1u : 0u, f)) continue;
            expand = true;
        }
        if (expand) {
            const uint32_t bb = w.b;
            if (!bit_of(e_cpl(), bb)) return W_NEED;
            uint32_t r0, r1;
            runs_of(bb, nruns, &r0, &r1);
            const uint32_t res = walk_runs<K>(w, r0, r1, T, thr, lim);
            if (res == W_DECIDED) return res;
            w.b = bb + 1u;
        }
    }
    return W_DONE;
}

__device__ __forceinline__ void set_bit(uint32_t* w, uint32_t b) { atomicOr(&w[b >> 5], 1u << (b & 31u)); }

// Does fold K expect to step through bin b (a predicted crossing or decision,
// a bin planned without a grid, or a step its sums could not take; for the
// exact walk also a tie, which the bound walks take as two ends)?
__device__ __forceinline__ bool fold_needs(int k, uint32_t b, bool exact) {
    const uint32_t pw = e_plan()[b];
    if (bit_of(e_xreq(k), b) || (pw & plan_must(k))) return true;
    if (k == FK_R && !(pw & PF_R)) return false;
    const uint32_t s0 = slot0(k);
    return exact ? (tie_bit(s0, b) || tie_bit(s0 + 1u, b)) : (bad_bit(s0, b) || bad_bit(s0 + 1u, b));
}

// ---- passes ----------------------------------------------------------------
// tau's grid units for the sums of slot `slot` (binade g); a step that
// cannot be summed, or a sum that could pass 2^32 over the bin's n
// candidates, marks the bin's sum invalid.
__device__ __forceinline__ void add_term(uint32_t slot, uint32_t b, float tau, int g, uint32_t n) {
    uint32_t fl = 0;
    uint32_t t = grid_term(tau, g, &fl);
    const bool tie = t == kTieTerm;
    if (tie) t = fl;  // the lower bound of the step; the tie bit says it may be one more
    const bool bad = t == kBigTerm || static_cast<uint64_t>(t) * n >= (1ull << 32);
    atomicAdd(&e_sum(slot)[b], bad ? 0u : t);
    if (bad || tie) {
        const uint32_t i = slot * kNB + b;
        const uint32_t bit = 1u << (i & 31u);
        const uint32_t old = atomicOr(&e_tie()[i >> 5], bit);
        if (bad || (old & bit)) atomicOr(&e_tieb()[i >> 5], bit);
    }
}

enum : int { EP_HIST = 0, EP_SR = 1, EP_A = 2, EP_CENSUS = 3, EP_SUB = 4 };

// One re-read of the row for the engine, its candidates (filter q, in total
// order) handled by mode:
//   EP_HIST    candidates and approximate masses (hardware exp2) per bin, the
//              smallest candidate's key, whether a candidate is NaN;
//   EP_SR      the grid sums of total and the draw, and the census;
//   EP_A       the grid sums of acc (terms p / T), and the census;
//   EP_CENSUS  the census alone;
//   EP_SUB     the crowded coarse bins' sub-histograms (kSub bins each, in
//              e_hkey, which holds no census yet).
// The row is read as in row_pass (16-byte blocks, the next tile in flight);
// each element takes one predicate and one branch into the mode's work.
template <int kMode>
__device__ __noinline__ void eng_pass(Fin& f_in, const Filt& q_in, const FBins& vb_in, float T) {
    const Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const FBins vb = vb_in;
    const uint32_t tid = threadIdx.x;
    if (kMode == EP_HIST) {
        for (uint32_t i = tid; i < kNB; i += kBlock) {
            e_cnt()[i] = 0u;
            e_mass()[i] = 0.0;
        }
        if (tid == 0) {
            e_sc()[SC_NAN] = 0u;
            e_sc()[SC_CMIN] = 0xFFFFFFFFu;
        }
    } else if (kMode == EP_SUB) {
        for (uint32_t i = tid; i < kCrowd * kSub; i += kBlock) e_hkey()[i] = 0u;
    } else if (kMode == EP_SR || kMode == EP_A) {
        const uint32_t nslot = kMode == EP_SR ? 4u : 2u;
        for (uint32_t i = tid; i < nslot * kNB; i += kBlock) e_sum(0)[i] = 0u;
        for (uint32_t i = tid; i < nslot * kNB / 32u; i += kBlock) {
            e_tie()[i] = 0u;
            e_tieb()[i] = 0u;
        }
    }
    TSM_LDS_SYNC();
    const float t = f.m.t;
    const float y0 = vb.vb.y0;
    const float l2t = 1.4426950408889634f / t;
    const uint64_t* tab = e_exptab();
    uint32_t kmin = 0xFFFFFFFFu;
    bool nan = false;

    const uint32_t n = f.n;
    const bool penal = f.m.penal;
    const TSM_GLOBAL_AS float* rowp = global_as(f.rowp);
    const TSM_GLOBAL_AS uint32_t* mrow = global_as(f.mrow);
    const uint32_t head = static_cast<uint32_t>((reinterpret_cast<uintptr_t>(f.rowp) >> 2) & 3u);
    const TSM_GLOBAL_AS float* base = rowp - head;  // 16-byte aligned
    const uint32_t span = head + n, nblk = (span + 3u) / 4u, full = span / 4u;
    constexpr uint32_t kTB = kReTile / 4u;
    constexpr uint32_t kPer = kTB / kBlock;
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
    for (uint32_t tl = 0; tl < ntiles; tl++) {
        if (tl + 1u < ntiles) {
#pragma unroll
            for (uint32_t k = 0; k < kPer; k++) nxt[k] = load_blk((tl + 1u) * kTB + tid + k * kBlock);
        }
        const uint32_t tb = tl * kReTile;
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
            const uint32_t j = tl * kTB + tid + k * kBlock;
            const float xv[4] = {cur[k].x, cur[k].y, cur[k].z, cur[k].w};
#pragma unroll
            for (uint32_t e = 0; e < 4u; e++) {
                const uint32_t i = 4u * j + e;
                const uint32_t id = i - head;
                bool keep = j < nblk && i >= head && i < span;
                float y = xv[e];
                if (penal) {
                    const uint32_t li = (i - tb) & (kReTile - 1u);
                    const uint32_t c = (f.cnt()[li >> 1] >> ((li & 1u) << 4)) & 0xFFFFu;
                    if (c) y = penalize(y, c, f.m, f.P);
                }
                if (q.use_cut) keep = keep && y >= q.cut;
                if (q.use_max) keep = keep && composite(total_key(y), id) <= q.max_comp;
                if (q.need_allowed && keep) keep = (mrow[id >> 5] >> (id & 31u)) & 1u;
                if (q.use_minp && keep) {
                    keep = !(y < q.minp_lo);
                    if (keep && !(y >= q.minp_hi)) keep = glibc_expf_lds((y - q.y0) / t, tab) >= q.minp;
                }
                if (kMode == EP_SUB) {
                    if (keep && y == y) {
                        const uint32_t c = vb.vb.bin(y);
#pragma unroll
                        for (uint32_t s = 0; s < kCrowd; s++) {
                            if (c != vb.cr[s]) continue;
                            const float x = vb.frac(y, c) * static_cast<float>(kSub);
                            const uint32_t j = x < static_cast<float>(kSub - 1u) ? static_cast<uint32_t>(x) : kSub - 1u;
                            atomicAdd(&e_hkey()[s * kSub + j], 1u);
                        }
                    }
                    continue;
                }
                const uint32_t b = vb.bin(y);
                if (kMode == EP_HIST) {
                    const bool isnan = y != y;
                    nan |= keep && isnan;
                    keep = keep && !isnan;
                    const double m = static_cast<double>(__builtin_amdgcn_exp2f((y - y0) * l2t));
                    const uint32_t kk = total_key(y);
                    kmin = keep && kk < kmin ? kk : kmin;
                    if (keep) {
                        atomicAdd(&e_cnt()[b], 1u);
                        atomicAdd(&e_mass()[b], m);
                    }
                } else {
                    if (kMode != EP_CENSUS) {
                        const uint32_t pw = e_plan()[b];
                        const uint32_t nb = e_cnt()[b];
                        const float p = glibc_expf_lds((y - y0) / t, tab);
                        if (kMode == EP_SR) {
                            const int gs = static_cast<int>(pw & 0xFFu) - 128;
                            const int gr = static_cast<int>((pw >> 8) & 0xFFu) - 128;
                            const bool ds = keep && !(pw & PF_MUST_S);
                            const bool dr = keep && (pw & PF_R) && !(pw & PF_MUST_R);
                            if (ds) {
                                add_term(SL_S0, b, p, gs, nb);
                                if (pw & PF_TWO_S) add_term(SL_S1, b, p, gs + 1, nb);
                            }
                            if (dr) {
                                add_term(SL_R0, b, p, gr, nb);
                                if (pw & PF_TWO_R) add_term(SL_R1, b, p, gr + 1, nb);
                            }
                        } else {
                            const float qv = p / T;
                            const int ga = static_cast<int>((pw >> 16) & 0xFFu) - 128;
                            if (keep && !(pw & PF_MUST_A)) {
                                add_term(SL_S0, b, qv, ga, nb);
                                if (pw & PF_TWO_A) add_term(SL_S1, b, qv, ga + 1, nb);
                            }
                        }
                    }
                    if (keep && bit_of(e_req(), b)) census_insert(total_key(y), id, b);
                }
            }
        }
        if (tl + 1u < ntiles) {
#pragma unroll
            for (uint32_t k = 0; k < kPer; k++) cur[k] = nxt[k];
        }
    }
    if (kMode == EP_HIST) {
        TSM_LDS_SYNC();
        kmin = wave_min(kmin);
        if (lane_id() == 0 && kmin != 0xFFFFFFFFu) atomicMin(&e_sc()[SC_CMIN], kmin);
        if (nan) e_sc()[SC_NAN] = 1u;
    }
    TSM_LDS_SYNC();
}

// ---- plans ---------------------------------------------------------------------
// Relative error allowed between a fold and the approximate cumulative masses
// it is planned from (hardware exp2 terms, f64 sums; the f32 fold's own
// rounding drift): a bin whose fold value may lie on either side of a power of
// two gets both grids, or no sum at all when the range spans more.
constexpr double kPlanEps = 1e-4;
// The same for predicting where a fold will step value by value (census
// requests): tighter, since a miss costs a census round, not a wrong result.
constexpr double kPredEps = 2e-5;

__device__ __forceinline__ void plan_range(double lo, double hi, bool sub, uint32_t shift, uint32_t two,
                                           uint32_t must, uint32_t* pw) {
    const int e_lo = step_binade(static_cast<float>(lo), sub);
    const int e_hi = binade_of(static_cast<float>(hi));
    if (!(lo > 0.0) || e_hi - e_lo >= 2 || e_lo < -126) {
        *pw |= must;
        return;
    }
    *pw |= static_cast<uint32_t>(e_lo + 128) << shift;
    if (e_hi > e_lo) *pw |= two;
}

// Plans of total and the draw from the approximate masses, with the bins each
// is expected to step through.  Two bins per thread.
__device__ void plan_sr(Fin& f, float u, bool draw, bool topp) {
    const uint32_t tid = threadIdx.x;
    const uint32_t b0 = 2 * tid;
    for (uint32_t i = tid; i < 3u * kNB / 32u; i += kBlock) e_xreq(0)[i] = 0u;
    if (tid == 0) {
        e_sc()[SC_KLO] = 0xFFFFFFFFu;
        e_sc()[SC_KHI] = 0u;
    }
    const double m0 = e_mass()[b0], m1 = e_mass()[b0 + 1];
    const uint32_t c0 = e_cnt()[b0], c1 = e_cnt()[b0 + 1];
    double tot;
    const double P0 = block_excl_scan_f64(m0 + m1, f.miscd() + 8, &tot);  // barriers order the clears above
    const double Pb[2] = {P0, P0 + m0}, mb[2] = {m0, m1};
    const uint32_t cb[2] = {c0, c1};
    const double tp = static_cast<double>(f.P.top_p);
    const double eps2 = kPredEps;
    if (topp) {
#pragma unroll
        for (int k = 0; k < 2; k++)
            if (cb[k] && (Pb[k] + mb[k]) / tot >= tp - eps2 && Pb[k] / tot <= tp + eps2) {
                atomicMin(&e_sc()[SC_KLO], b0 + k);
                atomicMax(&e_sc()[SC_KHI], b0 + k);
            }
    }
    TSM_LDS_SYNC();
    const uint32_t klo = e_sc()[SC_KLO], khi = e_sc()[SC_KHI];
#pragma unroll
    for (int k = 0; k < 2; k++) {  // the kept mass's bounds: cumulative masses at the region's ends
        if (topp && klo != 0xFFFFFFFFu && b0 + k == klo) e_scd()[0] = Pb[k];
        if (topp && klo != 0xFFFFFFFFu && b0 + k == khi) e_scd()[1] = Pb[k] + mb[k];
    }
    TSM_LDS_SYNC();
    double M_lo = tot, M_hi = tot;
    if (topp && klo != 0xFFFFFFFFu) {
        M_lo = e_scd()[0];
        M_hi = e_scd()[1];
    }
    M_lo *= 1.0 - kPredEps;
    M_hi *= 1.0 + kPredEps;
    const double du = static_cast<double>(u);
    // r = u * mass - (total's fold so far) carries the drift of both f32
    // folds over the whole row (total's own reaches ~1e-5 of it): an absolute
    // margin of 1e-4 of the total
    const double slack = 1e-4 * tot;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const uint32_t b = b0 + k;
        if (!cb[k]) {
            e_plan()[b] = PF_MUST_S | PF_MUST_R | PF_MUST_A;
            continue;
        }
        uint32_t pw = 0;
        // total: the fold value at the bin's start is about Pb
        const double slo = Pb[k] * (1.0 - kPlanEps), shi = Pb[k] * (1.0 + kPlanEps);
        plan_range(slo, shi, false, 0u, PF_TWO_S, PF_MUST_S, &pw);
        if ((pw & PF_MUST_S) || binade_of(static_cast<float>((Pb[k] + mb[k]) * (1.0 + kPlanEps))) !=
                                     binade_of(static_cast<float>(slo)))
            set_bit(e_xreq(FK_S), b);
        if (draw) {
            // the draw: r at the bin's start is about u * M - Pb
            const double rlo = du * M_lo - Pb[k] * (1.0 + kPredEps) - slack,
                         rhi = du * M_hi - Pb[k] * (1.0 - kPredEps) + slack;
            if (rhi > 0.0) {
                pw |= PF_R;
                plan_range(rlo, rhi, true, 8u, PF_TWO_R, PF_MUST_R, &pw);
                // r may leave its binade (or reach zero) in this bin when the
                // lowest end value and the highest start value lie in
                // different binades
                const double elo = rlo - mb[k] * (1.0 + kPredEps);
                if ((pw & PF_MUST_R) || !(elo > 0.0) ||
                    binade_of(static_cast<float>(elo)) != step_binade(static_cast<float>(rhi), true))
                    set_bit(e_xreq(FK_R), b);
            }
        }
        if (topp && klo != 0xFFFFFFFFu && b >= klo && b <= khi) {
            set_bit(e_xreq(FK_A), b);
            if (draw) set_bit(e_xreq(FK_R), b);
        }
        e_plan()[b] = pw;
    }
    TSM_LDS_SYNC();
}

// acc's plan once total's walk has left the fold value at every bin start.
__device__ void plan_a(float T, float top_p) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t b = tid; b < kNB; b += kBlock) {
        const uint32_t n = e_cnt()[b];
        if (!n) continue;
        uint32_t pw = e_plan()[b] & ~(0xFFu << 16 | PF_TWO_A | PF_MUST_A);
        const double s = static_cast<double>(e_sstart()[b]);
        const double s_end = b + 1 < kNB ? static_cast<double>(e_sstart()[b + 1]) : static_cast<double>(T);
        const double a = s / T, a_end = s_end / T;
        const double lo = a * (1.0 - kPlanEps), hi = a * (1.0 + kPlanEps);
        plan_range(lo, hi, false, 16u, PF_TWO_A, PF_MUST_A, &pw);
        const bool before = a <= top_p * (1.0 + kPredEps);  // acc stops at top_p
        const bool decides = before && a_end * (1.0 + kPredEps) >= top_p;
        if (before && ((pw & PF_MUST_A) || decides ||
                       binade_of(static_cast<float>(a_end * (1.0 + kPredEps))) !=
                           binade_of(static_cast<float>(a * (1.0 - kPredEps)))))
            set_bit(e_xreq(FK_A), b);
        e_plan()[b] = pw;
    }
    TSM_LDS_SYNC();
}

// Clears the tie bits of slots 0 and 1 (total's, before acc's sums).
__device__ __forceinline__ void clear_ties01() {
    for (uint32_t i = threadIdx.x; i < 2u * kNB / 32u; i += kBlock) {
        e_tie()[i] = 0u;
        e_tieb()[i] = 0u;
    }
    TSM_LDS_SYNC();
}

// Keeps the lowest bins of the bitmap w (one word per lane of wave 0) while
// their candidates stay within cap_cnt and their number within cap_bins (the
// lowest bin is kept whatever its count when `first` is set); returns the
// candidates and bins kept, summed over the wave.
__device__ uint2 trim_bins(uint32_t& w, uint32_t cap_cnt, uint32_t cap_bins, bool first) {
    const uint32_t lane = lane_id();
    uint32_t cnt = 0;
    for (uint32_t bits = w; bits; bits &= bits - 1u) cnt += e_cnt()[32u * lane + static_cast<uint32_t>(__builtin_ctz(bits))];
    const uint32_t nb = static_cast<uint32_t>(__popc(w));
    const uint32_t pc = wave_incl_scan(cnt) - cnt, pb = wave_incl_scan(nb) - nb;
    const uint32_t anyb = first ? first_lane(wave_ballot(w != 0u)) : 64u;  // lane holding the lowest bin
    if (pc + cnt > cap_cnt || pb + nb > cap_bins) {
        uint32_t kept = 0, c = pc, k = pb;
        for (uint32_t bits = w; bits; bits &= bits - 1u) {
            const uint32_t i = static_cast<uint32_t>(__builtin_ctz(bits));
            const uint32_t ci = e_cnt()[32u * lane + i];
            const bool must = lane == anyb && kept == 0u && pc == 0u && pb == 0u;
            if (!must && (c + ci > cap_cnt || k + 1u > cap_bins)) break;
            kept |= 1u << i;
            c += ci;
            k++;
        }
        w = kept;
    }
    uint32_t kc = 0;
    for (uint32_t bits = w; bits; bits &= bits - 1u) kc += e_cnt()[32u * lane + static_cast<uint32_t>(__builtin_ctz(bits))];
    return make_uint2(wave_sum(kc), wave_sum(static_cast<uint32_t>(__popc(w))));
}

// Requests of a census round for fold K stopped at bin `from`: that bin and
// the bins after it that fold K expects to step through, then, in the room
// left, those of the folds still to come (acc's when acc_next, the draw's
// when draw).  Within kReqCnt candidates and kReqMax bins, lowest bins first.
__device__ void request_round(int K, uint32_t from, bool draw, bool acc_next, bool exact, bool whole = false) {
    const uint32_t tid = threadIdx.x;
    if (tid < kWave) {
        uint32_t cur = 0, later = 0;
        for (uint32_t i = 0; i < 32u; i++) {
            const uint32_t b = 32u * tid + i;
            if (!e_cnt()[b]) continue;
            if (b == from || (b > from && fold_needs(K, b, exact))) cur |= 1u << i;
            else if ((whole && fold_needs(K, b, exact)) || (K == FK_S && ((acc_next && bit_of(e_xreq(FK_A), b)) || (draw && fold_needs(FK_R, b, false)))) ||
                     (K == FK_A && draw && fold_needs(FK_R, b, false)))
                later |= 1u << i;
        }
        const uint2 used = trim_bins(cur, kReqCnt, kReqMax, true);
        const uint32_t room_c = used.x < kReqCnt ? kReqCnt - used.x : 0u;
        const uint32_t room_b = used.y < kReqMax ? kReqMax - used.y : 0u;
        trim_bins(later, room_c, room_b, false);
        e_req()[tid] = cur | later;
    }
    TSM_LDS_SYNC();
}

// Fold K's walk on wave 0 from w, with census rounds wherever the census
// lacks a bin the walk must step through.  Returns W_DONE or W_DECIDED with w
// updated, or W_NEED when a bin holds more distinct values than the census.
template <int K, int kB = 0>
__device__ __noinline__ uint32_t run_walk(Fin& f_in, const Filt& q_in, const FBins& vb_in, Walk& w_io,
                                          uint32_t bend, float T, float thr, uint32_t force, uint32_t lim,
                                          bool draw, bool acc_next) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const FBins vb = vb_in;
    const uint32_t tid = threadIdx.x;
    Walk w = w_io;
    uint32_t last_from = kNoBin;
    bool alone = false;
    for (;;) {
        const uint32_t nruns = e_sc()[SC_NRUNS];
        if (tid < kWave) {
            const uint32_t res = walk_bins<K, kB>(w, bend, nruns, T, thr, force, lim);
            if (tid == 0) {
                e_sc()[SC_RES] = res;
                e_sc()[SC_B] = w.b;
                e_sc()[SC_POS] = w.pos;
                e_sc()[SC_RUN] = w.run;
                e_sc()[SC_WITHIN] = w.within;
                e_sc()[SC_X] = __float_as_uint(w.x);
                e_sc()[SC_TIED] = w.tied;
            }
        }
        TSM_LDS_SYNC();
        const uint32_t res = e_sc()[SC_RES];
        w.b = e_sc()[SC_B];
        w.pos = e_sc()[SC_POS];
        w.run = e_sc()[SC_RUN];
        w.within = e_sc()[SC_WITHIN];
        w.x = __uint_as_float(e_sc()[SC_X]);
        w.tied = e_sc()[SC_TIED];
        TSM_LDS_SYNC();
        if (res != W_NEED) {
            w_io = w;
            return res;
        }
        if (w.b == last_from) {
            // the bin was requested and still overflowed the census: once more alone
            if (alone) {
                w_io = w;
                return W_NEED;
            }
            alone = true;
            if (tid < kNB / 32u) e_req()[tid] = 0u;
            TSM_LDS_SYNC();
            if (tid == 0) set_bit(e_req(), w.b);
            TSM_LDS_SYNC();
        } else {
            alone = false;
            // a walk with ties down is followed by one with ties up: its
            // needs before w.b come too
            request_round(K, w.b, draw, acc_next, kB == 0, kB == 1);
        }
        last_from = w.b;
        census_clear();
        eng_pass<EP_CENSUS>(f, q, vb, 0.0f);
        census_finish(vb, f.m.t);
    }
}

// Fold K's two bound walks at once: ties down (kB 1) on wave 0 from wl, ties
// up (kB 2) on wave 1 from wh, with shared census rounds wherever either
// lacks a bin.  The walks read the same sums and census and write their own
// bin-start records (e_sstart, e_shi; e_pstart gets the same positions from
// both).  Sets *rl and *rh; returns W_NEED when a bin holds more distinct
// values than the census, else W_DONE.
constexpr uint32_t kSc2 = 16;  // e_sc() words 16..29: the two walks' results, 7 words each
template <int K>
__device__ __noinline__ uint32_t run_walk2(Fin& f_in, const Filt& q_in, const FBins& vb_in, Walk& wl_io,
                                           Walk& wh_io, uint32_t* rl, uint32_t* rh, uint32_t bend, float T,
                                           float thr, uint32_t force, uint32_t lim, bool draw, bool acc_next) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const FBins vb = vb_in;
    const uint32_t tid = threadIdx.x, wid = tid / kWave;
    Walk w0 = wl_io, w1 = wh_io;
    uint32_t r0 = W_NEED, r1 = W_NEED;
    uint32_t from0 = kNoBin, from1 = kNoBin;  // the bin each walk last asked the census for
    bool alone = false;
    for (;;) {
        const uint32_t nruns = e_sc()[SC_NRUNS];
        if (wid < 2u && (wid == 0u ? r0 : r1) == W_NEED) {
            Walk w = wid == 0u ? w0 : w1;
            const uint32_t res = wid == 0u ? walk_bins<K, 1>(w, bend, nruns, T, thr, force, lim)
                                           : walk_bins<K, 2>(w, bend, nruns, T, thr, force, lim);
            if (lane_id() == 0) {
                uint32_t* o = e_sc() + kSc2 + 7u * wid;
                o[0] = res;
                o[1] = w.b;
                o[2] = w.pos;
                o[3] = w.run;
                o[4] = w.within;
                o[5] = __float_as_uint(w.x);
                o[6] = w.tied;
            }
        }
        TSM_LDS_SYNC();
#pragma unroll
        for (uint32_t j = 0; j < 2u; j++) {
            if ((j == 0u ? r0 : r1) != W_NEED) continue;
            const uint32_t* o = e_sc() + kSc2 + 7u * j;
            Walk& w = j == 0u ? w0 : w1;
            w.b = o[1];
            w.pos = o[2];
            w.run = o[3];
            w.within = o[4];
            w.x = __uint_as_float(o[5]);
            w.tied = o[6];
            if (j == 0u) r0 = o[0];
            else r1 = o[0];
        }
        TSM_LDS_SYNC();
        if (r0 != W_NEED && r1 != W_NEED) break;
        // a census round from the lower of the bins the walks stopped at; a
        // walk that stops again at the bin it last asked for gets that bin
        // alone, once
        const bool n0 = r0 == W_NEED, n1 = r1 == W_NEED;
        const uint32_t b = n0 && n1 ? min(w0.b, w1.b) : (n0 ? w0.b : w1.b);
        const bool again = (n0 && w0.b == b && from0 == b) || (n1 && w1.b == b && from1 == b);
        if (again) {
            if (alone) {
                wl_io = w0;
                wh_io = w1;
                *rl = r0;
                *rh = r1;
                return W_NEED;
            }
            alone = true;
            if (tid < kNB / 32u) e_req()[tid] = 0u;
            TSM_LDS_SYNC();
            if (tid == 0) set_bit(e_req(), b);
            TSM_LDS_SYNC();
        } else {
            alone = false;
            request_round(K, b, draw, acc_next, false, true);
        }
        if (n0 && w0.b == b) from0 = b;
        if (n1 && w1.b == b) from1 = b;
        census_clear();
        eng_pass<EP_CENSUS>(f, q, vb, 0.0f);
        census_finish(vb, f.m.t);
    }
    wl_io = w0;
    wh_io = w1;
    *rl = r0;
    *rh = r1;
    return W_DONE;
}

// The kept candidate at position pos (0-based, pos < kept count) when no step
// of the draw decides: its run and index within the run, from bin lb's runs.
__device__ __forceinline__ bool locate(uint32_t lb, uint32_t pos, uint32_t nruns, uint32_t* run, uint32_t* within) {
    uint32_t r0, r1;
    runs_of(lb, nruns, &r0, &r1);
    uint32_t at = e_pstart()[lb];
    for (uint32_t j = r0; j < r1; j++) {
        const uint32_t m = e_hcnt()[j];
        if (pos < at + m) {
            *run = j;
            *within = pos - at;
            return true;
        }
        at += m;
    }
    return false;
}

constexpr uint32_t kHot = 32;  // weight factor of coarse bins where a fold steps value by value
constexpr uint32_t kFineCap = 1024;  // candidates a fine bin's share of the weight may hold

// Does a coarse bin of approximate mass m after cumulative mass P (of tot)
// hold a predicted event: total crossing a power of two, acc = total / tot
// crossing one, top-p's decision, or r = u * mass - P crossing one or
// reaching zero?  The margins cover the gap between these estimates and the
// f32 folds.
__device__ __forceinline__ bool coarse_hot(double P, double m, double tot, float u, bool topp, bool draw,
                                           float top_p) {
    if (m <= 0.0) return false;
    const double lo = P * (1.0 - kPlanEps), hi = (P + m) * (1.0 + kPlanEps);
    if (!(lo > 0.0) || binade_of(static_cast<float>(lo)) != binade_of(static_cast<float>(hi))) return true;
    if (topp) {
        // acc stops at top_p: a bin that starts past it is never walked by acc
        const double tp = static_cast<double>(top_p) * tot;
        if (lo <= tp * (1.0 + kPlanEps)) {
            if (binade_of(static_cast<float>(lo / tot)) != binade_of(static_cast<float>(hi / tot))) return true;
            if (tp <= hi) return true;
        }
    }
    if (draw) {
        const double M = topp ? static_cast<double>(top_p) * tot : tot;
        const double rhi = static_cast<double>(u) * M * (1.0 + kPlanEps) - lo;
        const double rlo = static_cast<double>(u) * M * (1.0 - kPlanEps) - hi;
        if (rhi > 0.0 && (!(rlo > 0.0) || binade_of(static_cast<float>(rlo)) != binade_of(static_cast<float>(rhi))))
            return true;
    }
    return false;
}

// The last bin at or before `limit` where total's walks with ties down and up
// start from the same value: from there on that value is total's own.
__device__ uint32_t last_agree(uint32_t limit) {
    const uint32_t tid = threadIdx.x;
    if (tid == 0) e_sc()[SC_LAST] = 0u;
    TSM_LDS_SYNC();
    for (uint32_t b = tid; b <= limit && b < kNB; b += kBlock)
        if (__float_as_uint(e_sstart()[b]) == __float_as_uint(e_shi()[b])) atomicMax(&e_sc()[SC_LAST], b);
    TSM_LDS_SYNC();
    const uint32_t r = e_sc()[SC_LAST];
    TSM_LDS_SYNC();
    return r;
}

// After the fine layout's histogram: the coarse bins (this thread's two,
// with cnt0 / cnt1 candidates) holding a part of a fine bin with more
// candidates than a census round takes are crowded; up to kCrowd of them get
// a sub-histogram (one more pass) and are laid out from it (FBins).  Returns
// whether any was, so that the caller counts the fine bins again.
__device__ __noinline__ bool crowd_layout(Fin& f, const Filt& q, FBins& vb, uint32_t cnt0, uint32_t cnt1) {
    const uint32_t tid = threadIdx.x;
    if (tid == 0) e_crowd()[0] = 0u;
    TSM_LDS_SYNC();
#pragma unroll
    for (uint32_t k = 0; k < 2u; k++) {
        const uint32_t c = 2u * tid + k;
        if ((k == 0u ? cnt0 : cnt1) <= kReqCnt / 4u) continue;  // too few to crowd a fine bin
        const uint32_t l0 = e_lay()[c], l1 = c + 1u < kNB ? e_lay()[c + 1u] : l0 + (kNB - 1u);
        const uint32_t f0 = min(static_cast<uint32_t>(static_cast<float>(l0) * vb.scale), kNB - 1u);
        const uint32_t f1 = min(static_cast<uint32_t>(static_cast<float>(l1) * vb.scale), kNB - 1u);
        bool crowded = false;
        for (uint32_t j = f0; j <= f1 && !crowded; j++) crowded = e_cnt()[j] > kReqCnt;
        if (crowded) {
            const uint32_t sl = atomicAdd(&e_crowd()[0], 1u);
            if (sl < kCrowd) e_crowd()[1u + sl] = c;
        }
    }
    TSM_LDS_SYNC();
    const uint32_t nc = min(e_crowd()[0], kCrowd);
    if (nc == 0u) return false;
#pragma unroll
    for (uint32_t sl = 0; sl < kCrowd; sl++) vb.cr[sl] = sl < nc ? e_crowd()[1u + sl] : kNoBin;
    // the sub-histograms (by the coarse bins and fr only), then each crowded
    // bin's cumulative counts at its sub-bin edges, wave sl for slot sl
    eng_pass<EP_SUB>(f, q, vb, 0.0f);
    const uint32_t wid = tid / kWave, lane = lane_id();
    if (wid < nc) {
        constexpr uint32_t kPerLane = kSub / kWave;
        static_assert(kPerLane * kWave == kSub, "sub-bins per lane");
        uint32_t h[kPerLane], sum = 0;
#pragma unroll
        for (uint32_t i = 0; i < kPerLane; i++) {
            h[i] = e_hkey()[wid * kSub + lane * kPerLane + i];
            sum += h[i];
        }
        const uint32_t incl = wave_incl_scan(sum);
        const uint32_t n = wave_read(incl, kWave - 1u);
        uint16_t* F = e_cdf(wid);
        uint32_t cum = incl - sum;
#pragma unroll
        for (uint32_t i = 0; i < kPerLane; i++) {
            const uint32_t j = lane * kPerLane + i;
            F[j] = static_cast<uint16_t>(n ? (static_cast<uint64_t>(cum) * 65535u) / n : (j * 65535u) / kSub);
            cum += h[i];
        }
        if (lane == 0) F[kSub] = 65535u;
    }
    TSM_LDS_SYNC();
    return true;
}

// Sampler::distribution (sampler.rs:102-116) for a kept set of `keep`
// candidates (filter q, `len` candidates before the kept count): the first
// min(keep, stride) of them, best first, as (id, p_j / mass), written in
// chunks of up to kExactCap entries, each selected above the previous one's
// last composite, gathered and sorted.  Returns the best id (0 when nothing
// was written).
__device__ __noinline__ uint32_t write_dist_chunks(Fin& f, const Filt& q, uint32_t len, uint32_t keep,
                                                   const DistOut* dist, float y0, float t, float mass) {
    const uint32_t tid = threadIdx.x;
    const uint32_t k = min(keep, dist->stride);
    uint32_t done = 0, best = 0;
    uint64_t last = 0;
    while (done < k) {
        const uint32_t c = min(k - done, kExactCap);
        Filt qd = q;
        if (done) {
            qd.use_min = true;
            qd.min_comp = last;
        }
        if (done + c < len) {
            qd.use_max = true;
            qd.max_comp = select_kth(f, qd, c);
        }
        const uint32_t g = gather_pass(f, qd, kExactCap);
        if (g == 0u) break;
        sort_gathered(f, g);
        last = f.gcomp()[g - 1u];
        if (done == 0u) best = f.rid()[0];
        for (uint32_t j = tid; j < g; j += kBlock) {
            dist->ids[done + j] = f.rid()[j];
            dist->probs[done + j] = glibc_expf((f.ry()[j] - y0) / t) / mass;
        }
        done += g;
        TSM_LDS_SYNC();  // every thread has read gcomp before the next chunk's passes
    }
    if (keep > done && tid == 0) atomicOr(dist->status, TSM_STATUS_DIST_TRUNCATED);
    return best;
}

struct BigOut {
    Pick pick;
    bool small;  // at most kExactCap candidates: the caller finishes them exactly
};

// Rows with a nucleus larger than kExactCap (filter q, best value y0, the
// row's smallest value mlo): total, top-p, the kept mass and the draw by the
// reference's f32 folds.  q1 is q before min-p (min-p keeps at least the
// best candidate).
__device__ __noinline__ BigOut big_nucleus(Fin& f_in, const Filt& q_in, float y0, float mlo, float u,
                                           const DistOut* dist) {
    Fin f = f_in;  // a private copy: its fields stay in registers across LDS atomics
    const Filt q = q_in;
    const uint32_t tid = threadIdx.x;
    const float t = f.m.t;
    const bool topp = !(f.P.top_p >= 1.0f);
    const bool draw = dist == nullptr;
    BigOut out;
    out.small = false;
    out.pick.token = 0xFFFFFFFFu;
    out.pick.keep = 0;
    out.pick.prob = 0.0f;
    out.pick.mass = 0.0f;
    if (tid < 32u) e_exptab()[tid] = kExp2Tab[tid];
    TSM_LDS_SYNC();
    FBins vb;
    vb.vb.y0 = y0;
#pragma unroll
    for (uint32_t sl = 0; sl < kCrowd; sl++) vb.cr[sl] = kNoBin;
    {
        float span = fminf(30.5f, (y0 - mlo) / t);
        if (!(span > 0.0f)) span = 1.0f;
        vb.vb.mul = (static_cast<float>(kNB) / span) / t;
    }
    bool degenerate = !__builtin_isfinite(y0) || !(__builtin_isfinite(vb.vb.mul) && vb.vb.mul > 0.0f);
    uint32_t len = 0;
    if (!degenerate) {
        vb.scale = 0.0f;  // fine = coarse
        eng_pass<EP_HIST>(f, q, vb, 0.0f);
        // when the candidates fill under a quarter of the bins, bin them again
        // over their own range
        const uint32_t kmin = e_sc()[SC_CMIN];
        const bool nan1 = e_sc()[SC_NAN] != 0u;
        TSM_LDS_SYNC();  // read before a second histogram resets them
        if (!nan1 && kmin != 0xFFFFFFFFu) {
            const float cmin = key_to_float(kmin);
            if (vb.vb.bin(cmin) < kNB / 4u) {
                const float sp2 = ((y0 - cmin) / t) * 1.001f;
                const float mul2 = (static_cast<float>(kNB) / sp2) / t;
                if (sp2 > 0.0f && __builtin_isfinite(mul2) && mul2 > 0.0f) {
                    vb.vb.mul = mul2;
                    eng_pass<EP_HIST>(f, q, vb, 0.0f);
                }
            }
        }
        degenerate = e_sc()[SC_NAN] != 0u;
        const uint32_t c0 = e_cnt()[2 * tid], c1 = e_cnt()[2 * tid + 1];
        len = block_sum<kBlock>(c0 + c1, f.tmp());
        if (!degenerate && len > kExactCap) {
            // fine bins of about equal weight: a coarse bin weighs its count,
            // kHot times that where a fold is expected to step value by value
            // (a binade crossing of total, acc or r, top-p's decision, the
            // draw's end), so that those stretches are censused in small bins
            const double m0 = e_mass()[2 * tid], m1 = e_mass()[2 * tid + 1];
            double mtot;
            const double P0 = block_excl_scan_f64(m0 + m1, f.miscd() + 8, &mtot);
            const bool h0 = coarse_hot(P0, m0, mtot, u, topp, draw, f.P.top_p);
            const bool h1 = coarse_hot(P0 + m0, m1, mtot, u, topp, draw, f.P.top_p);
            // the hot factor, lowered when hot bins hold most candidates so
            // that a fine bin (a 1/kNB share of the weight) holds at most
            // kFineCap candidates, which the census can take
            const uint32_t hc = block_sum<kBlock>((h0 ? c0 : 0u) + (h1 ? c1 : 0u), f.tmp());
            uint32_t hot = kHot;
            if (hc > 0) {
                const uint64_t room = static_cast<uint64_t>(kNB) * kFineCap;
                const uint64_t cold = len - hc;
                const uint64_t k = room > cold ? (room - cold) / hc : 1u;
                hot = static_cast<uint32_t>(k < 1u ? 1u : (k > kHot ? kHot : k));
            }
            const uint32_t w0c = c0 * (h0 ? hot : 1u);
            const uint32_t w1c = c1 * (h1 ? hot : 1u);
            uint32_t wtot;
            const uint32_t W0 = block_excl_scan<kBlock>(w0c + w1c, f.tmp(), &wtot);
            e_lay()[2 * tid] = W0;
            e_lay()[2 * tid + 1] = W0 + w0c;
            vb.scale = static_cast<float>(kNB) / static_cast<float>(wtot);
            TSM_LDS_SYNC();
            eng_pass<EP_HIST>(f, q, vb, 0.0f);
            if (crowd_layout(f, q, vb, c0, c1)) eng_pass<EP_HIST>(f, q, vb, 0.0f);
        }
        if (!degenerate && len <= kExactCap) {
            out.small = true;
            out.pick.keep = len;
            return out;
        }
    }
    if (degenerate) {
        // NaN everywhere downstream (an infinite best value, or a NaN
        // candidate): total, acc and r are NaN, no step decides, and the
        // reference keeps every candidate and picks the last (sampler.rs:150)
        if (len == 0) len = count_pass<kNucGroup>(f, q);
        if (len <= kExactCap) {  // exact_finalize carries the NaNs as the reference does
            out.small = true;
            out.pick.keep = len;
            return out;
        }
        const uint64_t last = exact_at(f, q, ~0ull);
        out.pick.keep = len;
        out.pick.token = static_cast<uint32_t>(last);
        out.pick.mass = __uint_as_float(0x7FC00000u);
        out.pick.prob = out.pick.mass;
        if (dist) write_dist_chunks(f, q, len, len, dist, y0, t, out.pick.mass);
        return out;
    }
    // total's (and the draw's) plans, sums and census
    plan_sr(f, u, draw, topp);
    for (uint32_t i = tid; i < 4u * kNB / 32u; i += kBlock) {
        e_tie()[i] = 0u;
        e_tieb()[i] = 0u;
    }
    TSM_LDS_SYNC();
    request_round(FK_S, 0u, draw && !topp, topp, false);  // with top-p the draw's census waits for acc's
    census_clear();
    eng_pass<EP_SR>(f, q, vb, 0.0f);
    census_finish(vb, t);
    Walk w0;
    w0.x = 0.0f;
    w0.b = 0;
    w0.pos = 0;
    w0.run = w0.within = w0.tied = 0;
    // total: with every unresolved tie rounded down, then up; when both give
    // the same value it is total (the fold is monotone in each step), else
    // the ties are censused and stepped exactly
    float T;
    {
        Walk wl = w0, wh = w0;
        uint32_t rl, rh;
        if (run_walk2<FK_S>(f, q, vb, wl, wh, &rl, &rh, kNB, 0.0f, 0.0f, kNoBin, 0xFFFFFFFFu, draw, topp) == W_NEED)
            return out;
        T = wl.x;
        if (__float_as_uint(wl.x) != __float_as_uint(wh.x)) {
            // the exact walk from the last bin where both walks still agree
            const uint32_t ba = last_agree(kNB - 1u);
            Walk we = w0;
            we.x = e_sstart()[ba];
            we.b = ba;
            we.pos = e_pstart()[ba];
            if (run_walk<FK_S>(f, q, vb, we, kNB, 0.0f, 0.0f, kNoBin, 0xFFFFFFFFu, draw, topp) == W_NEED) return out;
            T = we.x;
        }
    }
    // total (sampler.rs:238)
    uint32_t keep = len, kb = kNoBin;
    float mass = T;
    if (topp) {
        plan_a(T, f.P.top_p);
        clear_ties01();
        request_round(FK_A, 0u, draw, false, false);
        census_clear();
        eng_pass<EP_A>(f, q, vb, T);
        census_finish(vb, t);
        // acc the same way: ties down and up at once; the same decision from both
        // is acc's, else the exact walk
        Walk wal = w0, wa = w0;
        uint32_t ral, ra;
        if (run_walk2<FK_A>(f, q, vb, wal, wa, &ral, &ra, kNB, T, f.P.top_p, kNoBin, 0xFFFFFFFFu, draw, false) ==
            W_NEED)
            return out;
        if (ra != ral || (ra == W_DECIDED && wa.pos != wal.pos)) {
            wa = w0;
            ra = run_walk<FK_A>(f, q, vb, wa, kNB, T, f.P.top_p, kNoBin, 0xFFFFFFFFu, draw, false);
            if (ra == W_NEED) return out;
        }
        if (ra == W_DECIDED) {  // acc >= top_p at candidate wa.pos - 1 (sampler.rs:241-243)
            keep = wa.pos;
            kb = e_rbin()[wa.run];
            if (__float_as_uint(e_sstart()[kb]) != __float_as_uint(e_shi()[kb])) {
                // total's value at bin kb still depends on a tie: total's sums
                // again (acc's took their slots) and its exact walk
                const uint32_t ba = last_agree(kb);
                request_round(FK_S, ba, false, false, true);
                census_clear();
                eng_pass<EP_SR>(f, q, vb, 0.0f);
                census_finish(vb, t);
                Walk we = w0;
                we.x = e_sstart()[ba];
                we.b = ba;
                we.pos = e_pstart()[ba];
                if (run_walk<FK_S>(f, q, vb, we, kb + 1u, 0.0f, 0.0f, kNoBin, 0xFFFFFFFFu, draw, false) == W_NEED)
                    return out;
                if (!bit_of(e_cpl(), kb)) {
                    if (tid < kNB / 32u) e_req()[tid] = 0u;
                    TSM_LDS_SYNC();
                    if (tid == 0) set_bit(e_req(), kb);
                    TSM_LDS_SYNC();
                    census_clear();
                    eng_pass<EP_CENSUS>(f, q, vb, 0.0f);
                    census_finish(vb, t);
                    if (!bit_of(e_cpl(), kb)) return out;
                }
            }
            if (tid < kWave) {  // the kept mass: total's fold through the kept part of bin kb
                Walk wm;
                wm.tied = 0;
                wm.x = e_sstart()[kb];
                wm.b = kb;
                wm.pos = e_pstart()[kb];
                uint32_t r0, r1;
                runs_of(kb, e_sc()[SC_NRUNS], &r0, &r1);
                walk_runs<FK_S>(wm, r0, r1, 0.0f, 0.0f, keep);
                if (tid == 0) e_sc()[SC_X] = __float_as_uint(wm.x);
            }
            TSM_LDS_SYNC();
            mass = __uint_as_float(e_sc()[SC_X]);
            TSM_LDS_SYNC();
        }
    }
    out.pick.keep = keep;
    out.pick.mass = mass;
    if (dist) {  // Sampler::distribution (sampler.rs:102-116): the kept candidates over mass
        out.pick.token = write_dist_chunks(f, q, len, keep, dist, y0, t, mass);
        return out;
    }
    // the draw (sampler.rs:142-150)
    Walk wr;
    wr.x = u * mass;
    wr.b = 0;
    wr.pos = 0;
    wr.run = wr.within = wr.tied = 0;
    const uint32_t bend = kb != kNoBin ? kb + 1u : kNB;
    // the draw with unresolved ties one way and the other at once; the same pick
    // from both is the draw's, else the exact walk
    Walk wrl = wr;
    uint32_t rrl, rr;
    if (run_walk2<FK_R>(f, q, vb, wrl, wr, &rrl, &rr, bend, 0.0f, 0.0f, kb, keep, draw, false) == W_NEED) return out;
    if (rr != rrl || (rr == W_DECIDED && wr.pos != wrl.pos)) {
        wr = wrl;
        wr.x = u * mass;
        wr.b = 0;
        wr.pos = 0;
        rr = run_walk<FK_R>(f, q, vb, wr, bend, 0.0f, 0.0f, kb, keep, draw, false);
    }
    if (rr == W_NEED) return out;
    uint32_t run = wr.run, within = wr.within;
    if (rr != W_DECIDED) {
        // no step reached r <= 0: the last kept candidate
        uint32_t lb = kb;
        if (lb == kNoBin) {
            if (tid == 0) e_sc()[SC_LAST] = 0u;
            TSM_LDS_SYNC();
            for (uint32_t b = tid; b < kNB; b += kBlock)
                if (e_cnt()[b]) atomicMax(&e_sc()[SC_LAST], b);
            TSM_LDS_SYNC();
            lb = e_sc()[SC_LAST];
        }
        if (!bit_of(e_cpl(), lb)) {
            if (tid < kNB / 32u) e_req()[tid] = 0u;
            TSM_LDS_SYNC();
            if (tid == 0) set_bit(e_req(), lb);
            TSM_LDS_SYNC();
            census_clear();
            eng_pass<EP_CENSUS>(f, q, vb, 0.0f);
            census_finish(vb, t);
            if (!bit_of(e_cpl(), lb)) return out;
        }
        if (!locate(lb, keep - 1u, e_sc()[SC_NRUNS], &run, &within)) return out;
    }
    const uint32_t key = e_hkey()[run];
    const uint32_t minid = e_hmin()[run];
    const float p = e_runp()[run];
    TSM_LDS_SYNC();
    // the pick is the (within+1)-th smallest id among the candidates of value key
    out.pick.token = within == 0u ? minid
                                  : static_cast<uint32_t>(exact_at(
                                        f, q, select_from(f, q, within + 1u, 3, static_cast<uint64_t>(~key) << 32, 32)));
    out.pick.prob = p / mass;
    return out;
}

}  // namespace nuc

// Rows without top-k (window > 1024): the cutoff set (sampler.rs:195-208),
// the window rule, truncation to want, min-p, then top-p and the draw, all
// by re-reading the row.  Up to 1024 survivors are finished by exact_finalize;
// larger sets by the value-bin folds above.  Both reproduce the reference's
// f32 arithmetic.
__device__ __noinline__ Pick reread_nucleus(Fin& f, uint32_t nallow, float u, const DistOut* dist) {
    (void)nallow;
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
    Filt q0;
    q0.order = ORD_TOTAL_Y;
    q0.use_cut = true;
    q0.cut = cut;
    q0.need_allowed = m.constrained;
    uint32_t n0 = 0xFFFFFFFFu;  // not counted
    if (m.constrained) {
        n0 = count_pass<kNucGroup>(f, q0);
        if (n0 == 0) {  // sampler.rs:211-221: every allowed id, by total_cmp
            q0.use_cut = false;
            n0 = count_pass<kNucGroup>(f, q0);
        }
    }
    Filt q1 = q0;
    if (m.want < f.n) {  // ranked.truncate(want)
        if (n0 == 0xFFFFFFFFu) n0 = count_pass<kNucGroup>(f, q0);
        if (n0 > m.want) {
            q1.use_max = true;
            q1.max_comp = select_kth(f, q0, m.want);
        }
    }
    Filt q2 = q1;
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
    }
    const nuc::BigOut bo = nuc::big_nucleus(f, q2, y0, mlo, u, dist);
    if (!bo.small) return bo.pick;
    if (bo.pick.keep == 0) {  // min-p left nothing: the best candidate alone
        q2 = q1;
        q2.use_max = true;
        q2.max_comp = select_kth(f, q1, 1);
    }
    return nucleus_exact(f, q2, u, dist);
}

}  // namespace tsm
