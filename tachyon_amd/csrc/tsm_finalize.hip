// tsm_finalize.hip - pass 2: one 1024-thread workgroup per row.
//
// Fast path (rows whose window is <= 1024, sampler.rs:193-194): merge the
// chunks' candidates in LDS (bitonic sort, value descending, id ascending),
// take the top `window`, apply the mask with the reference's window rule
// (sampler.rs:209-222), truncate to top-k, and run the reference's own
// sequential f32 arithmetic for probabilities, min-p, top-p and the draw
// (sampler.rs:231-246, :142-150) in one lane, so tokens are bit-exact.
//
// Re-read path (everything else: no top-k and a >1024 window, the
// whole-vocabulary mask fallback without complete allow lists, candidate
// overflow): the workgroup re-reads its row (L2 / MALL resident after the
// sweep) in tiles and answers order-statistic questions with 11-bit LDS radix
// histograms:
//   * select_kth: the k-th element in (value desc, id asc) order;
//   * mass_select: the first element whose cumulative probability reaches a
//     target (f64 partial sums; used when more than 1024 candidates remain).
// When at most 1024 candidates survive truncation and min-p they are
// gathered and finished by the same exact sequential code as the fast path.
#include "tsm_launch.h"

namespace tsm {

// ---- LDS layout (bytes) ------------------------------------------------------
constexpr uint32_t kOffA = 0;                          // 32 KB: merge composites / tile counts
constexpr uint32_t kOffB = kOffA + kMergeCap * 8;      // 12 KB: ranked y, id, p
constexpr uint32_t kOffC = kOffB + kExactCap * 12;     //  8 KB: P, q  | gather composites
constexpr uint32_t kOffD = kOffC + kExactCap * 8;      // 24 KB: histogram counts + f64 mass
constexpr uint32_t kOffE = kOffD + kBins * 12;         // chunk prefix offsets
constexpr uint32_t kMaxChunks = TSM_MAX_VOCAB / kChunk;
constexpr uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }
constexpr uint32_t kOffF = align16(kOffE + (kMaxChunks + 1) * 4);  // raw top-n composites
constexpr uint32_t kOffG = kOffF + 32 * 8;                         // misc words (f64 from M_D0)
static_assert(kOffF % 8 == 0 && (kOffG + 32 * 4) % 8 == 0, "u64/f64 LDS records are 8-byte aligned");
constexpr uint32_t kMisc = 96;  // 32 scalar words + 32 doubles
constexpr uint32_t kSmem = kOffG + kMisc * 4 + 32 * 4;    // + scan tmp
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
    M_NRAW = 11,
    M_FLAG = 12,
    M_STATS = 16,   // 6 words: candidate/allowed/penalized totals, flags, lists, lse
    M_D0 = 32,      // 32 doubles from here: [0] cumulative mass, [8..23] scan scratch
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
};

struct Fin {
    const float* rowp;
    const uint32_t* mrow;
    const uint32_t* hist;
    uint32_t hlen, n;
    RowMode m;
    tsm_row_params P;
    unsigned char* smem;
    uint32_t* cnt;
    uint64_t* comp;
    float* ry;
    uint32_t* rid;
    float* rp;
    float* rP;
    float* rq;
    uint64_t* gcomp;
    uint32_t* hcnt;
    double* hmass;
    uint64_t* big;  // C + D as one u64 array (4096 entries)
    uint32_t* coff;
    uint64_t* rawtop;
    uint32_t* misc;
    double* miscd;
    uint32_t* tmp;
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
    if (q.use_minp && !(glibc_expf((y - q.y0) / f.m.t) >= q.minp)) return false;
    return true;
}

// One re-read of the row in tiles; fn(id, raw, penalized) for every id.
template <class F>
__device__ void row_pass(Fin& f, F&& fn) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t tb = 0; tb < f.n; tb += kTile) {
        const uint32_t tl = min(kTile, f.n - tb);
        if (f.m.penal) {
            __syncthreads();
            for (uint32_t i = tid; i < kTile / 2; i += kFinThreads) f.cnt[i] = 0;
            __syncthreads();
            const uint32_t hc = min(f.hlen, TSM_MAX_HISTORY);
            for (uint32_t h = tid; h < hc; h += kFinThreads) {
                const uint32_t li = f.hist[h] - tb;
                if (li < tl) atomicAdd(&f.cnt[li >> 1], 1u << ((li & 1u) << 4));
            }
            __syncthreads();
        }
        for (uint32_t i = tid; i < tl; i += kFinThreads) {
            const uint32_t id = tb + i;
            const float x = f.rowp[id];
            float y = x;
            if (f.m.penal) {
                const uint32_t c = (f.cnt[i >> 1] >> ((i & 1u) << 4)) & 0xFFFFu;
                if (c) y = penalize(x, c, f.m, f.P);
            }
            fn(id, x, y);
        }
    }
    __syncthreads();
}

// Block-wide bitonic sort, ascending, of n u64 (n a power of two <= 4096).
__device__ void bitonic_sort(uint64_t* a, uint32_t n) {
    for (uint32_t k = 2; k <= n; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n; i += kFinThreads) {
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
            __syncthreads();
        }
}

__device__ __forceinline__ uint32_t pow2_ceil(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Counts filtered elements (one pass).
__device__ uint32_t count_pass(Fin& f, const Filt& q) {
    uint32_t local = 0;
    row_pass(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) local++;
    });
    return block_sum<kFinThreads>(local, f.tmp);
}

// Radix rounds over the 64-bit composite (~key << 32 | id, ids < 2^22): bits
// [lo, lo + width) per round; bits 22..31 are always zero and are skipped.
__constant__ int kRoundLo[5] = {53, 42, 32, 11, 0};
__constant__ int kRoundW[5] = {11, 11, 10, 11, 11};

// Count-based select starting at round r0 with the bits at and above
// position `known_lo` fixed to those of `known`.  Returns T such that exactly
// `need` filtered elements sharing those bits have composite <= T, or ~0 if
// fewer than `need` exist.
__device__ uint64_t select_from(Fin& f, const Filt& q, uint32_t need, int r0, uint64_t known,
                                int known_lo) {
    const uint32_t tid = threadIdx.x;
    for (int r = r0; r < 5; r++) {
        const int lo = kRoundLo[r], w = kRoundW[r];
        for (uint32_t i = tid; i < kBins; i += kFinThreads) f.hcnt[i] = 0;
        if (tid < 2) f.misc[M_FIND + tid] = 0xFFFFFFFFu;
        __syncthreads();
        const uint64_t kn = known;
        const int kl = known_lo;
        row_pass(f, [&](uint32_t id, float x, float y) {
            const uint64_t c = comp_of(q.order, id, x, y);
            if ((kl >= 64 || (c >> kl) == (kn >> kl)) && keep_el(f, q, id, y, c))
                atomicAdd(&f.hcnt[(c >> lo) & ((1u << w) - 1u)], 1u);
        });
        hist_find<kFinThreads>(f.hcnt, need, f.tmp, f.misc + M_FIND);
        const uint32_t d = f.misc[M_FIND];
        if (d == 0xFFFFFFFFu) return ~0ull;
        const uint32_t before = f.misc[M_FIND + 1];
        const uint32_t binc = f.hcnt[d];
        __syncthreads();
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
__device__ uint64_t exact_at(Fin& f, const Filt& q, uint64_t T) {
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
    unsigned long long* wtmp = reinterpret_cast<unsigned long long*>(f.miscd + 8);
    if ((threadIdx.x & (kWave - 1)) == 0) wtmp[threadIdx.x / kWave] = best;
    __syncthreads();
    unsigned long long all = 0;
    for (int w = 0; w < kFinThreads / kWave; w++) all = wtmp[w] > all ? wtmp[w] : all;
    __syncthreads();
    return all == 0 ? ~0ull : all - 1ull;
}

// Block-wide exclusive f64 scan (1024 threads).
__device__ double block_excl_scan_f64(double v, double* tmp, double* total) {
    constexpr int NW = kFinThreads / kWave;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    double inc = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const double w = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += w;
    }
    if (lane == kWave - 1) tmp[wid] = inc;
    __syncthreads();
    double before = 0.0, all = 0.0;
    for (int w = 0; w < NW; w++) {
        const double t = tmp[w];
        if (w < wid) before += t;
        all += t;
    }
    __syncthreads();
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
__device__ MassSel mass_select(Fin& f, const Filt& q, float y0, double target) {
    const uint32_t tid = threadIdx.x;
    uint64_t known = 0;
    int known_lo = 64;
    double cum_before = 0.0;
    uint32_t cnt_before = 0;
    double* dtmp = f.miscd + 8;
    for (int r = 0; r < 3; r++) {
        const int lo = kRoundLo[r], w = kRoundW[r];
        for (uint32_t i = tid; i < kBins; i += kFinThreads) {
            f.hcnt[i] = 0;
            f.hmass[i] = 0.0;
        }
        if (tid == 0) {
            f.misc[M_FIND] = 0xFFFFFFFFu;
            f.misc[M_FIND2] = 0;
        }
        __syncthreads();
        const uint64_t kn = known;
        const int kl = known_lo;
        row_pass(f, [&](uint32_t id, float x, float y) {
            const uint64_t c = comp_of(q.order, id, x, y);
            if ((kl >= 64 || (c >> kl) == (kn >> kl)) && keep_el(f, q, id, y, c)) {
                const uint32_t d = (c >> lo) & ((1u << w) - 1u);
                atomicAdd(&f.hcnt[d], 1u);
                atomicAdd(&f.hmass[d], static_cast<double>(glibc_expf((y - y0) / f.m.t)));
            }
        });
        // thread t owns bins 2t, 2t+1
        const uint32_t b0 = 2 * tid;
        const uint32_t c0 = f.hcnt[b0], c1 = f.hcnt[b0 + 1];
        const double m0 = f.hmass[b0], m1 = f.hmass[b0 + 1];
        double mtot;
        const double mb = block_excl_scan_f64(m0 + m1, dtmp, &mtot);
        uint32_t ctot;
        const uint32_t cb = block_excl_scan<kFinThreads>(c0 + c1, f.tmp, &ctot);
        const double base = cum_before + mb;
        uint32_t cand = 0xFFFFFFFFu;
        if (c0 > 0 && base + m0 >= target) cand = b0;
        else if (c1 > 0 && base + m0 + m1 >= target) cand = b0 + 1;
        if (cand != 0xFFFFFFFFu) atomicMin(&f.misc[M_FIND], cand);
        if (c0 + c1 > 0) atomicMax(&f.misc[M_FIND2], (c1 > 0 ? b0 + 1 : b0) + 1);  // last nonempty + 1
        __syncthreads();
        uint32_t d = f.misc[M_FIND];
        const bool overshoot = d == 0xFFFFFFFFu;  // read now: select_from below rewrites M_FIND
        if (overshoot) d = f.misc[M_FIND2] - 1;   // target beyond the total: last element
        if ((d >> 1) == tid) {
            const bool second = d & 1u;
            f.miscd[0] = base + (second ? m0 : 0.0);
            f.misc[M_CNT] = cb + (second ? c0 : 0u);
            f.misc[M_TOTAL] = second ? c1 : c0;
        }
        __syncthreads();
        cum_before = f.miscd[0];
        cnt_before += f.misc[M_CNT];
        const uint32_t ties = f.misc[M_TOTAL];
        known |= static_cast<uint64_t>(d) << lo;
        known_lo = lo;
        __syncthreads();
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
__device__ double mass_total(Fin& f, const Filt& q, float y0) {
    double local = 0.0;
    row_pass(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) local += static_cast<double>(glibc_expf((y - y0) / f.m.t));
    });
    double tot;
    block_excl_scan_f64(local, f.miscd + 8, &tot);
    return tot;
}

// Gathers filtered elements' composites into gcomp (caller guarantees <= cap).
__device__ uint32_t gather_pass(Fin& f, const Filt& q, uint32_t cap) {
    if (threadIdx.x == 0) f.misc[M_CNT] = 0;
    __syncthreads();
    row_pass(f, [&](uint32_t id, float x, float y) {
        const uint64_t c = comp_of(q.order, id, x, y);
        if (keep_el(f, q, id, y, c)) {
            const uint32_t pos = atomicAdd(&f.misc[M_CNT], 1u);
            if (pos < cap) f.gcomp[pos] = c;
        }
    });
    const uint32_t n = min(f.misc[M_CNT], cap);
    __syncthreads();
    return n;
}

// Sorts gcomp[0..n) and unpacks it into the ranked arrays (ids in the low word).
__device__ void sort_gathered(Fin& f, uint32_t n) {
    const uint32_t n2 = pow2_ceil(max(n, 1u));
    for (uint32_t i = n + threadIdx.x; i < n2; i += kFinThreads) f.gcomp[i] = ~0ull;
    __syncthreads();
    bitonic_sort(f.gcomp, n2);
    for (uint32_t j = threadIdx.x; j < n; j += kFinThreads) {
        const uint64_t c = f.gcomp[j];
        f.ry[j] = key_to_float(~static_cast<uint32_t>(c >> 32));
        f.rid[j] = static_cast<uint32_t>(c);
    }
    __syncthreads();
}

struct Pick {
    uint32_t token, keep;
    float prob;
    float mass;
};

// The reference's arithmetic on a ranked list of `len` (<= 1024) candidates,
// best first: p_j (sampler.rs:231-234), min-p (extension), top-p
// (sampler.rs:235-246), draw (sampler.rs:142-150).  Sequential sums run in
// one lane so every f32 rounding matches the CPU sampler.
__device__ Pick exact_finalize(Fin& f, uint32_t len, float u, bool draw) {
    const uint32_t tid = threadIdx.x;
    const float y0 = f.ry[0];
    for (uint32_t j = tid; j < len; j += kFinThreads) f.rp[j] = glibc_expf((f.ry[j] - y0) / f.m.t);
    if (tid == 0) f.misc[M_FIRST] = len;
    __syncthreads();
    if (!f.m.greedy && f.P.min_p > 0.0f) {
        for (uint32_t j = tid; j < len; j += kFinThreads)
            if (!(f.rp[j] >= f.P.min_p)) atomicMin(&f.misc[M_FIRST], j);
        __syncthreads();
        len = max(f.misc[M_FIRST], 1u);
    }
    const bool topp = !(f.m.greedy || f.P.top_p >= 1.0f);
    if (tid == 0) {
        float total = 0.0f;
        for (uint32_t j = 0; j < len; j++) {
            total += f.rp[j];
            f.rP[j] = total;
        }
    }
    __syncthreads();
    if (topp) {
        const float total = f.rP[len - 1];
        for (uint32_t j = tid; j < len; j += kFinThreads) f.rq[j] = f.rp[j] / total;
        __syncthreads();
    }
    if (tid == 0) {
        uint32_t keep = len;
        if (topp) {
            float acc = 0.0f;
            for (uint32_t j = 0; j < len; j++) {
                acc += f.rq[j];
                if (acc >= f.P.top_p) {
                    keep = j + 1;
                    break;
                }
            }
        }
        const float mass = f.rP[keep - 1];
        uint32_t pick = keep - 1;
        if (draw) {
            float r = u * mass;
            for (uint32_t j = 0; j < keep; j++) {
                r -= f.rp[j];
                if (r <= 0.0f) {
                    pick = j;
                    break;
                }
            }
        }
        f.misc[M_TOKEN] = f.rid[pick];
        f.misc[M_KEEP] = keep;
        f.misc[M_PROB] = __float_as_uint(f.rp[pick] / mass);
        f.misc[M_MASS] = __float_as_uint(mass);
    }
    __syncthreads();
    Pick p;
    p.token = f.misc[M_TOKEN];
    p.keep = f.misc[M_KEEP];
    p.prob = __uint_as_float(f.misc[M_PROB]);
    p.mass = __uint_as_float(f.misc[M_MASS]);
    return p;
}

// Writes the first min(keep, dist_stride) entries of the exact distribution.
__device__ void write_dist_exact(const Fin& f, const FinArgs& a, uint32_t row, const Pick& p) {
    const size_t o = static_cast<size_t>(row) * a.dist_stride;
    const uint32_t k = min(p.keep, a.dist_stride);
    for (uint32_t j = threadIdx.x; j < k; j += kFinThreads) {
        a.dist_ids[o + j] = f.rid[j];
        a.dist_probs[o + j] = f.rp[j] / p.mass;
    }
    if (p.keep > a.dist_stride && threadIdx.x == 0) atomicOr(a.status, TSM_STATUS_DIST_TRUNCATED);
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
    const bool ok = tid < g && allowed_bit(f, f.rid[tid]);
    const float yv = tid < g ? f.ry[tid] : 0.0f;
    const uint32_t idv = tid < g ? f.rid[tid] : 0u;
    uint32_t total;
    const uint32_t pos = block_excl_scan<kFinThreads>(ok ? 1u : 0u, f.tmp, &total);
    if (ok) {
        f.ry[pos] = yv;
        f.rid[pos] = idv;
    }
    __syncthreads();
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

__global__ __launch_bounds__(kFinThreads) void finalize_kernel(FinArgs a) {
    HIP_DYNAMIC_SHARED(unsigned char, smem_raw)
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t n = a.usable;
    const tsm_row_params P = a.params[row];
    uint32_t h0 = 0, hlen = 0;
    if (a.hist_off) {
        h0 = a.hist_off[row];
        const uint32_t h1 = a.hist_off[row + 1];
        hlen = h1 > h0 ? h1 - h0 : 0u;
    }
    Fin f;
    f.rowp = a.logits + static_cast<size_t>(row) * a.row_stride;
    f.mrow = a.mask ? a.mask + static_cast<size_t>(row) * a.mask_stride : nullptr;
    f.hist = a.hist_ids ? a.hist_ids + h0 : nullptr;
    f.hlen = hlen;
    f.n = n;
    f.m = row_mode(P, n, hlen, a.mask != nullptr);
    if (a.distribution) f.m = row_mode(P, n, hlen, false);  // distribution() takes no constraint
    f.P = P;
    f.smem = smem_raw;
    f.cnt = reinterpret_cast<uint32_t*>(smem_raw + kOffA);
    f.comp = reinterpret_cast<uint64_t*>(smem_raw + kOffA);
    f.ry = reinterpret_cast<float*>(smem_raw + kOffB);
    f.rid = reinterpret_cast<uint32_t*>(smem_raw + kOffB + kExactCap * 4);
    f.rp = reinterpret_cast<float*>(smem_raw + kOffB + kExactCap * 8);
    f.rP = reinterpret_cast<float*>(smem_raw + kOffC);
    f.rq = reinterpret_cast<float*>(smem_raw + kOffC + kExactCap * 4);
    f.gcomp = reinterpret_cast<uint64_t*>(smem_raw + kOffC);
    f.hcnt = reinterpret_cast<uint32_t*>(smem_raw + kOffD);
    f.hmass = reinterpret_cast<double*>(smem_raw + kOffD + kBins * 4);
    f.big = reinterpret_cast<uint64_t*>(smem_raw + kOffC);
    f.coff = reinterpret_cast<uint32_t*>(smem_raw + kOffE);
    f.rawtop = reinterpret_cast<uint64_t*>(smem_raw + kOffF);
    f.misc = reinterpret_cast<uint32_t*>(smem_raw + kOffG);
    f.miscd = reinterpret_cast<double*>(smem_raw + kOffG + M_D0 * 4);
    f.tmp = reinterpret_cast<uint32_t*>(smem_raw + kOffG + kMisc * 4);
    const RowMode& m = f.m;
    const uint32_t C = a.n_chunks;
    const ChunkStats* st = a.stats + static_cast<size_t>(row) * C;

    // ---- 1. chunk statistics: logsumexp, candidate totals, allowed count ----
    // (wave 0 reduces; C <= 256)
    if (tid < 64) {
        float mx = -INFINITY;
        uint32_t ncand = 0, nallow = 0, npen = 0, fl_or = 0, all_lists = 1;
        for (uint32_t c = tid; c < C; c += 64) {
            const ChunkStats s = st[c];
            mx = fmaxf(mx, s.raw_max);
            ncand += min(s.n_cand, kCandCap);
            nallow += s.n_allowed;
            npen += min(s.n_pen, kPenCap);
            fl_or |= s.flags;
            all_lists &= (s.flags & CS_ALLOW_LIST) ? 1u : 0u;
        }
        mx = wave_max(mx);
        double sum = 0.0;
        for (uint32_t c = tid; c < C; c += 64) {
            const ChunkStats s = st[c];
            if (s.raw_max != -INFINITY) sum += s.raw_sum * exp(static_cast<double>(s.raw_max - mx));
        }
        sum = wave_sum(sum);
        ncand = wave_sum(ncand);
        nallow = wave_sum(nallow);
        npen = wave_sum(npen);
        for (int o = 32; o > 0; o >>= 1) {
            fl_or |= __shfl_xor(fl_or, o, kWave);
            all_lists &= __shfl_xor(all_lists, o, kWave);
        }
        if (tid == 0) {
            f.misc[M_STATS + 0] = ncand;
            f.misc[M_STATS + 1] = nallow;
            f.misc[M_STATS + 2] = npen;
            f.misc[M_STATS + 3] = fl_or;
            f.misc[M_STATS + 4] = all_lists;
            // sampler.rs:298-304: lse = max + (f32) ln(sum exp((f64)(l - max)))
            f.misc[M_STATS + 5] = __float_as_uint(mx + static_cast<float>(log(sum)));
        }
    }
    __syncthreads();
    const uint32_t ncand = f.misc[M_STATS + 0], nallow = f.misc[M_STATS + 1], npen_tot = f.misc[M_STATS + 2];
    const uint32_t fl_or = f.misc[M_STATS + 3];
    const bool all_lists = f.misc[M_STATS + 4] != 0;
    const float lse = __uint_as_float(f.misc[M_STATS + 5]);
    const bool has_cand = (fl_or & CS_HAS_CAND) != 0;
    const bool cand_ok = has_cand && !(fl_or & CS_CAND_OVERFLOW) && ncand <= kMergeCap;

    // ---- 2. load and sort the candidates (value desc, id asc) ----
    uint32_t n2 = 0;
    if (cand_ok) {
        if (tid == 0) {
            uint32_t acc = 0;
            for (uint32_t c = 0; c < C; c++) {
                f.coff[c] = acc;
                acc += min(st[c].n_cand, kCandCap);
            }
            f.coff[C] = acc;
        }
        __syncthreads();
        n2 = pow2_ceil(max(ncand, 1u));
        for (uint32_t c = 0; c < C; c++) {
            const uint32_t o = f.coff[c], k = f.coff[c + 1] - o;
            const uint2* src = a.cand + (static_cast<size_t>(row) * C + c) * kCandCap;
            for (uint32_t i = tid; i < k; i += kFinThreads) {
                const uint2 e = src[i];
                const uint32_t id = e.y & 0x7FFFFFFFu;
                f.comp[o + i] = composite(canon_key(__uint_as_float(e.x)), (id << 1) | (e.y >> 31));
            }
        }
        for (uint32_t i = ncand + tid; i < n2; i += kFinThreads) f.comp[i] = ~0ull;
        __syncthreads();
        bitonic_sort(f.comp, n2);
    }

    // ---- 3. raw top-n for logprobs from the candidates ----
    // Non-penalized candidates carry their raw value; penalized ids come from
    // the chunks' penalized lists with their raw values.
    bool raw_ok = false;
    uint32_t nraw = 0;
    const bool want_lp = m.logprobs && a.out_top_ids != nullptr && m.nlp > 0;
    if (want_lp && m.nlp > a.top_stride) {  // the list must fit the row's slots
        if (tid == 0) atomicOr(a.status, TSM_STATUS_BAD_PARAMS);
        f.m.nlp = a.top_stride;
    }
    if (want_lp && cand_ok && !(fl_or & CS_PEN_OVERFLOW) && npen_tot + m.nlp <= kMergeCap) {
        // (a) first nlp non-penalized entries of the sorted list
        if (tid == 0) {
            uint32_t k = 0;
            for (uint32_t i = 0; i < ncand && k < m.nlp; i++) {
                const uint64_t c = f.comp[i];
                if ((c & 1ull) == 0) {
                    f.big[k++] = (c & 0xFFFFFFFF00000000ull) | ((c & 0xFFFFFFFFull) >> 1);
                }
            }
            f.misc[M_NRAW] = k;
        }
        __syncthreads();
        const uint32_t k0 = f.misc[M_NRAW];
        // (b) every penalized id with its raw value
        if (tid == 0) {
            uint32_t acc = k0;
            for (uint32_t c = 0; c < C; c++) {
                f.coff[c] = acc;
                acc += min(st[c].n_pen, kPenCap);
            }
            f.coff[C] = acc;
        }
        __syncthreads();
        for (uint32_t c = 0; c < C; c++) {
            const uint32_t o = f.coff[c], k = f.coff[c + 1] - o;
            const uint2* src = a.pen + (static_cast<size_t>(row) * C + c) * kPenCap;
            for (uint32_t i = tid; i < k; i += kFinThreads) {
                const uint2 e = src[i];
                f.big[o + i] = composite(canon_key(__uint_as_float(e.y)), e.x);
            }
        }
        const uint32_t tot = f.coff[C];
        const uint32_t p2 = pow2_ceil(max(tot, 1u));
        __syncthreads();
        for (uint32_t i = tot + tid; i < p2; i += kFinThreads) f.big[i] = ~0ull;
        __syncthreads();
        bitonic_sort(f.big, p2);
        nraw = min(tot, m.nlp);
        if (tid < nraw) f.rawtop[tid] = f.big[tid];
        __syncthreads();
        raw_ok = true;
    }

    // ---- 4. sampling ----
    const float u = (a.uniforms && !a.distribution) ? a.uniforms[row] : 0.0f;
    Pick pk;
    bool done = false;
    const bool none_allowed = m.constrained && nallow == 0;
    if (none_allowed) {
        // nothing allowed: argmax of the raw row, no draw (sampler.rs:139-141)
        uint32_t tok;
        if (raw_ok && nraw > 0) {
            tok = static_cast<uint32_t>(f.rawtop[0]);
        } else {
            Filt q;
            q.order = ORD_CANON_X;
            tok = static_cast<uint32_t>(exact_at(f, q, select_kth(f, q, 1)));
        }
        pk.token = tok;
        pk.keep = 0;
        pk.prob = 1.0f;
        pk.mass = 0.0f;
        done = true;
    }
    if (!done && m.topk && cand_ok) {
        // fast path: window = top `window` of the merged candidates
        const uint32_t W = m.window;
        const uint32_t wv = min(W, ncand);
        uint32_t len;
        if (m.constrained) {
            const bool in = tid < wv;
            uint32_t id = 0;
            float yv = 0.0f;
            bool ok = false;
            if (in) {
                const uint64_t c = f.comp[tid];
                id = static_cast<uint32_t>(c) >> 1;
                yv = key_to_float(~static_cast<uint32_t>(c >> 32));
                ok = allowed_bit(f, id);
            }
            uint32_t total;
            const uint32_t pos = block_excl_scan<kFinThreads>(ok ? 1u : 0u, f.tmp, &total);
            if (ok && pos < f.m.want) {
                f.ry[pos] = yv;
                f.rid[pos] = id;
            }
            __syncthreads();
            len = min(total, m.want);
        } else {
            for (uint32_t j = tid; j < min(wv, m.want); j += kFinThreads) {
                const uint64_t c = f.comp[j];
                f.ry[j] = key_to_float(~static_cast<uint32_t>(c >> 32));
                f.rid[j] = static_cast<uint32_t>(c) >> 1;
            }
            __syncthreads();
            len = min(wv, m.want);
        }
        if (len > 0) {
            pk = exact_finalize(f, len, u, !a.distribution);
            done = true;
        } else if (m.constrained && all_lists && nallow <= kMergeCap) {
            // whole-vocabulary fallback from the chunks' allow lists
            if (tid == 0) {
                uint32_t acc = 0;
                for (uint32_t c = 0; c < C; c++) {
                    f.coff[c] = acc;
                    acc += st[c].n_allowed;
                }
                f.coff[C] = acc;
            }
            __syncthreads();
            for (uint32_t c = 0; c < C; c++) {
                const uint32_t o = f.coff[c], k = f.coff[c + 1] - o;
                const uint2* src = a.allow + (static_cast<size_t>(row) * C + c) * kAllowCap;
                for (uint32_t i = tid; i < k; i += kFinThreads) {
                    const uint2 e = src[i];
                    f.comp[o + i] = composite(total_key(__uint_as_float(e.x)), e.y);
                }
            }
            const uint32_t p2 = pow2_ceil(max(nallow, 1u));
            for (uint32_t i = nallow + tid; i < p2; i += kFinThreads) f.comp[i] = ~0ull;
            __syncthreads();
            bitonic_sort(f.comp, p2);
            const uint32_t l2 = min(nallow, m.want);
            for (uint32_t j = tid; j < l2; j += kFinThreads) {
                const uint64_t c = f.comp[j];
                f.ry[j] = key_to_float(~static_cast<uint32_t>(c >> 32));
                f.rid[j] = static_cast<uint32_t>(c);
            }
            __syncthreads();
            pk = exact_finalize(f, l2, u, !a.distribution);
            done = true;
        }
    }
    if (!done) {
        if (m.topk) {
            uint32_t len = 0;
            bool have = false;
            if (!(cand_ok && m.constrained)) have = slow_topk_window(f, &len);
            if (!have) len = slow_fallback(f, nallow);
            pk = exact_finalize(f, len, u, !a.distribution);
        } else {
            // no top-k: cutoff set (sampler.rs:195-208), then the window rule
            float mall = -INFINITY, mal = -INFINITY;
            {
                float la = -INFINITY, lb = -INFINITY;
                row_pass(f, [&](uint32_t id, float x, float y) {
                    la = fmaxf(la, y);
                    if (m.constrained && allowed_bit(f, id)) lb = fmaxf(lb, y);
                });
                la = wave_max(la);
                lb = wave_max(lb);
                float* ftmp = reinterpret_cast<float*>(f.miscd + 8);
                if ((tid & 63) == 0) {
                    ftmp[tid / 64] = la;
                    ftmp[16 + tid / 64] = lb;
                }
                __syncthreads();
                for (int w = 0; w < 16; w++) {
                    mall = fmaxf(mall, ftmp[w]);
                    mal = fmaxf(mal, ftmp[16 + w]);
                }
                __syncthreads();
            }
            const float cut = mall - 30.0f * m.t;  // sampler.rs:198-199
            Filt q0;
            q0.order = ORD_TOTAL_Y;
            q0.use_cut = true;
            q0.cut = cut;
            float y0 = mall;
            uint32_t n0;
            if (m.constrained) {
                q0.need_allowed = true;
                n0 = count_pass(f, q0);
                if (n0 == 0) {  // sampler.rs:211-221
                    q0.use_cut = false;
                    n0 = nallow;
                }
                y0 = mal;
            } else {
                n0 = count_pass(f, q0);
            }
            Filt q1 = q0;
            uint32_t n1 = n0;
            if (n0 > m.want) {  // ranked.truncate(want)
                q1.use_max = true;
                q1.max_comp = select_kth(f, q0, m.want);
                n1 = m.want;
            }
            Filt q2 = q1;
            uint32_t n2c = n1;
            if (P.min_p > 0.0f) {  // extension: min-p prefix
                q2.use_minp = true;
                q2.y0 = y0;
                q2.minp = P.min_p;
                n2c = count_pass(f, q2);
                if (n2c == 0) {
                    q2 = q1;
                    q2.use_max = true;
                    q2.max_comp = select_kth(f, q1, 1);
                    n2c = 1;
                }
            }
            if (n2c <= kExactCap) {
                const uint32_t g = gather_pass(f, q2, kExactCap);
                sort_gathered(f, g);
                pk = exact_finalize(f, g, u, !a.distribution);
            } else {
                // more than 1024 candidates: exact-arithmetic cumulative sums
                const double total = mass_total(f, q2, y0);
                Filt q3 = q2;
                double mass = total;
                uint32_t keep = n2c;
                if (!(P.top_p >= 1.0f)) {
                    const MassSel sp = mass_select(f, q2, y0, static_cast<double>(P.top_p) * total);
                    q3.use_max = true;
                    q3.max_comp = sp.T;
                    mass = sp.cum;
                    keep = sp.rank;
                }
                if (a.distribution) {
                    Filt qd = q3;
                    const uint32_t k = min(keep, a.dist_stride);
                    if (k < keep) {
                        qd.use_max = true;
                        qd.max_comp = select_kth(f, q3, k);
                    }
                    const uint32_t g = gather_pass(f, qd, kExactCap);
                    sort_gathered(f, g);
                    const size_t o = static_cast<size_t>(row) * a.dist_stride;
                    for (uint32_t j = tid; j < g; j += kFinThreads) {
                        a.dist_ids[o + j] = f.rid[j];
                        a.dist_probs[o + j] = static_cast<float>(
                            static_cast<double>(glibc_expf((f.ry[j] - y0) / m.t)) / mass);
                    }
                    if (keep > a.dist_stride && tid == 0) atomicOr(a.status, TSM_STATUS_DIST_TRUNCATED);
                    if (tid == 0) a.out_keep[row] = keep;
                    return;
                }
                const MassSel sr = mass_select(f, q3, y0, static_cast<double>(u) * mass);
                const uint64_t ce = exact_at(f, q3, sr.T);
                const uint32_t ktok = static_cast<uint32_t>(ce);
                const float yk = key_to_float(~static_cast<uint32_t>(ce >> 32));
                pk.token = ktok;
                pk.keep = keep;
                pk.prob = static_cast<float>(static_cast<double>(glibc_expf((yk - y0) / m.t)) / mass);
                pk.mass = static_cast<float>(mass);
            }
        }
    }

    // ---- 5. outputs ----
    if (pk.token >= n) {  // a selection came back empty (e.g. NaN logits)
        if (tid == 0) atomicOr(a.status, TSM_STATUS_INTERNAL);
        pk.token = 0;
    }
    if (a.distribution) {
        if (pk.keep > 0) write_dist_exact(f, a, row, pk);
        if (tid == 0) a.out_keep[row] = pk.keep;
        return;
    }
    if (tid == 0) {
        a.out_token[row] = pk.token;
        if (a.out_prob) a.out_prob[row] = pk.prob;
        if (a.out_keep) a.out_keep[row] = pk.keep;
        if (m.logprobs && a.out_logprob) a.out_logprob[row] = f.rowp[pk.token] - lse;
    }
    if (want_lp) {
        if (!raw_ok) {
            Filt q;
            q.order = ORD_CANON_X;
            const uint64_t T = select_kth(f, q, m.nlp);
            q.use_max = true;
            q.max_comp = T;
            const uint32_t g = gather_pass(f, q, kExactCap);
            const uint32_t g2 = pow2_ceil(max(g, 1u));
            for (uint32_t i = g + tid; i < g2; i += kFinThreads) f.gcomp[i] = ~0ull;
            __syncthreads();
            bitonic_sort(f.gcomp, g2);
            nraw = min(g, m.nlp);
            if (tid < nraw) f.rawtop[tid] = f.gcomp[tid];
            __syncthreads();
        }
        if (tid < nraw) {
            const uint64_t c = f.rawtop[tid];
            const uint32_t id = static_cast<uint32_t>(c);
            const float x = key_to_float(~static_cast<uint32_t>(c >> 32));
            const size_t o = static_cast<size_t>(row) * a.top_stride + tid;
            a.out_top_ids[o] = id;
            if (a.out_top_lp) a.out_top_lp[o] = x - lse;
        }
    }
}

void launch_finalize(const FinArgs& a, uint32_t rows, hipStream_t stream) {
    hipLaunchKernelGGL(finalize_kernel, dim3(rows), dim3(kFinThreads), kSmem, stream, a);
}

hipError_t finalize_set_smem_attr() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&finalize_kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kSmem));
}

}  // namespace tsm
