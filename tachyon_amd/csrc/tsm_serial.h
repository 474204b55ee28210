// tsm_serial.h - the reference's per-row algorithm taken step by step by one
// wave, for rows whose logits hold a NaN.
//
// With a NaN among the values, top_n (sampler.rs:267-285) stops being an
// order statistic: `v > floor` is false for a NaN, partition_point's
// predicate `w >= v` is no longer monotone over a list that holds one, and
// where a value lands depends on the binary search's probe sequence.  The
// parallel selections of the sampling kernels assume a total order, so a row
// whose logits hold a NaN is sampled here instead, element by element in id
// order, with the insertion and the binary search done as the reference does
// them.  The probe sequence is that of slice::binary_search_by in Rust
// 1.87.0, the toolchain the reference's CI pins (.github/workflows/ci.yml:16-17,
// :64-65): size = len, base = 0; while size > 1 { half = size / 2; mid = base
// + half; the predicate moves base to mid; size -= half }; the position is
// base + pred(base).  The oracle restates the same order (the older halving
// search probes other positions and keeps other ids on such rows).  Such a
// row is pathological (one wave walks the whole row), so nothing here is
// tuned.
//
// Also in the reference's order: argmax (sampler.rs:314-322, the first index
// that nothing after it beats: 0 when x[0] is NaN), the mask filter and the
// whole-vocabulary fallback (sampler.rs:209-222), truncation, the
// probabilities and min-p, the top-p fold and the draw (sampler.rs:138-150,
// :231-246), each a sequential f32 loop in one lane.
#pragma once

#include "tsm_device.h"

namespace tsm {
namespace serial {

// LDS areas of the calling kernel, free while the wave runs here.
struct Lds {
    uint32_t* cnt;   // u32[tile / 2]: 16-bit history counts of the current tile
    float* val;      // f32[kMaxWindow]: the ranked values
    uint32_t* id;    // u32[kMaxWindow]: their ids
    uint64_t* comp;  // u64[kMaxWindow]: the fallback's composites
    float* p;        // f32[kMaxWindow]: p_j (may share comp's bytes)
    uint32_t tile;   // ids per count tile: a power of two
};

struct Row {
    const float* x;         // raw logits, ids [0, n)
    uint32_t n;
    const uint32_t* hist;   // the row's history ids (ids >= n are ignored), or null
    uint32_t hlen;
    const uint32_t* mrow;   // the row's mask words when the row is constrained, else null
    RowMode m;
    tsm_row_params P;
    float u;
};

struct Result {
    uint32_t token;
    uint32_t keep;   // kept count (0: nothing allowed, argmax of the raw row)
    uint32_t len;    // ranked count after truncation and min-p (p[0..len) hold p_j)
    float prob;      // p_pick / mass
    float mass;
};

__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_wave_barrier(); }

__device__ __forceinline__ float lane_f(float v, uint32_t l) {
    return __uint_as_float(wave_read(__float_as_uint(v), l));
}

// argmax (sampler.rs:314-322): best starts at 0 and moves to i when x[i] >
// x[best]; a NaN never beats anything and nothing beats a NaN at 0.
__device__ __noinline__ inline uint32_t argmax_ref(const float* x, uint32_t n) {
    const uint32_t lane = lane_id();
    const float x0 = x[0];
    if (x0 != x0) return 0u;
    // the first maximum among the non-NaN values (x[0] is one of them)
    float bv = x0;
    uint32_t bi = 0u;
    for (uint32_t i = lane; i < n; i += kWave) {
        const float v = x[i];
        if (v > bv) {  // false for NaN; ids rise within a lane, so ties keep the first
            bv = v;
            bi = i;
        }
    }
    // lanes agree on the largest value, then on its lowest id
    float m = bv;
    for (int o = 1; o < kWave; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
    uint32_t c = bv == m ? bi : 0xFFFFFFFFu;
    for (int o = 1; o < kWave; o <<= 1) c = min(c, static_cast<uint32_t>(__shfl_xor(static_cast<int>(c), o, kWave)));
    return c == 0xFFFFFFFFu ? 0u : c;
}

// Counts of the history ids in [t0, t0 + tile) into s.cnt (16 bits per id).
__device__ __noinline__ inline void tile_counts(const Row& r, const Lds& s, uint32_t t0) {
    const uint32_t lane = lane_id();
    for (uint32_t i = lane; i < s.tile / 2u; i += kWave) s.cnt[i] = 0u;
    wave_sync();
    const uint32_t hc = min(r.hlen, TSM_MAX_HISTORY);
    for (uint32_t h = lane; h < hc; h += kWave) {
        const uint32_t id = r.hist[h];
        const uint32_t li = id - t0;
        if (id < r.n && li < s.tile) atomicAdd(&s.cnt[li >> 1], 1u << ((li & 1u) << 4));
    }
    wave_sync();
}

// top_n(values, want) (sampler.rs:267-285) over the penalized row (penal) or
// the raw row: s.val / s.id get the list; returns its length.
__device__ __noinline__ inline uint32_t top_n_ref(const Row& r, const Lds& s, uint32_t want, bool penal) {
    const uint32_t lane = lane_id();
    uint32_t k = 0;
    float floor = -INFINITY;
    if (want == 0) return 0;
    for (uint32_t t0 = 0; t0 < r.n; t0 += s.tile) {
        if (penal) tile_counts(r, s, t0);
        const uint32_t t1 = min(t0 + s.tile, r.n);
        for (uint32_t base = t0; base < t1; base += kWave) {
            const uint32_t i = base + lane;
            const bool in = i < t1;
            float y = in ? r.x[i] : 0.0f;
            if (penal && in) {
                const uint32_t li = i - t0;
                const uint32_t c = (s.cnt[li >> 1] >> ((li & 1u) << 4)) & 0xFFFFu;
                if (c) y = penalize(y, c, r.m, r.P);
            }
            uint32_t done = 0;  // lanes below `done` are handled
            for (;;) {
                const uint64_t cand = wave_ballot(in && lane >= done && (k < want || y > floor));
                if (!cand) break;
                const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(cand));
                const float v = lane_f(y, l);
                // partition_point(|&(w, _)| w >= v) in Rust 1.87.0's probe order
                uint32_t at = 0;
                if (k) {
                    uint32_t size = k, b = 0;
                    while (size > 1u) {
                        const uint32_t half = size / 2u, mid = b + half;
                        if (s.val[mid] >= v) b = mid;
                        size -= half;
                    }
                    at = b + (s.val[b] >= v ? 1u : 0u);
                }
                if (k == want) k--;  // out.pop()
                // out.insert(at, ..): entries [at, k) move up one, top chunk first
                for (uint32_t c = k; c > at;) {
                    const uint32_t c0 = c > at + kWave ? c - kWave : at;
                    const uint32_t j = c0 + lane;
                    float tv = 0.0f;
                    uint32_t ti = 0;
                    if (j < c) {
                        tv = s.val[j];
                        ti = s.id[j];
                    }
                    wave_sync();
                    if (j < c) {
                        s.val[j + 1u] = tv;
                        s.id[j + 1u] = ti;
                    }
                    wave_sync();
                    c = c0;
                }
                if (lane == 0) {
                    s.val[at] = v;
                    s.id[at] = base + l;
                }
                wave_sync();
                k++;
                if (k == want) floor = s.val[want - 1u];
                done = l + 1u;
            }
        }
        if (penal) wave_sync();  // the next tile's counts overwrite these
    }
    return k;
}

__device__ __forceinline__ bool allows(const uint32_t* mrow, uint32_t id) { return (mrow[id >> 5] >> (id & 31u)) & 1u; }

// The whole-vocabulary fallback (sampler.rs:211-221): the allowed ids sorted
// by f32::total_cmp, best first (equal values by id, as the oracle orders
// them), truncated to `want`.  s.val / s.id get the list; returns its length.
__device__ __noinline__ inline uint32_t fallback_ref(const Row& r, const Lds& s, uint32_t want, bool penal) {
    const uint32_t lane = lane_id();
    uint32_t k = 0;
    uint64_t worst = ~0ull;  // the want-th composite once the list is full
    for (uint32_t t0 = 0; t0 < r.n; t0 += s.tile) {
        if (penal) tile_counts(r, s, t0);
        const uint32_t t1 = min(t0 + s.tile, r.n);
        for (uint32_t base = t0; base < t1; base += kWave) {
            const uint32_t i = base + lane;
            const bool in = i < t1 && allows(r.mrow, i);
            float y = in ? r.x[i] : 0.0f;
            if (penal && in) {
                const uint32_t li = i - t0;
                const uint32_t c = (s.cnt[li >> 1] >> ((li & 1u) << 4)) & 0xFFFFu;
                if (c) y = penalize(y, c, r.m, r.P);
            }
            const uint64_t me = composite(total_key(y), i);  // ascending = best first
            uint32_t done = 0;
            for (;;) {
                const uint64_t cand = wave_ballot(in && lane >= done && (k < want || me < worst));
                if (!cand) break;
                const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(cand));
                const uint64_t v = (static_cast<uint64_t>(wave_read(static_cast<uint32_t>(me >> 32), l)) << 32) |
                                   wave_read(static_cast<uint32_t>(me), l);
                // composites are distinct and totally ordered: any probe order
                // gives the same lower bound
                uint32_t lo = 0, hi = k;
                while (lo < hi) {
                    const uint32_t mid = lo + (hi - lo) / 2u;
                    if (s.comp[mid] < v) lo = mid + 1u;
                    else hi = mid;
                }
                const uint32_t at = lo;
                if (k == want) k--;
                for (uint32_t c = k; c > at;) {
                    const uint32_t c0 = c > at + kWave ? c - kWave : at;
                    const uint32_t j = c0 + lane;
                    uint64_t tv = 0;
                    if (j < c) tv = s.comp[j];
                    wave_sync();
                    if (j < c) s.comp[j + 1u] = tv;
                    wave_sync();
                    c = c0;
                }
                if (lane == 0) s.comp[at] = v;
                wave_sync();
                k++;
                if (k == want) worst = s.comp[want - 1u];
                done = l + 1u;
            }
        }
        if (penal) wave_sync();
    }
    for (uint32_t j = lane; j < k; j += kWave) {
        const uint64_t c = s.comp[j];
        s.val[j] = key_to_float(~static_cast<uint32_t>(c >> 32));
        s.id[j] = static_cast<uint32_t>(c);
    }
    wave_sync();
    return k;
}

// Sampler::pick / distribution for a top_n-path row (window <= kMaxWindow)
// or a greedy row of sample() (draw: with the uniform; else the kept set
// only).  Every lane returns the same result.
__device__ __noinline__ inline Result run(const Row& r, const Lds& s, bool draw) {
    const uint32_t lane = lane_id();
    const RowMode& m = r.m;
    Result res;
    res.len = 0;
    res.mass = 0.0f;
    if (draw && !m.constrained && m.greedy && !m.penal) {  // sample()'s shortcut (sampler.rs:79-82)
        res.token = argmax_ref(r.x, r.n);
        res.keep = 1u;
        res.prob = 1.0f;
        return res;
    }
    uint32_t len = top_n_ref(r, s, m.window, m.penal);
    if (m.constrained) {  // ranked.retain(allowed) (sampler.rs:209-210)
        uint32_t w = 0;
        for (uint32_t j0 = 0; j0 < len; j0 += kWave) {
            const uint32_t j = j0 + lane;
            float v = 0.0f;
            uint32_t id = 0;
            bool keep = false;
            if (j < len) {
                v = s.val[j];
                id = s.id[j];
                keep = allows(r.mrow, id);
            }
            const uint64_t b = wave_ballot(keep);
            wave_sync();
            if (keep) {
                s.val[w + lanes_below(b)] = v;
                s.id[w + lanes_below(b)] = id;
            }
            wave_sync();
            w += static_cast<uint32_t>(__popcll(b));
        }
        len = w;
        if (len == 0) len = fallback_ref(r, s, m.want, m.penal);
    }
    len = min(len, m.want);  // ranked.truncate(want)
    if (len == 0) {  // nothing allowed: argmax of the raw row, no draw (sampler.rs:139-141)
        res.token = argmax_ref(r.x, r.n);
        res.keep = 0;
        res.prob = 1.0f;
        return res;
    }
    // p_j in list order (sampler.rs:231-234), then the folds in one lane
    const float best = s.val[0];
    for (uint32_t j = lane; j < len; j += kWave) s.p[j] = glibc_expf((s.val[j] - best) / m.t);
    wave_sync();
    uint32_t keep = 0, pick = 0;
    float prob = 0.0f, mass = 0.0f;
    if (lane == 0) {
        if (!m.greedy && r.P.min_p > 0.0f) {  // min-p: the best-first prefix with p_j >= min_p, at least one
            uint32_t c = 0;
            while (c < len && s.p[c] >= r.P.min_p) c++;
            len = c > 1u ? c : 1u;
        }
        keep = len;
        if (!m.greedy && !(r.P.top_p >= 1.0f)) {  // sampler.rs:238-246
            float total = 0.0f;
            for (uint32_t j = 0; j < len; j++) total += s.p[j];
            float acc = 0.0f;
            for (uint32_t j = 0; j < len; j++) {
                acc += s.p[j] / total;
                if (acc >= r.P.top_p) {
                    keep = j + 1u;
                    break;
                }
            }
        }
        for (uint32_t j = 0; j < keep; j++) mass += s.p[j];  // sampler.rs:142
        pick = keep - 1u;
        if (draw) {
            float rr = r.u * mass;
            for (uint32_t j = 0; j < keep; j++) {
                rr -= s.p[j];
                if (rr <= 0.0f) {
                    pick = j;
                    break;
                }
            }
        }
        prob = s.p[pick] / mass;
    }
    res.len = wave_read(len, 0);
    res.keep = wave_read(keep, 0);
    res.token = s.id[wave_read(pick, 0)];
    res.prob = lane_f(prob, 0);
    res.mass = lane_f(mass, 0);
    return res;
}

}  // namespace serial
}  // namespace tsm
