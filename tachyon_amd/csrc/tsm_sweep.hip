// tsm_sweep.hip - pass 1 of the sampling pipeline: one coalesced read of
// every logit.
//
// Grid: (chunks, rows).  A 256-thread workgroup owns one 16384-id chunk of one
// row and holds all of it in registers (16 float4 per thread), so everything
// below costs no further HBM traffic:
//   * the row's history ids that fall in the chunk are counted into an LDS
//     array of u16 counters, and penalties (sampler.rs:165-175 + presence /
//     frequency) are applied in registers;
//   * raw max and sum exp(x - max) for the logsumexp (sampler.rs:298-304);
//   * a superset of the chunk's best Wc penalized values (ties -> lower id)
//     is found without sorting: the Wc-th largest of the 2048 group maxima
//     (8 values each) is a lower bound with >= Wc values above it, located by
//     a two-round 11-bit LDS radix select; every value at or above it is
//     written out as a candidate (typically ~1.1 Wc of them);
//   * for sparse masks, every allowed id of the chunk is listed, so the
//     reference's whole-vocabulary fallback (sampler.rs:211-221) needs no
//     second read.
// Wc = the row's window (top_n size, sampler.rs:186-194), raised so the raw
// top-n for logprobs is covered as well: a raw top-n id either is penalized
// (listed separately with its raw value) or ranks within n + (#penalized) by
// penalized value.
#include "tsm_launch.h"

namespace tsm {

template <bool kVec>
__global__ __launch_bounds__(kSweepThreads) void sweep_kernel(SweepArgs a) {
    const uint32_t chunk = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const uint32_t n = a.usable;
    const uint32_t base = chunk * kChunk;
    const uint32_t len = min(kChunk, n - base);
    const bool full = len == kChunk;
    const size_t slot = static_cast<size_t>(row) * a.n_chunks + chunk;
    const tsm_row_params P = a.params[row];
    uint32_t h0 = 0, hlen = 0;
    if (a.hist_off) {
        h0 = a.hist_off[row];
        const uint32_t h1 = a.hist_off[row + 1];
        hlen = h1 > h0 ? h1 - h0 : 0u;
    }
    const RowMode m = row_mode(P, n, hlen, a.mask != nullptr);

    __shared__ uint32_t s_cnt[kChunk / 2];  // u16 history counts, two per word
    __shared__ uint32_t s_h1[kBins];
    __shared__ uint32_t s_h2[kBins];
    __shared__ uint32_t s_mask[kChunk / 32];
    __shared__ uint32_t s_tmp[16];
    __shared__ uint32_t s_sel[4];
    __shared__ uint32_t s_ctr[4];  // 0: distinct history ids, 1: candidates, 2: pen slots, 3: allow slots
    __shared__ float s_wmax[kSweepThreads / kWave];
    __shared__ double s_wsum[kSweepThreads / kWave];

    // ---- 1. issue the chunk's loads first; HBM latency overlaps the setup ----
    float v[kSweepVec][4];
    const float* rowp = a.logits + static_cast<size_t>(row) * a.row_stride + base;
#pragma unroll
    for (int j = 0; j < kSweepVec; j++) {
        const uint32_t li = 4u * (j * kSweepThreads + tid);
        if (kVec && (full || li + 3 < len)) {
            const float4 f = *reinterpret_cast<const float4*>(rowp + li);
            v[j][0] = f.x;
            v[j][1] = f.y;
            v[j][2] = f.z;
            v[j][3] = f.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) v[j][q] = (li + q < len) ? rowp[li + q] : -INFINITY;
        }
    }

    // ---- 2. LDS setup: histograms, counters, history counts, mask words ----
    for (uint32_t i = tid; i < kBins; i += kSweepThreads) {
        s_h1[i] = 0;
        s_h2[i] = 0;
    }
    if (tid < 4) {
        s_ctr[tid] = 0;
        s_sel[tid] = 0xFFFFFFFFu;
    }
    if (m.penal) {
        uint4* c4 = reinterpret_cast<uint4*>(s_cnt);
        for (uint32_t i = tid; i < kChunk / 8; i += kSweepThreads) c4[i] = make_uint4(0, 0, 0, 0);
    }
    uint32_t my_allowed = 0;
    if (m.constrained) {
        const uint32_t nw = (len + 31) / 32;
        const uint32_t* mrow = a.mask + static_cast<size_t>(row) * a.mask_stride + base / 32;
        for (uint32_t w = tid; w < nw; w += kSweepThreads) {
            uint32_t word = mrow[w];
            if (w == nw - 1 && (len & 31)) word &= (1u << (len & 31)) - 1u;
            s_mask[w] = word;
            my_allowed += __popc(word);
        }
    }
    __syncthreads();
    if (m.penal) {
        const uint32_t hc = min(hlen, TSM_MAX_HISTORY);
        if (hlen > TSM_MAX_HISTORY && chunk == 0 && tid == 0) atomicOr(a.status, TSM_STATUS_HISTORY_TOO_LONG);
        for (uint32_t h = tid; h < hc; h += kSweepThreads) {
            const uint32_t li = a.hist_ids[h0 + h] - base;
            if (li < len) {
                const uint32_t sh = (li & 1u) << 4;
                const uint32_t old = atomicAdd(&s_cnt[li >> 1], 1u << sh);
                if (((old >> sh) & 0xFFFFu) == 0) atomicAdd(&s_ctr[0], 1u);
            }
        }
    }

    // ---- 3. raw max and sum exp(x - max) per thread (logsumexp partials) ----
    float mt = -INFINITY;
#pragma unroll
    for (int j = 0; j < kSweepVec; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) mt = fmaxf(mt, v[j][q]);
    float st = 0.0f;
    if (m.logprobs && mt != -INFINITY) {
#pragma unroll
        for (int j = 0; j < kSweepVec; j++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                st += __builtin_amdgcn_exp2f((v[j][q] - mt) * 1.44269504088896341f);
    }
    __syncthreads();  // history counts complete
    const uint32_t npen = m.penal ? s_ctr[0] : 0u;

    // ---- 4. penalties, in registers ----
    if (npen > 0) {
        uint2* pslot = a.pen + slot * kPenCap;
#pragma unroll
        for (int j = 0; j < kSweepVec; j++) {
            const uint32_t li = 4u * (j * kSweepThreads + tid);
            if (li < len) {
                const uint2 c2 = *reinterpret_cast<const uint2*>(&s_cnt[li >> 1]);
                if (c2.x | c2.y) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t c = ((q < 2 ? c2.x : c2.y) >> ((q & 1) * 16)) & 0xFFFFu;
                        if (c) {
                            const float x = v[j][q];
                            v[j][q] = penalize(x, c, m, P);
                            if (m.logprobs) {
                                const uint32_t pos = atomicAdd(&s_ctr[2], 1u);
                                if (pos < kPenCap) pslot[pos] = make_uint2(base + li + q, __float_as_uint(x));
                            }
                        }
                    }
                }
            }
        }
    }

    // ---- 5. sparse mask: list every allowed id of the chunk ----
    uint32_t n_allowed = 0;
    if (m.constrained) {
        n_allowed = block_sum<kSweepThreads>(my_allowed, s_tmp);
        if (n_allowed <= kAllowCap) {
            uint2* aslot = a.allow + slot * kAllowCap;
#pragma unroll
            for (int j = 0; j < kSweepVec; j++) {
                const uint32_t li = 4u * (j * kSweepThreads + tid);
                if (li < len) {
                    const uint32_t bits = (s_mask[li >> 5] >> (li & 31u)) & 0xFu;
                    if (bits) {
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            if ((bits >> q) & 1u) {
                                const uint32_t pos = atomicAdd(&s_ctr[3], 1u);
                                aslot[pos] = make_uint2(__float_as_uint(v[j][q]), base + li + q);
                            }
                    }
                }
            }
        }
    }

    // ---- 6. candidates: every value at or above a bound with >= Wc above ----
    const uint32_t lp_need = (m.logprobs && m.nlp > 0) ? m.nlp + npen : 0u;
    const uint32_t Wc = m.topk ? max(m.window, lp_need) : lp_need;
    uint32_t flags = 0;
    if (Wc > 0) {
        flags |= CS_HAS_CAND;
        float thr = -INFINITY;  // emit y >= thr
        if (Wc > kCandCap) {
            flags |= CS_CAND_OVERFLOW;
        } else if (Wc < len) {
            uint32_t gd[kGroups];  // ~key of each group max; all-ones = empty group
#pragma unroll
            for (int g = 0; g < kGroups; g++) {
                const uint32_t li0 = 4u * ((kGroupVec * g) * kSweepThreads + tid);
                float gm = -INFINITY;
#pragma unroll
                for (int jj = 0; jj < kGroupVec; jj++)
#pragma unroll
                    for (int q = 0; q < 4; q++) gm = fmaxf(gm, v[kGroupVec * g + jj][q]);
                gd[g] = (full || li0 < len) ? ~canon_key(gm) : 0xFFFFFFFFu;
            }
#pragma unroll
            for (int g = 0; g < kGroups; g++)
                if (gd[g] != 0xFFFFFFFFu) atomicAdd(&s_h1[gd[g] >> 21], 1u);
            __syncthreads();
            hist_find<kSweepThreads>(s_h1, Wc, s_tmp, s_sel);
            const uint32_t b1 = s_sel[0];
            if (b1 != 0xFFFFFFFFu) {
                const uint32_t need = Wc - s_sel[1];
#pragma unroll
                for (int g = 0; g < kGroups; g++)
                    if (gd[g] != 0xFFFFFFFFu && (gd[g] >> 21) == b1)
                        atomicAdd(&s_h2[(gd[g] >> 10) & (kBins - 1)], 1u);
                __syncthreads();
                hist_find<kSweepThreads>(s_h2, need, s_tmp, s_sel + 2);
                const uint32_t kt = ~((b1 << 21) | (s_sel[2] << 10) | 0x3FFu);  // lowest key kept
                thr = kt <= 0x007FFFFFu ? -INFINITY : key_to_float(kt);
            }
        }
        if (!(flags & CS_CAND_OVERFLOW)) {
            uint2* cslot = a.cand + slot * kCandCap;
#pragma unroll
            for (int j = 0; j < kSweepVec; j++) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t li = 4u * (j * kSweepThreads + tid) + q;
                    if ((full || li < len) && v[j][q] >= thr) {
                        bool pen = false;
                        if (npen > 0) pen = ((s_cnt[li >> 1] >> ((li & 1u) << 4)) & 0xFFFFu) != 0;
                        const uint32_t pos = atomicAdd(&s_ctr[1], 1u);
                        if (pos < kCandCap)
                            cslot[pos] = make_uint2(__float_as_uint(v[j][q]),
                                                    (base + li) | (pen ? 0x80000000u : 0u));
                    }
                }
            }
        }
    }

    // ---- 7. chunk statistics ----
    const int lane = tid & (kWave - 1), wid = tid / kWave;
    const float wm = wave_max(mt);
    double sc = 0.0;
    if (m.logprobs && mt != -INFINITY) sc = static_cast<double>(st) * exp(static_cast<double>(mt - wm));
    sc = wave_sum(sc);
    if (lane == 0) {
        s_wmax[wid] = wm;
        s_wsum[wid] = sc;
    }
    __syncthreads();
    if (tid == 0) {
        float cm = -INFINITY;
        for (int w = 0; w < kSweepThreads / kWave; w++) cm = fmaxf(cm, s_wmax[w]);
        double cs = 0.0;
        if (cm != -INFINITY)
            for (int w = 0; w < kSweepThreads / kWave; w++)
                if (s_wmax[w] != -INFINITY) cs += s_wsum[w] * exp(static_cast<double>(s_wmax[w] - cm));
        ChunkStats s;
        s.raw_sum = cs;
        s.raw_max = cm;
        s.n_cand = s_ctr[1];
        s.n_pen = npen;
        s.n_allowed = n_allowed;
        if (s.n_cand > kCandCap) flags |= CS_CAND_OVERFLOW;
        if (m.logprobs && npen > kPenCap) flags |= CS_PEN_OVERFLOW;
        if (m.constrained && n_allowed <= kAllowCap) flags |= CS_ALLOW_LIST;
        s.flags = flags;
        s.pad = 0;
        a.stats[slot] = s;
    }
}

template __global__ void sweep_kernel<true>(SweepArgs);
template __global__ void sweep_kernel<false>(SweepArgs);

void launch_sweep(const SweepArgs& a, uint32_t rows, bool vec, hipStream_t stream) {
    dim3 grid(a.n_chunks, rows);
    if (vec)
        hipLaunchKernelGGL(sweep_kernel<true>, grid, dim3(kSweepThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(sweep_kernel<false>, grid, dim3(kSweepThreads), 0, stream, a);
}

}  // namespace tsm
