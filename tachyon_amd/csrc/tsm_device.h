// tsm_device.h - constants, scratch records and device helpers shared by the
// sampling kernels (gfx950, wave64).  Compiled with -ffp-contract=off: every
// float/double operation below rounds on its own unless an fma is written out.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tachyon_sampler.h"

namespace tsm {

// ---- geometry --------------------------------------------------------------
constexpr int kWave = 64;
constexpr int kBlock = 1024;           // one workgroup (16 waves) per row
constexpr int kVec = 2;                // float4 loads per thread per tile
constexpr uint32_t kTile = kBlock * kVec * 4;  // 8192 ids per tile of the streaming pass
constexpr uint32_t kMaxWindow = 1024;  // top_n path bound (sampler.rs:193)
constexpr uint32_t kWideWindow = 256;  // constrained window floor (sampler.rs:186-187)
constexpr uint32_t kExactCap = 1024;   // longest ranked list finished exactly
constexpr uint32_t kWaveList = 64;     // longest ranked list the single-wave finish takes
constexpr uint32_t kBitmapWords = 8192;  // history bitmap: rows of up to 262144 ids
constexpr uint32_t kHashSlots = 4096;    // history count table (histories up to kHistFast ids)
constexpr uint32_t kHistFast = kHashSlots / 2;
constexpr uint32_t kBins = 2048;       // radix histogram bins (11-bit digits)

// ---- per-row mode (sampler.rs:161-190 + extensions) -------------------------
struct RowMode {
    float t;                // temperature, 1 when greedy
    uint32_t want;          // kept after truncation (A3)
    uint32_t window;        // ranked before the mask filter (A3)
    uint32_t nlp;           // logprob alternatives
    bool greedy, topk, constrained, logprobs, pen_rep, pen_pf, penal;
};

__device__ __host__ inline RowMode row_mode(const tsm_row_params& p, uint32_t n,
                                            uint32_t hist_len, bool have_mask) {
    RowMode m;
    m.greedy = p.temperature <= 0.0f;
    m.t = m.greedy ? 1.0f : p.temperature;
    m.want = m.greedy ? 1u : (p.top_k == 0 ? n : (p.top_k < n ? p.top_k : n));
    m.constrained = have_mask && (p.flags & TSM_ROW_CONSTRAINED);
    uint32_t w = m.want > kWideWindow ? m.want : kWideWindow;
    m.window = m.constrained ? (w < n ? w : n) : m.want;
    m.topk = m.window <= kMaxWindow;
    m.logprobs = (p.flags & TSM_ROW_LOGPROBS) != 0;
    uint32_t nl = p.n_logprobs < TSM_MAX_LOGPROBS ? p.n_logprobs : TSM_MAX_LOGPROBS;
    m.nlp = m.logprobs ? (nl < n ? nl : n) : 0u;
    m.pen_rep = hist_len > 0 && p.repetition_penalty != 1.0f;
    m.pen_pf = hist_len > 0 && (p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f);
    m.penal = m.pen_rep || m.pen_pf;
    return m;
}

// Repetition penalty (sampler.rs:172) then presence/frequency (extension),
// for an id that occurs `c` > 0 times in the row's history.
__device__ __forceinline__ float penalize(float l, uint32_t c, const RowMode& m,
                                          const tsm_row_params& p) {
    if (m.pen_rep) l = l > 0.0f ? l / p.repetition_penalty : l * p.repetition_penalty;
    if (m.pen_pf) {
        float fc = p.frequency_penalty * static_cast<float>(c);
        l = l - fc;
        l = l - p.presence_penalty;
    }
    return l;
}

// ---- order keys ---------------------------------------------------------------
// f32::total_cmp order as an unsigned key (sort_unstable_by, sampler.rs:207).
__device__ __forceinline__ uint32_t total_key(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// IEEE order with -0 == +0, as top_n's >= / > compare (sampler.rs:274-275).
__device__ __forceinline__ uint32_t canon_key(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u << 1) == 0) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// Composite sort key, ascending = best first: value descending, id ascending.
__device__ __forceinline__ uint64_t composite(uint32_t key, uint32_t low) {
    return (static_cast<uint64_t>(~key) << 32) | low;
}

// ---- glibc expf, bit for bit ---------------------------------------------------
// Rust's f32::exp calls glibc expf on linux-gnu (sampler.rs:234).  glibc's
// expf (sysdeps/ieee754/flt-32/e_expf.c, Szabolcs Nagy's method) evaluates
// 2^(k/32) * 2^(r/32) in double with a 32-entry table and a cubic, and its
// x86-64 FMA build fuses r = x*N/ln2 - k and the polynomial.  This is the same
// method, written out with the same fused operations; it was checked against
// the host's glibc expf on every float in [-104, 88.8] (2.24e9 inputs, 0
// mismatches) and tests/test_gpu_parity.py re-checks it on the device.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// The method with its 2^(i/32) table read through tab(i) (u64 bit patterns).
template <class Tab>
__device__ __forceinline__ float glibc_expf_core(float x, Tab tab) {
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                          // |x| >= 88 or x is nan/inf
        if (ux == 0xff800000u) return 0.0f;           // exp(-inf) = 0
        if (abstop >= 0x7f8u) return x + x;           // +inf or nan
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;          // underflow to +0
    }
    const double invln2n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = static_cast<double>(x);
    const double z = invln2n * xd;
    double kd = z + shift;
    const uint64_t ki = static_cast<uint64_t>(__double_as_longlong(kd));
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);
    uint64_t t = tab(static_cast<uint32_t>(ki % 32));
    t += ki << 47;
    const double s = __longlong_as_double(static_cast<long long>(t));
    const double zz = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
    y = y * s;
    return static_cast<float>(y);
}
__device__ __forceinline__ float glibc_expf(float x) {
    return glibc_expf_core(x, [](uint32_t i) { return kExp2Tab[i]; });
}
// The same with the table copied into LDS (a per-lane table index reads LDS
// instead of issuing a memory load).
__device__ __forceinline__ float glibc_expf_lds(float x, const uint64_t* tab) {
    return glibc_expf_core(x, [tab](uint32_t i) { return tab[i]; });
}

// ---- LDS ----------------------------------------------------------------------
// Base of the workgroup's dynamic LDS.  Every LDS structure is addressed from
// here at a fixed offset, so no LDS pointer is ever stored in memory and the
// compiler always sees LDS accesses (ds_*) rather than generic ones.
__device__ __forceinline__ unsigned char* lds_base() {
    HIP_DYNAMIC_SHARED(unsigned char, tsm_lds)
    return tsm_lds;
}

// Row data read by the re-read passes: a pointer in the global address space
// gives global loads (vector memory counter only) where a generic pointer
// would give flat loads, which also wait on LDS traffic.
#ifndef TSM_GLOBAL_AS
#define TSM_GLOBAL_AS __attribute__((address_space(1)))
#endif
template <class T>
__device__ __forceinline__ const TSM_GLOBAL_AS T* global_as(const T* p) {
    return (const TSM_GLOBAL_AS T*)p;
}

// A 16-byte load (one dwordx4) through a global-address-space pointer p,
// 16-byte aligned.
#ifndef TSM_HAVE_LOAD4
typedef float tsm_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load4(const TSM_GLOBAL_AS float* p) {
    const tsm_v4f v = *reinterpret_cast<const TSM_GLOBAL_AS tsm_v4f*>(p);
    return make_float4(v.x, v.y, v.z, v.w);
}
#endif

// Memory the kernel only reads, at addresses uniform over the workgroup (the
// row's parameters, history offsets and uniform): loads through the constant
// address space become scalar loads, which count on their own counter, so
// waiting for them does not wait for the vector loads already in flight.
#ifndef TSM_CONST_AS
#define TSM_CONST_AS __attribute__((address_space(4)))
#endif
template <class T>
__device__ __forceinline__ const TSM_CONST_AS T* const_as(const T* p) {
    return (const TSM_CONST_AS T*)p;
}

// ---- wave / block primitives (wave64) -----------------------------------------
__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
// Inclusive prefix sum over the wave with DPP row shifts and row broadcasts
// (row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast 15 and 31
// carry the row totals across rows); no LDS traffic.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));
    return v;
}

// Reductions over the wave with DPP moves (row_shr 1, 2, 4, 8 inside each
// 16-lane row, then row_bcast 15 and 31 across rows), the pattern of
// wave_incl_scan: lane 63 ends with the whole wave's result, which is then
// broadcast.  A few VALU cycles per step, against a round trip through the LDS
// crossbar for each step of a shuffle butterfly.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v, uint32_t old) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), kCtrl, kRowMask, 0xf, false));
}
template <class Op>
__device__ __forceinline__ uint32_t dpp_reduce32(uint32_t v, uint32_t idty, Op op) {
    v = op(v, dpp_mov<0x111, 0xf>(v, idty));
    v = op(v, dpp_mov<0x112, 0xf>(v, idty));
    v = op(v, dpp_mov<0x114, 0xf>(v, idty));
    v = op(v, dpp_mov<0x118, 0xf>(v, idty));
    v = op(v, dpp_mov<0x142, 0xa>(v, idty));
    v = op(v, dpp_mov<0x143, 0xc>(v, idty));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}
template <class Op>
__device__ __forceinline__ uint64_t dpp_reduce64(uint64_t v, uint64_t idty, Op op) {
    auto step = [&](auto mov) {
        const uint32_t lo = mov(static_cast<uint32_t>(v), static_cast<uint32_t>(idty));
        const uint32_t hi = mov(static_cast<uint32_t>(v >> 32), static_cast<uint32_t>(idty >> 32));
        v = op(v, (static_cast<uint64_t>(hi) << 32) | lo);
    };
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x111, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x112, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x114, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x118, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x142, 0xa>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x143, 0xc>(x, o); });
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), 63));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), 63));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t wave_sum_dpp(uint32_t v) {
    return dpp_reduce32(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    return __uint_as_float(dpp_reduce32(__float_as_uint(v), __float_as_uint(-INFINITY), [](uint32_t a, uint32_t b) {
        return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
}
__device__ __forceinline__ uint64_t wave_min_u64_dpp(uint64_t v) {
    return dpp_reduce64(v, ~0ull, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
    return dpp_reduce64(v, 0ull, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
// Reductions over the first 16 lanes (one DPP row): row_shr 1, 2, 4, 8, then
// lane 15 holds the result.  Used to combine per-wave partials that lanes
// 0..15 have read from LDS in one round trip.
template <class Op>
__device__ __forceinline__ uint32_t dpp_reduce16(uint32_t v, uint32_t idty, Op op) {
    v = op(v, dpp_mov<0x111, 0xf>(v, idty));
    v = op(v, dpp_mov<0x112, 0xf>(v, idty));
    v = op(v, dpp_mov<0x114, 0xf>(v, idty));
    v = op(v, dpp_mov<0x118, 0xf>(v, idty));
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 15));
}
template <class Op>
__device__ __forceinline__ uint64_t dpp_reduce16_64(uint64_t v, uint64_t idty, Op op) {
    auto step = [&](auto mov) {
        const uint32_t lo = mov(static_cast<uint32_t>(v), static_cast<uint32_t>(idty));
        const uint32_t hi = mov(static_cast<uint32_t>(v >> 32), static_cast<uint32_t>(idty >> 32));
        v = op(v, (static_cast<uint64_t>(hi) << 32) | lo);
    };
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x111, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x112, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x114, 0xf>(x, o); });
    step([](uint32_t x, uint32_t o) { return dpp_mov<0x118, 0xf>(x, o); });
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), 15));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), 15));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t row_sum16(uint32_t v) {
    return dpp_reduce16(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ uint32_t row_min16(uint32_t v) {
    return dpp_reduce16(v, ~0u, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t row_max16(uint32_t v) {
    return dpp_reduce16(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint64_t row_min16_u64(uint64_t v) {
    return dpp_reduce16_64(v, ~0ull, [](uint64_t a, uint64_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint64_t row_max16_u64(uint64_t v) {
    return dpp_reduce16_64(v, 0ull, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ float wave_max(float v) { return wave_max_dpp(v); }
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) { return wave_sum_dpp(v); }
__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
    return dpp_reduce32(v, ~0u, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    return dpp_reduce32(v, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ double wave_sum_f64_dpp(double v) {
    return __longlong_as_double(static_cast<long long>(dpp_reduce64(
        static_cast<uint64_t>(__double_as_longlong(v)), 0ull, [](uint64_t a, uint64_t b) {
            return static_cast<uint64_t>(__double_as_longlong(__longlong_as_double(static_cast<long long>(a)) +
                                                              __longlong_as_double(static_cast<long long>(b))));
        })));
}

// Value of `v` in lane `lane` (uniform), as a scalar broadcast.
__device__ __forceinline__ uint32_t wave_read(uint32_t v, uint32_t lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(lane)));
}
// A value every active lane holds alike, moved to a scalar register.
__device__ __forceinline__ uint32_t wave_uniform(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}
// Mask of the lanes whose predicate holds (bit i = lane i).
__device__ __forceinline__ uint64_t wave_ballot(bool p) { return static_cast<uint64_t>(__ballot(p)); }
// Number of lanes below this one whose bit is set in `mask`.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}
// Load of an LDS word that other waves update with atomics meanwhile.
__device__ __forceinline__ uint32_t lds_load_relaxed(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Publishing a count of records written to LDS: every lane fences its LDS
// writes and then raises the count (read-modify-write, so the updates of all
// lanes form one release sequence); a reader loads the count and fences
// before reading the records.  The fences order LDS operations only
// ("local"), so neither side waits for the wave's global loads in flight, as
// a plain release / acquire at workgroup scope would (it orders global
// memory too).
__device__ __forceinline__ void lds_publish_max(uint32_t* p, uint32_t v) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint32_t lds_load_acquire(uint32_t* p) {
    const uint32_t v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return v;
}

// Workgroup barrier for LDS communication.  Every exchange between the
// threads of a workgroup in these kernels goes through LDS (global memory is
// only read, or written for the host), so the barrier fences LDS alone: a
// __syncthreads() would also wait for every global load in flight, which
// stalls the row's prefetched tiles at each barrier.
#define TSM_LDS_SYNC()                                                   \
    do {                                                                 \
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  \
        __builtin_amdgcn_s_barrier();                                    \
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");  \
    } while (0)

// Exclusive prefix sum over the block; `tmp` holds >= nwaves+1 words of LDS.
// Returns the prefix; *total gets the block sum.  Contains two barriers.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* tmp, uint32_t* total) {
    constexpr int NW = NT / kWave;
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    static_assert(NW <= 16, "one DPP row combines the waves");
    uint32_t inc = wave_incl_scan(v);
    if (lane == kWave - 1) tmp[wid] = inc;
    TSM_LDS_SYNC();
    // lanes 0..NW-1 read the waves' totals in one round trip
    const uint32_t t = lane < NW ? tmp[lane] : 0u;
    const uint32_t before = row_sum16(lane < wid ? t : 0u), all = row_sum16(t);
    TSM_LDS_SYNC();
    *total = all;
    return before + inc - v;
}

template <int NT>
__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t* tmp) {
    constexpr int NW = NT / kWave;
    static_assert(NW <= 16, "one DPP row combines the waves");
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) tmp[threadIdx.x / kWave] = v;
    TSM_LDS_SYNC();
    const uint32_t all = row_sum16(lane_id() < NW ? tmp[lane_id()] : 0u);
    TSM_LDS_SYNC();
    return all;
}

template <int NT>
__device__ __forceinline__ uint32_t block_min(uint32_t v, uint32_t* tmp) {
    constexpr int NW = NT / kWave;
    static_assert(NW <= 16, "one DPP row combines the waves");
    v = wave_min(v);
    if ((threadIdx.x & (kWave - 1)) == 0) tmp[threadIdx.x / kWave] = v;
    TSM_LDS_SYNC();
    const uint32_t all = row_min16(lane_id() < NW ? tmp[lane_id()] : 0xFFFFFFFFu);
    TSM_LDS_SYNC();
    return all;
}

// Finds, in a histogram of kBins counts laid out by ascending digit, the
// first digit whose inclusive cumulative count reaches `need` (>= 1).
// Writes {digit, count strictly before it} to out[0..1]; leaves out untouched
// when the total is below `need`.  Block of NT threads, NT * per == kBins.
template <int NT>
__device__ __forceinline__ void hist_find(const uint32_t* hist, uint32_t need, uint32_t* tmp,
                                          uint32_t* out) {
    constexpr int per = kBins / NT;
    const int t = threadIdx.x;
    uint32_t c[per];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < per; i++) {
        c[i] = hist[t * per + i];
        sum += c[i];
    }
    uint32_t total;
    uint32_t before = block_excl_scan<NT>(sum, tmp, &total);
    if (before < need && before + sum >= need) {
        uint32_t run = before;
#pragma unroll
        for (int i = 0; i < per; i++) {
            if (run + c[i] >= need) {
                out[0] = t * per + i;
                out[1] = run;
                break;
            }
            run += c[i];
        }
    }
    TSM_LDS_SYNC();
}

}  // namespace tsm
