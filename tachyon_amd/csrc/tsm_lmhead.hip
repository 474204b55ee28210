// tsm_lmhead.hip - the logits producer: Tachyon's output layer on the GPU.
//
// For each logit row r the reference computes xb = rmsnorm(x[r]) in f32
// (model.rs:702-709 over kernels.rs:522-528) and then logits[r][v] =
// dot_bf16(W[v], xb) over the bf16 lm_head matrix W [vocab, dim]
// (model.rs:711-715, weights.rs:230-239, kernels.rs:1411-1413).  Here:
//
//   lm_prep_kernel  one workgroup per row: the rmsnorm in f32, then the row
//                   as bf16 MFMA operands in the caller's workspace: hi =
//                   bf16(xb), and with TSM_LM_SPLIT also lo = bf16(xb - hi),
//                   so that hi + lo carries xb to within 2^-17 of itself and
//                   the products with bf16 weights stay exact in f32.  Rows
//                   past `rows` up to the tile are zero.
//   lm_gemm_kernel  logits = A W^T on v_mfma_f32_16x16x32_bf16.  A workgroup
//                   (4 waves) owns 256 rows x 128 vocab ids; wave w the rows
//                   64w..64w+63 (4 x 8 MFMA tiles of 16 x 16, 128 f32
//                   accumulators per lane).  The weight tile of each k-step
//                   (128 ids x 64 k, 16 KB) is loaded cooperatively four
//                   steps ahead into a register ring (4 x 16 B per thread
//                   per step), written to one of two LDS buffers the step
//                   before it is used, and read back as MFMA fragments by
//                   every wave; one barrier per step.  A's fragments (the
//                   workspace, 2-4 MB, resident in L2) are loaded by each
//                   wave straight into registers one step ahead.
//
// Both operands are contiguous along k (A's rows, W's rows), so every MFMA
// fragment (8 consecutive k of one row) is one 16-byte load.
#include <cstdarg>
#include <cstdio>
#include <type_traits>

#include <hip/hip_runtime.h>

#include "tachyon_sampler.h"

namespace tsm {
namespace lm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 raw bytes

constexpr uint32_t kThreads = 256;            // 4 waves
constexpr uint32_t kTileM = 256;              // rows per workgroup (64 per wave)
constexpr uint32_t kTileN = 128;              // vocab ids per workgroup
constexpr uint32_t kStepK = 64;               // k per step: two MFMA k-halves of 32
constexpr uint32_t kRing = 4;                 // weight steps in flight per thread
constexpr uint32_t kRowB = kStepK * 2 + 16;   // LDS bytes per weight row (16 B pad: no bank conflicts)
constexpr uint32_t kBufB = kTileN * kRowB;    // one LDS weight buffer (18,432 B)
constexpr uint32_t kChunks = kTileN * kStepK * 2 / 16 / kThreads;  // 16-byte weight chunks per thread per step
static_assert(kChunks == 4, "weight tile split");

struct PrepArgs {
    const float* x;
    const float* norm_w;
    uint16_t* ahi;
    uint16_t* alo;  // null unless split
    float eps;
    uint32_t rows, rows_pad, dim, x_stride;
};

struct GemmArgs {
    const uint16_t* ahi;
    const uint16_t* alo;  // null unless split
    const uint16_t* w;
    float* logits;
    uint32_t rows, dim, vocab, ld;
};

// f32 -> bf16, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// One workgroup per (padded) row: the rmsnorm of kernels.rs:522-528,
// ss = (sum of x^2) / dim, inv = 1 / sqrt(ss + eps), out = x * inv * g, all
// in f32 (the sum in tree order rather than the reference's left fold).
__global__ __launch_bounds__(kThreads) void lm_prep_kernel(PrepArgs a) {
    __shared__ float part[kThreads / 64];
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    uint16_t* hi = a.ahi + static_cast<size_t>(r) * a.dim;
    uint16_t* lo = a.alo ? a.alo + static_cast<size_t>(r) * a.dim : nullptr;
    if (r >= a.rows) {  // padding rows of the last tile
        for (uint32_t k = tid; k < a.dim; k += kThreads) {
            hi[k] = 0;
            if (lo) lo[k] = 0;
        }
        return;
    }
    const float* x = a.x + static_cast<size_t>(r) * a.x_stride;
    float s = 0.0f;
    for (uint32_t k = tid; k < a.dim; k += kThreads) s += x[k] * x[k];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((tid & 63u) == 0) part[tid >> 6] = s;
    __syncthreads();
    const float ss = ((part[0] + part[1]) + (part[2] + part[3])) / static_cast<float>(a.dim);
    const float inv = 1.0f / sqrtf(ss + a.eps);
    for (uint32_t k = tid; k < a.dim; k += kThreads) {
        const float o = x[k] * inv * a.norm_w[k];
        const uint16_t h = bf16_rne(o);
        hi[k] = h;
        if (lo) lo[k] = bf16_rne(o - bf16_f32(h));
    }
}

__device__ __forceinline__ bf16x8 frag(const uint16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
}

// Workgroup (blockIdx.x: 128 vocab ids, blockIdx.y: 256 rows).  A holds
// gridDim.y * 256 rows (the padding zero), so its loads need no bounds; the
// weight rows past `vocab` are clamped to the last one and their results are
// not stored.
template <bool kSplit>
__global__ __launch_bounds__(kThreads) void lm_gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) uint8_t lds[2 * kBufB];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * kTileN;
    const uint32_t m0 = blockIdx.y * kTileM + wave * 64u;
    const uint32_t dim = a.dim, nsteps = dim / kStepK;

    // this thread's weight chunks: rows (tid >> 3) + 32 i, k offset 8 * (tid & 7)
    const uint16_t* wp[kChunks];
    uint32_t woff[kChunks];
#pragma unroll
    for (uint32_t i = 0; i < kChunks; i++) {
        const uint32_t row = (tid >> 3) + 32u * i;
        const uint32_t v = min(n0 + row, a.vocab - 1u);
        wp[i] = a.w + static_cast<size_t>(v) * dim + 8u * (tid & 7u);
        woff[i] = row * kRowB + 16u * (tid & 7u);
    }
    // this lane's A fragments: rows m0 + 16 i + (lane & 15), k offset 8 * (lane >> 4)
    const size_t aoff = static_cast<size_t>(m0 + (lane & 15u)) * dim + 8u * (lane >> 4);
    const uint16_t* ah = a.ahi + aoff;
    const uint16_t* al = kSplit ? a.alo + aoff : nullptr;
    // this lane's weight fragments in LDS: row 16 j + (lane & 15), bytes 16 * (lane >> 4)
    const uint32_t foff = (lane & 15u) * kRowB + 16u * (lane >> 4);

    u32x4 ring[kRing][kChunks];
    auto issue = [&](uint32_t s, u32x4 (&dst)[kChunks]) __attribute__((always_inline)) {
        const uint32_t k0 = s * kStepK;
#pragma unroll
        for (uint32_t i = 0; i < kChunks; i++) dst[i] = *reinterpret_cast<const u32x4*>(wp[i] + k0);
    };
    auto stage = [&](const u32x4 (&src)[kChunks], uint32_t buf) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < kChunks; i++) *reinterpret_cast<u32x4*>(lds + buf * kBufB + woff[i]) = src[i];
    };
    bf16x8 ahf[2][4][2], alf[2][4][2];
    auto load_a = [&](uint32_t s, uint32_t set) __attribute__((always_inline)) {
        const uint32_t k0 = s * kStepK;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const size_t o = static_cast<size_t>(16u * i) * dim + k0 + 32u * h;
                ahf[set][i][h] = frag(ah + o);
                if (kSplit) alf[set][i][h] = frag(al + o);
            }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One k-step s = s0 + Q (Q a compile-time ring slot, so that every
    // register array is indexed by constants): stage step s + 1, fetch A of
    // step s + 1, put step s + kRing in flight, then the MFMAs of step s.
    // The loads and stores are unconditional (a step past the last one reads
    // the last one again, into a buffer no step reads), so that no two paths
    // meet with different ring slots: the ring then stays in registers.
    auto body = [&](uint32_t s0, auto qc) __attribute__((always_inline)) {
        constexpr uint32_t Q = decltype(qc)::value;
        const uint32_t s = s0 + Q;
        // every wave is done with buffer (s + 1) & 1 (step s - 1) and sees
        // step s in buffer s & 1
        __syncthreads();
        stage(ring[(Q + 1u) % kRing], (s + 1u) & 1u);
        load_a(min(s + 1u, nsteps - 1u), (Q + 1u) & 1u);
        issue(min(s + kRing, nsteps - 1u), ring[Q]);
        if (s >= nsteps) return;
        const uint8_t* wb = lds + (s & 1u) * kBufB + foff;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            bf16x8 wf[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
                wf[j] = *reinterpret_cast<const bf16x8*>(wb + j * 16u * kRowB + 64u * h);
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
#pragma unroll
                for (uint32_t j = 0; j < 8; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahf[Q & 1u][i][h], wf[j], acc[i][j], 0, 0, 0);
                    if (kSplit)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alf[Q & 1u][i][h], wf[j], acc[i][j], 0, 0, 0);
                }
        }
    };
    using C0 = std::integral_constant<uint32_t, 0>;
    using C1 = std::integral_constant<uint32_t, 1>;
    using C2 = std::integral_constant<uint32_t, 2>;
    using C3 = std::integral_constant<uint32_t, 3>;
    static_assert(kRing == 4, "the ring slots below");

    // prologue: steps 0 .. kRing - 1 in flight, step 0 staged, A of step 0 loaded
    issue(0, ring[0]);
    issue(min(1u, nsteps - 1u), ring[1]);
    issue(min(2u, nsteps - 1u), ring[2]);
    issue(min(3u, nsteps - 1u), ring[3]);
    stage(ring[0], 0);
    load_a(0, 0);
    for (uint32_t s0 = 0; s0 < nsteps; s0 += kRing) {
        body(s0, C0{});
        body(s0, C1{});
        body(s0, C2{});
        body(s0, C3{});
    }

    // lane l holds rows 4 (l >> 4) + e, column l & 15 of each 16 x 16 tile
#pragma unroll
    for (uint32_t i = 0; i < 4; i++)
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) {
            const uint32_t row = m0 + 16u * i + 4u * (lane >> 4) + e;
            if (row >= a.rows) continue;
            float* out = a.logits + static_cast<size_t>(row) * a.ld;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {
                const uint32_t col = n0 + 16u * j + (lane & 15u);
                if (col < a.vocab) out[col] = acc[i][j][e];
            }
        }
}

void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

uint32_t rows_pad(uint32_t rows) { return (rows + kTileM - 1u) / kTileM * kTileM; }

}  // namespace lm
}  // namespace tsm

extern "C" {

size_t tsm_lm_head_workspace(uint32_t rows, uint32_t dim, uint32_t flags) {
    const size_t copies = (flags & TSM_LM_SPLIT) ? 2u : 1u;
    return static_cast<size_t>(tsm::lm::rows_pad(rows)) * dim * 2u * copies;
}

int tsm_lm_head(void* stream, const float* x, uint32_t x_stride, const float* norm_w, float eps,
                const uint16_t* w, uint32_t rows, uint32_t dim, uint32_t vocab, uint32_t flags, void* workspace,
                size_t workspace_bytes, float* logits, uint32_t ld, char* err, size_t errlen) {
    using tsm::lm::set_err;
    if (flags & ~static_cast<uint32_t>(TSM_LM_SPLIT)) return set_err(err, errlen, "unknown flags 0x%x", flags), 1;
    if (rows == 0 || rows > TSM_LM_MAX_ROWS)
        return set_err(err, errlen, "rows %u is outside [1, %u]", rows, TSM_LM_MAX_ROWS), 1;
    if (dim == 0 || dim % tsm::lm::kStepK != 0 || dim > TSM_LM_MAX_DIM)
        return set_err(err, errlen, "dim %u must be a positive multiple of %u, at most %u", dim, tsm::lm::kStepK,
                       TSM_LM_MAX_DIM), 1;
    if (vocab == 0 || vocab > TSM_MAX_VOCAB)
        return set_err(err, errlen, "vocab %u is outside [1, %u]", vocab, TSM_MAX_VOCAB), 1;
    if (!x || !norm_w || !w || !logits || !workspace)
        return set_err(err, errlen, "x, norm_w, w, workspace and logits must be set"), 1;
    if (x_stride < dim) return set_err(err, errlen, "x_stride %u is below dim %u", x_stride, dim), 1;
    if (ld < vocab) return set_err(err, errlen, "ld %u is below vocab %u", ld, vocab), 1;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(workspace) & 15u))
        return set_err(err, errlen, "w and workspace must be 16-byte aligned"), 1;
    const size_t need = tsm_lm_head_workspace(rows, dim, flags);
    if (workspace_bytes < need)
        return set_err(err, errlen, "workspace holds %zu bytes; %zu needed", workspace_bytes, need), 1;
    const bool split = (flags & TSM_LM_SPLIT) != 0;
    const uint32_t rp = tsm::lm::rows_pad(rows);
    uint16_t* ahi = static_cast<uint16_t*>(workspace);
    uint16_t* alo = split ? ahi + static_cast<size_t>(rp) * dim : nullptr;
    const hipStream_t st = static_cast<hipStream_t>(stream);

    tsm::lm::PrepArgs p;
    p.x = x;
    p.norm_w = norm_w;
    p.ahi = ahi;
    p.alo = alo;
    p.eps = eps;
    p.rows = rows;
    p.rows_pad = rp;
    p.dim = dim;
    p.x_stride = x_stride;
    hipLaunchKernelGGL(tsm::lm::lm_prep_kernel, dim3(rp), dim3(tsm::lm::kThreads), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "prep launch failed: %s", hipGetErrorString(e)), 1;

    tsm::lm::GemmArgs g;
    g.ahi = ahi;
    g.alo = alo;
    g.w = w;
    g.logits = logits;
    g.rows = rows;
    g.dim = dim;
    g.vocab = vocab;
    g.ld = ld;
    const dim3 grid((vocab + tsm::lm::kTileN - 1u) / tsm::lm::kTileN, rp / tsm::lm::kTileM);
    if (split) hipLaunchKernelGGL(tsm::lm::lm_gemm_kernel<true>, grid, dim3(tsm::lm::kThreads), 0, st, g);
    else hipLaunchKernelGGL(tsm::lm::lm_gemm_kernel<false>, grid, dim3(tsm::lm::kThreads), 0, st, g);
    e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "gemm launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

}  // extern "C"
