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
//                   the products with bf16 weights stay exact in f32.  The
//                   operands are stored in MFMA fragment order (frag_pos), so
//                   that a wave's fragment load is 1 KB in one piece; rows
//                   past `rows` up to the tile are zero.
//   lm_gemm_kernel  logits = A W^T on v_mfma_f32_16x16x32_bf16.  A workgroup
//                   (8 waves, two per SIMD) owns R rows x 128 vocab ids, R
//                   the smallest of 32, 64, 128, 256 that holds the batch
//                   (Tile); each wave owns 32 rows and 128 / (8 / (R / 32))
//                   ids (at R = 256: 2 x 8 MFMA tiles of 16 x 16, 64 f32
//                   accumulators per lane).  The weight tile of each
//                   k-step (128 ids x 64 k, 16 KB) is loaded cooperatively
//                   four steps ahead into a register ring (2 x 16 B per thread
//                   per step), staged into one of three LDS buffers two steps
//                   before it is used, and read back as MFMA fragments by
//                   every wave half a step ahead of its MFMAs; one barrier per
//                   step.  A's fragments (the workspace, 2-4 MB, resident in
//                   L2) are loaded by each wave straight into registers one
//                   step ahead.
//
// Measured at 256 rows x dim 4096 x vocab 151,936 (MI355X): about 470 us
// (bf16 activations) and 690 us (split), against 175 us for the bytes at
// 8 TB/s; one row (decoding) about 270 us.
// One wave per SIMD issues these MFMAs at about half the peak rate (a
// microbenchmark of independent MFMAs: 52% with one wave, 76% with two),
// hence the 8-wave workgroup; the loads of both operands, the LDS reads and
// the barrier each add to the step time (variants with each switched off).
//
// Both operands are contiguous along k (A's rows, W's rows), so every MFMA
// fragment (8 consecutive k of one row) is one 16-byte load.
#include <cstdarg>
#include <cstdio>
#include <type_traits>
#include <utility>

#include <hip/hip_runtime.h>

#include "tachyon_sampler.h"

namespace tsm {
namespace lm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 raw bytes

constexpr uint32_t kPrepThreads = 256;  // the prep kernel: 4 waves per row
constexpr uint32_t kPrepChunks = 16;    // 8-value chunks per prep thread: dim up to 32768

constexpr uint32_t kTileN = 128;              // vocab ids per workgroup
constexpr uint32_t kStepK = 64;               // k per step: two MFMA k-halves of 32
constexpr uint32_t kRing = 4;                 // weight steps in flight per thread
constexpr uint32_t kASets = 2;                // A steps held per wave (the one in use and the next)
constexpr uint32_t kRowB = kStepK * 2 + 16;   // LDS bytes per weight row (16 B pad: no bank conflicts)
constexpr uint32_t kBufB = kTileN * kRowB;    // one LDS weight buffer (18,432 B)
static_assert(kRing % kASets == 0, "A sets follow the ring slots");
static_assert(kRing >= 3, "a step is staged two steps ahead");

// A workgroup's shape: TM rows x kTileN ids, WM waves along the rows and WN
// along the vocabulary (8 waves, two per SIMD).
template <uint32_t TM, uint32_t WM, uint32_t WN>
struct Tile {
    static constexpr uint32_t kTileM = TM, kWavesM = WM, kWavesN = WN;
    static constexpr uint32_t kThreads = 64 * WM * WN;
    static constexpr uint32_t kRowsW = TM / WM;                // rows per wave
    static constexpr uint32_t kMBlk = kRowsW / 16;             // 16-row MFMA blocks per wave
    static constexpr uint32_t kNBlk = kTileN / WN / 16;        // 16-id MFMA blocks per wave
    static constexpr uint32_t kChunks = kTileN * kStepK * 2 / 16 / kThreads;  // 16-byte weight chunks per thread per step
    static_assert(kChunks * kThreads * 16 == kTileN * kStepK * 2, "weight tile split");
    static_assert(kMBlk >= 1 && kNBlk >= 1 && kRowsW % 16 == 0, "whole MFMA blocks");
};
// Every shape but the smallest gives a wave 32 rows; fewer rows per
// workgroup spread the waves along the vocabulary instead, so that a small
// batch does not pay for a 256-row tile's MFMA work.
using Tile256 = Tile<256, 8, 1>;  // a wave owns 32 rows x 128 ids
using Tile128 = Tile<128, 4, 2>;  // 32 rows x 64 ids
using Tile64 = Tile<64, 2, 4>;    // 32 rows x 32 ids
using Tile32 = Tile<32, 1, 8>;    // 32 rows x 16 ids
using Tile16 = Tile<16, 1, 8>;    // 16 rows x 16 ids (decoding)

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

// The operands' layout in the workspace: MFMA fragment order.  The 16 x 32
// block (rows 16 rb.., k 32 kc..) is 1 KB, lane l's 8 values (row 16 rb +
// (l & 15), k 32 kc + 8 (l >> 4) ..) at bytes 16 l, and the blocks of one
// row block follow each other along k; so a wave's fragment load reads 1 KB
// in one piece.  frag_pos is the element offset of (row, k), k a multiple of 8.
__device__ __forceinline__ size_t frag_pos(uint32_t row, uint32_t k, uint32_t dim) {
    const uint32_t lane = (row & 15u) + 16u * ((k >> 3) & 3u);
    return ((static_cast<size_t>(row >> 4) * (dim >> 5) + (k >> 5)) * 64u + lane) * 8u;
}

// One workgroup per (padded) row: the rmsnorm of kernels.rs:522-528,
// ss = (sum of x^2) / dim, inv = 1 / sqrt(ss + eps), out = x * inv * g, all
// in f32 (the sum in tree order rather than the reference's left fold).
__global__ __launch_bounds__(kPrepThreads) void lm_prep_kernel(PrepArgs a) {
    __shared__ float part[kPrepThreads / 64];
    static_assert(kPrepThreads == 256, "the reduction below sums four wave partials");
    static_assert(kPrepThreads * kPrepChunks * 8 >= TSM_LM_MAX_DIM, "a row fits the threads' chunks");
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    const uint32_t nchunk = a.dim / 8u;  // 8 consecutive k per chunk: one lane's fragment
    if (r >= a.rows) {  // padding rows of the last tile
        const u32x4 z = {0u, 0u, 0u, 0u};
        for (uint32_t c = tid; c < nchunk; c += kPrepThreads) {
            *reinterpret_cast<u32x4*>(a.ahi + frag_pos(r, 8u * c, a.dim)) = z;
            if (a.alo) *reinterpret_cast<u32x4*>(a.alo + frag_pos(r, 8u * c, a.dim)) = z;
        }
        return;
    }
    // the row is read once: each thread keeps its chunks (8 values each, at
    // most kPrepChunks) in registers between the sum of squares and the
    // normalization
    const float* x = a.x + static_cast<size_t>(r) * a.x_stride;
    f32x4 v[kPrepChunks][2];
    float s = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kPrepChunks; j++) {
        const uint32_t c = tid + j * kPrepThreads;
        if (c < nchunk) {
            // x rows are 16-byte aligned only when x_stride and the base are; read by element
#pragma unroll
            for (uint32_t e = 0; e < 4; e++) {
                v[j][0][e] = x[8u * c + e];
                v[j][1][e] = x[8u * c + 4u + e];
            }
#pragma unroll
            for (uint32_t e = 0; e < 4; e++) s += v[j][0][e] * v[j][0][e];
#pragma unroll
            for (uint32_t e = 0; e < 4; e++) s += v[j][1][e] * v[j][1][e];
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((tid & 63u) == 0) part[tid >> 6] = s;
    __syncthreads();
    const float ss = ((part[0] + part[1]) + (part[2] + part[3])) / static_cast<float>(a.dim);
    const float inv = 1.0f / sqrtf(ss + a.eps);
#pragma unroll
    for (uint32_t j = 0; j < kPrepChunks; j++) {
        const uint32_t c = tid + j * kPrepThreads;
        if (c >= nchunk) continue;
        uint32_t hw[4], lw[4];
#pragma unroll
        for (uint32_t e = 0; e < 8; e += 2) {
            const uint32_t k = 8u * c + e;
            const float o0 = v[j][e >> 2][e & 3u] * inv * a.norm_w[k];
            const float o1 = v[j][e >> 2][(e & 3u) + 1u] * inv * a.norm_w[k + 1u];
            const uint16_t h0 = bf16_rne(o0), h1 = bf16_rne(o1);
            hw[e / 2] = static_cast<uint32_t>(h0) | (static_cast<uint32_t>(h1) << 16);
            lw[e / 2] = static_cast<uint32_t>(bf16_rne(o0 - bf16_f32(h0))) |
                        (static_cast<uint32_t>(bf16_rne(o1 - bf16_f32(h1))) << 16);
        }
        const size_t pos = frag_pos(r, 8u * c, a.dim);
        *reinterpret_cast<u32x4*>(a.ahi + pos) = u32x4{hw[0], hw[1], hw[2], hw[3]};
        if (a.alo) *reinterpret_cast<u32x4*>(a.alo + pos) = u32x4{lw[0], lw[1], lw[2], lw[3]};
    }
}

// Calls f(std::integral_constant<uint32_t, Q>) for Q = 0 .. N-1 in order:
// register arrays indexed by Q are then indexed by constants.
template <uint32_t N, class F, uint32_t... Q>
__device__ __forceinline__ void each_slot_(F&& f, std::integer_sequence<uint32_t, Q...>) {
    (f(std::integral_constant<uint32_t, Q>{}), ...);
}
template <uint32_t N, class F>
__device__ __forceinline__ void each_slot(F&& f) {
    each_slot_<N>(f, std::make_integer_sequence<uint32_t, N>{});
}

__device__ __forceinline__ bf16x8 frag(const uint16_t* p) {
    return *reinterpret_cast<const bf16x8*>(p);
}

// Workgroup (blockIdx.x: 128 vocab ids, blockIdx.y: 256 rows).  A holds
// gridDim.y * 256 rows (the padding zero), so its loads need no bounds; the
// weight rows past `vocab` are clamped to the last one and their results are
// not stored.
template <bool kSplit, class T>
__global__ __launch_bounds__(T::kThreads) void lm_gemm_kernel(GemmArgs a) {
    constexpr uint32_t kTileM = T::kTileM, kWavesM = T::kWavesM, kWavesN = T::kWavesN, kThreads = T::kThreads;
    constexpr uint32_t kRowsW = T::kRowsW, kMBlk = T::kMBlk, kNBlk = T::kNBlk, kChunks = T::kChunks;
    __shared__ __align__(16) uint8_t lds[3 * kBufB];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * kTileN;
    const uint32_t wn0 = (wave / kWavesM) * (kTileN / kWavesN);  // this wave's first id in the tile
    const uint32_t m0 = blockIdx.y * kTileM + (wave % kWavesM) * kRowsW;
    const uint32_t dim = a.dim, nsteps = dim / kStepK;

    // this thread's weight chunks: rows (tid >> 3) + (kThreads / 8) i, k offset 8 * (tid & 7)
    const uint16_t* wp[kChunks];
    uint32_t woff[kChunks];
#pragma unroll
    for (uint32_t i = 0; i < kChunks; i++) {
        const uint32_t row = (tid >> 3) + (kThreads / 8u) * i;
        const uint32_t v = min(n0 + row, a.vocab - 1u);
        wp[i] = a.w + static_cast<size_t>(v) * dim + 8u * (tid & 7u);
        woff[i] = row * kRowB + 16u * (tid & 7u);
    }
    // this lane's A fragments: rows m0 + 16 i + (lane & 15), k offset 8 * (lane >> 4)
    const size_t aoff = static_cast<size_t>(m0 >> 4) * (dim >> 5) * 512u + 8u * lane;
    const uint16_t* ah = a.ahi + aoff;
    const uint16_t* al = kSplit ? a.alo + aoff : nullptr;
    // this lane's weight fragments in LDS: row 16 j + (lane & 15), bytes 16 * (lane >> 4)
    const uint32_t foff = (wn0 + (lane & 15u)) * kRowB + 16u * (lane >> 4);

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
    bf16x8 ahf[kASets][kMBlk][2], alf[kASets][kMBlk][2];
    auto load_a = [&](uint32_t s, uint32_t set) __attribute__((always_inline)) {
        const uint32_t k0 = s * kStepK;
#pragma unroll
        for (uint32_t i = 0; i < kMBlk; i++)
#pragma unroll
            for (uint32_t h = 0; h < 2; h++) {
                const size_t o = (static_cast<size_t>(i) * (dim >> 5) + (k0 >> 5) + h) * 512u;
                ahf[set][i][h] = frag(ah + o);
                if (kSplit) alf[set][i][h] = frag(al + o);
            }
    };

    f32x4 acc[kMBlk][kNBlk];
#pragma unroll
    for (uint32_t i = 0; i < kMBlk; i++)
#pragma unroll
        for (uint32_t j = 0; j < kNBlk; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // One k-step s = s0 + Q (Q a compile-time ring slot, so that every
    // register array is indexed by constants): stage step s + 1, fetch A of
    // step s + 1, put step s + kRing in flight, then the MFMAs of step s.
    // Half-step h of step t: the weight fragments (k 32 h .. 32 h + 31 of
    // the tile's 64) from LDS buffer t % 3.
    auto read_w = [&](bf16x8 (&wf)[kNBlk], uint32_t t, uint32_t h) __attribute__((always_inline)) {
        const uint8_t* wb = lds + (t % 3u) * kBufB + foff + 64u * h;
#pragma unroll
        for (uint32_t j = 0; j < kNBlk; j++) wf[j] = *reinterpret_cast<const bf16x8*>(wb + j * 16u * kRowB);
    };
    auto mfmas = [&](const bf16x8 (&wf)[kNBlk], const bf16x8 (&a)[kMBlk][2], uint32_t h) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < kMBlk; i++)
#pragma unroll
            for (uint32_t j = 0; j < kNBlk; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][h], wf[j], acc[i][j], 0, 0, 0);
    };
    bf16x8 wc[kNBlk], wn[kNBlk];  // this half-step's weight fragments and the next one's

    // Step s = s0 + Q (Q a compile-time ring slot, so that every register
    // array is indexed by constants).  Three LDS buffers: step t is staged
    // into buffer t % 3 at step t - 2 and read at steps t - 1 (its first
    // half) and t (its second), so each half-step's LDS reads overlap the
    // MFMAs of the one before.  The loads and stores are unconditional (a
    // step past the last one reads the last one again, into a buffer no
    // MFMA uses), so that no two paths meet with different ring slots: the
    // ring then stays in registers.
    auto body = [&](uint32_t s0, auto qc) __attribute__((always_inline)) {
        constexpr uint32_t Q = decltype(qc)::value;
        const uint32_t s = s0 + Q;
        // every wave is done with buffer (s + 2) % 3 (step s - 1) and sees
        // step s + 1 in buffer (s + 1) % 3
        __syncthreads();
        stage(ring[(Q + 2u) % kRing], (s + 2u) % 3u);
        load_a(min(s + kASets - 1u, nsteps - 1u), (Q + kASets - 1u) % kASets);
        issue(min(s + kRing, nsteps - 1u), ring[Q]);
        read_w(wn, s, 1);
        const bool live = s < nsteps;
        if (live) {
            mfmas(wc, ahf[Q % kASets], 0);
            if (kSplit) mfmas(wc, alf[Q % kASets], 0);
        }
        read_w(wc, s + 1u, 0);
        if (live) {
            mfmas(wn, ahf[Q % kASets], 1);
            if (kSplit) mfmas(wn, alf[Q % kASets], 1);
        }
    };

    // prologue: steps 0 .. kRing - 1 in flight, steps 0 and 1 staged, A of
    // the first kASets - 1 steps loaded, the first half of step 0 read
    each_slot<kRing>([&](auto qc) __attribute__((always_inline)) {
        constexpr uint32_t Q = decltype(qc)::value;
        issue(min(Q, nsteps - 1u), ring[Q]);
    });
    stage(ring[0], 0);
    stage(ring[1], 1);
    each_slot<kASets - 1>([&](auto qc) __attribute__((always_inline)) {
        constexpr uint32_t Q = decltype(qc)::value;
        load_a(min(Q, nsteps - 1u), Q);
    });
    __syncthreads();
    read_w(wc, 0, 0);
    for (uint32_t s0 = 0; s0 < nsteps; s0 += kRing)
        each_slot<kRing>([&](auto qc) __attribute__((always_inline)) { body(s0, qc); });

    // lane l holds rows 4 (l >> 4) + e, column l & 15 of each 16 x 16 tile
#pragma unroll
    for (uint32_t i = 0; i < kMBlk; i++)
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) {
            const uint32_t row = m0 + 16u * i + 4u * (lane >> 4) + e;
            if (row >= a.rows) continue;
            float* out = a.logits + static_cast<size_t>(row) * a.ld;
#pragma unroll
            for (uint32_t j = 0; j < kNBlk; j++) {
                const uint32_t col = n0 + wn0 + 16u * j + (lane & 15u);
                if (col < a.vocab) out[col] = acc[i][j][e];
            }
        }
}

// ---- the Q8 lm_head ------------------------------------------------------------
// Tachyon's Q8 matrices (weights.rs:64-70, llama.cpp's Q8_0): per row, blocks
// of 32 int8 values, each block with an f16 scale.  The reference quantizes
// each activation row per 32-value block too (quantize_input, weights.rs:
// 652-664, over kernels.rs:84-100) and sums the blocks' integer dots, each
// times the weight block's scale and the activation block's scale, in f32
// in block order (the scalar dot_q8_with, kernels.rs:1420-1430).
//
//   lm_q8_prep_kernel  one workgroup per row: the rmsnorm with the sum of
//                      squares as the reference's left fold (the squares
//                      computed by every thread into LDS, then added in order
//                      by one lane), so the normalized values and their
//                      quantization are the reference's own; then the int8
//                      values in MFMA fragment order (q8_frag_pos) and the
//                      block scales (q8_scale_pos), 8 lanes per block.
//   lm_q8_gemm_kernel  the integer block dots on v_mfma_i32_16x16x64_i8, a
//                      pair of blocks (64 bytes of a row) at a time: each
//                      lane loads 16 contiguous weight bytes and 16
//                      activation bytes (lane group g: bytes 16 g .. 16 g +
//                      15 of the pair), and two MFMAs per 16 x 16 tile take
//                      the same weight fragment against the activation
//                      fragment with one block's lane groups (g >> 1 == h)
//                      kept and the other's zeroed, so each MFMA sums
//                      exactly one block's 32 products.  Each block's sum is
//                      converted and scaled in f32 and added in block order,
//                      as the reference does.  The
//                      f32 work (convert, two products, a sum per row, id
//                      and block: 4 VALU operations against 32 MACs on the
//                      matrix cores) bounds the kernel at large batches and
//                      the weight stream at small ones; a wave keeps the
//                      operands of the next kQ8Ring pairs in flight in a
//                      register ring, issued in the order they are used.
//                      Tiles by batch size (Q8Tile): a wave owns RB row
//                      blocks x JB id blocks of 16; WR x WN waves.
constexpr uint32_t kQ8Block = 32;       // values per quantization block
constexpr uint32_t kQ8Threads = 1024;   // prep kernel (one round of the quantization at dim 4096)
constexpr uint32_t kQ8Stage = 4096;     // squares staged per round of the prep's fold
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <uint32_t RB_, uint32_t JB_, uint32_t WR_, uint32_t WN_, uint32_t RING_ = 2>
struct Q8Tile {
    static constexpr uint32_t RB = RB_, JB = JB_, WR = WR_, WN = WN_, kRing = RING_;
    static constexpr uint32_t kRows = 16u * RB * WR, kIds = 16u * JB * WN, kThreads = 64u * WR * WN;
};

struct Q8PrepArgs {
    const float* x;
    const float* norm_w;
    int8_t* aq;
    float* as;
    float eps;
    uint32_t rows, rows_pad, dim, x_stride;
};
struct Q8GemmArgs {
    const int8_t* aq;
    const float* as;
    const int8_t* wq;
    const uint16_t* ws;
    float* logits;
    uint32_t rows, rows_pad, dim, vocab, ld;
};

// Byte offset of value kin (of 0..31) of block b of `row` in the
// activations' fragment order: per 16-row block and pair of blocks (np pairs
// a row) 1 KB, lane (row & 15) + 16 g holding bytes 16 g .. 16 g + 15 of the
// row's pair (block 2p + (g >> 1), values 16 (g & 1) ..), the same place the
// weight fragment holds them.
__device__ __forceinline__ size_t q8_frag_pos(uint32_t row, uint32_t b, uint32_t kin, uint32_t np) {
    const uint32_t g = 2u * (b & 1u) + (kin >> 4);
    return ((static_cast<size_t>(row >> 4) * np + (b >> 1)) * 64u + (row & 15u) + 16u * g) * 16u + (kin & 15u);
}

// Index of row `row`'s scale of block b: per 16-row block and quantization
// block, the 16 rows' scales side by side, so a lane's 4 rows are one float4.
__device__ __forceinline__ size_t q8_scale_pos(uint32_t row, uint32_t b, uint32_t nb) {
    return (static_cast<size_t>(row >> 4) * nb + b) * 16u + (row & 15u);
}

// f16 bits to f32 for finite values, as kernels.rs f16_finite: the bits
// shifted into place, then scaled by 2^112.
__device__ __forceinline__ float q8_f16(uint32_t h) {
    const uint32_t u = ((h & 0x8000u) << 16) | ((h & 0x7FFFu) << 13);
    return __uint_as_float(u) * __uint_as_float(0x77800000u);
}

// Rust's `(v * id).round() as i8`: halves away from zero, saturating, NaN to 0.
__device__ __forceinline__ uint32_t q8_quant(float v, float id) {
    const float r = roundf(v * id);
    const int q = r != r ? 0 : r >= 127.0f ? 127 : r <= -128.0f ? -128 : static_cast<int>(r);
    return static_cast<uint32_t>(q) & 0xFFu;
}

__global__ __launch_bounds__(kQ8Threads) void lm_q8_prep_kernel(Q8PrepArgs a) {
    static_assert(kQ8Threads % 8u == 0 && kQ8Stage % 32u == 0, "8 lanes per block; whole blocks per stage");
    __shared__ f32x4 sq[kQ8Stage / 4u];
    __shared__ float inv_s;
    const uint32_t r = blockIdx.x, tid = threadIdx.x;
    const uint32_t nb = a.dim / kQ8Block, np = (nb + 1u) / 2u;
    if (r >= a.rows) {  // padding rows of the last row block: every slot of the row 0
        for (uint32_t c = tid; c < 16u * np; c += kQ8Threads)
            *reinterpret_cast<uint32_t*>(a.aq + q8_frag_pos(r, 2u * (c >> 4) + ((c >> 3) & 1u), 4u * (c & 7u), np)) =
                0u;
        for (uint32_t b = tid; b < nb; b += kQ8Threads) a.as[q8_scale_pos(r, b, nb)] = 0.0f;
        return;
    }
    const float* x = a.x + static_cast<size_t>(r) * a.x_stride;
    // ss = sum of x^2 as a left fold (kernels.rs:522-528 over dot_f32): each
    // square is rounded on its own (no fused multiply-add), so the threads
    // form them and one lane adds them in order, a stage at a time
    float ss = 0.0f;
    float* sqf = reinterpret_cast<float*>(sq);
    for (uint32_t c0 = 0; c0 < a.dim; c0 += kQ8Stage) {
        const uint32_t len = a.dim - c0 < kQ8Stage ? a.dim - c0 : kQ8Stage;  // a multiple of 32
        __syncthreads();
        for (uint32_t i = tid; i < len; i += kQ8Threads) {
            const float v = x[c0 + i];
            sqf[i] = v * v;
        }
        __syncthreads();
        if (tid == 0)
            for (uint32_t i = 0; i < len / 4u; i += 8u) {
                f32x4 v[8];
#pragma unroll
                for (uint32_t j = 0; j < 8u; j++) v[j] = sq[i + j];
#pragma unroll
                for (uint32_t j = 0; j < 8u; j++) {
                    ss = ss + v[j][0];
                    ss = ss + v[j][1];
                    ss = ss + v[j][2];
                    ss = ss + v[j][3];
                }
            }
    }
    if (tid == 0) {
        ss = ss / static_cast<float>(a.dim);
        inv_s = 1.0f / sqrtf(ss + a.eps);
    }
    __syncthreads();
    const float inv = inv_s;
    // quantize_q8 per block (kernels.rs:84-100): 8 lanes per block, 4
    // values each; the block's maximum |v| over the 8 lanes (a maximum of
    // non-negative values: the same in any order)
    const uint32_t sub = tid & 7u;
    for (uint32_t b = tid >> 3; b < nb; b += kQ8Threads / 8u) {
        const uint32_t k = kQ8Block * b + 4u * sub;
        float v[4];
        float amax = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4u; j++) {
            v[j] = x[k + j] * inv * a.norm_w[k + j];
            amax = fmaxf(amax, fabsf(v[j]));
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 8));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        uint32_t w = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4u; j++) w |= q8_quant(v[j], id) << (8u * j);
        *reinterpret_cast<uint32_t*>(a.aq + q8_frag_pos(r, b, 4u * sub, np)) = w;
        // an odd nb's last pair has no second block: its slots hold 0
        if (b + 1u == nb && (nb & 1u)) *reinterpret_cast<uint32_t*>(a.aq + q8_frag_pos(r, b + 1u, 4u * sub, np)) = 0u;
        if (sub == 0) a.as[q8_scale_pos(r, b, nb)] = d;
    }
}

// One pair of blocks' operands for a wave: per id block the weight
// fragment (16 bytes: both blocks) and the ids' scales (f16 bits), from HBM;
// per row block the activation fragment (16 bytes: both blocks) and the
// rows' scales of both blocks, from L2.  A ring of T::kRing slots: the loads
// of pair p + kRing are issued as pair p is done, weights and activations
// together, so the waits on the load counter (which retires loads in order)
// never hold a load that is needed later than one still in flight.  With
// kPaired (nb a multiple of 8, wscale 16-byte aligned) the ids' scales come
// a round of kQ8SRound pairs at a time, one 16-byte load per id block (lane
// group g: the scales of pairs 16t + 4g .. 16t + 4g + 3), passed to the
// other lane groups with ds_bpermute: a 128-byte line of an id's scales is
// read by two loads, not sixteen.  Otherwise two 2-byte loads per id block
// and pair.
constexpr uint32_t kQ8SRound = 16;
constexpr uint32_t q8_lcm(uint32_t a, uint32_t b) {
    uint32_t m = a;
    while (m % b) m += a;
    return m;
}
template <class T>
struct Q8Slot {
    i32x4 bf[T::JB];
    uint32_t wsh[T::JB][2];
    i32x4 af[T::RB];
    f32x4 xs[T::RB][2];
};

template <class T, bool kPaired>
__global__ __launch_bounds__(T::kThreads) void lm_q8_gemm_kernel(Q8GemmArgs a) {
    constexpr uint32_t RB = T::RB, JB = T::JB, R = T::kRing, U = q8_lcm(T::kRing, kQ8SRound);
    static_assert(kQ8SRound == 16, "a round's scales: four pairs per lane group");
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wid = tid >> 6;
    const uint32_t wr = wid % T::WR, wn = wid / T::WR;
    const uint32_t nb = a.dim / kQ8Block, np = (nb + 1u) / 2u, nrb = a.rows_pad / 16u;
    const uint32_t rb0 = blockIdx.y * (RB * T::WR) + wr * RB;           // row blocks rb0 .. rb0 + RB - 1
    const uint32_t n0 = blockIdx.x * T::kIds + wn * (16u * JB);         // ids n0 + 16 j + (lane & 15)
    f32x4 acc[RB][JB];
#pragma unroll
    for (uint32_t i = 0; i < RB; i++)
#pragma unroll
        for (uint32_t j = 0; j < JB; j++) acc[i][j] = f32x4{-0.0f, -0.0f, -0.0f, -0.0f};  // Rust's f32 sum starts at -0.0
    bool rbok[RB];
    const int8_t* abase[RB];
    const float* sbase[RB];
#pragma unroll
    for (uint32_t i = 0; i < RB; i++) {
        rbok[i] = rb0 + i < nrb;
        const uint32_t rb = rbok[i] ? rb0 + i : 0u;
        abase[i] = a.aq + static_cast<size_t>(rb) * np * 1024u + lane * 16u;
        sbase[i] = a.as + static_cast<size_t>(rb) * nb * 16u + 4u * (lane >> 4);
    }
    bool idok[JB];
    const int8_t* wrow[JB];
    const uint16_t* wsrow[JB];
#pragma unroll
    for (uint32_t j = 0; j < JB; j++) {
        const uint32_t id = n0 + 16u * j + (lane & 15u);
        idok[j] = id < a.vocab;
        const uint32_t idc = idok[j] ? id : 0u;
        wrow[j] = a.wq + static_cast<size_t>(idc) * a.dim + 16u * (lane >> 4);
        wsrow[j] = a.ws + static_cast<size_t>(idc) * nb;
    }
    const i32x4 zi = {0, 0, 0, 0};
    const f32x4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool upper = lane >= 32u;  // lane groups 2 and 3: the pair's second block
    // pair p: blocks 2p and, when it exists, 2p + 1 (the last pair of an odd
    // nb has one block: lane groups 2 and 3 then load no weights, which would
    // lie past the row's end)
    auto load = [&](Q8Slot<T>& o, uint32_t p) {
        const bool two = 2u * p + 1u < nb;
#pragma unroll
        for (uint32_t j = 0; j < JB; j++) {
            o.bf[j] = two || !upper ? *reinterpret_cast<const i32x4*>(wrow[j] + static_cast<size_t>(p) * 64u) : zi;
            if (!kPaired) {
                o.wsh[j][0] = wsrow[j][2u * p];
                o.wsh[j][1] = two ? wsrow[j][2u * p + 1u] : 0u;
            }
        }
#pragma unroll
        for (uint32_t i = 0; i < RB; i++) {
            const float* sp = sbase[i] + static_cast<size_t>(2u * p) * 16u;
            o.af[i] = rbok[i] ? *reinterpret_cast<const i32x4*>(abase[i] + static_cast<size_t>(p) * 1024u) : zi;
            o.xs[i][0] = rbok[i] ? *reinterpret_cast<const f32x4*>(sp) : zf;
            o.xs[i][1] = rbok[i] && two ? *reinterpret_cast<const f32x4*>(sp + 16) : zf;
        }
    };
    // kPaired: the scales of pairs 16t .. 16t + 15, lane group g holding
    // pairs 16t + 4g .. 16t + 4g + 3 (dword d: pair 16t + 4g + d, its two
    // blocks' scales); np is a multiple of 4, so a group's pairs all exist
    // or none do
    auto load_s = [&](u32x4 (&sc)[JB], uint32_t t) {
        const uint32_t p = kQ8SRound * t + 4u * (lane >> 4);
#pragma unroll
        for (uint32_t j = 0; j < JB; j++)
            sc[j] = p < np ? *reinterpret_cast<const u32x4*>(wsrow[j] + 2u * p) : u32x4{0u, 0u, 0u, 0u};
    };
    // the scales of pair 16t + u (u the same in every lane) from lane group u / 4
    auto take_s = [&](Q8Slot<T>& o, const u32x4 (&sc)[JB], uint32_t u) {
#pragma unroll
        for (uint32_t j = 0; j < JB; j++) {
            const uint32_t v = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(
                static_cast<int>(4u * ((lane & 15u) + 16u * (u >> 2))), static_cast<int>(sc[j][u & 3u])));
            o.wsh[j][0] = v & 0xFFFFu;
            o.wsh[j][1] = v >> 16;
        }
    };
    auto scale_add_one = [&](const Q8Slot<T>& o, uint32_t h) {
        float wsc[JB];
#pragma unroll
        for (uint32_t j = 0; j < JB; j++) wsc[j] = q8_f16(o.wsh[j][h]);
#pragma unroll
        for (uint32_t i = 0; i < RB; i++) {
            if (!rbok[i]) continue;
            const i32x4 ah = (upper == (h != 0)) ? o.af[i] : zi;  // block h's lane groups only
#pragma unroll
            for (uint32_t j = 0; j < JB; j++) {
                const i32x4 s = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, o.bf[j], zi, 0, 0, 0);
#pragma unroll
                for (uint32_t e = 0; e < 4; e++)
                    acc[i][j][e] = acc[i][j][e] + static_cast<float>(s[e]) * wsc[j] * o.xs[i][h][e];
            }
        }
    };
    Q8Slot<T> ring[R];
    u32x4 scur[JB], snext[JB];
    if (kPaired) load_s(snext, 0);
#pragma unroll
    for (uint32_t u = 0; u < R; u++)
        if (u < np) load(ring[u], u);
    // U pairs a round (a multiple of the ring and of the scale round), so
    // every slot and lane group below is fixed at compile time
    for (uint32_t p0 = 0; p0 < np; p0 += U) {
#pragma unroll
        for (uint32_t u = 0; u < U; u++) {
            const uint32_t p = p0 + u;
            if (p >= np) break;
            if (kPaired && u % kQ8SRound == 0) {
#pragma unroll
                for (uint32_t j = 0; j < JB; j++) scur[j] = snext[j];
                if (p + kQ8SRound < np) load_s(snext, p / kQ8SRound + 1u);
            }
            Q8Slot<T>& o = ring[u % R];
            if (kPaired) take_s(o, scur, u % kQ8SRound);
            // the pair's blocks in order
            scale_add_one(o, 0);
            if (2u * p + 1u < nb) scale_add_one(o, 1);
            if (p + R < np) load(o, p + R);
        }
    }
    // lane l holds rows 4 (l >> 4) + e, id l & 15 of each 16 x 16 tile
#pragma unroll
    for (uint32_t i = 0; i < RB; i++) {
        if (!rbok[i]) continue;
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) {
            const uint32_t row = 16u * (rb0 + i) + 4u * (lane >> 4) + e;
            if (row >= a.rows) continue;
            float* out = a.logits + static_cast<size_t>(row) * a.ld;
#pragma unroll
            for (uint32_t j = 0; j < JB; j++)
                if (idok[j]) out[n0 + 16u * j + (lane & 15u)] = acc[i][j][e];
        }
    }
}

// The paired-scale path for batches of up to 32 rows (nb a multiple of 8,
// wq and wscale 16-byte aligned): a step is four pairs, 256 contiguous bytes
// of each weight row (two cache lines), loaded 16 lanes to a row so that
// every load reads whole lines, and turned into the fragment layout through
// a transpose buffer of the wave's own in LDS (rows padded to kQ8L2Stride
// bytes).  A step's lines go to LDS as it starts, which frees their
// registers for the next step's loads; each pair's activations are loaded as
// the pair two before it is done (so loads are issued in the order they are
// used, as above).  A wave owns RB row blocks (1 up to 16 rows, 2 up to 32)
// x 2 id blocks: with one row block the registers leave room for three waves
// a SIMD.
constexpr uint32_t kQ8L2Stride = 272;
template <class T>
__global__ __launch_bounds__(T::kThreads) void lm_q8_gemm_line_kernel(Q8GemmArgs a) {
    constexpr uint32_t RB = T::RB, JB = T::JB, W = T::kThreads / 64u;
    __shared__ __attribute__((aligned(16))) uint8_t tbuf[W][JB][16][kQ8L2Stride];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wid = tid >> 6;
    const uint32_t wn = wid / T::WR;
    const uint32_t nb = a.dim / kQ8Block, np = nb / 2u, ns = np / 4u;
    const uint32_t rb0 = blockIdx.y * (RB * T::WR) + (wid % T::WR) * RB;  // row blocks rb0 .. rb0 + RB - 1
    const uint32_t n0 = blockIdx.x * T::kIds + wn * (16u * JB);
    f32x4 acc[RB][JB];
#pragma unroll
    for (uint32_t i = 0; i < RB; i++)
#pragma unroll
        for (uint32_t j = 0; j < JB; j++) acc[i][j] = f32x4{-0.0f, -0.0f, -0.0f, -0.0f};
    bool rbok[RB];
    const int8_t* abase[RB];
    const float* sbase[RB];
#pragma unroll
    for (uint32_t i = 0; i < RB; i++) {
        rbok[i] = rb0 + i < a.rows_pad / 16u;
        const uint32_t rb = rbok[i] ? rb0 + i : 0u;
        abase[i] = a.aq + static_cast<size_t>(rb) * np * 1024u + lane * 16u;
        sbase[i] = a.as + static_cast<size_t>(rb) * nb * 16u + 4u * (lane >> 4);
    }
    // weight rows as 32-bit offsets from the workgroup's first id (a tile's
    // rows span at most kIds * dim bytes); ids past the vocabulary read the
    // tile's first row
    const uint32_t t0 = blockIdx.x * T::kIds;
    const int8_t* const wq0 = a.wq + static_cast<size_t>(t0) * a.dim;
    const uint16_t* const ws0 = a.ws + static_cast<size_t>(t0) * nb;
    bool idok[JB];
    uint32_t wsoff[JB];
    uint32_t wloff[JB][4];
#pragma unroll
    for (uint32_t j = 0; j < JB; j++) {
        const uint32_t r = n0 - t0 + 16u * j + (lane & 15u);
        idok[j] = t0 + r < a.vocab;
        wsoff[j] = (idok[j] ? r : 0u) * nb;
#pragma unroll
        for (uint32_t q = 0; q < 4u; q++) {
            const uint32_t lr = n0 - t0 + 16u * j + 4u * q + (lane >> 4);
            wloff[j][q] = (t0 + lr < a.vocab ? lr : 0u) * a.dim + 16u * (lane & 15u);
        }
    }
    uint8_t* const wbase = &tbuf[wid][0][lane >> 4][16u * (lane & 15u)];
    const uint8_t* const rbase = &tbuf[wid][0][lane & 15u][16u * (lane >> 4)];
    const i32x4 zi = {0, 0, 0, 0};
    const f32x4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool upper = lane >= 32u;
    i32x4 wl[JB][4];
    struct Act {
        i32x4 af[RB];
        f32x4 xs[RB][2];
    };
    auto load_w = [&](uint32_t s) {
#pragma unroll
        for (uint32_t j = 0; j < JB; j++)
#pragma unroll
            for (uint32_t q = 0; q < 4u; q++)
                wl[j][q] = *reinterpret_cast<const i32x4*>(wq0 + wloff[j][q] + 256u * s);
    };
    auto load_a = [&](Act& x, uint32_t p) {
#pragma unroll
        for (uint32_t i = 0; i < RB; i++) {
            const float* sp = sbase[i] + static_cast<size_t>(2u * p) * 16u;
            x.af[i] = rbok[i] ? *reinterpret_cast<const i32x4*>(abase[i] + static_cast<size_t>(p) * 1024u) : zi;
            x.xs[i][0] = rbok[i] ? *reinterpret_cast<const f32x4*>(sp) : zf;
            x.xs[i][1] = rbok[i] ? *reinterpret_cast<const f32x4*>(sp + 16) : zf;
        }
    };
    auto load_s = [&](u32x4 (&sc)[JB], uint32_t r) {
        const uint32_t p = kQ8SRound * r + 4u * (lane >> 4);
#pragma unroll
        for (uint32_t j = 0; j < JB; j++)
            sc[j] = p < np ? *reinterpret_cast<const u32x4*>(ws0 + wsoff[j] + 2u * p) : u32x4{0u, 0u, 0u, 0u};
    };
    Act act[2];
    u32x4 scur[JB], snext[JB];
    load_s(snext, 0);
    load_w(0);
    load_a(act[0], 0);
    load_a(act[1], 1);
    for (uint32_t s0 = 0; s0 < ns; s0 += kQ8SRound / 4u) {
#pragma unroll
        for (uint32_t v = 0; v < kQ8SRound / 4u; v++) {
            const uint32_t s = s0 + v;
            if (s >= ns) break;
            if (v == 0) {
#pragma unroll
                for (uint32_t j = 0; j < JB; j++) scur[j] = snext[j];
                if (s0 + kQ8SRound / 4u < ns) load_s(snext, s0 / (kQ8SRound / 4u) + 1u);
            }
#pragma unroll
            for (uint32_t j = 0; j < JB; j++)
#pragma unroll
                for (uint32_t q = 0; q < 4u; q++)
                    *reinterpret_cast<i32x4*>(wbase + j * (16u * kQ8L2Stride) + q * (4u * kQ8L2Stride)) = wl[j][q];
            if (s + 1u < ns) load_w(s + 1u);
#pragma unroll
            for (uint32_t t = 0; t < 4u; t++) {
                const uint32_t u = 4u * v + t;  // the pair's place in the scale round
                const uint32_t p = 4u * s + t;
                Act& x = act[t & 1u];
                i32x4 bf[JB];
                float wsc[JB][2];
#pragma unroll
                for (uint32_t j = 0; j < JB; j++) {
                    bf[j] = *reinterpret_cast<const i32x4*>(rbase + j * (16u * kQ8L2Stride) + t * 64u);
                    const uint32_t sv = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(
                        static_cast<int>(4u * ((lane & 15u) + 16u * (u >> 2))), static_cast<int>(scur[j][u & 3u])));
                    wsc[j][0] = q8_f16(sv & 0xFFFFu);
                    wsc[j][1] = q8_f16(sv >> 16);
                }
#pragma unroll
                for (uint32_t h = 0; h < 2u; h++)  // the pair's blocks in order
#pragma unroll
                    for (uint32_t i = 0; i < RB; i++) {
                        if (!rbok[i]) continue;
                        const i32x4 ah = (upper == (h != 0)) ? x.af[i] : zi;
#pragma unroll
                        for (uint32_t j = 0; j < JB; j++) {
                            const i32x4 sm = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, bf[j], zi, 0, 0, 0);
#pragma unroll
                            for (uint32_t e = 0; e < 4; e++)
                                acc[i][j][e] = acc[i][j][e] + static_cast<float>(sm[e]) * wsc[j][h] * x.xs[i][h][e];
                        }
                    }
                if (p + 2u < np) load_a(x, p + 2u);
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < RB; i++) {
        if (!rbok[i]) continue;
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) {
            const uint32_t row = 16u * (rb0 + i) + 4u * (lane >> 4) + e;
            if (row >= a.rows) continue;
            float* out = a.logits + static_cast<size_t>(row) * a.ld;
#pragma unroll
            for (uint32_t j = 0; j < JB; j++)
                if (idok[j]) out[n0 + 16u * j + (lane & 15u)] = acc[i][j][e];
        }
    }
}

// With paired scales batches of up to 32 rows take the whole-line kernel
// (its own tiles: 16 or 32 rows x 128 ids), the others the pair-at-a-time
// kernel.
template <class T, bool kPaired>
void launch_q8_gemm(const Q8GemmArgs& g, hipStream_t st) {
    const dim3 grid((g.vocab + T::kIds - 1u) / T::kIds, (g.rows_pad + T::kRows - 1u) / T::kRows);
    if constexpr (kPaired && T::JB == 2u) hipLaunchKernelGGL((lm_q8_gemm_line_kernel<T>), grid, dim3(T::kThreads), 0, st, g);
    else hipLaunchKernelGGL((lm_q8_gemm_kernel<T, kPaired>), grid, dim3(T::kThreads), 0, st, g);
}

template <bool kPaired>
void launch_q8_tiles(const Q8GemmArgs& g, hipStream_t st) {
    // tiles by batch (rows x ids): 16 x 128 (whole lines) or 16 x 256, 32 x 128 (whole lines) or 32 x 256,
    // 64 x 256, 128 x 128, 256 x 64
    const uint32_t rp = g.rows_pad;
    if (rp <= 16u) {
        if constexpr (kPaired) launch_q8_gemm<Q8Tile<1, 2, 1, 4>, true>(g, st);
        else launch_q8_gemm<Q8Tile<1, 4, 1, 4>, false>(g, st);
    } else if (rp <= 32u) {
        if constexpr (kPaired) launch_q8_gemm<Q8Tile<2, 2, 1, 4>, true>(g, st);
        else launch_q8_gemm<Q8Tile<2, 4, 1, 4>, false>(g, st);
    }
    else if (rp <= 64u) launch_q8_gemm<Q8Tile<2, 4, 2, 4>, kPaired>(g, st);
    else if (rp <= 128u) launch_q8_gemm<Q8Tile<2, 4, 4, 2>, kPaired>(g, st);
    else launch_q8_gemm<Q8Tile<2, 4, 8, 1>, kPaired>(g, st);
}

void set_err(char* err, size_t errlen, const char* fmt, ...) {
    if (!err || errlen == 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

// The workgroup tile's rows for a batch: the smallest tile that holds it, up to 256.
uint32_t tile_rows(uint32_t rows) {
    return rows <= 16u ? 16u : rows <= 32u ? 32u : rows <= 64u ? 64u : rows <= 128u ? 128u : 256u;
}
uint32_t rows_pad(uint32_t rows) { return (rows + tile_rows(rows) - 1u) / tile_rows(rows) * tile_rows(rows); }

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
    hipLaunchKernelGGL(tsm::lm::lm_prep_kernel, dim3(rp), dim3(tsm::lm::kPrepThreads), 0, st, p);
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
    const uint32_t tm = tsm::lm::tile_rows(rows);
    const dim3 grid((vocab + tsm::lm::kTileN - 1u) / tsm::lm::kTileN, rp / tm);
    auto launch = [&](auto tile) {
        using T = decltype(tile);
        if (split) hipLaunchKernelGGL((tsm::lm::lm_gemm_kernel<true, T>), grid, dim3(T::kThreads), 0, st, g);
        else hipLaunchKernelGGL((tsm::lm::lm_gemm_kernel<false, T>), grid, dim3(T::kThreads), 0, st, g);
    };
    if (tm == 16u) launch(tsm::lm::Tile16{});
    else if (tm == 32u) launch(tsm::lm::Tile32{});
    else if (tm == 64u) launch(tsm::lm::Tile64{});
    else if (tm == 128u) launch(tsm::lm::Tile128{});
    else launch(tsm::lm::Tile256{});
    e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "gemm launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

size_t tsm_lm_head_q8_workspace(uint32_t rows, uint32_t dim) {
    // the activation fragments (1 KB per 16 rows and pair of blocks), then
    // the f32 block scales
    const size_t rp = (static_cast<size_t>(rows) + 15u) / 16u * 16u, nb = dim / tsm::lm::kQ8Block;
    return rp * ((nb + 1u) / 2u) * 64u + rp * nb * 4u;
}

int tsm_lm_head_q8(void* stream, const float* x, uint32_t x_stride, const float* norm_w, float eps, const int8_t* wq,
                   const uint16_t* wscale, uint32_t rows, uint32_t dim, uint32_t vocab, void* workspace,
                   size_t workspace_bytes, float* logits, uint32_t ld, char* err, size_t errlen) {
    using tsm::lm::set_err;
    if (rows == 0 || rows > TSM_LM_MAX_ROWS)
        return set_err(err, errlen, "rows %u is outside [1, %u]", rows, TSM_LM_MAX_ROWS), 1;
    if (dim == 0 || dim % tsm::lm::kQ8Block != 0 || dim > TSM_LM_MAX_DIM)
        return set_err(err, errlen, "dim %u must be a positive multiple of %u, at most %u", dim, tsm::lm::kQ8Block,
                       TSM_LM_MAX_DIM), 1;
    if (vocab == 0 || vocab > TSM_MAX_VOCAB)
        return set_err(err, errlen, "vocab %u is outside [1, %u]", vocab, TSM_MAX_VOCAB), 1;
    if (!x || !norm_w || !wq || !wscale || !logits || !workspace)
        return set_err(err, errlen, "x, norm_w, wq, wscale, workspace and logits must be set"), 1;
    if (x_stride < dim) return set_err(err, errlen, "x_stride %u is below dim %u", x_stride, dim), 1;
    if (ld < vocab) return set_err(err, errlen, "ld %u is below vocab %u", ld, vocab), 1;
    if ((reinterpret_cast<uintptr_t>(wq) & 15u) || (reinterpret_cast<uintptr_t>(wscale) & 1u) ||
        (reinterpret_cast<uintptr_t>(workspace) & 15u))
        return set_err(err, errlen, "wq and workspace must be 16-byte and wscale 2-byte aligned"), 1;
    const size_t need = tsm_lm_head_q8_workspace(rows, dim);
    if (workspace_bytes < need)
        return set_err(err, errlen, "workspace holds %zu bytes; %zu needed", workspace_bytes, need), 1;
    const uint32_t rp = (rows + 15u) / 16u * 16u;
    const size_t aqb = static_cast<size_t>(rp) * ((dim / tsm::lm::kQ8Block + 1u) / 2u) * 64u;
    int8_t* aq = static_cast<int8_t*>(workspace);
    float* as = reinterpret_cast<float*>(static_cast<char*>(workspace) + aqb);
    const hipStream_t st = static_cast<hipStream_t>(stream);

    tsm::lm::Q8PrepArgs p;
    p.x = x;
    p.norm_w = norm_w;
    p.aq = aq;
    p.as = as;
    p.eps = eps;
    p.rows = rows;
    p.rows_pad = rp;
    p.dim = dim;
    p.x_stride = x_stride;
    hipLaunchKernelGGL(tsm::lm::lm_q8_prep_kernel, dim3(rp), dim3(tsm::lm::kQ8Threads), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "prep launch failed: %s", hipGetErrorString(e)), 1;
    tsm::lm::Q8GemmArgs g;
    g.aq = aq;
    g.as = as;
    g.wq = wq;
    g.ws = wscale;
    g.logits = logits;
    g.rows = rows;
    g.rows_pad = rp;
    g.dim = dim;
    g.vocab = vocab;
    g.ld = ld;
    // the weight scales 16 pairs at a time when dim is a multiple of 256 and
    // wscale 16-byte aligned, else 2 bytes a pair
    if ((dim / tsm::lm::kQ8Block) % 8u == 0 && (reinterpret_cast<uintptr_t>(wscale) & 15u) == 0)
        tsm::lm::launch_q8_tiles<true>(g, st);
    else
        tsm::lm::launch_q8_tiles<false>(g, st);
    e = hipGetLastError();
    if (e != hipSuccess) return set_err(err, errlen, "gemm launch failed: %s", hipGetErrorString(e)), 1;
    return 0;
}

}  // extern "C"
