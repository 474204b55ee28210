// lmhead_oracle.cpp - CPU restatement of Tachyon's output layer for a Bf16
// or Q8 lm_head, TEST INFRASTRUCTURE ONLY.
//
// The parity checker of the logits producer (tsm_lm_head): tests/ load it
// through ctypes, inside libtachyon_oracle.so.  The product library never
// links, loads or calls it.
//
// It follows the reference's portable scalar path:
//   rmsnorm      kernels.rs:522-528 over dot_f32 (kernels.rs:1407-1409): a
//                left fold of x*x in f32, / len, 1 / sqrt(ss + eps), then
//                v * inv * g per element;
//   dot_bf16     kernels.rs:1411-1413: a left fold of bf16_to_f32(w) * x in
//                f32;
//   the matmul   weights.rs:230-239 (Bf16 arm): out[i * rows + r] =
//                dot_bf16(W[r], x[i]);
//   Q8           quantize_q8 of each x row (kernels.rs:84-100, as
//                quantize_input, weights.rs:652-664), then per weight row
//                the scalar dot_q8_with (kernels.rs:1420-1430): integer block
//                dots, each times the row's f16 block scale and the x
//                block's scale, summed over blocks in order.
// (On aarch64 the reference folds with NEON accumulators instead, so its
// own results differ by summation order from platform to platform; the GPU
// tests hold both to a bound on that difference.)
//
// Pinning (tests/test_oracle.py): closed forms (constant rows, one-hot
// weights, small integers whose sums are exact) checked against numpy.
#include <cmath>
#include <cstdint>
#include <cstring>

namespace {

float bf16_to_f32(uint16_t h) {
    const uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" {

// rmsnorm (kernels.rs:522-528) of one row of n values.
void or_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* out) {
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / static_cast<float>(n);
    const float inv = 1.0f / std::sqrt(ss + eps);
    for (uint32_t i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

// The Bf16 matmul (weights.rs:230-239): out[i * ld + r] = dot_bf16(W[r], x[i])
// for t rows of x (dim values each) and `rows` rows of W.
void or_matmul_bf16(const uint16_t* w, uint32_t rows, uint32_t dim, const float* x, uint32_t t, float* out,
                    uint32_t ld) {
    for (uint32_t i = 0; i < t; i++)
        for (uint32_t r = 0; r < rows; r++) {
            const uint16_t* wr = w + static_cast<size_t>(r) * dim;
            const float* xi = x + static_cast<size_t>(i) * dim;
            float s = 0.0f;
            for (uint32_t k = 0; k < dim; k++) s += bf16_to_f32(wr[k]) * xi[k];
            out[static_cast<size_t>(i) * ld + r] = s;
        }
}

// f16 bits to f32 for finite values (kernels.rs f16_finite): the bits
// shifted into place, then scaled by 2^112 (which also renormalizes
// subnormals).
static float f16_finite(uint16_t h) {
    const uint32_t hh = static_cast<uint32_t>(h) & 0x7FFFu, sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t u = sign | (hh << 13);
    float f, m;
    std::memcpy(&f, &u, 4);
    const uint32_t two112 = 0x77800000u;
    std::memcpy(&m, &two112, 4);
    return f * m;
}

// quantize_q8 (kernels.rs:84-100): per block of 32 values, d = max|x| / 127,
// q = round(x / d) (Rust's f32::round, halves away from zero; `as i8`
// saturates, NaN to 0), scales[b] = d.
void or_quantize_q8(const float* x, uint32_t n, float* scales, int8_t* qs) {
    for (uint32_t b = 0; b < n / 32u; b++) {
        float amax = 0.0f;
        for (uint32_t j = 0; j < 32u; j++) amax = std::fmax(amax, std::fabs(x[32u * b + j]));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        for (uint32_t j = 0; j < 32u; j++) {
            const float r = std::round(x[32u * b + j] * id);
            qs[32u * b + j] = r != r ? 0 : r >= 127.0f ? 127 : r <= -128.0f ? -128 : static_cast<int8_t>(r);
        }
        scales[b] = d;
    }
}

// The Q8 matmul (weights.rs:474-560, int_matmul over Q8Rows, weights.rs:344-374):
// each row of x is quantized (quantize_input, weights.rs:652-664), then
// out[i * ld + r] = sum over blocks b, in order, of (s_b as f32) * f16(wscale[r][b])
// * xs[i][b], s_b the exact integer dot of the block's 32 weights and values
// (the scalar dot_q8_with, kernels.rs:1420-1430).
void or_matmul_q8(const int8_t* wq, const uint16_t* wscale, uint32_t rows, uint32_t dim, const float* x,
                  uint32_t t, float* out, uint32_t ld) {
    const uint32_t nb = dim / 32u;
    float* xs = new float[nb];
    int8_t* xq = new int8_t[dim];
    for (uint32_t i = 0; i < t; i++) {
        or_quantize_q8(x + static_cast<size_t>(i) * dim, dim, xs, xq);
        for (uint32_t r = 0; r < rows; r++) {
            const int8_t* w = wq + static_cast<size_t>(r) * dim;
            const uint16_t* ws = wscale + static_cast<size_t>(r) * nb;
            float acc = -0.0f;  // the neutral element of Rust's f32 Sum (Rust 1.87)
            for (uint32_t b = 0; b < nb; b++) {
                int32_t s = 0;
                for (uint32_t j = 0; j < 32u; j++) s += static_cast<int32_t>(w[32u * b + j]) * xq[32u * b + j];
                acc += static_cast<float>(s) * f16_finite(ws[b]) * xs[b];
            }
            out[static_cast<size_t>(i) * ld + r] = acc;
        }
    }
    delete[] xs;
    delete[] xq;
}

}  // extern "C"
