// lmhead_oracle.cpp - CPU restatement of Tachyon's output layer for a Bf16
// lm_head, TEST INFRASTRUCTURE ONLY.
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
//                dot_bf16(W[r], x[i]).
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

}  // extern "C"
