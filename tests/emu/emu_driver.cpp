// emu_driver.cpp - runs one tsm_sample / tsm_distribution call of the C ABI
// (include/tachyon_sampler.h) on the CPU emulation of the kernels.
// TEST INFRASTRUCTURE ONLY.
//
//   emu_driver <input.bin> <output.bin>
//
// Input (little endian): u32 magic 'TSMW', mode (0 sample, 1 distribution),
// rows, row_stride, usable, mask_stride (0: no mask), hist_total
// (0xFFFFFFFF: no history), top_stride, dist_stride, kinds (0: the batch's
// row_kinds left unknown, 1: computed with tsm_row_kind as a caller would);
// then
// logits f32[rows*row_stride], params (40 B each)[rows],
// hist_offsets u32[rows+1] + hist_ids u32[hist_total] (if history),
// mask u32[rows*mask_stride] (if mask), uniforms f32[rows].
// Output: u32 rc, u32 status, then for mode 0 token u32[rows],
// logprob f32[rows], top_ids u32[rows*top_stride], top_lp f32[rows*top_stride],
// prob f32[rows], keep u32[rows]; for mode 1 ids u32[rows*dist_stride],
// probs f32[rows*dist_stride], keep u32[rows].  On rc != 0 the error text
// follows instead.
//
// Every array gets its own exact-size allocation, so the sanitizers see an
// access one past any of them.
#include <hip/hip_runtime.h>

#include <vector>

#include "tachyon_sampler.h"

namespace {

struct Reader {
    FILE* f;
    uint32_t u32() {
        uint32_t v;
        if (std::fread(&v, 4, 1, f) != 1) std::abort();
        return v;
    }
    template <class T>
    T* dev(size_t n) {  // exact-size "device" buffer filled from the file
        if (n == 0) return nullptr;
        T* p = static_cast<T*>(std::malloc(n * sizeof(T)));
        if (std::fread(p, sizeof(T), n, f) != n) std::abort();
        return p;
    }
};

template <class T>
T* zeros(size_t n) {
    if (n == 0) return nullptr;
    T* p = static_cast<T*>(std::malloc(n * sizeof(T)));
    std::memset(p, 0xEE, n * sizeof(T));
    return p;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: emu_driver in.bin out.bin\n");
        return 2;
    }
    FILE* in = std::fopen(argv[1], "rb");
    if (!in) return 2;
    Reader R{in};
    if (R.u32() != 0x574D5354u) return 3;
    const uint32_t mode = R.u32(), rows = R.u32(), row_stride = R.u32(), usable = R.u32();
    const uint32_t mask_stride = R.u32(), hist_total = R.u32(), top_stride = R.u32(), dist_stride = R.u32();
    const uint32_t kinds_mode = R.u32();
    tsm_batch b{};
    b.logits = R.dev<float>(static_cast<size_t>(rows) * row_stride);
    b.rows = rows;
    b.row_stride = row_stride;
    b.usable = usable;
    b.mask_stride = mask_stride;
    b.params = R.dev<tsm_row_params>(rows);
    if (hist_total != 0xFFFFFFFFu) {
        b.hist_offsets = R.dev<uint32_t>(rows + 1);
        b.hist_ids = hist_total ? R.dev<uint32_t>(hist_total) : static_cast<uint32_t*>(std::malloc(4));
    }
    if (mask_stride) b.mask = R.dev<uint32_t>(static_cast<size_t>(rows) * mask_stride);
    b.uniforms = R.dev<float>(rows);
    if (kinds_mode == 1) {  // as a caller would: from the host-side parameters and history lengths
        for (uint32_t r = 0; r < rows; r++) {
            const uint32_t hl = b.hist_offsets ? b.hist_offsets[r + 1] - b.hist_offsets[r] : 0u;
            b.row_kinds |= tsm_row_kind(&b.params[r], usable, hl, mode == 0 && b.mask != nullptr);
        }
    }
    std::fclose(in);

    char err[512] = {0};
    tsm_ctx* ctx = tsm_create(0, rows, usable, err, sizeof(err));
    FILE* out = std::fopen(argv[2], "wb");
    auto put = [&](const void* p, size_t bytes) { std::fwrite(p, 1, bytes, out); };
    if (!ctx) {
        const uint32_t rc = 100, st = 0;
        put(&rc, 4);
        put(&st, 4);
        put(err, std::strlen(err));
        std::fclose(out);
        return 0;
    }
    int rc;
    uint32_t status = 0;
    if (mode == 0) {
        tsm_outputs o{};
        o.token = zeros<uint32_t>(rows);
        o.logprob = zeros<float>(rows);
        o.top_stride = top_stride;
        o.top_ids = zeros<uint32_t>(static_cast<size_t>(rows) * top_stride);
        o.top_logprobs = zeros<float>(static_cast<size_t>(rows) * top_stride);
        o.prob = zeros<float>(rows);
        o.keep = zeros<uint32_t>(rows);
        rc = tsm_sample(ctx, nullptr, &b, &o, err, sizeof(err));
        char e2[256];
        tsm_status(ctx, &status, e2, sizeof(e2));
        const uint32_t urc = static_cast<uint32_t>(rc);
        put(&urc, 4);
        put(&status, 4);
        if (rc != 0) {
            put(err, std::strlen(err));
        } else {
            put(o.token, rows * 4);
            put(o.logprob, rows * 4);
            if (top_stride) {
                put(o.top_ids, static_cast<size_t>(rows) * top_stride * 4);
                put(o.top_logprobs, static_cast<size_t>(rows) * top_stride * 4);
            }
            put(o.prob, rows * 4);
            put(o.keep, rows * 4);
        }
    } else {
        uint32_t* ids = zeros<uint32_t>(static_cast<size_t>(rows) * dist_stride);
        float* ps = zeros<float>(static_cast<size_t>(rows) * dist_stride);
        uint32_t* keep = zeros<uint32_t>(rows);
        rc = tsm_distribution(ctx, nullptr, &b, ids, ps, dist_stride, keep, err, sizeof(err));
        char e2[256];
        tsm_status(ctx, &status, e2, sizeof(e2));
        const uint32_t urc = static_cast<uint32_t>(rc);
        put(&urc, 4);
        put(&status, 4);
        if (rc != 0) {
            put(err, std::strlen(err));
        } else {
            put(ids, static_cast<size_t>(rows) * dist_stride * 4);
            put(ps, static_cast<size_t>(rows) * dist_stride * 4);
            put(keep, rows * 4);
        }
    }
    std::fclose(out);
    tsm_destroy(ctx);
    return 0;
}
