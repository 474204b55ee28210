// tsm_sample.h - argument record of the sampling kernel and its host-side
// launcher (defined in tsm_sample.hip).
#pragma once

#include "tsm_device.h"

namespace tsm {

struct SampleArgs {
    const float* logits;
    const tsm_row_params* params;
    const uint32_t* hist_ids;
    const uint32_t* hist_off;
    const uint32_t* mask;
    const float* uniforms;
    uint32_t* status;
    uint32_t* out_token;
    float* out_logprob;
    uint32_t* out_top_ids;
    float* out_top_lp;
    float* out_prob;
    uint32_t* out_keep;
    uint32_t* dist_ids;
    float* dist_probs;
    uint32_t row_stride, usable, mask_stride, top_stride, dist_stride;
    uint32_t distribution;  // 1: write the kept distribution instead of drawing
    uint32_t skip_split;    // 1: rows the split kernel takes are sampled there (this kernel skips them)
    uint32_t skip_lean;     // 1: rows the lean kernel takes are sampled there (sample_kernel skips them)
    uint32_t general;       // 1: sample_kernel runs too (the lean kernel leaves it the rows it does not take)
};

// Queues the whole-row kernels of one sampling step (one workgroup per row)
// on `stream`: the lean kernel (the common top-k rows) when `lean`, the
// general kernel (every other row) when `general`.
void launch_sample(const SampleArgs& a, uint32_t rows, bool vec_loads, bool lean, bool general, hipStream_t stream);
// Whether the lean kernel takes a row (host and device).
__host__ __device__ inline bool lean_takes(const RowMode& m, const tsm_row_params& p, uint32_t hist_len, uint32_t n,
                                           bool distribution) {
    const bool fast_hist = !m.penal || (hist_len <= kHistFast && n <= 32u * kBitmapWords);
    const bool lowers = p.repetition_penalty >= 1.0f && p.repetition_penalty <= 3.4e38f && p.frequency_penalty >= 0.0f &&
                        p.frequency_penalty <= 3.4e38f && p.presence_penalty >= 0.0f && p.presence_penalty <= 3.4e38f;
    return !distribution && m.topk && fast_hist && (!m.penal || lowers) && m.want <= kWaveList;
}
// Raises the kernel's dynamic LDS limit to what it uses (call once per device).
hipError_t sample_set_smem_attr();

}  // namespace tsm
