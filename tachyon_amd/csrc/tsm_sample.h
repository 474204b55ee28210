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
};

// Queues one sampling step (one workgroup per row) on `stream`.
void launch_sample(const SampleArgs& a, uint32_t rows, bool vec_loads, hipStream_t stream);
// Raises the kernel's dynamic LDS limit to what it uses (call once per device).
hipError_t sample_set_smem_attr();

}  // namespace tsm
