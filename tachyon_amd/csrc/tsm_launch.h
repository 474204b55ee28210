// tsm_launch.h - argument records of the two kernels of a sampling step and
// their host-side launchers (defined next to each kernel).
#pragma once

#include "tsm_device.h"

namespace tsm {

struct SweepArgs {
    const float* logits;
    const tsm_row_params* params;
    const uint32_t* hist_ids;
    const uint32_t* hist_off;
    const uint32_t* mask;
    ChunkStats* stats;
    uint2* cand;    // [rows*chunks][kCandCap]  (value bits, id | penalized<<31)
    uint2* pen;     // [rows*chunks][kPenCap]   (id, raw value bits)
    uint2* allow;   // [rows*chunks][kAllowCap] (value bits, id)
    uint32_t* status;
    uint32_t row_stride, usable, mask_stride, n_chunks;
};

struct FinArgs {
    const float* logits;
    const tsm_row_params* params;
    const uint32_t* hist_ids;
    const uint32_t* hist_off;
    const uint32_t* mask;
    const float* uniforms;
    const ChunkStats* stats;
    const uint2* cand;
    const uint2* pen;
    const uint2* allow;
    uint32_t* status;
    uint32_t* out_token;
    float* out_logprob;
    uint32_t* out_top_ids;
    float* out_top_lp;
    float* out_prob;
    uint32_t* out_keep;
    uint32_t* dist_ids;
    float* dist_probs;
    uint32_t row_stride, usable, mask_stride, n_chunks, top_stride, dist_stride;
    uint32_t distribution;  // 1: write the kept distribution instead of drawing
};

void launch_sweep(const SweepArgs& a, uint32_t rows, bool vec, hipStream_t stream);
void launch_finalize(const FinArgs& a, uint32_t rows, hipStream_t stream);
hipError_t finalize_set_smem_attr();

}  // namespace tsm
