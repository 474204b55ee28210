// tsm_probe.hip - test helper (not part of the product library): evaluates
// the device restatement of glibc expf (tsm::glibc_expf) over an array so a
// GPU test can compare it bit for bit with the host's glibc expf.
#include "../../tachyon_amd/csrc/tsm_device.h"

__global__ void probe_expf_kernel(const float* x, float* y, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = tsm::glibc_expf(x[i]);
}

extern "C" int tsm_probe_expf(const float* x, float* y, uint32_t n, void* stream) {
    const uint32_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(probe_expf_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), x, y, n);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}
