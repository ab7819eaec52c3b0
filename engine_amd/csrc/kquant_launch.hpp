// Internal launcher API between the C-ABI host layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ribn_amd {

// Members one wave-GEMV launch accumulates; larger batches are split by the host.
constexpr int kWaveMaxMembers = 4;

hipError_t launch_dequant(int value_type, const uint8_t* w, uint32_t wbytes, float* out, uint32_t nblocks,
                          hipStream_t stream);

hipError_t launch_gemv_exact(int value_type, const uint8_t* w, uint32_t wbytes, const float* x, float* y,
                             int K, int N, int members, hipStream_t stream);

// gamma == nullptr: plain GEMV; otherwise RMSNorm(x; gamma, eps) is fused into the activation load.
hipError_t launch_gemv_wave(int value_type, const uint8_t* w, uint32_t wbytes, const float* x, float* y, int K,
                            int N, int members, const float* gamma, float eps, int cu_count, hipStream_t stream);

hipError_t launch_rms_norm(const float* x, const float* w, float* y, int length, int members, float eps,
                           hipStream_t stream);

}  // namespace ribn_amd
