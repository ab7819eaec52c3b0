// Matrix-core peak probe (measurement only; no counterpart in the reference,
// whose roofline notes ask for the MFMA peak to be confirmed by a measured
// microbenchmark). Every wave of a full grid issues independent MFMAs on
// register operands, sixteen accumulators deep, so the matrix pipes never
// wait on a dependency or on memory; the achieved rate is the chip's dense
// peak for that instruction. (Eight chains per wave, even with four waves
// per SIMD, hold v_mfma_f32_16x16x32_f16 to 1.39-1.41 PFLOP/s: its result
// latency needs more independent instructions in flight than that.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "abi_internal.hpp"
#include "ribn_amd.h"

using namespace ribn_amd_abi;

namespace {

typedef _Float16 p_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 p_bf8 __attribute__((ext_vector_type(8)));
typedef float p_f4 __attribute__((ext_vector_type(4)));
typedef float p_f16v __attribute__((ext_vector_type(16)));

constexpr int kChains = 16;  // independent accumulators per wave

// FLOPs of one instruction: 2 * M * N * K.
constexpr double kFlops[4] = {2.0 * 16 * 16 * 32, 2.0 * 32 * 32 * 16, 2.0 * 16 * 16 * 32, 2.0 * 16 * 16 * 4};

template <int KIND>
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* sink, int iters) {
    const int lane = threadIdx.x & 63;
    // operands that differ per lane, so nothing folds at compile time
    const float seed = 1.0f + 1e-3f * (float)lane;
    if constexpr (KIND == 0 || KIND == 2) {
        p_f4 acc[kChains];
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = p_f4{0.f, 0.f, 0.f, 0.f};
        if constexpr (KIND == 0) {
            p_half8 a, b;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                a[j] = (_Float16)(seed * (float)(j + 1) * 1e-3f);
                b[j] = (_Float16)(seed * (float)(8 - j) * 1e-3f);
            }
            for (int i = 0; i < iters; ++i) {
#pragma unroll
                for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
            }
        } else {
            p_bf8 a, b;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                a[j] = (__bf16)(seed * (float)(j + 1) * 1e-3f);
                b[j] = (__bf16)(seed * (float)(8 - j) * 1e-3f);
            }
            for (int i = 0; i < iters; ++i) {
#pragma unroll
                for (int c = 0; c < kChains; ++c)
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
            }
        }
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
        if (s == -1.0f) sink[blockIdx.x] = s;  // never true: keeps the work
    } else if constexpr (KIND == 1) {
        p_f16v acc[kChains / 2];
#pragma unroll
        for (int c = 0; c < kChains / 2; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[c][i] = 0.f;
        p_half8 a, b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            a[j] = (_Float16)(seed * (float)(j + 1) * 1e-3f);
            b[j] = (_Float16)(seed * (float)(8 - j) * 1e-3f);
        }
        for (int i = 0; i < iters; ++i) {
            // two 32x32 instructions per chain step: as many flops per
            // iteration as the 16x16 kinds
#pragma unroll
            for (int c = 0; c < kChains / 2; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
        }
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < kChains / 2; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) s += acc[c][i];
        if (s == -1.0f) sink[blockIdx.x] = s;
    } else {
        p_f4 acc[kChains];
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = p_f4{0.f, 0.f, 0.f, 0.f};
        const float a = seed * 1e-3f, b = seed * 2e-3f;
        for (int i = 0; i < iters; ++i) {
#pragma unroll
            for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
        }
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
        if (s == -1.0f) sink[blockIdx.x] = s;
    }
}

// Instructions per wave per iteration.
constexpr int kPerIter[4] = {kChains, kChains / 2, kChains, kChains};

}  // namespace

extern "C" {

ribn_amd_status ribn_amd_probe_mfma_peak(ribn_amd_context* ctx, uint32_t kind, uint32_t iterations,
                                         double* tflops) {
    if (!ctx || !tflops) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (kind > 3) return fail(RIBN_AMD_INVALID_ARGUMENT, 3, kind, "unknown MFMA kind %u", kind);
    if (iterations == 0 || iterations > (1u << 20)) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, 1u << 20, iterations, "iterations must be 1..%u", 1u << 20);
    }
    DeviceGuard guard(ctx->device);
    // four waves on every SIMD of every CU (one 256-thread workgroup per
    // SIMD's worth), two rounds of residency
    const int blocks = ctx->cu_count * 8;
    float* sink = nullptr;
    hipError_t e = hipMalloc(&sink, (size_t)blocks * sizeof(float));
    if (e != hipSuccess) return driver(e, "hipMalloc probe sink");
    hipEvent_t t0 = nullptr, t1 = nullptr;
    e = hipEventCreate(&t0);
    if (e == hipSuccess) e = hipEventCreate(&t1);
    auto launch = [&](int iters) {
        switch (kind) {
        case 0: hipLaunchKernelGGL(mfma_peak_kernel<0>, dim3(blocks), dim3(256), 0, ctx->stream, sink, iters); break;
        case 1: hipLaunchKernelGGL(mfma_peak_kernel<1>, dim3(blocks), dim3(256), 0, ctx->stream, sink, iters); break;
        case 2: hipLaunchKernelGGL(mfma_peak_kernel<2>, dim3(blocks), dim3(256), 0, ctx->stream, sink, iters); break;
        default: hipLaunchKernelGGL(mfma_peak_kernel<3>, dim3(blocks), dim3(256), 0, ctx->stream, sink, iters); break;
        }
        return hipGetLastError();
    };
    if (e == hipSuccess) e = launch(16);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(t0, ctx->stream);
    if (e == hipSuccess) e = launch((int)iterations);
    if (e == hipSuccess) e = hipEventRecord(t1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(t1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, t0, t1);
    if (t0) hipEventDestroy(t0);
    if (t1) hipEventDestroy(t1);
    hipFree(sink);
    if (e != hipSuccess) return driver(e, "MFMA peak probe");
    const double insts = (double)blocks * 4.0 * (double)iterations * (double)kPerIter[kind];
    *tflops = insts * kFlops[kind] / ((double)ms * 1e-3) / 1e12;
    return ok();
}

}  // extern "C"
