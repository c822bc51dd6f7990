// Achievable MFMA rate on this device: a loop of independent matrix instructions from
// registers only (no memory traffic inside the loop), on every CU. The benchmark reports it
// beside the datasheet peaks, so that a kernel's fraction of the peak can be read against what
// the matrix cores sustain in practice (the reference's profiler times whole layer calls and
// has no counterpart).
//
// Each wave keeps kAcc accumulator tiles and issues one MFMA into each per iteration, so
// consecutive instructions never depend on each other; two workgroups of 8 waves per CU (four
// waves per SIMD).
#include "kernels.h"

namespace delrec {

namespace {

typedef float pk_floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 pk_bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kAcc = 8;
constexpr int kPeakBlock = 512;

}  // namespace

// kind 0: v_mfma_f32_16x16x32_bf16 (16384 flops per instruction); kind 1:
// v_mfma_f32_16x16x4_f32 (2048 flops per instruction)
template <int KIND>
__global__ void __launch_bounds__(kPeakBlock) peak_mfma_kernel(int iters, float* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    pk_floatx4 acc[kAcc];
#pragma unroll
    for (int q = 0; q < kAcc; ++q) acc[q] = pk_floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (KIND == 0) {
        pk_bf16x8 a, b;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            a[e] = (__bf16)(1.0f + 0.001f * (float)(lane + e));
            b[e] = (__bf16)(1.0f - 0.001f * (float)(lane + e));
        }
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int q = 0; q < kAcc; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[q], 0, 0, 0);
        }
    } else {
        const float a = 1.0f + 0.001f * (float)lane, b = 1.0f - 0.001f * (float)lane;
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int q = 0; q < kAcc; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[q], 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < kAcc; ++q) s += acc[q][0] + acc[q][1] + acc[q][2] + acc[q][3];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

int peak_mfma_blocks(int cus) { return 2 * cus; }

double launch_peak_mfma(int kind, int iters, float* sink, int blocks, hipStream_t stream) {
    const double waves = (double)blocks * (kPeakBlock / 64);
    const double per = kind == 0 ? 16384.0 : 2048.0;
    if (kind == 0)
        hipLaunchKernelGGL(peak_mfma_kernel<0>, dim3(blocks), dim3(kPeakBlock), 0, stream, iters, sink);
    else
        hipLaunchKernelGGL(peak_mfma_kernel<1>, dim3(blocks), dim3(kPeakBlock), 0, stream, iters, sink);
    return waves * iters * kAcc * per;
}

}  // namespace delrec
