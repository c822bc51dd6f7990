// Sums of the lag-correlation GEMM's split partials and the dense delay-gradient epilogue.
//
//   lag_finish  dW, dd (and ds) from the split partials of the lag-correlation GEMM.
//   max_to_host the maximum of a device vector, written straight into pinned host memory.
//   (The axonal dW GEMM and its partial sums are device bodies in dw_gemm.h, launched
//   beside the other reductions of the axonal backward in axonal.hip.)
#include "common.h"
#include "kernels.h"

namespace delrec {

// ---------------------------------------------------------------------------------------
// Sums of the lag-GEMM partials (lagmm.hip) into dW, dd and ds.
__global__ void lag_finish_kernel(LagGemm p, float* dW, float* dd) {
    const size_t NN = (size_t)p.N * p.N;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= NN) return;
    // the partials' column position -> the column (the event-driven correlation's order);
    // there, silent columns' sums are 0 and the sparse tiles' columns hold one partial per
    // 64-row chunk (the even ones)
    const int jp = (int)(idx % p.N);
    int k0 = 0, kd = 1;
    if (p.cls) {
        if (jp < p.cls[0]) k0 = p.KS;
        else if (jp < (p.cls[0] + p.cls[1]) / 64 * 64) kd = 2;
    }
    float aw = 0.0f, ad = 0.0f;
#pragma unroll 8
    for (int k = k0; k < p.KS; k += kd) {
        aw += p.pw[(size_t)k * NN + idx];
        if (p.pd) ad += p.pd[(size_t)k * NN + idx];
    }
    const int j = p.perm ? p.perm[jp] : jp;
    const size_t out = idx - jp + j;
    if (dW) dW[out] = aw;
    if (dd) {
        const float s = p.s ? p.s[j] : p.s_uniform;
        dd[out] = load_w(p.W, p.w_bf16, out) * (ad / (s * s));
    }
}

__global__ void lag_ds_kernel(LagGemm p, float* ds) {
    const int jp = blockIdx.x * blockDim.x + threadIdx.x;
    if (jp >= p.N) return;
    const int j = p.perm ? p.perm[jp] : jp;
    const size_t NN = (size_t)p.N * p.N;
    int k0 = 0, kd = 1;   // as lag_finish_kernel
    if (p.cls) {
        if (jp < p.cls[0]) k0 = p.KS;
        else if (jp < (p.cls[0] + p.cls[1]) / 64 * 64) kd = 2;
    }
    float acc = 0.0f;
    for (int i = 0; i < p.N; ++i) {
        float c = 0.0f;
        for (int k = k0; k < p.KS; k += kd) c += p.ps[(size_t)k * NN + (size_t)i * p.N + jp];
        acc += load_w(p.W, p.w_bf16, (size_t)i * p.N + j) * c;
    }
    ds[j] = acc;
}

void launch_lag_finish(const LagGemm& a, float* dW, float* dd, float* ds, hipStream_t stream) {
    const size_t NN = (size_t)a.N * a.N;
    hipLaunchKernelGGL(lag_finish_kernel, dim3((unsigned)((NN + 255) / 256)), dim3(256), 0, stream,
                       a, dW, dd);
    if (ds && a.ps)
        hipLaunchKernelGGL(lag_ds_kernel, dim3((a.N + 255) / 256), dim3(256), 0, stream, a, ds);
}

// ---------------------------------------------------------------------------------------
// Closed-form delay gradient on an explicit lag stack (the reference's _delay_grad hook).
__global__ void delay_grad_kernel(const float* C, const float* W, const float* d, float s, int N,
                                  int Lm, float* dd) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)N * N) return;
    const float c = 1.0f + d[idx];
    float acc = 0.0f;
    for (int l = 1; l < Lm; ++l) acc += tri_dsign((float)l, c, s) * C[idx * Lm + l];
    dd[idx] = W[idx] * (acc / (s * s));
}

void launch_delay_grad(const float* C, const float* W, const float* d, float sigma, int N, int Lm,
                       float* dd, hipStream_t stream) {
    const size_t NN = (size_t)N * N;
    hipLaunchKernelGGL(delay_grad_kernel, dim3((unsigned)((NN + 255) / 256)), dim3(256), 0, stream,
                       C, W, d, 1.0f + sigma, N, Lm, dd);
}

// ---------------------------------------------------------------------------------------
// max(x[0 .. n)) into a slot of pinned host memory (delrec_max_post): one workgroup.
__global__ void __launch_bounds__(256) max_to_host_kernel(const float* __restrict__ x, int n, uint32_t ticket,
                                                          unsigned long long* slot) {
    block_max_to_host(x, n, ticket, slot);
}

void launch_max_to_host(const float* x, int n, uint32_t ticket, unsigned long long* slot, hipStream_t stream) {
    hipLaunchKernelGGL(max_to_host_kernel, dim3(1), dim3(256), 0, stream, x, n, ticket, slot);
}

}  // namespace delrec
