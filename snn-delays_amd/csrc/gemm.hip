// MFMA (fp32, v_mfma_f32_16x16x4f32) reductions over the (t, b) axis of the backward.
//
//   dw_gemm     dW[i,j] = sum_{t,b} gr[t,b,i] * z[t,b,j]: the axonal weight gradient, the
//               reference's host GEMM at recdel_base.py:327-330. 128x128 tiles, split-K
//               into deterministic partials (no atomics), summed by sum_partials.
//   lag_finish  dW, dd (and ds) from the split partials of the lag-correlation GEMM.
//
// MFMA 16x16x4 f32 operand layout (wave64): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; accumulator register r of lane l holds D[4*(l/16) + r][l%16].
#include "kernels.h"

namespace delrec {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kDwTile = 64;
constexpr int kDwKt = 32;
constexpr int kDwPitch = kDwTile + 4;

// 64x64 output tile per workgroup (4 waves of 32x32, 2x2 MFMA blocks each); the K range
// of the split is staged through two LDS buffers 32 rows at a time, the next stage's
// global loads (float4) held in registers while the current stage is multiplied.
__global__ void __launch_bounds__(256) dw_gemm_kernel(const float* __restrict__ A,
                                                      const float* __restrict__ Bm, int K, int N,
                                                      int kchunk, float* __restrict__ partial) {
    __shared__ float sA[2][kDwKt][kDwPitch];
    __shared__ float sB[2][kDwKt][kDwPitch];
    const int i0 = blockIdx.x * kDwTile, j0 = blockIdx.y * kDwTile, ks = blockIdx.z;
    const int kb = ks * kchunk, ke = min(K, kb + kchunk);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wi = w >> 1, wj = w & 1;
    const int lr = lane >> 4, lc = lane & 15;
    const bool vec = (N & 3) == 0;
    // staging assignment: 32 rows x 16 float4 per matrix = 512 float4, 2 per thread
    const int r0 = threadIdx.x >> 4, c4 = (threadIdx.x & 15) * 4;
    floatx4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[a][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    float4 ra[2], rb[2];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = k0 + r0 + 16 * h;
            const bool kin = k < ke;
            if (vec) {
                ra[h] = (kin && i0 + c4 < N) ? *reinterpret_cast<const float4*>(A + (size_t)k * N + i0 + c4)
                                             : float4{0.f, 0.f, 0.f, 0.f};
                rb[h] = (kin && j0 + c4 < N) ? *reinterpret_cast<const float4*>(Bm + (size_t)k * N + j0 + c4)
                                             : float4{0.f, 0.f, 0.f, 0.f};
            } else {
                float a4[4], b4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a4[e] = (kin && i0 + c4 + e < N) ? A[(size_t)k * N + i0 + c4 + e] : 0.0f;
                    b4[e] = (kin && j0 + c4 + e < N) ? Bm[(size_t)k * N + j0 + c4 + e] : 0.0f;
                }
                ra[h] = float4{a4[0], a4[1], a4[2], a4[3]};
                rb[h] = float4{b4[0], b4[1], b4[2], b4[3]};
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<float4*>(&sA[buf][r0 + 16 * h][c4]) = ra[h];
            *reinterpret_cast<float4*>(&sB[buf][r0 + 16 * h][c4]) = rb[h];
        }
    };

    int buf = 0;
    if (kb < ke) {
        fetch(kb);
        stash(0);
    }
    __syncthreads();
    for (int k0 = kb; k0 < ke; k0 += kDwKt) {
        const bool more = k0 + kDwKt < ke;
        if (more) fetch(k0 + kDwKt);
#pragma unroll
        for (int kk = 0; kk < kDwKt; kk += 4) {
            float av[2], bv[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                av[q] = sA[buf][kk + lr][wi * 32 + q * 16 + lc];
                bv[q] = sB[buf][kk + lr][wj * 32 + q * 16 + lc];
            }
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a], bv[c], acc[a][c], 0, 0, 0);
        }
        if (more) stash(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    float* P = partial + (size_t)ks * N * N;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + wi * 32 + a * 16 + 4 * lr + r;
                const int j = j0 + wj * 32 + c * 16 + lc;
                if (i < N && j < N) P[(size_t)i * N + j] = acc[a][c][r];
            }
}

__global__ void sum_partials_kernel(const float* __restrict__ partial, int ks, size_t count,
                                    float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= count) return;
    float acc = 0.0f;
    for (int k = 0; k < ks; ++k) acc += partial[(size_t)k * count + idx];
    out[idx] = acc;
}

void launch_dw_gemm(const float* A, const float* Bm, int K, int N, int ks, float* partial,
                    hipStream_t stream) {
    const int tiles = (N + kDwTile - 1) / kDwTile;
    const int kchunk = (K + ks - 1) / ks;
    hipLaunchKernelGGL(dw_gemm_kernel, dim3(tiles, tiles, ks), dim3(256), 0, stream, A, Bm, K,
                       N, kchunk, partial);
}

void launch_sum_partials(const float* partial, int ks, size_t count, float* out, hipStream_t stream) {
    const unsigned blocks = (unsigned)((count + 255) / 256);
    hipLaunchKernelGGL(sum_partials_kernel, dim3(blocks), dim3(256), 0, stream, partial, ks, count, out);
}

// ---------------------------------------------------------------------------------------
// Sums of the lag-GEMM partials (lagmm.hip) into dW, dd and ds.
__global__ void lag_finish_kernel(LagGemm p, float* dW, float* dd) {
    const size_t NN = (size_t)p.N * p.N;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= NN) return;
    float aw = 0.0f, ad = 0.0f;
    for (int k = 0; k < p.KS; ++k) {
        aw += p.pw[(size_t)k * NN + idx];
        if (p.pd) ad += p.pd[(size_t)k * NN + idx];
    }
    if (dW) dW[idx] = aw;
    if (dd) {
        const int j = (int)(idx % p.N);
        const float s = p.s ? p.s[j] : p.s_uniform;
        dd[idx] = load_w(p.W, p.w_bf16, idx) * (ad / (s * s));
    }
}

__global__ void lag_ds_kernel(LagGemm p, float* ds) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= p.N) return;
    const size_t NN = (size_t)p.N * p.N;
    float acc = 0.0f;
    for (int i = 0; i < p.N; ++i) {
        float c = 0.0f;
        for (int k = 0; k < p.KS; ++k) c += p.ps[(size_t)k * NN + (size_t)i * p.N + j];
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

}  // namespace delrec
