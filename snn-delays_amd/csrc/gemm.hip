// Reductions over the (t, b) axis of the axonal backward, and the sums of split partials.
//
//   dw_gemm     dW[i,j] = sum_{t,b} gr[t,b,i] * z[t,b,j]: the axonal weight gradient, the
//               reference's host GEMM at recdel_base.py:327-330, on bf16 MFMA with split
//               fp32 operands. 128x128 tiles, split-K into deterministic partials (no
//               atomics), summed by sum_partials.
//   lag_finish  dW, dd (and ds) from the split partials of the lag-correlation GEMM.
#include "kernels.h"

namespace delrec {

typedef float floatx4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDwTile = 128;   // output tile (i and j) per workgroup
constexpr int kDwKt = 32;      // rows of k per stage (one MFMA K)

__device__ __forceinline__ uint32_t dw_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// dW[i, j] = sum_k A[k, i] * Bm[k, j] on bf16 MFMA (v_mfma_f32_16x16x32_bf16) with both fp32
// operands split into bf16 halves, x = hi + lo with hi = bf16(x), lo = bf16(x - hi): each
// tile takes hi*hi + hi*lo + lo*hi (the lo*lo term is below 2^-32 of the product), so a
// product carries a relative error of about 2^-16, accumulated in fp32. 128x128 output
// tile per workgroup (4 waves of 64x64), split over k (blockIdx.z) into deterministic
// partials. Each stage of 32 rows is read from global memory as 8-row runs of one column
// (coalesced across the workgroup's columns), split, and stored in LDS k-blocked -- the 8
// consecutive k of one column as 16 bytes, the run an MFMA lane supplies -- while the
// previous stage is multiplied.
// MFMA lane layout: lane l supplies A[l%16][8g .. 8g+7], B[8g .. 8g+7][l%16] (g = l/16, the
// same k order for both operands); accumulator register r of lane l holds D[4g + r][l%16].
__global__ void __launch_bounds__(256) dw_gemm_kernel(const float* __restrict__ A,
                                                      const float* __restrict__ Bm, int K, int N,
                                                      int kchunk, float* __restrict__ partial) {
    // [buffer][operand A/B][hi/lo][k block][column] of 16-byte runs
    __shared__ uint4 sm[2][2][2][kDwKt / 8][kDwTile];
    const int i0 = blockIdx.x * kDwTile, j0 = blockIdx.y * kDwTile, ks = blockIdx.z;
    const int kb = ks * kchunk, ke = min(K, kb + kchunk);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1;
    const int g = lane >> 4, lc = lane & 15;
    // staging: per operand 4 k-blocks x 128 columns = 512 runs, two per thread
    const int col = tid & (kDwTile - 1), kq = tid >> 7;

    floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    float ra[2][8], rb[2][8];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int kbase = k0 + (kq + 2 * h) * 8;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = kbase + e;
                const bool kin = k < ke;
                ra[h][e] = (kin && i0 + col < N) ? A[(size_t)k * N + i0 + col] : 0.0f;
                rb[h][e] = (kin && j0 + col < N) ? Bm[(size_t)k * N + j0 + col] : 0.0f;
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t ah[4], al[4], bh[4], bl[4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const uint32_t a0 = dw_bf16_bits(ra[h][e]), a1 = dw_bf16_bits(ra[h][e + 1]);
                const uint32_t b0 = dw_bf16_bits(rb[h][e]), b1 = dw_bf16_bits(rb[h][e + 1]);
                ah[e / 2] = a0 | (a1 << 16);
                bh[e / 2] = b0 | (b1 << 16);
                al[e / 2] = dw_bf16_bits(ra[h][e] - __uint_as_float(a0 << 16)) |
                            (dw_bf16_bits(ra[h][e + 1] - __uint_as_float(a1 << 16)) << 16);
                bl[e / 2] = dw_bf16_bits(rb[h][e] - __uint_as_float(b0 << 16)) |
                            (dw_bf16_bits(rb[h][e + 1] - __uint_as_float(b1 << 16)) << 16);
            }
            const int kbk = kq + 2 * h;
            sm[buf][0][0][kbk][col] = uint4{ah[0], ah[1], ah[2], ah[3]};
            sm[buf][0][1][kbk][col] = uint4{al[0], al[1], al[2], al[3]};
            sm[buf][1][0][kbk][col] = uint4{bh[0], bh[1], bh[2], bh[3]};
            sm[buf][1][1][kbk][col] = uint4{bl[0], bl[1], bl[2], bl[3]};
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
        bf16x8 fah[4], fal[4], fbh[4], fbl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            fah[q] = __builtin_bit_cast(bf16x8, sm[buf][0][0][g][wi * 64 + q * 16 + lc]);
            fal[q] = __builtin_bit_cast(bf16x8, sm[buf][0][1][g][wi * 64 + q * 16 + lc]);
            fbh[q] = __builtin_bit_cast(bf16x8, sm[buf][1][0][g][wj * 64 + q * 16 + lc]);
            fbl[q] = __builtin_bit_cast(bf16x8, sm[buf][1][1][g][wj * 64 + q * 16 + lc]);
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fah[a], fbh[c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fah[a], fbl[c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fal[a], fbh[c], acc[a][c], 0, 0, 0);
            }
        if (more) stash(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    float* P = partial + (size_t)ks * N * N;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + wi * 64 + a * 16 + 4 * g + r;
                const int j = j0 + wj * 64 + c * 16 + lc;
                if (i < N && j < N) P[(size_t)i * N + j] = acc[a][c][r];
            }
}

// out[idx] = sum_k partial[k][idx]. A workgroup owns 64 float4 of the output; wave w sums
// the partials k = w, w + 4, ... (loads issued together), and wave 0 adds the four in
// order, so the result does not depend on timing.
__global__ void __launch_bounds__(256) sum_partials_kernel(const float* __restrict__ partial, int ks,
                                                           size_t count, float* __restrict__ out) {
    __shared__ float4 red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t idx = ((size_t)blockIdx.x * 64 + lane) * 4;
    const bool full = idx + 4 <= count;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    if (full) {
        int k = w;
        for (; k + 12 < ks; k += 16) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[u] = *reinterpret_cast<const float4*>(partial + (size_t)(k + 4 * u) * count + idx);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
            }
        }
        for (; k < ks; k += 4) {
            const float4 v = *reinterpret_cast<const float4*>(partial + (size_t)k * count + idx);
            acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
        }
    } else {
        float t4[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = w; k < ks; k += 4)
            for (int e = 0; e < 4; ++e)
                if (idx + e < count) t4[e] += partial[(size_t)k * count + idx + e];
        acc = float4{t4[0], t4[1], t4[2], t4[3]};
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w == 0) {
        float4 r = red[0][lane];
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            r.x += red[q][lane].x; r.y += red[q][lane].y; r.z += red[q][lane].z; r.w += red[q][lane].w;
        }
        if (full) {
            *reinterpret_cast<float4*>(out + idx) = r;
        } else {
            const float rr[4] = {r.x, r.y, r.z, r.w};
            for (int e = 0; e < 4; ++e)
                if (idx + e < count) out[idx + e] = rr[e];
        }
    }
}

void launch_dw_gemm(const float* A, const float* Bm, int K, int N, int ks, float* partial,
                    hipStream_t stream) {
    const int tiles = (N + kDwTile - 1) / kDwTile;
    const int kchunk = ((K + ks - 1) / ks + kDwKt - 1) / kDwKt * kDwKt;   // whole stages
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
#pragma unroll 8
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
