// Device bodies of the axonal weight gradient and of the sums of split partials, shared by
// the launches that run them beside other reductions of the backward.
//
//   dw_gemm_tile   dW[i,j] = sum_{t,b} gr[t,b,i] * z[t,b,j]: the reference's host GEMM at
//                  recdel_base.py:327-330, on bf16 MFMA with three-term fp32 operands; one
//                  128x128 output tile over one k chunk per workgroup, written as a
//                  deterministic partial (no atomics).
//   sum_partials_block  out[idx] = sum_k partial[k][idx] in a fixed order.
#pragma once

#include "kernels.h"

namespace delrec {

typedef float dw_floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 dw_bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDwTile = 128;   // output tile (i and j) per workgroup
constexpr int kDwKt = 32;      // rows of k per stage (one MFMA K)
constexpr int kDwThreads = 256;

// LDS of one stage: [operand A/B][hi/mid/lo][k block][column] of 16-byte runs (48 KiB)
struct DwStage {
    uint4 v[2][3][kDwKt / 8][kDwTile];
};

__device__ __forceinline__ uint32_t dw_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// dW[i, j] = sum_k A[k, i] * Bm[k, j] on bf16 MFMA (v_mfma_f32_16x16x32_bf16) with both fp32
// operands split into three bf16 terms, x = hi + mid + lo with hi = bf16(x),
// mid = bf16(x - hi), lo = bf16(x - hi - mid) (x is held to about 2^-27): each tile takes
// the six products whose order is at least 2^-16 of the whole (hi*hi, hi*mid, mid*hi,
// hi*lo, mid*mid, lo*hi), dropping mid*lo, lo*mid and lo*lo (about 2^-24 together), so a
// product is as accurate as an fp32 one, accumulated in fp32. Tile (ti, tj) of
// 128x128 outputs (4 waves of 64x64) over k chunk kz. Each stage of 32 rows is read from
// global memory as 8-row runs of one column (coalesced across the workgroup's columns) into
// registers while the previous stage is multiplied, then split and stored in LDS k-blocked
// -- the 8 consecutive k of one column as 16 bytes, the run an MFMA lane supplies.
// MFMA lane layout: lane l supplies A[l%16][8g .. 8g+7], B[8g .. 8g+7][l%16] (g = l/16, the
// same k order for both operands); accumulator register r of lane l holds D[4g + r][l%16].
__device__ __forceinline__ void dw_gemm_tile(const float* __restrict__ A, const float* __restrict__ Bm,
                                             int K, int N, int kchunk, float* __restrict__ partial,
                                             int ti, int tj, int kz, DwStage& sm) {
    const int i0 = ti * kDwTile, j0 = tj * kDwTile;
    const int kb = kz * kchunk, ke = min(K, kb + kchunk);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1;
    const int g = lane >> 4, lc = lane & 15;
    // staging: per operand 4 k-blocks x 128 columns = 512 runs, two per thread
    const int col = tid & (kDwTile - 1), kq = tid >> 7;

    dw_floatx4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = dw_floatx4{0.f, 0.f, 0.f, 0.f};

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
    // x = hi + mid + lo as the bf16 bit patterns of one pair of consecutive k
    auto split3 = [](float x0, float x1, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
        const uint32_t h0 = dw_bf16_bits(x0), h1 = dw_bf16_bits(x1);
        const float r0 = x0 - __uint_as_float(h0 << 16), r1 = x1 - __uint_as_float(h1 << 16);
        const uint32_t m0 = dw_bf16_bits(r0), m1 = dw_bf16_bits(r1);
        const uint32_t l0 = dw_bf16_bits(r0 - __uint_as_float(m0 << 16));
        const uint32_t l1 = dw_bf16_bits(r1 - __uint_as_float(m1 << 16));
        hi = h0 | (h1 << 16);
        mid = m0 | (m1 << 16);
        lo = l0 | (l1 << 16);
    };
    auto stash = [&]() {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t a3[3][4], b3[3][4];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                split3(ra[h][e], ra[h][e + 1], a3[0][e / 2], a3[1][e / 2], a3[2][e / 2]);
                split3(rb[h][e], rb[h][e + 1], b3[0][e / 2], b3[1][e / 2], b3[2][e / 2]);
            }
            const int kbk = kq + 2 * h;
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                sm.v[0][q][kbk][col] = uint4{a3[q][0], a3[q][1], a3[q][2], a3[q][3]};
                sm.v[1][q][kbk][col] = uint4{b3[q][0], b3[q][1], b3[q][2], b3[q][3]};
            }
        }
    };

    if (kb < ke) {
        fetch(kb);
        stash();
    }
    __syncthreads();
    for (int k0 = kb; k0 < ke; k0 += kDwKt) {
        const bool more = k0 + kDwKt < ke;
        if (more) fetch(k0 + kDwKt);
        dw_bf16x8 fa[3][4], fb[3][4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                fa[pl][q] = __builtin_bit_cast(dw_bf16x8, sm.v[0][pl][g][wi * 64 + q * 16 + lc]);
                fb[pl][q] = __builtin_bit_cast(dw_bf16x8, sm.v[1][pl][g][wj * 64 + q * 16 + lc]);
            }
        // every wave holds its fragments in registers before the stage is overwritten
        __syncthreads();
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[0][a], fb[2][c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[1][a], fb[1][c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[2][a], fb[0][c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[0][a], fb[1][c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[1][a], fb[0][c], acc[a][c], 0, 0, 0);
                acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[0][a], fb[0][c], acc[a][c], 0, 0, 0);
            }
        if (more) stash();
        __syncthreads();
    }
    float* P = partial + (size_t)kz * N * N;
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

// out[idx] = sum_k partial[k][idx] over the 64 float4 of block `blk` (256 threads): wave w
// sums the partials k = w, w + 4, ... (eight loads issued together), and wave 0 adds the four in
// order, so the result does not depend on timing.
__device__ __forceinline__ void sum_partials_block(const float* __restrict__ partial, int ks, size_t count,
                                                   float* __restrict__ out, int blk, float4 (&red)[4][64]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t idx = ((size_t)blk * 64 + lane) * 4;
    const bool full = idx + 4 <= count;
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    if (full) {
        int k = w;
        for (; k + 28 < ks; k += 32) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = *reinterpret_cast<const float4*>(partial + (size_t)(k + 4 * u) * count + idx);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
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

}  // namespace delrec
