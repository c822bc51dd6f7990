// Lag-correlation GEMM of the synaptic / hybrid backward on bf16 MFMA (gfx950).
//
// The weight and delay gradients of a per-connection delay need, for every lag l in the
// window, C_l[i,j] = sum_{t,b} gr[t+l, b, i] * y[t, b, j] (the reference materialises the
// (N, N, L) stack of these, synaptic_eventdriven.py:441-468, synaptic_hybrid.py:196-208).
// Here every C_l is produced tile by tile on MFMA and folded at once into
//   pw[i,j] += h(l; d_ij, s_j) C_l[i,j]      (dW)
//   pd[i,j] += sign(l-1-d_ij)[|l-1-d_ij| <= s_j] C_l[i,j]      (dd, before W/s^2)
//   ps[i,j] += dh/ds(l; d_ij, s_j) C_l[i,j]  (use_sig_p)
// so the stack never exists.
//
// Operands are bf16. Spikes are exactly 0 or 1 in bf16. gr is split into gr_hi =
// bf16(gr) and gr_lo = bf16(gr - gr_hi), and each tile takes both products, so a term
// carries a relative error below 2^-16 of gr (fp32 accumulation). The packed operands use
// a k-blocked layout, element (k, m) at ((k / 8) * Np + m) * 8 + k % 8, so one 16-byte load
// holds the 8 consecutive k of one column that an MFMA lane supplies; a row k is
// (t * Bp + b) with the batch padded to Bp = 8n, so a time shift is a whole number of
// blocks.
//
// Relative lags: column j's spike train is stored shifted by its first lag lo_j,
// Y'[t, b, j] = y[t - lo_j, b, j], and the kernel walks r = 0 .. R-1 with l = lo_j + r.
// Synaptic delays use lo_j = 1, R = L - 1 (every lag). A hybrid delay base[j] + offset[i,j]
// with integer offsets puts every connection of column j within R = (max - min offset) +
// ceil(2s) + 4 lags of lo_j, so the hybrid runs R instead of L - 1 lags.
//
// MFMA v_mfma_f32_16x16x32_bf16 (wave64): lane l supplies A[l%16][8g .. 8g+7] and
// B[8g .. 8g+7][l%16] with g = l/16 (the same k order for A and B); accumulator register r
// of lane l holds D[4g + r][l%16].
#include "kernels.h"

namespace delrec {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kLT = 128;   // output tile (i and j) per workgroup
constexpr int kLK = 32;    // rows of k per stage
constexpr int kLKB = kLK / 8;

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// gr (T, B, N) fp32 -> gr_hi, gr_lo in the k-blocked layout (Kp rows, Np columns; padding
// rows and columns are zero).
__global__ void pack_gr_kernel(const float* __restrict__ gr, int T, int B, int Bp, int N, int Np,
                               int Kp, uint4* __restrict__ hi, uint4* __restrict__ lo) {
    const size_t total = (size_t)(Kp / 8) * Np;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int kb = (int)(q / Np), m = (int)(q - (size_t)kb * Np);
        uint32_t h[4], l[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            float v[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int k = kb * 8 + e + f;
                const int t = k / Bp, b = k - (k / Bp) * Bp;
                v[f] = (t < T && b < B && m < N) ? gr[((size_t)t * B + b) * N + m] : 0.0f;
            }
            const uint32_t h0 = bf16_rne_bits(v[0]), h1 = bf16_rne_bits(v[1]);
            const uint32_t l0 = bf16_rne_bits(v[0] - __uint_as_float(h0 << 16));
            const uint32_t l1 = bf16_rne_bits(v[1] - __uint_as_float(h1 << 16));
            h[e / 2] = h0 | (h1 << 16);
            l[e / 2] = l0 | (l1 << 16);
        }
        hi[q] = uint4{h[0], h[1], h[2], h[3]};
        lo[q] = uint4{l[0], l[1], l[2], l[3]};
    }
}

// spike bits (B, ceil(T/32), N) -> Y'[t, b, j] = y[t - lo_j, b, j] in bf16 (1.0 = 0x3F80),
// k-blocked; lo == NULL means lo_j = 1.
__global__ void pack_spikes_kernel(const uint32_t* __restrict__ bits, const int* __restrict__ lo,
                                   int T, int B, int Bp, int N, int Np, int Kp,
                                   uint4* __restrict__ out) {
    const int TW = (T + 31) >> 5;
    const size_t total = (size_t)(Kp / 8) * Np;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int kb = (int)(q / Np), j = (int)(q - (size_t)kb * Np);
        const int shift = (j < N) ? (lo ? lo[j] : 1) : 0;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t v[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int k = kb * 8 + e + f;
                const int t = k / Bp, b = k - (k / Bp) * Bp;
                const int ts = t - shift;
                bool on = false;
                if (j < N && t < T && b < B && ts >= 0)
                    on = (bits[((size_t)b * TW + (ts >> 5)) * N + j] >> (ts & 31)) & 1u;
                v[f] = on ? 0x3F80u : 0u;
            }
            w[e / 2] = v[0] | (v[1] << 16);
        }
        out[q] = uint4{w[0], w[1], w[2], w[3]};
    }
}

// Hybrid lag range: one workgroup reduces the offsets to their min / max, then writes the
// number of relative lags R (meta[0]), the smallest offset (meta[1]) and each column's
// first lag lo_j.
__global__ void __launch_bounds__(1024) lag_range_kernel(const int8_t* __restrict__ off,
                                                         const float* __restrict__ base, int N, int L,
                                                         float s, int* __restrict__ meta,
                                                         int* __restrict__ lo) {
    __shared__ int smin[16], smax[16];
    __shared__ int s_omin, s_full;
    const size_t NN = (size_t)N * N;
    int mn = 127, mx = -128;
    for (size_t q = threadIdx.x; q < NN; q += blockDim.x) {
        const int v = off[q];
        mn = min(mn, v);
        mx = max(mx, v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        mn = min(mn, __shfl_xor(mn, o));
        mx = max(mx, __shfl_xor(mx, o));
    }
    if ((threadIdx.x & 63) == 0) {
        smin[threadIdx.x >> 6] = mn;
        smax[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int a = 127, z = -128;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
            a = min(a, smin[w]);
            z = max(z, smax[w]);
        }
        int R = (z - a) + (int)ceilf(2.0f * s) + 4;
        const bool full = R >= L - 1;
        if (full) R = L - 1;
        meta[0] = max(R, 1);
        meta[1] = a;
        s_omin = a;
        s_full = full ? 1 : 0;
    }
    __syncthreads();
    const int omin = s_omin;
    const bool full = s_full != 0;
    for (int j = threadIdx.x; j < N; j += blockDim.x)
        lo[j] = full ? 1 : max(1, (int)floorf(1.0f + base[j] + (float)omin - s) - 1);
}

__device__ __forceinline__ float lag_conn_delay(const LagBf16& p, int i, int j) {
    if (p.d) return p.d[(size_t)i * p.N + j];
    return p.base[j] + 0.0f + 1.0f * (float)p.off[(size_t)i * p.N + j];
}

// 128x128 output tile per workgroup, 4 waves of 64x64 (4x4 MFMA blocks), split over k
// (blockIdx.z). Per relative lag r: the k range of the split (rows k < (T - r) * Bp) is
// staged through two LDS buffers 32 rows at a time (gr_hi, gr_lo shifted by r * Bp rows,
// Y' unshifted), the next stage's 16-byte global loads held in registers meanwhile; then
// the tile of C_{lo_j + r} is folded into the per-element sums.
constexpr int kCP = kLT + 4;   // pitch of the delay tile in LDS (conflict-free epilogue reads)

template <bool DS>
__global__ void __launch_bounds__(256) lag_bf16_kernel(LagBf16 p) {
    __shared__ uint4 sbuf[2][3][kLKB * kLT];
    __shared__ float scc[kLT * kCP];        // 1 + d_ij of the tile
    const int N = p.N, Np = p.Np, T = p.T, Bp = p.Bp;
    const int i0 = blockIdx.x * kLT, j0 = blockIdx.y * kLT;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1;
    const int g = lane >> 4, lc = lane & 15;
    const int R = p.meta ? p.meta[0] : p.R;
    const int steps_all = (T * Bp + kLK - 1) / kLK;
    const int per = (steps_all + (int)gridDim.z - 1) / (int)gridDim.z;
    const int sb = (int)blockIdx.z * per, se = min(steps_all, sb + per);

    for (int q = tid; q < kLT * kLT; q += 256) {
        const int ii = q >> 7, jj = q & (kLT - 1);
        const int i = i0 + ii, j = j0 + jj;
        scc[ii * kCP + jj] = (i < N && j < N) ? 1.0f + lag_conn_delay(p, i, j) : 0.0f;
    }
    // this lane's output elements: i = i0 + wi*64 + mb*16 + 4g + e, j = j0 + wj*64 + nb*16 + lc
    float sj[4];
    int loj[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        const int j = j0 + wj * 64 + nb * 16 + lc;
        const int jc = j < N ? j : 0;
        sj[nb] = p.s ? p.s[jc] : p.s_uniform;
        loj[nb] = p.lo ? p.lo[jc] : 1;
    }
    float ow[4][4][4], od[4][4][4], os[DS ? 4 : 1][4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ow[mb][nb][e] = 0.0f;
                od[mb][nb][e] = 0.0f;
                if (DS) os[DS ? mb : 0][nb][e] = 0.0f;
            }

    // staging: each operand stage is kLKB * kLT = 512 uint4, two per thread
    uint4 st[3][2];
    auto fetch = [&](int step, size_t ashift_blocks) {
        const size_t kb0 = (size_t)step * kLKB;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = tid + h * 256;
            const int kb = c >> 7, m = c & (kLT - 1);
            st[0][h] = p.ahi[(kb0 + ashift_blocks + kb) * Np + i0 + m];
            st[1][h] = p.alo[(kb0 + ashift_blocks + kb) * Np + i0 + m];
            st[2][h] = p.yb[(kb0 + kb) * Np + j0 + m];
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = tid + h * 256;
            sbuf[buf][0][c] = st[0][h];
            sbuf[buf][1][c] = st[1][h];
            sbuf[buf][2][c] = st[2][h];
        }
    };

    for (int r = 0; r < R; ++r) {
        const int kend = (T - r) * Bp;              // rows k with t + r < T
        const int se_r = min(se, (kend + kLK - 1) / kLK);
        if (se_r <= sb) break;                      // later lags have fewer rows still
        const size_t ashift = (size_t)r * (Bp / 8); // blocks of the gr shift r * Bp
        floatx4 acc[4][4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

        fetch(sb, ashift);
        stash(0);
        __syncthreads();
        int buf = 0;
        for (int step = sb; step < se_r; ++step) {
            const bool more = step + 1 < se_r;
            if (more) fetch(step + 1, ashift);
            bf16x8 ah[4], al[4], bv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                ah[q] = __builtin_bit_cast(bf16x8, sbuf[buf][0][g * kLT + wi * 64 + q * 16 + lc]);
                al[q] = __builtin_bit_cast(bf16x8, sbuf[buf][1][g * kLT + wi * 64 + q * 16 + lc]);
                bv[q] = __builtin_bit_cast(bf16x8, sbuf[buf][2][g * kLT + wj * 64 + q * 16 + lc]);
            }
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int nb = 0; nb < 4; ++nb) {
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[mb], bv[nb], acc[mb][nb], 0, 0, 0);
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[mb], bv[nb], acc[mb][nb], 0, 0, 0);
                }
            if (more) stash(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }

        // fold C_l, l = lo_j + r, into the per-element sums (lags past L - 1 do not exist)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const int l = loj[nb] + r;
            const float lf = (float)l;
            const bool in = l <= p.L - 1;
            const float sv = sj[nb], s2 = sv * sv;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float C = in ? acc[mb][nb][e] : 0.0f;
                    const float cv = scc[(wi * 64 + mb * 16 + 4 * g + e) * kCP + wj * 64 + nb * 16 + lc];
                    ow[mb][nb][e] += tri_weight(lf, cv, sv, s2) * C;
                    od[mb][nb][e] += tri_dsign(lf, cv, sv) * C;
                    if (DS) os[DS ? mb : 0][nb][e] += tri_ds(lf, cv, sv, s2) * C;
                }
        }
    }

    const size_t NN = (size_t)N * N;
    const size_t base_o = (size_t)blockIdx.z * NN;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = i0 + wi * 64 + mb * 16 + 4 * g + e;
                const int j = j0 + wj * 64 + nb * 16 + lc;
                if (i >= N || j >= N) continue;
                const size_t o = base_o + (size_t)i * N + j;
                p.pw[o] = ow[mb][nb][e];
                p.pd[o] = od[mb][nb][e];
                if (DS) p.ps[o] = os[DS ? mb : 0][nb][e];
            }
}

void launch_lag_range(const int8_t* off, const float* base, int N, int L, float s, int* meta, int* lo,
                      hipStream_t stream) {
    hipLaunchKernelGGL(lag_range_kernel, dim3(1), dim3(1024), 0, stream, off, base, N, L, s, meta, lo);
}

int lag_bf16_splits(int T, int Bp, int Np, int cus) {
    const int tiles = (Np / kLT) * (Np / kLT);
    const int steps = (T * Bp + kLK - 1) / kLK;
    const int want = (cus + tiles - 1) / tiles;
    return std::max(1, std::min(want, steps / 8 > 0 ? steps / 8 : 1));
}

void launch_lag_bf16(const LagBf16& a, const float* gr, const uint32_t* bits, hipStream_t stream) {
    const size_t total = (size_t)(a.Kp / 8) * a.Np;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(pack_gr_kernel, dim3(blocks), dim3(256), 0, stream, gr, a.T, a.B, a.Bp, a.N,
                       a.Np, a.Kp, const_cast<uint4*>(a.ahi), const_cast<uint4*>(a.alo));
    hipLaunchKernelGGL(pack_spikes_kernel, dim3(blocks), dim3(256), 0, stream, bits, a.lo, a.T, a.B,
                       a.Bp, a.N, a.Np, a.Kp, const_cast<uint4*>(a.yb));
    const dim3 grid(a.Np / kLT, a.Np / kLT, a.KS);
    if (a.ps)
        hipLaunchKernelGGL(lag_bf16_kernel<true>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(lag_bf16_kernel<false>, grid, dim3(256), 0, stream, a);
}

}  // namespace delrec
