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
// Operands are bf16. Spikes are exactly 0 or 1 in bf16. gr is split into three terms,
// gr_hi = bf16(gr), gr_mid = bf16(gr - gr_hi), gr_lo = bf16(gr - gr_hi - gr_mid), and each
// tile takes all three products, so a term is as accurate as gr itself in fp32 (the
// split holds gr to about 2^-27; fp32 accumulation). For bf16 W the weight gradient leaves
// as bf16 (rounded to 2^-9) and the tiles take hi and mid only (gr to about 2^-17 per term,
// 2^8 times finer than that rounding): a third fewer products. The packed operands use
// a k-blocked layout, element (k, m) at ((k / 8) * Np + m) * 8 + k % 8, so one 16-byte load
// holds the 8 consecutive k of one column that an MFMA lane supplies; a row k is
// (t * Bp + b) with the batch padded to a multiple of 32, so a 32-row batch chunk of one
// time step is 4 whole k-blocks.
//
// Relative lags: column j's spike train is stored shifted by its first lag lo_j,
// Y'[t, b, j] = y[t - lo_j, b, j], and the kernel walks r = 0 .. R-1 with l = lo_j + r, where
// [lo_j, lo_j + R_j) is the exact range of lags on the triangle support of some connection
// of column j and R is the widest R_j of a 64-column tile (hybrid: (max - min offset) +
// 2s, give or take one; synaptic: up to L - 1).
//
// MFMA v_mfma_f32_16x16x32_bf16 (wave64): lane l supplies A[l%16][8g .. 8g+7] and
// B[8g .. 8g+7][l%16] with g = l/16 (the same k order for A and B); accumulator register r
// of lane l holds D[4g + r][l%16].
#include "kernels.h"

namespace delrec {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// gr (T, B, N) fp32 -> gr_hi, gr_mid, gr_lo in the k-blocked layout (Kp rows, Np columns;
// padding rows and columns are zero); lo == NULL skips the third plane (two-plane tiles).
__global__ void pack_gr_kernel(const float* __restrict__ gr, int T, int B, int Bp, int N, int Np,
                               int Kp, uint4* __restrict__ hi, uint4* __restrict__ mid,
                               uint4* __restrict__ lo) {
    const size_t total = (size_t)(Kp / 8) * Np;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int kb = (int)(q / Np), m = (int)(q - (size_t)kb * Np);
        uint32_t h[4], md[4], l[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t hb[2], mb[2], lb[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int k = kb * 8 + e + f;
                const int t = k / Bp, b = k - (k / Bp) * Bp;
                const float v = (t < T && b < B && m < N) ? gr[((size_t)t * B + b) * N + m] : 0.0f;
                hb[f] = bf16_rne_bits(v);
                const float r = v - __uint_as_float(hb[f] << 16);
                mb[f] = bf16_rne_bits(r);
                lb[f] = bf16_rne_bits(r - __uint_as_float(mb[f] << 16));
            }
            h[e / 2] = hb[0] | (hb[1] << 16);
            md[e / 2] = mb[0] | (mb[1] << 16);
            l[e / 2] = lb[0] | (lb[1] << 16);
        }
        hi[q] = uint4{h[0], h[1], h[2], h[3]};
        mid[q] = uint4{md[0], md[1], md[2], md[3]};
        if (lo) lo[q] = uint4{l[0], l[1], l[2], l[3]};
    }
}

// spike bits (B, ceil(T/32), N) -> Y'[t, b, j] = y[t - lo_j, b, j] in bf16 (1.0 = 0x3F80),
// k-blocked (row k = t * Bp + b, Kp = T * Bp); lo == NULL means lo_j = 1. One thread per
// column, batch octet and 32-step chunk: each of the octet's 8 rows reads the two spike words
// that cover the chunk's shifted steps once (steps before 0 read 0), and the chunk's 32
// 16-byte outputs follow, consecutive columns on consecutive lanes.
__global__ void pack_spikes_kernel(const uint32_t* __restrict__ bits, const int* __restrict__ lo,
                                   int T, int B, int Bp, int N, int Np, uint4* __restrict__ out) {
    const int TW = (T + 31) >> 5;
    const int BO = Bp / 8;
    const size_t total = (size_t)TW * BO * Np;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(q % (size_t)Np);
        const size_t r = q / (size_t)Np;
        const int bo = (int)(r % (size_t)BO), tc = (int)(r / (size_t)BO);
        const int shift = (j < N) ? (lo ? lo[j] : 1) : 0;
        // step 32 tc + e reads y at ts0 + e, ts0 = 32 tc - shift: bits off .. off + 31 of the
        // word pair (w0, w0 + 1), w0 = floor(ts0 / 32)
        const int ts0 = 32 * tc - shift;
        const int w0 = ts0 >= 0 ? ts0 / 32 : -((31 - ts0) / 32);
        const int off = ts0 - 32 * w0;
        uint32_t m[8];   // bit e: y(32 tc + e - shift) of batch row 8 bo + rr
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int b = 8 * bo + rr;
            uint64_t v = 0;
            if (j < N && b < B) {
                const size_t row = (size_t)b * TW;
                const uint32_t wl = (w0 >= 0 && w0 < TW) ? bits[(row + w0) * N + j] : 0u;
                const uint32_t wh = (w0 + 1 >= 0 && w0 + 1 < TW) ? bits[(row + w0 + 1) * N + j] : 0u;
                v = ((((uint64_t)wh) << 32) | wl) >> off;
            }
            m[rr] = (uint32_t)v;
        }
        const int ne = min(32, T - 32 * tc);
        for (int e = 0; e < ne; ++e) {
            uint32_t w[4];
#pragma unroll
            for (int pr = 0; pr < 4; ++pr)
                w[pr] = (((m[2 * pr] >> e) & 1u) ? 0x3F80u : 0u) | (((m[2 * pr + 1] >> e) & 1u) ? 0x3F800000u : 0u);
            out[((size_t)(32 * tc + e) * BO + bo) * Np + j] = uint4{w[0], w[1], w[2], w[3]};
        }
    }
}

__device__ __forceinline__ float lag_conn_delay(const LagBf16& p, int i, int j) {
    if (p.d) return p.d[(size_t)i * p.N + j];
    return p.base[j] + 0.0f + 1.0f * (float)p.off[(size_t)i * p.N + j];
}

// Lag range of each column: the first and last integer lag l in [1, L-1] on the closed
// support |l - (1 + d_ij)| <= s_j of some connection (i, j), decided by the fp32 test the
// fold uses (tap_range), so a lag outside [lo_j, lo_j + rc_j) has zero weight and zero
// derivative for every receiver. Also each column's smallest offset (hybrid). A workgroup
// covers 64 columns with 16 lanes over the receivers.
__global__ void __launch_bounds__(1024) lag_cols_kernel(LagBf16 p) {
    __shared__ int sa[16][64], sz[16][64], so[16][64], sx[16][64];
    const int jl = threadIdx.x & 63, il = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + jl;
    int a = 0x7fffffff, z = -0x7fffffff, om = 127, ox = -128;
    if (j < p.N) {
        const float s = p.s ? p.s[j] : p.s_uniform;
        for (int i = il; i < p.N; i += 16) {
            int l0, l1;
            tap_range(1.0f + lag_conn_delay(p, i, j), s, p.L, l0, l1);
            if (l0 <= l1) {
                a = min(a, l0);
                z = max(z, l1);
            }
            if (p.off) {
                const int o = p.off[(size_t)i * p.N + j];
                om = min(om, o);
                ox = max(ox, o);
            }
        }
    }
    sa[il][jl] = a;
    sz[il][jl] = z;
    so[il][jl] = om;
    sx[il][jl] = ox;
    __syncthreads();
    if (il == 0 && j < p.N) {
        for (int q = 1; q < 16; ++q) {
            a = min(a, sa[q][jl]);
            z = max(z, sz[q][jl]);
            om = min(om, so[q][jl]);
            ox = max(ox, sx[q][jl]);
        }
        p.lo[j] = a <= z ? a : 1;
        p.rc[j] = a <= z ? z - a + 1 : 0;
        p.om[j] = om;
        p.ox[j] = ox;
    }
}

// meta[0] = widest column lag range, meta[1] / meta[2] = smallest / largest offset (hybrid)
__global__ void __launch_bounds__(1024) lag_meta_kernel(const int* __restrict__ rc,
                                                        const int* __restrict__ om,
                                                        const int* __restrict__ ox, int N,
                                                        int* __restrict__ meta) {
    __shared__ int sr[16], so[16], sx[16];
    int r = 0, o = 127, x = -128;
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        r = max(r, rc[j]);
        o = min(o, om[j]);
        x = max(x, ox[j]);
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        r = max(r, __shfl_xor(r, k));
        o = min(o, __shfl_xor(o, k));
        x = max(x, __shfl_xor(x, k));
    }
    if ((threadIdx.x & 63) == 0) {
        sr[threadIdx.x >> 6] = r;
        so[threadIdx.x >> 6] = o;
        sx[threadIdx.x >> 6] = x;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
            r = max(r, sr[w]);
            o = min(o, so[w]);
            x = max(x, sx[w]);
        }
        meta[0] = r;
        meta[1] = o;
        meta[2] = x;
    }
}

// ---------------------------------------------------------------------------------------
// Windowed lag GEMM. Workgroup: a 64 x 64 output tile (4 waves of 32 x 32, 2 x 2 MFMA
// blocks each) and one 32-row batch chunk bc of every time step (the k split: partial
// sums per chunk). A time slice of an operand is the chunk's 4 k-blocks at time t.
//
// For the relative lags r = q0 .. q0 + RL - 1 of one pass, C_r = sum_tau A(tau) Y'(tau - r)
// with A = (gr_hi, gr_mid, gr_lo). Step n reads the gr slice tau = q0 + n once and multiplies it
// with the spike slices n - r', r' < RL, which stay in registers: a window of kWY slots
// holds slice sigma in slot sigma mod kWY, so step n refills slot (n + P) mod kWY (slice
// n + P, P = kWY - RL ahead) after its last reader, step n - 1, and the gr slices rotate
// through kWA slots (kWA - 1 ahead). The loop body is unrolled over kWY steps, so every
// slot is a fixed register set and each load is waited for only where it is first read.
// One descriptor per operand spans the chunk's slices 0 .. T-1, so slices at or past T
// read as zeros; slice t is the byte offset t * (Bp / 8) * Np * 16 plus the lane's column.
constexpr int kWT = 64;    // output tile (i and j)

__device__ __forceinline__ bf16x8 load16(i32x4 rs, int voff) {
    return __builtin_bit_cast(bf16x8, raw_buffer_load_i32x4(rs, voff, 0, 0));
}

template <int RL, int kWY, int kWA, bool DS, int NP>
__device__ __forceinline__ void lag_win_body(const LagBf16& p, int i0, int j0, int bc, int rt) {
    constexpr int P = kWY - RL;   // spike slices loaded ahead
    static_assert(kWY % kWA == 0 && P >= 1, "window slots");
    const int N = p.N, Np = p.Np, T = p.T;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const uint32_t slice = (uint32_t)(p.Bp / 8) * Np * 16;   // bytes per time slice
    const size_t chunk = (size_t)bc * 4 * Np;                  // uint4 offset of the chunk
    const uint32_t span = (uint32_t)T * slice - (uint32_t)(chunk * 16);
    const i32x4 rhi = buffer_rsrc(p.ahi + chunk, span);
    const i32x4 rmd = buffer_rsrc(p.amd + chunk, span);
    const i32x4 rlo = buffer_rsrc(p.alo + chunk, span);
    const i32x4 ryb = buffer_rsrc(p.yb + chunk, span);
    // lane offsets of the first 16-column block; the second is 256 bytes further
    const uint32_t va = (uint32_t)(g * Np + i0 + wi * 32 + lc) * 16;
    const uint32_t vy = (uint32_t)(g * Np + j0 + wj * 32 + lc) * 16;
    float sj[2];
    int loj[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int j = j0 + wj * 32 + nb * 16 + lc;
        const int jc = j < N ? j : 0;
        sj[nb] = p.s ? p.s[jc] : p.s_uniform;
        loj[nb] = p.lo[jc];
    }
    const bf16x8 zero = __builtin_bit_cast(bf16x8, i32x4{0, 0, 0, 0});
    const size_t NN = (size_t)N * N;

    for (int q0 = 0; q0 < max(rt, 1) && q0 < T; q0 += RL) {
        floatx4 acc[RL][2][2];
#pragma unroll
        for (int r = 0; r < RL; ++r)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) acc[r][mb][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
        bf16x8 yw[kWY][2], ah[kWA][2], am[kWA][2], al[kWA][2];
#pragma unroll
        for (int sl = 0; sl < kWY; ++sl) {
            if (sl < P) {   // slices 0 .. P-1; the other slots hold slices -RL+1 .. -1
                const uint32_t o = vy + (uint32_t)sl * slice;
                yw[sl][0] = load16(ryb, o);
                yw[sl][1] = load16(ryb, o + 256);
            } else {
                yw[sl][0] = zero;
                yw[sl][1] = zero;
            }
        }
#pragma unroll
        for (int sl = 0; sl < kWA - 1; ++sl) {
            const uint32_t o = va + (uint32_t)(q0 + sl) * slice;
            ah[sl][0] = load16(rhi, o);
            ah[sl][1] = load16(rhi, o + 256);
            am[sl][0] = load16(rmd, o);
            am[sl][1] = load16(rmd, o + 256);
            if constexpr (NP > 2) {
                al[sl][0] = load16(rlo, o);
                al[sl][1] = load16(rlo, o + 256);
            }
        }
        const int nsteps = T - q0;
        // running offsets of the next spike slice (n + P) and the next gr slice (q0 + n + kWA - 1)
        uint32_t oy = vy + (uint32_t)P * slice;
        uint32_t oa = va + (uint32_t)(q0 + kWA - 1) * slice;
        for (int n0 = 0; n0 < nsteps; n0 += kWY) {
#pragma unroll
            for (int u = 0; u < kWY; ++u) {
                {
                    yw[(u + P) % kWY][0] = load16(ryb, oy);
                    yw[(u + P) % kWY][1] = load16(ryb, oy + 256);
                    ah[(u + kWA - 1) % kWA][0] = load16(rhi, oa);
                    ah[(u + kWA - 1) % kWA][1] = load16(rhi, oa + 256);
                    am[(u + kWA - 1) % kWA][0] = load16(rmd, oa);
                    am[(u + kWA - 1) % kWA][1] = load16(rmd, oa + 256);
                    if constexpr (NP > 2) {
                        al[(u + kWA - 1) % kWA][0] = load16(rlo, oa);
                        al[(u + kWA - 1) % kWA][1] = load16(rlo, oa + 256);
                    }
                    oy += slice;
                    oa += slice;
                }
                // keep the refills at the top of the step, ahead of this step's products
                __builtin_amdgcn_sched_barrier(0);
                const int sa = u % kWA;
#pragma unroll
                for (int r = 0; r < RL; ++r)
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
                            acc[r][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                ah[sa][mb], yw[(u - r + kWY) % kWY][nb], acc[r][mb][nb], 0, 0, 0);
#pragma unroll
                for (int r = 0; r < RL; ++r)
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
                            acc[r][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                am[sa][mb], yw[(u - r + kWY) % kWY][nb], acc[r][mb][nb], 0, 0, 0);
                if constexpr (NP > 2) {
#pragma unroll
                    for (int r = 0; r < RL; ++r)
#pragma unroll
                        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                            for (int nb = 0; nb < 2; ++nb)
                                acc[r][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    al[sa][mb], yw[(u - r + kWY) % kWY][nb], acc[r][mb][nb], 0, 0, 0);
                }
            }
        }

        // fold C_l, l = lo_j + q0 + r, into this chunk's partial sums (lags past L - 1 do
        // not exist)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int j = j0 + wj * 32 + nb * 16 + lc;
            const float sv = sj[nb], s2 = sv * sv;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = i0 + wi * 32 + mb * 16 + 4 * g + e;
                    if (i >= N || j >= N) continue;
                    const float cv = 1.0f + lag_conn_delay(p, i, j);
                    float ow = 0.0f, od = 0.0f, os = 0.0f;
#pragma unroll
                    for (int r = 0; r < RL; ++r) {
                        const int l = loj[nb] + q0 + r;
                        const float C = l <= p.L - 1 ? acc[r][mb][nb][e] : 0.0f;
                        const float lf = (float)l;
                        ow += tri_weight(lf, cv, sv, s2) * C;
                        od += tri_dsign(lf, cv, sv) * C;
                        if (DS) os += tri_ds(lf, cv, sv, s2) * C;
                    }
                    const size_t o = (size_t)bc * NN + (size_t)i * N + j;
                    if (q0 > 0) {
                        ow += p.pw[o];
                        od += p.pd[o];
                        if (DS) os += p.ps[o];
                    }
                    p.pw[o] = ow;
                    p.pd[o] = od;
                    if (DS) p.ps[o] = os;
                }
        }
    }
}

// one workgroup per (output tile, batch chunk); the chunk is the fastest index, so with 8
// chunks the workgroups of one chunk share an XCD (workgroups are dealt to the XCDs in
// turn) and its L2 holds the slices they all stream. Tiles of at most 6 lags run 6-lag
// passes (the hybrid of 5 offsets and 2 taps), of at most 8 lags 8-lag passes, of at most 10
// lags 10-lag passes, wider ones 12-lag passes; the launch of each variant skips the others'
// tiles (each variant gets the whole register file to itself).
template <int RL, bool DS, int NP>
__global__ void __launch_bounds__(256) lag_win_kernel(LagBf16 p) {
    const int nbc = p.Bp / 32;
    const int bc = (int)blockIdx.x % nbc, tile = (int)blockIdx.x / nbc;
    const int tj = p.Np / kWT;
    const int i0 = (tile / tj) * kWT, j0 = (tile % tj) * kWT;
    const int j = j0 + (int)(threadIdx.x & 63);
    int rt = j < p.N ? p.rc[j] : 0;   // the tile's lags: the widest range among its columns
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) rt = max(rt, __shfl_xor(rt, k));
    rt = __builtin_amdgcn_readfirstlane(rt);
    // each launch takes the tiles whose widest range its pass width serves best
    if (RL == 6 && rt > 6) return;
    if (RL == 8 && (rt <= 6 || rt > 8)) return;
    if (RL == 10 && (rt <= 8 || rt > 10)) return;
    if (RL == 12 && rt <= 10) return;
    // gr-slice registers: 3 slots (2 slices ahead) beside a 12-slot spike window (6-, 8- and
    // 10-lag passes), 4 slots (3 ahead) beside the 16-slot one (12-lag passes)
    lag_win_body<RL, RL <= 10 ? 12 : 16, RL <= 10 ? 3 : 4, DS, NP>(p, i0, j0, bc, rt);
}

template <bool DS, int NP>
void launch_lag_win(const LagBf16& a, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((lag_win_kernel<6, DS, NP>), grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL((lag_win_kernel<8, DS, NP>), grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL((lag_win_kernel<10, DS, NP>), grid, dim3(256), 0, stream, a);
    hipLaunchKernelGGL((lag_win_kernel<12, DS, NP>), grid, dim3(256), 0, stream, a);
}

void launch_lag_cols(const LagBf16& a, hipStream_t stream) {
    hipLaunchKernelGGL(lag_cols_kernel, dim3((a.N + 63) / 64), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(lag_meta_kernel, dim3(1), dim3(1024), 0, stream, a.rc, a.om, a.ox, a.N, a.meta);
}

void launch_lag_bf16(const LagBf16& a, const float* gr, const uint32_t* bits, hipStream_t stream) {
    const size_t total = (size_t)(a.Kp / 8) * a.Np;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(pack_gr_kernel, dim3(blocks), dim3(256), 0, stream, gr, a.T, a.B, a.Bp, a.N,
                       a.Np, a.Kp, const_cast<uint4*>(a.ahi), const_cast<uint4*>(a.amd),
                       a.planes == 2 ? nullptr : const_cast<uint4*>(a.alo));
    const size_t chunks = (size_t)((a.T + 31) / 32) * (a.Bp / 8) * a.Np;
    const unsigned sblocks = (unsigned)std::min<size_t>((chunks + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(pack_spikes_kernel, dim3(sblocks), dim3(256), 0, stream, bits, a.lo, a.T, a.B,
                       a.Bp, a.N, a.Np, const_cast<uint4*>(a.yb));
    const int tiles = (a.Np / kWT) * (a.Np / kWT);
    const dim3 grid((unsigned)(tiles * (a.Bp / 32)));
    if (a.planes == 2) {
        if (a.ps) launch_lag_win<true, 2>(a, grid, stream); else launch_lag_win<false, 2>(a, grid, stream);
    } else {
        if (a.ps) launch_lag_win<true, 3>(a, grid, stream); else launch_lag_win<false, 3>(a, grid, stream);
    }
}

}  // namespace delrec
