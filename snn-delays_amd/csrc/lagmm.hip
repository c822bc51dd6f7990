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

#include <cstdio>
#include <cstdlib>

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
// k-blocked (row k = t * Bp + b, Kp = T * Bp); lo == NULL means lo_j = 1. Column position jp
// holds column perm[jp] (jp when perm is NULL); with the class sizes cls, only the positions
// from the first 64-column tile that holds a dense column on (the dense kernel's tiles). One
// thread per position, batch octet and 32-step chunk: each of the octet's 8 rows reads the two
// spike words that cover the chunk's shifted steps once (steps before 0 read 0), and the
// chunk's 32 16-byte outputs follow, consecutive positions on consecutive lanes.
__global__ void pack_spikes_kernel(const uint32_t* __restrict__ bits, const int* __restrict__ lo,
                                   const int* __restrict__ perm, const int* __restrict__ cls, int T, int B,
                                   int Bp, int N, int Np, uint4* __restrict__ out) {
    const int TW = (T + 31) >> 5;
    const int BO = Bp / 8;
    const int first = cls ? (cls[0] + cls[1]) / 64 * 64 : 0;
    const int cols = Np - first;
    const size_t total = (size_t)TW * BO * cols;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int jp = first + (int)(q % (size_t)cols);
        const int j = perm ? perm[jp] : (jp < N ? jp : -1);
        const size_t r = q / (size_t)cols;
        const int bo = (int)(r % (size_t)BO), tc = (int)(r / (size_t)BO);
        const int shift = (j >= 0) ? (lo ? lo[j] : 1) : 0;
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
            if (j >= 0 && b < B) {
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
            out[((size_t)(32 * tc + e) * BO + bo) * Np + jp] = uint4{w[0], w[1], w[2], w[3]};
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
    // column position jp -> column (the event-driven form's order), -1 for padding
    auto colj = [&](int jp) { return p.perm ? (jp < Np ? p.perm[jp] : -1) : (jp < N ? jp : -1); };
    float sj[2];
    int loj[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int j = colj(j0 + wj * 32 + nb * 16 + lc);
        const int jc = j >= 0 ? j : 0;
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
            const int jp = j0 + wj * 32 + nb * 16 + lc, j = colj(jp);
            const float sv = sj[nb], s2 = sv * sv;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = i0 + wi * 32 + mb * 16 + 4 * g + e;
                    if (i >= N || j < 0) continue;
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
                    const size_t o = (size_t)bc * NN + (size_t)i * N + jp;
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
    if (p.cls) {   // event-driven form: only the tiles that hold a dense column
        const int n1 = p.cls[0] + p.cls[1], n2 = n1 + p.cls[2];
        if (j0 + kWT <= n1 || j0 >= n2) return;
    }
    const int jp = j0 + (int)(threadIdx.x & 63);
    const int j = p.perm ? (jp < p.Np ? p.perm[jp] : -1) : (jp < p.N ? jp : -1);
    int rt = j >= 0 ? p.rc[j] : 0;   // the tile's lags: the widest range among its columns
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) rt = max(rt, __shfl_xor(rt, k));
    rt = __builtin_amdgcn_readfirstlane(rt);
    // each launch takes the tiles whose widest range its pass width serves best
    if (RL == 6 && rt > 6) return;
    if (RL == 8 && (rt <= 6 || rt > 8)) return;
    if (RL == 10 && (rt <= 8 || rt > 10)) return;
    if (RL == 12 && rt <= 10) return;
    // gr-slice registers: 3 slots (2 slices ahead) beside a 12-slot spike window (6-, 8- and
    // 10-lag passes) or a 15-slot one (12-lag passes; a 16-slot window with 4 gr slots left
    // more spilled registers in the step loop: 11.5 against 8.9 ms at T250 B256 N1024 sigma 4)
    lag_win_body<RL, RL <= 10 ? 12 : 15, 3, DS, NP>(p, i0, j0, bc, rt);
}

// ---------------------------------------------------------------------------------------
// The same correlation, event-driven over the spike columns (bf16 W: hi + mid gr planes). A
// spike column j contributes C_l[., j] only through its spikes, and the recurrent layers'
// spike trains are sparse and uneven (C5's first layer: 70 % of the columns never fire, 20 %
// fire at 10-30 %). The contraction runs over the 64 batch rows of a chunk at one step, in
// groups of four rows, and each column falls in one of three classes, counted on the device
// from the shifted trains themselves:
//  silent  no spike: C_l[., j] = 0, no products;
//  sparse  never more than two spikes in a group: the spikes are the exact compressed operand
//          of the 4:2 sparse MFMA (v_smfmac_f32_16x16x64_bf16: values bf16 1.0, or 0 where a
//          group has fewer), half the dense issue;
//  dense   some group with three or four spikes: the dense kernel above (lag_win_kernel) on
//          the spike operand packed in the same column order.
// The columns are reordered by class (stable) so that 64-column tiles hold one class where
// they can (a tile takes the heaviest class among its columns); the partial sums stay in that
// order and lag_finish puts each column back. The sparse kernel's output is C^T: rows j
// (spike columns), columns i.
//
// Sparse operand lanes: the A lane l is row l % 16, values 2gg, 2gg + 1 in group 4 (l / 16) + gg
// with their 2-bit positions in bits 4gg .. 4gg + 3 of the index, so lane group g = l / 16
// covers batch rows 16g .. 16g + 15 of the 64-row chunk; a B lane supplies rows 8g .. 8g + 7
// and 32 + 8g .. + 7 of its receiver (slots 0-7, 8-15): the k-blocks g and g + 4 of the chunk
// in the dense kernel's gr planes.

// 16 spike bits (bit q = batch row 16g + q) -> one sparse A lane as a code word: bits 0-15 the
// value positions, 16-23 two value bits per group (value 2gg at bit 16 + 2gg, 2gg + 1 at
// 17 + 2gg), bit 24 set when a group holds more than two spikes. Positions ascend in a group.
__host__ __device__ inline uint32_t sp_code16(uint32_t m) {
    uint32_t idx = 0, vb = 0, over = 0;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
        const uint32_t n = (m >> (4 * gg)) & 15u;
        const uint32_t l1 = n & (0u - n), n2 = n ^ l1, l2 = n2 & (0u - n2);
        over |= n2 ^ l2;
        const uint32_t p1 = l1 ? (uint32_t)__builtin_ctz(l1) : 0u, p2 = l2 ? (uint32_t)__builtin_ctz(l2) : 0u;
        uint32_t q0 = 0, q1 = 1, v = 0;
        if (l2) { q0 = p1; q1 = p2; v = 3; }
        else if (l1 && p1 == 0) { v = 1; }
        else if (l1) { q1 = p1; v = 2; }
        idx |= (q0 | (q1 << 2)) << (4 * gg);
        vb |= v << (2 * gg);
    }
    return idx | (vb << 16) | ((over != 0u ? 1u : 0u) << 24);
}

// a code word's values as the 8 bf16 of the sparse A operand
__device__ __forceinline__ bf16x8 sp_values(uint32_t c) {
    uint32_t w[4];
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
        const uint32_t b0 = (c >> (16 + 2 * gg)) & 1u, b1 = (c >> (17 + 2 * gg)) & 1u;
        w[gg] = (b0 | (b1 << 16)) * 0x3F80u;
    }
    return __builtin_bit_cast(bf16x8, uint4{w[0], w[1], w[2], w[3]});
}

// the 16 batch rows 64c + 16g + rr of column j over the steps 32 tc .. 32 tc + 31 of the
// shifted train Y'[t] = y[t - shift]: m[rr] bit e = Y'[32 tc + e] (0 outside 0 .. T-1)
__device__ __forceinline__ void sp_rows(const uint32_t* __restrict__ bits, int T, int B, int N, int j, int shift,
                                        int c, int g, int tc, uint32_t (&m)[16]) {
    const int TW = (T + 31) >> 5;
    const int ts0 = 32 * tc - shift;
    const int w0 = ts0 >= 0 ? ts0 / 32 : -((31 - ts0) / 32);
    const int off = ts0 - 32 * w0;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
        const int b = 64 * c + 16 * g + rr;
        uint64_t v = 0;
        if (j >= 0 && j < N && b < B) {
            const size_t row = (size_t)b * TW;
            const uint32_t wl = (w0 >= 0 && w0 < TW) ? bits[(row + w0) * N + j] : 0u;
            const uint32_t wh = (w0 + 1 >= 0 && w0 + 1 < TW) ? bits[(row + w0 + 1) * N + j] : 0u;
            v = ((((uint64_t)wh) << 32) | wl) >> off;
        }
        m[rr] = (uint32_t)v;
    }
}

__device__ __forceinline__ uint32_t sp_step16(const uint32_t (&m)[16], int e) {
    uint32_t mk = 0;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) mk |= ((m[rr] >> e) & 1u) << rr;
    return mk;
}

__global__ void lag_zero_kernel(int* __restrict__ p, int n) {
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < n; q += gridDim.x * blockDim.x) p[q] = 0;
}

// cnt[j] = spikes of column j's shifted train, cnt[Np + j] = its groups of four batch rows
// with more than two spikes at one step. One thread per (column, chunk, lane group, 32 steps).
__global__ void lag_count_kernel(const uint32_t* __restrict__ bits, const int* __restrict__ lo, int T, int B,
                                 int Bp, int N, int Np, int* __restrict__ cnt) {
    const int TW = (T + 31) >> 5, NC = Bp / 64;
    const size_t total = (size_t)TW * NC * 4 * N;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int j = (int)(q % (size_t)N);
        size_t r = q / (size_t)N;
        const int g = (int)(r & 3);
        r >>= 2;
        const int c = (int)(r % (size_t)NC), tc = (int)(r / (size_t)NC);
        uint32_t m[16];
        sp_rows(bits, T, B, N, j, lo[j], c, g, tc, m);
        int spk = 0, ovf = 0;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) spk += __builtin_popcount(m[rr]);
        if (spk) {
            const int ne = min(32, T - 32 * tc);
            for (int e = 0; e < ne; ++e) ovf += (int)(sp_code16(sp_step16(m, e)) >> 24);
            atomicAdd(&cnt[j], spk);
            if (ovf) atomicAdd(&cnt[Np + j], ovf);
        }
    }
}

// The column order: silent columns, then sparse, then dense (each in column order), then the
// padding columns N .. Np-1 (perm = -1); cls[0..2] = the class sizes. One workgroup.
__global__ void __launch_bounds__(1024) lag_perm_kernel(const int* __restrict__ cnt, int N, int Np,
                                                        int* __restrict__ perm, int* __restrict__ cls) {
    __shared__ int sc[4][1024];
    __shared__ int tot[4];
    const int tid = threadIdx.x, per = (Np + 1023) / 1024;
    const int a = min(Np, tid * per), z = min(Np, a + per);
    auto klass = [&](int j) { return j >= N ? 3 : (cnt[Np + j] > 0 ? 2 : (cnt[j] > 0 ? 1 : 0)); };
    int n[4] = {0, 0, 0, 0};
    for (int j = a; j < z; ++j) ++n[klass(j)];
#pragma unroll
    for (int k = 0; k < 4; ++k) sc[k][tid] = n[k];
    __syncthreads();
    // inclusive scans of the four count arrays (Hillis-Steele)
    for (int d = 1; d < 1024; d <<= 1) {
        int v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = tid >= d ? sc[k][tid - d] : 0;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) sc[k][tid] += v[k];
        __syncthreads();
    }
    if (tid == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) tot[k] = sc[k][1023];
    }
    __syncthreads();
    int pos[4];
    pos[0] = sc[0][tid] - n[0];
    pos[1] = tot[0] + sc[1][tid] - n[1];
    pos[2] = tot[0] + tot[1] + sc[2][tid] - n[2];
    pos[3] = tot[0] + tot[1] + tot[2] + sc[3][tid] - n[3];
    for (int j = a; j < z; ++j) {
        const int k = klass(j);
        perm[pos[k]++] = k == 3 ? -1 : j;
    }
    if (tid == 0) {
        cls[0] = tot[0];
        cls[1] = tot[1];
        cls[2] = tot[2];
    }
}

// the shifted spike trains of the sparse tiles' columns (positions below the first tile that
// holds a dense column) as code words at ((t * NC + c) * 4 + g) * Np + jp. One thread per
// (position, chunk, lane group, 32 steps).
__global__ void pack_spikes_sp_kernel(const uint32_t* __restrict__ bits, const int* __restrict__ lo,
                                      const int* __restrict__ perm, const int* __restrict__ cls, int T, int B,
                                      int Bp, int N, int Np, uint32_t* __restrict__ code) {
    const int TW = (T + 31) >> 5, NC = Bp / 64;
    const int lim = (cls[0] + cls[1]) / 64 * 64;
    const size_t total = (size_t)TW * NC * 4 * lim;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int jp = (int)(q % (size_t)lim);
        size_t r = q / (size_t)lim;
        const int g = (int)(r & 3);
        r >>= 2;
        const int c = (int)(r % (size_t)NC), tc = (int)(r / (size_t)NC);
        const int j = perm[jp];
        uint32_t m[16];
        sp_rows(bits, T, B, N, j, j >= 0 ? lo[j] : 0, c, g, tc, m);
        const int ne = min(32, T - 32 * tc);
        for (int e = 0; e < ne; ++e)
            code[(((size_t)(32 * tc + e) * NC + c) * 4 + g) * Np + jp] = sp_code16(sp_step16(m, e));
    }
}

typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

__device__ uint32_t lw_buffer_load_u32(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");

// Sparse tiles. Workgroup: a 64 x 64 output tile (receivers i0 .., column positions j0 ..),
// one 64-row chunk bc; waves of JB column blocks (16) x IB receiver blocks (16), JB x IB = 4
// (JB = 4: each wave 16 receivers x all 64 columns). Step n reads the gr slice q0 + n (both
// planes; per lane and block the k-blocks g and g + 4 of the chunk: K = 64) and multiplies it
// with the code words of slices n - r, r < RL, held expanded in a window of KWY = RL + P
// slots (loaded P steps ahead); gr rotates through KWA slots (KWA - 1 steps ahead). The
// chunk's sums go to the partial of its first 32 rows (the partials are per 32-row chunk, as
// the dense kernel's; lag_finish reads the even ones for these columns).
template <int RL, int JB, int IB, bool DS, int KWA = 2, int P = 2>
__device__ __forceinline__ void lag_win_sp_body(const LagBf16& p, int i0, int j0, int bc, int rt,
                                                float (*tw)[65], float (*td)[65], float (*ts)[65]) {
    constexpr int KWY = RL + P;
    static_assert(JB * IB == 4 && KWY % KWA == 0 && KWY % P == 0, "wave shape / window slots");
    const int N = p.N, Np = p.Np, T = p.T, NC = p.Bp / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, lc = lane & 15;
    const int iw = IB == 1 ? 16 * w : 32 * (w >> 1);      // the wave's first receiver (tile-relative)
    const int jw = IB == 1 ? 0 : 32 * (w & 1);           // and first column position
    // gr planes (k-blocked): slice t, k-block kb of the chunk, receiver i at uint4
    // (t * Bp / 8 + 8 bc + kb) * Np + i
    const uint32_t gslice = (uint32_t)(p.Bp / 8) * Np * 16;
    const size_t gch = (size_t)bc * 8 * Np;
    const uint32_t gspan = (uint32_t)T * gslice - (uint32_t)(gch * 16);
    const i32x4 rhi = buffer_rsrc(p.ahi + gch, gspan);
    const i32x4 rmd = buffer_rsrc(p.amd + gch, gspan);
    const uint32_t va = (uint32_t)(g * Np + i0 + iw + lc) * 16;
    const uint32_t vhalf = (uint32_t)4 * Np * 16;
    // code words: slice t at u32 ((t * NC + bc) * 4 + g) * Np + jp
    const uint32_t cslice = (uint32_t)NC * 4 * Np * 4;
    const size_t cch = (size_t)bc * 4 * Np;
    const i32x4 rcd = buffer_rsrc(p.ycode + cch, (uint32_t)T * cslice - (uint32_t)(cch * 4));
    const uint32_t vc = (uint32_t)(g * Np + j0 + jw + lc) * 4;
    const size_t NN = (size_t)N * N;
    auto load_b = [&](const i32x4& rs, uint32_t o) {
        const i32x4 x0 = raw_buffer_load_i32x4(rs, (int)o, 0, 0);
        const i32x4 x1 = raw_buffer_load_i32x4(rs, (int)(o + vhalf), 0, 0);
        return u32x8{(uint32_t)x0.x, (uint32_t)x0.y, (uint32_t)x0.z, (uint32_t)x0.w,
                     (uint32_t)x1.x, (uint32_t)x1.y, (uint32_t)x1.z, (uint32_t)x1.w};
    };

    for (int q0 = 0; q0 < max(rt, 1) && q0 < T; q0 += RL) {
        floatx4 acc[RL][JB][IB];
#pragma unroll
        for (int r = 0; r < RL; ++r)
#pragma unroll
            for (int jb = 0; jb < JB; ++jb)
#pragma unroll
                for (int ib = 0; ib < IB; ++ib) acc[r][jb][ib] = floatx4{0.f, 0.f, 0.f, 0.f};
        {
            bf16x8 sv[KWY][JB];
            uint32_t si[KWY][JB];
            uint32_t raw[P][JB];
            u32x8 bh[KWA][IB], bm[KWA][IB];
            const bf16x8 zero = __builtin_bit_cast(bf16x8, i32x4{0, 0, 0, 0});
#pragma unroll
            for (int sl = 0; sl < KWY; ++sl)     // slots P .. KWY-1 hold slices -RL .. -1 (zeros)
#pragma unroll
                for (int jb = 0; jb < JB; ++jb) {
                    sv[sl][jb] = zero;
                    si[sl][jb] = 0u;
                }
#pragma unroll
            for (int sl = 0; sl < P; ++sl)
#pragma unroll
                for (int jb = 0; jb < JB; ++jb)
                    raw[sl][jb] = lw_buffer_load_u32(rcd, (int)(vc + (uint32_t)jb * 64 + (uint32_t)sl * cslice), 0, 0);
#pragma unroll
            for (int sl = 0; sl < KWA - 1; ++sl)
#pragma unroll
                for (int ib = 0; ib < IB; ++ib) {
                    bh[sl][ib] = load_b(rhi, va + (uint32_t)ib * 256 + (uint32_t)(q0 + sl) * gslice);
                    bm[sl][ib] = load_b(rmd, va + (uint32_t)ib * 256 + (uint32_t)(q0 + sl) * gslice);
                }
            const int nsteps = T - q0;
            uint32_t oy = vc + (uint32_t)P * cslice;                 // code slice n + P
            uint32_t oa = va + (uint32_t)(q0 + KWA - 1) * gslice;    // gr slice q0 + n + KWA - 1
            for (int n0 = 0; n0 < nsteps; n0 += KWY) {
#pragma unroll
                for (int u = 0; u < KWY; ++u) {
                    // slice n = n0 + u enters its slot
#pragma unroll
                    for (int jb = 0; jb < JB; ++jb) {
                        const uint32_t c = raw[u % P][jb];
                        sv[u][jb] = sp_values(c);
                        si[u][jb] = c & 0xFFFFu;
                    }
#pragma unroll
                    for (int jb = 0; jb < JB; ++jb)
                        raw[u % P][jb] = lw_buffer_load_u32(rcd, (int)(oy + (uint32_t)jb * 64), 0, 0);
#pragma unroll
                    for (int ib = 0; ib < IB; ++ib) {
                        bh[(u + KWA - 1) % KWA][ib] = load_b(rhi, oa + (uint32_t)ib * 256);
                        bm[(u + KWA - 1) % KWA][ib] = load_b(rmd, oa + (uint32_t)ib * 256);
                    }
                    oy += cslice;
                    oa += gslice;
                    __builtin_amdgcn_sched_barrier(0);
                    const int sa = u % KWA;
                    // one pass per gr plane, so that consecutive products go to different
                    // accumulators
#pragma unroll
                    for (int pl = 0; pl < 2; ++pl)
#pragma unroll
                        for (int r = 0; r < RL; ++r)
#pragma unroll
                            for (int jb = 0; jb < JB; ++jb)
#pragma unroll
                                for (int ib = 0; ib < IB; ++ib) {
                                    const int sl = (u - r + KWY) % KWY;
                                    acc[r][jb][ib] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(
                                        sv[sl][jb], __builtin_bit_cast(bf16x16, pl == 0 ? bh[sa][ib] : bm[sa][ib]),
                                        acc[r][jb][ib], (int)si[sl][jb], 0, 0);
                                }
                }
            }
        }

        // fold C_l, l = lo_j + q0 + r, through LDS (C^T on the lanes: column position ..4g + e,
        // receiver i = ..lc) into this chunk's partial sums, stored in the column order
#pragma unroll
        for (int jb = 0; jb < JB; ++jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int jl = jw + jb * 16 + 4 * g + e, jp = j0 + jl;
                const int j = jp < Np ? p.perm[jp] : -1;
                const int jc = j >= 0 ? j : 0;
                const float sv0 = p.s ? p.s[jc] : p.s_uniform, s2 = sv0 * sv0;
                const int loj = p.lo[jc];
#pragma unroll
                for (int ib = 0; ib < IB; ++ib) {
                    const int il = iw + ib * 16 + lc, i = i0 + il;
                    float ow = 0.0f, od = 0.0f, os = 0.0f;
                    if (i < N && j >= 0) {
                        const float cv = 1.0f + lag_conn_delay(p, i, j);
#pragma unroll
                        for (int r = 0; r < RL; ++r) {
                            const int l = loj + q0 + r;
                            const float C = l <= p.L - 1 ? acc[r][jb][ib][e] : 0.0f;
                            const float lf = (float)l;
                            ow += tri_weight(lf, cv, sv0, s2) * C;
                            od += tri_dsign(lf, cv, sv0) * C;
                            if (DS) os += tri_ds(lf, cv, sv0, s2) * C;
                        }
                    }
                    tw[il][jl] = ow;
                    td[il][jl] = od;
                    if (DS) ts[il][jl] = os;
                }
            }
        __syncthreads();
        {
            const int il = tid >> 2, i = i0 + il;
#pragma unroll 4
            for (int x = 0; x < 16; ++x) {
                const int jl = (tid & 3) * 16 + x, jp = j0 + jl;
                if (i >= N || jp >= N) continue;        // positions N .. Np-1 hold the padding
                const size_t o = (size_t)(2 * bc) * NN + (size_t)i * N + jp;
                float ow = tw[il][jl], od = td[il][jl], os = DS ? ts[il][jl] : 0.0f;
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
        __syncthreads();
    }
}

// one workgroup per (output tile, 64-row chunk), the chunk fastest (as the dense kernel), for
// the tiles below the first dense column that are not silent: 6-, 8- and 10-lag passes (wider
// tiles in several 6-lag passes)
template <int RL, bool DS>
__global__ void __launch_bounds__(256) lag_win_sp_kernel(LagBf16 p) {
    __shared__ float tw[64][65], td[64][65], ts[DS ? 64 : 1][65];
    const int nbc = p.Bp / 64;
    const int bc = (int)blockIdx.x % nbc, tile = (int)blockIdx.x / nbc;
    const int tj = p.Np / kWT;
    const int i0 = (tile / tj) * kWT, j0 = (tile % tj) * kWT;
    const int n0 = p.cls[0], n1 = n0 + p.cls[1];
    if (j0 + kWT > n1) return;                           // a dense column, or padding only
    if (j0 + kWT <= n0) return;                          // silent: lag_finish takes 0
    const int jp = j0 + (int)(threadIdx.x & 63);
    const int jj = p.perm[jp];
    int rt = jj >= 0 ? p.rc[jj] : 0;
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) rt = max(rt, __shfl_xor(rt, k));
    rt = __builtin_amdgcn_readfirstlane(rt);
    if (RL == 6 && rt > 6 && rt <= 10) return;
    if (RL == 8 && (rt <= 6 || rt > 8)) return;
    if (RL == 10 && (rt <= 8 || rt > 10)) return;
    // 6-lag passes: 2 x 2 waves with gr two steps ahead (three slots); 4 x 1 waves with one
    // step ahead, a fifth of the L1 traffic for the B operand, measured 5 % slower (C5)
    if constexpr (RL == 6)
        lag_win_sp_body<RL, 2, 2, DS, 3, 3>(p, i0, j0, bc, rt, tw, td, ts);
    else
        lag_win_sp_body<RL, 2, 2, DS>(p, i0, j0, bc, rt, tw, td, ts);
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

bool lag_bf16_sparse(const LagBf16& a) {
    // DELREC_LAG_SPARSE=0 turns the form off, =1 takes it whatever the grid
    const char* e = std::getenv("DELREC_LAG_SPARSE");
    const bool off = e && e[0] == '0', force = e && e[0] == '1';
    // bf16 W (two gr planes; the third plane's buffer holds the event-driven form's arrays),
    // whole 64-row chunks, and a dense grid of at least 4096 workgroups (16 per CU): below
    // that the correlation takes one workgroup's walk over the steps whatever its share of the
    // work, and two launches (sparse and dense tiles) take two walks (C3, 512 workgroups:
    // 0.39 ms dense, 0.60 ms split)
    const size_t wgs = (size_t)(a.Np / kWT) * (a.Np / kWT) * (a.Bp / 32);
    return !off && a.planes == 2 && a.Bp % 64 == 0 && (force || wgs >= 4096);
}

namespace {

// the event-driven form's arrays in the third gr plane's room (unused with two planes):
// column counts [2][Np], order [Np], class sizes [4], code words [T][Bp / 64][4][Np]
struct LagSpRoom {
    int* cnt;
    int* perm;
    int* cls;
    uint32_t* code;
};

LagSpRoom lag_sp_room(const LagBf16& a) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    char* base = reinterpret_cast<char*>(const_cast<uint4*>(a.alo));
    LagSpRoom r;
    size_t o = 0;
    r.cnt = reinterpret_cast<int*>(base + o);
    o += up((size_t)2 * a.Np * sizeof(int));
    r.perm = reinterpret_cast<int*>(base + o);
    o += up((size_t)a.Np * sizeof(int));
    r.cls = reinterpret_cast<int*>(base + o);
    o += 256;
    r.code = reinterpret_cast<uint32_t*>(base + o);
    return r;
}

}  // namespace

void launch_col_order(const int* cnt, int N, int Np, int* perm, int* cls, hipStream_t stream) {
    hipLaunchKernelGGL(lag_perm_kernel, dim3(1), dim3(1024), 0, stream, cnt, N, Np, perm, cls);
}

const int* lag_bf16_perm(const LagBf16& a) { return lag_bf16_sparse(a) ? lag_sp_room(a).perm : nullptr; }
const int* lag_bf16_cls(const LagBf16& a) { return lag_bf16_sparse(a) ? lag_sp_room(a).cls : nullptr; }

void launch_lag_bf16(const LagBf16& a, const float* gr, const uint32_t* bits, hipStream_t stream) {
    const bool ev = lag_bf16_sparse(a);
    if (std::getenv("DELREC_LOG_PLAN"))
        std::fprintf(stderr, "[delrec] lag correlation: %s spikes\n", ev ? "event-driven" : "dense");
    const size_t total = (size_t)(a.Kp / 8) * a.Np;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(pack_gr_kernel, dim3(blocks), dim3(256), 0, stream, gr, a.T, a.B, a.Bp, a.N,
                       a.Np, a.Kp, const_cast<uint4*>(a.ahi), const_cast<uint4*>(a.amd),
                       a.planes == 2 ? nullptr : const_cast<uint4*>(a.alo));
    LagBf16 b = a;
    const size_t chunks = (size_t)((a.T + 31) / 32) * (a.Bp / 8) * a.Np;
    const unsigned sblocks = (unsigned)std::min<size_t>((chunks + 255) / 256, 65535u * 4);
    const int tiles = (a.Np / kWT) * (a.Np / kWT);
    if (ev) {
        // column classes and order, the sparse tiles' code words, then the dense kernel on the
        // tiles from the first dense column on (its spike operand in the same order)
        const LagSpRoom rm = lag_sp_room(a);
        const int NC = a.Bp / 64, TW = (a.T + 31) / 32;
        hipLaunchKernelGGL(lag_zero_kernel, dim3((2 * a.Np + 255) / 256), dim3(256), 0, stream, rm.cnt, 2 * a.Np);
        const size_t tc = (size_t)TW * NC * 4 * a.N;
        hipLaunchKernelGGL(lag_count_kernel, dim3((unsigned)std::min<size_t>((tc + 255) / 256, 65535u * 4)),
                           dim3(256), 0, stream, bits, a.lo, a.T, a.B, a.Bp, a.N, a.Np, rm.cnt);
        hipLaunchKernelGGL(lag_perm_kernel, dim3(1), dim3(1024), 0, stream, rm.cnt, a.N, a.Np, rm.perm, rm.cls);
        const size_t th = (size_t)TW * NC * 4 * a.Np;
        hipLaunchKernelGGL(pack_spikes_sp_kernel, dim3((unsigned)std::min<size_t>((th + 255) / 256, 65535u * 4)),
                           dim3(256), 0, stream, bits, a.lo, rm.perm, rm.cls, a.T, a.B, a.Bp, a.N, a.Np, rm.code);
        b.ycode = rm.code;
        b.perm = rm.perm;
        b.cls = rm.cls;
        const dim3 grid((unsigned)(tiles * NC));
        if (a.ps) {
            hipLaunchKernelGGL((lag_win_sp_kernel<6, true>), grid, dim3(256), 0, stream, b);
            hipLaunchKernelGGL((lag_win_sp_kernel<8, true>), grid, dim3(256), 0, stream, b);
            hipLaunchKernelGGL((lag_win_sp_kernel<10, true>), grid, dim3(256), 0, stream, b);
        } else {
            hipLaunchKernelGGL((lag_win_sp_kernel<6, false>), grid, dim3(256), 0, stream, b);
            hipLaunchKernelGGL((lag_win_sp_kernel<8, false>), grid, dim3(256), 0, stream, b);
            hipLaunchKernelGGL((lag_win_sp_kernel<10, false>), grid, dim3(256), 0, stream, b);
        }
    }
    hipLaunchKernelGGL(pack_spikes_kernel, dim3(sblocks), dim3(256), 0, stream, bits, a.lo, b.perm, b.cls, a.T, a.B,
                       a.Bp, a.N, a.Np, const_cast<uint4*>(a.yb));
    const dim3 grid((unsigned)(tiles * (a.Bp / 32)));
    if (a.planes == 2) {
        if (a.ps) launch_lag_win<true, 2>(b, grid, stream); else launch_lag_win<false, 2>(b, grid, stream);
    } else {
        if (a.ps) launch_lag_win<true, 3>(b, grid, stream); else launch_lag_win<false, 3>(b, grid, stream);
    }
}

}  // namespace delrec
