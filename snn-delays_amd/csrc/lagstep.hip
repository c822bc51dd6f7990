// Synaptic / hybrid scans as one lag-stacked GEMM per time step, on bf16 MFMA (gfx950).
//
// With per-connection weights M_l[i,j] = W_ij * h(l; d_ij, s_j) (h = max(0, s - |l - c|) / s^2,
// c = 1 + d, the triangle of reference delays.py:48-63), the recurrent input of step t and
// the future gradient of the backward are
//   rec(t)[b, i]  = sum_{l=1..Lw} sum_j y(t - l)[b, j]  M_l[i, j]
//   gfut(t)[b, j] = sum_{l=1..Lw} sum_i gr(t + l)[b, i] M_l[i, j],      Lw = L - 1,
// i.e. a (B x Lw*N) by (Lw*N x N) product per step whose left operand is a window of a
// batch-major history: with the history stored [b][time][N], the window of step t is a
// plain strided matrix (row b at b * lda, k = lag slot * N + neuron). Every lag of every
// connection is a dense MFMA product: the triangle's empty lags cost MFMA time instead of
// per-tap VALU work.
//
// Time blocking. Streaming all of M every step would make the scan HBM-bound, so the steps
// go in blocks of P: the lags l > P of a whole block depend only on spikes (gradients)
// from before (after) the block, so one GEMM with B * P rows (row (b, step of the block))
// covers them and reads their part of M once per block; each step then runs a split-K GEMM
// over its P near lags (their part of M stays in cache) and one LIF launch that adds both
// sets of partial sums in a fixed order and advances the neurons.
// This replaces the per-connection gathers of the reference's scans
// (synaptic_eventdriven.py:106-164, :323-364) where their rings do not fit one CU's LDS.
//
// Precision: spikes are exact in bf16. M is stored as two bf16 planes, M ~ hi + lo (relative
// error about 2^-17); the backward also splits gr into hi + lo and takes hi*hi + hi*lo + lo*hi
// (about 2^-16). Accumulation is fp32.
//
// Layouts. A packed operand P with K rows and Np columns is k-blocked: element (k, n) at
// ((k / 8) * Np + n) * 8 + k % 8, so one 16-byte load holds the 8 consecutive k of one column
// that an MFMA lane supplies. Forward: k = q * Nk + j with lag l = Lw - q (q ascending is
// time ascending), columns i. Backward: k = q * Nk + i with lag l = q + 1, columns j. The
// neuron count is padded to Nk = 32n so a 32-row k stage never straddles two lags.
#include "kernels.h"

namespace delrec {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ bf16x8 load16(i32x4 rs, uint32_t voff) {
    return __builtin_bit_cast(bf16x8, raw_buffer_load_i32x4(rs, (int)voff, 0, 0));
}

__device__ __forceinline__ float lagw_delay(const LagStepPack& p, int i, int j) {
    if (p.d) return p.d[(size_t)i * p.N + j];
    return p.base[j] + 0.0f + 1.0f * (float)p.off[(size_t)i * p.N + j];
}

// One thread per (8-block of the contracted neuron, output column); it reads its 8
// connections' weight, delay and half-width once and writes their 16-byte runs for every
// lag of both planes.
template <bool FWD>
__global__ void __launch_bounds__(256) pack_lagw_kernel(LagStepPack p) {
    const int NB = p.Nk / 8;
    const size_t total = (size_t)NB * p.Np;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int kb = (int)(idx / p.Np), col = (int)(idx - (size_t)kb * p.Np);
    float w[8], c[8], sv[8], s2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int i = FWD ? col : kb * 8 + e;
        const int j = FWD ? kb * 8 + e : col;
        const bool ok = i < p.N && j < p.N;
        const int ic = ok ? i : 0, jc = ok ? j : 0;
        w[e] = ok ? load_w(p.W, p.w_bf16, (size_t)ic * p.N + jc) : 0.0f;
        c[e] = 1.0f + lagw_delay(p, ic, jc);
        sv[e] = p.s ? p.s[jc] : p.s_uniform;
        s2[e] = sv[e] * sv[e];
    }
    const size_t plane = (size_t)p.Lw * NB * p.Np;
    for (int q = 0; q < p.Lw; ++q) {
        const float l = (float)(FWD ? p.Lw - q : q + 1);
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t h2[2], l2[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const float m = w[e + f] * tri_weight(l, c[e + f], sv[e + f], s2[e + f]);
                h2[f] = bf16_bits_rne(m);
                l2[f] = bf16_bits_rne(m - __uint_as_float(h2[f] << 16));
            }
            hi[e / 2] = h2[0] | (h2[1] << 16);
            lo[e / 2] = l2[0] | (l2[1] << 16);
        }
        const size_t o = ((size_t)q * NB + kb) * p.Np + col;
        p.out[o] = uint4{hi[0], hi[1], hi[2], hi[3]};
        p.out[plane + o] = uint4{lo[0], lo[1], lo[2], lo[3]};
    }
}

// ---------------------------------------------------------------------------------------
// Split-K GEMM of one step: part[ks][b][n] = sum over the split's k of A[b][k] * P[k][n].
// Workgroup: 128 rows x 2 WN columns (4 waves of 64 x WN, 4 x WN / 16 MFMA blocks each) and
// one k split; 32-k stages go global -> registers (S stages ahead, fixed register slots:
// the loop is unrolled over S) -> LDS (double-buffered, one barrier per stage) -> fragment
// registers (double-buffered: the next stage's fragments load while this stage multiplies).
// WN = 128 halves the LDS bytes read per MFMA (a wave reads 64 rows and 128 columns of a
// stage for 32 x PA blocks) -- the form of the long products; WN = 64 keeps more workgroups
// for the short ones.
// PA = 1: A x (P_hi + P_lo). PA = 2: A_hi x P_hi + A_hi x P_lo + A_lo x P_hi. PB = 1 (a one-
// plane P, e.g. bf16 weights): A x P, or A_hi x P + A_lo x P.
// Block order: workgroups are dealt to the 8 XCDs in turn (XCD = id mod 8), so when KS is a
// multiple of 8 each XCD takes KS / 8 whole k splits with all their row and column tiles:
// the A tile of a (row tile, split) and the P tile of a (column tile, split) are then
// fetched into one L2 and shared there by every workgroup that reads them. Otherwise (the
// per-block GEMM: many row tiles, few splits) each XCD takes a quarter of the row tiles
// times half of the column tiles, so each A tile is fetched by 2 XCDs and each P tile by 4.
template <int PA, int PB, int S, int WN>
__global__ void __launch_bounds__(256) lagstep_gemm_kernel(LagStepGemm p) {
    extern __shared__ uint4 lds_u4[];
    constexpr int NC = 2 * WN;            // workgroup columns
    constexpr int NBW = WN / 16;          // MFMA column blocks per wave
    constexpr int BH = NC / 64;           // uint4 of a P plane staged per thread per stage
    constexpr int BUF = PA * 512 + PB * 4 * NC;   // uint4 per LDS stage buffer
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const int NT = p.Np / NC;
    const int BT = (p.rows + 127) / 128;
    const int id = (int)blockIdx.x;
    int bt, nt, ks;
    if ((p.KS & 7) == 0) {
        const int xcd = id & 7, slot = id >> 3;
        const int kl = slot / (BT * NT), rem = slot - kl * (BT * NT);
        ks = xcd * (p.KS >> 3) + kl;
        bt = rem / NT;
        nt = rem - bt * NT;
    } else if ((BT & 3) == 0 && (NT & 1) == 0) {
        // each XCD takes a (BT / 4) x (NT / 2) block of tiles with every k split
        const int xcd = id & 7, slot = id >> 3;
        const int bb = BT >> 2, nn = NT >> 1;
        ks = slot / (bb * nn);
        const int rem = slot - ks * (bb * nn);
        bt = (xcd >> 1) * bb + rem / nn;
        nt = (xcd & 1) * nn + rem % nn;
    } else {
        bt = id / (NT * p.KS);
        const int rest = id - bt * (NT * p.KS);
        ks = rest / NT;
        nt = rest - ks * NT;
    }
    const int b0 = bt * 128, n0 = nt * NC;
    const int nst = p.Kt / 32;
    const int per = (nst + p.KS - 1) / p.KS;
    const int s0 = ks * per;
    const int ns = max(min(nst, s0 + per) - s0, 0);

    i32x4 ra[PA], rb[PB];
    const uint32_t abytes = (uint32_t)((size_t)p.B * p.lda * 2);
    ra[0] = buffer_rsrc(p.a0, abytes);
    if (PA > 1) ra[PA - 1] = buffer_rsrc(p.a1, abytes);
    const uint32_t pbytes = (uint32_t)((size_t)(p.Kt / 8) * p.Np * 16);
    rb[0] = buffer_rsrc(p.p0, pbytes);
    if (PB > 1) rb[PB - 1] = buffer_rsrc(p.p1, pbytes);
    // staging: thread tid stages A uint4 c = tid + 256 h (k-block c >> 7, row c & 127) and
    // P uint4 c = tid + 256 h (k-block c / NC, column c % NC)
    uint32_t oa[2], ob[BH];
    const uint32_t bstep = (uint32_t)(4 * p.Np * 16);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = tid + 256 * h, kb = c >> 7, r = c & 127;
        const int rr = b0 + r;   // rows past p.rows land past the descriptor's end: zeros
        oa[h] = (uint32_t)(((size_t)(rr / p.rp) * p.lda + (size_t)(rr % p.rp) * p.rs + p.aoff +
                            (size_t)s0 * 32 + kb * 8) * 2);
    }
#pragma unroll
    for (int h = 0; h < BH; ++h) {
        const int c = tid + 256 * h, kb = c / NC, r = c % NC;
        ob[h] = (uint32_t)((((size_t)s0 * 4 + kb) * p.Np + n0 + r) * 16);
    }
    uint4 sa[S][PA][2], sb[S][PB][BH];
    auto issue = [&](int slot) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int q = 0; q < PA; ++q)
                sa[slot][q][h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(ra[q], (int)oa[h], 0, 0));
            oa[h] += 64;
        }
#pragma unroll
        for (int h = 0; h < BH; ++h) {
#pragma unroll
            for (int q = 0; q < PB; ++q)
                sb[slot][q][h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(rb[q], (int)ob[h], 0, 0));
            ob[h] += bstep;
        }
    };
    auto stash = [&](int slot, int buf) {
#pragma unroll
        for (int q = 0; q < PA; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) lds_u4[buf * BUF + q * 512 + tid + 256 * h] = sa[slot][q][h];
#pragma unroll
        for (int q = 0; q < PB; ++q)
#pragma unroll
            for (int h = 0; h < BH; ++h) lds_u4[buf * BUF + PA * 512 + q * 4 * NC + tid + 256 * h] = sb[slot][q][h];
    };
    floatx4 acc[4][NBW];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) acc[mb][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

    bf16x8 fa[2][PA][4], fb[2][PB][NBW];  // fragments: the stage being multiplied and the next
    auto frags = [&](int f, int buf) {
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int q = 0; q < PA; ++q)
                fa[f][q][x] = __builtin_bit_cast(bf16x8, lds_u4[buf * BUF + q * 512 + g * 128 + wi * 64 + x * 16 + lc]);
#pragma unroll
        for (int x = 0; x < NBW; ++x)
#pragma unroll
            for (int q = 0; q < PB; ++q)
                fb[f][q][x] = __builtin_bit_cast(bf16x8, lds_u4[buf * BUF + PA * 512 + q * 4 * NC + g * NC + wj * WN + x * 16 + lc]);
    };

#pragma unroll
    for (int q = 0; q < S; ++q) issue(q);
    stash(0, 0);
    stash(1, 1);
    barrier_lds();
    frags(0, 0);
    static_assert(S % 2 == 0 && S >= 4, "an even number of register stages keeps the LDS buffer static");
    // iteration i: fragments of stage i + 1 are read (LDS buffer (i + 1) % 2, ready since the
    // last barrier) while stage i's are multiplied; stage i + 2 goes into buffer i % 2, whose
    // stage i is already in registers; the global loads run S stages ahead
    for (int s = 0; s < ns; s += S) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            issue(u);   // stage s + u + S into the slot stage s + u left (stashed two stages ago)
            frags((u + 1) & 1, (u + 1) & 1);
            if (s + u < ns) {
                const int f = u & 1;
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                    for (int nb = 0; nb < NBW; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[f][0][mb], fb[f][0][nb], acc[mb][nb], 0, 0, 0);
                if (PB > 1) {
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                        for (int nb = 0; nb < NBW; ++nb)
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[f][0][mb], fb[f][PB - 1][nb], acc[mb][nb], 0, 0, 0);
                }
                if (PA > 1) {
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                        for (int nb = 0; nb < NBW; ++nb)
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[f][PA - 1][mb], fb[f][0][nb], acc[mb][nb], 0, 0, 0);
                }
            }
            stash((u + 2) % S, u & 1);
            barrier_lds();
        }
    }

    float* out = p.part + (size_t)ks * p.rows * p.Np;
    if (p.cm) {
        // column-major: a lane's 4 accumulator rows are 16 contiguous bytes of its column
        // (16-byte aligned when the row count is a multiple of 4)
        const bool v4 = (p.rows & 3) == 0;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int r = b0 + wi * 64 + mb * 16 + 4 * g;
#pragma unroll
            for (int nb = 0; nb < NBW; ++nb) {
                float* o = out + (size_t)(n0 + wj * WN + nb * 16 + lc) * p.rows + r;
                if (v4 && r + 3 < p.rows) {
                    *reinterpret_cast<floatx4*>(o) = acc[mb][nb];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (r + e < p.rows) o[e] = acc[mb][nb][e];
                }
            }
        }
        return;
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = b0 + wi * 64 + mb * 16 + 4 * g + e;
            if (r >= p.rows) continue;
#pragma unroll
            for (int nb = 0; nb < NBW; ++nb) out[(size_t)r * p.Np + n0 + wj * WN + nb * 16 + lc] = acc[mb][nb][e];
        }
}

// The same product in 256 x 256 tiles for a two-plane A and a one-plane P (the hybrid's
// per-block far product): 8 waves of 64 x 128 (4 x 8 MFMA blocks, 128 accumulator registers
// each; a 4-wave 128 x 128 split needs all 256 AGPRs and the register allocator shuffles
// them) and one k split per workgroup. A 32-k stage moves 256 rows x 2 planes of A and 256
// columns of P through LDS (48 KB, double-buffered) from one register stage of global loads
// (in flight while the previous stage multiplies): half the staged bytes per MFMA of the
// 128 x 256 tile. Row mapping and partial layout (row-major) as lagstep_gemm_kernel.
__global__ void __launch_bounds__(512) lagstep_gemm256_kernel(LagStepGemm p) {
    extern __shared__ uint4 lds_u4[];
    constexpr int TR = 256, NC = 256;
    constexpr int ABUF = 2 * 4 * TR;      // A: plane q, k-block kb, row r at q * 1024 + kb * 256 + r
    constexpr int BUF = ABUF + 4 * NC;    // P: k-block kb, column c at ABUF + kb * 256 + c
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const int NT = p.Np / NC;
    const int id = (int)blockIdx.x;
    const int ks = id % p.KS, tile = id / p.KS;
    const int bt = tile / NT, nt = tile - bt * NT;
    const int b0 = bt * TR, n0 = nt * NC;
    const int nst = p.Kt / 32;
    const int per = (nst + p.KS - 1) / p.KS;
    const int s0 = ks * per;
    const int ns = max(min(nst, s0 + per) - s0, 0);

    const uint32_t abytes = (uint32_t)((size_t)p.B * p.lda * 2);
    const i32x4 ra0 = buffer_rsrc(p.a0, abytes), ra1 = buffer_rsrc(p.a1, abytes);
    const uint32_t pbytes = (uint32_t)((size_t)(p.Kt / 8) * p.Np * 16);
    const i32x4 rb = buffer_rsrc(p.p0, pbytes);
    // staging: thread tid stages A uint4 c = tid + 512 h (k-block c >> 8, row c & 255) of both
    // planes and P uint4 c = tid + 512 h (k-block c >> 8, column c & 255), h < 2
    uint32_t oa[2], ob[2];
    const uint32_t bstep = (uint32_t)(4 * p.Np * 16);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = tid + 512 * h, kb = c >> 8, r = c & 255;
        const int rr = b0 + r;   // rows past p.rows land past the descriptor's end: zeros
        oa[h] = (uint32_t)(((size_t)(rr / p.rp) * p.lda + (size_t)(rr % p.rp) * p.rs + p.aoff +
                            (size_t)s0 * 32 + kb * 8) * 2);
        ob[h] = (uint32_t)((((size_t)s0 * 4 + kb) * p.Np + n0 + r) * 16);
    }
    uint4 sa[2][2], sb[2];   // one register stage: [plane][h], [h]
    auto issue = [&]() {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            sa[0][h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(ra0, (int)oa[h], 0, 0));
            sa[1][h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(ra1, (int)oa[h], 0, 0));
            oa[h] += 64;
            sb[h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(rb, (int)ob[h], 0, 0));
            ob[h] += bstep;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            lds_u4[buf * BUF + tid + 512 * h] = sa[0][h];
            lds_u4[buf * BUF + 1024 + tid + 512 * h] = sa[1][h];
            lds_u4[buf * BUF + ABUF + tid + 512 * h] = sb[h];
        }
    };
    floatx4 acc[4][8];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf) {
        bf16x8 fb[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
            fb[nb] = __builtin_bit_cast(bf16x8, lds_u4[buf * BUF + ABUF + g * 256 + wj * 128 + nb * 16 + lc]);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const bf16x8 a0 = __builtin_bit_cast(bf16x8, lds_u4[buf * BUF + g * 256 + wi * 64 + mb * 16 + lc]);
            const bf16x8 a1 = __builtin_bit_cast(bf16x8, lds_u4[buf * BUF + 1024 + g * 256 + wi * 64 + mb * 16 + lc]);
#pragma unroll
            for (int nb = 0; nb < 8; ++nb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, fb[nb], acc[mb][nb], 0, 0, 0);
#pragma unroll
            for (int nb = 0; nb < 8; ++nb)
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, fb[nb], acc[mb][nb], 0, 0, 0);
        }
    };

    issue();
    stash(0);
    barrier_lds();
    issue();
    // stage s in LDS buffer s % 2 while stage s + 1's loads are in flight in the registers;
    // those go to the other buffer after stage s multiplies, then stage s + 2's loads issue
    // (past the last stage they read zeros or bytes no stage uses)
    for (int s = 0; s < ns; ++s) {
        compute(s & 1);
        stash((s + 1) & 1);
        barrier_lds();
        issue();
    }

    float* out = p.part + (size_t)ks * p.rows * p.Np;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = b0 + wi * 64 + mb * 16 + 4 * g + e;
            if (r >= p.rows) continue;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) out[(size_t)r * p.Np + n0 + wj * 128 + nb * 16 + lc] = acc[mb][nb][e];
        }
}

// ---------------------------------------------------------------------------------------
// Far lags of a block of P steps without LDS:
//   out[tt][b][n] = sum_q sum_k H[b][(base + tt + q) * Nk + k] * M[q][k][n],  q < Lf, tt < P,
// the Hankel form of the block rows (row tt reads the history shifted by tt slices). For a
// 32-k chunk the loop walks q: M(q) is loaded once and multiplied by the P history slices
// q .. q + P - 1, which stay in a register window of W slots (slice sigma in slot sigma mod W,
// refilled W - P slices ahead after its last reader, like the windowed lag GEMM), the M
// slices rotating through SM slots. A wave owns 32 rows x 32 columns x P block rows (the P
// accumulator sets in AGPRs); slices of q >= Lf read zeros through the M descriptor's bound.
template <int PA, int P, int W, int SM>
__global__ void __launch_bounds__(256) lagblock_kernel(LagStepGemm p) {
    static_assert(W % SM == 0 && W > P, "window slots");
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const int BT = (p.B + 63) / 64, NT = p.Np / 64;
    const int id = (int)blockIdx.x;
    int bt, nt, ks;
    if ((BT * NT * p.KS) % 8 == 0 && (NT * p.KS) % 8 == 0) {
        // the BT row tiles that share an M tile (column tile, split) sit on one XCD
        const int xcd = id & 7, slot = id >> 3;
        bt = slot % BT;
        const int pair = (slot / BT) * 8 + xcd;
        ks = pair / NT;
        nt = pair - ks * NT;
    } else {
        bt = id % BT;
        const int rest = id / BT;
        nt = rest % NT;
        ks = rest / NT;
    }
    const int b0 = bt * 64 + wi * 32, n0 = nt * 64 + wj * 32;
    const int nch = p.Nk / 32;                       // 32-k chunks of one lag slice
    const int per = (nch + p.KS - 1) / p.KS;
    const int c0 = ks * per, c1 = min(nch, c0 + per);
    const int Lf = p.Kt / p.Nk;

    i32x4 rh[PA], rm[2];
    const uint32_t hbytes = (uint32_t)((size_t)p.B * p.lda * 2);
    rh[0] = buffer_rsrc(p.a0, hbytes);
    if (PA > 1) rh[PA - 1] = buffer_rsrc(p.a1, hbytes);
    const uint32_t qstep = (uint32_t)((size_t)(p.Nk / 8) * p.Np * 16);   // bytes per lag slice
    rm[0] = buffer_rsrc(p.p0, (uint32_t)Lf * qstep);
    rm[1] = buffer_rsrc(p.p1, (uint32_t)Lf * qstep);
    const uint32_t hstep = (uint32_t)p.Nk * 2;                           // bytes per history slice
    uint32_t vh[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
        vh[mb] = (uint32_t)(((size_t)(b0 + mb * 16 + lc) * p.lda + p.aoff + 8 * g) * 2);
    const uint32_t vm = (uint32_t)((size_t)g * p.Np + n0 + lc) * 16;

    floatx4 acc[P][2][2];
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) acc[t][mb][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int c = c0; c < c1; ++c) {
        bf16x8 hw[W][PA][2], mw[SM][2][2];
        // history slices 0 .. W - 2 of this chunk, M slices 0 .. SM - 2
        uint32_t oh = (uint32_t)c * 64;   // byte offset of the chunk within a slice
        uint32_t om = vm + (uint32_t)c * 4 * p.Np * 16;
#pragma unroll
        for (int sl = 0; sl < W - 1; ++sl) {
#pragma unroll
            for (int q = 0; q < PA; ++q)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) hw[sl][q][mb] = load16(rh[q], vh[mb] + oh);
            oh += hstep;
        }
#pragma unroll
        for (int sl = 0; sl < SM - 1; ++sl) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                mw[sl][q][0] = load16(rm[q], om);
                mw[sl][q][1] = load16(rm[q], om + 256);
            }
            om += qstep;
        }
        for (int q0 = 0; q0 < Lf; q0 += W) {
#pragma unroll
            for (int u = 0; u < W; ++u) {
                // refill: history slice q + W - 1 into the slot slice q - 1 left, M(q + SM - 1)
#pragma unroll
                for (int q = 0; q < PA; ++q)
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb) hw[(u + W - 1) % W][q][mb] = load16(rh[q], vh[mb] + oh);
                oh += hstep;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    mw[(u + SM - 1) % SM][q][0] = load16(rm[q], om);
                    mw[(u + SM - 1) % SM][q][1] = load16(rm[q], om + 256);
                }
                om += qstep;
                __builtin_amdgcn_sched_barrier(0);
                const int sm = u % SM;
#pragma unroll
                for (int t = 0; t < P; ++t)
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
                            acc[t][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                hw[(u + t) % W][0][mb], mw[sm][0][nb], acc[t][mb][nb], 0, 0, 0);
#pragma unroll
                for (int t = 0; t < P; ++t)
#pragma unroll
                    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
                            acc[t][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                hw[(u + t) % W][0][mb], mw[sm][1][nb], acc[t][mb][nb], 0, 0, 0);
                if (PA > 1) {
#pragma unroll
                    for (int t = 0; t < P; ++t)
#pragma unroll
                        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                            for (int nb = 0; nb < 2; ++nb)
                                acc[t][mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                    hw[(u + t) % W][PA - 1][mb], mw[sm][0][nb], acc[t][mb][nb], 0, 0, 0);
                }
            }
        }
    }

    float* out = p.part + (size_t)ks * p.rows * p.Np;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int b = b0 + mb * 16 + 4 * g + e;
            if (b >= p.B) continue;
#pragma unroll
            for (int t = 0; t < P; ++t)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    out[((size_t)b * P + t) * p.Np + n0 + nb * 16 + lc] = acc[t][mb][nb][e];
        }
}

// ---------------------------------------------------------------------------------------
// LIF steps. One thread per (b, neuron) over the padded width Nk: the history columns past
// N are written as zeros.

// forward step t: rec = sum_ks part + bias; u = charge(v, x + rec * m); spike, reset; outputs
// y, u, the spike bit, and y(t) into the history at time index t + Lw
__global__ void __launch_bounds__(256) lagstep_lif_fwd_kernel(LagStepLif p) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)p.B * p.Nk) return;
    const int b = (int)(idx / p.Nk), i = (int)(idx - (size_t)b * p.Nk);
    const int t = p.t;
    uint16_t* hrow = p.hist + (size_t)b * p.lda + (size_t)(t + p.Lw) * p.Nk;
    if (i >= p.N) {
        hrow[i] = 0;
        return;
    }
    const Lif k = p.lif;
    const size_t bi = (size_t)b * p.N + i;
    // the partial sums in a fixed order; unrolled so that their loads are in flight together
    float r = 0.0f;
#pragma unroll 8
    for (int q = 0; q < p.KS; ++q) r += p.part[((size_t)q * p.B + b) * p.Np + i];
#pragma unroll 4
    for (int q = 0; q < p.KSF; ++q) r += p.fpart[((size_t)q * p.B * p.P + (size_t)b * p.P + p.tt) * p.Np + i];
    r += p.bias ? p.bias[i] : 0.0f;
    const float m = p.drop ? p.drop[bi] : 1.0f;
    const size_t o = (size_t)t * p.B * p.N + bi;
    const float a = p.x[o] + r * m;
    const float v = t == 0 ? k.v0 : p.state[bi];
    const float u = lif_charge(k, v, a);
    const float y = lif_fire(k, u);
    p.state[bi] = lif_reset(k, u, y);
    p.y[o] = y;
    p.u[o] = u;
    const int TW = (p.T + 31) >> 5;
    uint32_t* wp = p.bits + ((size_t)b * TW + (t >> 5)) * p.N + i;
    const uint32_t bit = (y != 0.0f ? 1u : 0u) << (t & 31);
    *wp = (t & 31) == 0 ? bit : (*wp | bit);
    hrow[i] = y != 0.0f ? 0x3F80 : 0;
}

// backward step t: gfut = sum_ks part; du = LIF backward (gy + gfut, u, y, lam); dx, gr, the
// db partial, and gr(t) split into the hi / lo histories
__global__ void __launch_bounds__(256) lagstep_lif_bwd_kernel(LagStepLif p) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)p.B * p.Nk) return;
    const int b = (int)(idx / p.Nk), j = (int)(idx - (size_t)b * p.Nk);
    const int t = p.t;
    const size_t ho = (size_t)b * p.lda + (size_t)t * p.Nk + j;
    if (j >= p.N) {
        p.hist[ho] = 0;
        p.hist2[ho] = 0;
        return;
    }
    const Lif k = p.lif;
    const size_t bj = (size_t)b * p.N + j;
    float gf = 0.0f;
#pragma unroll 8
    for (int q = 0; q < p.KS; ++q) gf += p.part[((size_t)q * p.B + b) * p.Np + j];
#pragma unroll 4
    for (int q = 0; q < p.KSF; ++q) gf += p.fpart[((size_t)q * p.B * p.P + (size_t)b * p.P + p.tt) * p.Np + j];
    const size_t o = (size_t)t * p.B * p.N + bj;
    const float u = p.u[o];
    const float y = lif_fire(k, u);
    const bool last = t == p.T - 1;
    const float lam = last ? 0.0f : p.state[bj];
    const float du = lif_backward(k, p.gy[o] + gf, u, y, lam);
    p.state[bj] = k.decay * du;
    const float da = lif_dx(k, du);
    const float gr = da * (p.drop ? p.drop[bj] : 1.0f);
    p.dx[o] = da;
    if (p.drop) p.gr[o] = gr;   // else gr == dx: the lag correlation reads dx
    p.dbp[bj] = last ? gr : p.dbp[bj] + gr;
    const uint32_t hi = bf16_bits_rne(gr);
    p.hist[ho] = (uint16_t)hi;
    p.hist2[ho] = (uint16_t)bf16_bits_rne(gr - __uint_as_float(hi << 16));
}

__global__ void fill_u4_kernel(uint4* __restrict__ p, size_t n) {
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (size_t)gridDim.x * blockDim.x)
        p[q] = uint4{0u, 0u, 0u, 0u};
}

// h[b * lda + off0 + e] = 0 for b < B, e < n
__global__ void fill_rows_u16_kernel(uint16_t* __restrict__ h, int B, size_t lda, size_t off0, size_t n) {
    const size_t total = (size_t)B * n;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
        const size_t b = q / n;
        h[b * lda + off0 + (q - b * n)] = 0;
    }
}

// ---------------------------------------------------------------------------------------

// k splits of a per-step GEMM: none when the tiles alone fill three quarters of the CUs;
// else enough workgroups for every CU, rounded up to a multiple of 8 where that keeps to two
// workgroups per CU and the k range allows, so that each XCD takes whole splits (its L2 then
// holds only its k slice of both operands, fetched once) -- e.g. 512 x 2048 outputs with
// k = 10240: 8 splits of 64 tiles rather than 4, which leave each XCD a column half of the
// operand
int lagstep_splits(int B, int Np, int Kt, int cus, int nc) {
    const int tiles = ((B + 127) / 128) * (Np / nc);
    if (tiles * 4 >= cus * 3) return 1;
    const int nst = Kt / 32;
    const int cap = std::max(1, nst / 8);
    int ks = std::max(1, std::min((cus + tiles - 1) / tiles, cap));
    const int up = (ks + 7) / 8 * 8;
    if (ks > 1 && up <= cap && tiles * up <= 2 * cus) ks = up;
    return ks;
}

void launch_pack_lagw(const LagStepPack& a, bool fwd, hipStream_t stream) {
    const size_t total = (size_t)(a.Nk / 8) * a.Np;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (fwd)
        hipLaunchKernelGGL(pack_lagw_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(pack_lagw_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
}

// zero rows [t0, t1) of every batch row of a [B][lda / Nk][Nk] history
void launch_hist_zero(uint16_t* h, int B, size_t lda, int Nk, int t0, int t1, hipStream_t stream) {
    const size_t n = (size_t)(t1 - t0) * Nk;
    if (n == 0) return;
    const unsigned blocks = (unsigned)std::min<size_t>(((size_t)B * n + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_rows_u16_kernel, dim3(blocks), dim3(256), 0, stream, h, B, lda, (size_t)t0 * Nk, n);
}

// the whole history (B * lda bf16; lda is a multiple of 32): the far-lag kernel's window
// reads a few slices past its last lag, which must hold finite values (0 * NaN is NaN)
void launch_hist_clear(uint16_t* h, int B, size_t lda, hipStream_t stream) {
    const size_t n = (size_t)B * lda / 8;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(fill_u4_kernel, dim3(blocks), dim3(256), 0, stream, reinterpret_cast<uint4*>(h), n);
}

constexpr int kLagStepStages = 4;
constexpr int kLagStepBlock = 8;   // steps per block (near lags per step)
int lagstep_block() { return kLagStepBlock; }

size_t lagstep_gemm_lds(int pa, int pb, int wn) {
    return (size_t)2 * (pa * 512 + pb * 4 * 2 * wn) * sizeof(uint4);
}

#define DELREC_LAGSTEP_GEMM(PAV, PBV, WNV)                                                     \
    if (pa == PAV && pb == PBV && wn == WNV) {                                                 \
        ensure_lds((const void*)lagstep_gemm_kernel<PAV, PBV, kLagStepStages, WNV>, lds);     \
        hipLaunchKernelGGL((lagstep_gemm_kernel<PAV, PBV, kLagStepStages, WNV>), dim3(grid), dim3(256), lds, \
                           stream, g);                                                         \
        return;                                                                                \
    }

// wn = 128 (128 x 256 tiles; Np a multiple of 256) for a one-plane P, else 64
void launch_lagstep_gemm(const LagStepGemm& g, int pa, hipStream_t stream, int pb, int wn) {
    const int grid = ((g.rows + 127) / 128) * (g.Np / (2 * wn)) * g.KS;
    const size_t lds = lagstep_gemm_lds(pa, pb, wn);
    DELREC_LAGSTEP_GEMM(1, 2, 64)
    DELREC_LAGSTEP_GEMM(2, 2, 64)
    DELREC_LAGSTEP_GEMM(2, 1, 64)
    DELREC_LAGSTEP_GEMM(2, 1, 128)
}

// k splits of lagstep_gemm256_kernel: enough workgroups for the CUs, at least 8 stages each
int lagstep_gemm256_splits(int rows, int Np, int Kt, int cus) {
    const int tiles = ((rows + 255) / 256) * (Np / 256);
    const int cap = std::max(1, Kt / 32 / 8);
    return std::max(1, std::min((cus + tiles - 1) / tiles, cap));
}

size_t lagstep_gemm256_lds() { return (size_t)2 * (2 * 4 * 256 + 4 * 256) * sizeof(uint4); }

void launch_lagstep_gemm256(const LagStepGemm& g, hipStream_t stream) {
    const int grid = ((g.rows + 255) / 256) * (g.Np / 256) * g.KS;
    const size_t lds = lagstep_gemm256_lds();
    ensure_lds((const void*)lagstep_gemm256_kernel, lds);
    hipLaunchKernelGGL(lagstep_gemm256_kernel, dim3(grid), dim3(512), lds, stream, g);
}

// far lags of a block: rows (b, tt) of g.part with g.rp == kLagStepBlock
int lagblock_splits(int B, int Np, int Nk, int cus) {
    const int tiles = ((B + 63) / 64) * (Np / 64);
    const int nch = Nk / 32;
    const int want = (cus + tiles - 1) / tiles;
    return std::max(1, std::min(want, nch));
}

void launch_lagblock(const LagStepGemm& g, int pa, hipStream_t stream) {
    const int grid = ((g.B + 63) / 64) * (g.Np / 64) * g.KS;
    if (pa == 1)
        hipLaunchKernelGGL((lagblock_kernel<1, kLagStepBlock, 12, 4>), dim3(grid), dim3(256), 0, stream, g);
    else
        hipLaunchKernelGGL((lagblock_kernel<2, kLagStepBlock, 10, 2>), dim3(grid), dim3(256), 0, stream, g);
}

void launch_lagstep_lif(const LagStepLif& l, bool fwd, hipStream_t stream) {
    const size_t n = (size_t)l.B * l.Nk;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (fwd)
        hipLaunchKernelGGL(lagstep_lif_fwd_kernel, dim3(blocks), dim3(256), 0, stream, l);
    else
        hipLaunchKernelGGL(lagstep_lif_bwd_kernel, dim3(blocks), dim3(256), 0, stream, l);
}

}  // namespace delrec
