// Hybrid scans with the integer offsets as the lag axis, on bf16 MFMA (gfx950): the form for
// hybrid delays d_ij = base_j + off_ij whose rings do not fit one CU's LDS. The reference runs
// the hybrid as its per-connection scatter / gather (synaptic_eventdriven.py:106-164,
// :323-364, launched by synaptic_hybrid.py:139-211).
//
// Write off_ij = omin + e_ij with e in [0, D), and give each source the triangle of its
// smallest delay, c_j = 1 + (base_j + omin), with its KF taps h_j(lof_j + f), f < KF (every
// lag >= 1: the entry point checks d_min >= s - 1). Connection (i, j)'s taps are then the
// source's, shifted by e_ij steps:
//   rec_i(t)  = sum_j W_ij sum_f h_j(lof_j + f) y_j(t - lof_j - f - e_ij)
//             = sum_e sum_j W^(e)_ij z_j(t - e),  z_j(t) = sum_f h_j(lof_j + f) y_j(t - lof_j - f),
//   gfut_j(t) = sum_i W_ij sum_f h_j(lof_j + f) gr_i(t + lof_j + f + e_ij)
//             = sum_f h_j(lof_j + f) G_j(t + lof_j + f),  G_j(tau) = sum_e sum_i W^(e)_ij gr_i(tau + e),
// with W^(e) = W * [off - omin == e] (exact in bf16 for bf16 W). z_j is the source's axonal
// trace and G the offset-stacked product. Each step runs one (B x D*N) by (D*N x N) product
// over a batch-major history window -- the lag-stacked GEMM of lagstep.hip with the D offsets
// in place of the L - 1 lags (C5: 5 products per connection instead of 66) -- and one LIF
// launch that adds the split-K partials in a fixed order. (The forward of bf16 W takes the
// scatter on arrival further down, which walks only the spikes.)
//
// The per-source time shift lof_j sits on the contracted side in the forward (z_j is formed
// by the LIF thread that owns neuron j, from its own spike-history word), and on the output
// side in the backward: G_j(tau) is first needed at step tau - lof_j. So the backward splits
// the sources: "near" ones (lof_j < P) get G_j(t + 1) from a per-step product over their
// columns only, "far" ones (lof_j >= P) get G_j(tau) for the P steps tau = t0 + 1 .. t0 + P of a
// block from one product at the block's start t0 whose rows are (b, tau) -- every one of
// those G is first read at a step <= t0, and the history it reads (gr(t0 + 1 ..)) is complete.
// For C5 (lof_j = floor(base_j) + 1, base U[0, 60], P = 4) the per-step product shrinks to the
// 5 % of near columns and the rest runs as 2048-row products. Both write a ring of G_j(tau)
// in a [slot][j][b] layout (b fastest, whole 256-byte rows through an LDS transpose); the
// per-step LIF reads G_j(t + lof_j + f) from it.
//
// Precision: spikes are exact; z and gr are split into bf16 hi + lo planes (relative error
// about 2^-16); W^(e) is one bf16 plane for bf16 W, or hi + lo planes for fp32 W
// (hi*hi + hi*lo + lo*hi). Accumulation is fp32. Connection (i, j)'s triangle is evaluated at
// c_j + e_ij where the reference evaluates 1 + fp32(base_j + off_ij): the two differ only when
// that sum rounds in fp32, by at most half an ulp of the delay (about 4e-6 at d = 60).
#include "kernels.h"

namespace delrec {

namespace {

typedef __bf16 bf16x8h __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t hyb_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

}  // namespace

// P[(q, kk), col] for q < D offset slices of the contracted neuron kk:
//   forward  (contracted j, output i): W_ij when off_ij - omin == D - 1 - q (slice q ascending
//            is time ascending: history slice t + q of step t holds z(t - D + 1 + q));
//   backward (contracted i, output j): W_ij when off_ij - omin == q.
// One thread per (8-block of the contracted neuron, output column), k-blocked layout
// ((k / 8) * Np + col) * 8 + k % 8; planes: hi (and lo for fp32 W).
template <bool FWD>
__global__ void __launch_bounds__(256) hyb_pack_kernel(HybPack p) {
    const int NB = p.Nk / 8;
    const size_t total = (size_t)NB * p.Np;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int kb = (int)(idx / p.Np), col = (int)(idx - (size_t)kb * p.Np);
    float w[8];
    int e8[8];
    // backward columns through the optional source permutation (columns past nc are 0)
    const int jc = (!FWD && p.perm) ? (col < p.nc ? p.perm[p.c0 + col] : p.N) : col;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int i = FWD ? col : kb * 8 + e;
        const int j = FWD ? kb * 8 + e : jc;
        const bool ok = i < p.N && j < p.N;
        const size_t c = ok ? (size_t)i * p.N + j : 0;
        w[e] = ok ? load_w(p.W, p.w_bf16, c) : 0.0f;
        e8[e] = ok ? (int)p.off[c] - p.omin : -1;   // -1: no connection
        if (ok && e8[e] < 0) e8[e] = -2;               // -2: outside the range
    }
    // an offset outside the caller's range [omin, omin + D) would drop its connection: it is
    // packed as a NaN weight in slice 0 instead, so that the products it enters become NaN
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (e8[e] >= p.D) e8[e] = -2;
    const size_t plane = (size_t)p.D * NB * p.Np;
    for (int q = 0; q < p.D; ++q) {
        const int want = FWD ? p.D - 1 - q : q;
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t h2[2], l2[2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int ef = e8[e + f];
                const float m = ef == want ? w[e + f] : (ef < -1 && q == 0 ? __builtin_nanf("") : 0.0f);
                h2[f] = hyb_bf16_rne(m);
                l2[f] = hyb_bf16_rne(m - __uint_as_float(h2[f] << 16));
            }
            hi[e / 2] = h2[0] | (h2[1] << 16);
            lo[e / 2] = l2[0] | (l2[1] << 16);
        }
        const size_t o = ((size_t)q * NB + kb) * p.Np + col;
        p.out[o] = uint4{hi[0], hi[1], hi[2], hi[3]};
        if (p.planes > 1) p.out[plane + o] = uint4{lo[0], lo[1], lo[2], lo[3]};
    }
}

// Each source's first lag of non-zero weight lof_j and its KF tap weights h[f * N + j] at the
// smallest offset: c_j = 1 + (base_j + 0 + 1 * omin), the parametrisation's fp32 sum.
// The offset-stacked and arrival forms need that first lag >= 1 for every source (the
// caller's d_min = min_j base_j + omin >= s - 1); a source that breaks it would lose the taps
// of lags < 1 silently, so its taps are written as NaN instead (every output it reaches
// becomes NaN).
__global__ void __launch_bounds__(256) hyb_taps_kernel(HybTaps p) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= p.N) return;
    const float c = 1.0f + (p.base[j] + 0.0f + 1.0f * (float)p.omin);
    const float s = p.s, s2 = s * s;
    const int first = (int)floorf(c - s) + 1;
    const int lof = max(1, first);
    p.lof[j] = lof;
    const bool bad = first < 1;
    for (int f = 0; f < p.KF; ++f)
        p.h[(size_t)f * p.N + j] = bad ? __builtin_nanf("") : tri_weight((float)(lof + f), c, s, s2);
}

// Forward step t, one thread per (b, neuron i) over the padded width Nk: rec = sum_ks part +
// bias; u = charge(v, x + rec * m); spike, reset; outputs y, u and the spike bit; the
// neuron's spike-history word(s) (bit k = y(t - k)) and, as a source, its trace z(t + 1)
// split into the hi / lo history planes at slice t + D.
template <int HW>
__global__ void __launch_bounds__(256) hyb_lif_fwd_kernel(HybLif p) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)p.B * p.Nk) return;
    const int b = (int)(idx / p.Nk), i = (int)(idx - (size_t)b * p.Nk);
    const int t = p.t;
    const size_t ho = (size_t)b * p.lda + (size_t)(t + p.D) * p.Nk + i;
    if (i >= p.N) {
        p.hhi[ho] = 0;
        p.hlo[ho] = 0;
        return;
    }
    const Lif k = p.lif;
    const size_t BN = (size_t)p.B * p.N, bi = (size_t)b * p.N + i;
    float r = 0.0f;
#pragma unroll 8
    for (int q = 0; q < p.KS; ++q) r += p.part[((size_t)q * p.B + b) * p.Np + i];
    r += p.bias ? p.bias[i] : 0.0f;
    const float m = p.drop ? p.drop[bi] : 1.0f;
    const size_t o = (size_t)t * BN + bi;
    const float a = p.x[o] + r * m;
    const float v = t == 0 ? k.v0 : p.state[bi];
    const float u = lif_charge(k, v, a);
    const float y = lif_fire(k, u);
    p.state[bi] = lif_reset(k, u, y);
    p.y[o] = y;
    p.u[o] = u;
    const int TW = (p.T + 31) >> 5;
    uint32_t* wp = p.bits + ((size_t)b * TW + (t >> 5)) * p.N + i;
    const uint32_t yb = y != 0.0f ? 1u : 0u;
    *wp = (t & 31) == 0 ? (yb << (t & 31)) : (*wp | (yb << (t & 31)));
    uint64_t h[HW];
#pragma unroll
    for (int w = 0; w < HW; ++w) h[w] = t == 0 ? 0ull : p.hist[(size_t)w * BN + bi];
#pragma unroll
    for (int w = HW - 1; w > 0; --w) h[w] = (h[w] << 1) | (h[w - 1] >> 63);
    h[0] = (h[0] << 1) | (uint64_t)yb;
#pragma unroll
    for (int w = 0; w < HW; ++w) p.hist[(size_t)w * BN + bi] = h[w];
    // z(t + 1) = sum_f h(lof + f) y(t + 1 - lof - f): bit lof + f - 1 of the history
    const int lof = p.lof[i];
    float z = 0.0f;
    for (int f = 0; f < p.KF; ++f) {
        const int kb = lof + f - 1;
        const uint64_t word = HW == 1 ? h[0] : (kb < 64 ? h[0] : h[HW - 1]);
        const float hf = p.h[(size_t)f * p.N + i];
        z += ((word >> (kb & 63)) & 1ull) ? hf : 0.0f;
    }
    const uint32_t hi = hyb_bf16_rne(z);
    p.hhi[ho] = (uint16_t)hi;
    p.hlo[ho] = (uint16_t)hyb_bf16_rne(z - __uint_as_float(hi << 16));
}

// Backward step t over a tile of 16 sources / neurons j0 .. j0 + 15 x 64 batch rows (256
// threads; 1024 workgroups at C5: twice the loads in flight of 32-source tiles, which were
// 2 % slower, and 8-source tiles 9 %), three phases:
//  1 G_j(t + 1) of the tile's near sources, the near product's columns ntile[x] ..
//    ntile[x + 1] - 1: sum_ks npart[ks][c][b] in a fixed order (column-major partials, one
//    column per wave, 16 partials in flight per lane), into LDS;
//  2 (transposed: one source per wave at a time, its 64 batch rows on the lanes): those
//    G(t + 1) into ring slot (t + 1) mod R; then gfut_j(t) = sum_f h_j(lof_j + f) G_j(t + lof_j
//    + f), from LDS for tau = t + 1 (lof_j = 1, f = 0: always a near source) and from the
//    ring otherwise (0 for tau >= T: gr past the last step is 0), all ring reads of the
//    wave's sources issued before any is used;
//  3 (row-major): the LIF backward on gy + gfut, outputs dx (and gr when it differs), the db
//    partial, and gr(t) split into the hi / lo history planes at slice t.
// The ring slot of tau is rewritten with G(tau - R) only after every step that reads G(tau)
// (steps >= tau - L + 1) has run, for R >= L - 1; this step's reads (tau >= t + 2) and writes
// (tau = t + 1) never share a slot.
constexpr int kHybTapsMax = 8;
constexpr int kHybBwdTile = 16;

template <int KF>
__global__ void __launch_bounds__(256) hyb_bwd_lif_kernel(HybBwd p) {
    constexpr int JT = kHybBwdTile;
    __shared__ float sg[JT][65];
    __shared__ float sf[JT][65];
    __shared__ int ncl[JT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j0 = blockIdx.x * JT, b0 = blockIdx.y * 64;
    const int t = p.t, N = p.N, B = p.B, T = p.T, R = p.R;
    const int lo = p.ntile[blockIdx.x], nn = p.ntile[blockIdx.x + 1] - lo;
    if (tid < JT) ncl[tid] = -1;
    // loads that do not wait for this step's G, issued first so that their latency overlaps
    // phases 1 and 2: the LIF operands of phase 3 and the ring reads of phase 2
    // phase 3 lays a wave over LR = 64 / JT rows of JT columns; 4 LR rows per pass
    constexpr int LR = 64 / JT;
    const int jl3 = lane & (JT - 1), j3 = j0 + jl3;
    const int r0 = LR * w + lane / JT;
    const size_t BN = (size_t)B * N;
    const bool last = t == T - 1;
    constexpr int E3 = 64 / (4 * LR);
    float uu[E3], gyv[E3], lam[E3], dbv[E3], mv[E3];
#pragma unroll
    for (int e = 0; e < E3; ++e) {
        const int b = b0 + r0 + 4 * LR * e;
        const bool ok = b < B && j3 < N;
        const size_t bj = (size_t)(ok ? b : 0) * N + (ok ? j3 : 0), o = (size_t)t * BN + bj;
        uu[e] = ok ? p.u_in[o] : 0.0f;
        gyv[e] = ok ? p.gy[o] : 0.0f;
        lam[e] = (ok && !last) ? p.state[bj] : 0.0f;
        dbv[e] = (ok && !last && p.dbp) ? p.dbp[bj] : 0.0f;
        mv[e] = (ok && p.drop) ? p.drop[bj] : 1.0f;
    }
    constexpr int E = JT / 4;
    const int tm = t % R;
    float got[E][KF], hv[E][KF];
    int lofv[E];
    {
        const int b = b0 + lane;
        const bool bok = b < B;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = j0 + w + 4 * e;
            lofv[e] = j < N ? p.lof[j] : 0;
#pragma unroll
            for (int f = 0; f < KF; ++f) {
                hv[e][f] = (j < N && f < p.KF) ? p.h[(size_t)f * N + j] : 0.0f;
                const int d = lofv[e] + f;   // tau - t, in [1, L - 1]
                int sl = tm + d;
                sl = sl >= R ? sl - R : sl;
                // tau >= t + 2 only: slot (t + 1) mod R, written in phase 2, is never read
                const bool rd = j < N && f < p.KF && d >= 2 && t + d < T && bok;
                got[e][f] = rd ? p.ring[((size_t)sl * N + j) * B + b] : 0.0f;
            }
        }
    }
    barrier_lds();   // LDS only: the loads above stay in flight
    // phase 1: one near column per wave at a time, its 64 batch rows on the lanes (the
    // partials are column-major: 256 contiguous bytes per partial)
    {
        const int b = b0 + lane;
        const size_t qs = (size_t)p.Nnp * B;
        for (int cl = w; cl < nn; cl += 4) {
            float g = 0.0f;
            if (b < B) {
                const float* src = p.npart + (size_t)(lo + cl) * B + b;
                int q = 0;
                for (; q + 16 <= p.KSn; q += 16) {
                    float v[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] = src[(size_t)(q + e) * qs];
#pragma unroll
                    for (int e = 0; e < 16; ++e) g += v[e];
                }
                for (; q < p.KSn; ++q) g += src[(size_t)q * qs];
            }
            sg[cl][lane] = g;
            if (lane == 0) ncl[p.perm[lo + cl] - j0] = cl;
        }
    }
    barrier_lds();
    // phase 2
    {
        const int b = b0 + lane;
        const bool bok = b < B;
        const int s1 = tm + 1 == R ? 0 : tm + 1;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int cl = w + 4 * e;
            if (cl < nn && t + 1 < T && bok) p.ring[((size_t)s1 * N + p.perm[lo + cl]) * B + b] = sg[cl][lane];
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int jl = w + 4 * e, j = j0 + jl;
            float gf = 0.0f;
            if (j < N) {
                const int cl = ncl[jl];
                const float g1 = cl >= 0 && t + 1 < T ? sg[cl][lane] : 0.0f;   // near G(t + 1)
#pragma unroll
                for (int f = 0; f < KF; ++f) gf = fmaf(hv[e][f], lofv[e] + f == 1 ? g1 : got[e][f], gf);
            }
            sf[jl][lane] = gf;
        }
    }
    barrier_lds();
    // phase 3: column jl = lane % JT, rows LR w + lane / JT + 4 LR e (operands loaded on entry)
    {
        const Lif k = p.lif;
        const int jl = jl3, j = j3;
#pragma unroll
        for (int e = 0; e < E3; ++e) {
            const int r = r0 + 4 * LR * e, b = b0 + r;
            if (b >= B || j >= p.Nk) continue;
            const size_t ho = (size_t)b * p.lda + (size_t)t * p.Nk + j;
            if (j >= N) {
                p.hhi[ho] = 0;
                p.hlo[ho] = 0;
                continue;
            }
            const float gf = sf[jl][r];
            const size_t bj = (size_t)b * N + j, o = (size_t)t * BN + bj;
            const float y = lif_fire(k, uu[e]);
            const float du = lif_backward(k, gyv[e] + gf, uu[e], y, lam[e]);
            p.state[bj] = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * mv[e];
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            if (p.dbp) p.dbp[bj] = last ? gr : dbv[e] + gr;
            const uint32_t hi = hyb_bf16_rne(gr);
            p.hhi[ho] = (uint16_t)hi;
            p.hlo[ho] = (uint16_t)hyb_bf16_rne(gr - __uint_as_float(hi << 16));
        }
    }
}

// The far product of the block that starts at step t0 (rows (b, tt), tau = t0 + 1 + tt):
// G_j(tau) = sum_ks fpart[ks][b * P + tt][c] for far column c (source perm[Nn + c]) into
// ring slot tau mod R. Tile: 64 far columns x 64 batch rows of one tt, summed row-major and
// stored through an LDS transpose as 256-byte ring rows. Its consumers are steps
// tau - lof_j - f <= t0 (lof_j >= P), none of which has run.
__global__ void __launch_bounds__(256) hyb_bwd_far_kernel(HybBwd p) {
    __shared__ float sg[64][65];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c0 = blockIdx.x * 64, b0 = blockIdx.y * 64, tt = blockIdx.z;
    const int B = p.B, N = p.N, P = p.P;
    const int tau = p.t0 + 1 + tt;
    if (tau >= p.T) return;   // G past the last step is 0 and never read
    {
        const int c = c0 + lane;
        const bool cok = c < p.Nf;
        float g[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) g[e] = 0.0f;
        for (int q = 0; q < p.KSf; ++q) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int b = b0 + w + 4 * e;
                v[e] = (cok && b < B) ? p.fpart[((size_t)q * B * P + (size_t)b * P + tt) * p.Nfp + c] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 16; ++e) g[e] += v[e];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) sg[lane][w + 4 * e] = g[e];
    }
    __syncthreads();
    const int b = b0 + lane;
    const size_t slot = (size_t)(tau % p.R) * N;
#pragma unroll 4
    for (int e = 0; e < 16; ++e) {
        const int cl = w + 4 * e, c = c0 + cl;
        if (c < p.Nf && b < B) p.ring[(slot + p.perm[p.Nn + c]) * B + b] = sg[cl][lane];
    }
}

// ---------------------------------------------------------------------------------------
// Forward of the hybrid as an event-driven scatter on arrival, one batch row per workgroup
// (bf16 W, at most 2048 neurons: NPT = 1 or 2 per lane of a block of at most 1024 lanes,
// each lane's neurons being both receivers and sources).
//
// A spike of source j at step tau reaches receiver i through tap f at tau + lof_j + f + e_ij,
// so it "arrives" at step t = tau + lof_j and its contributions then land e_ij + f steps
// ahead: at step t the walked sources are those with y_j(t - lof_j) = 1 (bit lof_j - 1 of the
// source's own spike-history word), and the pending recurrent input of each receiver only
// needs a ring of D + KF - 1 slots (C5: 6; the per-connection scatter needs L, 67), rounded
// up to a power of two R (C5: 8) so that a slot wraps by a mask: R slots plus KF - 1 mirror
// slots after slot R - 1, so a connection's KF taps are the slots s .. s + KF - 1 from
// s = (t + e) mod R with no wrap; the mirror slot R + m is read and cleared with slot m.
// The ring is slot-major, ring[slot][receiver] with a pitch of NR = NPT * 1024 receivers, so
// the lanes of a wave always hit 64 distinct banks whatever slot each connection selects, and
// the taps of a run are immediate offsets of one address. (C5: 9 slots of 2048 receivers,
// 74 KB, so two rows' workgroups share a CU.) Per connection: the packed word
// bf16(W) << 16 | (offset - smallest offset) in the low half word (one 4-byte load), the
// slot, and KF read-modify-writes w * h_j(lof_j + f) of the run. Where the R slots are
// exactly 2^16 bytes (C3: 16 x 4 KB, C5: 8 x 8 KB) the low half holds the offset times the
// slot bytes, so a 16-bit add of (t mod R) * slot bytes wraps the slot by itself and one add
// places the receiver: two VALU instead of three (offset byte-add, mask, scale-add).
//
// Per step: every wave walks the arrival list of step t (flattened from per-wave segments,
// sources in a fixed order) over its own receivers, 64 arrivals at a time: lane a of the
// wave holds arrival a's source and tap weights, which reach the whole wave by readlane, so
// the only memory reads of the walk are the packed words, fetched a chunk of CH arrivals
// ahead into the other of two word buffers (CH = 32 with one neuron per lane, 4 with two),
// each load taking the source row's offset in its scalar offset. A receiver's ring column is
// only ever written by its own lane, so the scatter needs no barrier; then each lane runs the
// LIF of its receivers on their ring slot, shifts each
// source's spike into its history word and appends the sources arriving at t + 1 to its
// wave's segment of the other list buffer; one LDS barrier per step.
constexpr int kArriveWaves = 16;   // list segments per buffer (a 1024-lane block)

template <int NPT, int KF, int HW, int CH, bool WS>
__global__ void __launch_bounds__(1024, NPT) hyb_fwd_arrive_kernel(HybScat p) {
    extern __shared__ float smem[];
    constexpr int NR = NPT * 1024;
    constexpr int SH = NPT == 1 ? 12 : 13;   // log2 of a slot's bytes (WS: the offset field's shift)
    const int N = p.N, T = p.T, B = p.B, R = p.R, RP = p.RP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6;
    float* ring = smem;                                                             // [RP][NR]
    int* cnt = reinterpret_cast<int*>(ring + (size_t)RP * NR);                      // [2][16]
    uint16_t* seg = reinterpret_cast<uint16_t*>(cnt + 2 * kArriveWaves);            // [2][16][NPT * 64]
    const int TW = (T + 31) >> 5;
    const size_t BN = (size_t)B * N;
    const Lif k = p.lif;

    for (int q = tid; q < RP * NR; q += BS) ring[q] = 0.0f;
    if (tid < 2 * kArriveWaves) cnt[tid] = 0;    // nothing arrives at step 0; absent waves stay 0

    int idx[NPT], lof[NPT];
    bool act[NPT];
    float v[NPT], m[NPT], bias[NPT];
    uint64_t hist[NPT][HW];
    uint32_t word[NPT];
#pragma unroll
    for (int c = 0; c < NPT; ++c) {
        idx[c] = tid + c * BS;
        act[c] = idx[c] < N;
        const int i = act[c] ? idx[c] : 0;
        lof[c] = p.lof[i];
        v[c] = k.v0;
        m[c] = p.drop ? p.drop[(size_t)b * N + i] : 1.0f;
        bias[c] = p.bias ? p.bias[i] : 0.0f;
#pragma unroll
        for (int w = 0; w < HW; ++w) hist[c][w] = 0ull;
        word[c] = 0u;
    }
    // one descriptor for the packed connections; source o's words start o * N in, a lane
    // past N reads beyond the matrix (0: weight 0, no contribution)
    const i32x4 rw = buffer_rsrc(p.wpk, (uint32_t)((size_t)N * N * 4u));
    int wio[NPT];
#pragma unroll
    for (int c = 0; c < NPT; ++c) wio[c] = act[c] ? idx[c] * 4 : 0x40000000;
    __syncthreads();

    int tm = 0;   // t mod R
    for (int t = 0; t < T; ++t) {
        // this step's input, issued first so that the scatter hides its latency
        float xs[NPT];
#pragma unroll
        for (int c = 0; c < NPT; ++c) xs[c] = act[c] ? p.x[(size_t)t * BN + (size_t)b * N + idx[c]] : 0.0f;

        // ---- scatter of the sources arriving at t
        const int bsel = t & 1;
        int cw[kArriveWaves];
        {
            const int4* c4 = reinterpret_cast<const int4*>(cnt + bsel * kArriveWaves);
#pragma unroll
            for (int q = 0; q < kArriveWaves / 4; ++q) {
                const int4 v4 = c4[q];
                cw[4 * q] = v4.x; cw[4 * q + 1] = v4.y; cw[4 * q + 2] = v4.z; cw[4 * q + 3] = v4.w;
            }
        }
        int total = 0;
#pragma unroll
        for (int w2 = 0; w2 < kArriveWaves; ++w2) total += cw[w2];
        for (int base = 0; base < total; base += 64) {
            // lane a: arrival base + a -- its source and tap weights
            int src = 0;
            float hs[KF];
            {
                const int f = base + lane;
                int acc = 0, sgi = 0, pos = 0;
                bool found = false;
#pragma unroll
                for (int w2 = 0; w2 < kArriveWaves; ++w2) {
                    if (!found && f < acc + cw[w2]) {
                        sgi = w2;
                        pos = f - acc;
                        found = true;
                    }
                    acc += cw[w2];
                }
                src = found ? (int)seg[(bsel * kArriveWaves + sgi) * (NPT * 64) + pos] : 0;
#pragma unroll
                for (int q = 0; q < KF; ++q) hs[q] = found ? p.h[(size_t)q * N + src] : 0.0f;
            }
            const int nf = min(64, total - base);
            // the words of CH arrivals from f: the source row's offset rides in the scalar
            // offset of the load (uniform), the lane's column in the vector offset
            auto fetch = [&](uint32_t (&wb)[CH][NPT], int f) {
#pragma unroll
                for (int e = 0; e < CH; ++e) {
                    const int o = __builtin_amdgcn_readlane(src, (f + e) & 63);
#pragma unroll
                    for (int c = 0; c < NPT; ++c)
                        wb[e][c] = __float_as_uint(raw_buffer_load_f32(rw, wio[c], o * N * 4, 0));
                }
            };
            // two word buffers in turn: chunk f0's words in one while the next chunk's load
            // into the other
            uint32_t wa[CH][NPT], wz[CH][NPT];
            fetch(wa, 0);
            auto scatter = [&](const uint32_t (&wc)[CH][NPT], int f0) {
#pragma unroll
                for (int e = 0; e < CH; ++e) {
                    if (f0 + e >= nf) break;
                    float hf[KF];
#pragma unroll
                    for (int q = 0; q < KF; ++q)
                        hf[q] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hs[q]), (f0 + e) & 63));
                    // the NPT receivers of a lane lie in distinct ring columns: all their taps
                    // are read before any is written, one LDS round trip per arrival
                    float* run[NPT];
                    float wf[NPT], old[NPT][KF];
#pragma unroll
                    for (int c = 0; c < NPT; ++c) {
                        const uint32_t wv = wc[e][c];
                        // the offset byte holds offset - smallest offset, in [0, D) for the
                        // offsets the caller describes; R is a power of two, so the slot wraps
                        // by a mask (one byte-add and one AND), and a byte outside that range
                        // still lands in the ring. A lane past N reads the word 0: weight 0
                        // into its own column
                        wf[c] = __uint_as_float(wv & 0xFFFF0000u);
                        if constexpr (WS) {
                            // the field is the offset's slot bytes and R slots are 2^16 bytes:
                            // a 16-bit add wraps the slot, one add places the receiver
                            const uint32_t ab = (uint16_t)((uint16_t)wv + (uint16_t)(tm << SH));
                            run[c] = reinterpret_cast<float*>(reinterpret_cast<char*>(ring + idx[c]) + ab);
                        } else {
                            const int sl = (tm + (int)(wv & 0xFFu)) & (R - 1);
                            run[c] = ring + sl * NR + idx[c];
                        }
#pragma unroll
                        for (int q = 0; q < KF; ++q) old[c][q] = run[c][q * NR];
                    }
#pragma unroll
                    for (int c = 0; c < NPT; ++c)
#pragma unroll
                        for (int q = 0; q < KF; ++q) run[c][q * NR] = fmaf(wf[c], hf[q], old[c][q]);
                }
            };
            for (int f0 = 0; f0 < nf; f0 += 2 * CH) {
                if (f0 + CH < nf) fetch(wz, f0 + CH);
                scatter(wa, f0);
                if (f0 + CH >= nf) break;
                if (f0 + 2 * CH < nf) fetch(wa, f0 + 2 * CH);
                scatter(wz, f0 + CH);
            }
        }

        // ---- LIF of this lane's receivers, then each source's history and next arrival
        bool next[NPT];
#pragma unroll
        for (int c = 0; c < NPT; ++c) {
            float* col = ring + idx[c];
            float rec = col[tm * NR];
            col[tm * NR] = 0.0f;
            if (tm < KF - 1) {
                rec += col[(R + tm) * NR];
                col[(R + tm) * NR] = 0.0f;
            }
            const float r = rec + bias[c];
            const float a = xs[c] + r * m[c];
            const float u = lif_charge(k, v[c], a);
            const float yv = lif_fire(k, u);
            const bool fire = act[c] && yv != 0.0f;
            v[c] = lif_reset(k, u, yv);
            if (act[c]) {
                const size_t o = (size_t)t * BN + (size_t)b * N + idx[c];
                p.y[o] = fire ? 1.0f : 0.0f;
                p.u[o] = u;
            }
            word[c] |= (fire ? 1u : 0u) << (t & 31);
            if (((t & 31) == 31 || t == T - 1) && act[c]) {
                p.bits[((size_t)b * TW + (t >> 5)) * N + idx[c]] = word[c];
                word[c] = 0u;
            }
#pragma unroll
            for (int w = HW - 1; w > 0; --w) hist[c][w] = (hist[c][w] << 1) | (hist[c][w - 1] >> 63);
            hist[c][0] = (hist[c][0] << 1) | (fire ? 1ull : 0ull);
            // y(t + 1 - lof) is bit lof - 1 of the updated history
            const int kb = lof[c] - 1;
            const uint64_t hw = HW == 1 ? hist[c][0] : (kb < 64 ? hist[c][0] : hist[c][HW - 1]);
            next[c] = act[c] && ((hw >> (kb & 63)) & 1ull);
        }
        const int nsel = (t + 1) & 1;
        uint16_t* myseg = seg + (nsel * kArriveWaves + wave) * (NPT * 64);
        int filled = 0;
#pragma unroll
        for (int c = 0; c < NPT; ++c) {
            const uint64_t bal = __ballot(next[c]);
            if (next[c]) myseg[filled + __popcll(bal & ((1ull << lane) - 1ull))] = (uint16_t)idx[c];
            filled += __popcll(bal);
        }
        if (lane == 0) cnt[nsel * kArriveWaves + wave] = filled;
        tm = (tm + 1) & (R - 1);
        barrier_lds();
    }
}

// wpk[o * N + i] = bf16 bits of W[i, o] << 16 | uint8(offset[i, o] - smallest offset) << a.sh
// (launch_pack_hybrid with the smallest offset and a.sh: the slot bytes' log2 where R slots
// of them are 2^16 bytes, else 0)
bool launch_hyb_fwd_arrive(const HybScat& a, int npt, int hw, int block, size_t lds, hipStream_t stream) {
#define DELREC_ARRIVE_WS(NPTV, KFV, HWV, WSV)                                                     \
    if (npt == NPTV && a.KF <= KFV && hw == HWV && (a.sh > 0) == WSV) {                          \
        constexpr int CHV = NPTV == 1 ? 32 : 4;                                                   \
        ensure_lds((const void*)hyb_fwd_arrive_kernel<NPTV, KFV, HWV, CHV, WSV>, lds);           \
        hipLaunchKernelGGL((hyb_fwd_arrive_kernel<NPTV, KFV, HWV, CHV, WSV>), dim3(a.B), dim3(block), lds, stream, a); \
        return true;                                                                             \
    }
#define DELREC_ARRIVE(NPTV, KFV, HWV) DELREC_ARRIVE_WS(NPTV, KFV, HWV, true) DELREC_ARRIVE_WS(NPTV, KFV, HWV, false)
    DELREC_ARRIVE(1, 2, 1) DELREC_ARRIVE(1, 2, 2) DELREC_ARRIVE(2, 2, 1) DELREC_ARRIVE(2, 2, 2)
    DELREC_ARRIVE(1, 4, 1) DELREC_ARRIVE(1, 4, 2) DELREC_ARRIVE(2, 4, 1) DELREC_ARRIVE(2, 4, 2)
#undef DELREC_ARRIVE
#undef DELREC_ARRIVE_WS
    return false;
}

// ---------------------------------------------------------------------------------------

// steps per block of the backward's far product: C5 measured 90 ms per scan at 4, 94 at 8,
// 104 at 6, 114 at 16, 123 at 3 (128 x 256 far tiles); 80 at 4, 93 at 8, 104 at 5, 341 at 2
// with the 256 x 256 far tiles
constexpr int kHybBlock = 4;

HybStepDims hybstep_dims(int T, int B, int N, int L, int D, int KF, int cus) {
    HybStepDims q{};
    q.Nk = (N + 31) / 32 * 32;
    q.Np = (N + 127) / 128 * 128;
    q.D = D;
    q.KF = KF;
    q.R = std::max(L, 2);
    q.HW = (std::max(L - 1, 1) + 63) / 64;
    q.Kt = D * q.Nk;
    q.P = kHybBlock;
    q.lda = (size_t)(T + D + q.P + 1) * q.Nk;   // slices past the last step read as 0 (the far
                                                // product of the first block reaches T + P + D - 2)
    q.plane = (size_t)(q.Kt / 8) * q.Np;
    q.KS = lagstep_splits(B, q.Np, q.Kt, cus);
    // offsets of 16 or fewer, taps of 8 or fewer, a spike history of two 64-bit words, and
    // 32-bit byte offsets for every operand a GEMM addresses (incl. rows of a partial tile)
    q.ok = D >= 1 && D <= 16 && KF >= 1 && KF <= 8 && q.HW <= 2 &&
           (size_t)(B + 128) * q.lda * 2 < ((size_t)1 << 32) && q.plane * 16 < ((size_t)1 << 32);
    return q;
}

void launch_hyb_pack(const HybPack& a, bool fwd, hipStream_t stream) {
    const size_t total = (size_t)(a.Nk / 8) * a.Np;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (fwd)
        hipLaunchKernelGGL(hyb_pack_kernel<true>, dim3(blocks), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(hyb_pack_kernel<false>, dim3(blocks), dim3(256), 0, stream, a);
}

void launch_hyb_taps(const HybTaps& a, hipStream_t stream) {
    hipLaunchKernelGGL(hyb_taps_kernel, dim3((a.N + 255) / 256), dim3(256), 0, stream, a);
}

void launch_hyb_lif(const HybLif& l, int hw, hipStream_t stream) {
    const size_t n = (size_t)l.B * l.Nk;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (hw == 1)
        hipLaunchKernelGGL(hyb_lif_fwd_kernel<1>, dim3(blocks), dim3(256), 0, stream, l);
    else
        hipLaunchKernelGGL(hyb_lif_fwd_kernel<2>, dim3(blocks), dim3(256), 0, stream, l);
}

// the LIF tiles cover Nk neurons (the history planes' padding columns are written as 0)
void launch_hyb_bwd_lif(const HybBwd& a, hipStream_t stream) {
    const dim3 grid(a.Nk / kHybBwdTile, (a.B + 63) / 64);
    if (a.KF <= 2)
        hipLaunchKernelGGL(hyb_bwd_lif_kernel<2>, grid, dim3(256), 0, stream, a);
    else if (a.KF <= 4)
        hipLaunchKernelGGL(hyb_bwd_lif_kernel<4>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(hyb_bwd_lif_kernel<8>, grid, dim3(256), 0, stream, a);
}

int hyb_bwd_tile() { return kHybBwdTile; }

void launch_hyb_bwd_far(const HybBwd& a, hipStream_t stream) {
    if (a.Nf <= 0) return;
    const dim3 grid((a.Nf + 63) / 64, (a.B + 63) / 64, a.P);
    hipLaunchKernelGGL(hyb_bwd_far_kernel, grid, dim3(256), 0, stream, a);
}

int hyb_bwd_far_cols(int planes) { return planes == 1 ? 256 : 128; }

HybBwdSizes hyb_bwd_sizes(const HybStepDims& q, int B, int cus, int fcol) {
    HybBwdSizes z{};
    // any padded column count of either part: near columns in multiples of 128 up to Np, far
    // ones in multiples of fcol up to Np rounded up to fcol; the two parts' padded counts add
    // up to at most N + 127 + fcol - 1 < Np + 384
    for (int c = 128; c <= q.Np; c += 128)
        z.npart = std::max(z.npart, (size_t)lagstep_splits(B, c, q.Kt, cus) * B * c);
    // (256-column far parts may run either far kernel: the larger split count sizes them)
    for (int c = fcol; c <= (q.Np + fcol - 1) / fcol * fcol; c += fcol) {
        int ks = lagstep_splits(B * q.P, c, q.Kt, cus, fcol);
        if (fcol == 256) ks = std::max(ks, lagstep_gemm256_splits(B * q.P, c, q.Kt, cus));
        z.fpart = std::max(z.fpart, (size_t)ks * B * q.P * c);
    }
    z.planes = (size_t)(q.Kt / 8) * (q.Np + 384);
    return z;
}

}  // namespace delrec
