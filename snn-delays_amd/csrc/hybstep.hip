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

// The backward runs in blocks of P steps t0 - P + 1 .. t0, latest block first, as four launches
// per block (no launch per step):
//  1 the far product (lagstep.hip): G_j(tau) of the far sources (lof_j >= P) for the P steps
//    tau = t0 + 1 .. t0 + P, rows (b, tau); its history slices (> t0) are complete;
//  2 hyb_bwd_farblk_kernel: those G into the ring and the whole block's LIF backward of the
//    far sources: gfut_j(t) = sum_f h_j(f) G_j(t + lof_j + f) reads only tau >= t + P > t0;
//    it writes the far sources' gr(t) into the history for the block's slices, and 0 for the
//    near sources' columns there;
//  3 the near product (lagstep.hip): G_j(t + 1) of the near sources for the block's steps t,
//    rows (b, t + 1), which reads the block's slices with the near columns still 0;
//  4 hyb_bwd_near_kernel: per batch row, the near sources' chain through the block, latest
//    step first, adding the part the product could not see -- sum_i W_ij gr_i(t + 1 + e_ij)
//    over near receivers i whose step t + 1 + e_ij lies in the block -- from an LDS window of
//    the near gr it produces.
// Batch rows are independent, so step 4 needs no synchronisation beyond its workgroup, and
// the only sequential chain left inside a block is the near sources' (C5: 5 % of them).

namespace {

__device__ __forceinline__ float hyb_sel4(const float (&g)[kHybBlockMax], int i) {
    float v = g[0];
#pragma unroll
    for (int q = 1; q < kHybBlockMax; ++q) v = i == q ? g[q] : v;
    return v;
}

}  // namespace

// Step 2: a tile of 64 neurons x 16 batch rows per workgroup, in three phases:
//  1 (64 neurons on the lanes, 4 rows per wave: coalesced over j) the far sources' G(tau),
//    tau = t0 + 1 .. t0 + P, summed over the product's splits (split groups of 4 loads in
//    flight) into LDS; the LIF operands u, gy into registers; 0 into the history at the
//    block's slices for the near and padding columns;
//  2 (16 rows on the lanes, 4 neurons each: the ring [slot][j][b] has b fastest) those G into
//    the ring, and each source's window of the P + KF - 1 values G_j(tau), tau = t0 - P + 1 +
//    lof_j + w, that the block's taps read -- from LDS for tau <= t0 + P, else from the ring
//    (written by earlier launches), 0 past the last step -- into LDS;
//  3 (neurons on the lanes again) the LIF backward of the block's steps, latest first, with
//    gfut_j(t) = sum_f h_j(f) window[t - (t0 - P + 1) + f].
constexpr int kSplitGroup = 4;
constexpr int kFarRows = 16;

template <int KF>
__global__ void __launch_bounds__(256) hyb_bwd_farblk_kernel(HybBwd p) {
    constexpr int W = kHybBlockMax + KF - 1;
    __shared__ float sG[kHybBlockMax][kFarRows][65];
    __shared__ float sW[W][kFarRows][65];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j0 = blockIdx.x * 64, b0 = blockIdx.y * kFarRows;
    const int t0 = p.t0, P = p.P, T = p.T, N = p.N, B = p.B, R = p.R;
    const int tb = max(t0 - P + 1, 0);
    const int ns = t0 - tb + 1;                       // steps in this block
    const int tbase = t0 - P + 1;
    const size_t BN = (size_t)B * N;
    const Lif k = p.lif;
    const bool first = t0 == T - 1;
    // the ring values phase 2 reads (its own lane mapping: row b0 + lane % 16, neurons
    // 16 w + 4 (lane / 16) + q), issued first so that they arrive during phase 1
    const int r2 = lane & (kFarRows - 1), b2 = b0 + r2;
    int lof2[4];
    float v2[4][W];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int jj = j0 + 16 * w + 4 * (lane >> 4) + q;
        const int l = jj < N ? p.lof[jj] : 0;
        lof2[q] = (jj < N && l >= P && b2 < B) ? l : -1;
#pragma unroll
        for (int x = 0; x < W; ++x) {
            const int tau = tbase + l + x;
            const bool rd = lof2[q] >= 0 && x < P + p.KF - 1 && tau < T && tau > t0 + P;
            v2[q][x] = rd ? p.ring[((size_t)(tau % R) * N + jj) * B + b2] : 0.0f;
        }
    }
    // phase 1: lane = neuron j0 + lane, rows b0 + 4 w + rr
    const int j = j0 + lane;
    const bool inj = j < p.Nk;
    const int lof = j < N ? p.lof[j] : 0;
    const bool far = j < N && lof >= P;
    const int c = far ? p.colf[j] : 0;
    constexpr int RW = kFarRows / 4;                  // rows per wave
    float uu[RW][kHybBlockMax], gyv[RW][kHybBlockMax];
    {
        const size_t kstride = (size_t)B * P * p.Nfp;
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {
            const int r = 4 * w + rr, b = b0 + r;
            const bool ok = far && b < B;
            float g[kHybBlockMax];
#pragma unroll
            for (int tt = 0; tt < kHybBlockMax; ++tt) g[tt] = 0.0f;
            const float* fp = p.fpart + (size_t)(ok ? b : 0) * P * p.Nfp + c;
            for (int k0 = 0; k0 < p.KSf; k0 += kSplitGroup) {
                float v[kSplitGroup][kHybBlockMax];
#pragma unroll
                for (int q = 0; q < kSplitGroup; ++q)
#pragma unroll
                    for (int tt = 0; tt < kHybBlockMax; ++tt)
                        v[q][tt] = (ok && k0 + q < p.KSf && tt < P && t0 + 1 + tt < T)
                                       ? fp[(size_t)(k0 + q) * kstride + (size_t)tt * p.Nfp] : 0.0f;
#pragma unroll
                for (int q = 0; q < kSplitGroup; ++q)
#pragma unroll
                    for (int tt = 0; tt < kHybBlockMax; ++tt) g[tt] += v[q][tt];
            }
#pragma unroll
            for (int tt = 0; tt < kHybBlockMax; ++tt) {
                sG[tt][r][lane] = g[tt];
                const int t = t0 - tt;
                const bool live = ok && tt < ns;
                const size_t o = (size_t)(live ? t : 0) * BN + (size_t)(ok ? b : 0) * N + (far ? j : 0);
                uu[rr][tt] = live ? p.u_in[o] : 0.0f;
                gyv[rr][tt] = live ? p.gy[o] : 0.0f;
            }
            if (inj && !far && b < B) {
                const size_t hrow = (size_t)b * p.lda + (size_t)p.PF * p.Nk + j;
                for (int q = 0; q < ns; ++q) {
                    p.hhi[hrow + (size_t)(t0 - q) * p.Nk] = 0;
                    p.hlo[hrow + (size_t)(t0 - q) * p.Nk] = 0;
                }
            }
        }
    }
    barrier_lds();   // (LDS only: no global value written here is read back in this launch)
    // phase 2: lane = row b0 + lane % 16; neurons 16 w + 4 (lane / 16) + q
    {
        const int r = r2, b = b2;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int jl = 16 * w + 4 * (lane >> 4) + q, jj = j0 + jl;
            const int lj = lof2[q];
            if (lj < 0) continue;
#pragma unroll
            for (int tt = 0; tt < kHybBlockMax; ++tt)
                if (tt < P && t0 + 1 + tt < T)
                    p.ring[((size_t)((t0 + 1 + tt) % R) * N + jj) * B + b] = sG[tt][r][jl];
#pragma unroll
            for (int x = 0; x < W; ++x) {
                const int tau = tbase + lj + x;
                sW[x][r][jl] = (tau <= t0 + P && tau < T) ? sG[max(tau - t0 - 1, 0)][r][jl] : v2[q][x];
            }
        }
    }
    barrier_lds();
    // phase 3: lane = neuron j0 + lane, rows 4 w + rr
    if (!far) return;
    float hv[KF];
#pragma unroll
    for (int f = 0; f < KF; ++f) hv[f] = f < p.KF ? p.h[(size_t)f * N + j] : 0.0f;
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const int r = 4 * w + rr, b = b0 + r;
        if (b >= B) break;
        const size_t bj = (size_t)b * N + j;
        const size_t hrow = (size_t)b * p.lda + (size_t)p.PF * p.Nk + j;
        float lam = first ? 0.0f : p.state[bj];
        float db = (p.dbp && !first) ? p.dbp[bj] : 0.0f;
        const float m = p.drop ? p.drop[bj] : 1.0f;
#pragma unroll
        for (int tt = 0; tt < kHybBlockMax; ++tt) {
            if (tt >= ns) break;
            const int t = t0 - tt, row = t - tbase;
            float gf = 0.0f;
#pragma unroll
            for (int f = 0; f < KF; ++f) gf = fmaf(hv[f], sW[row + f][r][lane], gf);
            const float y = lif_fire(k, uu[rr][tt]);
            const float du = lif_backward(k, gyv[rr][tt] + gf, uu[rr][tt], y, lam);
            lam = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * m;
            const size_t o = (size_t)t * BN + bj;
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            db += gr;
            const uint32_t hi = hyb_bf16_rne(gr);
            p.hhi[hrow + (size_t)t * p.Nk] = (uint16_t)hi;
            p.hlo[hrow + (size_t)t * p.Nk] = (uint16_t)hyb_bf16_rne(gr - __uint_as_float(hi << 16));
        }
        p.state[bj] = lam;
        if (p.dbp) p.dbp[bj] = db;
    }
}

// Step 4: RB = 2 batch rows per workgroup (one workgroup per CU at B = 512), 1024 threads (four
// waves per SIMD to hide the LDS and VALU latencies of a short chain). An item is one near
// source (compact index c, source perm[c]) and batch row: thread q owns item q for the LIF.
// On entry, from global memory, all of it independent of the chain: each item's u, gy, older
// ring values and state into registers, the block's near product summed over its splits and
// the packed near-to-near weights wnp[ci][c] into LDS. Per step t, latest first:
//  a G_j(t + 1) = that product row + sum over near receivers ci of w * gr_ci(t + 1 + e) from
//    the LDS window of the block's near gr (slot s = step t0 - P + 1 + s; slots >= P, steps
//    past the block, stay 0: the product already holds those) -- four threads per item, each
//    a quarter of the receivers, summed across the four lanes; into the ring and an LDS copy
//    of the block's G (tau <= t0 + 1);
//  b the LIF backward of the items: gfut from that copy (tau <= t0 + 1) or the ring (written
//    by earlier launches), gr into the history and the window.
constexpr int kNearRows = 2;
constexpr int kNearThreads = 1024;
static_assert(kHybNearMax * kNearRows <= kNearThreads / 2, "at least two threads per item");

namespace {

// the window holds each near receiver's slots contiguously, at an odd pitch: the lanes of a
// wave (sources c, same receiver ci) read slots row + 1 + e of one run -- distinct words in
// distinct banks, or one broadcast word
__host__ __device__ inline int near_ldw(int nslot) { return nslot | 1; }

}  // namespace

template <int KF>
__global__ void __launch_bounds__(kNearThreads) hyb_bwd_near_kernel(HybBwd p) {
    constexpr int RB = kNearRows, NT = kNearThreads;
    extern __shared__ float sm[];
    const int Nn = p.Nn, P = p.P, D = p.D, T = p.T, N = p.N, B = p.B, R = p.R, t0 = p.t0;
    const int nslot = P + D;
    const int ldw = near_ldw(nslot);                  // per-receiver pitch of the window
    const int Nq = (Nn + 15) & ~15;                   // receivers padded: sp parts of groups of 4
    uint32_t* wl = reinterpret_cast<uint32_t*>(sm);   // [Nq][Nn] packed weights (rows >= Nn: 0)
    float* grw = sm + (size_t)Nq * Nn;                // [RB][Nq][ldw]: gr of near receiver ci at slot s
    float* gnp = grw + (size_t)RB * Nq * ldw;         // [P][RB][Nn]: the near product, summed
    float* gq = gnp + (size_t)P * RB * Nn;            // [P][RB][Nn]: G(tau), slot tau - (t0 - P + 2)
    const int tid = threadIdx.x;
    const int b0 = blockIdx.x * RB;
    const int tb = max(t0 - P + 1, 0);
    const int ns = t0 - tb + 1;
    const int tbase = t0 - P + 1;                     // step of window slot 0
    const size_t BN = (size_t)B * N;
    const Lif k = p.lif;
    const bool first = t0 == T - 1;
    // start-up loads: the item's source, then its u, gy, older ring values and state; the
    // block product's partials (16 splits per round) and the packed weights
    const int ci_ = tid % Nn, ri_ = tid / Nn, bi_ = b0 + ri_;
    const bool own = tid < Nn * RB && bi_ < B;
    const int j = own ? p.perm[ci_] : 0;
    const int lofj = own ? p.lof[j] : 0;
    const size_t bj = (size_t)(own ? bi_ : 0) * N + j;
    float hv[KF], uu[kHybBlockMax], gyv[kHybBlockMax], rg[kHybBlockMax][KF];
#pragma unroll
    for (int f = 0; f < KF; ++f) hv[f] = (own && f < p.KF) ? p.h[(size_t)f * N + j] : 0.0f;
#pragma unroll
    for (int tt = 0; tt < kHybBlockMax; ++tt) {
        const int t = t0 - tt;
        const bool live = own && tt < ns;
        const size_t o = (size_t)(live ? t : 0) * BN + bj;
        uu[tt] = live ? p.u_in[o] : 0.0f;
        gyv[tt] = live ? p.gy[o] : 0.0f;
#pragma unroll
        for (int f = 0; f < KF; ++f) {
            const int tau = t + lofj + f;
            const bool rd = live && f < p.KF && tau < T && tau > t0 + 1;
            rg[tt][f] = rd ? p.ring[((size_t)(tau % R) * N + j) * B + bi_] : 0.0f;
        }
    }
    float lam = (own && !first) ? p.state[bj] : 0.0f;
    float db = (own && !first && p.dbp) ? p.dbp[bj] : 0.0f;
    const float mv = (own && p.drop) ? p.drop[bj] : 1.0f;
    {
        constexpr int GI = (kHybBlockMax * RB * kHybNearMax + NT - 1) / NT;   // product items per thread
        const size_t ks_stride = (size_t)B * P * p.Nnp;
        const int ng = P * RB * Nn;
        float gs[GI];
#pragma unroll
        for (int e = 0; e < GI; ++e) gs[e] = 0.0f;
        for (int k0 = 0; k0 < p.KSn; k0 += 8) {
            float v[GI][8];
#pragma unroll
            for (int e = 0; e < GI; ++e) {
                const int q = tid + NT * e, c = q % Nn, rr = q / Nn, r = rr % RB, row = rr / RB, b = b0 + r;
                const bool ok = q < ng && b < B;
                const float* src = p.npart + ((size_t)(ok ? b : 0) * P + (ok ? row : 0)) * p.Nnp + (ok ? c : 0);
#pragma unroll
                for (int x = 0; x < 8; ++x) v[e][x] = (ok && k0 + x < p.KSn) ? src[(size_t)(k0 + x) * ks_stride] : 0.0f;
            }
#pragma unroll
            for (int e = 0; e < GI; ++e)
#pragma unroll
                for (int x = 0; x < 8; ++x) gs[e] += v[e][x];
        }
#pragma unroll
        for (int e = 0; e < GI; ++e) {
            const int q = tid + NT * e;
            if (q < ng) gnp[q] = gs[e];
        }
    }
    {
        constexpr int WH = (kHybNearMax * kHybNearMax + 2 * NT - 1) / (2 * NT);   // weights per thread and round
        const int nw = Nn * Nn;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            uint32_t v[WH];
#pragma unroll
            for (int e = 0; e < WH; ++e) {
                const int q = (h2 * WH + e) * NT + tid;
                v[e] = q < nw ? p.wnp[q] : 0u;
            }
#pragma unroll
            for (int e = 0; e < WH; ++e) {
                const int q = (h2 * WH + e) * NT + tid;
                if (q < nw) wl[q] = v[e];
            }
        }
        for (int q = nw + tid; q < Nq * Nn; q += NT) wl[q] = 0u;
    }
    for (int q = tid; q < RB * Nq * ldw; q += NT) grw[q] = 0.0f;
    barrier_lds();
    // phase a mapping: sp = 4 (or 2 past 256 items) threads per item, item ia = tid / sp, part
    // pa = tid % sp (receivers ci = sp m + pa)
    const int sp = Nn * RB <= NT / 4 ? 4 : 2;
    const int ia = tid / sp, pa = tid % sp;
    const bool aown = ia < Nn * RB && b0 + ia / Nn < B;
    const int ca = aown ? ia % Nn : 0, ra = aown ? ia / Nn : 0, ba = b0 + ra;   // idle threads: item 0's
    const int ja = aown ? p.perm[ca] : 0;                                     // (in-bounds) reads
#pragma unroll
    for (int tt = 0; tt < kHybBlockMax; ++tt) {
        if (tt >= ns) break;                          // (static indices into the item arrays)
        const int t = t0 - tt;
        const int row = t - tbase;                    // the product's row of tau = t + 1
        // a: G(t + 1). A valid offset e < D always lands in the window: row + 1 + e < P + D
        {
            float acc = 0.0f;
            const uint32_t* wc = wl + (size_t)pa * Nn + (aown ? ca : 0);
            const float* gw = grw + ((size_t)ra * Nq + pa) * ldw + row + 1;
            const int nm = Nq / sp;                   // a multiple of 4
            for (int m0 = 0; m0 < nm; m0 += 4) {
                uint32_t pw[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) pw[x] = wc[(size_t)(sp * (m0 + x)) * Nn];
                float gv[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) gv[x] = gw[(size_t)(sp * (m0 + x)) * ldw + (int)(pw[x] & 0xFu)];
#pragma unroll
                for (int x = 0; x < 4; ++x) acc = fmaf(__uint_as_float(pw[x] & ~0xFu), gv[x], acc);
            }
            acc += __shfl_xor(acc, 1);
            if (sp == 4) acc += __shfl_xor(acc, 2);
            if (aown && pa == 0) {
                const float sum = acc + gnp[((size_t)row * RB + ra) * Nn + ca];
                gq[((size_t)row * RB + ra) * Nn + ca] = sum;
                if (t + 1 < T) p.ring[((size_t)((t + 1) % R) * N + ja) * B + ba] = sum;
            }
        }
        barrier_lds();
        // b: the LIF backward of the thread's item
        if (own) {
            float gf = 0.0f;
#pragma unroll
            for (int f = 0; f < KF; ++f) {
                const int tau = t + lofj + f;
                float gv = rg[tt][f];
                if (tau <= t0 + 1) gv = tau < T ? gq[((size_t)(tau - tbase - 1) * RB + ri_) * Nn + ci_] : 0.0f;
                gf = fmaf(hv[f], gv, gf);
            }
            const float y = lif_fire(k, uu[tt]);
            const float du = lif_backward(k, gyv[tt] + gf, uu[tt], y, lam);
            lam = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * mv;
            const size_t o = (size_t)t * BN + bj;
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            db += gr;
            const size_t ho = (size_t)bi_ * p.lda + (size_t)(p.PF + t) * p.Nk + j;
            const uint32_t hi = hyb_bf16_rne(gr);
            p.hhi[ho] = (uint16_t)hi;
            p.hlo[ho] = (uint16_t)hyb_bf16_rne(gr - __uint_as_float(hi << 16));
            grw[((size_t)ri_ * Nq + ci_) * ldw + row] = gr;
        }
        barrier_lds();
    }
    if (own) {
        p.state[bj] = lam;
        if (p.dbp) p.dbp[bj] = db;
    }
}

// wnp[ci][c]: the weight of the near connection receiver perm[ci] <- source perm[c], its low 4
// bits replaced by the offset - omin (< 16): bf16 W exact, fp32 W to 2^-19 relative (finer than
// the products' two bf16 planes); one thread per pair
__global__ void __launch_bounds__(256) hyb_near_pack_kernel(HybPack p, uint32_t* __restrict__ wnp) {
    const int Nn = p.nc;
    const size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (size_t)Nn * Nn) return;
    const int ci = (int)(q / Nn), c = (int)(q - (size_t)ci * Nn);
    const size_t o = (size_t)p.perm[ci] * p.N + p.perm[c];
    const int e = (int)p.off[o] - p.omin;
    // an offset outside the caller's range [omin, omin + D): a NaN weight at offset 0
    const bool bad = e < 0 || e >= p.D;
    const float w = bad ? __builtin_nanf("") : load_w(p.W, p.w_bf16, o);
    wnp[q] = (__float_as_uint(w) & ~0xFu) | (uint32_t)(bad ? 0 : e);
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
// the taps of a run are immediate offsets of one address. (C5: 9 slots of 2048 receivers and
// the lists, 82 KB, so one row's workgroup per CU: a ring without the mirror slot, 74 KB at
// 64 VGPRs, ran two per CU at the same speed -- the LDS traffic sets the pace, not the
// occupancy.) Per connection: the packed word
// bf16(W) << 16 | (offset - smallest offset) in the low half word (one 4-byte load), the
// slot, and KF read-modify-writes w * h_j(lof_j + f) of the run. Where the R slots are
// exactly 2^16 bytes (C3: 16 x 4 KB, C5: 8 x 8 KB) the low half holds the offset times the
// slot bytes plus the receiver's column bytes, so a 16-bit add of (t mod R) * slot bytes
// wraps the slot by itself and is the run's LDS address: one VALU instead of three (offset
// byte-add, mask, scale-add) -- ten VALU per arrival and wave at two receivers per lane.
// The packed rows have one word per lane column (NPT * block), so every lane reads a word of
// its own column, weight 0 past N.
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
typedef __attribute__((address_space(3))) char lds_char;

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

    if constexpr (WS) {
        // the packed offset fields are absolute LDS byte addresses: the ring must start at LDS
        // address 0 (no static LDS in this kernel, so the dynamic array does); otherwise every
        // output of the row is NaN
        if ((uint32_t)(size_t)(lds_char*)ring != 0u) {
            for (size_t q = tid; q < (size_t)T * N; q += BS) {
                const size_t t = q / N, i = q - t * N;
                p.u[t * BN + (size_t)b * N + i] = __builtin_nanf("");
                p.y[t * BN + (size_t)b * N + i] = __builtin_nanf("");
            }
            return;
        }
    }
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
    // one descriptor for the packed connections; source o's words start o * NPT * BS in, one
    // per lane column (the columns past N hold weight 0 in their own ring column)
    const int pitch = NPT * BS;
    const i32x4 rw = buffer_rsrc(p.wpk, (uint32_t)((size_t)N * pitch * 4u));
    int wio[NPT];
#pragma unroll
    for (int c = 0; c < NPT; ++c) wio[c] = idx[c] * 4;
    __syncthreads();

    int tm = 0;   // t mod R
    for (int t = 0; t < T; ++t) {
        // this step's input, issued first so that the scatter hides its latency
        float xs[NPT];
#pragma unroll
        for (int c = 0; c < NPT; ++c) xs[c] = act[c] ? p.x[(size_t)t * BN + (size_t)b * N + idx[c]] : 0.0f;

        // ---- scatter of the sources arriving at t
        const int bsel = t & 1;
        const uint32_t tmsh = (uint32_t)tm << SH;   // this step's slot bytes (WS)
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
                        wb[e][c] = __float_as_uint(raw_buffer_load_f32(rw, wio[c], o * pitch * 4, 0));
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
                        // still lands in the ring. A column past N holds weight 0 (its own
                        // ring column)
                        wf[c] = __uint_as_float(wv & 0xFFFF0000u);
                        if constexpr (WS) {
                            // the field is the offset's slot bytes plus the receiver's column
                            // bytes and R slots are 2^16 bytes: one 16-bit add of the step's
                            // slot bytes wraps the slot and is the byte address in the ring
                            // (one SDWA add whose 16-bit result is zero-extended: the
                            // compiler's form is an add and a mask)
                            uint32_t ab;
                            asm("v_add_u32_sdwa %0, %1, %2 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD"
                                : "=v"(ab) : "v"(wv), "v"(tmsh));
                            run[c] = (float*)(lds_char*)(size_t)ab;
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

// wpk[o * npt * block + i] = bf16 bits of W[i, o] << 16 | the offset field (launch_pack_hybrid
// with the smallest offset, a.sh: the slot bytes' log2 where R slots of them are 2^16 bytes,
// else 0, and the pitch npt * block)
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

HybStepDims hybstep_dims(int T, int B, int N, int L, int D, int KF, int cus) {
    HybStepDims q{};
    q.Nk = (N + 31) / 32 * 32;
    q.Np = (N + 127) / 128 * 128;
    q.D = D;
    q.KF = KF;
    q.R = std::max(L, 2);
    q.HW = (std::max(L - 1, 1) + 63) / 64;
    q.Kt = D * q.Nk;
    q.P = kHybBlockMax;
    q.PF = kHybBlockMax;   // zero slices before slice 0: the near product of a last block that
                           // starts before step 0 reads from slice t0 - P + 2 >= 2 - P
    q.lda = (size_t)(q.PF + T + D + q.P + 1) * q.Nk;   // slices past the last step read as 0 (the
                                                       // far product of the first block reaches
                                                       // T + P + D - 2)
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

void launch_hyb_bwd_farblk(const HybBwd& a, hipStream_t stream) {
    const dim3 grid((a.Nk + 63) / 64, (a.B + kFarRows - 1) / kFarRows);
    if (a.KF <= 2)
        hipLaunchKernelGGL(hyb_bwd_farblk_kernel<2>, grid, dim3(256), 0, stream, a);
    else if (a.KF <= 4)
        hipLaunchKernelGGL(hyb_bwd_farblk_kernel<4>, grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(hyb_bwd_farblk_kernel<8>, grid, dim3(256), 0, stream, a);
}

size_t hyb_bwd_near_lds(int P, int D, int Nn) {
    const size_t Nq = (size_t)(Nn + 15) & ~(size_t)15;
    return (Nq * Nn + (size_t)kNearRows * Nq * near_ldw(P + D) + (size_t)2 * P * kNearRows * Nn) * sizeof(float);
}

bool launch_hyb_bwd_near(const HybBwd& a, hipStream_t stream) {
    if (a.Nn <= 0) return true;
    if (a.Nn > kHybNearMax || a.P > kHybBlockMax || a.D > 16) return false;
    const size_t lds = hyb_bwd_near_lds(a.P, a.D, a.Nn);   // the caller checked it fits
    const dim3 grid((a.B + kNearRows - 1) / kNearRows);
#define DELREC_NEAR(KFV)                                                                         \
    ensure_lds((const void*)hyb_bwd_near_kernel<KFV>, lds);                                      \
    hipLaunchKernelGGL(hyb_bwd_near_kernel<KFV>, grid, dim3(kNearThreads), lds, stream, a);
    if (a.KF <= 2) { DELREC_NEAR(2) } else if (a.KF <= 4) { DELREC_NEAR(4) } else { DELREC_NEAR(8) }
#undef DELREC_NEAR
    return true;
}

// The backward's split of the sources by first lag, on the device: perm = the near sources
// (lof < P) in index order, then the far ones; colf[j] = j's far column (-1 for near ones).
// One workgroup of 1024 threads walks the sources in chunks twice (the near count, then the
// positions), so every store lands in [0, N) whatever the counts. The host chose the kernels'
// shapes from its own near count Nn: where the two disagree (the first lags changed between
// that count and this launch) the taps are overwritten with NaN, so that every output the
// backward writes is NaN rather than silently wrong.
__global__ void __launch_bounds__(1024) hyb_split_kernel(const int* __restrict__ lof, int N, int P, int Nn,
                                                         int* __restrict__ perm, int* __restrict__ colf,
                                                         float* __restrict__ h, int KF) {
    __shared__ int wsum[16];
    __shared__ int total;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    auto block_scan = [&](bool flag, int& before, int& all) {   // exclusive rank, chunk total
        const uint64_t bal = __ballot(flag);
        const int rank = __popcll(bal & ((1ull << lane) - 1ull));
        __syncthreads();
        if (lane == 0) wsum[w] = __popcll(bal);
        __syncthreads();
        int pre = 0, sum = 0;
        for (int q = 0; q < 16; ++q) {
            pre += q < w ? wsum[q] : 0;
            sum += wsum[q];
        }
        before = pre + rank;
        all = sum;
    };
    int nn = 0;
    for (int j0 = 0; j0 < N; j0 += 1024) {
        const int j = j0 + tid;
        int before, all;
        block_scan(j < N && lof[j] < P, before, all);
        nn += all;
    }
    int near = 0;
    for (int j0 = 0; j0 < N; j0 += 1024) {
        const int j = j0 + tid;
        const bool flag = j < N && lof[j] < P;
        int before, all;
        block_scan(flag, before, all);
        if (j < N) {
            const int pn = near + before;           // near sources before j
            if (flag) {
                perm[pn] = j;
                colf[j] = -1;
            } else {
                perm[nn + (j - pn)] = j;
                colf[j] = j - pn;
            }
        }
        near += all;
    }
    if (tid == 0) total = nn;
    __syncthreads();
    if (total != Nn)
        for (size_t q = tid; q < (size_t)KF * N; q += 1024) h[q] = __builtin_nanf("");
}

void launch_hyb_split(const int* lof, int N, int P, int Nn, int* perm, int* colf, float* h, int KF,
                      hipStream_t stream) {
    hipLaunchKernelGGL(hyb_split_kernel, dim3(1), dim3(1024), 0, stream, lof, N, P, Nn, perm, colf, h, KF);
}

void launch_hyb_near_pack(const HybPack& a, uint32_t* wnp, hipStream_t stream) {
    const size_t n = (size_t)a.nc * a.nc;
    if (n == 0) return;
    hipLaunchKernelGGL(hyb_near_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, wnp);
}

int hyb_bwd_far_cols(int planes) { return planes == 1 ? 256 : 128; }

HybBwdSizes hyb_bwd_sizes(const HybStepDims& q, int B, int cus, int fcol) {
    HybBwdSizes z{};
    // any block length P <= kHybBlockMax (rows B * P) and any padded column count of either
    // part: near columns in multiples of 128 up to kHybNearMax, far ones in multiples of fcol
    // up to Np rounded up to fcol; the two parts' padded counts add up to at most
    // N + 127 + fcol - 1 < Np + 384
    for (int P = 1; P <= kHybBlockMax; P *= 2) {
        for (int c = 128; c <= std::min(q.Np, kHybNearMax); c += 128)
            z.npart = std::max(z.npart, (size_t)lagstep_splits(B * P, c, q.Kt, cus) * B * P * c);
        // (the near product on the sparse MFMA: one 256-column tile; the near-block product:
        // 128-column tiles; both for blocks of 4 steps)
        if (P == 4) {
            z.npart = std::max(z.npart, (size_t)far_sparse_splits(B * P, 256, q.Nk, cus) * B * P * 256);
            for (int c = 128; c <= std::min(q.Np, kHybNearMax); c += 128)
                z.npart = std::max(z.npart, (size_t)near_block_splits(B * P, c, q.Nk, cus) * B * P * c);
        }
        // (256-column far parts may run either far kernel: the larger split count sizes them)
        for (int c = fcol; c <= (q.Np + fcol - 1) / fcol * fcol; c += fcol) {
            int ks = lagstep_splits(B * P, c, q.Kt, cus, fcol);
            if (fcol == 256) ks = std::max(ks, lagstep_gemm256_splits(B * P, c, q.Kt, cus));
            z.fpart = std::max(z.fpart, (size_t)ks * B * P * c);
        }
    }
    z.planes = (size_t)(q.Kt / 8) * (q.Np + 384);
    return z;
}

}  // namespace delrec
