// Axonal delayed-LIF recurrent scan for gfx950: forward and reverse-time BPTT.
//
// One workgroup owns one batch row for the whole sequence (batch rows are independent
// through the recurrence), so no step ever waits on another CU. Receiver i is served by
// G consecutive lanes, each holding a chunk of CH weights of W's row i in VGPRs (the
// "resident" form, N <= 256 in fp32) or streaming the chunk from L2 (N > 256). Each
// neuron keeps its own spike history as a register bitmask (bit l-1 = spike l steps ago),
// so the delayed trace z_j = sum_l h(l; d_j) y[t-l, j] needs no memory traffic; z is
// broadcast to the GEMV through a double-buffered LDS vector: one barrier per step.
//
// Reference behaviour replaced: recdel_fwd_kernel / recdel_bwd_kernel
// (src/delrec/triton_kernels/recdel_base.py:34-129, :189-285), with the dmask loop and
// autograd through build_mask (:327-342, :421-435) folded into per-neuron accumulators.
#include <utility>

#include "common.h"
#include "kernels.h"
#include "dw_gemm.h"

namespace delrec {

// ---------------------------------------------------------------------------------------
// Spike history helpers: HW 64-bit words, bit (l-1) of the concatenation = y[t-l].
template <int HW>
struct History {
    uint64_t w[HW];
    __device__ void clear() {
#pragma unroll
        for (int k = 0; k < HW; ++k) w[k] = 0;
    }
    __device__ void push(uint32_t y) {  // newest spike becomes lag 1
#pragma unroll
        for (int k = HW - 1; k > 0; --k) w[k] = (w[k] << 1) | (w[k - 1] >> 63);
        w[0] = (w[0] << 1) | (uint64_t)y;
    }
    __device__ float bit(int l) const {  // spike l steps ago, l >= 1
        const int p = l - 1;
        if (p >= 64 * HW) return 0.0f;
        return (float)((w[p >> 6] >> (p & 63)) & 1ull);
    }
    // shift towards older times: bit(l) <- bit(l+1); `oldest` enters at lag 64*HW
    __device__ void pull(uint32_t oldest) {
#pragma unroll
        for (int k = 0; k < HW - 1; ++k) w[k] = (w[k] >> 1) | (w[k + 1] << 63);
        w[HW - 1] = (w[HW - 1] >> 1) | ((uint64_t)oldest << 63);
    }
};

__device__ __forceinline__ uint32_t spike_bit(const uint32_t* bits, int TW, int N, int b, int tau, int j) {
    if (tau < 0) return 0u;
    return (bits[((size_t)b * TW + (tau >> 5)) * N + j] >> (tau & 31)) & 1u;
}

// Spike bits of one neuron read backwards in time, one 32-step word at a time, with the
// next older word loaded a word ahead so the stream never waits on memory.
struct SpikeStream {
    const uint32_t* col;   // &bits[b][0][j]; word w at col[w * N]
    int N, widx;
    uint32_t cur, pre;
    __device__ void init(const uint32_t* bits, int TW, int Nn, int b, int j, int tau) {
        N = Nn;
        col = bits + (size_t)b * TW * Nn + j;
        widx = tau >> 5;   // arithmetic shift: -1 for tau in [-32, -1]
        cur = widx >= 0 ? col[(size_t)widx * N] : 0u;
        pre = widx >= 1 ? col[(size_t)(widx - 1) * N] : 0u;
    }
    // bit of time tau; successive calls must go down by one
    __device__ uint32_t bit(int tau) {
        if (tau < 0) return 0u;
        if ((tau >> 5) != widx) {
            widx = tau >> 5;
            cur = pre;
            pre = widx >= 1 ? col[(size_t)(widx - 1) * N] : 0u;
        }
        return (cur >> (tau & 31)) & 1u;
    }
};

// Delayed trace of one neuron from its history (forward tap modes).
template <int HW>
__device__ __forceinline__ float axonal_trace(const History<HW>& h, int taps, float c, float s,
                                              float s2, int lo, int hi, int lag, float frac) {
    if (taps == DELREC_TAPS_SOFT) {
        float z = 0.0f;
        for (int l = lo; l <= hi; ++l) {
            const float yv = h.bit(l);
            z += tri_weight((float)l, c, s, s2) * yv;
        }
        return z;
    }
    if (taps == DELREC_TAPS_ROUND) return h.bit(lag);
    return (1.0f - frac) * h.bit(lag) + frac * h.bit(lag + 1);
}

// ---------------------------------------------------------------------------------------
// Forward.
constexpr int kPrefetch = 4;      // steps of x loaded ahead of use (forward)
constexpr int kPrefetchBwd = 3;   // steps of gy / u loaded ahead of use (backward)

template <int CH, bool RES, int HW>
__global__ void __launch_bounds__(1024) axonal_fwd_kernel(AxFwd p) {
    extern __shared__ float smem[];
    float* zbuf = smem;                               // [2][NZ]
    const int N = p.N, T = p.T, B = p.B, G = p.G, NZ = p.NZ;
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int i = tid / G, g = tid - (tid / G) * G;
    const bool act = i < N;
    const int ic = act ? i : 0;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;

    // resident weight chunk: W[i, g*CH + c]
    float wr[RES ? CH : 1];
    if constexpr (RES) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int j = g * CH + c;
            wr[c] = (act && j < N) ? load_w(p.W, p.w_bf16, (size_t)i * N + j) : 0.0f;
        }
    }
    const int jbeg = g * p.CHS, jend = min(N, jbeg + p.CHS);   // streaming chunk

    // this neuron as a source of the delayed trace: its tap weights, computed once
    const float c = 1.0f + p.d[ic];
    const float s = p.s ? p.s[ic] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool fast = p.taps == DELREC_TAPS_SOFT && nt <= kMaxTaps && HW == 1;
    float wq[kMaxTaps];
#pragma unroll
    for (int q = 0; q < kMaxTaps; ++q) wq[q] = (q < nt) ? tri_weight((float)(lo + q), c, s, s2) : 0.0f;
    const int lag = p.lag ? p.lag[ic] : 1;
    const float frac = p.frac ? p.frac[ic] : 0.0f;
    const float m = p.drop ? p.drop[(size_t)b * N + ic] : 1.0f;
    const float bias = p.bias ? p.bias[ic] : 0.0f;

    for (int q = tid; q < 2 * NZ; q += blockDim.x) zbuf[q] = 0.0f;
    __syncthreads();

    History<HW> hist;
    hist.clear();
    float v = k.v0;
    uint32_t word = 0;
    const size_t BN = (size_t)B * N;
    const size_t row = (size_t)b * N + ic;
    float xq[kPrefetch];
#pragma unroll
    for (int q = 0; q < kPrefetch; ++q) xq[q] = (act && q < T) ? p.x[(size_t)q * BN + row] : 0.0f;
    if (act && g == 0 && p.z) p.z[row] = 0.0f;

    for (int t = 0; t < T; ++t) {
        const float* zc = zbuf + (t & 1) * NZ;
        float acc = 0.0f;
        if constexpr (RES) {
            const float4* z4 = reinterpret_cast<const float4*>(zc + g * CH);
#pragma unroll
            for (int q = 0; q < CH / 4; ++q) {
                const float4 zz = z4[q];
                acc = fmaf(wr[4 * q + 0], zz.x, acc);
                acc = fmaf(wr[4 * q + 1], zz.y, acc);
                acc = fmaf(wr[4 * q + 2], zz.z, acc);
                acc = fmaf(wr[4 * q + 3], zz.w, acc);
            }
        } else {
            for (int j = jbeg; j < jend; ++j)
                acc = fmaf(act ? load_w(p.Wt, p.w_bf16, (size_t)j * N + i) : 0.0f, zc[j], acc);
        }
        acc = group_sum(acc, G);

        const float xv = xq[0];
#pragma unroll
        for (int q = 0; q < kPrefetch - 1; ++q) xq[q] = xq[q + 1];
        xq[kPrefetch - 1] = (act && t + kPrefetch < T) ? p.x[(size_t)(t + kPrefetch) * BN + row] : 0.0f;

        const float r = acc + bias;
        const float a = xv + r * m;
        const float u = lif_charge(k, v, a);
        const float y = lif_fire(k, u);
        v = lif_reset(k, u, y);
        const uint32_t yb = y != 0.0f ? 1u : 0u;
        hist.push(yb);
        word |= yb << (t & 31);
        if (act && g == 0) {
            const size_t o = (size_t)t * BN + row;
            p.y[o] = y;
            p.u[o] = u;
            if (p.rec) p.rec[o] = r;
            if ((t & 31) == 31 || t == T - 1) p.bits[((size_t)b * TW + (t >> 5)) * N + i] = word;
        }
        if ((t & 31) == 31) word = 0;
        if (t + 1 < T) {
            float zn;
            if (fast) {
                const uint64_t hs = hist.w[0] >> (lo - 1);
                zn = 0.0f;
#pragma unroll
                for (int q = 0; q < kMaxTaps; ++q) zn += wq[q] * (float)((hs >> q) & 1ull);
            } else {
                zn = axonal_trace<HW>(hist, p.taps, c, s, s2, lo, hi, lag, frac);
            }
            if (act && g == 0) {
                zbuf[((t + 1) & 1) * NZ + i] = zn;
                if (p.z) p.z[(size_t)(t + 1) * BN + row] = zn;
            }
        }
        barrier_lds();
    }
}

// ---------------------------------------------------------------------------------------
// Backward (reverse time). Lane group of G serves source j (a column of W).
template <int CH, bool RES, int HW>
__global__ void __launch_bounds__(1024) axonal_bwd_kernel(AxBwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B, G = p.G, NZ = p.NZ, R = p.R, NP = p.NP;
    float* grbuf = smem;                 // [2][NZ]
    float* ring = smem + 2 * NZ;         // [R][NP] future gz
    float* htab = ring + R * NP;         // [kMaxTaps][NP] tap weights of each source
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int j = tid / G, g = tid - (tid / G) * G;
    const bool act = j < N;
    const int jc = act ? j : 0;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;

    float wc[RES ? CH : 1];               // column chunk W[g*CH + c, j]
    if constexpr (RES) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int i = g * CH + c;
            wc[c] = (act && i < N) ? load_w(p.W, p.w_bf16, (size_t)i * N + j) : 0.0f;
        }
    }
    const int ibeg = g * p.CHS, iend = min(N, ibeg + p.CHS);

    const float c = 1.0f + p.d[jc];
    const float s = p.s ? p.s[jc] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool soft = p.mode == DELREC_BWD_SOFT;
    const bool fast = soft && nt <= kMaxTaps && HW == 1;
    const bool need_ds = p.s != nullptr;

    const int lag = p.lag ? p.lag[jc] : 1;
    const float m = p.drop ? p.drop[(size_t)b * N + jc] : 1.0f;

    for (int q = tid; q < 2 * NZ + R * NP; q += blockDim.x) smem[q] = 0.0f;
    if (act && g == 0) {
#pragma unroll
        for (int q = 0; q < kMaxTaps; ++q)
            htab[q * NP + j] = (q < nt) ? tri_weight((float)(lo + q), c, s, s2) : 0.0f;
    }
    __syncthreads();

    // past spikes of j relative to step t: bit(l) = y[t-l]; start at t = T-1
    History<HW> past;
    past.clear();
    for (int l = 64 * HW; l >= 1; --l) past.push(act ? spike_bit(p.bits, TW, N, b, T - 1 - l, jc) : 0u);

    const size_t BN = (size_t)B * N;
    const size_t rowj = (size_t)b * N + jc;
    float gq[kPrefetchBwd], uq[kPrefetchBwd];
#pragma unroll
    for (int q = 0; q < kPrefetchBwd; ++q) {
        const int tt = T - 1 - q;
        gq[q] = (act && tt >= 0) ? p.gy[(size_t)tt * BN + rowj] : 0.0f;
        uq[q] = (act && tt >= 0) ? p.u[(size_t)tt * BN + rowj] : 0.0f;
    }
    float lam = 0.0f, db_acc = 0.0f, dd_acc = 0.0f, ds_acc = 0.0f;
    int tmod = (T - 1) % R;

    for (int t = T - 1; t >= 0; --t) {
        // future gradient through the delayed trace
        float gfut = 0.0f;
        if (fast) {
#pragma unroll
            for (int q = 0; q < kMaxTaps; ++q) {
                const int l = lo + q;
                if (q < nt && t + l < T) {
                    int slot = tmod + l;
                    if (slot >= R) slot -= R;
                    gfut += htab[q * NP + jc] * ring[slot * NP + jc];
                }
            }
        } else if (soft) {
            for (int l = lo; l <= hi && t + l < T; ++l) {
                int slot = tmod + l;
                if (slot >= R) slot -= R;
                gfut += tri_weight((float)l, c, s, s2) * ring[slot * NP + jc];
            }
        } else if (t + lag < T) {
            int slot = tmod + lag;
            if (slot >= R) slot -= R;
            gfut = ring[slot * NP + jc];
        }
        const float gy = gq[0], u = uq[0];
#pragma unroll
        for (int q = 0; q < kPrefetchBwd - 1; ++q) {
            gq[q] = gq[q + 1];
            uq[q] = uq[q + 1];
        }
        const int tn = t - kPrefetchBwd;
        gq[kPrefetchBwd - 1] = (act && tn >= 0) ? p.gy[(size_t)tn * BN + rowj] : 0.0f;
        uq[kPrefetchBwd - 1] = (act && tn >= 0) ? p.u[(size_t)tn * BN + rowj] : 0.0f;

        const float y = lif_fire(k, u);
        const float du = lif_backward(k, gy + gfut, u, y, lam);
        lam = k.decay * du;
        const float da = lif_dx(k, du);       // dL/d(input of the charge)
        const float gr = da * m;
        if (act && g == 0) {
            const size_t o = (size_t)t * BN + rowj;
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            grbuf[(t & 1) * NZ + j] = gr;
        }
        db_acc += gr;
        barrier_lds();

        // gz_j = sum_i gr_i W[i, j]
        const float* gb = grbuf + (t & 1) * NZ;
        float acc = 0.0f;
        if constexpr (RES) {
            const float4* g4 = reinterpret_cast<const float4*>(gb + g * CH);
#pragma unroll
            for (int q = 0; q < CH / 4; ++q) {
                const float4 gg = g4[q];
                acc = fmaf(wc[4 * q + 0], gg.x, acc);
                acc = fmaf(wc[4 * q + 1], gg.y, acc);
                acc = fmaf(wc[4 * q + 2], gg.z, acc);
                acc = fmaf(wc[4 * q + 3], gg.w, acc);
            }
        } else {
            for (int i = ibeg; i < iend; ++i)
                acc = fmaf(act ? load_w(p.W, p.w_bf16, (size_t)i * N + j) : 0.0f, gb[i], acc);
        }
        const float gz = group_sum(acc, G);
        if (act) ring[tmod * NP + j] = gz;

        // delay / half-width gradients: dL/dh[j,l] = gz_t * y[t-l]
        if (fast && !need_ds) {
            const uint32_t ps = (uint32_t)(past.w[0] >> (lo - 1));
            float sd = 0.0f;
#pragma unroll
            for (int q = 0; q < kMaxTaps; ++q)
                sd += (q < nt && ((ps >> q) & 1u)) ? tri_dsign((float)(lo + q), c, s) : 0.0f;
            dd_acc += gz * sd;
        } else if (soft) {
            float sd = 0.0f, sds = 0.0f;
            for (int l = lo; l <= hi; ++l) {
                const float yv = past.bit(l);
                sd += tri_dsign((float)l, c, s) * yv;
                if (need_ds) sds += tri_ds((float)l, c, s, s2) * yv;
            }
            dd_acc += gz * sd;
            ds_acc += gz * sds;
        } else {
            dd_acc += gz * (past.bit(lag + 1) - past.bit(lag));
        }

        // slide the past window one step back
        if (t > 0) past.pull(act ? spike_bit(p.bits, TW, N, b, t - 1 - 64 * HW, jc) : 0u);
        tmod = tmod == 0 ? R - 1 : tmod - 1;
    }
    if (act && g == 0) {
        p.part[(size_t)0 * B * N + rowj] = db_acc;
        p.part[(size_t)1 * B * N + rowj] = soft ? dd_acc / s2 : dd_acc;
        p.part[(size_t)2 * B * N + rowj] = ds_acc;
    }
}

// ---------------------------------------------------------------------------------------
// Tiled forms for N <= 256 (the fast path). The GEMV lanes hold an RI x CJ tile of W in
// VGPRs: lane (grp, jcg) owns receivers grp*RI .. +RI and sources jcg*CJ .. +CJ, the NJ
// chunk lanes of a group sit in one DPP row and reduce there with a butterfly that leaves
// the RI row sums in every lane of the group. Neuron i = grp*RI + a lives on lane
// (grp, jcg = a) of its own group, so the recurrent input reaches it inside the wave;
// only z (forward) / gr (backward) cross waves, through LDS with a chunk pitch of CJ + 4
// floats (the NJ chunk reads of a row hit distinct banks): one barrier per step.
template <int CJ>
__device__ __forceinline__ int zpos(int j) { return (j / CJ) * (CJ + 4) + (j % CJ); }

template <int RI> struct TiledThreads { static constexpr int value = RI >= 4 ? 512 : 1024; };

// acc[a] of the lane's group for the lane's own a: a dot product with the lane's constant
// one-hot mask (exact for finite sums; a select chain on a lane index would be lowered to
// an indexed scratch access)
template <int RI>
struct OneHot {
    float m[RI];
    __device__ __forceinline__ void init(int sel) {
#pragma unroll
        for (int a = 0; a < RI; ++a) m[a] = (sel == a) ? 1.0f : 0.0f;
    }
    __device__ __forceinline__ float pick(const float (&acc)[RI]) const {
        float r = acc[0] * m[0];
#pragma unroll
        for (int a = 1; a < RI; ++a) r = fmaf(acc[a], m[a], r);
        return r;
    }
};

template <int RI, int NJ, int HW, int CJ>
__global__ void __launch_bounds__(TiledThreads<RI>::value) axonal_fwd_tiled(AxFwd p) {
    extern __shared__ float smem[];
    constexpr int CJP = CJ + 4;
    const int N = p.N, T = p.T, B = p.B, NZ = p.NZ;
    float* zbuf = smem;                 // [2][NZ], NZ = NJ * CJP
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int grp = tid / NJ, jcg = tid - (tid / NJ) * NJ;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;

    float w[RI][CJ];
    load_w_tile<RI, CJ>(w, p.W, p.w_bf16, N, [&](int a, int c, int& i, int& j) {
        i = grp * RI + a;
        j = jcg * CJ + c;
    });

    // neuron lanes: neuron i = grp * RI + jcg on the lanes jcg < RI
    const bool nl = jcg < RI && grp * RI + jcg < N;
    OneHot<RI> sel;
    sel.init(jcg);
    const int i = nl ? grp * RI + jcg : 0;
    const float c = 1.0f + p.d[i];
    const float s = p.s ? p.s[i] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool fast = p.taps == DELREC_TAPS_SOFT && nt <= kMaxTaps && HW == 1;
    float wq[kMaxTaps];
#pragma unroll
    for (int q = 0; q < kMaxTaps; ++q) wq[q] = (q < nt) ? tri_weight((float)(lo + q), c, s, s2) : 0.0f;
    const int lag = p.lag ? p.lag[i] : 1;
    const float frac = p.frac ? p.frac[i] : 0.0f;
    const float m = p.drop ? p.drop[(size_t)b * N + i] : 1.0f;
    const float bias = p.bias ? p.bias[i] : 0.0f;

    for (int q = tid; q < 2 * NZ; q += blockDim.x) zbuf[q] = 0.0f;
    __syncthreads();

    History<HW> hist;
    hist.clear();
    float v = k.v0;
    uint32_t word = 0;
    const size_t BN = (size_t)B * N;
    const size_t row = (size_t)b * N + i;
    float xq[kPrefetch];
#pragma unroll
    for (int q = 0; q < kPrefetch; ++q) xq[q] = (nl && q < T) ? p.x[(size_t)q * BN + row] : 0.0f;
    if (nl && p.z) p.z[row] = 0.0f;

    // one time step; `xs` is this step's prefetch slot, refilled with x[t + kPrefetch]
    auto step = [&](const int t, float& xs) {
        // GEMV: r_i = sum_j W[i, j] z_j over this lane's tile, reduced across the row
        const float4* z4 = reinterpret_cast<const float4*>(zbuf + (t & 1) * NZ + jcg * CJP);
        float acc[RI];
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = 0.0f;
#pragma unroll
        for (int q = 0; q < CJ / 4; ++q) {
            const float4 zz = z4[q];
#pragma unroll
            for (int a = 0; a < RI; ++a) {
                acc[a] = fmaf(w[a][4 * q + 0], zz.x, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 1], zz.y, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 2], zz.z, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 3], zz.w, acc[a]);
            }
        }
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = group_sum_t<NJ>(acc[a]);

        if (nl) {
            const float xv = xs;
            xs = (t + kPrefetch < T) ? p.x[(size_t)(t + kPrefetch) * BN + row] : 0.0f;
            const float r = sel.pick(acc) + bias;
            const float a = xv + r * m;
            const float u = lif_charge(k, v, a);
            const float y = lif_fire(k, u);
            v = lif_reset(k, u, y);
            const uint32_t yb = y != 0.0f ? 1u : 0u;
            hist.push(yb);
            word |= yb << (t & 31);
            const size_t o = (size_t)t * BN + row;
            p.y[o] = y;
            p.u[o] = u;
            if (p.rec) p.rec[o] = r;
            if ((t & 31) == 31 || t == T - 1) {
                p.bits[((size_t)b * TW + (t >> 5)) * N + i] = word;
                word = 0;
            }
            if (t + 1 < T) {
                float zn;
                if (fast) {
                    const uint32_t hs = (uint32_t)(hist.w[0] >> (lo - 1));
                    zn = 0.0f;
#pragma unroll
                    for (int q = 0; q < kMaxTaps; ++q) zn += ((hs >> q) & 1u) ? wq[q] : 0.0f;
                } else {
                    zn = axonal_trace<HW>(hist, p.taps, c, s, s2, lo, hi, lag, frac);
                }
                zbuf[((t + 1) & 1) * NZ + zpos<CJ>(i)] = zn;
                if (p.z) p.z[(size_t)(t + 1) * BN + row] = zn;
            }
        }
        barrier_lds();
    };

    for (int t0 = 0; t0 < T; t0 += kPrefetch) {
#pragma unroll
        for (int q = 0; q < kPrefetch; ++q)
            if (t0 + q < T) step(t0 + q, xq[q]);
    }
}

// ---------------------------------------------------------------------------------------
// Spike-driven forward for N <= 256. Wave w owns the source block j = 32w .. 32w + 31 for
// every receiver (lane l holds W[RI*l + a][32w + c] in VGPRs) and runs the LIF chain of
// those 32 neurons on its lanes 0..31. Its delayed trace z(t) stays in the lane of the
// source; a wave ballot of z != 0 gives the active columns of the block, and the
// contraction walks only those (the column index is wave-uniform, so the weight column
// is picked with GPR-index addressing and z with readlane). At typical firing rates that
// is a small fraction of the dense product. The per-wave partial sums of every receiver
// cross waves through LDS: one barrier per step, no z traffic through memory.
constexpr int kPrefetchWave = 8;   // steps of x loaded ahead of use

typedef float wcol32 __attribute__((ext_vector_type(32)));

template <int RI>
__device__ __forceinline__ void store_partials(float* dst, const float (&acc)[RI]) {
    if constexpr (RI == 4) {
        *reinterpret_cast<float4*>(dst) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else if constexpr (RI == 2) {
        *reinterpret_cast<float2*>(dst) = make_float2(acc[0], acc[1]);
    } else {
        dst[0] = acc[0];
    }
}

template <int RI, int HW>
__global__ void __launch_bounds__(512) axonal_fwd_wave(AxFwd p) {
    extern __shared__ float smem[];
    constexpr int ROWS = 64 * RI;                  // receivers covered by one wave's lanes
    const int N = p.N, T = p.T, B = p.B;
    const int NW = blockDim.x >> 6;                // waves = source blocks of 32
    float* part = smem;                            // [2][NW][ROWS]
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int wv = tid >> 6, l = tid & 63;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;

    wcol32 w[RI];
    load_w_tile<RI, 32>(w, p.W, p.w_bf16, N, [&](int a, int c, int& i, int& j) {
        i = RI * l + a;
        j = 32 * wv + c;
    });

    // neuron lanes: neuron i = 32 * wv + l on lanes l < 32
    const bool nl = l < 32 && 32 * wv + l < N;
    const int i = nl ? 32 * wv + l : 0;
    const float c = 1.0f + p.d[i];
    const float s = p.s ? p.s[i] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool fast = p.taps == DELREC_TAPS_SOFT && nt <= kMaxTaps && HW == 1;
    float wq[kMaxTaps];
#pragma unroll
    for (int q = 0; q < kMaxTaps; ++q) wq[q] = (q < nt) ? tri_weight((float)(lo + q), c, s, s2) : 0.0f;
    const int lag = p.lag ? p.lag[i] : 1;
    const float frac = p.frac ? p.frac[i] : 0.0f;
    const float m = p.drop ? p.drop[(size_t)b * N + i] : 1.0f;
    const float bias = p.bias ? p.bias[i] : 0.0f;

    History<HW> hist;
    hist.clear();
    float v = k.v0;
    uint32_t word = 0;
    const size_t BN = (size_t)B * N;
    const size_t row = (size_t)b * N + i;
    float xq[kPrefetchWave];
#pragma unroll
    for (int q = 0; q < kPrefetchWave; ++q) xq[q] = (nl && q < T) ? p.x[(size_t)q * BN + row] : 0.0f;
    if (nl && p.z) p.z[row] = 0.0f;

    float zcur = 0.0f;         // z(t) of this lane's source (0 off the neuron lanes)
    uint32_t zmask = 0;        // lanes of this wave whose z(t) != 0 (wave-uniform)

    // one time step; `xs` is this step's prefetch slot, refilled with x[t + kPrefetchWave]
    // (static slots: a register with a load in flight is never moved)
    auto step = [&](const int t, float& xs) {
        float acc[RI];
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = 0.0f;
        uint32_t mk = __builtin_amdgcn_readfirstlane(zmask);
        while (mk) {
            const int cc = __builtin_ctz(mk);
            mk &= mk - 1u;
            const float zc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(zcur), cc));
#pragma unroll
            for (int a = 0; a < RI; ++a) acc[a] = fmaf(w[a][cc], zc, acc[a]);
        }
        float* pt = part + (t & 1) * NW * ROWS;
        store_partials<RI>(pt + wv * ROWS + RI * l, acc);
        // refill the slot on every lane, outside the divergent region and with a clamped
        // (always valid) step, so the load never has to land before a later step reads it
        const float xv = xs;
        xs = p.x[(size_t)min(t + kPrefetchWave, T - 1) * BN + row];
        barrier_lds();

        float zn = 0.0f;
        if (nl && t < T) {
            float r = 0.0f;
            for (int q = 0; q < NW; ++q) r += pt[q * ROWS + i];
            r += bias;
            const float a = xv + r * m;
            const float u = lif_charge(k, v, a);
            const float y = lif_fire(k, u);
            v = lif_reset(k, u, y);
            const uint32_t yb = y != 0.0f ? 1u : 0u;
            hist.push(yb);
            word |= yb << (t & 31);
            const size_t o = (size_t)t * BN + row;
            p.y[o] = y;
            p.u[o] = u;
            if (p.rec) p.rec[o] = r;
            if ((t & 31) == 31 || t == T - 1) {
                p.bits[((size_t)b * TW + (t >> 5)) * N + i] = word;
                word = 0;
            }
            if (t + 1 < T) {
                if (fast) {
                    const uint32_t hs = (uint32_t)(hist.w[0] >> (lo - 1));
#pragma unroll
                    for (int q = 0; q < kMaxTaps; ++q) zn += ((hs >> q) & 1u) ? wq[q] : 0.0f;
                } else {
                    zn = axonal_trace<HW>(hist, p.taps, c, s, s2, lo, hi, lag, frac);
                }
                if (p.z) p.z[(size_t)(t + 1) * BN + row] = zn;
            }
        }
        zcur = zn;
        zmask = (uint32_t)__ballot(zn != 0.0f);
    };

    // whole blocks of kPrefetchWave steps (a step t >= T does no neuron work): a guard
    // around a step would make its prefetch slot a merge that waits for the load
    for (int t0 = 0; t0 < T; t0 += kPrefetchWave) {
#pragma unroll
        for (int q = 0; q < kPrefetchWave; ++q) step(t0 + q, xq[q]);
    }
}

// The same spike-driven scan specialised for the common regime (chosen by the host):
// soft triangle taps of a uniform half-width s with at most KF lags of non-zero weight
// (KF >= ceil(2s)) inside one 64-step history word, charge u = decay * v + a, hard reset
// to 0, no recurrent-input output.
//
// The step is software-pipelined around the one dependency that really crosses a step:
// a source whose first non-zero tap is at lag 1 ("fast", d < 2 + ... ) needs this step's
// spike to form its z(t+1); every other source's z(t+1) is fixed by spikes up to t-1.
// So while the LDS reads of r(t)'s partial sums are in flight, each wave forms the
// pre-step traces zpre(t+1) and contracts its slow active columns for step t+1; after
// the LIF only the fast sources' lag-1 term and their (few) columns remain on the
// critical path. Stores and the x prefetch use buffer descriptors in SGPRs.
// f(std::integral_constant<int, Q>{}) for Q = 0, 1, ... in order (an unrolled loop whose
// index is a compile-time constant in the body)
template <class F, int... Q>
__device__ __forceinline__ void unroll_steps(std::integer_sequence<int, Q...>, F&& f) {
    (f(std::integral_constant<int, Q>{}), ...);
}

// spike-history window of HW 64-bit words: bits sh .. sh + 31 (sh >= -1; bit -1 reads 0)
template <int HW>
__device__ __forceinline__ uint32_t hist_bits(const uint64_t (&h)[HW], int sh) {
    if constexpr (HW == 1) {
        return (uint32_t)(sh >= 0 ? (h[0] >> sh) : (h[0] << 1));
    } else {
        if (sh < 0) return (uint32_t)(h[0] << 1);
        const int wi = sh >> 6, bi = sh & 63;
        uint64_t lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            lo = (k == wi) ? h[k] : lo;
            hi = (k == wi + 1) ? h[k] : hi;
        }
        return (uint32_t)(bi ? ((lo >> bi) | (hi << (64 - bi))) : lo);
    }
}

template <int RI, int KF, int HW>
__device__ __forceinline__ void axonal_fwd_wave_fast_body(const AxFwd& p, float* smem) {
    constexpr int ROWS = 64 * RI;
    constexpr int NWMAX = 8;
    const int N = p.N, T = p.T, B = p.B;
    float* part = smem;                            // [2][NWMAX][ROWS]
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int wv = tid >> 6, l = tid & 63;
    const int TW = (T + 31) >> 5;
    const float decay = p.lif.decay, vth = p.lif.vth;

    wcol32 w[RI];
    load_w_tile<RI, 32>(w, p.W, p.w_bf16, N, [&](int a, int c, int& i, int& j) {
        i = RI * l + a;
        j = 32 * wv + c;
    });

    const bool nl = l < 32 && 32 * wv + l < N;
    const int i = nl ? 32 * wv + l : 0;
    const float c = 1.0f + p.d[i];
    const float s = p.s_uniform;
    const float s2 = s * s;
    // lags of non-zero weight: l > c - s, l >= 1 (at most KF of them: l < c + s)
    const int lof = max(1, (int)floorf(c - s) + 1);
    // L = 0: the window was not read by the caller; every lag of non-zero weight lies
    // below c + s <= L - 1, so the cap only matters for the lags a history cannot hold
    const int lcap = p.L > 0 ? p.L - 1 : 64 * HW;
    int wq[KF];                // tap weights as bit patterns (masked by the spike bits)
#pragma unroll
    for (int q = 0; q < KF; ++q) {
        const int lq = lof + q;
        wq[q] = __float_as_int(lq <= lcap ? tri_weight((float)lq, c, s, s2) : 0.0f);
    }
    const bool fastn = nl && lof == 1;             // z(t+1) needs y(t)
    const bool slown = nl && lof >= 2;
    const float w0 = fastn ? __int_as_float(wq[0]) : 0.0f;
    const float m = p.drop ? p.drop[(size_t)b * N + i] : 1.0f;
    const float bias = p.bias ? p.bias[i] : 0.0f;

    for (int q = tid; q < 2 * NWMAX * ROWS; q += blockDim.x) part[q] = 0.0f;
    __syncthreads();

    // hist bit k = y(t-1-k) at the start of step t. zpre(t+1) = sum_q w_q y(t+1-lof-q)
    // over the known spikes: bit (lof - 2 + q); for a fast source the q = 0 term is y(t).
    uint64_t hist[HW];
#pragma unroll
    for (int k = 0; k < HW; ++k) hist[k] = 0;
    float v = 0.0f;
    uint32_t word = 0;
    const size_t BN = (size_t)B * N;
    const uint32_t row_bytes = (uint32_t)BN * 4u;  // one step of a (T, B, N) tensor
    const uint32_t all_bytes = (uint32_t)T * row_bytes;   // at most 1 GiB (host check)
    const uint32_t voff = (uint32_t)(b * N + i) * 4u;     // this lane's byte offset within a step
    // One descriptor per tensor for the whole scan and one moving byte offset per lane: the
    // offset of step t is voff + t * row_bytes, which lies past the buffer end for steps
    // t >= T (stores dropped, loads read 0). Lanes without a neuron start past the end and
    // stay there (no wrap: twice the tensor plus a few steps fits 32 bits). Every memory
    // operation of a step is unconditional, so the compiler's counts of outstanding loads /
    // stores are exact and a prefetched value never waits on later stores.
    float* const zout = p.z;
    const i32x4 xr = buffer_rsrc(p.x, all_bytes), yr = buffer_rsrc(p.y, all_bytes);
    const i32x4 ur = buffer_rsrc(p.u, all_bytes), zr = buffer_rsrc(zout, zout ? all_bytes : 0u);
    const i32x4 br = buffer_rsrc(p.bits, (uint32_t)B * TW * N * 4u);
    const uint32_t boff = nl ? (uint32_t)(b * TW * N + i) * 4u : (uint32_t)kOutOfRange;   // word of steps 0..31
    const uint32_t n4 = (uint32_t)N * 4u;
    uint32_t vo = nl ? voff : all_bytes;           // y, u of step t; z of step t + 1 one row on
    uint32_t vx = voff + (uint32_t)kPrefetchWave * row_bytes;   // x of step t + P
    float xq[kPrefetchWave];
#pragma unroll
    for (int q = 0; q < kPrefetchWave; ++q) xq[q] = raw_buffer_load_f32(xr, voff + (uint32_t)q * row_bytes, 0, 0);
    if (nl && zout) zout[(size_t)b * N + i] = 0.0f;

    float zcur = 0.0f;                             // z(t) of this lane's source
    uint32_t mkf = 0;                              // fast sources with z(t) != 0
    float acc_s[RI];                               // slow columns of W z(t)
#pragma unroll
    for (int a = 0; a < RI; ++a) acc_s[a] = 0.0f;

    // step t = t0 + Q of a group of kPrefetchWave (Q a compile-time constant: only the last
    // step of a group can end a 32-step spike word)
    auto step = [&](const int t, float& xs, auto qc) {
        constexpr int Q = decltype(qc)::value;
        // fast columns of z(t) on top of the slow part formed during the previous step
        float acc[RI];
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = acc_s[a];
        uint32_t mk = __builtin_amdgcn_readfirstlane(mkf);
        while (mk) {
            const int cc = __builtin_ctz(mk);
            mk &= mk - 1u;
            // the weight column in one indexed-register run, then the spike value
            float wt[RI];
#pragma unroll
            for (int a = 0; a < RI; ++a) wt[a] = w[a][cc];
            __builtin_amdgcn_sched_barrier(0);
            const float zc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(zcur), cc));
#pragma unroll
            for (int a = 0; a < RI; ++a) acc[a] = fmaf(wt[a], zc, acc[a]);
        }
        float* pt = part + (t & 1) * NWMAX * ROWS;
        store_partials<RI>(pt + wv * ROWS + RI * l, acc);
        barrier_lds();
        float pr[NWMAX];                           // r(t) partials, read before the slow work
#pragma unroll
        for (int q = 0; q < NWMAX; ++q) pr[q] = pt[q * ROWS + i];

        // in the shadow of those reads: zpre(t+1) and the slow columns of W z(t+1)
        const uint32_t hs = hist_bits<HW>(hist, lof - 2);
        float zpre = 0.0f;
#pragma unroll
        for (int q = 0; q < KF; ++q) zpre += __int_as_float(wq[q] & -(int)((hs >> q) & 1u));
        const bool next = t + 1 < T;
        zpre = next ? zpre : 0.0f;
#pragma unroll
        for (int a = 0; a < RI; ++a) acc_s[a] = 0.0f;
        uint32_t ms = __builtin_amdgcn_readfirstlane((uint32_t)__ballot(slown && zpre != 0.0f));
        while (ms) {
            const int cc = __builtin_ctz(ms);
            ms &= ms - 1u;
            float wt[RI];
#pragma unroll
            for (int a = 0; a < RI; ++a) wt[a] = w[a][cc];
            __builtin_amdgcn_sched_barrier(0);
            const float zc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(zpre), cc));
#pragma unroll
            for (int a = 0; a < RI; ++a) acc_s[a] = fmaf(wt[a], zc, acc_s[a]);
        }

        // r(t) and the LIF step
        float r = pr[0];
#pragma unroll
        for (int q = 1; q < NWMAX; ++q) r += pr[q];
        r += bias;
        const float a = xs + r * m;
        const float u = v * decay + a;
        const bool fire = u - vth >= 0.0f;
        v = fire ? 0.0f : u;
#pragma unroll
        for (int k = HW - 1; k > 0; --k) hist[k] = (hist[k] << 1) | (hist[k - 1] >> 63);
        hist[0] = (hist[0] << 1) | (uint64_t)(fire ? 1u : 0u);
        word |= (fire ? 1u : 0u) << (t & 31);
        // z(t+1): the fast sources add their lag-1 tap
        float zn = (fastn && fire) ? w0 + zpre : zpre;
        zn = (nl && next) ? zn : 0.0f;
        mkf = (uint32_t)__ballot(fastn && zn != 0.0f);
        zcur = zn;

        // outputs; steps t >= T store nothing (their offsets lie past the buffer end)
        raw_buffer_store_f32(fire ? 1.0f : 0.0f, yr, vo, 0, 0);
        raw_buffer_store_f32(u, ur, vo, 0, 0);
        raw_buffer_store_f32(zn, zr, vo + row_bytes, 0, 0);
        vo += row_bytes;
        // the spike-bit word of steps 32k .. 32k+31, written at its last step
        bool flush = t == T - 1;
        if constexpr (Q == kPrefetchWave - 1) flush = flush || ((t & 31) == 31 && t < T);
        if (flush) raw_buffer_store_f32(__uint_as_float(word), br, boff + (uint32_t)(t >> 5) * n4, 0, 0);
        if constexpr (Q == kPrefetchWave - 1) {
            if ((t & 31) == 31) word = 0;
        }
        // refill the slot after its value is used (no copy, so no wait on the load)
        xs = raw_buffer_load_f32(xr, vx, 0, 0);
        vx += row_bytes;
    };

    for (int t0 = 0; t0 < T; t0 += kPrefetchWave)
        unroll_steps(std::make_integer_sequence<int, kPrefetchWave>{},
                     [&](auto qc) { step(t0 + decltype(qc)::value, xq[decltype(qc)::value], qc); });
}

template <int RI, int NJ, int HW, int CJ>
__global__ void __launch_bounds__(TiledThreads<RI>::value) axonal_bwd_tiled(AxBwd p) {
    extern __shared__ float smem[];
    constexpr int CJP = CJ + 4;
    const int N = p.N, T = p.T, B = p.B, NZ = p.NZ, R = p.R, NP = p.NP;
    float* grbuf = smem;                 // [2][NZ]
    float* ring = smem + 2 * NZ;         // [R][NP]: column j holds gz_j of the future steps
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int grp = tid / NJ, jcg = tid - (tid / NJ) * NJ;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;

    // tile of W^T: sources grp*RI + a (rows of the GEMV), receivers jcg*CJ + c (columns)
    float w[RI][CJ];
    load_w_tile<RI, CJ>(w, p.W, p.w_bf16, N, [&](int a, int cc, int& i, int& j) {
        j = grp * RI + a;
        i = jcg * CJ + cc;
    });

    // Source j = grp*RI + a runs its LIF chain on lane (grp, a). Its dL/dz is stored (gz)
    // for the delay-gradient pass, which keeps that work off the sequential scan.
    const bool nl = jcg < RI && grp * RI + jcg < N;                      // LIF lanes
    const int j = nl ? grp * RI + jcg : 0;
    OneHot<RI> sel;
    sel.init(jcg % RI);
    const float c = 1.0f + p.d[j];
    const float s = p.s ? p.s[j] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool soft = p.mode == DELREC_BWD_SOFT;
    const bool fast = soft && nt <= kMaxTaps && HW == 1;
    float wq[kMaxTaps];
#pragma unroll
    for (int q = 0; q < kMaxTaps; ++q) wq[q] = (q < nt) ? tri_weight((float)(lo + q), c, s, s2) : 0.0f;
    const int lag = p.lag ? p.lag[j] : 1;
    const float m = p.drop ? p.drop[(size_t)b * N + j] : 1.0f;

    for (int q = tid; q < 2 * NZ + R * NP; q += blockDim.x) smem[q] = 0.0f;
    __syncthreads();

    const size_t BN = (size_t)B * N;
    const size_t rowj = (size_t)b * N + j;
    float gq[kPrefetchBwd], uq[kPrefetchBwd];
#pragma unroll
    for (int q = 0; q < kPrefetchBwd; ++q) {
        const int tt = T - 1 - q;
        gq[q] = (nl && tt >= 0) ? p.gy[(size_t)tt * BN + rowj] : 0.0f;
        uq[q] = (nl && tt >= 0) ? p.u[(size_t)tt * BN + rowj] : 0.0f;
    }
    float lam = 0.0f, db_acc = 0.0f;

    // gz(t+1) of this lane's source: W^T-tile contraction of gr(t+1), reduced in the group
    auto contract = [&](int buf) {
        const float4* g4 = reinterpret_cast<const float4*>(grbuf + buf * NZ + jcg * CJP);
        float acc[RI];
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = 0.0f;
#pragma unroll
        for (int q = 0; q < CJ / 4; ++q) {
            const float4 gg = g4[q];
#pragma unroll
            for (int a = 0; a < RI; ++a) {
                acc[a] = fmaf(w[a][4 * q + 0], gg.x, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 1], gg.y, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 2], gg.z, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 3], gg.w, acc[a]);
            }
        }
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = group_sum_t<NJ>(acc[a]);
        return sel.pick(acc);
    };

    int tn1 = T % R;                                   // slot of time t + 1
    // one reverse step; `gs`, `us` are this step's prefetch slots, refilled with step t - P
    auto step = [&](const int t, float& gs, float& us) {
        const float gz1 = contract((t + 1) & 1);       // gz(t+1); gr(T) = 0
        const int tm = tn1 == 0 ? R - 1 : tn1 - 1;     // slot of time t
        if (nl) {
            ring[tn1 * NP + j] = gz1;
            if (t + 1 < T) p.gz[(size_t)(t + 1) * BN + rowj] = gz1;
            float gfut = 0.0f;
            if (fast) {
                // taps past the support weigh 0 and ring slots of times >= T hold 0
                int sb = tm + lo;
                if (sb >= R) sb -= R;
#pragma unroll
                for (int q = 0; q < kMaxTaps; ++q) {
                    int slot = sb + q;
                    if (slot >= R) slot -= R;
                    gfut += wq[q] * ring[slot * NP + j];
                }
            } else if (soft) {
                for (int l = lo; l <= hi && t + l < T; ++l) {
                    int slot = tm + l;
                    if (slot >= R) slot -= R;
                    gfut += tri_weight((float)l, c, s, s2) * ring[slot * NP + j];
                }
            } else if (t + lag < T) {
                int slot = tm + lag;
                if (slot >= R) slot -= R;
                gfut = ring[slot * NP + j];
            }
            const float gy = gs, u = us;
            const int tn = t - kPrefetchBwd;
            gs = tn >= 0 ? p.gy[(size_t)tn * BN + rowj] : 0.0f;
            us = tn >= 0 ? p.u[(size_t)tn * BN + rowj] : 0.0f;

            const float y = lif_fire(k, u);
            const float du = lif_backward(k, gy + gfut, u, y, lam);
            lam = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * m;
            const size_t o = (size_t)t * BN + rowj;
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            grbuf[(t & 1) * NZ + zpos<CJ>(j)] = gr;
            db_acc += gr;
        }
        barrier_lds();
        tn1 = tm;
    };

    // steps T-1, T-2, ... in groups of kPrefetchBwd; slot q holds step T-1-(n*P+q)
    for (int t0 = T - 1; t0 >= 0; t0 -= kPrefetchBwd) {
#pragma unroll
        for (int q = 0; q < kPrefetchBwd; ++q)
            if (t0 - q >= 0) step(t0 - q, gq[q], uq[q]);
    }
    const float gz0 = contract(0);                     // gz(0)
    if (nl) {
        p.gz[rowj] = gz0;
        p.part[(size_t)0 * B * N + rowj] = db_acc;
    }
}

// Picks the history length from d itself (block-uniform): one 64-step word when every
// neuron's lags of non-zero weight fit, else four words (256 lags). When the caller asked
// for max d on the host, workgroup 0 first writes it into the readback slot (the store's
// trip to host memory then overlaps the scan).
//
// Without a window length from the caller (L = 0) a neuron with a lag of non-zero weight
// beyond 256 cannot be held: the scan then writes NaN into y, u (and z) instead of dropping
// those taps, and posts NaN as max d, which the backward's window-length read rejects.
// (Every workgroup tests all N neurons, so the decision is the same in all of them.)
template <int RI, int KF>
__global__ void __launch_bounds__(512) axonal_fwd_wave_fast(AxFwd p) {
    extern __shared__ float smem[];
    const int l = threadIdx.x & 63, i = 32 * (threadIdx.x >> 6) + l;
    bool longer = false, beyond = false;
    if (l < 32 && i < p.N) {
        const float c = 1.0f + p.d[i];
        const float s = p.s_uniform, s2 = s * s;
        const int lof = max(1, (int)floorf(c - s) + 1);
        longer = lof + KF - 1 > 64;
#pragma unroll
        for (int q = 0; q < KF; ++q) {
            const int lq = lof + q;
            beyond |= p.L == 0 && lq > 256 && tri_weight((float)lq, c, s, s2) > 0.0f;
        }
    }
    beyond = __syncthreads_or(beyond);
    if (p.mx_slot && blockIdx.x == 0) block_max_to_host(p.d, p.N, p.mx_ticket, p.mx_slot, beyond);
    if (beyond) {
        const float nan = __builtin_nanf("");
        const size_t BN = (size_t)p.B * p.N;
        for (size_t q = threadIdx.x; q < (size_t)p.T * p.N; q += blockDim.x) {
            const size_t t = q / p.N, o = t * BN + (size_t)blockIdx.x * p.N + (q - t * p.N);
            p.y[o] = nan;
            p.u[o] = nan;
            if (p.z) p.z[o] = nan;
        }
        return;
    }
    if (__syncthreads_or(longer)) axonal_fwd_wave_fast_body<RI, KF, 4>(p, smem);
    else axonal_fwd_wave_fast_body<RI, KF, 1>(p, smem);
}

// The sum over the 8 lanes of a group of a[jcg & 3] (jcg = lane mod 8, bits b1 b0): lanes i
// and 7 - i add all four values (half-row mirror), then the quad halves them: keep two values
// and add the partner's (lane ^ 2), keep one and add the partner's (lane ^ 1). 13 VALU in
// place of a butterfly over all four values and a one-hot pick (16).
__device__ __forceinline__ float reduce_scatter_4x8(float (&a)[4], bool b1, bool b0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] += dpp<0x141>(a[k]);   // row_half_mirror: lane 7 - i
    float x0 = b1 ? a[2] : a[0], x1 = b1 ? a[3] : a[1];
    const float y0 = b1 ? a[0] : a[2], y1 = b1 ? a[1] : a[3];
    x0 += dpp<0x4E>(y0);                                     // quad_perm [2,3,0,1]: lane ^ 2
    x1 += dpp<0x4E>(y1);
    float x = b0 ? x1 : x0;
    const float y = b0 ? x0 : x1;
    x += dpp<0xB1>(y);                                       // quad_perm [1,0,3,2]: lane ^ 1
    return x;
}

// The tiled backward specialised for the common regime (chosen by the host): soft taps of
// a uniform half-width s (KF >= ceil(2s) lags of non-zero weight, one history word), the
// ATan surrogate, decay charge, hard reset to 0, reset not detached.
//
// Per step: the W^T-tile contraction and row butterfly, then straight-line lane work:
// the future-gradient taps read KF consecutive ring slots from one address (the ring
// keeps a mirror of its first KF - 1 slots after its end, so a run of taps never wraps),
// the LIF backward without mode switches (the surrogate takes a hardware reciprocal:
// 1-2 ulp), and unconditional buffer loads / stores (lanes without a source and steps
// outside [0, T) address past the buffer end), so the compiler's counts of outstanding
// memory operations are exact and a prefetched value never waits on later stores.
constexpr int kPrefetchBwdFast = 4;

template <int RI, int NJ, int CJ, int KF>
__global__ void __launch_bounds__(TiledThreads<RI>::value) axonal_bwd_tiled_fast(AxBwd p) {
    extern __shared__ float smem[];
    constexpr int CJP = CJ + 4;
    const int N = p.N, T = p.T, B = p.B, NZ = p.NZ, R = p.R, NP = p.NP;
    float* grbuf = smem;                 // [2][NZ]
    float* ring = smem + 2 * NZ;         // [R + KF - 1][NP]: slot (time mod R), mirrored
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int grp = tid / NJ, jcg = tid - (tid / NJ) * NJ;

    float w[RI][CJ];
    load_w_tile<RI, CJ>(w, p.W, p.w_bf16, N, [&](int a, int cc, int& i, int& j) {
        j = grp * RI + a;
        i = jcg * CJ + cc;
    });

    const bool nl = jcg < RI && grp * RI + jcg < N;
    const int j = nl ? grp * RI + jcg : 0;
    OneHot<RI> sel;
    sel.init(jcg % RI);
    const float c = 1.0f + p.d[j];
    const float s = p.s_uniform;
    const float s2 = s * s;
    const int lof = max(1, (int)floorf(c - s) + 1);
    float wq[KF];
#pragma unroll
    for (int q = 0; q < KF; ++q) {
        const int lq = lof + q;
        wq[q] = lq <= p.L - 1 ? tri_weight((float)lq, c, s, s2) : 0.0f;
    }
    const float m = p.drop ? p.drop[(size_t)b * N + j] : 1.0f;
    const float decay = p.lif.decay, vth = p.lif.vth;
    const float half_alpha = 0.5f * p.lif.alpha, za = 1.5707963267948966f * p.lif.alpha;

    for (int q = tid; q < 2 * NZ + (R + KF - 1) * NP; q += blockDim.x) smem[q] = 0.0f;
    __syncthreads();

    const size_t BN = (size_t)B * N;
    const uint32_t row_bytes = (uint32_t)BN * 4u;
    const int voff = (b * N + j) * 4;
    const int soff = nl ? voff : kOutOfRange;
    float* const grout = p.gr;

    float gq[kPrefetchBwdFast], uq[kPrefetchBwdFast];
#pragma unroll
    for (int q = 0; q < kPrefetchBwdFast; ++q) {
        const int tt = T - 1 - q;
        const uint32_t nb = tt >= 0 ? row_bytes : 0u;
        gq[q] = raw_buffer_load_f32(buffer_rsrc(p.gy + (size_t)max(tt, 0) * BN, nb), voff, 0, 0);
        uq[q] = raw_buffer_load_f32(buffer_rsrc(p.u + (size_t)max(tt, 0) * BN, nb), voff, 0, 0);
    }
    float lam = 0.0f, db_acc = 0.0f;

    auto contract = [&](int buf) {
        const float4* g4 = reinterpret_cast<const float4*>(grbuf + buf * NZ + jcg * CJP);
        float acc[RI];
#pragma unroll
        for (int a = 0; a < RI; ++a) acc[a] = 0.0f;
#pragma unroll
        for (int q = 0; q < CJ / 4; ++q) {
            const float4 gg = g4[q];
#pragma unroll
            for (int a = 0; a < RI; ++a) {
                acc[a] = fmaf(w[a][4 * q + 0], gg.x, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 1], gg.y, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 2], gg.z, acc[a]);
                acc[a] = fmaf(w[a][4 * q + 3], gg.w, acc[a]);
            }
        }
        if constexpr (RI == 4 && NJ == 8) {
            return reduce_scatter_4x8(acc, (jcg & 2) != 0, (jcg & 1) != 0);
        } else {
#pragma unroll
            for (int a = 0; a < RI; ++a) acc[a] = group_sum_t<NJ>(acc[a]);
            return sel.pick(acc);
        }
    };

    // byte addresses walked backwards in time: gz of step t + 1, dx and gr of step t, and
    // the prefetch of gy / u at step t - P
    const uint64_t step_b = (uint64_t)row_bytes;
    uint64_t gza = (uint64_t)p.gz + (uint64_t)T * step_b, dxa = (uint64_t)p.dx + (uint64_t)(T - 1) * step_b;
    uint64_t gra = (uint64_t)grout + (uint64_t)(T - 1) * step_b;
    const int tp0 = T - 1 - kPrefetchBwdFast;
    uint64_t gya = (uint64_t)p.gy + (uint64_t)max(tp0, 0) * step_b, uau = (uint64_t)p.u + (uint64_t)max(tp0, 0) * step_b;
    const uint32_t grbytes = grout ? row_bytes : 0u;
    // byte address of ring slot (t + lof) mod R in this lane's column, for the current t
    const int slot_bytes = NP * 4;
    int tn1 = T % R;                                   // slot of time t + 1
    int tap = (T - 1 + lof) % R * slot_bytes + j * 4;  // slot of time t + lof, t = T - 1

    auto step = [&](const int t, float& gs, float& us) {
        // taps of the future gradient, times t + lof + q (slots of times >= T hold 0), read
        // before the contraction: they are this lane's own slots of earlier steps, except the
        // first tap of a lag-1 source, time t + 1, which is gz(t+1) itself (with R >= L + 8
        // ring slots no other tap reaches the slot written in this step)
        const float* rp = reinterpret_cast<const float*>(reinterpret_cast<const char*>(ring) + tap);
        float rq[KF];
#pragma unroll
        for (int q = 0; q < KF; ++q) rq[q] = rp[q * NP];
        const float gz1 = contract((t + 1) & 1);       // gz(t+1); gr(T) = 0
        const int tm = tn1 == 0 ? R - 1 : tn1 - 1;     // slot of time t
        // publish gz(t+1) in its slot (and the mirror) and for the delay-gradient pass
        if (nl) {
            ring[tn1 * NP + j] = gz1;
            if (tn1 < KF - 1) ring[(tn1 + R) * NP + j] = gz1;
        }
        raw_buffer_store_f32(gz1, step_rsrc(gza, t + 1 < T ? row_bytes : 0u), soff, 0, 0);
        gza -= step_b;
        rq[0] = lof == 1 ? gz1 : rq[0];
        float gfut = 0.0f;
#pragma unroll
        for (int q = 0; q < KF; ++q) gfut = fmaf(wq[q], rq[q], gfut);
        // LIF backward (hard reset to 0, ATan surrogate, reset not detached)
        const float u = us;
        const float y = (u - vth >= 0.0f) ? 1.0f : 0.0f;
        const float gY = gs + gfut;
        const float zz = za * (u - vth);
        const float sg = half_alpha * __builtin_amdgcn_rcpf(1.0f + zz * zz);
        const float gS = gY - lam * u;
        const float du = lam * (1.0f - y) + gS * sg;
        lam = decay * du;
        const float gr = du * m;
        // steps t < 0 (the tail of the last group) contribute nothing and must not
        // overwrite gr(0), which the final contraction reads
        db_acc += t >= 0 ? gr : 0.0f;
        if (nl && t >= 0) grbuf[(t & 1) * NZ + zpos<CJ>(j)] = gr;   // LDS only: no memory counter
        const bool live = t >= 0;
        raw_buffer_store_f32(du, step_rsrc(dxa, live ? row_bytes : 0u), soff, 0, 0);
        raw_buffer_store_f32(gr, step_rsrc(gra, live ? grbytes : 0u), soff, 0, 0);
        dxa -= step_b;
        gra -= step_b;
        // refill the prefetch slots with step t - P (after their values are used); the
        // addresses stop at step 0 (those loads return 0)
        const int tp = t - kPrefetchBwdFast;
        const uint32_t nb = tp >= 0 ? row_bytes : 0u;
        gs = raw_buffer_load_f32(step_rsrc(gya, nb), voff, 0, 0);
        us = raw_buffer_load_f32(step_rsrc(uau, nb), voff, 0, 0);
        if (tp > 0) {
            gya -= step_b;
            uau -= step_b;
        }
        barrier_lds();
        tn1 = tm;
        tap -= slot_bytes;
        if (tap < j * 4) tap += R * slot_bytes;
    };

    // steps T-1, T-2, ... in whole groups of P (a step t < 0 stores nothing)
    for (int t0 = T - 1; t0 >= 0; t0 -= kPrefetchBwdFast) {
#pragma unroll
        for (int q = 0; q < kPrefetchBwdFast; ++q) step(t0 - q, gq[q], uq[q]);
    }
    const float gz0 = contract(0);                     // gz(0)
    if (nl) {
        p.gz[(size_t)b * N + j] = gz0;
        p.part[(size_t)0 * B * N + (size_t)b * N + j] = db_acc;
    }
}

// Delay / half-width gradient partials after the tiled scan, per (b, j):
//   dd_j += sum_t gz_j(t) sum_l dh/dd(l) y_j(t - l)   (soft: the closed-form triangle
//   derivative / s^2; straight: y(t - lag - 1) - y(t - lag)),  ds_j likewise with dh/ds.
// The sequence is cut into 32-step segments; a thread handles one segment at a time: it
// first pushes the 64*HW spikes before its segment into a History register (as the
// forward does), loads its 32 gz values together, then walks the segment. Block (64 j,
// kDelayY segment lanes) of one batch row: the segment lanes' sums are added in a fixed
// order through LDS, and the per-row partials part[1][b][j] (dd), part[2][b][j] (ds) are
// summed over the batch by reduce_rows together with the scan's db partials.
constexpr int kDelaySeg = 32;
constexpr int kDelayY = 4;

__host__ __device__ int axonal_delay_segments(int T) { return (T + kDelaySeg - 1) / kDelaySeg; }

// Block (bx, b): sources 64 bx .. 64 bx + 63 of batch row b; thread (tx, ty) of 64 x kDelayY.
template <int HW>
__device__ __forceinline__ void axonal_delay_grad_block(const AxBwd& p, int bx, int b, int tx, int ty,
                                                        float (&red)[2][kDelayY][64]) {
    const int N = p.N, T = p.T, B = p.B;
    const size_t BN = (size_t)B * N;
    const int S = axonal_delay_segments(T);
    const int jr = bx * 64 + tx;
    const bool act = jr < N;
    const int j = act ? jr : 0;
    const size_t rem = (size_t)b * N + j;
    const float c = 1.0f + p.d[j];
    const float s = p.s ? p.s[j] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int nt = hi - lo + 1;
    const bool soft = p.mode == DELREC_BWD_SOFT;
    const bool need_ds = p.s != nullptr;
    const bool fast = soft && !need_ds && nt <= kMaxTaps && HW == 1;
    const int lag = p.lag ? p.lag[j] : 1;
    float dsg[kMaxTaps];
#pragma unroll
    for (int k = 0; k < kMaxTaps; ++k) dsg[k] = (k < nt) ? tri_dsign((float)(lo + k), c, s) : 0.0f;
    const int TW = (T + 31) >> 5;
    const uint32_t* col = p.bits + (size_t)b * TW * N + j;

    float dd = 0.0f, ds = 0.0f;
    for (int seg = ty; seg < S; seg += kDelayY) {
        const int t0 = seg * kDelaySeg;
        float gzq[kDelaySeg];
#pragma unroll
        for (int e = 0; e < kDelaySeg; ++e)
            gzq[e] = (t0 + e < T) ? p.gz[(size_t)(t0 + e) * BN + rem] : 0.0f;

        // bit(l) = y(t0 - l): word w of the row holds steps 32w .. 32w + 31 (bit k = step
        // 32w + k), so lags 1..32 are the bit-reversed word seg - 1, lags 33..64 word seg - 2
        History<HW> past;
#pragma unroll
        for (int h = 0; h < HW; ++h) {
            const int w1 = seg - 2 * h - 1, w2 = seg - 2 * h - 2;
            const uint32_t a1 = w1 >= 0 ? col[(size_t)w1 * N] : 0u;
            const uint32_t a2 = w2 >= 0 ? col[(size_t)w2 * N] : 0u;
            past.w[h] = (uint64_t)__brev(a1) | ((uint64_t)__brev(a2) << 32);
        }
        const uint32_t word = col[(size_t)seg * N];                    // steps t0 .. t0 + 31

        float dds = 0.0f, dss = 0.0f;
#pragma unroll
        for (int e = 0; e < kDelaySeg; ++e) {
            if (t0 + e >= T) break;
            const float gz = gzq[e];
            if (fast) {
                const uint32_t ps = (uint32_t)(past.w[0] >> (lo - 1));
                float sd = 0.0f;
#pragma unroll
                for (int k = 0; k < kMaxTaps; ++k) sd += ((ps >> k) & 1u) ? dsg[k] : 0.0f;
                dds += gz * sd;
            } else if (soft) {
                float sd = 0.0f, sds = 0.0f;
                for (int l = lo; l <= hi; ++l) {
                    const float yv = past.bit(l);
                    sd += tri_dsign((float)l, c, s) * yv;
                    if (need_ds) sds += tri_ds((float)l, c, s, s2) * yv;
                }
                dds += gz * sd;
                dss += gz * sds;
            } else {
                dds += gz * (past.bit(lag + 1) - past.bit(lag));
            }
            past.push((word >> e) & 1u);
        }
        dd += soft ? dds / s2 : dds;
        ds += dss;
    }
    red[0][ty][tx] = dd;
    red[1][ty][tx] = ds;
    __syncthreads();
    if (ty == 0 && act) {
        float a0 = red[0][0][tx], a1 = red[1][0][tx];
#pragma unroll
        for (int y = 1; y < kDelayY; ++y) {
            a0 += red[0][y][tx];
            a1 += red[1][y][tx];
        }
        p.part[(size_t)1 * BN + rem] = a0;
        p.part[(size_t)2 * BN + rem] = a1;
    }
}

// Sum the per-row partials over the batch: out_k[j] = sum_b part[k][b][j]. Block (bx, kk) of
// threads (tx, ty) of CW x 16: CW consecutive neurons x 16 batch stripes, reduced through
// LDS in stripe order (the same sums for every CW).
template <int CW>
__device__ __forceinline__ void reduce_rows_block(const float* part, int B, int N, float* o0, float* o1,
                                                  float* o2, int bx, int kk, int tx, int ty,
                                                  float (&red)[16][CW + 1]) {
    float* out = kk == 0 ? o0 : (kk == 1 ? o1 : o2);
    if (!out) return;   // uniform over the block
    const int j = bx * CW + tx;
    const float* src = part + (size_t)kk * B * N;
    float acc = 0.0f;
    if (j < N) {
#pragma unroll 4
        for (int b = ty; b < B; b += 16) acc += src[(size_t)b * N + j];
    }
    red[ty][tx] = acc;
    __syncthreads();
    if (ty == 0 && j < N) {
        float t = 0.0f;
        for (int r = 0; r < 16; ++r) t += red[r][tx];
        out[j] = t;
    }
}

__global__ void __launch_bounds__(1024) reduce_rows_kernel(const float* part, int B, int N,
                                                           float* o0, float* o1, float* o2) {
    __shared__ float red[16][65];
    reduce_rows_block<64>(part, B, N, o0, o1, o2, blockIdx.x, blockIdx.y, threadIdx.x, threadIdx.y, red);
}

// The reductions after the axonal backward scan, as two launches on the caller's stream (no
// second stream: its fork and join cost more than the overlap they buy):
//   tail: blocks [0, ndw) the dW GEMM tiles (tile (ti, tj) of k chunk kz; the tiles of
//         one chunk on one XCD), then the delay / half-width gradient rows;
//   sums: blocks [0, nsum) the dW split-K sums, then the batch reductions of db, dd, ds
//         (16 neurons per block).
// Both job kinds of a launch only read what earlier launches wrote, so they run side by
// side; the longer dW blocks go first so that all of them start in the first round.
template <int HW>
__global__ void __launch_bounds__(kDwThreads, 2) axonal_bwd_tail_kernel(AxBwd p, AxTail q) {
    __shared__ DwStage sm;   // 48 KiB: one dW stage, or the delay blocks' 2 KiB of partials
    int bid = blockIdx.x;
    if (bid < q.ndw) {
        // the tiles of one k chunk read the same rows of both operands: with ks a multiple of
        // 8 they all go to one XCD (workgroup id mod 8), so the second reads hit its L2
        const int tt = q.tiles * q.tiles;
        int kz, r;
        if ((q.ks & 7) == 0) {
            const int slot = bid >> 3;
            kz = (slot / tt) * 8 + (bid & 7);
            r = slot % tt;
        } else {
            kz = bid / tt;
            r = bid - kz * tt;
        }
        dw_gemm_tile(q.A, q.Bz, q.K, p.N, q.kchunk, q.gpart, r % q.tiles, r / q.tiles, kz, sm);
        return;
    }
    bid -= q.ndw;
    axonal_delay_grad_block<HW>(p, bid % q.nbx, bid / q.nbx, threadIdx.x & 63, threadIdx.x >> 6,
                                *reinterpret_cast<float(*)[2][kDelayY][64]>(&sm));
}

__global__ void __launch_bounds__(kDwThreads) axonal_bwd_sums_kernel(AxTail q, const float* part, int B,
                                                                     int N) {
    __shared__ float4 sm[4][64];   // 4 KiB: the partial sums' wave totals, or the row stripes
    int bid = blockIdx.x;
    if (bid < q.nsum) {
        sum_partials_block(q.gpart, q.ks, (size_t)N * N, q.dW, bid, sm);
        return;
    }
    bid -= q.nsum;
    const int nb16 = (N + 15) / 16;
    reduce_rows_block<16>(part, B, N, q.o0, q.o1, q.o2, bid % nb16, bid / nb16, threadIdx.x & 15,
                          threadIdx.x >> 4, *reinterpret_cast<float(*)[16][17]>(&sm));
}

void launch_axonal_bwd_tail(const AxBwd& p, const AxTail& q, hipStream_t stream) {
    const int blocks = q.ndelay + q.ndw;
    if (blocks <= 0) return;
    const int lags = std::max(p.L - 1, 1);
    if (lags <= 64)
        hipLaunchKernelGGL(axonal_bwd_tail_kernel<1>, dim3(blocks), dim3(kDwThreads), 0, stream, p, q);
    else if (lags <= 128)
        hipLaunchKernelGGL(axonal_bwd_tail_kernel<2>, dim3(blocks), dim3(kDwThreads), 0, stream, p, q);
    else
        hipLaunchKernelGGL(axonal_bwd_tail_kernel<4>, dim3(blocks), dim3(kDwThreads), 0, stream, p, q);
}

void launch_axonal_bwd_sums(const AxTail& q, const float* part, int B, int N, hipStream_t stream) {
    const int blocks = q.nsum + 3 * ((N + 15) / 16);
    hipLaunchKernelGGL(axonal_bwd_sums_kernel, dim3(blocks), dim3(kDwThreads), 0, stream, q, part, B, N);
}

// ---------------------------------------------------------------------------------------
// Launchers.
#define DELREC_AX_CASE(CHV, RESV, HWV)                                                      \
    if (ch == CHV && res == RESV && hw == HWV) {                                            \
        if (fwd) {                                                                          \
            ensure_lds((const void*)axonal_fwd_kernel<CHV, RESV, HWV>, lds);        \
            hipLaunchKernelGGL((axonal_fwd_kernel<CHV, RESV, HWV>), dim3(grid), dim3(block), \
                               lds, stream, *fa);                                           \
        } else {                                                                            \
            ensure_lds((const void*)axonal_bwd_kernel<CHV, RESV, HWV>, lds);        \
            hipLaunchKernelGGL((axonal_bwd_kernel<CHV, RESV, HWV>), dim3(grid), dim3(block), \
                               lds, stream, *ba);                                           \
        }                                                                                   \
        return true;                                                                        \
    }

#define DELREC_AX_HW(CHV, RESV) DELREC_AX_CASE(CHV, RESV, 1) DELREC_AX_CASE(CHV, RESV, 2) \
    DELREC_AX_CASE(CHV, RESV, 4)

bool launch_axonal(bool fwd, const AxFwd* fa, const AxBwd* ba, int ch, bool res, int hw,
                   int grid, int block, size_t lds, hipStream_t stream) {
    DELREC_AX_HW(1, false)
    return false;
}

#define DELREC_AXT_CASE(RIV, NJV, HWV, CJV)                                                 \
    if (ri == RIV && nj == NJV && hw == HWV && cj == CJV) {                                  \
        if (fwd) {                                                                          \
            ensure_lds((const void*)axonal_fwd_tiled<RIV, NJV, HWV, CJV>, lds);              \
            hipLaunchKernelGGL((axonal_fwd_tiled<RIV, NJV, HWV, CJV>), dim3(grid), dim3(block), \
                               lds, stream, *fa);                                           \
        } else {                                                                            \
            ensure_lds((const void*)axonal_bwd_tiled<RIV, NJV, HWV, CJV>, lds);              \
            hipLaunchKernelGGL((axonal_bwd_tiled<RIV, NJV, HWV, CJV>), dim3(grid), dim3(block), \
                               lds, stream, *ba);                                           \
        }                                                                                   \
        return true;                                                                        \
    }
#define DELREC_AXT_HW(RIV, NJV, CJV) \
    DELREC_AXT_CASE(RIV, NJV, 1, CJV) DELREC_AXT_CASE(RIV, NJV, 2, CJV) DELREC_AXT_CASE(RIV, NJV, 4, CJV)

// (RI, NJ, CJ) triples chosen by the host layout for N <= 256
bool launch_axonal_tiled(bool fwd, const AxFwd* fa, const AxBwd* ba, int ri, int nj, int cj, int hw,
                         int grid, int block, size_t lds, hipStream_t stream) {
    DELREC_AXT_HW(1, 1, 16) DELREC_AXT_HW(1, 2, 16) DELREC_AXT_HW(1, 4, 16) DELREC_AXT_HW(1, 8, 16)
    DELREC_AXT_HW(2, 16, 16) DELREC_AXT_HW(4, 16, 16) DELREC_AXT_HW(8, 16, 16)
    DELREC_AXT_HW(4, 8, 32)
    return false;
}

#define DELREC_AXW_CASE(RIV, HWV)                                                         \
    if (ri == RIV && hw == HWV) {                                                           \
        ensure_lds((const void*)axonal_fwd_wave<RIV, HWV>, lds);                            \
        hipLaunchKernelGGL((axonal_fwd_wave<RIV, HWV>), dim3(grid), dim3(64 * nw), lds, stream, p); \
        return true;                                                                        \
    }

bool launch_axonal_fwd_wave_fast(const AxFwd& p, int ri, int kf, int nw, int grid, hipStream_t stream) {
    const size_t lds = (size_t)2 * 8 * 64 * ri * sizeof(float);
#define DELREC_AXWF_CASE(RIV, KFV)                                                          \
    if (ri == RIV && kf == KFV) {                                                           \
        ensure_lds((const void*)axonal_fwd_wave_fast<RIV, KFV>, lds);                       \
        hipLaunchKernelGGL((axonal_fwd_wave_fast<RIV, KFV>), dim3(grid), dim3(64 * nw), lds, stream, p); \
        return true;                                                                        \
    }
    DELREC_AXWF_CASE(1, 2) DELREC_AXWF_CASE(2, 2) DELREC_AXWF_CASE(4, 2)
    DELREC_AXWF_CASE(1, 4) DELREC_AXWF_CASE(2, 4) DELREC_AXWF_CASE(4, 4)
    DELREC_AXWF_CASE(1, 8) DELREC_AXWF_CASE(2, 8) DELREC_AXWF_CASE(4, 8)
    return false;
}

bool launch_axonal_fwd_wave(const AxFwd& p, int ri, int hw, int nw, int grid, size_t lds,
                            hipStream_t stream) {
    DELREC_AXW_CASE(1, 1) DELREC_AXW_CASE(1, 2) DELREC_AXW_CASE(1, 4)
    DELREC_AXW_CASE(2, 1) DELREC_AXW_CASE(2, 2) DELREC_AXW_CASE(2, 4)
    DELREC_AXW_CASE(4, 1) DELREC_AXW_CASE(4, 2) DELREC_AXW_CASE(4, 4)
    return false;
}

bool launch_axonal_bwd_tiled_fast(const AxBwd& p, int ri, int nj, int cj, int kf, int grid, int block,
                                  size_t lds, hipStream_t stream) {
#define DELREC_AXBF_CASE(RIV, NJV, CJV, KFV)                                                 \
    if (ri == RIV && nj == NJV && cj == CJV && kf == KFV) {                                  \
        ensure_lds((const void*)axonal_bwd_tiled_fast<RIV, NJV, CJV, KFV>, lds);            \
        hipLaunchKernelGGL((axonal_bwd_tiled_fast<RIV, NJV, CJV, KFV>), dim3(grid), dim3(block), lds, stream, p); \
        return true;                                                                         \
    }
#define DELREC_AXBF_KF(RIV, NJV, CJV) \
    DELREC_AXBF_CASE(RIV, NJV, CJV, 2) DELREC_AXBF_CASE(RIV, NJV, CJV, 4) DELREC_AXBF_CASE(RIV, NJV, CJV, 8)
    DELREC_AXBF_KF(1, 1, 16) DELREC_AXBF_KF(1, 2, 16) DELREC_AXBF_KF(1, 4, 16) DELREC_AXBF_KF(1, 8, 16)
    DELREC_AXBF_KF(2, 16, 16) DELREC_AXBF_KF(4, 16, 16) DELREC_AXBF_KF(8, 16, 16)
    DELREC_AXBF_KF(4, 8, 32)
    return false;
}

void launch_reduce_rows(const float* part, int B, int N, float* o0, float* o1, float* o2,
                        hipStream_t stream) {
    dim3 grid((N + 63) / 64, 3);
    hipLaunchKernelGGL(reduce_rows_kernel, grid, dim3(64, 16), 0, stream, part, B, N, o0, o1, o2);
}

}  // namespace delrec
