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
#include "common.h"
#include "kernels.h"

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

    // this neuron as a source of the delayed trace
    const float dval = p.d[ic];
    const float c = 1.0f + dval;
    const float s = p.s ? p.s[ic] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
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
    float xq0 = act ? p.x[row] : 0.0f;
    float xq1 = (act && T > 1) ? p.x[BN + row] : 0.0f;
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
        for (int msk = G >> 1; msk > 0; msk >>= 1) acc += wave_xor(acc, msk);

        const float xv = xq0;
        xq0 = xq1;
        if (act && t + 2 < T) xq1 = p.x[(size_t)(t + 2) * BN + row];

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
            const float zn = act ? axonal_trace<HW>(hist, p.taps, c, s, s2, lo, hi, lag, frac) : 0.0f;
            if (act && g == 0) {
                zbuf[((t + 1) & 1) * NZ + i] = zn;
                if (p.z) p.z[(size_t)(t + 1) * BN + row] = zn;
            }
        }
        __syncthreads();
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

    const float dval = p.d[jc];
    const float c = 1.0f + dval;
    const float s = p.s ? p.s[jc] : p.s_uniform;
    const float s2 = s * s;
    int lo, hi;
    tap_range(c, s, p.L, lo, hi);
    const int lag = p.lag ? p.lag[jc] : 1;
    const float m = p.drop ? p.drop[(size_t)b * N + jc] : 1.0f;

    for (int q = tid; q < 2 * NZ + R * NP; q += blockDim.x) smem[q] = 0.0f;
    __syncthreads();

    // past spikes of j relative to step t: bit(l) = y[t-l]; start at t = T-1
    History<HW> past;
    past.clear();
    for (int l = 64 * HW; l >= 1; --l) past.push(act ? spike_bit(p.bits, TW, N, b, T - 1 - l, jc) : 0u);

    const size_t BN = (size_t)B * N;
    const size_t rowj = (size_t)b * N + jc;
    float lam = 0.0f, db_acc = 0.0f, dd_acc = 0.0f, ds_acc = 0.0f;
    int tmod = (T - 1) % R;

    for (int t = T - 1; t >= 0; --t) {
        // future gradient through the delayed trace
        float gfut = 0.0f;
        if (p.mode == DELREC_BWD_SOFT) {
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
        const size_t o = (size_t)t * BN + rowj;
        const float gy = act ? p.gy[o] : 0.0f;
        const float u = act ? p.u[o] : 0.0f;
        const float y = lif_fire(k, u);
        const float du = lif_backward(k, gy + gfut, u, y, lam);
        lam = k.decay * du;
        const float da = lif_dx(k, du);       // dL/d(input of the charge)
        const float gr = da * m;
        if (act && g == 0) {
            p.dx[o] = da;
            if (p.gr) p.gr[o] = gr;
            grbuf[(t & 1) * NZ + j] = gr;
        }
        db_acc += gr;
        __syncthreads();

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
        for (int msk = G >> 1; msk > 0; msk >>= 1) acc += wave_xor(acc, msk);
        const float gz = acc;
        if (act) ring[tmod * NP + j] = gz;

        // delay / half-width gradients: dL/dh[j,l] = gz_t * y[t-l]
        if (p.mode == DELREC_BWD_SOFT) {
            float sd = 0.0f, sds = 0.0f;
            for (int l = lo; l <= hi; ++l) {
                const float yv = past.bit(l);
                sd += tri_dsign((float)l, c, s) * yv;
                sds += tri_ds((float)l, c, s, s2) * yv;
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
        p.part[(size_t)1 * B * N + rowj] = (p.mode == DELREC_BWD_SOFT) ? dd_acc / s2 : dd_acc;
        p.part[(size_t)2 * B * N + rowj] = ds_acc;
    }
}

// Sum the per-row partials over the batch: out_k[j] = sum_b part[k][b][j].
__global__ void reduce_rows_kernel(const float* part, int B, int N, float* o0, float* o1, float* o2) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int kk = blockIdx.y;
    if (j >= N) return;
    float* out = kk == 0 ? o0 : (kk == 1 ? o1 : o2);
    if (!out) return;
    const float* src = part + (size_t)kk * B * N;
    float acc = 0.0f;
    for (int b = 0; b < B; ++b) acc += src[(size_t)b * N + j];
    out[j] = acc;
}

// ---------------------------------------------------------------------------------------
// Launchers.
#define DELREC_AX_CASE(CHV, RESV, HWV)                                                      \
    if (ch == CHV && res == RESV && hw == HWV) {                                            \
        if (fwd) {                                                                          \
            (void)hipFuncSetAttribute((const void*)axonal_fwd_kernel<CHV, RESV, HWV>,             \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);      \
            hipLaunchKernelGGL((axonal_fwd_kernel<CHV, RESV, HWV>), dim3(grid), dim3(block), \
                               lds, stream, *fa);                                           \
        } else {                                                                            \
            (void)hipFuncSetAttribute((const void*)axonal_bwd_kernel<CHV, RESV, HWV>,             \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);      \
            hipLaunchKernelGGL((axonal_bwd_kernel<CHV, RESV, HWV>), dim3(grid), dim3(block), \
                               lds, stream, *ba);                                           \
        }                                                                                   \
        return true;                                                                        \
    }

#define DELREC_AX_HW(CHV, RESV) DELREC_AX_CASE(CHV, RESV, 1) DELREC_AX_CASE(CHV, RESV, 2) \
    DELREC_AX_CASE(CHV, RESV, 4)

bool launch_axonal(bool fwd, const AxFwd* fa, const AxBwd* ba, int ch, bool res, int hw,
                   int grid, int block, size_t lds, hipStream_t stream) {
    DELREC_AX_HW(4, true)
    DELREC_AX_HW(8, true)
    DELREC_AX_HW(16, true)
    DELREC_AX_HW(32, true)
    DELREC_AX_HW(64, true)
    DELREC_AX_HW(1, false)
    return false;
}

void launch_reduce_rows(const float* part, int B, int N, float* o0, float* o1, float* o2,
                        hipStream_t stream) {
    dim3 grid((N + 255) / 256, 3);
    hipLaunchKernelGGL(reduce_rows_kernel, grid, dim3(256), 0, stream, part, B, N, o0, o1, o2);
}

}  // namespace delrec
