// Synaptic / hybrid delayed-LIF recurrent scan for gfx950.
//
// Forward (event-driven): one workgroup per batch row; lane i owns receivers
// i, i + blockDim, ... and their column of a ring of pending recurrent input
// (ring[(t + l) mod R][i], R = L slots). Each step the fired sources are compacted with
// wave ballots + popcount prefix into an LDS list, then every lane scatters
// W[i,o] * h(l; d_io, s_o) for each fired source o into its own ring column: no atomics,
// no cross-lane hazards, two barriers per step (reference _ed_scatter_compact_kernel,
// synaptic_eventdriven.py:106-164, whose global-memory ring and .cg/volatile
// compaction this replaces). Hybrid delays are read as base[o] + offsets[i,o] (int8)
// instead of a materialised float (N, N) tensor.
//
// Backward (dense, reverse time): lane j owns sources; the future recurrent-input
// gradients gr[t + l, :] live in an LDS ring, and gfut_j = sum_i W[i,j] sum_l h(l; d_ij)
// gr[t+l, i] is gathered for every j (reference _ed_bwd_kernel,
// synaptic_eventdriven.py:323-364). The weight / delay gradients are then formed by the
// lag-correlation GEMM (gemm.hip).
#include "kernels.h"

namespace delrec {

__device__ __forceinline__ float syn_delay_t(const SynFwd& p, int o, int i) {
    if (p.dt) return p.dt[(size_t)o * p.N + i];
    return p.base[o] + 0.0f + 1.0f * (float)p.offt[(size_t)o * p.N + i];
}

__device__ __forceinline__ float syn_delay(const SynBwd& p, int i, int j) {
    if (p.d) return p.d[(size_t)i * p.N + j];
    return p.base[j] + 0.0f + 1.0f * (float)p.off[(size_t)i * p.N + j];
}

template <int NPT>
__global__ void __launch_bounds__(1024) syn_fwd_kernel(SynFwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B, R = p.R, NP = p.NP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = BS >> 6;
    const bool lds_ring = p.gring == nullptr;
    float* ring = lds_ring ? smem : p.gring + (size_t)b * R * N;
    const int pitch = lds_ring ? NP : N;
    int* fired = reinterpret_cast<int*>(smem + (lds_ring ? (size_t)R * NP : 0));
    int* wcnt = fired + p.NF;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;
    const size_t BN = (size_t)B * N;

    int idx[NPT];
    bool act[NPT];
    float v[NPT], m[NPT], bias[NPT], xq0[NPT], xq1[NPT];
    uint32_t word[NPT];
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
        idx[q] = tid + q * BS;
        act[q] = idx[q] < N;
        const int ic = act[q] ? idx[q] : 0;
        v[q] = k.v0;
        m[q] = p.drop ? p.drop[(size_t)b * N + ic] : 1.0f;
        bias[q] = p.bias ? p.bias[ic] : 0.0f;
        const size_t row = (size_t)b * N + ic;
        xq0[q] = act[q] ? p.x[row] : 0.0f;
        xq1[q] = (act[q] && T > 1) ? p.x[BN + row] : 0.0f;
        word[q] = 0;
        for (int r = 0; r < R; ++r)
            if (act[q]) ring[(size_t)r * pitch + idx[q]] = 0.0f;
    }
    __syncthreads();

    int tmod = 0;
    for (int t = 0; t < T; ++t) {
        uint64_t bal[NPT];
#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            float rec = 0.0f;
            if (act[q]) {
                float* cell = ring + (size_t)tmod * pitch + idx[q];
                rec = *cell;
                *cell = 0.0f;
            }
            const float xv = xq0[q];
            xq0[q] = xq1[q];
            const size_t row = (size_t)b * N + (act[q] ? idx[q] : 0);
            if (act[q] && t + 2 < T) xq1[q] = p.x[(size_t)(t + 2) * BN + row];
            const float r = rec + bias[q];
            const float a = xv + r * m[q];
            const float u = lif_charge(k, v[q], a);
            const float y = act[q] ? lif_fire(k, u) : 0.0f;
            v[q] = lif_reset(k, u, y);
            const uint32_t yb = y != 0.0f ? 1u : 0u;
            word[q] |= yb << (t & 31);
            if (act[q]) {
                const size_t o = (size_t)t * BN + row;
                p.y[o] = y;
                p.u[o] = u;
                if ((t & 31) == 31 || t == T - 1) p.bits[((size_t)b * TW + (t >> 5)) * N + idx[q]] = word[q];
            }
            if ((t & 31) == 31) word[q] = 0;
            bal[q] = __ballot(yb != 0u);
            if (lane == 0) wcnt[q * nwaves + wave] = __popcll(bal[q]);
        }
        __syncthreads();
        int nf = 0;
        for (int sgi = 0; sgi < NPT * nwaves; ++sgi) nf += wcnt[sgi];
#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            if (bal[q] >> lane & 1ull) {
                int off = 0;
                for (int sgi = 0; sgi < q * nwaves + wave; ++sgi) off += wcnt[sgi];
                off += __popcll(bal[q] & ((1ull << lane) - 1ull));
                fired[off] = idx[q];
            }
        }
        __syncthreads();
        // scatter the fired sources into the ring (lags >= 1: slot (t + l) mod R)
        for (int f = 0; f < nf; ++f) {
            const int o = fired[f];
            const float so = p.s ? p.s[o] : p.s_uniform;
            const float s2 = so * so;
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                if (!act[q]) continue;
                const int i = idx[q];
                const float w = load_w(p.Wt, p.w_bf16, (size_t)o * N + i);
                const float c = 1.0f + syn_delay_t(p, o, i);
                int lo, hi;
                tap_range(c, so, p.L, lo, hi);
                for (int l = lo; l <= hi; ++l) {
                    const float h = tri_weight((float)l, c, so, s2);
                    if (h == 0.0f) continue;
                    int slot = tmod + l;
                    if (slot >= R) slot -= R;
                    float* cell = ring + (size_t)slot * pitch + i;
                    *cell = *cell + w * h;
                }
            }
        }
        tmod = tmod + 1 == R ? 0 : tmod + 1;
    }
}

template <int NPT>
__global__ void __launch_bounds__(1024) syn_bwd_kernel(SynBwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B, R = p.R, NP = p.NP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    const bool lds_ring = p.gring == nullptr;
    float* ring = lds_ring ? smem : p.gring + (size_t)b * R * N;
    const int pitch = lds_ring ? NP : N;
    const Lif k = p.lif;
    const size_t BN = (size_t)B * N;

    int idx[NPT];
    bool act[NPT];
    float lam[NPT], m[NPT], s[NPT], dbacc[NPT];
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
        idx[q] = tid + q * BS;
        act[q] = idx[q] < N;
        const int jc = act[q] ? idx[q] : 0;
        lam[q] = 0.0f;
        dbacc[q] = 0.0f;
        m[q] = p.drop ? p.drop[(size_t)b * N + jc] : 1.0f;
        s[q] = p.s ? p.s[jc] : p.s_uniform;
        for (int r = 0; r < R; ++r)
            if (act[q]) ring[(size_t)r * pitch + idx[q]] = 0.0f;
    }
    __syncthreads();

    int tmod = (T - 1) % R;
    for (int t = T - 1; t >= 0; --t) {
        float gf[NPT];
#pragma unroll
        for (int q = 0; q < NPT; ++q) gf[q] = 0.0f;
        for (int i = 0; i < N; ++i) {
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                if (!act[q]) continue;
                const int j = idx[q];
                const float w = load_w(p.W, p.w_bf16, (size_t)i * N + j);
                const float c = 1.0f + syn_delay(p, i, j);
                const float sv = s[q], s2 = sv * sv;
                int lo, hi;
                tap_range(c, sv, p.L, lo, hi);
                float acc = 0.0f;
                for (int l = lo; l <= hi && t + l < T; ++l) {
                    int slot = tmod + l;
                    if (slot >= R) slot -= R;
                    acc += tri_weight((float)l, c, sv, s2) * ring[(size_t)slot * pitch + i];
                }
                gf[q] = fmaf(w, acc, gf[q]);
            }
        }
#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            if (!act[q]) continue;
            const int j = idx[q];
            const size_t o = (size_t)t * BN + (size_t)b * N + j;
            const float u = p.u[o];
            const float y = lif_fire(k, u);
            const float du = lif_backward(k, p.gy[o] + gf[q], u, y, lam[q]);
            lam[q] = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * m[q];
            p.dx[o] = da;
            p.gr[o] = gr;
            dbacc[q] += gr;
            ring[(size_t)tmod * pitch + j] = gr;
        }
        __syncthreads();
        tmod = tmod == 0 ? R - 1 : tmod - 1;
    }
#pragma unroll
    for (int q = 0; q < NPT; ++q)
        if (act[q]) p.part[(size_t)b * N + idx[q]] = dbacc[q];
}

void launch_syn_fwd(const SynFwd& a, int block, size_t lds, hipStream_t stream) {
    const int npt = (a.N + block - 1) / block;
    if (npt == 1) {
        (void)hipFuncSetAttribute((const void*)syn_fwd_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_fwd_kernel<1>, dim3(a.B), dim3(block), lds, stream, a);
    } else if (npt == 2) {
        (void)hipFuncSetAttribute((const void*)syn_fwd_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_fwd_kernel<2>, dim3(a.B), dim3(block), lds, stream, a);
    } else {
        (void)hipFuncSetAttribute((const void*)syn_fwd_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_fwd_kernel<4>, dim3(a.B), dim3(block), lds, stream, a);
    }
}

void launch_syn_bwd(const SynBwd& a, int block, size_t lds, hipStream_t stream) {
    const int npt = (a.N + block - 1) / block;
    if (npt == 1) {
        (void)hipFuncSetAttribute((const void*)syn_bwd_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_bwd_kernel<1>, dim3(a.B), dim3(block), lds, stream, a);
    } else if (npt == 2) {
        (void)hipFuncSetAttribute((const void*)syn_bwd_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_bwd_kernel<2>, dim3(a.B), dim3(block), lds, stream, a);
    } else {
        (void)hipFuncSetAttribute((const void*)syn_bwd_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipLaunchKernelGGL(syn_bwd_kernel<4>, dim3(a.B), dim3(block), lds, stream, a);
    }
}

// ---------------------------------------------------------------------------------------
// Plain multi-step LIF layer: one lane per (b, n), sequential over t.
__global__ void lif_fwd_kernel(delrec_lif_fwd_args a, Lif k) {
    const size_t BN = (size_t)a.B * a.N;
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= BN) return;
    float v = k.v0;
    for (int t = 0; t < a.T; ++t) {
        const size_t o = (size_t)t * BN + e;
        const float u = lif_charge(k, v, a.x[o]);
        const float y = lif_fire(k, u);
        v = lif_reset(k, u, y);
        a.y[o] = y;
        a.u[o] = u;
    }
}

__global__ void lif_bwd_kernel(delrec_lif_bwd_args a, Lif k) {
    const size_t BN = (size_t)a.B * a.N;
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= BN) return;
    float lam = 0.0f;
    for (int t = a.T - 1; t >= 0; --t) {
        const size_t o = (size_t)t * BN + e;
        const float u = a.u[o];
        const float du = lif_backward(k, a.gy[o], u, lif_fire(k, u), lam);
        lam = k.decay * du;
        a.dx[o] = lif_dx(k, du);
    }
}

void launch_lif(bool fwd, const delrec_lif_fwd_args* fa, const delrec_lif_bwd_args* ba,
                const Lif& k, hipStream_t stream) {
    const size_t BN = fwd ? (size_t)fa->B * fa->N : (size_t)ba->B * ba->N;
    const unsigned blocks = (unsigned)((BN + 255) / 256);
    if (fwd) hipLaunchKernelGGL(lif_fwd_kernel, dim3(blocks), dim3(256), 0, stream, *fa, k);
    else hipLaunchKernelGGL(lif_bwd_kernel, dim3(blocks), dim3(256), 0, stream, *ba, k);
}

}  // namespace delrec
