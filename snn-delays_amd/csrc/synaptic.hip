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
// Backward (dense, reverse time): lane j owns sources and gathers
// gfut_j = sum_i W[i,j] sum_l h(l; d_ij) gr[t+l, i] from a source-major ring of future
// recurrent-input gradients (reference _ed_bwd_kernel, synaptic_eventdriven.py:323-364).
// The weight / delay gradients are then formed by the lag-correlation GEMM (lagmm.hip).
#include <type_traits>

#include "kernels.h"

namespace delrec {

__device__ __forceinline__ float syn_delay_t(const SynFwd& p, int o, int i) {
    if (p.dt) return p.dt[(size_t)o * p.N + i];
    return p.base[o] + 0.0f + 1.0f * (float)p.offt[(size_t)o * p.N + i];
}

template <int NPT, bool GRING>
__global__ void __launch_bounds__(1024) syn_fwd_kernel(SynFwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B, R = p.R, NP = p.NP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = BS >> 6;
    float* ring = GRING ? p.gring + (size_t)b * R * N : smem;
    const int pitch = GRING ? N : NP;
    int* fired = reinterpret_cast<int*>(smem + (GRING ? 0 : (size_t)R * NP));
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

    // the per-connection data of a fired source o for this lane's receivers
    auto load_src = [&](int o, float (&w)[NPT], float (&dl)[NPT]) {
#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            const int i = act[q] ? idx[q] : 0;
            w[q] = load_w(p.Wt, p.w_bf16, (size_t)o * N + i);
            dl[q] = p.dt ? p.dt[(size_t)o * N + i]
                         : p.base[o] + 0.0f + 1.0f * (float)p.offt[(size_t)o * N + i];
        }
    };

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
        // scatter the fired sources into the ring (lags >= 1: slot (t + l) mod R); the next
        // source's weights and delays load while this one is scattered, and the taps of a
        // source are read and written four at a time
        float wn[NPT], dn[NPT];
        int on = 0;
        if (nf > 0) {
            on = fired[0];
            load_src(on, wn, dn);
        }
        for (int f = 0; f < nf; ++f) {
            const int o = on;
            float w[NPT], dl[NPT];
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                w[q] = wn[q];
                dl[q] = dn[q];
            }
            if (f + 1 < nf) {
                on = fired[f + 1];
                load_src(on, wn, dn);
            }
            const float so = p.s ? p.s[o] : p.s_uniform;
            const float is2 = 1.0f / (so * so);
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                if (!act[q]) continue;
                const int i = idx[q];
                const float c = 1.0f + dl[q];
                int lo, hi;
                tap_range(c, so, p.L, lo, hi);
                const float wq = w[q] * is2;
                for (int l0 = lo; l0 <= hi; l0 += 4) {
                    float* cell[4];
                    float old[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        int slot = tmod + min(l0 + e, hi);
                        slot = slot >= R ? slot - R : slot;
                        cell[e] = ring + (size_t)slot * pitch + i;
                        old[e] = *cell[e];
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int l = l0 + e;
                        if (l <= hi) *cell[e] = old[e] + wq * fmaxf(so - fabsf((float)l - c), 0.0f);
                    }
                }
            }
        }
        tmod = tmod + 1 == R ? 0 : tmod + 1;
    }
}

// Event-driven forward with the ring in LDS, one receiver per lane (N <= 1024), at most
// KF lags of non-zero weight per connection (KF >= ceil(2 s_max)).
//
// Per step: the LIF of every receiver (its recurrent input waits in its own ring column),
// then each wave writes the receivers that fired into its own segment of a double-buffered
// LDS list: one barrier per step. Lane k of every wave then finds the k-th fired source
// of the flattened list (wave segments in order) and holds its index, so the sources are
// walked in a fixed order with readlane. The walk goes in chunks of 8 sources: the weight
// and delay (or offset) of the next chunk's sources are loaded while the current chunk is
// scattered, through buffer descriptors whose base is the source's column of W^T / d^T
// (SGPRs), so a load costs no address arithmetic. Each lane adds
// W[i,o] / s_o^2 * max(0, s_o - |l - c_io|) at lags l = lof .. lof + KF - 1 (lof the first
// lag of non-zero weight, >= 1) into its own ring column: no atomics, no hazards between
// lanes. x is prefetched 8 steps ahead in fixed registers and every global load / store
// of a step is unconditional (inactive lanes address past the buffer end).
constexpr int kScatterChunk = 8;
constexpr int kPrefetchSynBwd = 4;   // steps of gy / u loaded ahead (hybrid backward)
constexpr int kScatterPrefetch = 8;

template <int KF, bool HYB, bool WBF>
__global__ void __launch_bounds__(1024) syn_fwd_scatter(SynFwd p) {
    extern __shared__ float smem[];
    constexpr bool PACKED = HYB && WBF;
    const int N = p.N, T = p.T, B = p.B, R = p.R, NP = p.NP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = BS >> 6;
    float* ring = smem;                                               // [R][NP]
    float4* srcl = reinterpret_cast<float4*>(smem + (size_t)R * NP);  // [N] base, s, 1/s^2
    float* dummy = reinterpret_cast<float*>(srcl + N);                // [64] writes of lanes past N
    int* seg = reinterpret_cast<int*>(dummy + 64);                    // [2][nwaves][64]
    int* cnt = seg + 2 * nwaves * 64;                                  // [2][nwaves]
    const int TW = (T + 31) >> 5;
    const size_t BN = (size_t)B * N;
    const bool act = tid < N;
    const int i = act ? tid : 0;
    const float vth = p.lif.vth;
    const Lif k = p.lif;
    const float m = p.drop ? p.drop[(size_t)b * N + i] : 1.0f;
    const float bias = p.bias ? p.bias[i] : 0.0f;

    // the lane's ring column (lanes past N write a private dummy cell: no branches, no
    // access to another receiver's column)
    float* const colp = act ? ring + tid : dummy + lane;
    const int cst = act ? NP : 0;
    for (int r = 0; r < R; ++r) colp[r * cst] = 0.0f;
    for (int q = tid; q < N; q += BS) {
        const float sq = p.s ? p.s[q] : p.s_uniform;
        srcl[q] = make_float4(HYB ? p.base[q] : 0.0f, sq, 1.0f / (sq * sq), 0.0f);
    }
    __syncthreads();

    const uint32_t row_bytes = (uint32_t)BN * 4u;
    const uint64_t step_b = (uint64_t)row_bytes;
    const int voff = (b * N + i) * 4;
    const int soff = act ? voff : kOutOfRange;
    const int boff = act ? (b * TW * N + i) * 4 : kOutOfRange;
    uint64_t xa = (uint64_t)p.x + (uint64_t)kScatterPrefetch * step_b;
    uint64_t ya = (uint64_t)p.y, ua = (uint64_t)p.u;
    float xq[kScatterPrefetch];
#pragma unroll
    for (int q = 0; q < kScatterPrefetch; ++q)
        xq[q] = raw_buffer_load_f32(step_rsrc((uint64_t)p.x + (uint64_t)q * step_b, q < T ? row_bytes : 0u), voff, 0, 0);

    // one descriptor per matrix; source o's column starts o * N elements in; a lane past N
    // reads beyond the matrix (0)
    const uint32_t nn = (uint32_t)N * (uint32_t)N;
    const i32x4 rw = buffer_rsrc(PACKED ? (const void*)p.wpk : p.Wt, nn * (PACKED ? 4u : (WBF ? 2u : 4u)));
    const i32x4 rd = buffer_rsrc(HYB ? (const void*)p.offt : (const void*)p.dt, nn * (HYB ? 1u : 4u));
    const int wsz = PACKED ? 4 : (WBF ? 2 : 4), dsz = HYB ? 1 : 4;
    const int wio = act ? i * wsz : 0x40000000, dio = act ? i * dsz : 0x40000000;
    // a source's weight and delay (or offset) as loaded, decoded only where they are used:
    // a decode right after the load would make the prefetch wait for it
    auto load_src = [&](int o, uint32_t& w, uint32_t& dl) {
        if constexpr (PACKED) {
            w = __float_as_uint(raw_buffer_load_f32(rw, wio + o * N * 4, 0, 0));
            dl = 0u;
        } else {
            if constexpr (WBF) w = (uint32_t)raw_buffer_load_u16(rw, wio + o * N * 2, 0, 0);
            else w = __float_as_uint(raw_buffer_load_f32(rw, wio + o * N * 4, 0, 0));
            if constexpr (HYB) dl = (uint32_t)(int32_t)raw_buffer_load_i8(rd, dio + o * N, 0, 0);
            else dl = __float_as_uint(raw_buffer_load_f32(rd, dio + o * N * 4, 0, 0));
        }
    };
    auto decode_src = [&](uint32_t w, uint32_t dl, float& wf, float& df) {
        if constexpr (PACKED) {
            wf = __uint_as_float(w & 0xFFFF0000u);
            df = (float)(int8_t)(w & 0xFFu);
        } else {
            wf = WBF ? __uint_as_float(w << 16) : __uint_as_float(w);
            df = HYB ? (float)(int32_t)dl : __uint_as_float(dl);
        }
    };

    float v = k.v0;
    uint32_t word = 0;
    int tmod = 0;
    auto step = [&](const int t, float& xs) {
        // LIF of this receiver: its recurrent input for step t waits in ring slot tmod
        float* cell = colp + tmod * cst;
        const float rec = *cell;
        *cell = 0.0f;
        const float r = rec + bias;
        const float a = xs + r * m;
        const float u = lif_charge(k, v, a);
        const bool fire = act && (u - vth >= 0.0f);
        v = lif_reset(k, u, fire ? 1.0f : 0.0f);
        word |= (fire ? 1u : 0u) << (t & 31);
        const bool live = t < T;
        raw_buffer_store_f32(fire ? 1.0f : 0.0f, step_rsrc(ya, live ? row_bytes : 0u), soff, 0, 0);
        raw_buffer_store_f32(u, step_rsrc(ua, live ? row_bytes : 0u), soff, 0, 0);
        const bool flush = ((t & 31) == 31 || t == T - 1) && live;
        raw_buffer_store_f32(__uint_as_float(word), step_rsrc((uint64_t)p.bits + (uint64_t)(t >> 5) * N * 4u,
                                                            flush ? (uint32_t)((size_t)B * TW * N * 4u) : 0u),
                             boff, 0, 0);
        if ((t & 31) == 31) word = 0;
        ya += step_b;
        ua += step_b;
        const int tn = t + kScatterPrefetch;
        xs = raw_buffer_load_f32(step_rsrc(xa, tn < T ? row_bytes : 0u), voff, 0, 0);
        xa += step_b;

        // fired receivers of this wave into its segment (buffer t & 1)
        const int bsel = t & 1;
        const uint64_t bal = __ballot(fire && live);
        if (fire && live) seg[(bsel * nwaves + wave) * 64 + __popcll(bal & ((1ull << lane) - 1ull))] = tid;
        if (lane == 0) cnt[bsel * nwaves + wave] = __popcll(bal);
        barrier_lds();

        // flattened list: lane q of every wave finds fired source number base + q
        int total = 0;
        int cw[16];
#pragma unroll
        for (int w2 = 0; w2 < 16; ++w2) {
            cw[w2] = w2 < nwaves ? cnt[bsel * nwaves + w2] : 0;
            total += cw[w2];
        }
        for (int base = 0; base < total; base += 64) {
            int src = 0;
            {
                int f = base + lane, acc = 0, sgi = 0, pos = 0;
                bool found = false;
#pragma unroll
                for (int w2 = 0; w2 < 16; ++w2) {
                    if (!found && f < acc + cw[w2]) {
                        sgi = w2;
                        pos = f - acc;
                        found = true;
                    }
                    acc += cw[w2];
                }
                src = found ? seg[(bsel * nwaves + sgi) * 64 + pos] : 0;
            }
            const int nf = min(64, total - base);
            // chunked walk: the next chunk's weights / delays load while this one scatters
            // (sources past nf read source 0: valid addresses, values unused; every load is
            // unconditional so the compiler's memory counts stay exact)
            uint32_t wn[kScatterChunk], dn[kScatterChunk];
#pragma unroll
            for (int e = 0; e < kScatterChunk; ++e) load_src(__builtin_amdgcn_readlane(src, e), wn[e], dn[e]);
            for (int f0 = 0; f0 < nf; f0 += kScatterChunk) {
                uint32_t wc[kScatterChunk], dc[kScatterChunk];
#pragma unroll
                for (int e = 0; e < kScatterChunk; ++e) {
                    wc[e] = wn[e];
                    dc[e] = dn[e];
                }
                if (f0 + kScatterChunk < nf) {
#pragma unroll
                    for (int e = 0; e < kScatterChunk; ++e)
                        load_src(__builtin_amdgcn_readlane(src, (f0 + kScatterChunk + e) & 63), wn[e], dn[e]);
                }
#pragma unroll
                for (int e = 0; e < kScatterChunk; ++e) {
                    if (f0 + e >= nf) break;
                    const int o = __builtin_amdgcn_readlane(src, (f0 + e) & 63);
                    const float4 sp = srcl[o];                 // base, s, 1/s^2
                    const float so = sp.y;
                    float wv, dv;
                    decode_src(wc[e], dc[e], wv, dv);
                    const float c = HYB ? 1.0f + (sp.x + 0.0f + 1.0f * dv) : 1.0f + dv;
                    const float wq = wv * sp.z;
                    // lags of non-zero weight: l > c - s, l >= 1; the ring slot of t + l
                    const int lof = max(1, (int)floorf(c - so) + 1);
                    int sl = tmod + lof;
                    sl = sl >= R ? sl - R : sl;
                    // the KF taps land in distinct slots (KF < R): read them all, then write
                    float* cp[KF];
                    float old[KF];
#pragma unroll
                    for (int q = 0; q < KF; ++q) {
                        cp[q] = colp + __umul24((uint32_t)sl, (uint32_t)cst);   // slot * pitch < 2^24
                        sl = sl + 1 == R ? 0 : sl + 1;
                    }
#pragma unroll
                    for (int q = 0; q < KF; ++q) old[q] = *cp[q];
#pragma unroll
                    for (int q = 0; q < KF; ++q) {
                        const float hv = fmaxf(so - fabsf((float)(lof + q) - c), 0.0f);
                        *cp[q] = old[q] + wq * hv;
                    }
                }
            }
        }
        tmod = tmod + 1 == R ? 0 : tmod + 1;
    };

    for (int t0 = 0; t0 < T; t0 += kScatterPrefetch) {
#pragma unroll
        for (int q = 0; q < kScatterPrefetch; ++q) step(t0 + q, xq[q]);
    }
}

// wpk[o * pitch + i] = W[i*N + o] << 16 | a low half from off[i*N + o] - omin, through 32 x 32
// LDS tiles. The low half: with sh = 0, offset - omin in the low byte; with sh > 0 (the
// arrival forward, whose R ring slots are exactly 2^16 bytes of 2^sh each), (offset - omin) <<
// sh plus the receiver's column bytes i * 4 (< 2^sh), so that a 16-bit add of the step's slot
// bytes gives the connection's LDS byte address in the ring (at LDS address 0) directly. With
// D > 0 the offsets must lie in [omin, omin + D) (the ring the arrival forward sizes from the
// caller's range): a connection outside it would land in another slot, so it is packed as a
// NaN weight at offset 0 instead (its receiver's outputs become NaN as soon as its source
// fires). The columns past N (up to pitch) weight 0, in their own ring column.
__global__ void __launch_bounds__(256) pack_hybrid_kernel(const uint16_t* __restrict__ W,
                                                         const int8_t* __restrict__ off, int N, int omin,
                                                         int sh, int D, int pitch, uint32_t* __restrict__ wpk) {
    __shared__ uint32_t tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    for (int r = threadIdx.y; r < 32; r += 8) {
        const int i = by + r, o = bx + threadIdx.x;
        const uint32_t col = sh > 0 ? (uint32_t)i * 4u : 0u;
        uint32_t v = col;
        if (i < N && o < N) {
            const int e = (int)off[(size_t)i * N + o] - omin;
            if (D > 0 && (e < 0 || e >= D))
                v = 0x7FC00000u | col;
            else
                v = ((uint32_t)W[(size_t)i * N + o] << 16) | ((((uint32_t)(uint8_t)e << sh) + col) & 0xFFFFu);
        }
        tile[r][threadIdx.x] = v;
    }
    __syncthreads();
    for (int r = threadIdx.y; r < 32; r += 8) {
        const int o = bx + r, i = by + threadIdx.x;
        if (i < pitch && o < N) wpk[(size_t)o * pitch + i] = tile[threadIdx.x][r];
    }
}

void launch_pack_hybrid(const uint16_t* W, const int8_t* off, int N, uint32_t* wpk, hipStream_t stream, int omin,
                        int sh, int D, int pitch) {
    if (pitch < N) pitch = N;
    const dim3 grid((N + 31) / 32, (pitch + 31) / 32), block(32, 8);
    hipLaunchKernelGGL(pack_hybrid_kernel, grid, block, 0, stream, W, off, N, omin, sh, D, pitch, wpk);
}

// Forward in gather form, for rings too large for LDS: lane i owns receiver i and sums
//   rec_i(t) = sum_j W_ij sum_l max(0, s_j - |l - c_ij|) / s_j^2 * y_j(t - l),  c_ij = 1 + d_ij,
// over every source each step. The spike history of each source is a bit word in LDS
// (bit l-1 = y_j(t - l), HW words of 64 lags, double-buffered so one barrier per step
// suffices); a connection reads the KT bits from its first lag lo_ij = max(1, ceil(c_ij - s_j))
// and adds the weight of each set bit. W and d (or the int8 offsets) stream in row-blocked
// chunks of 16 sources, one chunk ahead; sources silent for the whole window are skipped by
// the wave (the history word is wave-uniform).
template <int HW>
__device__ __forceinline__ uint32_t hist_window(const uint64_t (&h)[HW], int sh) {
    if (HW == 1) return (uint32_t)(h[0] >> sh);
    const uint64_t lo64 = sh < 64 ? (h[0] >> sh) | (sh ? h[HW - 1] << (64 - sh) : 0ull) : (h[HW - 1] >> (sh - 64));
    return (uint32_t)lo64;
}

template <int NPT, bool HYB, int HW>
__global__ void __launch_bounds__(1024) syn_fwd_gather_kernel(SynFwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    uint64_t* hist = reinterpret_cast<uint64_t*>(smem);          // [2][HW][N]
    float* s_l = reinterpret_cast<float*>(hist + (size_t)2 * HW * N);
    float* base_l = s_l + N;
    const Lif k = p.lif;
    const int TW = (T + 31) >> 5;
    const size_t BN = (size_t)B * N;
    const uint32_t wmask = p.KT >= 32 ? 0xFFFFFFFFu : ((1u << p.KT) - 1u);
    const bool wbf = p.w_bf16 != 0;

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
    }
    for (int j = tid; j < N; j += BS) {
#pragma unroll
        for (int w = 0; w < 2 * HW; ++w) hist[(size_t)w * N + j] = 0ull;
        s_l[j] = p.s ? p.s[j] : p.s_uniform;
        base_l[j] = HYB ? p.base[j] : 0.0f;
    }
    __syncthreads();

    const int NC = (N + 15) >> 4;
    uint32_t wa[NPT][16], da[NPT][16], wb2[NPT][16], db2[NPT][16];
    auto fetch = [&](int c, uint32_t (&cw)[NPT][16], uint32_t (&cd)[NPT][16]) {
#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            const size_t blk = (size_t)c * N + (act[q] ? idx[q] : 0);
            const int nw = wbf ? 2 : 4;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                if (h < nw) {
                    const uint4 x4 = static_cast<const uint4*>(p.Wr)[blk * nw + h];
                    cw[q][4 * h] = x4.x; cw[q][4 * h + 1] = x4.y; cw[q][4 * h + 2] = x4.z; cw[q][4 * h + 3] = x4.w;
                }
            }
            if (HYB) {
                const uint4 x4 = reinterpret_cast<const uint4*>(p.offr)[blk];
                cd[q][0] = x4.x; cd[q][1] = x4.y; cd[q][2] = x4.z; cd[q][3] = x4.w;
            } else {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint4 x4 = reinterpret_cast<const uint4*>(p.dr)[blk * 4 + h];
                    cd[q][4 * h] = x4.x; cd[q][4 * h + 1] = x4.y; cd[q][4 * h + 2] = x4.z; cd[q][4 * h + 3] = x4.w;
                }
            }
        }
    };

    for (int t = 0; t < T; ++t) {
        const uint64_t* hc = hist + (size_t)(t & 1) * HW * N;          // history through t - 1
        uint64_t* hn = hist + (size_t)((t + 1) & 1) * HW * N;
        float acc[NPT];
#pragma unroll
        for (int q = 0; q < NPT; ++q) acc[q] = 0.0f;

        auto gather = [&](int c, const uint32_t (&w32)[NPT][16], const uint32_t (&d32)[NPT][16]) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int j = c * 16 + e;
                if (j >= N) break;
                uint64_t h[HW];
                bool any = false;
#pragma unroll
                for (int w = 0; w < HW; ++w) {
                    h[w] = hc[(size_t)w * N + j];
                    any = any || h[w] != 0ull;
                }
                if (!any) continue;                    // j silent over the whole window
                const float sj = s_l[j];
                const float isj = 1.0f / (sj * sj);
#pragma unroll
                for (int q = 0; q < NPT; ++q) {
                    const float wv = wbf ? __uint_as_float((e & 1) ? (w32[q][e >> 1] & 0xFFFF0000u)
                                                                   : (w32[q][e >> 1] << 16))
                                         : __uint_as_float(w32[q][e]);
                    float dv;
                    if (HYB) {
                        const int off = ((int)(d32[q][e >> 2] << (24 - 8 * (e & 3)))) >> 24;
                        dv = base_l[j] + 0.0f + 1.0f * (float)off;
                    } else {
                        dv = __uint_as_float(d32[q][e]);
                    }
                    const float cc = 1.0f + dv;
                    const int lo = max(1, (int)ceilf(cc - sj));
                    uint32_t win = hist_window<HW>(h, lo - 1) & wmask;
                    float a = 0.0f;
                    while (win) {
                        const int bpos = __ffs(win) - 1;
                        win &= win - 1u;
                        a += fmaxf(sj - fabsf((float)(lo + bpos) - cc), 0.0f);
                    }
                    acc[q] = fmaf(wv, a * isj, acc[q]);
                }
            }
        };
        fetch(0, wa, da);
        for (int c = 0; c < NC; c += 2) {
            if (c + 1 < NC) fetch(c + 1, wb2, db2);
            gather(c, wa, da);
            if (c + 1 < NC) {
                if (c + 2 < NC) fetch(c + 2, wa, da);
                gather(c + 1, wb2, db2);
            }
        }

#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            const float xv = xq0[q];
            xq0[q] = xq1[q];
            const size_t row = (size_t)b * N + (act[q] ? idx[q] : 0);
            if (act[q] && t + 2 < T) xq1[q] = p.x[(size_t)(t + 2) * BN + row];
            const float r = acc[q] + bias[q];
            const float a = xv + r * m[q];
            const float u = lif_charge(k, v[q], a);
            const float y = act[q] ? lif_fire(k, u) : 0.0f;
            v[q] = lif_reset(k, u, y);
            const uint32_t yb = y != 0.0f ? 1u : 0u;
            word[q] |= yb << (t & 31);
            if (act[q]) {
                const int i = idx[q];
                const size_t o = (size_t)t * BN + row;
                p.y[o] = y;
                p.u[o] = u;
                if ((t & 31) == 31 || t == T - 1) p.bits[((size_t)b * TW + (t >> 5)) * N + i] = word[q];
                uint64_t carry = yb;
#pragma unroll
                for (int w = 0; w < HW; ++w) {
                    const uint64_t old = hc[(size_t)w * N + i];
                    hn[(size_t)w * N + i] = (old << 1) | carry;
                    carry = old >> 63;
                }
            }
            if ((t & 31) == 31) word[q] = 0;
        }
        __syncthreads();
    }
}

// Backward scan. Lane j owns source j (NPT sources per lane). The future gr of every
// receiver i sits in a source-major ring row: ring[i * RP + slot], slot = time mod R, plus
// KT mirror slots (slot s < KT is also written at R + s) so that a run of KT taps starting
// at any slot never wraps. Each step every lane walks i = 0 .. N-1 over the same ring row
// (all lanes gather inside one row), with W^T[j, i..] and d^T[j, i..] (or the int8
// offsets) streamed in chunks of 16 receivers from blocked copies in which a wave's lanes
// read adjacent 16-byte runs, one chunk ahead of the gather:
//   general:  gfut_j = sum_i W_ij sum_{q<KT} max(0, s - |lo_ij + q - c_ij|) gr_i(t + lo_ij + q) / s^2
//             with c_ij = 1 + d_ij and lo_ij = max(1, ceil(c_ij - s));
//   hybrid:   the taps of column j are those of c_j = 1 + base_j shifted by the integer
//             offset, so the KT weights are per-lane constants and a connection only adds
//             its offset to the slot (int8 offsets, 2 bytes per connection with bf16 W).
// The ring is in LDS when N * RP floats fit, else in the workspace (one row per receiver,
// so a step's gathers of all lanes stay within one cache-line run per i).
template <int NPT, int KT, bool HYB, int MAXT, bool GRING>
__global__ void __launch_bounds__(MAXT) syn_bwd_kernel(SynBwd p) {
    extern __shared__ float smem[];
    constexpr int KA = (HYB && KT > 0) ? KT : 1;        // per-tap accumulators (hybrid, fixed KT)
    const int N = p.N, T = p.T, B = p.B, R = p.R, RP = p.RP;
    const int kt = KT > 0 ? KT : p.KT;                  // KT == 0: the tap count is a runtime value
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    float* ring = GRING ? p.gring + (size_t)b * N * RP : smem;
    const Lif k = p.lif;
    const size_t BN = (size_t)B * N;
    const bool wbf = p.w_bf16 != 0;

    int idx[NPT];
    bool act[NPT];
    float lam[NPT], m[NPT], dbacc[NPT], sv[NPT], is2[NPT], cj[NPT];
    float hq[NPT][KA];
    int lob[NPT];
    bool chk[NPT];
#pragma unroll
    for (int q = 0; q < NPT; ++q) {
        idx[q] = tid + q * BS;
        act[q] = idx[q] < N;
        const int jc = act[q] ? idx[q] : 0;
        lam[q] = 0.0f;
        dbacc[q] = 0.0f;
        m[q] = p.drop ? p.drop[(size_t)b * N + jc] : 1.0f;
        sv[q] = p.s ? p.s[jc] : p.s_uniform;
        is2[q] = 1.0f / (sv[q] * sv[q]);
        lob[q] = 1;
        chk[q] = false;
        cj[q] = 0.0f;
        if (HYB) {
            // unclamped first lag of the closed support of c_j (a connection adds its offset)
            const float c = 1.0f + p.base[jc];
            int lo = (int)ceilf(c - sv[q]);
            if (fabsf((float)(lo - 1) - c) <= sv[q]) lo -= 1;
            if (fabsf((float)lo - c) > sv[q]) lo += 1;
            lob[q] = lo;
            cj[q] = c;
#pragma unroll
            for (int e = 0; e < KA; ++e) hq[q][e] = fmaxf(sv[q] - fabsf((float)(lo + e) - c), 0.0f);
            // some connection of j reaches a lag <= 0 (the zero offsets of the padded W^T
            // columns i >= N count too)
            chk[q] = lo + min(p.meta[1], 0) < 1;
        }
        for (int r = 0; r < p.RS; ++r)
            if (act[q]) ring[(size_t)idx[q] * RP + r] = 0.0f;
    }
    // lanes whose connections may reach lags <= 0 take the masked gather, wave by wave
    bool any_chk = false;
#pragma unroll
    for (int q = 0; q < NPT; ++q) any_chk = any_chk || chk[q];
    any_chk = __any(any_chk) != 0;
    __syncthreads();

    float gq[NPT][2], uq[NPT][2];
#pragma unroll
    for (int q = 0; q < NPT; ++q)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const int tt = T - 1 - f;
            const size_t o = (size_t)(tt >= 0 ? tt : 0) * BN + (size_t)b * N + (act[q] ? idx[q] : 0);
            gq[q][f] = (act[q] && tt >= 0) ? p.gy[o] : 0.0f;
            uq[q][f] = (act[q] && tt >= 0) ? p.u[o] : 0.0f;
        }

    int tmod = (T - 1) % R;
    for (int t = T - 1; t >= 0; --t) {
        float acc[NPT][KA];
#pragma unroll
        for (int q = 0; q < NPT; ++q)
#pragma unroll
            for (int e = 0; e < KA; ++e) acc[q][e] = 0.0f;

        // stream the chunks of 16 receivers: W^T (and d^T / offsets^T) of chunk c + 1 are
        // loaded while chunk c is gathered
        uint32_t wa[NPT][16], da[NPT][16], wb[NPT][16], db[NPT][16];
        auto fetch = [&](int c, uint32_t (&cw)[NPT][16], uint32_t (&cd)[NPT][16]) {
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                const size_t blk = (size_t)c * N + (act[q] ? idx[q] : 0);
                const int nw = wbf ? 2 : 4;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    if (h < nw) {
                        const uint4 v = static_cast<const uint4*>(p.Wt)[blk * nw + h];
                        cw[q][4 * h] = v.x; cw[q][4 * h + 1] = v.y; cw[q][4 * h + 2] = v.z; cw[q][4 * h + 3] = v.w;
                    }
                }
                if (HYB) {
                    const uint4 v = reinterpret_cast<const uint4*>(p.offt)[blk];
                    cd[q][0] = v.x; cd[q][1] = v.y; cd[q][2] = v.z; cd[q][3] = v.w;
                } else {
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const uint4 v = reinterpret_cast<const uint4*>(p.dt)[blk * 4 + h];
                        cd[q][4 * h] = v.x; cd[q][4 * h + 1] = v.y; cd[q][4 * h + 2] = v.z; cd[q][4 * h + 3] = v.w;
                    }
                }
            }
        };
        auto gather = [&](int c, const uint32_t (&w32)[NPT][16], const uint32_t (&d32)[NPT][16],
                          auto checked) {
            constexpr bool CHK = decltype(checked)::value;
#pragma unroll
            for (int q = 0; q < NPT; ++q) {
                float wf[16];
                if (wbf) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        wf[e] = __uint_as_float((e & 1) ? (w32[q][e >> 1] & 0xFFFF0000u) : (w32[q][e >> 1] << 16));
                } else {
#pragma unroll
                    for (int e = 0; e < 16; ++e) wf[e] = __uint_as_float(w32[q][e]);
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int i = min(c * 16 + e, N - 1);  // W^T is zero past N
                    const float* row = ring + (size_t)i * RP;
                    const float w = wf[e];
                    if (HYB) {
                        const int off = ((int)(d32[q][e >> 2] << (24 - 8 * (e & 3)))) >> 24;
                        const int lag0 = lob[q] + off;
                        if (!CHK) {                        // every lag lag0 + f >= 1
                            int slot = tmod + lag0;
                            slot = slot >= R ? slot - R : slot;
                            if (KT > 0) {
#pragma unroll
                                for (int f = 0; f < KA; ++f) acc[q][f] = fmaf(w, row[slot + f], acc[q][f]);
                            } else {
                                float a = 0.0f;
                                for (int f = 0; f < kt; ++f)
                                    a = fmaf(fmaxf(sv[q] - fabsf((float)(lob[q] + f) - cj[q]), 0.0f), row[slot + f], a);
                                acc[q][0] = fmaf(w, a, acc[q][0]);
                            }
                        } else if (KT > 0) {
                            // lags <= 0 do not exist: read a valid slot, weigh it 0
#pragma unroll
                            for (int f = 0; f < KA; ++f) {
                                int slot = tmod + max(lag0 + f, 1);
                                slot = slot >= R ? slot - R : slot;
                                const float g = row[slot];
                                acc[q][f] = fmaf(w, (lag0 + f >= 1) ? g : 0.0f, acc[q][f]);
                            }
                        } else {
                            float a = 0.0f;
                            for (int f = 0; f < kt; ++f) {
                                int slot = tmod + max(lag0 + f, 1);
                                slot = slot >= R ? slot - R : slot;
                                const float g = row[slot];
                                a = fmaf(fmaxf(sv[q] - fabsf((float)(lob[q] + f) - cj[q]), 0.0f),
                                         (lag0 + f >= 1) ? g : 0.0f, a);
                            }
                            acc[q][0] = fmaf(w, a, acc[q][0]);
                        }
                    } else {
                        const float c1 = 1.0f + __uint_as_float(d32[q][e]);
                        const int lo = max(1, (int)ceilf(c1 - sv[q]));
                        int slot = tmod + lo;
                        slot = slot >= R ? slot - R : slot;
                        const float x0 = (float)lo - c1;
                        float a = 0.0f;
                        if (KT > 0) {
#pragma unroll
                            for (int f = 0; f < (KT > 0 ? KT : 1); ++f)
                                a = fmaf(fmaxf(sv[q] - fabsf(x0 + (float)f), 0.0f), row[slot + f], a);
                        } else {
                            for (int f = 0; f < kt; ++f)
                                a = fmaf(fmaxf(sv[q] - fabsf(x0 + (float)f), 0.0f), row[slot + f], a);
                        }
                        acc[q][0] = fmaf(w, a, acc[q][0]);
                    }
                }
            }
        };
        auto gather_any = [&](int c, const uint32_t (&w32)[NPT][16], const uint32_t (&d32)[NPT][16]) {
            if (HYB && any_chk) gather(c, w32, d32, std::true_type{});
            else gather(c, w32, d32, std::false_type{});
        };
        // chunks of 16 receivers, ping-ponged between two register buffers: chunk c + 1 is
        // loaded while chunk c is gathered
        const int NC = (N + 15) >> 4;
        fetch(0, wa, da);
        for (int c = 0; c < NC; c += 2) {
            if (c + 1 < NC) fetch(c + 1, wb, db);
            gather_any(c, wa, da);
            if (c + 1 < NC) {
                if (c + 2 < NC) fetch(c + 2, wa, da);
                gather_any(c + 1, wb, db);
            }
        }

#pragma unroll
        for (int q = 0; q < NPT; ++q) {
            float gf = 0.0f;
            if (HYB && KT > 0) {
#pragma unroll
                for (int f = 0; f < KA; ++f) gf = fmaf(hq[q][f], acc[q][f], gf);
            } else {
                gf = acc[q][0];
            }
            gf *= is2[q];
            const float gyv = gq[q][0], u = uq[q][0];
            gq[q][0] = gq[q][1];
            uq[q][0] = uq[q][1];
            const int tn = t - 2;
            const size_t on = (size_t)(tn >= 0 ? tn : 0) * BN + (size_t)b * N + (act[q] ? idx[q] : 0);
            gq[q][1] = (act[q] && tn >= 0) ? p.gy[on] : 0.0f;
            uq[q][1] = (act[q] && tn >= 0) ? p.u[on] : 0.0f;
            if (!act[q]) continue;
            const int j = idx[q];
            const size_t o = (size_t)t * BN + (size_t)b * N + j;
            const float y = lif_fire(k, u);
            const float du = lif_backward(k, gyv + gf, u, y, lam[q]);
            lam[q] = k.decay * du;
            const float da = lif_dx(k, du);
            const float gr = da * m[q];
            p.dx[o] = da;
            if (p.drop) p.gr[o] = gr;   // else gr == dx: the lag correlation reads dx
            dbacc[q] += gr;
            float* row = ring + (size_t)j * RP;
            row[tmod] = gr;
            if (tmod < kt) row[tmod + R] = gr;
        }
        __syncthreads();
        tmod = tmod == 0 ? R - 1 : tmod - 1;
    }
#pragma unroll
    for (int q = 0; q < NPT; ++q)
        if (act[q]) p.part[(size_t)b * N + idx[q]] = dbacc[q];
}

template <int NPT>
void launch_syn_fwd_n(const SynFwd& a, int block, size_t lds, hipStream_t stream) {
    if (a.gring) {
        ensure_lds((const void*)syn_fwd_kernel<NPT, true>, lds);
        hipLaunchKernelGGL((syn_fwd_kernel<NPT, true>), dim3(a.B), dim3(block), lds, stream, a);
    } else {
        ensure_lds((const void*)syn_fwd_kernel<NPT, false>, lds);
        hipLaunchKernelGGL((syn_fwd_kernel<NPT, false>), dim3(a.B), dim3(block), lds, stream, a);
    }
}

template <int NPT, bool HYB, int HW>
void launch_syn_fwd_g(const SynFwd& a, int block, size_t lds, hipStream_t stream) {
    ensure_lds((const void*)syn_fwd_gather_kernel<NPT, HYB, HW>, lds);
    hipLaunchKernelGGL((syn_fwd_gather_kernel<NPT, HYB, HW>), dim3(a.B), dim3(block), lds, stream, a);
}

template <int NPT>
void launch_syn_fwd_gather(const SynFwd& a, int block, size_t lds, hipStream_t stream) {
    const bool hyb = a.offr != nullptr;
    if (a.HW == 1) {
        if (hyb) launch_syn_fwd_g<NPT, true, 1>(a, block, lds, stream);
        else launch_syn_fwd_g<NPT, false, 1>(a, block, lds, stream);
    } else {
        if (hyb) launch_syn_fwd_g<NPT, true, 2>(a, block, lds, stream);
        else launch_syn_fwd_g<NPT, false, 2>(a, block, lds, stream);
    }
}

#define DELREC_SCAT_CASE(KFV, HYBV, WBFV)                                                    \
    if (kf == KFV && hyb == HYBV && wbf == WBFV) {                                           \
        ensure_lds((const void*)syn_fwd_scatter<KFV, HYBV, WBFV>, lds);                     \
        hipLaunchKernelGGL((syn_fwd_scatter<KFV, HYBV, WBFV>), dim3(a.B), dim3(block), lds, stream, a); \
        return true;                                                                         \
    }
#define DELREC_SCAT_KF(HYBV, WBFV) \
    DELREC_SCAT_CASE(2, HYBV, WBFV) DELREC_SCAT_CASE(4, HYBV, WBFV) DELREC_SCAT_CASE(8, HYBV, WBFV)

bool launch_syn_fwd_scatter(const SynFwd& a, int kf, int block, size_t lds, hipStream_t stream) {
    const bool hyb = a.offt != nullptr, wbf = a.w_bf16 != 0;
    DELREC_SCAT_KF(false, false) DELREC_SCAT_KF(false, true) DELREC_SCAT_KF(true, false) DELREC_SCAT_KF(true, true)
    return false;
}

void launch_syn_fwd(const SynFwd& a, int block, size_t lds, hipStream_t stream) {
    const int npt = (a.N + block - 1) / block;
    if (a.Wr) {
        if (npt == 1) launch_syn_fwd_gather<1>(a, block, lds, stream);
        else if (npt == 2) launch_syn_fwd_gather<2>(a, block, lds, stream);
        else launch_syn_fwd_gather<4>(a, block, lds, stream);
        return;
    }
    if (npt == 1) launch_syn_fwd_n<1>(a, block, lds, stream);
    else if (npt == 2) launch_syn_fwd_n<2>(a, block, lds, stream);
    else launch_syn_fwd_n<4>(a, block, lds, stream);
}

template <int NPT, int KT, bool HYB, int MAXT>
void launch_syn_bwd_k(const SynBwd& a, int block, size_t lds, hipStream_t stream) {
    if (a.gring) {
        hipLaunchKernelGGL((syn_bwd_kernel<NPT, KT, HYB, MAXT, true>), dim3(a.B), dim3(block), 0, stream, a);
    } else {
        ensure_lds((const void*)syn_bwd_kernel<NPT, KT, HYB, MAXT, false>, lds);
        hipLaunchKernelGGL((syn_bwd_kernel<NPT, KT, HYB, MAXT, false>), dim3(a.B), dim3(block), lds, stream, a);
    }
}

// Hybrid backward with the ring in LDS, one source per lane (N <= 1024), KT = 2 or 4 taps.
// The same dense reverse gather as syn_bwd_kernel,
//   gfut_j = is2 * sum_f hq_j[f] * sum_i W[i,j] gr_i(t + lob_j + off_ij + f),
// with the per-connection work cut to an offset decode, one slot add and wrap, one LDS
// address (the 16 rows of a chunk are immediate offsets) and a KT-wide read: the lane's
// base slot (t + lob_j + min offset) mod R is formed once per step. Receivers stream in
// groups of 4 chunks of 16 (blocked W^T and offsets^T), the next group's operands in
// flight while the current group is gathered; past the last chunk the descriptor bounds
// read 0. CHK: some connection may reach a lag <= 0 (negative base), those taps weigh 0.
template <int KT, bool WBF, int MAXT>
__global__ void __launch_bounds__(MAXT) syn_bwd_hyb(SynBwd p) {
    // SPLIT (1024-thread blocks): lanes l and l + 32 of a wave hold the same source and
    // gather over the two halves of the receivers, so four waves share each SIMD (128 VGPRs)
    constexpr bool SPLIT = MAXT > 512;
    // chunks of 16 receivers per group: two groups of operands stay in registers
    constexpr int kBwdGroup = SPLIT ? 1 : 4;
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B, R = p.R, RP = p.RP;
    const int b = blockIdx.x, tid = threadIdx.x, BS = blockDim.x;
    float* ring = smem;                                   // [rows][RP]
    const size_t BN = (size_t)B * N;
    const int half = SPLIT ? (tid >> 5) & 1 : 0;
    const int jloc = SPLIT ? (tid >> 6) * 32 + (tid & 31) : tid;
    const bool act = jloc < N;
    const bool writer = act && half == 0;                 // the lane that stores for source j
    const int j = act ? (p.order ? p.order[jloc] : jloc) : 0;   // this lane's source
    const Lif k = p.lif;
    const float m = p.drop ? p.drop[(size_t)b * N + j] : 1.0f;
    const float sv = p.s_uniform;
    const float is2 = 1.0f / (sv * sv);
    const float c = 1.0f + p.base[j];
    int lob = (int)ceilf(c - sv);
    if (fabsf((float)(lob - 1) - c) <= sv) lob -= 1;
    if (fabsf((float)lob - c) > sv) lob += 1;
    float hq[KT];
#pragma unroll
    for (int f = 0; f < KT; ++f) hq[f] = fmaxf(sv - fabsf((float)(lob + f) - c), 0.0f);
    const int omin = p.meta[1];
    const int NC0 = (N + 15) >> 4;
    const int NC = SPLIT ? (NC0 + 1) / 2 : NC0;           // chunks of 16 receivers per lane
    const int NG = (NC + kBwdGroup - 1) / kBwdGroup;
    const int rows = (SPLIT ? 2 : 1) * NG * kBwdGroup * 16;
    const int cbase = half * NC;                          // the lane's first chunk
    const bool chk = __syncthreads_or(act && lob + min(omin, 0) < 1) != 0;
    // no-wrap form: each ring row mirrors its first E = (max - min offset) + KT slots after
    // slot R - 1, so a connection's slot needs no wrap (when the longer rows fit the LDS)
    const int E = p.meta[2] - omin + KT;
    const int RPn = (R + E) | 1;
    // it reads the offsets as byte slot offsets (offset - smallest) * 4, which needs a span <= 63
    const bool nowrap = !chk && E <= R && rows * RPn <= p.ldsf && p.offq && p.meta[2] - omin <= 63;
    const int RPu = nowrap ? RPn : RP;

    for (int q = tid; q < rows * RPu; q += BS) ring[q] = 0.0f;
    __syncthreads();

    // blocked W^T: receivers 16c .. 16c+15 of source j at ((c*N + j)*16) elements
    const uint32_t wbytes = (uint32_t)((size_t)p.NT * N * (WBF ? 2 : 4));
    const uint32_t obytes = (uint32_t)((size_t)p.NT * N);
    const i32x4 rw = buffer_rsrc(p.Wt, wbytes), ro = buffer_rsrc(nowrap ? (const void*)p.offq : (const void*)p.offt, obytes);
    const int wcs = N * 16 * (WBF ? 2 : 4), ocs = N * 16;   // bytes per chunk
    // the blocked operands are laid out by lane slot (jloc), in the order the host chose
    const int wj = act ? jloc * 16 * (WBF ? 2 : 4) + cbase * wcs : kOutOfRange;
    const int oj = act ? jloc * 16 + cbase * ocs : kOutOfRange;
    constexpr int WV = WBF ? 2 : 4;                          // uint4 of W per chunk
    struct Chunk { uint4 w[WV]; uint4 o; };
    auto fetch = [&](int cidx, Chunk& ch) {
        const int cw = cidx * wcs, co = cidx * ocs;
#pragma unroll
        for (int h = 0; h < WV; ++h) {
            const i32x4 v = raw_buffer_load_i32x4(rw, wj + cw + 16 * h, 0, 0);
            ch.w[h] = make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
        }
        const i32x4 ov = raw_buffer_load_i32x4(ro, oj + co, 0, 0);
        ch.o = make_uint4((uint32_t)ov.x, (uint32_t)ov.y, (uint32_t)ov.z, (uint32_t)ov.w);
    };
    const uint32_t row_bytes = (uint32_t)BN * 4u;
    const uint64_t step_b = (uint64_t)row_bytes;
    const int voff = (b * N + j) * 4;
    const int soff = writer ? voff : kOutOfRange;

    float gq[kPrefetchSynBwd], uq[kPrefetchSynBwd];
    const int tp0 = T - 1 - kPrefetchSynBwd;
    uint64_t gya = (uint64_t)p.gy + (uint64_t)max(tp0, 0) * step_b, uau = (uint64_t)p.u + (uint64_t)max(tp0, 0) * step_b;
    uint64_t dxa = (uint64_t)p.dx + (uint64_t)(T - 1) * step_b, gra = (uint64_t)p.gr + (uint64_t)(T - 1) * step_b;
#pragma unroll
    for (int q = 0; q < kPrefetchSynBwd; ++q) {
        const int tt = T - 1 - q;
        const uint32_t nb = tt >= 0 ? row_bytes : 0u;
        gq[q] = raw_buffer_load_f32(step_rsrc((uint64_t)p.gy + (uint64_t)max(tt, 0) * step_b, nb), voff, 0, 0);
        uq[q] = raw_buffer_load_f32(step_rsrc((uint64_t)p.u + (uint64_t)max(tt, 0) * step_b, nb), voff, 0, 0);
    }
    float lam = 0.0f, dbacc = 0.0f;
    int tmod = (T - 1) % R;
    float* const own = act ? ring + (size_t)j * RPu : ring + (size_t)(rows - 1) * RPu;   // never read for j >= N
    const int mirror = nowrap ? E : KT;   // slots written twice

    auto gather_group = [&](const Chunk (&cg)[kBwdGroup], int g0, int tbo, float (&acc)[KT], auto checked,
                            auto nowrapped) {
        constexpr bool CHK = decltype(checked)::value;
        constexpr bool NW = decltype(nowrapped)::value;
#pragma unroll
        for (int cc = 0; cc < kBwdGroup; ++cc) {
            const float* rowc = ring + (size_t)(cbase + g0 + cc) * 16 * RPu;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t ow = (e < 4) ? cg[cc].o.x : (e < 8) ? cg[cc].o.y : (e < 12) ? cg[cc].o.z : cg[cc].o.w;
                const float* rp;
                int off = 0;
                if constexpr (NW) {
                    // tbo holds the base slot in bytes; one byte-select add per connection
                    const uint32_t sl4 = (uint32_t)tbo + ((ow >> (8 * (e & 3))) & 0xFFu);
                    rp = reinterpret_cast<const float*>(reinterpret_cast<const char*>(rowc + e * RPu) + sl4);
                } else {
                    off = ((int)(ow << (24 - 8 * (e & 3)))) >> 24;
                    int sl = tbo + off;
                    sl = sl >= R ? sl - R : sl;
                    rp = rowc + e * RPu + sl;
                }
                float wv;
                if constexpr (WBF) {
                    const uint4& wq = cg[cc].w[e >> 3];
                    const int e8 = e & 7;
                    const uint32_t w2 = (e8 < 2) ? wq.x : (e8 < 4) ? wq.y : (e8 < 6) ? wq.z : wq.w;
                    wv = __uint_as_float((e & 1) ? (w2 & 0xFFFF0000u) : (w2 << 16));
                } else {
                    const uint4& wq = cg[cc].w[e >> 2];
                    const int e4 = e & 3;
                    wv = __uint_as_float(e4 == 0 ? wq.x : e4 == 1 ? wq.y : e4 == 2 ? wq.z : wq.w);
                }
                if constexpr (!CHK) {
#pragma unroll
                    for (int f = 0; f < KT; ++f) acc[f] = fmaf(wv, rp[f], acc[f]);
                } else {
#pragma unroll
                    for (int f = 0; f < KT; ++f) {
                        // lags <= 0 do not exist: such a tap weighs 0 (its slot holds a valid,
                        // unrelated value)
                        const float gv = rp[f];
                        acc[f] = fmaf(wv, (lob + off + f >= 1) ? gv : 0.0f, acc[f]);
                    }
                }
            }
        }
    };

    auto step = [&](const int t, float& gs, float& us, auto checked, auto nowrapped) {
        float acc[KT];
#pragma unroll
        for (int f = 0; f < KT; ++f) acc[f] = 0.0f;
        // base slot of the smallest lag lob + omin (wrapped into [0, R)); a connection adds
        // off - omin >= 0 (and one more wrap)
        int tbo = tmod + lob + omin;
        tbo %= R;
        tbo = tbo < 0 ? tbo + R : tbo;
        if constexpr (decltype(nowrapped)::value) tbo *= 4;   // bytes; offsets arrive as (off - omin) * 4
        else tbo -= omin;
        Chunk ca[kBwdGroup], cb[kBwdGroup];
#pragma unroll
        for (int cc = 0; cc < kBwdGroup; ++cc) fetch(cc, ca[cc]);
        for (int g = 0; g < NG; g += 2) {
#pragma unroll
            for (int cc = 0; cc < kBwdGroup; ++cc) fetch((g + 1) * kBwdGroup + cc, cb[cc]);
            gather_group(ca, g * kBwdGroup, tbo, acc, checked, nowrapped);
            if (g + 1 < NG) {
#pragma unroll
                for (int cc = 0; cc < kBwdGroup; ++cc) fetch((g + 2) * kBwdGroup + cc, ca[cc]);
                gather_group(cb, (g + 1) * kBwdGroup, tbo, acc, checked, nowrapped);
            }
        }
        if constexpr (SPLIT) {
#pragma unroll
            for (int f = 0; f < KT; ++f) acc[f] += __shfl_xor(acc[f], 32);
        }
        float gf = 0.0f;
#pragma unroll
        for (int f = 0; f < KT; ++f) gf = fmaf(hq[f], acc[f], gf);
        gf *= is2;
        const float gyv = gs, u = us;
        const float y = lif_fire(k, u);
        const float du = lif_backward(k, gyv + gf, u, y, lam);
        lam = k.decay * du;
        const float da = lif_dx(k, du);
        const float gr = da * m;
        const bool live = t >= 0;
        raw_buffer_store_f32(da, step_rsrc(dxa, live ? row_bytes : 0u), soff, 0, 0);
        // gr differs from dx only under a dropout mask: otherwise the store is dropped (a
        // zero-sized descriptor) and the lag correlation reads dx
        raw_buffer_store_f32(gr, step_rsrc(gra, (live && p.drop) ? row_bytes : 0u), soff, 0, 0);
        dxa -= step_b;
        gra -= step_b;
        dbacc += (live && act) ? gr : 0.0f;
        if (writer && live) {
            own[tmod] = gr;
            if (tmod < mirror) own[tmod + R] = gr;
        }
        const int tp = t - kPrefetchSynBwd;
        const uint32_t nb = tp >= 0 ? row_bytes : 0u;
        gs = raw_buffer_load_f32(step_rsrc(gya, nb), voff, 0, 0);
        us = raw_buffer_load_f32(step_rsrc(uau, nb), voff, 0, 0);
        if (tp > 0) {
            gya -= step_b;
            uau -= step_b;
        }
        barrier_lds();
        tmod = tmod == 0 ? R - 1 : tmod - 1;
    };

    auto run = [&](auto checked, auto nowrapped) {
        for (int t0 = T - 1; t0 >= 0; t0 -= kPrefetchSynBwd) {
#pragma unroll
            for (int q = 0; q < kPrefetchSynBwd; ++q) step(t0 - q, gq[q], uq[q], checked, nowrapped);
        }
    };
    if (chk) run(std::true_type{}, std::false_type{});
    else if (nowrap) run(std::false_type{}, std::true_type{});
    else run(std::false_type{}, std::false_type{});
    if (writer) p.part[(size_t)b * N + j] = dbacc;
}

// The same hybrid backward in the offset-stacked form, one MAC per connection. With
// e_ij = off_ij - omin and c_j = lob_j + omin (>= 1: the host takes this form only when every
// lag is >= 1),
//   gfut_j(t) = is2 * sum_f hq_j[f] * G_j(t + c_j + f),   G_j(tau) = sum_i W[i,j] gr_i(tau + e_ij).
// Step t forms G_j(t + 1) (gr(t + 1 .. t + D) are all known) into a per-source history of
// RG = L slots and reads the older G_j(t + c_j + f) back from it; c_j + f = 1 is this step's own
// G. The gr ring then spans only the D steps t + 1 .. t + D: Dg = D + 1 slots per receiver row
// (gr(t) goes to the slot no read of step t touches), each value stored twice, at slots s and
// s + Dg, so a step's run starts at the same slot b0 = (t + 1) mod Dg in every lane and a
// connection reads slot b0 + e_ij with no wrap. The lanes of a wave read one receiver row
// within D consecutive slots (a broadcast over distinct banks); a connection costs the W
// decode, one address add (the offset byte, held as e * 4) and one FMA, the row within a
// chunk being an immediate offset (the row pitch GS >= 2 D is a compile-time constant).
// Two lanes per source (l and l + 32 of a wave), each over half the receivers.
// LDS: rows * GS floats of ring, then RG x (blockDim / 2) floats of G history.
template <int KT, bool WBF, int GS>
__global__ void __launch_bounds__(1024) syn_bwd_hyb_g(SynBwd p) {
    extern __shared__ float smem[];
    const int N = p.N, T = p.T, B = p.B;
    const int b = blockIdx.x, tid = threadIdx.x;
    const int half = (tid >> 5) & 1;
    const int jloc = (tid >> 6) * 32 + (tid & 31);
    const bool act = jloc < N;
    const bool writer = act && half == 0;                 // the lane that stores for source j
    const int j = act ? (p.order ? p.order[jloc] : jloc) : 0;
    const Lif k = p.lif;
    const float m = p.drop ? p.drop[(size_t)b * N + j] : 1.0f;
    const float sv = p.s_uniform;
    const float is2 = 1.0f / (sv * sv);
    const float cj = 1.0f + p.base[j];
    int lob = (int)ceilf(cj - sv);
    if (fabsf((float)(lob - 1) - cj) <= sv) lob -= 1;
    if (fabsf((float)lob - cj) > sv) lob += 1;
    float hq[KT];
#pragma unroll
    for (int f = 0; f < KT; ++f) hq[f] = fmaxf(sv - fabsf((float)(lob + f) - cj), 0.0f);
    const int omin = p.meta[1];
    const int D = p.meta[2] - omin + 1;
    const int Dg = D + 1;
    const int c0 = lob + omin;                            // tau - t of tap 0
    const int NC0 = (N + 15) >> 4;
    const int NC = (NC0 + 1) / 2;                         // chunks of 16 receivers per lane
    const int rows = 2 * NC * 16;
    const int NL = (int)blockDim.x / 2;                   // G-history pitch (lane slots)
    const int RG = p.L;
    float* ring = smem;                                   // [rows][GS]
    float* ghist = smem + (size_t)rows * GS;              // [RG][NL]
    // the offsets' span must fit the ring pitch (the host sized GS from the caller's
    // off_count): a wider one makes every output NaN instead of reading other rows
    // and every tap of non-zero weight must lie at a lag >= 1 (tap f at c0 + f, c0 = lob + omin
    // with the offsets' own smallest value; lob may be a zero-weight edge tap): a caller's
    // d_min that claimed so wrongly gives NaN, not dropped taps
    bool low = false;
#pragma unroll
    for (int f = 0; f < KT; ++f) low = low || (c0 + f < 1 && hq[f] > 0.0f);
    const bool bad = 2 * D > GS || RG < 2 || __syncthreads_or(act && low) != 0;
    for (int q = tid; q < rows * GS + RG * NL; q += blockDim.x) smem[q] = 0.0f;
    __syncthreads();

    const uint32_t wbytes = (uint32_t)((size_t)p.NT * N * (WBF ? 2 : 4));
    const uint32_t obytes = (uint32_t)((size_t)p.NT * N);
    const i32x4 rw = buffer_rsrc(p.Wt, wbytes), ro = buffer_rsrc(p.offq, obytes);
    const int wcs = N * 16 * (WBF ? 2 : 4), ocs = N * 16;   // bytes per chunk
    const int cbase = half * NC;                          // the lane's first chunk
    const int wj = act ? jloc * 16 * (WBF ? 2 : 4) + cbase * wcs : kOutOfRange;
    const int oj = act ? jloc * 16 + cbase * ocs : kOutOfRange;
    constexpr int WV = WBF ? 2 : 4;                       // uint4 of W per chunk
    struct Chunk { uint4 w[WV]; uint4 o; };
    auto fetch = [&](int cidx, Chunk& ch) {
        const int cw = cidx * wcs, co = cidx * ocs;
#pragma unroll
        for (int h = 0; h < WV; ++h) {
            const i32x4 v = raw_buffer_load_i32x4(rw, wj + cw + 16 * h, 0, 0);
            ch.w[h] = make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
        }
        const i32x4 ov = raw_buffer_load_i32x4(ro, oj + co, 0, 0);
        ch.o = make_uint4((uint32_t)ov.x, (uint32_t)ov.y, (uint32_t)ov.z, (uint32_t)ov.w);
    };
    const size_t BN = (size_t)B * N;
    const uint32_t row_bytes = (uint32_t)BN * 4u;
    const uint64_t step_b = (uint64_t)row_bytes;
    const int voff = (b * N + j) * 4;
    const int soff = writer ? voff : kOutOfRange;

    float gq[kPrefetchSynBwd], uq[kPrefetchSynBwd];
    const int tp0 = T - 1 - kPrefetchSynBwd;
    uint64_t gya = (uint64_t)p.gy + (uint64_t)max(tp0, 0) * step_b, uau = (uint64_t)p.u + (uint64_t)max(tp0, 0) * step_b;
    uint64_t dxa = (uint64_t)p.dx + (uint64_t)(T - 1) * step_b, gra = (uint64_t)p.gr + (uint64_t)(T - 1) * step_b;
#pragma unroll
    for (int q = 0; q < kPrefetchSynBwd; ++q) {
        const int tt = T - 1 - q;
        const uint32_t nb = tt >= 0 ? row_bytes : 0u;
        gq[q] = raw_buffer_load_f32(step_rsrc((uint64_t)p.gy + (uint64_t)max(tt, 0) * step_b, nb), voff, 0, 0);
        uq[q] = raw_buffer_load_f32(step_rsrc((uint64_t)p.u + (uint64_t)max(tt, 0) * step_b, nb), voff, 0, 0);
    }
    float lam = 0.0f, dbacc = 0.0f;
    int b0 = T % Dg;                                      // (t + 1) mod Dg
    int g1 = T % RG;                                      // (t + 1) mod RG
    float* const own = ring + (size_t)(act ? j : 0) * GS; // this source's row as a receiver
    float* const gown = ghist + jloc;

    auto gather = [&](const Chunk& ch, int cidx, float acc) {
        // the chunk's 16 receiver rows from slot b0: row e at the immediate offset e * GS
        const char* rowc = reinterpret_cast<const char*>(ring + (size_t)(cbase + cidx) * 16 * GS + b0);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t ow = (e < 4) ? ch.o.x : (e < 8) ? ch.o.y : (e < 12) ? ch.o.z : ch.o.w;
            const uint32_t sl4 = (ow >> (8 * (e & 3))) & 0xFFu;
            const float gv = *reinterpret_cast<const float*>(rowc + sl4 + e * GS * 4);
            float wv;
            if constexpr (WBF) {
                const uint4& wq = ch.w[e >> 3];
                const int e8 = e & 7;
                const uint32_t w2 = (e8 < 2) ? wq.x : (e8 < 4) ? wq.y : (e8 < 6) ? wq.z : wq.w;
                wv = __uint_as_float((e & 1) ? (w2 & 0xFFFF0000u) : (w2 << 16));
            } else {
                const uint4& wq = ch.w[e >> 2];
                const int e4 = e & 3;
                wv = __uint_as_float(e4 == 0 ? wq.x : e4 == 1 ? wq.y : e4 == 2 ? wq.z : wq.w);
            }
            acc = fmaf(wv, gv, acc);
        }
        return acc;
    };

    auto step = [&](const int t, float& gs, float& us) {
        float acc = 0.0f;
        Chunk ca, cb;
        fetch(0, ca);
        for (int c = 0; c < NC; c += 2) {
            fetch(c + 1, cb);
            acc = gather(ca, c, acc);
            if (c + 1 < NC) {
                fetch(c + 2, ca);
                acc = gather(cb, c + 1, acc);
            }
        }
        const float G = acc + __shfl_xor(acc, 32);        // G_j(t + 1)
        if (writer) gown[(size_t)g1 * NL] = G;
        float gf = 0.0f;
#pragma unroll
        for (int f = 0; f < KT; ++f) {
            // tau - t = c0 + f; a tap of weight 0 outside lags 1 .. L - 1 reads some slot in
            // range, which it weighs by 0
            const int dd = min(max(c0 + f, 1), RG);
            int sl = g1 + dd - 1;
            sl = sl >= RG ? sl - RG : sl;
            const float gv = dd == 1 ? G : (t + dd < T ? gown[(size_t)sl * NL] : 0.0f);
            gf = fmaf(hq[f], gv, gf);
        }
        gf *= is2;
        const float gyv = gs, u = us;
        const float y = lif_fire(k, u);
        const float du = lif_backward(k, gyv + gf, u, y, lam);
        lam = k.decay * du;
        const float da = bad ? __builtin_nanf("") : lif_dx(k, du);
        const float gr = da * m;
        const bool live = t >= 0;
        raw_buffer_store_f32(da, step_rsrc(dxa, live ? row_bytes : 0u), soff, 0, 0);
        // gr differs from dx only under a dropout mask: otherwise the store is dropped (a
        // zero-sized descriptor) and the lag correlation reads dx
        raw_buffer_store_f32(gr, step_rsrc(gra, (live && p.drop) ? row_bytes : 0u), soff, 0, 0);
        dxa -= step_b;
        gra -= step_b;
        dbacc += (live && act) ? gr : 0.0f;
        // gr(t) into slot t mod Dg (no read of this step touches it) and its mirror
        const int sw = b0 == 0 ? Dg - 1 : b0 - 1;
        if (writer && live && !bad) {
            own[sw] = gr;
            if (sw + Dg < 2 * D) own[sw + Dg] = gr;
        }
        const int tp = t - kPrefetchSynBwd;
        const uint32_t nb = tp >= 0 ? row_bytes : 0u;
        gs = raw_buffer_load_f32(step_rsrc(gya, nb), voff, 0, 0);
        us = raw_buffer_load_f32(step_rsrc(uau, nb), voff, 0, 0);
        if (tp > 0) {
            gya -= step_b;
            uau -= step_b;
        }
        barrier_lds();
        b0 = sw;
        g1 = g1 == 0 ? RG - 1 : g1 - 1;
    };

    for (int t0 = T - 1; t0 >= 0; t0 -= kPrefetchSynBwd) {
#pragma unroll
        for (int q = 0; q < kPrefetchSynBwd; ++q) step(t0 - q, gq[q], uq[q]);
    }
    if (writer) p.part[(size_t)b * N + j] = dbacc;
}

__global__ void pack_offq_kernel(const int8_t* __restrict__ offt, size_t n, const int* __restrict__ meta,
                                 uint8_t* __restrict__ offq) {
    const int omin = meta[1];
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (size_t)gridDim.x * blockDim.x)
        offq[q] = (uint8_t)(((int)offt[q] - omin) * 4);
}

// order[k] = the source with the k-th smallest key (first lag lob, index): the first lag of
// non-zero weight of each hybrid source, computed as syn_bwd_hyb does. One workgroup.
__global__ void __launch_bounds__(1024) sort_by_first_lag_kernel(const float* base, float sv, int N,
                                                                 int* order) {
    __shared__ int key[1024];
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        const float c = 1.0f + base[j];
        int lob = (int)ceilf(c - sv);
        if (fabsf((float)(lob - 1) - c) <= sv) lob -= 1;
        if (fabsf((float)lob - c) > sv) lob += 1;
        key[j] = lob;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        const int kj = key[j];
        int pos = 0;
        for (int q = 0; q < N; ++q) {
            const int kq = key[q];
            pos += (kq < kj || (kq == kj && q < j)) ? 1 : 0;
        }
        order[pos] = j;
    }
}

void launch_sort_by_first_lag(const float* base, float s, int N, int* order, hipStream_t stream) {
    hipLaunchKernelGGL(sort_by_first_lag_kernel, dim3(1), dim3(1024), 0, stream, base, s, N, order);
}

void launch_pack_offq(const int8_t* offt, size_t n, const int* meta, uint8_t* offq, hipStream_t stream) {
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(pack_offq_kernel, dim3(blocks), dim3(256), 0, stream, offt, n, meta, offq);
}

#define DELREC_SBH_CASE(KTV, WBFV)                                                          \
    if (kt == KTV && wbf == WBFV) {                                                          \
        if (split) {                                                                         \
            ensure_lds((const void*)syn_bwd_hyb<KTV, WBFV, 1024>, lds);                      \
            hipLaunchKernelGGL((syn_bwd_hyb<KTV, WBFV, 1024>), dim3(a.B), dim3(block), lds, stream, a); \
        } else {                                                                             \
            ensure_lds((const void*)syn_bwd_hyb<KTV, WBFV, 512>, lds);                       \
            hipLaunchKernelGGL((syn_bwd_hyb<KTV, WBFV, 512>), dim3(a.B), dim3(block), lds, stream, a); \
        }                                                                                    \
        return true;                                                                         \
    }

// LDS of syn_bwd_hyb_g for a ring pitch gs, or 0 when no compiled pitch holds 2 D slots
size_t syn_bwd_hyb_g_lds(int N, int L, int D, int* gs) {
    const int g = 2 * D <= 16 ? 16 : 2 * D <= 24 ? 24 : 0;
    *gs = g;
    if (!g || N > 512 || L < 2) return 0;
    const int NC = ((N + 15) / 16 + 1) / 2;
    const int block = 2 * ((N + 31) / 32 * 32);
    return ((size_t)2 * NC * 16 * g + (size_t)L * (block / 2)) * sizeof(float);
}

#define DELREC_SBHG_CASE(KTV, WBFV, GSV)                                                    \
    if (kt == KTV && wbf == WBFV && gs == GSV) {                                             \
        ensure_lds((const void*)syn_bwd_hyb_g<KTV, WBFV, GSV>, lds);                         \
        hipLaunchKernelGGL((syn_bwd_hyb_g<KTV, WBFV, GSV>), dim3(a.B), dim3(block), lds, stream, a); \
        return true;                                                                         \
    }

bool launch_syn_bwd_hyb_g(const SynBwd& a, int D, size_t max_lds, hipStream_t stream) {
    int gs = 0;
    const size_t lds = syn_bwd_hyb_g_lds(a.N, a.L, D, &gs);
    if (!lds || lds > max_lds || !a.offq || !a.meta) return false;
    const int block = 2 * ((a.N + 31) / 32 * 32);
    const int kt = a.KT;
    const bool wbf = a.w_bf16 != 0;
    DELREC_SBHG_CASE(2, true, 16) DELREC_SBHG_CASE(2, true, 24) DELREC_SBHG_CASE(2, false, 16)
    DELREC_SBHG_CASE(2, false, 24) DELREC_SBHG_CASE(4, true, 16) DELREC_SBHG_CASE(4, true, 24)
    DELREC_SBHG_CASE(4, false, 16) DELREC_SBHG_CASE(4, false, 24)
    return false;
}

// blocks of up to 512 threads (two waves per SIMD, 256 VGPRs: the operand groups stay in
// registers); larger blocks take syn_bwd_kernel
bool launch_syn_bwd_hyb(const SynBwd& a, int block, size_t lds, hipStream_t stream) {
    // up to 512 sources: the split form, two lanes per source (DELREC_SYN_BWD_SPLIT=0: one)
    const char* e = getenv("DELREC_SYN_BWD_SPLIT");
    const bool split = a.N <= 512 && !(e && e[0] == '0');
    if (split) block = 2 * ((a.N + 31) / 32 * 32);
    else if (block > 512) return false;
    const int kt = a.KT;
    const bool wbf = a.w_bf16 != 0;
    DELREC_SBH_CASE(2, false) DELREC_SBH_CASE(2, true) DELREC_SBH_CASE(4, false) DELREC_SBH_CASE(4, true)
    return false;
}

// tap runs compiled for fixed lengths; other lengths take the runtime-count variant (KT = 0)
template <int NPT, bool HYB, int MAXT>
void launch_syn_bwd_kt(const SynBwd& a, int block, size_t lds, hipStream_t stream) {
    if (HYB && a.KT == 2) launch_syn_bwd_k<NPT, 2, HYB, MAXT>(a, block, lds, stream);
    else if (a.KT == 4) launch_syn_bwd_k<NPT, 4, HYB, MAXT>(a, block, lds, stream);
    else if (!HYB && a.KT == 8) launch_syn_bwd_k<NPT, 8, HYB, MAXT>(a, block, lds, stream);
    else if (!HYB && a.KT == 12) launch_syn_bwd_k<NPT, 12, HYB, MAXT>(a, block, lds, stream);
    else launch_syn_bwd_k<NPT, 0, HYB, MAXT>(a, block, lds, stream);
}

// blocks of up to 512 threads get the 256-VGPR variants (two waves per SIMD)
bool launch_syn_bwd(const SynBwd& a, int block, size_t lds, hipStream_t stream) {
    const int npt = (a.N + block - 1) / block;
    const bool hyb = a.offt != nullptr;
    if (npt == 1 && block <= 512) {
        if (hyb) launch_syn_bwd_kt<1, true, 512>(a, block, lds, stream);
        else launch_syn_bwd_kt<1, false, 512>(a, block, lds, stream);
    } else if (npt == 1) {
        if (hyb) launch_syn_bwd_kt<1, true, 1024>(a, block, lds, stream);
        else launch_syn_bwd_kt<1, false, 1024>(a, block, lds, stream);
    } else if (npt == 2) {
        if (hyb) launch_syn_bwd_kt<2, true, 1024>(a, block, lds, stream);
        else launch_syn_bwd_kt<2, false, 1024>(a, block, lds, stream);
    } else {
        if (hyb) launch_syn_bwd_kt<4, true, 1024>(a, block, lds, stream);
        else launch_syn_bwd_kt<4, false, 1024>(a, block, lds, stream);
    }
    return true;
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
