// The Linear layer that follows a recurrent delayed-LIF layer in the SNN_* stacks
// (torch.nn.Linear in the Sequential of reference networks.py:140-181, applied to the
// layer's spike output), as a binary-activation GEMM on bf16 MFMA (gfx950):
//   out[t][b][m] = bias[m] + sum_k y[t][b][k] * W[m][k],   y in {0, 1},
// read straight from the scans' spike bits (B, ceil(T/32), K) -- 1/32 of the fp32 spikes.
//
// The spikes are exact in bf16; W^T is split into bf16 hi + mid + lo planes (about 2^-25
// relative per weight, below fp32's own rounding; accumulation fp32), so each tile takes
// three products. A workgroup owns 128 consecutive steps of one batch row (four 32-step
// spike words per neuron) by 128 output columns: per 32-neuron stage it stages the 4 x 32
// spike words and the W planes' 32 x 128 blocks in LDS, and each lane expands its A fragment
// (16 rows x 8 neurons) from the words.
#include "kernels.h"

#include <algorithm>

namespace delrec {

namespace {

typedef float sl_floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 sl_bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t sl_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

constexpr int kSpikeLinearPlanes = 3;

}  // namespace

// W^T planes, k-blocked: element (k, m) = W[m][k'] at ((k / 8) * Mp + m) * 8 + k % 8, hi, mid
// and lo planes in turn, k' = perm[k] (k without an order); columns m >= M and rows without a
// neuron are 0.
__global__ void __launch_bounds__(256) spike_linear_pack_kernel(SpikeLinear p, uint4* out) {
    const size_t total = (size_t)(p.Kp / 8) * p.Mp;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int kb = (int)(idx / p.Mp), m = (int)(idx - (size_t)kb * p.Mp);
    uint32_t pl[kSpikeLinearPlanes][4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        uint32_t v2[kSpikeLinearPlanes][2];
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            const int kp = kb * 8 + e + f;
            const int k = p.perm ? p.perm[kp] : kp;
            float r = (m < p.M && k >= 0 && k < p.K) ? p.W[(size_t)m * p.K + k] : 0.0f;
#pragma unroll
            for (int q = 0; q < kSpikeLinearPlanes; ++q) {   // each plane the remainder's bf16
                v2[q][f] = sl_bf16_rne(r);
                r -= __uint_as_float(v2[q][f] << 16);
            }
        }
#pragma unroll
        for (int q = 0; q < kSpikeLinearPlanes; ++q) pl[q][e / 2] = v2[q][0] | (v2[q][1] << 16);
    }
#pragma unroll
    for (int q = 0; q < kSpikeLinearPlanes; ++q)
        out[q * total + idx] = uint4{pl[q][0], pl[q][1], pl[q][2], pl[q][3]};
}

// Tile: 128 steps t0 .. t0 + 127 of batch row b x 128 columns n0 .. n0 + 127; 4 waves of
// 64 x 64 (4 x 4 MFMA blocks, three W planes). Stage s covers neuron positions 32 s .. 32 s +
// 31; with an activity order the stages wholly below the first spiking neuron are skipped
// (their spike words are all 0). Loads of stage s + 2 are issued while stage s multiplies;
// stage s + 1 goes to LDS after it; one barrier per stage.
__global__ void __launch_bounds__(256) spike_linear_kernel(SpikeLinear p, const uint4* wp) {
    constexpr int PL = kSpikeLinearPlanes;
    __shared__ uint4 sw[2][PL][512];     // [buffer][plane][k-block * 128 + column]
    __shared__ __align__(16) uint32_t sa[2][4][32];   // [buffer][32-step word][neuron of the stage]
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const int NT = p.Mp / 128, TT = (p.T + 127) / 128, TW = (p.T + 31) >> 5;
    const int id = (int)blockIdx.x;
    const int nt = id % NT, rest = id / NT, tt = rest % TT, b = rest / TT;
    const int t0 = tt * 128, n0 = nt * 128;
    const int nst = p.Kp / 32;
    const int s0 = p.cls ? min(p.cls[0] / 32, nst) : 0;
    const size_t plane = (size_t)(p.Kp / 8) * p.Mp;
    const i32x4 rw = buffer_rsrc(wp, (uint32_t)(PL * plane * 16));
    const i32x4 rb = buffer_rsrc(p.bits, (uint32_t)((size_t)p.B * TW * p.ldb * 4));
    // staging: W uint4 c = tid + 256 h (k-block c >> 7, column c & 127) of both planes; the
    // spike word of (32-step block tid >> 5, neuron tid & 31) for threads below 128
    uint32_t ow[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int c = tid + 256 * h, kb = c >> 7, col = c & 127;
        ow[h] = (uint32_t)(((size_t)kb * p.Mp + n0 + col) * 16);
    }
    const uint32_t wstep = (uint32_t)(4 * p.Mp * 16);
    const int tb = tid >> 5, kk = tid & 31;
    const bool aload = tid < 128 && (t0 >> 5) + tb < TW;
    const uint32_t oa0 = aload ? (uint32_t)((((size_t)b * TW + (t0 >> 5) + tb) * p.ldb + kk) * 4) : 0x7ffffff0u;
    uint4 rwv[2][PL][2];   // [register set][plane][h]
    uint32_t rav[2];
    auto issue = [&](int set, int s) {
#pragma unroll
        for (int q = 0; q < PL; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                rwv[set][q][h] = __builtin_bit_cast(
                    uint4, raw_buffer_load_i32x4(rw, (int)(ow[h] + (uint32_t)s * wstep + (uint32_t)q * (uint32_t)(plane * 16)), 0, 0));
        // neurons past K read past the row: another neuron's word, weighted by the zero rows
        // of W's padding -- unless past the buffer, which reads 0
        rav[set] = __float_as_uint(raw_buffer_load_f32(rb, aload ? (int)(oa0 + (uint32_t)s * 128u) : 0x7ffffff0, 0, 0));
    };
    auto stash = [&](int set, int buf) {
#pragma unroll
        for (int q = 0; q < PL; ++q)
#pragma unroll
            for (int h = 0; h < 2; ++h) sw[buf][q][tid + 256 * h] = rwv[set][q][h];
        if (tid < 128) sa[buf][tb][kk] = rav[set];
    };
    sl_floatx4 acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = sl_floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int buf) {
        sl_bf16x8 fa[4], fb[PL][4];
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int q = 0; q < PL; ++q)
                fb[q][x] = __builtin_bit_cast(sl_bf16x8, sw[buf][q][g * 128 + wj * 64 + x * 16 + lc]);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int row = wi * 64 + mb * 16 + lc;   // step t0 + row
            const uint4* src = reinterpret_cast<const uint4*>(&sa[buf][row >> 5][g * 8]);
            const uint4 w0 = src[0], w1 = src[1];
            const int bit = row & 31;
            const uint32_t wd[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            uint32_t pk[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t a0 = ((wd[2 * e] >> bit) & 1u) * 0x3F80u;       // bf16 1.0 or 0
                const uint32_t a1 = ((wd[2 * e + 1] >> bit) & 1u) * 0x3F80u;
                pk[e] = a0 | (a1 << 16);
            }
            fa[mb] = __builtin_bit_cast(sl_bf16x8, uint4{pk[0], pk[1], pk[2], pk[3]});
        }
#pragma unroll
        for (int q = 0; q < PL; ++q)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int nb = 0; nb < 4; ++nb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[mb], fb[q][nb], acc[mb][nb], 0, 0, 0);
    };

    issue(0, s0);
    issue(1, s0 + 1);
    stash(0, 0);
    barrier_lds();
    for (int s = s0; s < nst; s += 2) {
        // stage s in LDS buffer 0, stage s + 1 in register set 1
        issue(0, s + 2);
        compute(0);
        stash(1, 1);
        barrier_lds();
        if (s + 1 >= nst) break;
        issue(1, s + 3);
        compute(1);
        stash(0, 0);
        barrier_lds();
    }

    // epilogue: rows t = t0 + wi * 64 + mb * 16 + 4 g + e, columns n0 + wj * 64 + nb * 16 + lc
    float bv[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
        const int m = n0 + wj * 64 + nb * 16 + lc;
        bv[nb] = (p.bias && m < p.M) ? p.bias[m] : 0.0f;
    }
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + wi * 64 + mb * 16 + 4 * g + e;
            if (t >= p.T) continue;
            float* o = p.out + ((size_t)t * p.B + b) * p.M;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) {
                const int m = n0 + wj * 64 + nb * 16 + lc;
                if (m < p.M) o[m] = acc[mb][nb][e] + bv[nb];
            }
        }
}

// g (T, B, M) fp32 into bf16 hi + mid + lo planes [plane][b][32-step word][8-step block][m]
// (8 steps of one output per uint4; steps past T are 0), once per call, so the K / 128 input
// tiles of the weight gradient stage the planes as they are instead of each splitting g
// again. One thread per (b, word, block, m).
// The input gradient dy = g W as one bf16 GEMM: each row of g (M fp32) becomes 3M bf16,
// [hi | lo | hi] with hi = bf16(x) and lo = bf16(x - hi), so that against W stacked as
// [W_hi; W_hi; W_lo] (3M x K) the product sums g_hi W_hi + g_lo W_hi + g_hi W_lo (about 2^-16
// relative per product, the missing g_lo W_lo included). One thread per 4 consecutive
// elements of a row (16-byte loads and 8-byte stores when M is a multiple of 4).
__global__ void __launch_bounds__(256) spike_linear_dx_split_kernel(const float* __restrict__ g, size_t rows, int M,
                                                                    uint16_t* __restrict__ out) {
    const int M4 = (M + 3) / 4;
    const size_t total = rows * (size_t)M4;
    const bool vec = (M & 3) == 0;
    for (size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += (size_t)gridDim.x * blockDim.x) {
        const size_t r = id / M4;
        const int m = (int)(id - r * M4) * 4;
        const float* src = g + r * M + m;
        uint16_t* dst = out + r * 3 * (size_t)M + m;
        if (vec) {
            const float4 v = *reinterpret_cast<const float4*>(src);
            const float x[4] = {v.x, v.y, v.z, v.w};
            uint32_t h[4], l[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h[e] = sl_bf16_rne(x[e]);
                l[e] = sl_bf16_rne(x[e] - __uint_as_float(h[e] << 16));
            }
            const uint2 hv = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
            *reinterpret_cast<uint2*>(dst) = hv;
            *reinterpret_cast<uint2*>(dst + M) = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
            *reinterpret_cast<uint2*>(dst + 2 * (size_t)M) = hv;
        } else {
            for (int e = 0; e < 4 && m + e < M; ++e) {
                const float x = src[e];
                const uint32_t h = sl_bf16_rne(x), l = sl_bf16_rne(x - __uint_as_float(h << 16));
                dst[e] = (uint16_t)h;
                dst[M + e] = (uint16_t)l;
                dst[2 * (size_t)M + e] = (uint16_t)h;
            }
        }
    }
}

void launch_spike_linear_dx_split(const float* g, size_t rows, int M, uint16_t* out, hipStream_t stream) {
    const size_t total = rows * (size_t)((M + 3) / 4);
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, (size_t)65535 * 8);
    hipLaunchKernelGGL(spike_linear_dx_split_kernel, dim3(blocks), dim3(256), 0, stream, g, rows, M, out);
}

__global__ void __launch_bounds__(256) spike_linear_gsplit_kernel(SpikeLinearDw p) {
    const int TW = (p.T + 31) >> 5;
    const size_t total = (size_t)p.B * TW * 4 * p.M;
    const size_t gstep = (size_t)p.B * p.M;
    for (size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(id % p.M);
        const size_t r = id / p.M;
        const int h = (int)(r & 3), wd = (int)((r >> 2) % TW), b = (int)(r / (4 * (size_t)TW));
        const int t0 = wd * 32 + 8 * h;
        uint32_t pl[kSpikeLinearPlanes][4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t v2[kSpikeLinearPlanes][2];
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                const int t = t0 + e + f;
                float v = t < p.T ? p.g[(size_t)t * gstep + (size_t)b * p.M + m] : 0.0f;
#pragma unroll
                for (int q = 0; q < kSpikeLinearPlanes; ++q) {
                    v2[q][f] = sl_bf16_rne(v);
                    v -= __uint_as_float(v2[q][f] << 16);
                }
            }
#pragma unroll
            for (int q = 0; q < kSpikeLinearPlanes; ++q) pl[q][e / 2] = v2[q][0] | (v2[q][1] << 16);
        }
        const size_t plane = (size_t)p.B * TW * 4 * p.M;
#pragma unroll
        for (int q = 0; q < kSpikeLinearPlanes; ++q) p.gp[q * plane + id] = make_uint4(pl[q][0], pl[q][1], pl[q][2], pl[q][3]);
    }
}

// The weight gradient of that Linear, dW[m][k] = sum_{t,b} g[t][b][m] * y[t][b][k], as the
// same binary-activation GEMM with the spikes on the other side: D = g^T (M x TB) . Y (TB x K).
// The contraction runs over stages of 32 steps of one batch row -- exactly one spike word per
// neuron -- so each lane expands its B fragment (8 steps of one neuron) from one word; g^T is
// split into bf16 hi + mid + lo planes (about 2^-25 relative, fp32 accumulation) before it.
// Tile: 128 outputs m x 256 inputs k per workgroup, 4 waves of 64 x 128; stages of a split in
// (batch row, word) order; loads of stage s + 1 in flight while stage s multiplies. The
// stages are split so that about two workgroups run per CU (one stage in flight each hides
// too little load latency: 23 ms at C5's 2048 x 2048 x 524288 with one, 12.5 ms with two);
// the input tiles of one output tile and split sit on one XCD, where they stream the same g
// columns from its L2. A 128 x 128 tile at two per CU takes 15 ms there.
__global__ void __launch_bounds__(256) spike_linear_dw_kernel(SpikeLinearDw p) {
    constexpr int PL = kSpikeLinearPlanes;
    __shared__ uint4 sa[2][PL][4 * 128];     // [buffer][plane][r-block * 128 + m]: 8 steps of g^T
    __shared__ uint32_t sb[2][256];          // [buffer][k]: the stage's spike words
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, g = lane >> 4, lc = lane & 15;
    const int MT = p.Mp / 128, KT = p.Kp / 256, TW = (p.T + 31) >> 5;
    const int id = (int)blockIdx.x;
    int mt, kt, ks;
    if (MT % 8 == 0) {
        // the input tiles of an output tile (and of one split) on one XCD: they stream the
        // same g columns, so all but the first read them from that XCD's L2
        const int xcd = id & 7, slot = id >> 3, rest = slot / KT;
        kt = slot - rest * KT;
        mt = xcd + 8 * (rest % (MT / 8));
        ks = rest / (MT / 8);
    } else {
        ks = id % p.KS;
        const int tile = id / p.KS;
        mt = tile / KT;
        kt = tile - mt * KT;
    }
    const int m0 = mt * 128, k0 = kt * 256;
    const int nst = p.B * TW;
    const int per = (nst + p.KS - 1) / p.KS;
    const int s0 = ks * per, s1 = min(nst, s0 + per);
    // staging: g^T from its three bf16 planes (split once by spike_linear_gsplit_kernel) --
    // uint4 u = tid + 256 x: plane u / 512, 8-step block (u / 128) % 4, output m = m0 + u % 128;
    // spikes -- thread tid loads the word of input k0 + tid
    uint4 rg[6];
    uint32_t rb = 0;
    auto issue = [&](int s) {
        const int b = s / TW, wd = s - b * TW;
#pragma unroll
        for (int x = 0; x < 6; ++x) {
            const int u = tid + 256 * x, q = u >> 9, h = (u >> 7) & 3, m = m0 + (u & 127);
            rg[x] = (s < s1 && m < p.M) ? p.gp[((((size_t)q * p.B + b) * TW + wd) * 4 + h) * p.M + m] : make_uint4(0u, 0u, 0u, 0u);
        }
        rb = (s < s1 && k0 + tid < p.ldb) ? p.bits[((size_t)b * TW + wd) * p.ldb + k0 + tid] : 0u;
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int x = 0; x < 6; ++x) {
            const int u = tid + 256 * x;
            sa[buf][u >> 9][((u >> 7) & 3) * 128 + (u & 127)] = rg[x];
        }
        sb[buf][tid] = rb;
    };
    sl_floatx4 acc[4][8];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) acc[mb][nb] = sl_floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf) {
        sl_bf16x8 fb[8];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {      // input k = k0 + wj 128 + nb 16 + lc, steps 8 g .. 8 g + 7
            const uint32_t wd = sb[buf][wj * 128 + nb * 16 + lc] >> (8 * g);
            uint32_t pk[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                pk[e] = (((wd >> (2 * e)) & 1u) * 0x3F80u) | ((((wd >> (2 * e + 1)) & 1u) * 0x3F80u) << 16);
            fb[nb] = __builtin_bit_cast(sl_bf16x8, uint4{pk[0], pk[1], pk[2], pk[3]});
        }
#pragma unroll
        for (int q = 0; q < PL; ++q)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const sl_bf16x8 fa = __builtin_bit_cast(sl_bf16x8, sa[buf][q][g * 128 + wi * 64 + mb * 16 + lc]);
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa, fb[nb], acc[mb][nb], 0, 0, 0);
            }
    };
    // a tile of silent input neurons (activity order) has dW = 0: no stages
    const int se = (p.cls && k0 + 256 <= p.cls[0]) ? s0 : s1;
    issue(s0);
    stash(0);
    barrier_lds();
    for (int s = s0; s < se; ++s) {
        const int buf = (s - s0) & 1;
        issue(s + 1);                 // past s1: zeros (no load)
        compute(buf);
        stash(buf ^ 1);
        barrier_lds();
    }
    // rows m = m0 + wi 64 + mb 16 + 4 g + e, column positions k0 + wj 128 + nb 16 + lc (the
    // input neurons perm[.] with an order)
    float* out = p.KS == 1 ? p.dW : p.part + (size_t)ks * p.M * p.K;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int m = m0 + wi * 64 + mb * 16 + 4 * g + e;
            if (m >= p.M) continue;
#pragma unroll
            for (int nb = 0; nb < 8; ++nb) {
                const int kp = k0 + wj * 128 + nb * 16 + lc;
                const int k = p.perm ? p.perm[kp] : kp;
                if (k >= 0 && k < p.K) out[(size_t)m * p.K + k] = acc[mb][nb][e];
            }
        }
}

// dW = sum over the splits of the partials, in split order
__global__ void __launch_bounds__(256) spike_linear_dw_sum_kernel(SpikeLinearDw p) {
    const size_t n = (size_t)p.M * p.K;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (size_t)gridDim.x * blockDim.x) {
        float v = 0.0f;
        for (int ks = 0; ks < p.KS; ++ks) v += p.part[(size_t)ks * n + q];
        p.dW[q] = v;
    }
}

void spike_linear_dw_dims(SpikeLinearDw& p, int cus) {
    p.Mp = (p.M + 127) / 128 * 128;
    p.Kp = (p.K + 255) / 256 * 256;
    const int tiles = (p.Mp / 128) * (p.Kp / 256);
    const int nst = p.B * ((p.T + 31) >> 5);
    // about four workgroups per CU when every tile works (two fit a CU at a time), so that the
    // tiles of spiking inputs alone -- those of silent inputs end at once -- still keep about
    // two per CU at C5's first layer (30 % spiking); >= 16 stages a split
    p.KS = std::max(1, std::min((4 * cus + tiles - 1) / tiles, std::max(1, nst / 16)));
}

size_t spike_linear_dw_ws(int T, int B, int K, int M, int cus) {
    SpikeLinearDw p{};
    p.T = T; p.B = B; p.K = K; p.M = M;
    spike_linear_dw_dims(p, cus);
    const size_t planes = (size_t)kSpikeLinearPlanes * B * ((T + 31) / 32) * 4 * M * sizeof(uint4);
    return planes + 256 + (p.KS > 1 ? (size_t)p.KS * M * K * sizeof(float) : 0);
}

size_t spike_linear_dw_planes(int T, int B, int M) {
    return (size_t)kSpikeLinearPlanes * B * ((T + 31) / 32) * 4 * M;
}

void launch_spike_linear_dw(const SpikeLinearDw& p, hipStream_t stream) {
    const size_t items = (size_t)p.B * ((p.T + 31) / 32) * 4 * p.M;
    hipLaunchKernelGGL(spike_linear_gsplit_kernel, dim3((unsigned)std::min<size_t>((items + 255) / 256, 65536)),
                       dim3(256), 0, stream, p);
    const unsigned grid = (unsigned)((p.Mp / 128) * (p.Kp / 256) * p.KS);
    hipLaunchKernelGGL(spike_linear_dw_kernel, dim3(grid), dim3(256), 0, stream, p);
    if (p.KS > 1) hipLaunchKernelGGL(spike_linear_dw_sum_kernel, dim3(1024), dim3(256), 0, stream, p);
}

void spike_linear_dims(SpikeLinear& p) {
    p.Kp = (p.K + 31) / 32 * 32;
    p.Mp = (p.M + 127) / 128 * 128;
}

size_t spike_linear_ws(int K, int M) {
    SpikeLinear p{};
    p.K = K;
    p.M = M;
    spike_linear_dims(p);
    return (size_t)kSpikeLinearPlanes * (p.Kp / 8) * p.Mp * sizeof(uint4);
}

// ---------------------------------------------------------------------------------------
// Input neurons in activity order: cnt[k] = 1 where neuron k spikes anywhere (cnt[KP ..] stay
// 0: no second class), the column order of the event-driven lag correlation (silent first,
// stably), and the spike words regathered in that order.
__global__ void spike_active_kernel(const uint32_t* __restrict__ bits, size_t rows, int K, int* __restrict__ cnt) {
    const size_t n = rows * K;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (size_t)gridDim.x * blockDim.x)
        if (bits[q]) cnt[q % K] = 1;   // every writer stores the same value
}

__global__ void spike_zero_kernel(int* __restrict__ p, int n) {
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < n; q += gridDim.x * blockDim.x) p[q] = 0;
}

__global__ void spike_gather_kernel(const uint32_t* __restrict__ bits, size_t rows, int K, int KP,
                                    const int* __restrict__ perm, uint32_t* __restrict__ out) {
    const size_t n = rows * KP;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < n; q += (size_t)gridDim.x * blockDim.x) {
        const int kp = (int)(q % KP);
        const int k = perm[kp];
        out[q] = k >= 0 ? bits[(q / KP) * K + k] : 0u;
    }
}

int spike_order_kp(int K) { return (K + 255) / 256 * 256; }

namespace {
size_t sl_up(size_t v) { return (v + 255) / 256 * 256; }
}

size_t spike_order_ws(int T, int B, int K) {
    const size_t KP = spike_order_kp(K), rows = (size_t)B * ((T + 31) / 32);
    return sl_up(2 * KP * sizeof(int)) + sl_up(KP * sizeof(int)) + 256 + sl_up(rows * KP * sizeof(uint32_t));
}

SpikeOrder spike_order_carve(void* base, int T, int B, int K) {
    const size_t KP = spike_order_kp(K);
    char* c = static_cast<char*>(base);
    SpikeOrder o;
    o.cnt = reinterpret_cast<int*>(c);
    c += sl_up(2 * KP * sizeof(int));
    o.perm = reinterpret_cast<int*>(c);
    c += sl_up(KP * sizeof(int));
    o.cls = reinterpret_cast<int*>(c);
    c += 256;
    o.bits = reinterpret_cast<uint32_t*>(c);
    (void)T;
    (void)B;
    return o;
}

void launch_spike_order(const uint32_t* bits, int T, int B, int K, const SpikeOrder& o, hipStream_t stream) {
    const int KP = spike_order_kp(K);
    const size_t rows = (size_t)B * ((T + 31) / 32);
    hipLaunchKernelGGL(spike_zero_kernel, dim3((2 * KP + 255) / 256), dim3(256), 0, stream, o.cnt, 2 * KP);
    const unsigned blocks = (unsigned)std::min<size_t>((rows * K + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(spike_active_kernel, dim3(blocks), dim3(256), 0, stream, bits, rows, K, o.cnt);
    launch_col_order(o.cnt, K, KP, o.perm, o.cls, stream);
    const unsigned gblocks = (unsigned)std::min<size_t>((rows * KP + 255) / 256, 65535u * 4);
    hipLaunchKernelGGL(spike_gather_kernel, dim3(gblocks), dim3(256), 0, stream, bits, rows, K, KP, o.perm, o.bits);
}

void launch_spike_linear(const SpikeLinear& p, uint4* wp, hipStream_t stream) {
    const size_t total = (size_t)(p.Kp / 8) * p.Mp;
    hipLaunchKernelGGL(spike_linear_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, p, wp);
    const unsigned grid = (unsigned)((size_t)p.B * ((p.T + 127) / 128) * (p.Mp / 128));
    hipLaunchKernelGGL(spike_linear_kernel, dim3(grid), dim3(256), 0, stream, p, (const uint4*)wp);
}

}  // namespace delrec
