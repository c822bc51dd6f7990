// The loss end of the SNN_* stacks, fused: the readout Linear's output (T, B, C) reduced over
// time -- summed (reference utils.py calc_loss_SSC), averaged (calc_loss_HAR / calc_loss_AL)
// or its maximum (calc_loss_SHD) -- optionally after a non-spiking leaky integrator (the SHD
// stack's LIF readout with an unreachable threshold, networks_shd.py:187-199), then the
// cross-entropy against the labels, averaged over the batch (torch.nn.CrossEntropyLoss), and
// in the same pass the gradient of that loss with respect to the readout's output.
//
// One workgroup per batch row: the classes on the threads, each thread walks its classes'
// time series forward (integrator, reduction, first maximum), the softmax over the classes is
// a workgroup reduction, and the gradient walks the series backward: for the integrator
// v_t = a v_{t-1} + c x_t, d(reduce)/d x_s = c sum_{t >= s} a^(t - s) d(reduce)/d v_t.
// A second single-workgroup launch averages the rows' losses in a fixed order.
#include "kernels.h"

namespace delrec {

namespace {

constexpr int kReadoutBlock = 256;

__device__ __forceinline__ float ro_block_reduce(float v, float* red, bool is_max) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float u = __shfl_xor(v, o);
        v = is_max ? fmaxf(v, u) : v + u;
    }
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (int q = 1; q < kReadoutBlock / 64; ++q) r = is_max ? fmaxf(r, red[q]) : r + red[q];
    return r;
}

}  // namespace

__global__ void __launch_bounds__(kReadoutBlock) readout_ce_kernel(ReadoutCe p) {
    extern __shared__ float smem[];
    float* red = smem;                     // [4] reduction scratch
    float* outc = smem + 4;                // [C] the reduced readout of this row
    const int b = blockIdx.x, tid = threadIdx.x;
    const int T = p.T, B = p.B, C = p.C;
    const size_t row = (size_t)B * C;
    const float a = p.decay, cin = p.in_scale;
    // forward: per class, the integrator and the time reduction (first maximum and its step)
    float mloc = -__builtin_inff();
    for (int c = tid; c < C; c += kReadoutBlock) {
        const float* x = p.logits + (size_t)b * C + c;
        float v = 0.0f, acc = 0.0f, best = -__builtin_inff();
        for (int t = 0; t < T; ++t) {
            const float xt = x[(size_t)t * row];
            if (p.integrator == 1) v = v * a + xt;
            else if (p.integrator == 2) v = v + (xt - v) / p.tau;
            else v = xt;
            if (p.reduce == DELREC_READOUT_MAX) {
                if (v > best) best = v;
            } else {
                acc += v;
            }
        }
        const float o = p.reduce == DELREC_READOUT_MAX ? best : (p.reduce == DELREC_READOUT_MEAN ? acc / (float)T : acc);
        outc[c] = o;
        if (p.out) p.out[(size_t)b * C + c] = o;
        mloc = fmaxf(mloc, o);
    }
    const float mx = ro_block_reduce(mloc, red, true);
    float sloc = 0.0f;
    for (int c = tid; c < C; c += kReadoutBlock) sloc += expf(outc[c] - mx);
    const float se = ro_block_reduce(sloc, red, false);
    const float lse = mx + logf(se);
    const int64_t lab = p.labels[b];
    if (tid == 0) p.rowloss[b] = (lab >= 0 && lab < C) ? lse - outc[lab] : __builtin_nanf("");
    // backward: d loss / d out_c = (softmax_c - [c == label]) / B, then back through the
    // reduction and the integrator, latest step first
    for (int c = tid; c < C; c += kReadoutBlock) {
        const float gout = (expf(outc[c] - lse) - (c == lab ? 1.0f : 0.0f)) / (float)B;
        const float* x = p.logits + (size_t)b * C + c;
        float* dx = p.dlogits + (size_t)b * C + c;
        int tmax = -1;
        if (p.reduce == DELREC_READOUT_MAX) {      // the step of the first maximum
            float v = 0.0f, best = -__builtin_inff();
            for (int t = 0; t < T; ++t) {
                const float xt = x[(size_t)t * row];
                if (p.integrator == 1) v = v * a + xt;
                else if (p.integrator == 2) v = v + (xt - v) / p.tau;
                else v = xt;
                if (v > best) { best = v; tmax = t; }
            }
        }
        const float gv = p.reduce == DELREC_READOUT_MEAN ? gout / (float)T : gout;
        float lam = 0.0f;                           // d loss / d v_t carried from t + 1
        for (int t = T - 1; t >= 0; --t) {
            const float dv = (p.reduce == DELREC_READOUT_MAX ? (t == tmax ? gout : 0.0f) : gv) + lam;
            dx[(size_t)t * row] = p.integrator ? dv * cin : dv;
            lam = p.integrator ? dv * a : 0.0f;
        }
    }
}

__global__ void __launch_bounds__(kReadoutBlock) readout_mean_kernel(ReadoutCe p) {
    __shared__ float red[4];
    float s = 0.0f;
    for (int b = threadIdx.x; b < p.B; b += kReadoutBlock) s += p.rowloss[b];
    const float tot = ro_block_reduce(s, red, false);
    if (threadIdx.x == 0) p.loss[0] = tot / (float)p.B;
}

void launch_readout_ce(const ReadoutCe& p, hipStream_t stream) {
    const size_t lds = (size_t)(4 + p.C) * sizeof(float);
    ensure_lds((const void*)readout_ce_kernel, lds);
    hipLaunchKernelGGL(readout_ce_kernel, dim3(p.B), dim3(kReadoutBlock), lds, stream, p);
    hipLaunchKernelGGL(readout_mean_kernel, dim3(1), dim3(kReadoutBlock), 0, stream, p);
}

}  // namespace delrec
