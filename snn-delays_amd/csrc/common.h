// Shared device helpers for the delayed-LIF kernels (gfx950, wave64).
//
// The whole library is compiled with -ffp-contract=off: the LIF charge, the triangle
// weights and the surrogate gradients are evaluated with the same separately rounded
// fp32 operations, in the same order, as the PyTorch scans they must match
// (spikingjelly LIFNode charge forms; reference triton_kernels/lif.py:25-56,
// surrogate.py:21-27, delays.py:13-29). Dot products that may be fused call fmaf().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/delrec.h"

namespace delrec {

constexpr int kWave = 64;

// ---------------------------------------------------------------- LIF neuron ----------

struct Lif {
    float tau, decay, vth, vr;
    int charge_mode;   // 0: v*decay + a   1: v - (v - vr)/tau + a   2: v + (a - v)/tau   3: v + (a - (v - vr))/tau
    int soft, detach, surr;
    float gamma, alpha;
    float v0;          // reset state: v_reset (0 for soft reset)
};

inline Lif make_lif(const delrec_lif& p) {
    Lif k;
    k.tau = p.tau;
    k.decay = p.decay;
    k.vth = p.v_threshold;
    k.vr = p.soft_reset ? 0.0f : p.v_reset;
    const bool reset0 = p.soft_reset || p.v_reset == 0.0f;
    k.charge_mode = p.decay_input ? (reset0 ? 2 : 3) : (reset0 ? 0 : 1);
    k.soft = p.soft_reset;
    k.detach = p.detach_reset;
    k.surr = p.surrogate;
    k.gamma = p.gamma;
    k.alpha = p.alpha;
    k.v0 = p.soft_reset ? 0.0f : p.v_reset;
    return k;
}

// Pre-reset membrane from the post-reset state v and the input a.
__device__ __forceinline__ float lif_charge(const Lif& k, float v, float a) {
    switch (k.charge_mode) {
        case 0: return v * k.decay + a;
        case 1: return (v - (v - k.vr) / k.tau) + a;
        case 2: return v + (a - v) / k.tau;
        default: return v + (a - (v - k.vr)) / k.tau;
    }
}

// Heaviside with H(0) = 1, evaluated as the reference does: (u - v_th) >= 0.
__device__ __forceinline__ float lif_fire(const Lif& k, float u) {
    return (u - k.vth >= 0.0f) ? 1.0f : 0.0f;
}

__device__ __forceinline__ float lif_reset(const Lif& k, float u, float y) {
    if (k.soft) return y != 0.0f ? u - k.vth : u;
    return y != 0.0f ? k.vr : u;
}

__device__ __forceinline__ float surrogate_grad(const Lif& k, float xg) {
    if (k.surr == 0) {
        const float inv = 1.0f / k.gamma;
        return inv * inv * fmaxf(k.gamma - fabsf(xg), 0.0f);
    }
    const float zz = (1.5707963267948966f * k.alpha) * xg;
    return (0.5f * k.alpha) / (1.0f + zz * zz);
}

// dL/du from dL/dy (gY), the carried dL/dv (lam), the saved membrane u and spike y.
__device__ __forceinline__ float lif_backward(const Lif& k, float gY, float u, float y, float lam) {
    const float sg = surrogate_grad(k, u - k.vth);
    if (k.soft) {
        const float gS = k.detach ? gY : gY - k.vth * lam;
        return lam + gS * sg;
    }
    const float gS = k.detach ? gY : gY - lam * (u - k.vr);
    return lam * (1.0f - y) + gS * sg;
}

// dL/dx from dL/du (the charge's input derivative).
__device__ __forceinline__ float lif_dx(const Lif& k, float du) {
    return k.charge_mode >= 2 ? du / k.tau : du;
}

// ---------------------------------------------------------------- triangle taps -------

// h(l; d, s) = max(0, s - |l - (1 + d)|) / (s*s)  (reference Eq. 7, delays.py:28).
__device__ __forceinline__ float tri_weight(float l, float c, float s, float s2) {
    return fmaxf(s - fabsf(l - c), 0.0f) / s2;
}

// d h / d d on the closed support |l - c| <= s with sign(0) = 0, without the 1/s^2.
__device__ __forceinline__ float tri_dsign(float l, float c, float s) {
    const float a = l - c;
    if (fabsf(a) > s) return 0.0f;
    return a > 0.0f ? 1.0f : (a < 0.0f ? -1.0f : 0.0f);
}

// d h / d s as autograd differentiates clamp(s - |l-c|, 0) / (s*s):
// [s - |l-c| >= 0] / s^2 - clamp(s - |l-c|, 0) / (s^2)^2 * 2s.
__device__ __forceinline__ float tri_ds(float l, float c, float s, float s2) {
    const float inner = s - fabsf(l - c);
    if (inner < 0.0f) return 0.0f;
    return 1.0f / s2 - (inner / (s2 * s2)) * (s + s);
}

// First and last integer lag >= 1 whose closed-support derivative may be non-zero:
// |l - c| <= s  ->  l in [ceil(c - s), floor(c + s)].
__device__ __forceinline__ void tap_range(float c, float s, int L, int& lo, int& hi) {
    lo = (int)ceilf(c - s);
    hi = (int)floorf(c + s);
    if (lo < 1) lo = 1;
    if (hi > L - 1) hi = L - 1;
}

// ---------------------------------------------------------------- weights -------------

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ float load_w(const void* W, int bf16, size_t idx) {
    return bf16 ? bf16_to_f32(((const uint16_t*)W)[idx]) : ((const float*)W)[idx];
}

// ---------------------------------------------------------------- wave helpers --------

__device__ __forceinline__ float wave_xor(float v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

}  // namespace delrec
