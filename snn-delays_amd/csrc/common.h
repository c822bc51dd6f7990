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

// First and last integer lag in [1, L-1] on the closed support |l - c| <= s (the lags
// whose weight or derivative may be non-zero), decided with the same fp32 test the
// weight functions use.
__device__ __forceinline__ void tap_range(float c, float s, int L, int& lo, int& hi) {
    lo = (int)ceilf(c - s);
    if (fabsf((float)(lo - 1) - c) <= s) lo -= 1;
    if (fabsf((float)lo - c) > s) lo += 1;
    hi = (int)floorf(c + s);
    if (fabsf((float)(hi + 1) - c) <= s) hi += 1;
    if (fabsf((float)hi - c) > s) hi -= 1;
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

// Fill a register tile t[a][c] = W[i][j] (0 outside the N x N matrix) with idx(a, c, i, j)
// giving the matrix indices. fp32 weights go through a buffer descriptor straight into
// the tile registers (an index outside W reads 0 from the hardware bounds check), so all
// loads are in flight before the first wait; bf16 weights are widened after loading.
template <int R, int C, class Tile, class Idx>
__device__ __forceinline__ void load_w_tile(Tile& t, const void* W, int bf16, int N, Idx idx);

// ---------------------------------------------------------------- buffer addressing ---
// Raw buffer loads / stores through a resource descriptor held in SGPRs: the per-lane
// offset is a VGPR that stays constant across steps while the (uniform) base moves, so
// address arithmetic costs no vector instructions. Accesses at or beyond `bytes` are
// dropped (stores) or return 0 (loads).
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__device__ void raw_buffer_store_f32(float v, i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.store.f32");
__device__ float raw_buffer_load_f32(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.f32");
__device__ uint16_t raw_buffer_load_u16(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i16");
__device__ int8_t raw_buffer_load_i8(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i8");
__device__ i32x4 raw_buffer_load_i32x4(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");

__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)base;
    i32x4 r;
    r.x = (int32_t)(uint32_t)a;
    r.y = (int32_t)((uint32_t)(a >> 32) & 0xffffu);   // stride 0
    r.z = (int32_t)bytes;                              // num_records
    r.w = 0x00020000;                                  // gfx9 family: 32-bit data format
    return r;
}

constexpr int kOutOfRange = 0x7ffffff0;   // a byte offset past every buffer used here

// Descriptor of one time step of a time-major tensor, walked step by step: the base
// address advances by a 64-bit add (device addresses fit in 48 bits, so the high word
// needs no masking against the stride field).
__device__ __forceinline__ i32x4 step_rsrc(uint64_t addr, uint32_t bytes) {
    i32x4 r;
    r.x = (int32_t)(uint32_t)addr;
    r.y = (int32_t)(uint32_t)(addr >> 32);
    r.z = (int32_t)bytes;
    r.w = 0x00020000;
    return r;
}

template <int R, int C, class Tile, class Idx>
__device__ __forceinline__ void load_w_tile(Tile& t, const void* W, int bf16, int N, Idx idx) {
    if (bf16) {
        const uint16_t* Wh = (const uint16_t*)W;
#pragma unroll
        for (int a = 0; a < R; ++a)
#pragma unroll
            for (int c = 0; c < C; ++c) {
                int i, j;
                idx(a, c, i, j);
                const bool ok = i < N && j < N;
                const float v = bf16_to_f32(Wh[ok ? (size_t)i * N + j : 0]);
                t[a][c] = ok ? v : 0.0f;
            }
    } else {
        const i32x4 rs = buffer_rsrc(W, (uint32_t)((size_t)N * N * 4u));
#pragma unroll
        for (int a = 0; a < R; ++a)
#pragma unroll
            for (int c = 0; c < C; ++c) {
                int i, j;
                idx(a, c, i, j);
                const int off = (i < N && j < N) ? (i * N + j) * 4 : kOutOfRange;
                t[a][c] = raw_buffer_load_f32(rs, off, 0, 0);
            }
    }
}

// ---------------------------------------------------------------- wave helpers --------

__device__ __forceinline__ float wave_xor(float v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G consecutive lanes (G a power of two); every lane of the
// group receives the total. DPP quad permutes / row mirrors for G <= 16.
__device__ __forceinline__ float group_sum(float v, int G) {
    if (G >= 2) v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    if (G >= 4) v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    if (G >= 8) v += dpp<0x141>(v);   // row_half_mirror: other quad of the 8-lane half row
    if (G >= 16) v += dpp<0x140>(v);  // row_mirror: other half of the 16-lane row
    if (G >= 32) v += wave_xor(v, 16);
    if (G >= 64) v += wave_xor(v, 32);
    return v;
}

// Workgroup barrier that orders LDS only: outstanding global loads (prefetches) and
// stores stay in flight across it. Every LDS access that must be visible to other
// waves is complete (lgkmcnt 0) before the barrier.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Compile-time group width: no runtime branches in the reduction.
template <int G>
__device__ __forceinline__ float group_sum_t(float v) {
    if constexpr (G >= 2) v += dpp<0xB1>(v);
    if constexpr (G >= 4) v += dpp<0x4E>(v);
    if constexpr (G >= 8) v += dpp<0x141>(v);
    if constexpr (G >= 16) v += dpp<0x140>(v);
    if constexpr (G >= 32) v += wave_xor(v, 16);
    if constexpr (G >= 64) v += wave_xor(v, 32);
    return v;
}

constexpr int kMaxTaps = 8;   // register-resident tap weights per neuron (fast path)

// max(x[0 .. n)) over the workgroup (NaN when an element is NaN, as torch.max), written by
// thread 0 with `ticket` into a slot of host memory, (ticket | value bits << 32), as one
// 8-byte system-scope store: a host reader sees either the old pair or the new one. Every
// thread of the workgroup (a multiple of 64 threads, at most 1024) calls it: it holds a
// barrier.
// With `poison` the posted value is NaN whatever x holds (a caller that found the
// maximum unusable, e.g. a window its kernel cannot hold).
__device__ __forceinline__ void block_max_to_host(const float* x, int n, uint32_t ticket,
                                                  unsigned long long* slot, bool poison = false) {
    __shared__ float wmax[16];
    float m = -INFINITY;
    int nan = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i];
        nan |= v != v;
        m = fmaxf(m, v);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    nan = __syncthreads_or(nan);
    if (threadIdx.x == 0) {
        float r = wmax[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, wmax[w]);
        if (nan || poison) r = __builtin_nanf("");
        const unsigned long long v = (unsigned long long)ticket | ((unsigned long long)__float_as_uint(r) << 32);
        __hip_atomic_store(slot, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace delrec
