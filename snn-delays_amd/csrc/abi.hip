// extern "C" entry points of libdelrec_hip.so (declared in include/delrec.h).
//
// Host side only: argument validation, workspace carving, launch-shape selection and
// kernel launches on the caller's stream. Nothing here allocates device memory or
// synchronises the stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <initializer_list>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "kernels.h"

using namespace delrec;

namespace {

constexpr size_t kAlign = 256;

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Carver {
    char* base;
    size_t cap, used = 0;
    Carver(void* p, size_t c) : base(static_cast<char*>(p)), cap(c) {}
    template <class T>
    T* take(size_t count) {
        const size_t bytes = align_up(count * sizeof(T));
        if (!base || used + bytes > cap) return nullptr;
        T* out = reinterpret_cast<T*>(base + used);
        used += bytes;
        return out;
    }
};

// Sizes only (no pointers): mirrors Carver so query_workspace and the entry points agree.
struct Counter {
    size_t used = 0;
    template <class T>
    void take(size_t count) { used += align_up(count * sizeof(T)); }
};

// dynamic LDS a launch may request: the per-workgroup limit less 1 KB, which holds the
// kernels' own static LDS (a __syncthreads_or takes 256 bytes)
int max_lds_bytes() {
    static const int cached = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            v = 65536;
        return v - 1024;
    }();
    return cached;
}

int num_cus() {
    static const int cached = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            v = 256;
        return v;
    }();
    return cached;
}

int finish_launch() {
    return hipGetLastError() == hipSuccess ? DELREC_OK : DELREC_ERR_LAUNCH;
}

bool lif_ok(const delrec_lif& l) {
    if (!(l.tau > 0.0f)) return false;
    if (l.surrogate != 0 && l.surrogate != 1) return false;
    if (l.surrogate == 0 && !(l.gamma > 0.0f)) return false;
    return true;
}

// ------------------------------------------------------------------ axonal layout ------
struct AxLayout {
    bool res;       // N <= 256: tiled kernels with W resident in VGPRs
    int G, CH, CHS, NZ, block, hw, ri;
    int np;         // padded neuron count of the tiled kernels' per-neuron LDS rows
};

bool axonal_layout(int N, int L, AxLayout& o) {
    const int lags = std::max(L - 1, 1);
    if (lags <= 64) o.hw = 1;
    else if (lags <= 128) o.hw = 2;
    else if (lags <= 256) o.hw = 4;
    else return false;
    if (N <= 256) {
        // CJ sources per lane chunk (32 for 128 < N <= 256: 4 x 32 tiles reduce over 8-lane
        // groups; DELREC_AXONAL_CJ=16 selects the 8 x 16 tiles), NJ chunk lanes per receiver
        // group (a power of two), RI receivers per lane with RI <= NJ: neuron i runs on lane
        // (i / RI, i % RI) of its own group.
        int cj = N > 128 ? 32 : 16;
        if (const char* e = getenv("DELREC_AXONAL_CJ"))
            if (atoi(e) == 16) cj = 16;
        int nj = 1;
        while (nj * cj < N) nj <<= 1;
        int ri = 1;
        if (cj == 32) {
            ri = 4;
        } else {
            // the smallest RI whose lanes fit the block (kernels with RI >= 4 run at most 512
            // threads, TiledThreads in axonal.hip)
            while (ri < 8 && ((N + ri - 1) / ri) * nj > (ri >= 4 ? 512 : 1024)) ri <<= 1;
            if (ri == 4 && nj == 16) ri = 8;
            if (const char* e = getenv("DELREC_AXONAL_RI")) {
                const int want = atoi(e);
                if (nj == 16 && (want == 2 || want == 4 || want == 8) &&
                    ((N + want - 1) / want) * nj <= (want >= 4 ? 512 : 1024))
                    ri = want;
            }
        }
        const int lanes = ((N + ri - 1) / ri) * nj;
        if (lanes > (ri >= 4 ? 512 : 1024) || ri > nj) return false;
        o.res = true;
        o.G = nj;
        o.ri = ri;
        o.CH = cj;
        o.CHS = cj;
        o.NZ = nj * (cj + 4);
        o.block = (lanes + 63) / 64 * 64;
        o.np = N;
    } else {
        o.res = false;
        o.ri = 0;
        int G = 1;
        while (G < 16) {
            const int rpw = 64 / (G * 2);
            const int npad = (N + rpw - 1) / rpw * rpw;
            if (npad * G * 2 > 1024) break;
            G <<= 1;
        }
        const int rpw = 64 / G;
        const int npad = (N + rpw - 1) / rpw * rpw;
        if (npad * G > 1024) return false;   // more receivers than threads of one workgroup
        o.G = G;
        o.CH = 1;
        o.CHS = (N + G - 1) / G;
        o.NZ = (G * o.CHS + 3) / 4 * 4;
        o.block = npad * G;
        o.np = N;
    }
    return true;
}

// true unless the environment variable is set to "0" (a kernel variant kept for comparison)
bool getenv_flag_off(const char* name) {
    const char* e = getenv(name);
    return !(e && strcmp(e, "0") == 0);
}

// The spike-driven forward (axonal_fwd_wave) serves N <= 256 unless DELREC_AXONAL_FWD=tiled
// selects the dense tiled scan (kept for comparison; read on every call).
bool axonal_fwd_wave_on() {
    const char* e = getenv("DELREC_AXONAL_FWD");
    return !(e && strcmp(e, "tiled") == 0);
}

// k splits of the dW GEMM: about one 128x128-tile workgroup per CU (the delay-gradient
// blocks launched beside them take the other slots; twice as many splits doubles the
// partials' HBM traffic for no gain), chunks of >= 128 rows
int dw_splits(int T, int B, int N) {
    const int tiles = (N + 127) / 128;
    const int want = (num_cus() + tiles * tiles - 1) / (tiles * tiles);
    return std::max(1, std::min(want, std::max(1, T * B / 128)));
}

template <class C>
void axonal_bwd_ws(C& c, int T, int B, int N, const AxLayout& lay) {
    c.template take<float>((size_t)3 * B * N);          // per-row partials
    c.template take<float>((size_t)T * B * N);          // gr (dropout / decay_input)
    c.template take<float>((size_t)dw_splits(T, B, N) * N * N);   // dW split-K partials
    if (lay.res) c.template take<float>((size_t)T * B * N);                         // gz
}

// ------------------------------------------------------------------ synaptic layout ----
struct SynLayout {
    int block, R, NP, NF;
    bool lds_ring;
    size_t lds;
};

SynLayout syn_layout(int N, int L, bool fwd) {
    SynLayout o;
    o.block = std::min(1024, (N + 63) / 64 * 64);
    o.R = std::max(L, 2);
    o.NP = N;
    o.NF = N;
    const int npt = (N + o.block - 1) / o.block;
    const size_t extra = fwd ? (size_t)(o.NF + npt * (o.block / 64) + 4) * sizeof(int) : 0;
    const size_t ring = (size_t)o.R * o.NP * sizeof(float);
    o.lds_ring = ring + extra <= (size_t)max_lds_bytes();
    o.lds = (o.lds_ring ? ring : 0) + extra;
    return o;
}

constexpr int kSynMaxTaps = 64;   // half-widths up to s = 31

// Backward ring of the synaptic / hybrid scan: source-major rows of R = L slots plus KT
// mirror slots, KT = taps walked per connection (from the largest half-width).
struct SynBwdLayout {
    int block, R, RS, RP, KT, NT;
    bool lds_ring;
    size_t lds;
};

int syn_taps(float s_max, bool hybrid) {
    // hybrid: taps of one column's triangle from its first closed-support lag (s == 1 needs 2);
    // synaptic: lags from max(1, ceil(c - s)) up to floor(c + s)
    const int need = hybrid ? (s_max == 1.0f ? 2 : (int)std::ceil(2.0f * s_max) + 1)
                            : (int)std::floor(2.0f * s_max) + 2;
    // compiled run lengths: 2 and 4 (hybrid), 4, 8 and 12 (synaptic); others run with a
    // runtime tap count
    for (int kt : hybrid ? std::initializer_list<int>{2, 4} : std::initializer_list<int>{4, 8, 12})
        if (kt >= need) return kt;
    return need <= kSynMaxTaps ? need : 0;
}

SynBwdLayout syn_bwd_layout(int N, int L, int KT) {
    SynBwdLayout o;
    o.block = std::min(1024, (N + 63) / 64 * 64);
    o.R = std::max(L, 2);
    o.KT = KT;
    o.RS = o.R + KT;
    o.RP = o.RS | 1;                         // odd pitch: a gather's lanes hit distinct banks
    o.NT = (N + 15) / 16 * 16;
    const size_t ring = (size_t)N * o.RP * sizeof(float);
    o.lds_ring = ring <= (size_t)max_lds_bytes();
    o.lds = o.lds_ring ? ring : 0;
    return o;
}

// the bf16 lag GEMM's packed operands: rows t * Bp + b with the batch padded to 32-row
// chunks (one partial sum per chunk), columns padded to a multiple of 128
struct LagPack {
    int Bp, Np, Kp, KS;
};

LagPack lag_pack(int T, int B, int N) {
    LagPack q;
    q.Bp = (B + 31) / 32 * 32;
    q.Np = (N + 127) / 128 * 128;
    q.Kp = T * q.Bp;
    q.KS = q.Bp / 32;
    return q;
}

// the forward's gather form: history words of 64 lags and the window of one connection
int syn_gather_words(int L) { return L - 1 <= 64 ? 1 : (L - 1 <= 128 ? 2 : 0); }
int syn_gather_taps(float s_max) { return (int)std::floor(2.0f * s_max) + 2; }

// The lag-stacked per-step GEMM scans (lagstep.hip) run where the rings of the gather /
// scatter scans do not fit one CU's LDS; DELREC_SYN_LAGSTEP=1 forces them (any size),
// =0 turns them off. Operands are addressed with 32-bit byte offsets.
struct LagStepDims {
    int Nk, Np, Lw, Kt;
    int P, Lf;          // steps per block (= near lags), far lags Lw - P
    int KS, KSF;        // k splits of the per-step near GEMM and of the per-block far GEMM
    size_t lda;         // history row pitch (elements): (T + Lw) * Nk
    size_t plane;       // uint4 per packed M plane
    bool ok;
};

LagStepDims lagstep_dims(int T, int B, int N, int L) {
    LagStepDims q{};
    q.Nk = (N + 31) / 32 * 32;
    q.Np = (N + 127) / 128 * 128;
    q.Lw = std::max(L - 1, 1);
    q.Kt = q.Lw * q.Nk;
    q.P = std::min(lagstep_block(), q.Lw);
    q.Lf = q.Lw - q.P;
    q.lda = (size_t)(T + q.Lw) * q.Nk;
    q.plane = (size_t)(q.Kt / 8) * q.Np;
    q.KS = lagstep_splits(B, q.Np, q.P * q.Nk, num_cus());
    q.KSF = q.Lf > 0 ? lagblock_splits(B, q.Np, q.Nk, num_cus()) : 0;
    // byte offsets of every history row a GEMM may address (incl. rows of a partial tile)
    q.ok = (size_t)(B + 128) * q.lda * 2 < ((size_t)1 << 32) && q.plane * 16 < ((size_t)1 << 32);
    return q;
}

// ceil(2 s_max): the most lags of non-zero weight a connection has (the flags' bits 8..15)
int lag_taps(float smax) { return std::min(255, std::max(0, (int)std::ceil(2.0f * smax))); }

// The lag-stacked form multiplies every lag of the window; it pays where a connection's
// taps are a fair share of the window (measured: 46 lags at 10 taps, C4, beat the gathers
// 7x), not for narrow triangles over long windows (the hybrid at sigma 0: 2 taps).
bool syn_lagstep(int T, int B, int N, int L, int taps) {
    const char* e = getenv("DELREC_SYN_LAGSTEP");
    if (e && e[0] == '0') return false;
    if (!lagstep_dims(T, B, N, L).ok) return false;
    if (e && e[0] == '1') return true;
    return !syn_layout(N, L, true).lds_ring && L - 1 <= 12 * std::max(taps, 1);
}

template <class C>
void lagstep_ws(C& c, int T, int B, int N, int L, bool fwd) {
    const LagStepDims q = lagstep_dims(T, B, N, L);
    c.template take<uint4>(2 * q.plane);                         // M planes
    c.template take<uint16_t>((size_t)B * q.lda);                // history (spikes / gr hi)
    if (!fwd) c.template take<uint16_t>((size_t)B * q.lda);      // gr lo
    c.template take<float>((size_t)q.KS * B * q.Np);             // near-lag partials
    c.template take<float>((size_t)std::max(q.KSF, 1) * B * q.P * q.Np);   // far-lag partials
    c.template take<float>((size_t)B * N);                       // v / lambda
}

// The offset-stacked hybrid scans (hybstep.hip): hybrid delays of one uniform half-width
// whose taps all lie at lags >= 1 (lags_ok: d_min >= s - 1), D = off_count offsets (at most
// 16), KF = ceil(2 s) taps per source (at most 8) and a window of at most 128 lags, where
// the rings of the per-connection scans do not fit one CU's LDS. DELREC_SYN_HYBSTEP=1
// forces them at any size (parity tests), =0 turns them off.
bool syn_hybstep(int T, int B, int N, int L, bool hybrid, int off_count, int taps, bool lags_ok) {
    const char* e = getenv("DELREC_SYN_HYBSTEP");
    if (e && e[0] == '0') return false;
    if (!hybrid || off_count <= 0 || !lags_ok) return false;
    if (!hybstep_dims(T, B, N, L, off_count, taps, num_cus()).ok) return false;
    if (e && e[0] == '1') return true;
    return !syn_layout(N, L, true).lds_ring;
}

// The hybrid forward as a scatter on arrival (hybstep.hip, hyb_fwd_arrive_kernel): bf16 W,
// one uniform half-width of at most 4 taps per source, all at lags >= 1, at most 16 offsets,
// 2048 neurons and two spike-history words; its ring of D + KF - 1 slots per receiver and
// the arrival lists fit LDS. DELREC_HYB_FWD=0 turns it off.
struct ArriveShape {
    bool ok;
    int npt, block, kf, R, RP, hw;
    int pitch;   // packed words per source row: npt * block, one per lane column
    int sh;   // the packed offset field's shift: log2 of a slot's bytes where R slots are 2^16 bytes, else 0
    size_t lds;
};
ArriveShape syn_arrive(int N, int L, bool hybrid, bool bf16, int off_count, int taps, bool lags_ok) {
    ArriveShape a{};
    if (!getenv_flag_off("DELREC_HYB_FWD")) return a;
    if (!hybrid || !bf16 || !lags_ok || off_count < 1 || off_count > 16 || taps < 1 || taps > 4) return a;
    if (N > 2048) return a;
    a.npt = N <= 1024 ? 1 : 2;
    a.block = a.npt == 1 ? (N + 63) / 64 * 64 : 1024;
    a.pitch = a.npt * a.block;
    a.kf = taps <= 2 ? 2 : 4;
    a.R = 1;   // D + KF - 1 slots, rounded up to a power of two (the kernel wraps by a mask)
    while (a.R < off_count + a.kf - 1) a.R *= 2;
    a.RP = a.R + a.kf - 1;
    const int slot_log2 = a.npt == 1 ? 12 : 13;   // npt * 1024 receivers x 4 bytes per slot
    a.sh = (a.R << slot_log2) == 65536 ? slot_log2 : 0;
    a.hw = (std::max(L - 1, 1) + 63) / 64;
    // ring [RP][npt * 1024], segment counts [2][16], arrival segments [2][16][npt * 64]
    a.lds = (size_t)a.RP * a.npt * 1024 * sizeof(float) + (size_t)2 * 16 * sizeof(int) +
            (size_t)2 * 16 * a.npt * 64 * sizeof(uint16_t);
    a.ok = a.hw <= 2 && a.lds <= (size_t)max_lds_bytes();
    return a;
}

template <class C>
void hybstep_ws(C& c, int T, int B, int N, int L, int D, int KF, bool fwd, bool bf16) {
    const HybStepDims q = hybstep_dims(T, B, N, L, D, KF, num_cus());
    const int planes = bf16 ? 1 : 2;
    if (fwd) {
        c.template take<uint4>(planes * q.plane);                // W^(e) planes
        c.template take<uint16_t>((size_t)B * q.lda);            // z history hi
        c.template take<uint16_t>((size_t)B * q.lda);            // z history lo
        c.template take<float>((size_t)q.KS * B * q.Np);         // split-K partials
        c.template take<float>((size_t)B * N);                   // v
        c.template take<int>((size_t)N);                         // first lag per source
        c.template take<float>((size_t)KF * N);                  // tap weights per source
        c.template take<uint64_t>((size_t)q.HW * B * N);         // spike-history words
        return;
    }
    const HybBwdSizes z = hyb_bwd_sizes(q, B, num_cus(), hyb_bwd_far_cols(planes));
    c.template take<uint4>(planes * z.planes);                   // near + far W^(e) planes
    c.template take<uint16_t>((size_t)B * q.lda);                // gr history hi
    c.template take<uint16_t>((size_t)B * q.lda);                // gr history lo
    c.template take<float>(std::max<size_t>(z.npart, 1));        // near partials
    c.template take<float>(std::max<size_t>(z.fpart, 1));        // far partials
    c.template take<float>((size_t)B * N);                       // lambda
    c.template take<int>((size_t)N);                             // first lag per source
    c.template take<float>((size_t)KF * N);                      // tap weights per source
    c.template take<int>((size_t)N);                             // source order
    c.template take<int>((size_t)N);                             // far column per source
    c.template take<uint32_t>((size_t)kHybNearMax * kHybNearMax); // W and offsets between near neurons
    c.template take<float>((size_t)q.R * N * B);                 // ring of G
}

template <class C>
void syn_fwd_ws(C& c, int T, int B, int N, int L, bool hybrid, bool bf16, int taps, int offc, bool lags_ok) {
    const ArriveShape ar = syn_arrive(N, L, hybrid, bf16, offc, taps, lags_ok);
    if (ar.ok) {
        c.template take<uint32_t>((size_t)N * ar.pitch);   // packed W^T | offsets^T
        c.template take<int>((size_t)N);            // first lag per source
        c.template take<float>((size_t)ar.kf * N);  // tap weights per source
        return;
    }
    if (syn_hybstep(T, B, N, L, hybrid, offc, taps, lags_ok)) {
        hybstep_ws(c, T, B, N, L, offc, taps, true, bf16);
        return;
    }
    if (syn_lagstep(T, B, N, L, taps)) {
        lagstep_ws(c, T, B, N, L, true);
        return;
    }
    const SynLayout lay = syn_layout(N, L, true);
    const size_t nb = (size_t)((N + 15) / 16) * 16 * N;   // blocked copies
    if (bf16) c.template take<uint16_t>(nb); else c.template take<float>(nb);
    if (hybrid) c.template take<int8_t>(nb); else c.template take<float>(nb);
    if (!lay.lds_ring) c.template take<float>((size_t)B * lay.R * N);
    if (hybrid && bf16) c.template take<uint32_t>((size_t)N * N);   // packed W^T | offsets^T
}

template <class C>
void syn_bwd_ws(C& c, int T, int B, int N, int L, int taps, bool hybrid, bool bf16, int offc, bool lags_ok) {
    // sized for the widest tap run, so the ring may always go to the workspace
    const SynBwdLayout lay = syn_bwd_layout(N, L, kSynMaxTaps);
    const LagPack q = lag_pack(T, B, N);
    const size_t packed = (size_t)q.Kp / 8 * q.Np;       // uint4 per packed operand
    c.template take<float>((size_t)T * B * N);          // gr
    c.template take<float>((size_t)B * N);              // db partials
    c.template take<float>((size_t)3 * q.KS * N * N);   // lag-GEMM partials
    c.template take<uint4>(packed);                     // gr_hi
    c.template take<uint4>(packed);                     // gr_mid
    c.template take<uint4>(packed);                     // gr_lo
    c.template take<uint4>(packed);                     // shifted spikes
    c.template take<int>((size_t)4 * N + 64);           // lag range per column, meta
    if (syn_hybstep(T, B, N, L, hybrid, offc, taps, lags_ok)) {
        hybstep_ws(c, T, B, N, L, offc, taps, false, bf16);
        return;
    }
    if (syn_lagstep(T, B, N, L, taps)) {
        lagstep_ws(c, T, B, N, L, false);
        return;
    }
    c.template take<float>((size_t)N * lay.NT);         // W^T (fp32 or bf16)
    c.template take<float>((size_t)N * lay.NT);         // d^T or the offsets^T
    c.template take<float>((size_t)B * N * lay.RP);     // ring when it does not fit LDS
    c.template take<uint8_t>((size_t)N * lay.NT);       // byte slot offsets (hybrid)
    c.template take<int>((size_t)N);                    // sources in first-lag order (hybrid)
}

// out[c * op + r] = in[r * n + c] for an (n, n) matrix; output columns r in [n, op) are 0
template <class E>
__global__ void transpose_kernel(const E* __restrict__ in, E* __restrict__ out, int n, int op) {
    __shared__ E tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    for (int k = threadIdx.y; k < 32; k += 8) {
        const int r = by + k, c = bx + threadIdx.x;
        tile[k][threadIdx.x] = (r < n && c < n) ? in[(size_t)r * n + c] : E(0);
    }
    __syncthreads();
    for (int k = threadIdx.y; k < 32; k += 8) {
        const int r = bx + k, c = by + threadIdx.x;
        if (r < n && c < op) out[(size_t)r * op + c] = tile[threadIdx.x][k];
    }
}

// Blocked copies for per-lane streaming of an (n, n) row-major matrix in runs of 16:
//   columns (ROWS = false): lane j reads i = 16c .. 16c+15 of column j,
//       out[((i / 16) * n + j) * 16 + i % 16] = in[i * n + j];
//   rows (ROWS = true): lane i reads j = 16c .. 16c+15 of row i,
//       out[((j / 16) * n + i) * 16 + j % 16] = in[i * n + j];
// a wave's lanes read adjacent runs; entries past n are zero (ceil(n / 16) runs per lane).
// With `order` (columns form only) lane slot k holds column order[k].
template <class E, bool ROWS>
__global__ void block_copy_kernel(const E* __restrict__ in, E* __restrict__ out, int n,
                                  const int* __restrict__ order) {
    const int nc = (n + 15) / 16;
    const size_t total = (size_t)nc * n;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total;
         q += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(q / n), slot = (int)(q - (size_t)c * n);
        const int lane = (!ROWS && order) ? order[slot] : slot;
        E v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int k = c * 16 + e;
            v[e] = k < n ? (ROWS ? in[(size_t)lane * n + k] : in[(size_t)k * n + lane]) : E(0);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) out[q * 16 + e] = v[e];
    }
}

template <class E, bool ROWS = false>
void block_transpose(const void* in, void* out, int n, hipStream_t s, const int* order = nullptr) {
    const size_t total = (size_t)((n + 15) / 16) * n;
    const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, 65535);
    hipLaunchKernelGGL((block_copy_kernel<E, ROWS>), dim3(blocks), dim3(256), 0, s,
                       static_cast<const E*>(in), static_cast<E*>(out), n, order);
}

template <class E>
void transpose(const void* in, void* out, int n, hipStream_t s, int op = 0) {
    if (op < n) op = n;
    const dim3 grid((n + 31) / 32, (op + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel<E>, grid, dim3(32, 8), 0, s, static_cast<const E*>(in),
                       static_cast<E*>(out), n, op);
}

// HIP-event brackets around the time-scan kernels (benchmark hook)
struct ScanTiming {
    std::vector<hipEvent_t> ev;    // two per launch
    std::vector<int32_t> kind;
    int used = 0;
};
ScanTiming g_scan;

bool scan_begin(int kind, hipStream_t s) {
    const int cap = (int)g_scan.kind.size();
    if (g_scan.used >= cap) return false;
    g_scan.kind[g_scan.used] = kind;
    return hipEventRecord(g_scan.ev[2 * g_scan.used], s) == hipSuccess;
}

void scan_end(bool on, hipStream_t s) {
    if (!on) return;
    if (hipEventRecord(g_scan.ev[2 * g_scan.used + 1], s) == hipSuccess) ++g_scan.used;
}

void scan_release() {
    for (hipEvent_t e : g_scan.ev) (void)hipEventDestroy(e);
    g_scan.ev.clear();
    g_scan.kind.clear();
    g_scan.used = 0;
}

// Ring of max readbacks: DELREC_MAX_SLOTS 8-byte slots of coherent pinned host memory, each
// (ticket, value bits) written by one store of max_to_host_kernel. Ticket 0 marks an empty
// slot; tickets count up from 1 (wrapping past 0).
struct MaxRing {
    unsigned long long* host = nullptr;
    std::atomic<uint32_t> next{1};
    bool ok = false;
};

MaxRing& max_ring() {
    static MaxRing r;
    static std::once_flag once;
    std::call_once(once, [] {
        void* p = nullptr;
        const size_t bytes = (size_t)DELREC_MAX_SLOTS * sizeof(unsigned long long);
        if (hipHostMalloc(&p, bytes, hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable) ==
            hipSuccess) {
            memset(p, 0, bytes);
            r.host = static_cast<unsigned long long*>(p);
            r.ok = true;
        }
    });
    return r;
}

// a fresh ticket and the device address of its slot
int max_slot(uint32_t& t, unsigned long long*& dslot) {
    MaxRing& r = max_ring();
    if (!r.ok) return DELREC_ERR_DEVICE;
    t = r.next.fetch_add(1);
    if (t == 0) t = r.next.fetch_add(1);
    void* dbase = nullptr;
    if (hipHostGetDevicePointer(&dbase, r.host, 0) != hipSuccess || !dbase) return DELREC_ERR_DEVICE;
    dslot = static_cast<unsigned long long*>(dbase) + t % DELREC_MAX_SLOTS;
    return DELREC_OK;
}

// Scratch of delrec_axonal_bwd_noalloc: device memory that belongs to the library's code
// object, one copy on every GPU the library runs on, held until the process ends. In host
// code `scratch` names a host-side stand-in, never the device address: host code uses the
// address scratch_address() looks up (per device) instead.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;

struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
};
ScratchSlot g_scratch[kMaxDevices];

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

// The current device's copy of `scratch`, looked up once per device (with that device
// current) on the first call that needs it.
int scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DELREC_ERR_DEVICE;
    ScratchSlot& slot = g_scratch[dev];
    std::call_once(slot.once, [&slot] {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) slot.ptr = p;
    });
    if (!slot.ptr) return DELREC_ERR_DEVICE;
    *out = slot.ptr;
    return DELREC_OK;
}

}  // namespace

void delrec::ensure_lds(const void* fn, size_t bytes) {
    // launches may come from several host threads (the autograd engine runs backward passes
    // on its own device thread)
    static std::mutex mu;
    static std::vector<std::pair<const void*, size_t>> done;
    std::lock_guard<std::mutex> lock(mu);
    for (auto& e : done)
        if (e.first == fn) {
            if (e.second >= bytes) return;
            (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
            e.second = bytes;
            return;
        }
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    done.emplace_back(fn, bytes);
}

namespace delrec {
namespace {

// The input neurons in activity order (the kernels then skip the silent ones), unless
// DELREC_SPIKE_ORDER=0 (natural order, the spike words read as given)
template <class P>
void spike_linear_order(P& p, void* room, hipStream_t s) {
    const char* e = getenv("DELREC_SPIKE_ORDER");
    p.ldb = p.K;
    if (e && e[0] == '0') return;
    const SpikeOrder o = spike_order_carve(room, p.T, p.B, p.K);
    launch_spike_order(p.bits, p.T, p.B, p.K, o, s);
    p.bits = o.bits;
    p.ldb = spike_order_kp(p.K);
    p.perm = o.perm;
    p.cls = o.cls;
}

}  // namespace
}  // namespace delrec

extern "C" {

int delrec_peak_mfma(int32_t kind, int32_t iters, float* sink, size_t sink_bytes, double* flops, void* stream) {
    if ((kind != 0 && kind != 1) || iters <= 0 || !sink || !flops) return DELREC_ERR_ARG;
    const int blocks = peak_mfma_blocks(num_cus());
    if (sink_bytes < (size_t)blocks * 512 * sizeof(float)) return DELREC_ERR_WORKSPACE;
    *flops = launch_peak_mfma(kind, iters, sink, blocks, static_cast<hipStream_t>(stream));
    return finish_launch();
}

const char* delrec_version(void) { return "delrec-mi355x " DELREC_ABI_VERSION " (gfx950)"; }

const char* delrec_strerror(int status) {
    switch (status) {
        case DELREC_OK: return "ok";
        case DELREC_ERR_ARG: return "invalid argument";
        case DELREC_ERR_UNSUPPORTED: return "unsupported regime";
        case DELREC_ERR_WORKSPACE: return "workspace missing or too small";
        case DELREC_ERR_LAUNCH: return "kernel launch failed";
        case DELREC_ERR_WINDOW: return "delay window too long for this layer size";
        case DELREC_ERR_DEVICE: return "device query failed";
        case DELREC_ERR_PENDING: return "device value not written within the time limit";
        case DELREC_ERR_STALE: return "readback slot reused by later posts";
        case DELREC_ERR_SCRATCH: return "sizes need more scratch than the no-alloc entry point holds (64 MiB)";
        default: return "unknown status";
    }
}

int delrec_query_workspace(int32_t kind, int32_t T, int32_t B, int32_t N, int32_t L,
                           int32_t flags, size_t* bytes) {
    if (!bytes || T <= 0 || B <= 0 || N <= 0 || L < 1) return DELREC_ERR_ARG;
    Counter c;
    const bool bf16 = flags & 1;
    switch (kind) {
        case DELREC_WS_AXONAL_FWD: {
            AxLayout lay;
            if (!axonal_layout(N, L, lay)) return DELREC_ERR_UNSUPPORTED;
            if (!lay.res) c.take<float>((size_t)N * N);
            break;
        }
        case DELREC_WS_AXONAL_BWD: {
            AxLayout lay;
            if (!axonal_layout(N, L, lay)) return DELREC_ERR_UNSUPPORTED;
            axonal_bwd_ws(c, T, B, N, lay);
            break;
        }
        case DELREC_WS_SYN_FWD:
            syn_fwd_ws(c, T, B, N, L, (flags & 2) != 0, bf16, (flags >> 8) & 0xff, (flags >> 16) & 0xff,
                       (flags & 4) != 0);
            break;
        case DELREC_WS_SYN_BWD:
            syn_bwd_ws(c, T, B, N, L, (flags >> 8) & 0xff, (flags & 2) != 0, bf16, (flags >> 16) & 0xff,
                       (flags & 4) != 0);
            break;
        case DELREC_WS_SPIKE_LINEAR:
            c.take<uint4>(spike_linear_ws(N, L) / sizeof(uint4));
            c.take<uint4>(spike_order_ws(T, B, N) / sizeof(uint4));
            break;
        case DELREC_WS_SPIKE_LINEAR_DW:
            c.take<uint4>(spike_order_ws(T, B, N) / sizeof(uint4));
            c.take<uint4>(spike_linear_dw_planes(T, B, L));
            c.take<float>((spike_linear_dw_ws(T, B, N, L, num_cus()) -
                           spike_linear_dw_planes(T, B, L) * sizeof(uint4)) / sizeof(float));
            break;
        case DELREC_WS_READOUT_CE:
            c.take<float>((size_t)B);
            break;
        default: return DELREC_ERR_ARG;
    }
    *bytes = c.used;
    return DELREC_OK;
}

// The straight-line forward applies: soft taps of a uniform half-width (at most 8 lags of
// non-zero weight), decay charge, hard reset to 0, no recurrent-input output, N <= 256.
bool axonal_fwd_common(const delrec_axonal_fwd_args* a) {
    const float span = ceilf(2.0f * a->s_uniform);
    // (the straight-line scan addresses each (T, B, N) output with 32-bit offsets: <= 1 GiB)
    return a->N <= 256 && axonal_fwd_wave_on() && a->taps == DELREC_TAPS_SOFT && !a->s &&
           a->s_uniform > 0.0f && span <= 8.0f && !a->lif.decay_input && !a->lif.soft_reset &&
           a->lif.v_reset == 0.0f && !a->rec &&
           (size_t)a->T * a->B * a->N * sizeof(float) <= ((size_t)1 << 30);
}

int delrec_axonal_fwd(const delrec_axonal_fwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || a->L < 0) return DELREC_ERR_ARG;
    // L = 0 (window not read by the caller) only where the kernel sizes its own history
    if (a->L == 0 && !axonal_fwd_common(a)) return DELREC_ERR_ARG;
    if (!a->x || !a->W || !a->d || !a->y || !a->u || !a->bits || !lif_ok(a->lif)) return DELREC_ERR_ARG;
    if (a->taps < 0 || a->taps > 2) return DELREC_ERR_ARG;
    if (a->taps != DELREC_TAPS_SOFT && !a->lag) return DELREC_ERR_ARG;
    if (a->taps == DELREC_TAPS_INTERP && !a->frac) return DELREC_ERR_ARG;
    AxLayout lay;
    if (!axonal_layout(a->N, a->L, lay)) return DELREC_ERR_WINDOW;
    const size_t lds = (size_t)2 * lay.NZ * sizeof(float);
    if (lds > (size_t)max_lds_bytes()) return DELREC_ERR_WINDOW;
    hipStream_t s = static_cast<hipStream_t>(stream);
    AxFwd p{};
    p.T = a->T; p.B = a->B; p.N = a->N; p.L = a->L;
    p.G = lay.G; p.NZ = lay.NZ; p.CHS = lay.CHS;
    p.x = a->x; p.W = a->W; p.Wt = nullptr; p.w_bf16 = a->w_bf16;
    p.bias = a->bias; p.d = a->d; p.s = a->s; p.s_uniform = a->s_uniform; p.drop = a->drop;
    p.taps = a->taps; p.lag = a->lag; p.frac = a->frac; p.lif = make_lif(a->lif);
    p.y = a->y; p.u = a->u; p.rec = a->rec; p.z = a->z; p.bits = a->bits;
    if (!lay.res) {
        Carver cv(a->workspace, a->workspace_bytes);
        void* wt = a->w_bf16 ? (void*)cv.take<uint16_t>((size_t)a->N * a->N)
                             : (void*)cv.take<float>((size_t)a->N * a->N);
        if (!wt) return DELREC_ERR_WORKSPACE;
        if (a->w_bf16) transpose<uint16_t>(a->W, wt, a->N, s); else transpose<float>(a->W, wt, a->N, s);
        p.Wt = wt;
    }
    // max d for the caller's host: written by the straight-line scan's first workgroup, else
    // by a small kernel ahead of the scan
    const bool fast = lay.res && axonal_fwd_wave_on() && axonal_fwd_common(a) && lay.hw <= 4;
    uint32_t mx_t = 0;
    if (a->dmax_ticket) {
        unsigned long long* slot = nullptr;
        if (int st = max_slot(mx_t, slot)) return st;
        if (fast) {
            p.mx_slot = slot;
            p.mx_ticket = mx_t;
        } else {
            launch_max_to_host(a->d, a->N, mx_t, slot, s);
        }
    }
    const bool timed = scan_begin(DELREC_WS_AXONAL_FWD, s);
    bool ok;
    if (lay.res && axonal_fwd_wave_on()) {
        // spike-driven form: ceil(N/32) waves of 32 source columns, RI receivers per lane
        const int nw = (a->N + 31) / 32;
        const int ri = a->N > 128 ? 4 : (a->N > 64 ? 2 : 1);
        // the straight-line variant (kf >= ceil(2s) lags of non-zero weight; it takes its
        // history length, one or four 64-step words, from d)
        const float span = ceilf(2.0f * a->s_uniform);
        const int kf = span <= 2.0f ? 2 : (span <= 4.0f ? 4 : 8);
        if (fast) {
            ok = launch_axonal_fwd_wave_fast(p, ri, kf, nw, a->B, s);
        } else {
            const size_t lds_w = (size_t)2 * nw * 64 * ri * sizeof(float);
            ok = launch_axonal_fwd_wave(p, ri, lay.hw, nw, a->B, lds_w, s);
        }
    } else {
        ok = lay.res ? launch_axonal_tiled(true, &p, nullptr, lay.ri, lay.G, lay.CH, lay.hw, a->B, lay.block, lds, s)
                     : launch_axonal(true, &p, nullptr, lay.CH, lay.res, lay.hw, a->B, lay.block, lds, s);
    }
    scan_end(timed && ok, s);
    if (!ok) return DELREC_ERR_UNSUPPORTED;
    if (a->dmax_ticket) *a->dmax_ticket = mx_t;
    return finish_launch();
}

int delrec_axonal_bwd(const delrec_axonal_bwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || a->L < 1) return DELREC_ERR_ARG;
    if (!a->gy || !a->u || !a->bits || !a->W || !a->d || !a->dx || !lif_ok(a->lif)) return DELREC_ERR_ARG;
    if (a->mode != DELREC_BWD_SOFT && a->mode != DELREC_BWD_STRAIGHT) return DELREC_ERR_ARG;
    if (a->mode == DELREC_BWD_STRAIGHT && !a->lag) return DELREC_ERR_ARG;
    if (a->dW && !a->z) return DELREC_ERR_ARG;
    AxLayout lay;
    if (!axonal_layout(a->N, a->L, lay)) return DELREC_ERR_WINDOW;
    // the tiled backward reads kMaxTaps consecutive ring slots from the first tap lag on
    const int R = std::max(a->L, 2) + (lay.res ? kMaxTaps : 0);
    const int NP = lay.res ? lay.np : a->N;
    // tiled: grbuf + ring; streamed: grbuf + ring + tap-weight table
    const size_t lds = ((size_t)2 * lay.NZ + (size_t)(R + (lay.res ? 0 : kMaxTaps)) * NP) * sizeof(float);
    if (lds > (size_t)max_lds_bytes()) return DELREC_ERR_WINDOW;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int T = a->T, B = a->B, N = a->N;
    Carver cv(a->workspace, a->workspace_bytes);
    float* part = cv.take<float>((size_t)3 * B * N);
    float* grbuf = cv.take<float>((size_t)T * B * N);
    const int ks = dw_splits(T, B, N);
    float* gemm_part = cv.take<float>((size_t)ks * N * N);
    float* gzbuf = lay.res ? cv.take<float>((size_t)T * B * N) : nullptr;
    if (!part || !grbuf || !gemm_part || (lay.res && !gzbuf)) return DELREC_ERR_WORKSPACE;
    const bool need_gr = a->drop != nullptr || a->lif.decay_input;

    AxBwd p{};
    p.T = T; p.B = B; p.N = N; p.L = a->L;
    p.G = lay.G; p.NZ = lay.NZ; p.CHS = lay.CHS; p.R = R; p.NP = NP;
    p.gy = a->gy; p.u = a->u; p.bits = a->bits; p.W = a->W; p.w_bf16 = a->w_bf16;
    p.d = a->d; p.s = a->s; p.s_uniform = a->s_uniform; p.drop = a->drop;
    p.mode = a->mode; p.lag = a->lag; p.lif = make_lif(a->lif);
    p.dx = a->dx; p.gr = need_gr ? grbuf : nullptr; p.part = part; p.gz = gzbuf;
    const bool timed = scan_begin(DELREC_WS_AXONAL_BWD, s);
    // the straight-line tiled backward: soft taps of a uniform half-width (kf >= ceil(2s)
    // lags of non-zero weight), one history word, ATan, decay charge, hard reset to 0
    const float span = ceilf(2.0f * a->s_uniform);
    const int kf = span <= 2.0f ? 2 : (span <= 4.0f ? 4 : 8);
    const bool common = lay.res && axonal_fwd_wave_on() && a->mode == DELREC_BWD_SOFT && lay.hw == 1 &&
                        !a->s && a->s_uniform > 0.0f && span <= 8.0f && a->lif.surrogate == 1 &&
                        !a->lif.decay_input && !a->lif.soft_reset && a->lif.v_reset == 0.0f &&
                        !a->lif.detach_reset;
    bool ok;
    if (common) {
        const size_t lds_f = ((size_t)2 * lay.NZ + (size_t)(R + kf - 1) * NP) * sizeof(float);
        ok = lds_f <= (size_t)max_lds_bytes() &&
             launch_axonal_bwd_tiled_fast(p, lay.ri, lay.G, lay.CH, kf, B, lay.block, lds_f, s);
    } else {
        ok = lay.res ? launch_axonal_tiled(false, nullptr, &p, lay.ri, lay.G, lay.CH, lay.hw, B, lay.block, lds, s)
                     : launch_axonal(false, nullptr, &p, lay.CH, lay.res, lay.hw, B, lay.block, lds, s);
    }
    scan_end(timed && ok, s);
    if (!ok) return DELREC_ERR_UNSUPPORTED;
    int st = finish_launch();
    if (st) return st;
    // dW = sum_{t,b} gr (x) z beside the delay-gradient pass (the tiled scan leaves db
    // partials in part[0], the segment pass adds dd / ds in part[1..2]; the streamed scan
    // writes all three), then the split-K sums beside the batch reductions
    const bool delays = lay.res && (a->dd || a->ds);
    AxTail q{};
    q.nbx = (N + 63) / 64;
    q.ndelay = delays ? q.nbx * B : 0;
    if (a->dW) {
        q.A = need_gr ? grbuf : a->dx;
        q.Bz = a->z;
        q.K = T * B;
        q.ks = ks;
        q.tiles = (N + 127) / 128;
        q.kchunk = ((q.K + ks - 1) / ks + 31) / 32 * 32;   // whole 32-row stages
        q.gpart = gemm_part;
        q.dW = a->dW;
        q.ndw = q.tiles * q.tiles * ks;
        q.nsum = (int)(((size_t)N * N + 255) / 256);
    }
    q.o0 = a->db;
    q.o1 = lay.res && !delays ? nullptr : a->dd;
    q.o2 = lay.res && !delays ? nullptr : a->ds;
    launch_axonal_bwd_tail(p, q, s);
    launch_axonal_bwd_sums(q, part, B, N, s);
    return finish_launch();
}

int delrec_axonal_bwd_noalloc(const delrec_axonal_bwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || a->L < 1) return DELREC_ERR_ARG;
    AxLayout lay;
    if (!axonal_layout(a->N, a->L, lay)) return DELREC_ERR_WINDOW;
    Counter c;
    axonal_bwd_ws(c, a->T, a->B, a->N, lay);
    if (c.used > kNoAllocScratchBytes) return DELREC_ERR_SCRATCH;
    void* ws = nullptr;
    if (int st = scratch_address(&ws)) return st;
    // the same launches as delrec_axonal_bwd, with this GPU's scratch as the workspace (every
    // workspace word is written before it is read, so nothing needs clearing between calls)
    delrec_axonal_bwd_args b = *a;
    b.workspace = ws;
    b.workspace_bytes = kNoAllocScratchBytes;
    return delrec_axonal_bwd(&b, stream);
}

// forward as one lag-stacked GEMM + one LIF launch per step
int syn_fwd_lagstep(const delrec_syn_fwd_args* a, hipStream_t s) {
    const int T = a->T, B = a->B, N = a->N;
    const LagStepDims q = lagstep_dims(T, B, N, a->L);
    Carver cv(a->workspace, a->workspace_bytes);
    uint4* planes = cv.take<uint4>(2 * q.plane);
    uint16_t* hist = cv.take<uint16_t>((size_t)B * q.lda);
    float* part = cv.take<float>((size_t)q.KS * B * q.Np);
    float* fpart = cv.take<float>((size_t)std::max(q.KSF, 1) * B * q.P * q.Np);
    float* state = cv.take<float>((size_t)B * N);
    if (!planes || !hist || !part || !fpart || !state) return DELREC_ERR_WORKSPACE;
    LagStepPack pk{};
    pk.N = N; pk.Nk = q.Nk; pk.Np = q.Np; pk.Lw = q.Lw;
    pk.W = a->W; pk.w_bf16 = a->w_bf16; pk.d = a->d; pk.base = a->base; pk.off = a->offsets;
    pk.s = a->s; pk.s_uniform = a->s_uniform; pk.out = planes;
    launch_pack_lagw(pk, true, s);
    launch_hist_clear(hist, B, q.lda, s);   // incl. the spikes before t = 0
    // packed k order: lag Lw first, lag 1 last; the far lags Lw .. P + 1 come first
    const size_t kfar = (size_t)q.Lf * q.Nk / 8 * q.Np;   // uint4 offset of the near lags
    LagStepGemm g{};   // near lags of one step: spikes t - P .. t - 1
    g.a0 = hist; g.a1 = nullptr; g.lda = q.lda; g.rs = 0; g.B = B; g.rows = B; g.rp = 1;
    g.p0 = planes + kfar; g.p1 = planes + q.plane + kfar; g.Np = q.Np; g.Kt = q.P * q.Nk;
    g.KS = q.KS; g.Nk = q.Nk; g.part = part;
    LagStepGemm gf = g;   // far lags of a block of P steps: row (b, tt) reads spikes t0 + tt - Lw ..
    gf.rows = B * q.P; gf.rp = q.P; gf.rs = q.Nk;
    gf.p0 = planes; gf.p1 = planes + q.plane; gf.Kt = q.Lf * q.Nk; gf.KS = q.KSF; gf.part = fpart;
    LagStepLif l{};
    l.T = T; l.B = B; l.N = N; l.Nk = q.Nk; l.Np = q.Np; l.KS = q.KS; l.Lw = q.Lw; l.lda = q.lda;
    l.part = part; l.fpart = q.Lf > 0 ? fpart : nullptr; l.KSF = q.Lf > 0 ? q.KSF : 0; l.P = q.P;
    l.x = a->x; l.bias = a->bias; l.drop = a->drop; l.lif = make_lif(a->lif);
    l.state = state; l.y = a->y; l.u = a->u; l.bits = a->bits; l.hist = hist;
    const bool timed = scan_begin(DELREC_WS_SYN_FWD, s);
    for (int t0 = 0; t0 < T; t0 += q.P) {
        if (q.Lf > 0) {
            gf.aoff = (size_t)t0 * q.Nk;
            launch_lagblock(gf, 1, s);
        }
        for (int t = t0; t < std::min(T, t0 + q.P); ++t) {
            g.aoff = (size_t)(t + q.Lf) * q.Nk;
            launch_lagstep_gemm(g, 1, s);
            l.t = t;
            l.tt = t - t0;
            launch_lagstep_lif(l, true, s);
        }
    }
    scan_end(timed, s);
    return finish_launch();
}

// forward as one offset-stacked GEMM + one LIF launch per step (hybstep.hip)
int syn_fwd_hybstep(const delrec_syn_fwd_args* a, int KF, hipStream_t s) {
    const int T = a->T, B = a->B, N = a->N;
    const HybStepDims q = hybstep_dims(T, B, N, a->L, a->off_count, KF, num_cus());
    const int planes = a->w_bf16 ? 1 : 2;
    Carver cv(a->workspace, a->workspace_bytes);
    uint4* P = cv.take<uint4>(planes * q.plane);
    uint16_t* hhi = cv.take<uint16_t>((size_t)B * q.lda);
    uint16_t* hlo = cv.take<uint16_t>((size_t)B * q.lda);
    float* part = cv.take<float>((size_t)q.KS * B * q.Np);
    float* state = cv.take<float>((size_t)B * N);
    int* lof = cv.take<int>((size_t)N);
    float* h = cv.take<float>((size_t)KF * N);
    uint64_t* hist = cv.take<uint64_t>((size_t)q.HW * B * N);
    if (!P || !hhi || !hlo || !part || !state || !lof || !h || !hist) return DELREC_ERR_WORKSPACE;
    HybPack pk{};
    pk.N = N; pk.Nk = q.Nk; pk.Np = q.Np; pk.D = q.D; pk.omin = a->off_min; pk.planes = planes;
    pk.W = a->W; pk.w_bf16 = a->w_bf16; pk.off = a->offsets; pk.out = P;
    launch_hyb_pack(pk, true, s);
    HybTaps tp{};
    tp.N = N; tp.KF = KF; tp.omin = a->off_min; tp.s = a->s_uniform; tp.base = a->base; tp.lof = lof; tp.h = h;
    launch_hyb_taps(tp, s);
    launch_hist_clear(hhi, B, q.lda, s);   // z before t = 0, and the slices past the last step
    launch_hist_clear(hlo, B, q.lda, s);
    LagStepGemm g{};   // step t: rec(t) from history slices t .. t + D - 1 = z(t - D + 1 .. t)
    g.a0 = hhi; g.a1 = hlo; g.lda = q.lda; g.rs = 0; g.B = B; g.rows = B; g.rp = 1;
    g.p0 = P; g.p1 = planes > 1 ? P + q.plane : nullptr; g.Np = q.Np; g.Kt = q.Kt; g.KS = q.KS;
    g.Nk = q.Nk; g.part = part;
    HybLif l{};
    l.T = T; l.B = B; l.N = N; l.Nk = q.Nk; l.Np = q.Np; l.KS = q.KS; l.D = q.D; l.KF = KF; l.R = q.R;
    l.lda = q.lda; l.part = part; l.lof = lof; l.h = h; l.bias = a->bias; l.drop = a->drop;
    l.lif = make_lif(a->lif); l.state = state; l.hhi = hhi; l.hlo = hlo;
    l.x = a->x; l.y = a->y; l.u = a->u; l.bits = a->bits; l.hist = hist;
    const bool timed = scan_begin(DELREC_WS_SYN_FWD, s);
    for (int t = 0; t < T; ++t) {
        g.aoff = (size_t)t * q.Nk;
        launch_lagstep_gemm(g, 2, s, planes);
        l.t = t;
        launch_hyb_lif(l, q.HW, s);
    }
    scan_end(timed, s);
    return finish_launch();
}

// forward as one event-driven scatter-on-arrival launch, one batch row per workgroup
int syn_fwd_arrive(const delrec_syn_fwd_args* a, const ArriveShape& ar, hipStream_t s) {
    const int N = a->N;
    Carver cv(a->workspace, a->workspace_bytes);
    uint32_t* wpk = cv.take<uint32_t>((size_t)N * ar.pitch);
    int* lof = cv.take<int>((size_t)N);
    float* h = cv.take<float>((size_t)ar.kf * N);
    if (!wpk || !lof || !h) return DELREC_ERR_WORKSPACE;
    launch_pack_hybrid(static_cast<const uint16_t*>(a->W), a->offsets, N, wpk, s, a->off_min, ar.sh,
                       a->off_count, ar.pitch);
    HybTaps tp{};   // kf rows: a run shorter than kf gets taps of weight 0 past its triangle
    tp.N = N; tp.KF = ar.kf; tp.omin = a->off_min; tp.s = a->s_uniform; tp.base = a->base; tp.lof = lof; tp.h = h;
    launch_hyb_taps(tp, s);
    HybScat p{};
    p.T = a->T; p.B = a->B; p.N = N; p.D = a->off_count; p.KF = ar.kf; p.R = ar.R; p.RP = ar.RP; p.sh = ar.sh;
    p.omin = a->off_min; p.x = a->x; p.bias = a->bias; p.drop = a->drop; p.lif = make_lif(a->lif);
    p.wpk = wpk; p.lof = lof; p.h = h; p.y = a->y; p.u = a->u; p.bits = a->bits;
    const bool timed = scan_begin(DELREC_WS_SYN_FWD, s);
    const bool launched = launch_hyb_fwd_arrive(p, ar.npt, ar.hw, ar.block, ar.lds, s);
    scan_end(timed, s);
    if (!launched) return DELREC_ERR_UNSUPPORTED;
    return finish_launch();
}

int delrec_syn_fwd(const delrec_syn_fwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || a->L < 1) return DELREC_ERR_ARG;
    if (!a->x || !a->W || !a->y || !a->u || !a->bits || !lif_ok(a->lif)) return DELREC_ERR_ARG;
    const bool hybrid = a->d == nullptr;
    if (hybrid && (!a->base || !a->offsets)) return DELREC_ERR_ARG;
    if (a->N > 4096) return DELREC_ERR_UNSUPPORTED;
    const SynLayout lay = syn_layout(a->N, a->L, true);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int N = a->N;
    const bool lags_ok = a->d_min >= a->s_uniform - 1.0f;
    const ArriveShape ar = syn_arrive(N, a->L, hybrid && !a->s, a->w_bf16 != 0, a->off_count,
                                      lag_taps(a->s_uniform), lags_ok);
    if (ar.ok) return syn_fwd_arrive(a, ar, s);
    if (syn_hybstep(a->T, a->B, N, a->L, hybrid && !a->s, a->off_count, lag_taps(a->s_uniform), lags_ok))
        return syn_fwd_hybstep(a, lag_taps(a->s_uniform), s);
    if (syn_lagstep(a->T, a->B, N, a->L, lag_taps(a->s ? a->s_max : std::max(a->s_max, a->s_uniform))))
        return syn_fwd_lagstep(a, s);
    const size_t nb = (size_t)((N + 15) / 16) * 16 * N;
    Carver cv(a->workspace, a->workspace_bytes);
    void* wt = a->w_bf16 ? (void*)cv.take<uint16_t>(nb) : (void*)cv.take<float>(nb);
    void* dt = hybrid ? (void*)cv.take<int8_t>(nb) : (void*)cv.take<float>(nb);
    float* gring = lay.lds_ring ? nullptr : cv.take<float>((size_t)a->B * lay.R * N);
    uint32_t* wpk = (hybrid && a->w_bf16) ? cv.take<uint32_t>((size_t)N * N) : nullptr;
    if (!wt || !dt || (!lay.lds_ring && !gring) || (hybrid && a->w_bf16 && !wpk)) return DELREC_ERR_WORKSPACE;

    SynFwd p{};
    p.T = a->T; p.B = a->B; p.N = N; p.L = a->L; p.R = lay.R; p.NP = lay.NP; p.NF = lay.NF;
    p.x = a->x; p.w_bf16 = a->w_bf16; p.bias = a->bias;
    p.base = a->base;
    p.s = a->s; p.s_uniform = a->s_uniform; p.drop = a->drop; p.lif = make_lif(a->lif);
    p.y = a->y; p.u = a->u; p.bits = a->bits;
    // a ring that fits LDS takes the event-driven scatter; otherwise the gather form reads
    // spike-history words (windows of up to 128 lags and 32 taps), else the workspace ring
    const int hw = syn_gather_words(a->L);
    const int kt = syn_gather_taps(a->s ? a->s_max : std::max(a->s_max, a->s_uniform));
    const bool gather = !lay.lds_ring && hw > 0 && kt <= 32;
    size_t lds = lay.lds;
    if (gather) {
        if (a->w_bf16) block_transpose<uint16_t, true>(a->W, wt, N, s); else block_transpose<float, true>(a->W, wt, N, s);
        if (hybrid) block_transpose<int8_t, true>(a->offsets, dt, N, s); else block_transpose<float, true>(a->d, dt, N, s);
        p.Wr = wt;
        p.dr = hybrid ? nullptr : static_cast<const float*>(dt);
        p.offr = hybrid ? static_cast<const int8_t*>(dt) : nullptr;
        p.HW = hw;
        p.KT = kt;
        lds = (size_t)2 * hw * N * sizeof(uint64_t) + (size_t)2 * N * sizeof(float);
    } else {
        if (a->w_bf16) transpose<uint16_t>(a->W, wt, N, s); else transpose<float>(a->W, wt, N, s);
        if (hybrid) transpose<int8_t>(a->offsets, dt, N, s); else transpose<float>(a->d, dt, N, s);
        p.Wt = wt;
        p.dt = hybrid ? nullptr : static_cast<const float*>(dt);
        p.offt = hybrid ? static_cast<const int8_t*>(dt) : nullptr;
        p.gring = gring;
    }
    const bool timed = scan_begin(DELREC_WS_SYN_FWD, s);
    // the chunked event-driven scatter: ring in LDS, one receiver per lane, at most 8
    // lags of non-zero weight per connection
    const float smax = a->s ? a->s_max : std::max(a->s_max, a->s_uniform);
    const float span = ceilf(2.0f * smax);
    const int kf = span <= 2.0f ? 2 : (span <= 4.0f ? 4 : 8);
    const int nwaves = lay.block / 64;
    const size_t lds_s = (size_t)lay.R * lay.NP * sizeof(float) + (size_t)N * 4 * sizeof(float) +
                         64 * sizeof(float) + (size_t)(2 * nwaves * 64 + 2 * nwaves) * sizeof(int);
    const bool scatter = !gather && lay.lds_ring && N <= 1024 && span <= 8.0f && smax > 0.0f &&
                         lds_s <= (size_t)max_lds_bytes() && getenv_flag_off("DELREC_SYN_SCATTER");
    if (scatter && wpk) {
        launch_pack_hybrid(static_cast<const uint16_t*>(a->W), a->offsets, N, wpk, s);
        p.wpk = wpk;
    }
    if (!(scatter && launch_syn_fwd_scatter(p, kf, lay.block, lds_s, s))) launch_syn_fwd(p, lay.block, lds, s);
    scan_end(timed, s);
    return finish_launch();
}

int delrec_spike_linear_fwd(const delrec_spike_linear_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->K <= 0 || a->M <= 0) return DELREC_ERR_ARG;
    if (!a->bits || !a->W || !a->out) return DELREC_ERR_ARG;
    SpikeLinear p{};
    p.T = a->T; p.B = a->B; p.K = a->K; p.M = a->M;
    p.bits = a->bits; p.W = a->W; p.bias = a->bias; p.out = a->out;
    spike_linear_dims(p);
    // 32-bit byte offsets: the spike words (in the activity order's pitch), the packed planes
    // and one output row block
    const int TW = (p.T + 31) / 32;
    if ((size_t)p.B * TW * spike_order_kp(p.K) * 4 >= ((size_t)1 << 31) ||
        spike_linear_ws(p.K, p.M) >= ((size_t)1 << 31))
        return DELREC_ERR_UNSUPPORTED;
    Carver cv(a->workspace, a->workspace_bytes);
    uint4* wp = cv.take<uint4>(spike_linear_ws(p.K, p.M) / sizeof(uint4));
    uint4* ob = cv.take<uint4>(spike_order_ws(p.T, p.B, p.K) / sizeof(uint4));
    if (!wp || !ob) return DELREC_ERR_WORKSPACE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    spike_linear_order(p, ob, s);
    launch_spike_linear(p, wp, s);
    return finish_launch();
}

int delrec_spike_linear_dw(const delrec_spike_linear_dw_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->K <= 0 || a->M <= 0) return DELREC_ERR_ARG;
    if (!a->bits || !a->g || !a->dW) return DELREC_ERR_ARG;
    SpikeLinearDw p{};
    p.T = a->T; p.B = a->B; p.K = a->K; p.M = a->M;
    p.bits = a->bits; p.g = a->g; p.dW = a->dW;
    spike_linear_dw_dims(p, num_cus());
    Carver cv(a->workspace, a->workspace_bytes);
    uint4* ob = cv.take<uint4>(spike_order_ws(p.T, p.B, p.K) / sizeof(uint4));
    p.gp = cv.take<uint4>(spike_linear_dw_planes(p.T, p.B, p.M));
    if (!ob || !p.gp) return DELREC_ERR_WORKSPACE;
    if (p.KS > 1) {
        p.part = cv.take<float>((size_t)p.KS * p.M * p.K);
        if (!p.part) return DELREC_ERR_WORKSPACE;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    spike_linear_order(p, ob, s);
    launch_spike_linear_dw(p, s);
    return finish_launch();
}

int delrec_spike_linear_dx_split(const float* g, int64_t rows, int32_t M, void* out, void* stream) {
    if (!g || !out || rows <= 0 || M <= 0) return DELREC_ERR_ARG;
    launch_spike_linear_dx_split(g, (size_t)rows, M, static_cast<uint16_t*>(out), static_cast<hipStream_t>(stream));
    return finish_launch();
}

int delrec_readout_ce(const delrec_readout_ce_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->C <= 0) return DELREC_ERR_ARG;
    if (!a->logits || !a->labels || !a->dlogits || !a->loss) return DELREC_ERR_ARG;
    if (a->reduce < DELREC_READOUT_SUM || a->reduce > DELREC_READOUT_MAX) return DELREC_ERR_ARG;
    if (a->integrator < 0 || a->integrator > 2 || (a->integrator && !(a->tau > 0.0f))) return DELREC_ERR_ARG;
    if ((size_t)(4 + a->C) * sizeof(float) > (size_t)max_lds_bytes()) return DELREC_ERR_UNSUPPORTED;
    Carver cv(a->workspace, a->workspace_bytes);
    float* rowloss = cv.take<float>((size_t)a->B);
    if (!rowloss) return DELREC_ERR_WORKSPACE;
    ReadoutCe p{};
    p.T = a->T; p.B = a->B; p.C = a->C; p.logits = a->logits; p.labels = a->labels;
    p.reduce = a->reduce; p.integrator = a->integrator; p.tau = a->tau;
    p.decay = a->integrator ? (float)(1.0 - 1.0 / (double)a->tau) : 0.0f;
    p.in_scale = a->integrator == 2 ? (float)(1.0 / (double)a->tau) : 1.0f;
    p.out = a->out; p.dlogits = a->dlogits; p.rowloss = rowloss; p.loss = a->loss;
    launch_readout_ce(p, static_cast<hipStream_t>(stream));
    return finish_launch();
}

int delrec_syn_bwd(const delrec_syn_bwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || a->L < 1) return DELREC_ERR_ARG;
    if (!a->gy || !a->u || !a->bits || !a->W || !a->dx || !lif_ok(a->lif)) return DELREC_ERR_ARG;
    if (!(a->s_max > 0.0f)) return DELREC_ERR_ARG;
    const bool hybrid = a->d == nullptr;
    if (hybrid && (!a->base || !a->offsets)) return DELREC_ERR_ARG;
    if (hybrid && a->s) return DELREC_ERR_UNSUPPORTED;     // the hybrid has one uniform half-width
    if (a->N > 4096) return DELREC_ERR_UNSUPPORTED;
    const int KT = syn_taps(hybrid ? a->s_uniform : (a->s ? a->s_max : std::max(a->s_max, a->s_uniform)), hybrid);
    if (KT == 0) return DELREC_ERR_UNSUPPORTED;             // half-width beyond the widest tap run
    const SynBwdLayout lay = syn_bwd_layout(a->N, a->L, KT);
    const SynBwdLayout wlay = syn_bwd_layout(a->N, a->L, kSynMaxTaps);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int T = a->T, B = a->B, N = a->N;
    const LagPack q = lag_pack(T, B, N);
    const size_t packed = (size_t)q.Kp / 8 * q.Np;
    // the lag GEMM addresses a packed operand with 32-bit byte offsets (plus a window of
    // slices past the end)
    if ((size_t)(T + 32) * (q.Bp / 8) * q.Np * 16 >= ((size_t)1 << 32)) return DELREC_ERR_UNSUPPORTED;
    Carver cv(a->workspace, a->workspace_bytes);
    float* gr = cv.take<float>((size_t)T * B * N);
    float* part = cv.take<float>((size_t)B * N);
    float* lagp = cv.take<float>((size_t)3 * q.KS * N * N);
    uint4* ahi = cv.take<uint4>(packed);
    uint4* amd = cv.take<uint4>(packed);
    uint4* alo = cv.take<uint4>(packed);
    uint4* yb = cv.take<uint4>(packed);
    int* meta = cv.take<int>((size_t)4 * N + 64);
    const int taps = lag_taps(hybrid ? a->s_uniform : (a->s ? a->s_max : std::max(a->s_max, a->s_uniform)));
    const bool hybstep = syn_hybstep(T, B, N, a->L, hybrid && !a->s, a->off_count, taps,
                                     a->d_min >= a->s_uniform - 1.0f);
    const bool lagstep = !hybstep && syn_lagstep(T, B, N, a->L, taps);
    void* wt = nullptr;
    void* dt = nullptr;
    float* gring = nullptr;
    uint8_t* offq = nullptr;
    int* order = nullptr;
    if (!lagstep && !hybstep) {
        wt = cv.take<float>((size_t)N * wlay.NT);
        dt = cv.take<float>((size_t)N * wlay.NT);
        gring = cv.take<float>((size_t)B * N * wlay.RP);
        offq = cv.take<uint8_t>((size_t)N * wlay.NT);
        order = cv.take<int>((size_t)N);
        if (!wt || !dt || !gring || !offq || !order) return DELREC_ERR_WORKSPACE;
    }
    if (!gr || !part || !lagp || !ahi || !amd || !alo || !yb || !meta) return DELREC_ERR_WORKSPACE;

    // the streamlined hybrid backward (syn_bwd_hyb: ring in LDS over the receivers rounded up
    // to groups of 64, one source per lane, N <= 512). Its lanes take the sources in
    // first-lag order: the 32 lanes an LDS access serves together then gather from nearby
    // slots of one ring row, which keeps them in distinct banks (any assignment gives the
    // same sums: each source's gather runs in its own lane); its blocked W^T and offsets are
    // laid out in that order, so a lane's runs stay adjacent to its neighbours'.
    const size_t hrows = (size_t)((N + 63) / 64 * 64);
    const size_t lds_h = hrows * lay.RP * sizeof(float);
    const bool hyb_fast = hybrid && !lagstep && !hybstep && N <= 512 && (lay.KT == 2 || lay.KT == 4) &&
                          lds_h <= (size_t)max_lds_bytes() && getenv_flag_off("DELREC_SYN_BWD_HYB");
    if (!lagstep && !hybstep) {
        if (hyb_fast) launch_sort_by_first_lag(a->base, a->s_uniform, N, order, s);
        const int* ord = hyb_fast ? order : nullptr;
        if (a->w_bf16) block_transpose<uint16_t>(a->W, wt, N, s, ord); else block_transpose<float>(a->W, wt, N, s, ord);
        if (hybrid) block_transpose<int8_t>(a->offsets, dt, N, s, ord);
        else block_transpose<float>(a->d, dt, N, s);
    }
    // each column's lag range for the lag GEMM, and the smallest offset (meta[1]) the
    // hybrid scan reads
    const size_t NN = (size_t)N * N;
    LagBf16 g{};
    g.T = T; g.B = B; g.Bp = q.Bp; g.N = N; g.Np = q.Np; g.L = a->L; g.Kp = q.Kp; g.KS = q.KS;
    g.ahi = ahi; g.amd = amd; g.alo = alo; g.yb = yb;
    g.planes = a->w_bf16 ? 2 : 3;   // bf16 W: dW leaves rounded to bf16, two gr planes suffice
    g.meta = meta; g.lo = meta + 64; g.rc = meta + 64 + N; g.om = meta + 64 + 2 * N; g.ox = meta + 64 + 3 * N;
    g.d = a->d; g.base = a->base; g.off = a->offsets; g.s = a->s; g.s_uniform = a->s_uniform;
    g.pw = lagp;
    g.pd = lagp + (size_t)q.KS * NN;
    g.ps = a->ds ? lagp + (size_t)2 * q.KS * NN : nullptr;
    launch_lag_cols(g, s);
    if (hybrid && !lagstep && !hybstep) launch_pack_offq(static_cast<const int8_t*>(dt), (size_t)N * lay.NT, meta, offq, s);

    if (hybstep) {
        // reverse-time scan in blocks of P steps, the sources split by first lag: far ones
        // (lof >= P) through one product per block whose rows are (b, step of the block) and one
        // launch for the block's LIF backward; near ones (lof < P) through a second product per
        // block and a per-batch-row chain through the block's steps (hybstep.hip)
        const int KF = taps;
        const HybStepDims hq = hybstep_dims(T, B, N, a->L, a->off_count, KF, num_cus());
        const int planes = a->w_bf16 ? 1 : 2;
        const int fcol = hyb_bwd_far_cols(planes);   // the far GEMM's workgroup columns
        const HybBwdSizes hz = hyb_bwd_sizes(hq, B, num_cus(), fcol);
        uint4* Pw = cv.take<uint4>(planes * hz.planes);
        uint16_t* ghi = cv.take<uint16_t>((size_t)B * hq.lda);
        uint16_t* glo = cv.take<uint16_t>((size_t)B * hq.lda);
        float* npart = cv.take<float>(std::max<size_t>(hz.npart, 1));
        float* fpart = cv.take<float>(std::max<size_t>(hz.fpart, 1));
        float* state = cv.take<float>((size_t)B * N);
        int* lof = cv.take<int>((size_t)N);
        float* h = cv.take<float>((size_t)KF * N);
        int* perm = cv.take<int>((size_t)N);
        int* colf = cv.take<int>((size_t)N);
        uint32_t* wnp = cv.take<uint32_t>((size_t)kHybNearMax * kHybNearMax);
        float* ring = cv.take<float>((size_t)hq.R * N * B);
        if (!Pw || !ghi || !glo || !npart || !fpart || !state || !lof || !h || !perm || !colf || !wnp || !ring)
            return DELREC_ERR_WORKSPACE;
        HybTaps tp{};
        tp.N = N; tp.KF = KF; tp.omin = a->off_min; tp.s = a->s_uniform; tp.base = a->base; tp.lof = lof; tp.h = h;
        launch_hyb_taps(tp, s);
        // the split by first lag: the near counts (lof < 4, lof < 2) come from the caller, who
        // computed them with the forward's own host read; without them the first lags are
        // read back here (one stream sync). The split itself runs on the device.
        int n4 = a->near_lt4, n2 = a->near_lt2;
        if (!a->near_known || n2 < 0 || n2 > n4 || n4 > N) {
            std::vector<int> lof_h(N);
            if (hipMemcpyAsync(lof_h.data(), lof, (size_t)N * sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
                hipStreamSynchronize(s) != hipSuccess)
                return DELREC_ERR_LAUNCH;
            n4 = n2 = 0;
            for (int j = 0; j < N; ++j) {
                n4 += lof_h[j] < 4 ? 1 : 0;
                n2 += lof_h[j] < 2 ? 1 : 0;
            }
        }
        // the longest block (at most kHybBlockMax = 4 steps) whose near sources the chain
        // takes; P = 1 has none (every lof >= 1)
        static_assert(kHybBlockMax == 4, "near counts for blocks of 4 and 2 steps");
        int P = kHybBlockMax, Nn = 0;
        for (;; P /= 2) {
            Nn = P == 4 ? n4 : P == 2 ? n2 : 0;
            if (P == 1 || (Nn <= kHybNearMax && hyb_bwd_near_lds(P, hq.D, Nn) <= (size_t)max_lds_bytes())) break;
        }
        const int Nf = N - Nn;
        launch_hyb_split(lof, N, P, Nn, perm, colf, h, KF, s);
        // The far product on the 4:2 sparse MFMA where it can (bf16 W, blocks of 4 steps, 3 .. 6
        // offsets; DELREC_FAR_SPARSE=0 keeps the dense one), the near one with
        // DELREC_NEAR_SPARSE=1 (at C5's 95 near columns its one 256-column tile at 8 k-splits
        // takes 36 us per block against 27 for the dense 128-column product): a compressed
        // W^T (values, then position words) in place of the dense planes, 256 columns per
        // tile. The plane room (Kt / 8) (Np + 384) holds either form of both parts: the
        // compressed one takes 5 Q / 32 <= 20 D / 128 uint4 per receiver and column.
        const int fq = planes == 1 && P == 4 ? far_sparse_q(hq.D) : 0;
        const size_t proom = (size_t)planes * hz.planes;
        const bool fits_lds = fq && far_sparse_lds(fq) <= (size_t)max_lds_bytes();
        const size_t nwv = Nn > 0 && fits_lds ? far_sparse_wv(hq.Nk, 256, fq) : 0;
        const int ksn = nwv ? far_sparse_splits(B * P, 256, hq.Nk, num_cus()) : 1;
        const char* nse = getenv("DELREC_NEAR_SPARSE");
        const bool nsparse = nwv > 0 && nse && strcmp(nse, "1") == 0 && nwv * 16 < ((size_t)1 << 31) &&
                             (size_t)ksn * B * P * 256 <= hz.npart;
        const int Nnp = nsparse ? 256 : (Nn + 127) / 128 * 128, Nfp = (Nf + fcol - 1) / fcol * fcol;
        const size_t nplane = (size_t)(hq.Kt / 8) * Nnp, fplane = (size_t)(hq.Kt / 8) * Nfp;
        const size_t nsize = nsparse ? nwv + (nwv + 3) / 4 : (size_t)planes * nplane;
        uint4* Pn = Pw;              // near planes: hi (, lo), or the compressed near W^T
        uint4* Pf = Pw + nsize;      // far planes: hi (, lo), or the compressed far W^T
        HybPack pk{};
        pk.N = N; pk.Nk = hq.Nk; pk.D = hq.D; pk.omin = a->off_min; pk.planes = planes;
        pk.W = a->W; pk.w_bf16 = a->w_bf16; pk.off = a->offsets; pk.perm = perm;
        if (Nn > 0) {
            pk.Np = Nnp; pk.c0 = 0; pk.nc = Nn; pk.out = Pn;
            if (nsparse)
                launch_far_sparse_pack(pk, fq, Pn, reinterpret_cast<uint32_t*>(Pn + nwv), s);
            else
                launch_hyb_pack(pk, false, s);
            launch_hyb_near_pack(pk, wnp, s);
        }
        const size_t fwv = Nf > 0 && fits_lds ? far_sparse_wv(hq.Nk, Nfp, fq) : 0;   // Nfp: 256 columns per tile
        FarSparse fs{};
        fs.a0 = ghi; fs.a1 = glo; fs.lda = hq.lda; fs.B = B; fs.rows = B * P; fs.Nk = hq.Nk; fs.Np = Nfp;
        fs.KS = fwv ? far_sparse_splits(B * P, Nfp, hq.Nk, num_cus()) : 1;
        fs.wv = Pf; fs.wi = reinterpret_cast<const uint32_t*>(Pf + fwv); fs.part = fpart;
        const bool sparse = fwv > 0 && getenv_flag_off("DELREC_FAR_SPARSE") &&
                            nsize + fwv + (fwv + 3) / 4 <= proom && fwv * 16 < ((size_t)1 << 31) &&
                            (size_t)fs.KS * B * P * Nfp <= hz.fpart;
        if (!sparse && nsize + (size_t)planes * fplane > proom) return DELREC_ERR_WORKSPACE;
        FarSparse fn = fs;   // the near product: 256 columns, its own splits and partials
        fn.Np = 256; fn.KS = ksn; fn.wv = Pn; fn.wi = reinterpret_cast<const uint32_t*>(Pn + nwv); fn.part = npart;
        // otherwise, for one W plane, blocks of 4 steps and D + 3 <= 8 slices, the dense near
        // product with the history staged once per slice (DELREC_NEAR_BLOCK=0 keeps the plain
        // strided GEMM)
        NearBlock nb{};
        nb.a0 = ghi; nb.a1 = glo; nb.lda = hq.lda; nb.B = B; nb.rows = B * P; nb.Nk = hq.Nk; nb.Np = Nnp;
        nb.w = Pn; nb.part = npart;
        nb.KS = near_block_splits(B * P, Nnp, hq.Nk, num_cus());
        const bool nblock = Nn > 0 && !nsparse && planes == 1 && P == 4 && near_block_ok(hq.D) &&
                            getenv_flag_off("DELREC_NEAR_BLOCK") && (size_t)nb.KS * B * P * Nnp <= hz.npart &&
                            near_block_lds(hq.D) <= (size_t)max_lds_bytes();
        if (Nf > 0) {
            pk.Np = Nfp; pk.c0 = Nn; pk.nc = Nf; pk.out = Pf;
            if (sparse)
                launch_far_sparse_pack(pk, fq, Pf, reinterpret_cast<uint32_t*>(Pf + fwv), s);
            else
                launch_hyb_pack(pk, false, s);
        }
        // gr before the first step (front pad) and past the last one (slices PF + T ..) are 0;
        // every column of the block's slices is written before a product reads them (the far
        // LIF launch writes the far gr and 0 for the near columns, the near chain fills those)
        const int hslices = (int)(hq.lda / hq.Nk);
        launch_hist_zero(ghi, B, hq.lda, hq.Nk, 0, hq.PF, s);
        launch_hist_zero(glo, B, hq.lda, hq.Nk, 0, hq.PF, s);
        launch_hist_zero(ghi, B, hq.lda, hq.Nk, hq.PF + T, hslices, s);
        launch_hist_zero(glo, B, hq.lda, hq.Nk, hq.PF + T, hslices, s);
        // gr == dx unless a dropout mask scales it
        const bool need_gr = a->drop != nullptr;
        LagStepGemm gf{};   // block t0: far G(t0 + 1 + tt), row (b, tt) shifted by tt slices
        gf.a0 = ghi; gf.a1 = glo; gf.lda = hq.lda; gf.rs = hq.Nk; gf.B = B; gf.rows = B * P; gf.rp = P;
        gf.p0 = Pf; gf.p1 = planes > 1 ? Pf + fplane : nullptr; gf.Np = Nfp; gf.Kt = hq.Kt; gf.Nk = hq.Nk;
        // one-plane P: 256 x 256 tiles of 8 waves (128 x 256 tiles of 4 waves with DELREC_FAR256=0)
        const bool far256 = planes == 1 && getenv_flag_off("DELREC_FAR256");
        gf.KS = Nf == 0 ? 1 : sparse ? fs.KS : far256 ? lagstep_gemm256_splits(B * P, Nfp, hq.Kt, num_cus())
                                                      : lagstep_splits(B * P, Nfp, hq.Kt, num_cus(), fcol);
        gf.part = fpart; gf.cm = 0;
        LagStepGemm gn = gf;   // block t0: near G(t0 - P + 2 + tt), the block's steps' t + 1
        gn.p0 = Pn; gn.p1 = planes > 1 ? Pn + nplane : nullptr; gn.Np = Nnp;
        gn.KS = Nn == 0 ? 1 : nsparse ? ksn : nblock ? nb.KS : lagstep_splits(B * P, Nnp, hq.Kt, num_cus());
        gn.part = npart;
        if (getenv("DELREC_LOG_PLAN"))
            fprintf(stderr, "[delrec] hybrid offset-stacked backward: T=%d B=%d N=%d D=%d P=%d; near sources %d "
                    "(product KS=%d%s, %d row tiles, chain of %d-row workgroups); far sources %d (product KS=%d, "
                    "%s tiles, %d row tiles); far LIF grid %d x %d\n", T, B, N, hq.D, P, Nn, Nn > 0 ? gn.KS : 0,
                    nsparse ? " sparse" : nblock ? " block" : "", (B * P + 127) / 128, 2, Nf, Nf > 0 ? gf.KS : 0,
                    sparse ? "sparse 128x256" : far256 ? "256x256" : "128x256",
                    (B * P + (far256 && !sparse ? 255 : 127)) / (far256 && !sparse ? 256 : 128), (hq.Nk + 63) / 64,
                    (B + 15) / 16);
        HybBwd l{};
        l.T = T; l.B = B; l.N = N; l.Nk = hq.Nk; l.KF = KF; l.R = hq.R; l.P = P; l.D = hq.D; l.PF = hq.PF;
        l.lda = hq.lda;
        l.npart = npart; l.KSn = Nn > 0 ? gn.KS : 0; l.Nnp = Nnp; l.Nn = Nn; l.perm = perm;
        l.fpart = fpart; l.KSf = Nf > 0 ? gf.KS : 0; l.Nfp = Nfp; l.Nf = Nf; l.colf = colf;
        l.wnp = wnp;
        l.lof = lof; l.h = h; l.drop = a->drop; l.lif = make_lif(a->lif); l.state = state;
        l.hhi = ghi; l.hlo = glo; l.u_in = a->u; l.gy = a->gy; l.dx = a->dx;
        l.gr = need_gr ? gr : nullptr; l.dbp = a->db ? part : nullptr; l.ring = ring;
        const bool timed = scan_begin(DELREC_WS_SYN_BWD, s);
        bool ok = true;
        for (int t0 = T - 1; t0 >= 0 && ok; t0 -= P) {
            if (Nf > 0) {
                gf.aoff = (size_t)(hq.PF + t0 + 1) * hq.Nk;
                fs.aoff = gf.aoff;
                if (sparse)
                    launch_far_sparse(fs, fq, s);
                else if (far256)
                    launch_lagstep_gemm256(gf, s);
                else
                    launch_lagstep_gemm(gf, 2, s, planes, fcol / 2);
            }
            l.t0 = t0;
            launch_hyb_bwd_farblk(l, s);
            if (Nn > 0) {
                gn.aoff = (size_t)(hq.PF + t0 - P + 2) * hq.Nk;
                fn.aoff = gn.aoff;
                nb.aoff = gn.aoff;
                if (nsparse)
                    launch_far_sparse(fn, fq, s);
                else if (nblock)
                    launch_near_block(nb, hq.D, s);
                else
                    launch_lagstep_gemm(gn, 2, s, planes);
                ok = launch_hyb_bwd_near(l, s);
            }
        }
        scan_end(timed, s);
        if (!ok) return DELREC_ERR_UNSUPPORTED;
        int st = finish_launch();
        if (st) return st;
        if (a->db) launch_reduce_rows(part, B, N, a->db, nullptr, nullptr, s);
        if (a->dW || a->dd || a->ds) {
            launch_lag_bf16(g, need_gr ? gr : a->dx, a->bits, s);
            LagGemm f{};
            f.N = N; f.KS = q.KS; f.W = a->W; f.w_bf16 = a->w_bf16; f.s = a->s; f.s_uniform = a->s_uniform;
            f.pw = g.pw; f.pd = g.pd; f.ps = g.ps; f.perm = lag_bf16_perm(g); f.cls = lag_bf16_cls(g);
            launch_lag_finish(f, a->dW, a->dd, a->ds, s);
        }
        return finish_launch();
    }

    if (lagstep) {
        // reverse-time scan as one lag-stacked GEMM + one LIF launch per step
        const LagStepDims ls = lagstep_dims(T, B, N, a->L);
        uint4* planes = cv.take<uint4>(2 * ls.plane);
        uint16_t* ghi = cv.take<uint16_t>((size_t)B * ls.lda);
        uint16_t* glo = cv.take<uint16_t>((size_t)B * ls.lda);
        float* lpart = cv.take<float>((size_t)ls.KS * B * ls.Np);
        float* fpart = cv.take<float>((size_t)std::max(ls.KSF, 1) * B * ls.P * ls.Np);
        float* state = cv.take<float>((size_t)B * N);
        if (!planes || !ghi || !glo || !lpart || !fpart || !state) return DELREC_ERR_WORKSPACE;
        LagStepPack pk{};
        pk.N = N; pk.Nk = ls.Nk; pk.Np = ls.Np; pk.Lw = ls.Lw;
        pk.W = a->W; pk.w_bf16 = a->w_bf16; pk.d = a->d; pk.base = a->base; pk.off = a->offsets;
        pk.s = a->s; pk.s_uniform = a->s_uniform; pk.out = planes;
        launch_pack_lagw(pk, false, s);
        launch_hist_clear(ghi, B, ls.lda, s);   // incl. gr past the last step
        launch_hist_clear(glo, B, ls.lda, s);
        // packed k order: lag 1 first; the near lags 1 .. P come first
        const size_t kfar = (size_t)ls.P * ls.Nk / 8 * ls.Np;
        LagStepGemm gg{};   // near lags of one step: gr t + 1 .. t + P
        gg.a0 = ghi; gg.a1 = glo; gg.lda = ls.lda; gg.rs = 0; gg.B = B; gg.rows = B; gg.rp = 1;
        gg.p0 = planes; gg.p1 = planes + ls.plane; gg.Np = ls.Np; gg.Kt = ls.P * ls.Nk; gg.KS = ls.KS;
        gg.Nk = ls.Nk; gg.part = lpart;
        LagStepGemm gf = gg;   // far lags of a block: row (b, tt) of step tb + tt reads gr from tb + tt + P + 1
        gf.rows = B * ls.P; gf.rp = ls.P; gf.rs = ls.Nk;
        gf.p0 = planes + kfar; gf.p1 = planes + ls.plane + kfar; gf.Kt = ls.Lf * ls.Nk; gf.KS = ls.KSF;
        gf.part = fpart;
        LagStepLif l{};
        l.T = T; l.B = B; l.N = N; l.Nk = ls.Nk; l.Np = ls.Np; l.KS = ls.KS; l.Lw = ls.Lw;
        l.lda = ls.lda; l.part = lpart; l.fpart = ls.Lf > 0 ? fpart : nullptr;
        l.KSF = ls.Lf > 0 ? ls.KSF : 0; l.P = ls.P;
        l.drop = a->drop; l.lif = make_lif(a->lif);
        l.state = state; l.u = const_cast<float*>(a->u); l.hist = ghi; l.hist2 = glo;
        l.gy = a->gy; l.dx = a->dx; l.gr = gr; l.dbp = part;
        const bool timed = scan_begin(DELREC_WS_SYN_BWD, s);
        for (int t1 = T - 1; t1 >= 0; t1 -= ls.P) {
            const int tb = t1 - ls.P + 1;   // the block's first step (rows of steps < 0 are unused)
            if (ls.Lf > 0) {
                gf.aoff = (size_t)(t1 + 2) * ls.Nk;
                launch_lagblock(gf, 2, s);
            }
            for (int t = t1; t >= std::max(tb, 0); --t) {
                gg.aoff = (size_t)(t + 1) * ls.Nk;
                launch_lagstep_gemm(gg, 2, s);
                l.t = t;
                l.tt = t - tb;
                launch_lagstep_lif(l, false, s);
            }
        }
        scan_end(timed, s);
        int st = finish_launch();
        if (st) return st;
        launch_reduce_rows(part, B, N, a->db, nullptr, nullptr, s);
        if (a->dW || a->dd || a->ds) {
            launch_lag_bf16(g, a->drop ? gr : a->dx, a->bits, s);
            LagGemm f{};
            f.N = N; f.KS = q.KS; f.W = a->W; f.w_bf16 = a->w_bf16; f.s = a->s; f.s_uniform = a->s_uniform;
            f.pw = g.pw; f.pd = g.pd; f.ps = g.ps; f.perm = lag_bf16_perm(g); f.cls = lag_bf16_cls(g);
            launch_lag_finish(f, a->dW, a->dd, a->ds, s);
        }
        return finish_launch();
    }

    SynBwd p{};
    p.T = T; p.B = B; p.N = N; p.L = a->L;
    p.R = lay.R; p.RS = lay.RS; p.RP = lay.RP; p.KT = lay.KT; p.NT = lay.NT;
    p.gy = a->gy; p.u = a->u; p.Wt = wt; p.w_bf16 = a->w_bf16;
    p.dt = hybrid ? nullptr : static_cast<const float*>(dt);
    p.base = a->base;
    p.offt = hybrid ? static_cast<const int8_t*>(dt) : nullptr;
    p.meta = hybrid ? meta : nullptr;
    p.s = a->s; p.s_uniform = a->s_uniform;
    p.drop = a->drop; p.lif = make_lif(a->lif);
    p.dx = a->dx; p.gr = gr; p.part = part; p.gring = lay.lds_ring ? nullptr : gring;
    const bool timed = scan_begin(DELREC_WS_SYN_BWD, s);
    // room for rows that also mirror the offset span (up to L more slots): the kernel
    // takes the no-wrap form when the span it finds fits
    const size_t lds_hx = std::max(lds_h, std::min((size_t)max_lds_bytes(),
                                                   hrows * (size_t)(2 * lay.R + lay.KT + 1) * sizeof(float)));
    p.ldsf = (int)(lds_hx / sizeof(float));
    p.offq = hybrid ? offq : nullptr;
    p.order = hyb_fast ? order : nullptr;
    // (no fallback from the hybrid kernels: their operands are in first-lag order). Where every
    // lag is >= 1 and the offsets span at most 12 steps, the offset-stacked form (one MAC per
    // connection; DELREC_SYN_BWD_HYB_G=0 keeps the per-tap gather)
    const bool hyb_g = hyb_fast && a->d_min >= a->s_uniform - 1.0f && a->off_count > 0 &&
                       getenv_flag_off("DELREC_SYN_BWD_HYB_G") &&
                       launch_syn_bwd_hyb_g(p, a->off_count, (size_t)max_lds_bytes(), s);
    const bool ok = hyb_g || (hyb_fast ? launch_syn_bwd_hyb(p, lay.block, lds_hx, s) : launch_syn_bwd(p, lay.block, lay.lds, s));
    scan_end(timed && ok, s);
    if (!ok) return DELREC_ERR_UNSUPPORTED;
    int st = finish_launch();
    if (st) return st;
    launch_reduce_rows(part, B, N, a->db, nullptr, nullptr, s);
    if (a->dW || a->dd || a->ds) {
        launch_lag_bf16(g, a->drop ? gr : a->dx, a->bits, s);
        LagGemm f{};
        f.N = N; f.KS = q.KS; f.W = a->W; f.w_bf16 = a->w_bf16; f.s = a->s; f.s_uniform = a->s_uniform;
        f.pw = g.pw; f.pd = g.pd; f.ps = g.ps; f.perm = lag_bf16_perm(g); f.cls = lag_bf16_cls(g);
        launch_lag_finish(f, a->dW, a->dd, a->ds, s);
    }
    return finish_launch();
}

int delrec_lif_fwd(const delrec_lif_fwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || !a->x || !a->y || !a->u || !lif_ok(a->lif))
        return DELREC_ERR_ARG;
    launch_lif(true, a, nullptr, make_lif(a->lif), static_cast<hipStream_t>(stream));
    return finish_launch();
}

int delrec_lif_bwd(const delrec_lif_bwd_args* a, void* stream) {
    if (!a || a->T <= 0 || a->B <= 0 || a->N <= 0 || !a->gy || !a->u || !a->dx || !lif_ok(a->lif))
        return DELREC_ERR_ARG;
    launch_lif(false, nullptr, a, make_lif(a->lif), static_cast<hipStream_t>(stream));
    return finish_launch();
}

int delrec_delay_grad(const float* C, const float* W, const float* d, float sigma, int32_t N,
                      int32_t Lm, float* dd, void* stream) {
    if (!C || !W || !d || !dd || N <= 0 || Lm < 1 || !(sigma >= 0.0f)) return DELREC_ERR_ARG;
    launch_delay_grad(C, W, d, sigma, N, Lm, dd, static_cast<hipStream_t>(stream));
    return finish_launch();
}

int delrec_max_post(const float* x, int32_t n, uint32_t* ticket, void* stream) {
    if (!x || n <= 0 || !ticket) return DELREC_ERR_ARG;
    uint32_t t = 0;
    unsigned long long* slot = nullptr;
    if (int st = max_slot(t, slot)) return st;
    launch_max_to_host(x, n, t, slot, static_cast<hipStream_t>(stream));
    *ticket = t;
    return finish_launch();
}

int delrec_max_take(uint32_t ticket, float* out, int32_t timeout_ms) {
    if (!out || ticket == 0) return DELREC_ERR_ARG;
    MaxRing& r = max_ring();
    if (!r.ok) return DELREC_ERR_DEVICE;
    const unsigned long long* slot = r.host + ticket % DELREC_MAX_SLOTS;
    const auto t0 = std::chrono::steady_clock::now();
    for (uint64_t spin = 1;; ++spin) {
        const unsigned long long v = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
        const uint32_t t = (uint32_t)v;
        if (t == ticket) {
            const uint32_t bits = (uint32_t)(v >> 32);
            memcpy(out, &bits, sizeof(bits));
            return DELREC_OK;
        }
        if (t != 0 && (int32_t)(t - ticket) > 0) return DELREC_ERR_STALE;   // a later post's value
        if ((spin & 1023) == 0) {
            const auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(
                                std::chrono::steady_clock::now() - t0).count();
            if (ms >= timeout_ms) return DELREC_ERR_PENDING;
            if (ms >= 1) std::this_thread::yield();
        }
    }
}

int delrec_scan_timing(int32_t capacity) {
    if (capacity < 0) return DELREC_ERR_ARG;
    scan_release();
    if (capacity == 0) return DELREC_OK;
    g_scan.ev.assign((size_t)2 * capacity, nullptr);
    for (hipEvent_t& e : g_scan.ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            e = nullptr;
            scan_release();
            return DELREC_ERR_DEVICE;
        }
    }
    g_scan.kind.assign((size_t)capacity, 0);
    return DELREC_OK;
}

int delrec_scan_timing_read(float* ms, int32_t* kinds, int32_t capacity) {
    if (!ms || !kinds || capacity < 0) return -DELREC_ERR_ARG;
    const int n = std::min(g_scan.used, (int)capacity);
    for (int k = 0; k < n; ++k) {
        if (hipEventSynchronize(g_scan.ev[2 * k + 1]) != hipSuccess) return -DELREC_ERR_DEVICE;
        if (hipEventElapsedTime(&ms[k], g_scan.ev[2 * k], g_scan.ev[2 * k + 1]) != hipSuccess)
            return -DELREC_ERR_DEVICE;
        kinds[k] = g_scan.kind[k];
    }
    return n;
}

}  // extern "C"
