// Kernel parameter blocks and launchers shared by the HIP sources and the C ABI layer.
#pragma once

#include "common.h"

namespace delrec {

struct AxFwd {
    int T, B, N, L;
    int G, NZ, CHS;            // lanes per receiver, padded z length, streamed chunk
    const float* x;
    const void* W;             // row-major (resident form)
    const void* Wt;            // transposed copy (streamed form)
    int w_bf16;
    const float* bias;
    const float* d;
    const float* s;
    float s_uniform;
    const float* drop;
    int taps;
    const int* lag;
    const float* frac;
    Lif lif;
    float* y;
    float* u;
    float* rec;
    float* z;
    uint32_t* bits;
    unsigned long long* mx_slot;   // NULL, or the readback slot workgroup 0 writes max d into
    uint32_t mx_ticket;
};

struct AxBwd {
    int T, B, N, L;
    int G, NZ, CHS, R, NP;     // lanes per source, padded gr length, streamed chunk, ring slots, ring pitch
    const float* gy;
    const float* u;
    const uint32_t* bits;
    const void* W;
    int w_bf16;
    const float* d;
    const float* s;
    float s_uniform;
    const float* drop;
    int mode;
    const int* lag;
    Lif lif;
    float* dx;
    float* gr;                 // (T,B,N) dL/drec, written when it differs from dx, else NULL
    float* part;               // [3][B][N] per-row partials of db, dd, ds
    float* gz;                 // (T,B,N) dL/dz of the tiled scan, read by the delay-gradient pass
};

struct SynFwd {
    int T, B, N, L, R, NP, NF;  // ring slots / pitch, fired-list capacity
    const float* x;
    const void* Wt;             // transposed: Wt[o*N + i] = W[i, o]
    int w_bf16;
    const float* bias;
    const float* dt;            // transposed delays dt[o*N + i], or NULL (hybrid)
    const float* base;
    const int8_t* offt;         // transposed hybrid offsets offt[o*N + i]
    const float* s;
    float s_uniform;
    const float* drop;
    Lif lif;
    float* y;
    float* u;
    uint32_t* bits;
    float* gring;               // global ring [B][R][N] when the ring does not fit LDS, else NULL
    // gather form (rings too large for LDS): W / d / offsets in row-blocked copies,
    // W[i][j] at ((j/16)*N + i)*16 + j%16; HW history words, KT taps per window
    int HW, KT;
    const void* Wr;
    const float* dr;
    const int8_t* offr;
    // hybrid with bf16 W: W^T and the offsets^T packed per connection,
    // wpk[o*N + i] = bf16(W[i, o]) << 16 | uint8(offset[i, o]), else NULL
    const uint32_t* wpk;
};

struct SynBwd {
    int T, B, N, L;
    int R;                      // ring slots (time mod R), R >= L
    int RS;                     // slots per ring row incl. the KT mirror slots
    int RP;                     // ring row pitch (floats)
    int KT;                     // taps walked per connection (2, 4, 8, 12, 16)
    int NT;                     // rows of the blocked W^T / d^T / offsets^T (multiple of 16)
    const float* gy;
    const float* u;
    const void* Wt;             // blocked W^T: W[i][j] at ((i/16)*N + j)*16 + i%16, 0 for i >= N
    int w_bf16;
    const float* dt;            // blocked d^T (synaptic), or NULL
    const float* base;          // hybrid base (N)
    const int8_t* offt;         // blocked hybrid offsets^T (int8), or NULL
    const int* meta;            // hybrid: meta[1] = smallest offset
    const float* s;
    float s_uniform;
    const float* drop;
    Lif lif;
    float* dx;
    float* gr;                  // (T,B,N) dL/drec (always written: the dW / dd GEMM reads it)
    float* part;                // [B][N] db partials
    float* gring;               // global ring [B][N][RP] when it does not fit LDS, else NULL
    int ldsf;                   // floats of LDS the hybrid backward was given
    const int* order;           // hybrid: source of each lane slot (first-lag order), or NULL
    const uint8_t* offq;        // blocked (offset - smallest offset) * 4 as bytes (hybrid), or NULL
};

// the split partials of the lag GEMM and what dd / ds are formed from
struct LagGemm {
    int N, KS;
    const void* W;
    int w_bf16;
    const float* s;
    float s_uniform;
    float* pw;                  // [KS][N][N] partial sum_l h * C_l
    float* pd;                  // [KS][N][N] partial sum_l sign * C_l, or NULL
    float* ps;                  // [KS][N][N] partial sum_l dh/ds * C_l, or NULL
    const int* perm;            // column order of the partials (event-driven form), or NULL
    const int* cls;             // and its class sizes (silent, sparse, dense), or NULL
};

// bf16-MFMA lag-correlation GEMM (lagmm.hip): operands packed in the k-blocked layout,
// batch padded to Bp = 32n (KS = Bp / 32 chunk partials)
struct LagBf16 {
    int T, B, Bp, N, Np, L, Kp, KS;
    const uint4* ahi;            // gr_hi (Kp, Np) k-blocked
    const uint4* amd;            // gr_mid
    const uint4* alo;            // gr_lo
    const uint4* yb;             // shifted spikes Y' (Kp, Np) k-blocked
    int* meta;                   // meta[0] = widest column lag range, meta[1] / [2] = smallest /
                                 // largest offset
    int* lo;                     // [N] first lag of each column
    int* rc;                     // [N] number of lags of each column
    int* om;                     // [N] smallest offset of each column (hybrid)
    int* ox;                     // [N] largest offset of each column (hybrid)
    const float* d;              // row-major, or NULL (hybrid)
    const float* base;
    const int8_t* off;
    const float* s;
    float s_uniform;
    float* pw;                   // [KS][N][N] partial sum_l h * C_l
    float* pd;                   // [KS][N][N] partial sum_l sign * C_l
    float* ps;                   // [KS][N][N] partial sum_l dh/ds * C_l, or NULL
    int planes;                  // gr planes multiplied: 3 (hi, mid, lo), or 2 (hi, mid) for bf16 W
    // the event-driven form (set by launch_lag_bf16): the sparse tiles' spike code words
    // [t][Bp / 64][4][Np] and the column order perm (class sizes cls[0..2]); NULL otherwise
    const uint32_t* ycode;
    const int* perm;
    const int* cls;
};

// lag-stacked per-step GEMM scans (lagstep.hip)
struct LagStepPack {             // M_l planes (hi, lo) of the forward or backward operand
    int N, Nk, Np, Lw;
    const void* W;
    int w_bf16;
    const float* d;              // row-major, or NULL (hybrid)
    const float* base;
    const int8_t* off;
    const float* s;
    float s_uniform;
    uint4* out;                  // 2 planes of (Lw * Nk / 8) x Np uint4
};

struct LagStepGemm {
    const uint16_t* a0;          // history (bf16); output row r reads k = 0 at element
    const uint16_t* a1;          //   (r / rp) * lda + (r % rp) * rs + aoff; a1: lo plane or NULL
    size_t lda, rs;
    size_t aoff;
    int B;                       // batch rows of the history
    int rows, rp;                // output rows (B * rp), rows per batch row
    const uint4* p0;             // packed M planes (first k-block of the product's lags)
    const uint4* p1;
    int Np, Kt, KS;
    int Nk;                      // padded neurons per history slice / lag slice
    float* part;                 // [KS][rows][Np], or [KS][Np][rows] when cm
    int cm;                      // column-major partials (a consumer that reads columns)
};

struct FarSparse {               // the hybrid backward's far product on the 4:2 sparse MFMA
    const uint16_t* a0;          // gr history, hi / lo planes [b][slice][Nk]; slice 0 of the
    const uint16_t* a1;          //   block's product at element aoff of each batch row
    size_t lda, aoff;
    int B, rows;                 // batch rows, product rows B * 4 (row b * 4 + step of the block)
    int Nk, Np, KS;              // receivers (multiple of 32), far columns (multiple of 256), k splits
    const uint4* wv;             // compressed W^T values [chunk][q][column block][lane]
    const uint32_t* wi;          // their position words, same order
    float* part;                 // [KS][rows][Np]
};

struct NearBlock {               // the hybrid backward's near product of a block (dense, bf16 W)
    const uint16_t* a0;          // gr history, hi / lo planes [b][slice][Nk]; the block's first
    const uint16_t* a1;          //   row step's slice at element aoff of each batch row
    size_t lda, aoff;
    int B, rows;                 // batch rows, product rows B * 4 (row b * 4 + step of the block)
    int Nk, Np, KS;              // receivers (multiple of 32), near columns (multiple of 128), k splits
    const uint4* w;              // W^(e) planes, k-blocked [(e Nk + i) / 8][Np], e < D
    float* part;                 // [KS][rows][Np]
};

struct LagStepLif {
    int T, B, N, Nk, Np, KS, t, Lw;
    size_t lda;
    const float* part;           // [KS][B][Np] near-lag partials of step t
    const float* fpart;          // [KSF][B * P][Np] far-lag partials of step t's block, or NULL
    int KSF, P, tt;              // far splits, steps per block, t's row in its block
    const float* x;              // forward input
    const float* bias;
    const float* drop;
    Lif lif;
    float* state;                // [B][N]: v (forward) or lambda (backward)
    float* y;
    float* u;                    // forward output / backward input
    uint32_t* bits;
    uint16_t* hist;              // forward: spikes; backward: gr hi
    uint16_t* hist2;             // backward: gr lo
    const float* gy;
    float* dx;
    float* gr;
    float* dbp;                  // [B][N] db partials
};

// offset-stacked hybrid scans (hybstep.hip)
struct HybPack {                 // W^(e) planes of the forward or backward operand
    int N, Nk, Np, D, omin, planes;
    const void* W;
    int w_bf16;
    const int8_t* off;
    uint4* out;                  // planes of (D * Nk / 8) x Np uint4
    // backward only, optional: output column c holds source perm[c0 + c] for c < nc (0 past)
    const int* perm;
    int c0, nc;
};

struct HybTaps {                 // each source's first lag and tap weights at the smallest offset
    int N, KF, omin;
    float s;
    const float* base;
    int* lof;                    // [N]
    float* h;                    // [KF][N]
};

struct HybLif {                  // one forward step of the offset-stacked scan
    int T, B, N, Nk, Np, KS, t, D, KF, R;
    size_t lda;                  // history row pitch (elements)
    const float* part;           // [KS][B][Np] partials of step t's product
    const int* lof;
    const float* h;
    const float* bias;
    const float* drop;
    Lif lif;
    float* state;                // [B][N]: v
    uint16_t* hhi;               // z history planes
    uint16_t* hlo;
    const float* x;
    float* y;
    float* u;
    uint32_t* bits;
    uint64_t* hist;              // [HW][B][N] spike-history words
};

// The hybrid backward with the sources split by first lag (hybstep.hip): "near" sources
// (lof < P) take G(t + 1) from a per-step product over their columns, "far" ones (lof >= P)
// from one product per block of P steps whose rows are (batch row, step of the block); both
// land in a ring of G_j(tau) that the LIF launch of each step reads.
struct HybBwd {
    int T, B, N, Nk, KF, R, P, D;
    int PF;                      // zero slices before slice 0 of the gr history
    size_t lda;                  // history row pitch (elements)
    int t0;                      // the block's latest step (its steps are t0 - P + 1 .. t0)
    const float* npart;          // [KSn][B * P][Nnp] partials of the block's near product
    int KSn, Nnp, Nn;            //   (row (b, tt): G(t0 - P + 2 + tt))
    const int* perm;             // [N]: the near sources ascending, then the far ones ascending
    const float* fpart;          // [KSf][B * P][Nfp] partials of the block's far product
    int KSf, Nfp, Nf;            //   (row (b, tt): G(t0 + 1 + tt))
    const int* colf;             // [N]: far column of source j (-1: near)
    const uint32_t* wnp;         // [Nn][Nn] W[perm[ci], perm[c]] between near neurons, the
                                 //   low 4 bits replaced by the offset - omin
    const int* lof;
    const float* h;              // [KF][N]
    const float* drop;
    Lif lif;
    float* state;                // [B][N] lambda
    uint16_t* hhi;               // gr history planes
    uint16_t* hlo;
    const float* u_in;
    const float* gy;
    float* dx;
    float* gr;                   // (T, B, N) when it differs from dx, else NULL
    float* dbp;                  // [B][N] db partials, or NULL
    float* ring;                 // [R][N][B]: G_j(tau) at slot tau mod R
};
constexpr int kHybBlockMax = 4;  // steps per block of the hybrid backward (P <= this)
constexpr int kHybNearMax = 160; // near sources the per-block near chain takes (LDS)
void launch_hyb_bwd_farblk(const HybBwd& a, hipStream_t stream);
bool launch_hyb_bwd_near(const HybBwd& a, hipStream_t stream);
void launch_hyb_near_pack(const HybPack& a, uint32_t* wnp, hipStream_t stream);
// perm / colf of the split by first lag (near: lof < P) on the device; taps h -> NaN when the
// device's near count differs from Nn
void launch_hyb_split(const int* lof, int N, int P, int Nn, int* perm, int* colf, float* h, int KF,
                      hipStream_t stream);
size_t hyb_bwd_near_lds(int P, int D, int Nn);

struct HybScat {                 // the hybrid forward as a scatter on arrival (bf16 W)
    int T, B, N, D, KF, R, RP, omin;   // KF: the compiled run length; R >= D + KF - 1 ring slots, a power of two
    int sh;                      // > 0: the offset field is (offset - omin) << sh, sh = log2 of the slot
                                 // bytes, R slots being 2^16 bytes
    const float* x;
    const float* bias;
    const float* drop;
    Lif lif;
    const uint32_t* wpk;         // wpk[o * N + i] = bf16(W[i, o]) << 16 | uint8(offset[i, o] - omin) << sh
    const int* lof;              // [N] first lag of each source
    const float* h;              // [KF][N] its tap weights (0 past its triangle)
    float* y;
    float* u;
    uint32_t* bits;
};
bool launch_hyb_fwd_arrive(const HybScat& a, int npt, int hw, int block, size_t lds, hipStream_t stream);

// Linear layer on spike inputs (spikelinear.hip): out[t][b][m] = bias[m] + sum_k y W[m][k]
// The input neurons of a spike Linear in activity order (silent ones first, then those that
// spike, stably; positions K .. KP-1 padding, perm -1): cnt [2][KP] counts, the order, the
// class sizes (cls[0] = silent neurons), and the spike words regathered in that order
// (B, ceil(T/32), KP). KP = K rounded up to 256.
struct SpikeOrder {
    int* cnt;
    int* perm;
    int* cls;
    uint32_t* bits;
};
int spike_order_kp(int K);
size_t spike_order_ws(int T, int B, int K);
SpikeOrder spike_order_carve(void* base, int T, int B, int K);
void launch_spike_order(const uint32_t* bits, int T, int B, int K, const SpikeOrder& o, hipStream_t stream);
// rows x M fp32 -> rows x 3M bf16 [hi | lo | hi] (the input gradient's split operand)
void launch_spike_linear_dx_split(const float* g, size_t rows, int M, uint16_t* out, hipStream_t stream);
void launch_col_order(const int* cnt, int N, int Np, int* perm, int* cls, hipStream_t stream);

struct SpikeLinear {
    int T, B, K, M, Kp, Mp;      // Kp = K rounded up to 32, Mp = M rounded up to 128
    const uint32_t* bits;        // (B, ceil(T/32), ldb) spike words
    int ldb;                     // their row pitch (K, or the order's KP)
    const int* perm;             // input neuron of each position (activity order), or NULL
    const int* cls;              // the order's class sizes (stages below cls[0] / 32 are skipped)
    const float* W;              // (M, K) fp32
    const float* bias;           // (M) or NULL
    float* out;                  // (T, B, M) fp32
};
void spike_linear_dims(SpikeLinear& p);
size_t spike_linear_ws(int K, int M);   // bytes of the packed W^T planes
void launch_spike_linear(const SpikeLinear& p, uint4* wp, hipStream_t stream);
struct SpikeLinearDw {           // dW[m][k] = sum_{t,b} g[t][b][m] y[t][b][k]
    int T, B, K, M, Kp, Mp, KS;  // Kp, Mp rounded up to 128; KS splits of the (b, word) stages
    const uint32_t* bits;        // (B, ceil(T/32), ldb)
    int ldb;                     // their row pitch (K, or the order's KP)
    const int* perm;             // input neuron of each column position, or NULL
    const int* cls;              // the order's class sizes (tiles of silent neurons: zeros)
    const float* g;              // (T, B, M)
    float* dW;                   // (M, K)
    float* part;                 // [KS][M][K] when KS > 1
    uint4* gp;                   // g's bf16 planes [3][B][ceil(T/32)][4][M] (8 steps per uint4)
};
struct ReadoutCe {               // time reduction (+ leaky integrator) + cross-entropy, fused
    int T, B, C;
    const float* logits;         // (T, B, C)
    const int64_t* labels;       // (B)
    int reduce;                  // DELREC_READOUT_*
    int integrator;              // 0 none, 1 v = decay v + x, 2 v = v + (x - v) / tau
    float tau, decay, in_scale;  // in_scale: d v_t / d x_t (1, or 1 / tau for form 2)
    float* out;                  // (B, C) or NULL
    float* dlogits;              // (T, B, C)
    float* rowloss;              // (B) workspace
    float* loss;                 // (1)
};
void launch_readout_ce(const ReadoutCe& p, hipStream_t stream);
void spike_linear_dw_dims(SpikeLinearDw& p, int cus);
size_t spike_linear_dw_planes(int T, int B, int M);   // uint4 of g's planes in the workspace
size_t spike_linear_dw_ws(int T, int B, int K, int M, int cus);
void launch_spike_linear_dw(const SpikeLinearDw& p, hipStream_t stream);

struct HybStepDims {
    int Nk, Np, D, KF, R, HW, Kt, KS, P, PF;
    size_t lda, plane;
    bool ok;
};
// the backward's largest near / far partials and packed planes over every split of the
// sources (the split is only known once the first lags are)
struct HybBwdSizes {
    size_t npart, fpart, planes;   // floats, floats, uint4 per W plane set (near + far)
};
HybBwdSizes hyb_bwd_sizes(const HybStepDims& q, int B, int cus, int fcol);
int hyb_bwd_far_cols(int planes);   // far columns per GEMM tile: 256 for one W plane, else 128

HybStepDims hybstep_dims(int T, int B, int N, int L, int D, int KF, int cus);
void launch_hyb_pack(const HybPack& a, bool fwd, hipStream_t stream);
void launch_hyb_taps(const HybTaps& a, hipStream_t stream);
void launch_hyb_lif(const HybLif& l, int hw, hipStream_t stream);   // forward step

// far product on the sparse MFMA: Q = ceil(D / 2) sparse products per 32 receivers (0: the
// offset count is outside the supported 3 .. 6); blocks of 4 steps, bf16 W only
int far_sparse_q(int D);
size_t far_sparse_lds(int Q);
size_t far_sparse_wv(int Nk, int Np, int Q);            // uint4 of values (and uint32 of positions)
int far_sparse_splits(int rows, int Np, int Nk, int cus);
void launch_far_sparse_pack(const HybPack& a, int Q, uint4* wv, uint32_t* wi, hipStream_t stream);
bool launch_far_sparse(const FarSparse& g, int Q, hipStream_t stream);
// near product of a block, dense with the history staged once per slice: D offsets with
// D + 3 <= 8, blocks of 4 steps, one W plane
bool near_block_ok(int D);
size_t near_block_lds(int D);
int near_block_splits(int rows, int Np, int Nk, int cus);
bool launch_near_block(const NearBlock& g, int D, hipStream_t stream);
int lagstep_splits(int B, int Np, int Kt, int cus, int nc = 128);   // nc: workgroup columns
int lagstep_block();
size_t lagstep_gemm_lds(int pa, int pb = 2, int wn = 64);
void launch_pack_lagw(const LagStepPack& a, bool fwd, hipStream_t stream);
void launch_hist_zero(uint16_t* h, int B, size_t lda, int Nk, int t0, int t1, hipStream_t stream);
void launch_hist_clear(uint16_t* h, int B, size_t lda, hipStream_t stream);
// pb = 1: one P plane (p1 unused)
void launch_lagstep_gemm(const LagStepGemm& g, int pa, hipStream_t stream, int pb = 2, int wn = 64);
// 256 x 256 tiles for a two-plane A and a one-plane P (Np a multiple of 256)
int lagstep_gemm256_splits(int rows, int Np, int Kt, int cus);
void launch_lagstep_gemm256(const LagStepGemm& g, hipStream_t stream);
void launch_lagstep_lif(const LagStepLif& l, bool fwd, hipStream_t stream);
int lagblock_splits(int B, int Np, int Nk, int cus);
void launch_lagblock(const LagStepGemm& g, int pa, hipStream_t stream);

// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per kernel and size (cached; the
// library is used from one host thread at a time)
void ensure_lds(const void* fn, size_t bytes);

bool launch_axonal(bool fwd, const AxFwd* fa, const AxBwd* ba, int ch, bool res, int hw,
                   int grid, int block, size_t lds, hipStream_t stream);
bool launch_axonal_tiled(bool fwd, const AxFwd* fa, const AxBwd* ba, int ri, int nj, int cj, int hw,
                         int grid, int block, size_t lds, hipStream_t stream);
// spike-driven forward for N <= 256: nw waves of 32 source columns, ri receivers per lane
bool launch_axonal_fwd_wave(const AxFwd& p, int ri, int hw, int nw, int grid, size_t lds,
                            hipStream_t stream);
// its specialisation for soft taps of a uniform half-width (kf >= ceil(2s) lags of
// non-zero weight, one history word), decay charge, hard reset to 0, no recurrent-input
// output
bool launch_axonal_fwd_wave_fast(const AxFwd& p, int ri, int kf, int nw, int grid, hipStream_t stream);
// tiled backward for soft taps of a uniform half-width (kf >= ceil(2s) lags of non-zero
// weight, one history word), ATan surrogate, decay charge, hard reset to 0, not detached;
// the ring holds R + kf - 1 slots
bool launch_axonal_bwd_tiled_fast(const AxBwd& p, int ri, int nj, int cj, int kf, int grid, int block,
                                  size_t lds, hipStream_t stream);
__host__ __device__ int axonal_delay_segments(int T);
void launch_reduce_rows(const float* part, int B, int N, float* o0, float* o1, float* o2,
                        hipStream_t stream);

// The reductions after the axonal backward scan, in two launches:
//   launch_axonal_bwd_tail: the dd / ds per-row partials (part[1], part[2]) from the tiled
//     scan's gz and the spike bits (ndelay blocks), beside the dW GEMM
//     dW[i,j] = sum_k A[k,i] * Bz[k,j] over K rows, split into ks chunks of partials (ndw
//     blocks);
//   launch_axonal_bwd_sums: dW = the sum of those partials (nsum blocks), beside the batch
//     sums of the per-row partials into o0, o1, o2 (3 * ceil(N / 16) blocks; a null output is
//     skipped).
struct AxTail {
    const float* A;     // (K, N): dL/drec
    const float* Bz;    // (K, N): z
    int K, kchunk, ks, tiles;
    float* gpart;       // [ks][N][N]
    float* dW;
    int ndw, ndelay, nsum, nbx;
    float* o0;
    float* o1;
    float* o2;
};
void launch_axonal_bwd_tail(const AxBwd& p, const AxTail& q, hipStream_t stream);
// *slot = ticket | max(x[0 .. n)) bits << 32, one system-scope 8-byte store (host memory)
void launch_max_to_host(const float* x, int n, uint32_t ticket, unsigned long long* slot, hipStream_t stream);
void launch_axonal_bwd_sums(const AxTail& q, const float* part, int B, int N, hipStream_t stream);

void launch_syn_fwd(const SynFwd& a, int block, size_t lds, hipStream_t stream);
// wpk[o*N + i] = W[i*N + o] (bf16 bits) << 16 | uint8(off[i*N + o] - omin) << sh (low 16 bits);
// D > 0: a connection whose off - omin lies outside [0, D) gets a NaN weight and offset 0
// peaks.hip: a register-only MFMA loop (kind 0: bf16 16x16x32, 1: fp32 16x16x4) over
// `blocks` workgroups; returns the flops one launch issues. sink: blocks * 512 floats.
int peak_mfma_blocks(int cus);
double launch_peak_mfma(int kind, int iters, float* sink, int blocks, hipStream_t stream);
// wpk[o * pitch + i]: bf16 W[i, o] << 16 | the offset's low field (see pack_hybrid_kernel);
// pitch >= N (0: N), columns N .. pitch-1 weight 0
void launch_pack_hybrid(const uint16_t* W, const int8_t* off, int N, uint32_t* wpk, hipStream_t stream,
                        int omin = 0, int sh = 0, int D = 0, int pitch = 0);
// event-driven forward, ring in LDS, one receiver per lane, kf >= ceil(2 s_max) taps
bool launch_syn_fwd_scatter(const SynFwd& a, int kf, int block, size_t lds, hipStream_t stream);
bool launch_syn_bwd(const SynBwd& a, int block, size_t lds, hipStream_t stream);
// hybrid backward, ring in LDS over ceil(N/64)*64 rows, one source per lane (N <= 512),
// KT = 2 or 4; false when it does not apply
// offq[q] = (offt[q] - meta[1]) * 4 (the byte slot offsets of the hybrid backward)
void launch_pack_offq(const int8_t* offt, size_t n, const int* meta, uint8_t* offq, hipStream_t stream);
// order[k] = the source with the k-th smallest (first lag lob, index) of the hybrid backward
// (one workgroup; N <= 1024)
void launch_sort_by_first_lag(const float* base, float s, int N, int* order, hipStream_t stream);
bool launch_syn_bwd_hyb(const SynBwd& a, int block, size_t lds, hipStream_t stream);
// the offset-stacked form of the hybrid backward (every lag >= 1, D offsets, N <= 512); false
// when it does not apply (the caller then takes launch_syn_bwd_hyb)
bool launch_syn_bwd_hyb_g(const SynBwd& a, int D, size_t max_lds, hipStream_t stream);
size_t syn_bwd_hyb_g_lds(int N, int L, int D, int* gs);
// each column's lag range (lo, rc, om) and meta[0..1]
void launch_lag_cols(const LagBf16& a, hipStream_t stream);
// packs gr / spikes, then the lag GEMM into a.pw / a.pd / a.ps
void launch_lag_bf16(const LagBf16& a, const float* gr, const uint32_t* bits, hipStream_t stream);
// whether launch_lag_bf16 takes the event-driven form (spike columns by class), and the
// column order and class sizes of the partial sums it leaves there (else NULL)
bool lag_bf16_sparse(const LagBf16& a);
const int* lag_bf16_perm(const LagBf16& a);
const int* lag_bf16_cls(const LagBf16& a);
// dW = sum_k pw; dd = W/s^2 * sum_k pd; ds[j] = sum_i W[i,j] * sum_k ps[i,j]
void launch_lag_finish(const LagGemm& a, float* dW, float* dd, float* ds, hipStream_t stream);

void launch_lif(bool fwd, const delrec_lif_fwd_args* fa, const delrec_lif_bwd_args* ba,
                const Lif& k, hipStream_t stream);
void launch_delay_grad(const float* C, const float* W, const float* d, float sigma, int N,
                       int Lm, float* dd, hipStream_t stream);

}  // namespace delrec
