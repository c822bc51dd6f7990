// The hybrid backward's per-block far product on the 4:2 sparse MFMA of gfx950
// (v_smfmac_f32_16x16x64_bf16).
//
// For a block of P = 4 steps starting at t0 (reverse time), the far sources j need
//   G_j(tau) = sum_i sum_e W^(e)_ij gr_i(tau + e),   tau = t0 + 1 + tt, tt < 4,
// with W^(e) = W [off_ij - omin == e]: every connection has exactly one offset, so along the
// contraction k = (receiver i, offset e) each row j of W^T holds one non-zero per receiver.
// Grouping k in fours as (receivers 2p, 2p + 1) x (offsets 2q, 2q + 1) leaves at most two
// non-zeros per group, which is the sparse MFMA's 4:2 format: W^T is the compressed operand
// (rows j), the gr history the dense one (columns (b, tt)), and D offsets cost Q = ceil(D / 2)
// sparse products of K = 64 per 32 receivers instead of D dense products of K = 32 -- 0.6 of
// the MFMA issue at D = 5, and the history is read once per block slice instead of once per
// (step, offset).
//
// Operand layouts (lane layout of the instruction: A lane l = row l % 16, compressed values
// 2g, 2g + 1 belong to sparsity group 4 (l / 16) + g, their 2-bit positions in bits 4g .. 4g + 3
// of the index word; B lane l = column l % 16, slot s = k 32 (s / 8) + 8 (l / 16) + s % 8;
// C lane l = column l % 16, element e = row 4 (l / 16) + e):
//  - group G of a 64-k product covers receiver pair pr(G) = 4 (G' / 2) + G' % 2 (+ 2 for
//    G >= 8, G' = G mod 8) of the 32-receiver chunk at offsets 2q, 2q + 1, positions
//    (2p, 2q), (2p + 1, 2q), (2p, 2q + 1), (2p + 1, 2q + 1); so lane group g of the dense
//    operand holds pairs 4g .. 4g + 3 = receivers 8g .. 8g + 7 at slices tau + 2q and
//    tau + 2q + 1: two 16-byte reads of the batch-major history, interleaved by 32-bit words;
//  - the compressed W^T is stored per (chunk, q, 16-column block, lane): 8 bf16 (16 bytes) and
//    a 32-bit index word (positions in the low 16 bits), so a wave loads a fragment as one
//    1 KB and one 256-byte run.
// Precision: bf16 W is exact; gr enters as its hi and lo bf16 planes (two products), fp32
// accumulation -- the dense kernel's arithmetic, summed in another order.
//
// Workgroup: 4 waves (one per SIMD), a tile of 256 columns j x 128 rows (b, tt) (32 batch
// rows); wave (wj, wc) owns 128 j x 64 rows: 8 x 4 blocks of 16 x 16, 128 accumulator
// registers. Per 32-receiver chunk the tile's history -- 32 batch rows x (3 + 2Q) slices x
// 64 bytes, both planes -- is staged through LDS (double-buffered, one register stage of
// loads in flight); the compressed W fragments come straight from global memory (L2) into
// registers, each q's fragments reloaded for the next chunk right after their last use.
// k is split over KS workgroups; partials as the dense product's, row-major [KS][rows][Np].
#include "kernels.h"

namespace delrec {

namespace {

typedef float fs_floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 fs_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 fs_bf16x16 __attribute__((ext_vector_type(16)));
typedef uint32_t fs_u32x8 __attribute__((ext_vector_type(8)));

__device__ uint32_t fs_buffer_load_u32(i32x4 rsrc, int voff, int soff, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");

constexpr int kFarSparseRows = 32;    // batch rows per tile (x 4 steps = 128 product rows)
constexpr int kFarSparsePairWords = 12;   // LDS words per receiver pair (slices + pad)

// pair of the 32-receiver chunk held by sparsity group G of a 64-k product
__host__ __device__ inline int fs_pair(int G) {
    const int h = G >> 3, g = G & 7;
    return 4 * (g >> 1) + (g & 1) + 2 * h;
}

}  // namespace

// One thread per (chunk, q, column block, lane): the 8 compressed values and positions of
// sparsity groups 4 (lane / 16) .. + 3 for column jb * 16 + lane % 16 (source perm[c0 + col];
// columns past nc are 0). An offset outside [omin, omin + D) packs a NaN weight into the
// q = 0 product, as the dense pack does, so that the results it enters are NaN.
__global__ void __launch_bounds__(256) far_sparse_pack_kernel(HybPack p, int Q, uint4* __restrict__ wv,
                                                              uint32_t* __restrict__ wi) {
    const int NJB = p.Np / 16, nch = p.Nk / 32;
    const size_t total = (size_t)nch * Q * NJB * 64;
    const size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int lane = (int)(id & 63);
    const size_t r1 = id >> 6;
    const int jb = (int)(r1 % NJB);
    const size_t r2 = r1 / NJB;
    const int q = (int)(r2 % Q), c = (int)(r2 / Q);
    const int col = jb * 16 + (lane & 15);
    const int j = col < p.nc ? p.perm[p.c0 + col] : -1;
    const uint16_t* Wh = static_cast<const uint16_t*>(p.W);
    uint32_t words[4];
    uint32_t idx = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int G = 4 * (lane >> 4) + g;
        const int i0 = c * 32 + 2 * fs_pair(G);
        // receiver i0 sits at position 0 (offset 2q) or 2 (2q + 1), i0 + 1 at 1 or 3
        int pos[2] = {0, 1};
        uint32_t val[2] = {0u, 0u};
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int i = i0 + r;
            if (j < 0 || i >= p.N) continue;
            const size_t o = (size_t)i * p.N + j;
            const int e = (int)p.off[o] - p.omin;
            if (e < 0 || e >= p.D) {
                if (q == 0) val[r] = 0x7FC0u;   // NaN
            } else if (e == 2 * q || e == 2 * q + 1) {
                val[r] = Wh[o];
                pos[r] = r + 2 * (e - 2 * q);
            }
        }
        // the two values of a group in ascending position
        const bool sw = pos[0] > pos[1];
        const uint32_t v0 = sw ? val[1] : val[0], v1 = sw ? val[0] : val[1];
        const int p0 = sw ? pos[1] : pos[0], p1 = sw ? pos[0] : pos[1];
        words[g] = v0 | (v1 << 16);
        idx |= (uint32_t)(p0 | (p1 << 2)) << (4 * g);
    }
    wv[id] = make_uint4(words[0], words[1], words[2], words[3]);
    wi[id] = idx;
}

template <int Q>
__global__ void __launch_bounds__(256) far_sparse_kernel(FarSparse p) {
    constexpr int S = 3 + 2 * Q;                          // staged slices per batch row
    constexpr int RB = kFarSparseRows;
    constexpr int PS = kFarSparsePairWords;               // words per pair: its S slices + pad
    constexpr int BS = 16 * PS + 4;                       // words per batch row: [pair][slice]
    static_assert(PS >= S && PS % 8 == 4 && BS % 64 == 4, "bank layout");
    constexpr int PL = RB * BS;                           // words per plane
    constexpr int BUF = 2 * PL;                           // words per buffer (two planes)
    constexpr int NS = S;                                 // staged uint4 per thread
    static_assert(2 * RB * 4 == 256, "staging shape: one thread per (plane, batch row, quarter)");
    extern __shared__ uint32_t lds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wj = w & 1, wc = w >> 1;
    const int lg = lane >> 4, lc = lane & 15;
    const int NCT = (p.rows + 4 * RB - 1) / (4 * RB), NJT = p.Np / 256;
    const int id = (int)blockIdx.x;
    int ct, jt, ks;
    if (NCT % 4 == 0 && NJT % 2 == 0) {
        // XCD x (= id mod 8) serves a quarter of the row tiles x half of the column tiles
        const int x = id & 7, slot = id >> 3, ncq = NCT / 4;
        ks = slot % p.KS;
        const int t = slot / p.KS;
        ct = (x & 3) * ncq + t % ncq;
        jt = (x >> 2) * (NJT / 2) + t / ncq;
    } else {
        ks = id % p.KS;
        const int t = id / p.KS;
        jt = t % NJT;
        ct = t / NJT;
    }
    const int b0 = ct * RB, n0 = jt * 256;
    const int nch = p.Nk / 32;
    const int per = (nch + p.KS - 1) / p.KS;
    const int c0 = ks * per, c1 = min(nch, c0 + per);
    const int NJB = p.Np / 16;

    const uint32_t hbytes = (uint32_t)((size_t)p.B * p.lda * 2);
    const i32x4 rh0 = buffer_rsrc(p.a0, hbytes), rh1 = buffer_rsrc(p.a1, hbytes);
    const size_t nfrag = (size_t)nch * Q * NJB * 64;
    const i32x4 rwv = buffer_rsrc(p.wv, (uint32_t)(nfrag * 16)), rwi = buffer_rsrc(p.wi, (uint32_t)(nfrag * 4));
    // staging: thread tid stages plane tid / 128 (wave-uniform), batch row b = (tid / 4) % 32
    // and 16-byte quarter r = tid % 4 (pairs 4r .. 4r + 3) of the chunk's 64 bytes; load h
    // takes slice (h + 2b) mod S, so that the four lanes of a row still read 64 contiguous
    // bytes while the rows of one LDS store spread over the banks (at most two lanes of a
    // half wave per bank; the rotation by b alone left up to four)
    const bool hpl = __builtin_amdgcn_readfirstlane(w) >= 2;
    const i32x4 rh = hpl ? rh1 : rh0;
    const int sb = (tid >> 2) & 31, sq = tid & 3;
    // batch rows past B land past the descriptor's end (zeros)
    const uint32_t ho = (uint32_t)(((size_t)(b0 + sb) * p.lda + p.aoff + sq * 8) * 2);
    const uint32_t hstep = (uint32_t)p.Nk * 2;
    const int hl = (hpl ? PL : 0) + sb * BS + 4 * sq * PS;   // word of (pair 4 sq, slice 0)
    uint4 sreg[NS];
    const int sr = (2 * sb) % S;
    auto slice_of = [&](int h) { return h + sr < S ? h + sr : h + sr - S; };
    auto issue_stage = [&](int c) {
#pragma unroll
        for (int h = 0; h < NS; ++h)
            sreg[h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(
                rh, (int)(ho + (uint32_t)c * 64 + (uint32_t)slice_of(h) * hstep), 0, 0));
    };
    // LDS: per plane and batch row, the chunk's 16 receiver pairs at a pitch of PS words,
    // each with its S slices in consecutive words, so that the two words of an operand group
    // (one pair at slices tau + 2q, tau + 2q + 1) are adjacent
    auto stash = [&](int buf) {
        uint32_t* d = lds + buf * BUF + hl;
#pragma unroll
        for (int h = 0; h < NS; ++h) {
            const int sl = slice_of(h);
            d[sl] = sreg[h].x;
            d[PS + sl] = sreg[h].y;
            d[2 * PS + sl] = sreg[h].z;
            d[3 * PS + sl] = sreg[h].w;
        }
    };
    // compressed W fragments of the wave's column blocks jb0 .. jb0 + 7 for q-step k (chunk
    // c0 + k / Q, q = k mod Q), in register slot k mod 2: loaded right after step k - 2, one
    // step ahead of their use
    const int jb0 = (n0 + wj * 128) / 16;
    uint4 av[2][8];
    uint32_t ai[2][8];
    auto load_w = [&](int k, int slot) {
        const int c = c0 + k / Q, q = k % Q;
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
            const size_t f = (((size_t)c * Q + q) * NJB + jb0 + jb) * 64 + lane;
            av[slot][jb] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(rwv, (int)(f * 16), 0, 0));
            ai[slot][jb] = fs_buffer_load_u32(rwi, (int)(f * 4), 0, 0);
        }
    };
    // the accumulators live in the AGPRs (the MFMA's AGPR form), which leaves the VGPRs to the
    // operands in flight
    asm volatile("; accumulators in AGPRs" ::"a"(0.0f));
    fs_floatx4 acc[8][4];
#pragma unroll
    for (int jb = 0; jb < 8; ++jb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[jb][cb] = fs_floatx4{0.f, 0.f, 0.f, 0.f};
    // dense-operand reads: column cb * 16 + lc of the wave's 64 rows is batch row
    // wc * 16 + cb * 4 + lc / 4, step tt = lc % 4; pairs 4 lg .. + 3 at slices tt + 2q, + 1.
    // Banks (word mod 64): tt adds 0 .. 3, the batch row 4 (BS = 4 mod 64) per row, lg 4 PS lg
    // (16, 32 or 48 mod 64): the 64 lanes of a read hit 64 distinct banks, each half wave 32
    // distinct banks mod 32
    const int bl = (wc * 16 + (lc >> 2)) * BS + 4 * lg * PS + (lc & 3);
    auto read_b = [&](const uint32_t* L, int cb, fs_bf16x16* bv) {
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) {
            const uint32_t* x = L + pl * PL + cb * 4 * BS;
            bv[pl] = __builtin_bit_cast(fs_bf16x16, fs_u32x8{x[0], x[1], x[PS], x[PS + 1], x[2 * PS], x[2 * PS + 1],
                                                             x[3 * PS], x[3 * PS + 1]});
        }
    };
    const int ncl = c1 - c0, nstep = ncl * Q;
    // One chunk = Q q-steps; q-step k (chunk k / Q) uses W slot k mod 2. In a step the 4
    // column blocks run 16 products each while the next block's operands are read (ping-pong
    // bA / bB; the next step's first block at the end). At a chunk's end: the next chunk's
    // history (loaded during this chunk) into the other buffer, a barrier, and the loads of
    // the chunk after it; then the compressed W of step k + 2 into the freed slot. Every load
    // and barrier is unconditional (indices clamped to the last chunk / step), and the loop
    // body is two chunks, so each slot and wait is static.
    fs_bf16x16 bA[2], bB[2];
    auto smfma = [&](int slot, int cb, const fs_bf16x16* bv) {
#pragma unroll
        for (int pl = 0; pl < 2; ++pl)
#pragma unroll
            for (int jb = 0; jb < 8; ++jb)
                acc[jb][cb] = __builtin_amdgcn_smfmac_f32_16x16x64_bf16(
                    __builtin_bit_cast(fs_bf16x8, av[slot][jb]), bv[pl], acc[jb][cb], (int)ai[slot][jb], 0, 0);
    };
    auto chunk = [&](int cl, int s0) {
        const uint32_t* L0 = lds + (cl & 1) * BUF + bl;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int k = cl * Q + q, slot = (s0 + q) & 1;
            const uint32_t* L = L0 + 2 * q;
            read_b(L, 1, bB);
            smfma(slot, 0, bA);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
            read_b(L, 2, bA);
            smfma(slot, 1, bB);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
            read_b(L, 3, bB);
            smfma(slot, 2, bA);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
            if (q == Q - 1) {
                stash((cl + 1) & 1);
                barrier_lds();
                issue_stage(c0 + min(cl + 2, ncl - 1));
                read_b(lds + ((cl + 1) & 1) * BUF + bl, 0, bA);
            } else {
                read_b(L + 2, 0, bA);
            }
            smfma(slot, 3, bB);
            load_w(min(k + 2, nstep - 1), slot);
        }
    };

    if (nstep > 0) {
        issue_stage(c0);
        load_w(0, 0);
        load_w(min(1, nstep - 1), 1);
        stash(0);
        barrier_lds();
        issue_stage(c0 + min(1, ncl - 1));
        read_b(lds + bl, 0, bA);
    }
    int cl = 0;
    for (; cl + 1 < ncl; cl += 2) {
        chunk(cl, 0);
        chunk(cl + 1, Q & 1);
    }
    if (cl < ncl) chunk(cl, 0);

    float* out = p.part + (size_t)ks * p.rows * p.Np;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int r = b0 * 4 + wc * 64 + cb * 16 + lc;
        if (r >= p.rows) continue;
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
            const int j = n0 + wj * 128 + jb * 16 + 4 * lg;
            *reinterpret_cast<fs_floatx4*>(out + (size_t)r * p.Np + j) = acc[jb][cb];
        }
    }
}

// ---------------------------------------------------------------------------------------
// The near product of a block, dense: G_j(tau) of the near sources (columns j, dense bf16
// W^(e) planes, k-blocked [(e Nk + i) / 8][Np]) for the block's rows (b, tt), tau = the block's
// first row step + tt, from the history slices tau + e. The product reads every history slice
// of a batch row once per 32-receiver chunk -- 32 batch rows x (D + 3) slices x 64 bytes x 2
// planes, staged through LDS -- and builds the rows (b, tt) of all D offsets from it, where
// a plain strided GEMM re-reads the window once per (step, offset): 4 (D) / (D + 3) of its
// history traffic. Workgroup: 4 waves, 128 rows (32 batch rows x 4 steps) x 128 columns, a
// wave 64 x 64 (4 x 4 blocks of v_mfma_f32_16x16x32_bf16, both gr planes); W and history
// double-buffered in LDS from one register stage of loads. LDS: batch row pitch 132 words
// and slice pitch 16 make the 16 lanes of a row block's 16-byte reads hit 16 distinct bank
// groups; the history rows are loaded at slices rotated by the batch row (stores at most
// two-way conflicted). k split over KS workgroups; partials row-major [KS][rows][Np].
constexpr int kNearBlockRows = 32;      // batch rows per tile (x 4 steps)
constexpr int kNearBlockSlices = 8;     // staged slices per batch row (D + 3 <= 8)
constexpr int kNearBlockBP = 33;        // uint4 per staged batch row (8 slices x 4 + 1)

template <int D>
__global__ void __launch_bounds__(256) near_block_kernel(NearBlock p) {
    constexpr int S = D + 3, SL = kNearBlockSlices, BP = kNearBlockBP, RB = kNearBlockRows;
    static_assert(S <= SL, "slices per batch row");
    constexpr int HPL = RB * BP;                  // uint4 per history plane
    constexpr int HB = 2 * HPL;                   // W after the two history planes
    constexpr int BUF = HB + D * 4 * 128;         // uint4 per buffer
    constexpr int NH = (2 * RB * S * 4 + 255) / 256;   // history uint4 staged per thread
    constexpr int NW = D * 4 * 128 / 256;              // W uint4 staged per thread
    static_assert(D * 4 * 128 % 256 == 0, "W staging");
    extern __shared__ uint4 nlds[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int wi = w >> 1, wj = w & 1, lg = lane >> 4, lc = lane & 15;
    const int NCT = (p.rows + 4 * RB - 1) / (4 * RB), NJT = p.Np / 128;
    const int id = (int)blockIdx.x;
    int ct, jt, ks;
    if (p.KS % 8 == 0) {
        // XCD x (= id mod 8) serves KS / 8 of the splits over every tile: their W slabs stay in
        // its L2 while the row tiles stream past
        const int x = id & 7, slot = id >> 3, kx = p.KS / 8;
        ks = x * kx + slot % kx;
        const int t = slot / kx;
        jt = t % NJT;
        ct = t / NJT;
    } else {
        ks = id % p.KS;
        const int t = id / p.KS;
        jt = t % NJT;
        ct = t / NJT;
    }
    const int b0 = ct * RB, n0 = jt * 128;
    const int nch = p.Nk / 32;
    const int per = (nch + p.KS - 1) / p.KS;
    const int c0 = ks * per, c1 = min(nch, c0 + per);

    const uint32_t hbytes = (uint32_t)((size_t)p.B * p.lda * 2);
    const i32x4 rh0 = buffer_rsrc(p.a0, hbytes), rh1 = buffer_rsrc(p.a1, hbytes);
    const i32x4 rw = buffer_rsrc(p.w, (uint32_t)((size_t)(D * p.Nk / 8) * p.Np * 16));
    // history staging: uint4 u = tid + 256 h: plane u / (RB S 4), batch row, slice (rotated
    // by the batch row), 16-byte quarter; W staging: uint4 u = tid + 256 h: (offset e,
    // k-block kb) = u / 128, column u % 128
    uint32_t ho[NH];
    int hl[NH];
    bool hp[NH], hv[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int u = tid + 256 * h;
        hv[h] = u < 2 * RB * S * 4;
        const int uu = hv[h] ? u : 0;
        const int pl = uu / (RB * S * 4), r = uu % (RB * S * 4);
        const int b = r / (S * 4), q = (r / 4) % S, qd = r % 4;
        const int sl = (q + b) % S;
        ho[h] = (uint32_t)(((size_t)(b0 + b) * p.lda + p.aoff + (size_t)sl * p.Nk + qd * 8) * 2);
        hl[h] = pl * HPL + b * BP + sl * 4 + qd;
        hp[h] = pl != 0;
    }
    uint32_t wo[NW];
#pragma unroll
    for (int h = 0; h < NW; ++h) {
        const int u = tid + 256 * h, ekb = u / 128, col = u % 128, e = ekb / 4, kb = ekb % 4;
        wo[h] = (uint32_t)((((size_t)e * p.Nk / 8 + kb) * p.Np + n0 + col) * 16);
    }
    uint4 sh[NH], sw[NW];
    auto issue = [&](int c) {
#pragma unroll
        for (int h = 0; h < NH; ++h)
            sh[h] = hv[h] ? __builtin_bit_cast(uint4, raw_buffer_load_i32x4(hp[h] ? rh1 : rh0, (int)(ho[h] + (uint32_t)c * 64), 0, 0))
                          : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int h = 0; h < NW; ++h)
            sw[h] = __builtin_bit_cast(uint4, raw_buffer_load_i32x4(rw, (int)(wo[h] + (uint32_t)c * 4 * p.Np * 16), 0, 0));
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int h = 0; h < NH; ++h)
            if (hv[h]) nlds[buf * BUF + hl[h]] = sh[h];
#pragma unroll
        for (int h = 0; h < NW; ++h) nlds[buf * BUF + HB + tid + 256 * h] = sw[h];
    };
    fs_floatx4 acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = fs_floatx4{0.f, 0.f, 0.f, 0.f};
    // A fragment of row block mb: row r = wi 64 + mb 16 + lc = batch row r / 4, step r % 4,
    // receivers 8 lg .. + 7 of the chunk at slice (r % 4) + e
    int ar[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int r = wi * 64 + mb * 16 + lc;
        ar[mb] = (r >> 2) * BP + (r & 3) * 4 + lg;
    }
    const int bc = wj * 64 + lc;
    if (c0 < c1) {
        issue(c0);
        stash(0);
        barrier_lds();
        if (c0 + 1 < c1) issue(c0 + 1);
    }
    for (int c = c0; c < c1; ++c) {
        const uint4* L = nlds + ((c - c0) & 1) * BUF;
#pragma unroll
        for (int e = 0; e < D; ++e) {
            fs_bf16x8 bf[4];
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) bf[nb] = __builtin_bit_cast(fs_bf16x8, L[HB + (e * 4 + lg) * 128 + bc + nb * 16]);
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) {
                fs_bf16x8 af[4];
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) af[mb] = __builtin_bit_cast(fs_bf16x8, L[pl * HPL + ar[mb] + e * 4]);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                    for (int nb = 0; nb < 4; ++nb)
                        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mb], bf[nb], acc[mb][nb], 0, 0, 0);
            }
        }
        if (c + 1 < c1) {
            stash(((c - c0) & 1) ^ 1);
            barrier_lds();
            if (c + 2 < c1) issue(c + 2);
        }
    }
    float* out = p.part + (size_t)ks * p.rows * p.Np;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const int r = b0 * 4 + wi * 64 + mb * 16 + 4 * lg + e4;
            if (r >= p.rows) continue;
#pragma unroll
            for (int nb = 0; nb < 4; ++nb) out[(size_t)r * p.Np + n0 + wj * 64 + nb * 16 + lc] = acc[mb][nb][e4];
        }
}

// ---------------------------------------------------------------------------------------

int far_sparse_q(int D) { return D >= 3 && D <= 6 ? (D + 1) / 2 : 0; }

size_t far_sparse_lds(int Q) {
    (void)Q;   // the pair pitch holds up to 12 slices (Q <= 4)
    return (size_t)2 * 2 * kFarSparseRows * (16 * kFarSparsePairWords + 4) * sizeof(uint32_t);
}

size_t far_sparse_wv(int Nk, int Np, int Q) { return (size_t)(Nk / 32) * Q * (Np / 16) * 64; }

int far_sparse_splits(int rows, int Np, int Nk, int cus) {
    const int tiles = ((rows + 4 * kFarSparseRows - 1) / (4 * kFarSparseRows)) * (Np / 256);
    const int nch = Nk / 32;
    if (tiles < 1) return 1;
    return std::max(1, std::min((cus + tiles - 1) / tiles, std::max(1, nch / 8)));
}

bool near_block_ok(int D) { return D >= 1 && D + 3 <= kNearBlockSlices; }

size_t near_block_lds(int D) {
    return (size_t)2 * (2 * kNearBlockRows * kNearBlockBP + D * 4 * 128) * sizeof(uint4);
}

int near_block_splits(int rows, int Np, int Nk, int cus) {
    const int tiles = ((rows + 4 * kNearBlockRows - 1) / (4 * kNearBlockRows)) * (Np / 128);
    const int nch = Nk / 32;
    if (tiles < 1) return 1;
    return std::max(1, std::min((cus + tiles - 1) / tiles, std::max(1, nch / 4)));
}

bool launch_near_block(const NearBlock& g, int D, hipStream_t stream) {
    const int tiles = ((g.rows + 4 * kNearBlockRows - 1) / (4 * kNearBlockRows)) * (g.Np / 128);
    const dim3 grid((unsigned)(tiles * g.KS));
    const size_t lds = near_block_lds(D);
#define DELREC_NEAR_BLOCK(DV)                                                                   \
    if (D == DV) {                                                                              \
        ensure_lds((const void*)near_block_kernel<DV>, lds);                                    \
        hipLaunchKernelGGL(near_block_kernel<DV>, grid, dim3(256), lds, stream, g);             \
        return true;                                                                            \
    }
    DELREC_NEAR_BLOCK(1) DELREC_NEAR_BLOCK(2) DELREC_NEAR_BLOCK(3) DELREC_NEAR_BLOCK(4) DELREC_NEAR_BLOCK(5)
#undef DELREC_NEAR_BLOCK
    return false;
}

void launch_far_sparse_pack(const HybPack& a, int Q, uint4* wv, uint32_t* wi, hipStream_t stream) {
    const size_t total = far_sparse_wv(a.Nk, a.Np, Q);
    hipLaunchKernelGGL(far_sparse_pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a, Q,
                       wv, wi);
}

bool launch_far_sparse(const FarSparse& g, int Q, hipStream_t stream) {
    const int tiles = ((g.rows + 4 * kFarSparseRows - 1) / (4 * kFarSparseRows)) * (g.Np / 256);
    const dim3 grid((unsigned)(tiles * g.KS));
    const size_t lds = far_sparse_lds(Q);
    if (Q == 3) {
        ensure_lds((const void*)far_sparse_kernel<3>, lds);
        hipLaunchKernelGGL(far_sparse_kernel<3>, grid, dim3(256), lds, stream, g);
        return true;
    }
    if (Q == 2) {
        ensure_lds((const void*)far_sparse_kernel<2>, lds);
        hipLaunchKernelGGL(far_sparse_kernel<2>, grid, dim3(256), lds, stream, g);
        return true;
    }
    return false;
}

}  // namespace delrec
