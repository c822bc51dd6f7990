/*
 * delrec.h — C ABI of the MI355X delayed-LIF recurrent layer (forward + BPTT backward).
 *
 * One shared library, libdelrec_hip.so, built for gfx950. Every entry point takes raw
 * device pointers, sizes and a hipStream_t (passed as void*), launches asynchronously on
 * that stream, allocates nothing, and returns a delrec_status (0 = ok). Scratch memory is
 * passed in by the caller, sized by delrec_query_workspace().
 *
 * Layouts (all row-major, contiguous):
 *   x, y, u, dx, gy      (T, B, N) float32, time-major
 *   W                    (N, N): W[i*N + j] is the weight from source j to receiver i;
 *                        float32, or bfloat16 when the args' w_bf16 flag is set
 *   d (axonal)           (N,)  float32 delay per source
 *   d (synaptic)         (N, N) float32 delay per connection, d[i*N + j]
 *   base, offsets        hybrid delays d[i*N+j] = base[j] + offsets[i*N+j]; offsets int8
 *   spike bits           (B, ceil(T/32), N) uint32: bit (t % 32) of word [b][t/32][i]
 *                        is the spike of neuron i at step t
 *
 * Reference interfaces replaced (paths relative to the DelRec repository):
 *   delrec_axonal_fwd   recdel_triton_forward + recdel_fwd_kernel
 *                       (src/delrec/triton_kernels/recdel_base.py:136-182, :34-129)
 *   delrec_axonal_bwd   recdel_triton_backward + recdel_bwd_kernel + the dW / dmask host
 *                       reductions + autograd through build_mask
 *                       (recdel_base.py:288-342, :189-285, :402-439)
 *   delrec_syn_fwd      _ed_scatter_compact_kernel as launched by EventDrivenSyn.forward
 *                       and HybridSynDelay.forward (synaptic_eventdriven.py:106-164,
 *                       :385-416; synaptic_hybrid.py:139-172)
 *   delrec_syn_bwd      _ed_bwd_kernel + the Cstack GEMMs + dW + dd/dp
 *                       (synaptic_eventdriven.py:323-364, :419-471;
 *                        synaptic_hybrid.py:174-211)
 *   delrec_delay_grad   _delay_grad / _hybrid_dd_kernel (synaptic_hybrid.py:83-126)
 *   delrec_lif_fwd/bwd  the plain multi-step LIF layer the SNN_* stacks build around the
 *                       recurrent layer (spikingjelly LIFNode, networks.py:82-100)
 */
#ifndef DELREC_H
#define DELREC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    DELREC_OK = 0,
    DELREC_ERR_ARG = 1,          /* bad size, null pointer or inconsistent flags       */
    DELREC_ERR_UNSUPPORTED = 2,  /* regime this build does not implement               */
    DELREC_ERR_WORKSPACE = 3,    /* workspace missing or smaller than queried          */
    DELREC_ERR_LAUNCH = 4,       /* a kernel launch failed (hipGetLastError)           */
    DELREC_ERR_WINDOW = 5,       /* window length L out of range for the on-chip ring  */
    DELREC_ERR_DEVICE = 6,       /* device query failed / not a gfx950 device          */
    DELREC_ERR_PENDING = 7,      /* delrec_max_take: the value did not arrive in time  */
    DELREC_ERR_STALE = 8,        /* delrec_max_take: the slot was reused by later posts */
    DELREC_ERR_SCRATCH = 9       /* delrec_axonal_bwd_noalloc: sizes beyond its scratch   */
} delrec_status;

/* Neuron constants (spikingjelly LIFNode semantics; reference lif.py:25-56). */
typedef struct {
    float tau;           /* membrane time constant                                      */
    float decay;         /* float(1 - 1/tau) evaluated in double by the caller          */
    float v_threshold;
    float v_reset;       /* ignored when soft_reset                                     */
    int32_t soft_reset;  /* 1: v_reset is None (v -= spike * v_threshold)              */
    int32_t decay_input; /* 1: h = v + (x - (v - v_reset)) / tau                       */
    int32_t detach_reset;
    int32_t surrogate;   /* 0 = triangle(gamma), 1 = atan(alpha): the reference's ids   */
    float gamma;
    float alpha;
} delrec_lif;

/* Forward tap modes of the axonal layer (reference FWD constexpr, recdel_base.py:59-61). */
enum { DELREC_TAPS_SOFT = 0, DELREC_TAPS_ROUND = 1, DELREC_TAPS_INTERP = 2 };

typedef struct {
    int32_t T, B, N, L;          /* L: window length, ceil(1 + max d + max s) + 1; 0:   */
                                 /* not read by the caller (soft taps, uniform s, decay */
                                 /* charge, hard reset to 0, no rec, N <= 256,          */
                                 /* T*B*N <= 2^28): the kernel takes its history length */
                                 /* from d, up to 256 lags; the caller checks L before  */
                                 /* the backward                                        */
    const float* x;              /* (T,B,N)                                             */
    const void* W;               /* (N,N) fp32 or bf16                                  */
    int32_t w_bf16;
    const float* bias;           /* (N) or NULL                                         */
    const float* d;              /* (N) delays (already STE-rounded when requested)      */
    const float* s;              /* (N) per-source half-width, or NULL -> s_uniform     */
    float s_uniform;             /* 1 + sigma                                           */
    const float* drop;           /* (B,N) fixed recurrent-dropout multiplier or NULL    */
    int32_t taps;                /* DELREC_TAPS_*                                       */
    const int32_t* lag;          /* (N) hard lag for ROUND / INTERP, else NULL          */
    const float* frac;           /* (N) INTERP weight of lag+1, else NULL               */
    delrec_lif lif;
    float* y;                    /* out (T,B,N) spikes                                  */
    float* u;                    /* out (T,B,N) pre-reset membrane                      */
    float* rec;                  /* out (T,B,N) recurrent input incl. bias, or NULL     */
    float* z;                    /* out (T,B,N) delayed source trace (for dW)           */
    uint32_t* bits;              /* out (B, ceil(T/32), N) spike bitmask                */
    void* workspace;             /* N > 256: transposed W                               */
    size_t workspace_bytes;
    uint32_t* dmax_ticket;       /* NULL, or out: the call also posts max d as by       */
                                 /* delrec_max_post (from inside the scan kernel where  */
                                 /* it can) and returns the ticket for delrec_max_take  */
} delrec_axonal_fwd_args;

/* Backward gfut modes (reference APPROX constexpr, recdel_base.py:216-233). */
enum { DELREC_BWD_SOFT = 0, DELREC_BWD_STRAIGHT = 1 };

typedef struct {
    int32_t T, B, N, L;
    const float* gy;             /* (T,B,N) upstream gradient                            */
    const float* u;              /* (T,B,N) saved membrane                               */
    const uint32_t* bits;        /* saved spike bitmask                                  */
    const float* z;              /* saved delayed trace                                  */
    const void* W;
    int32_t w_bf16;
    const float* d;
    const float* s;
    float s_uniform;
    const float* drop;
    int32_t mode;                /* DELREC_BWD_SOFT or DELREC_BWD_STRAIGHT               */
    const int32_t* lag;          /* (N) for STRAIGHT                                     */
    delrec_lif lif;
    float* dx;                   /* out (T,B,N)                                          */
    float* dW;                   /* out (N,N) float32, or NULL                           */
    float* db;                   /* out (N), or NULL                                     */
    float* dd;                   /* out (N), or NULL                                     */
    float* ds;                   /* out (N) gradient w.r.t. the half-width s, or NULL    */
    void* workspace;
    size_t workspace_bytes;
} delrec_axonal_bwd_args;

typedef struct {
    int32_t T, B, N, L;
    const float* x;
    const void* W;               /* (N,N) W[i*N+j], fp32 or bf16                         */
    int32_t w_bf16;
    const float* bias;
    const float* d;              /* (N,N) per-connection delays, or NULL when hybrid      */
    const float* base;           /* (N) hybrid base delay per source                     */
    const int8_t* offsets;       /* (N,N) hybrid integer offsets, offsets[i*N+j]         */
    const float* s;              /* (N) per-source half-width or NULL                    */
    float s_uniform;
    float s_max;                 /* largest half-width: max of s[], or s_uniform           */
    const float* drop;           /* (B,N) or NULL                                        */
    delrec_lif lif;
    float* y;
    float* u;
    uint32_t* bits;
    void* workspace;
    size_t workspace_bytes;
    /* hybrid only (0 otherwise): the offset range and a bound of the smallest delay, for
     * the offset-stacked and arrival scans, which apply when off_count > 0 (off_count =
     * largest - smallest offset + 1, at most 16) and d_min >= s_uniform - 1. Those forms give
     * every source the triangle of base[j] + off_min, so d_min must be at most
     * min over j of float32(base[j] + off_min) -- NOT the smallest materialised delay, which
     * can be larger when the source of the smallest base has no connection at off_min.
     * The caller reads them with the window length. A call that breaks either contract
     * (an offset outside [off_min, off_min + off_count), or a source whose taps reach a lag
     * < 1 in those forms) gets NaN in the outputs that connection or source reaches,
     * never silently dropped taps. */
    float d_min;
    int32_t off_min;
    int32_t off_count;
} delrec_syn_fwd_args;

typedef struct {
    int32_t T, B, N, L;
    const float* gy;
    const float* u;
    const float* y;              /* (T,B,N) saved spikes                                 */
    const uint32_t* bits;
    const void* W;
    int32_t w_bf16;
    const float* d;
    const float* base;
    const int8_t* offsets;
    const float* s;
    float s_uniform;
    float s_max;                 /* largest half-width: max of s[], or s_uniform           */
    const float* drop;
    delrec_lif lif;
    float* dx;                   /* out (T,B,N)                                          */
    float* dW;                   /* out (N,N) or NULL. With w_bf16 the lag correlation
                                    behind dW / dd / ds takes gr to about 2^-17 per term
                                    (fp32 W: 2^-25), below the bf16 rounding (2^-9) that
                                    a bf16 weight's gradient gets                        */
    float* dd;                   /* out (N,N) per-connection delay gradient, or NULL     */
    float* ds;                   /* out (N) half-width gradient, or NULL                 */
    float* db;                   /* out (N) or NULL                                      */
    void* workspace;
    size_t workspace_bytes;
    float d_min;                 /* hybrid: as in delrec_syn_fwd_args                    */
    int32_t off_min;
    int32_t off_count;
    /* hybrid, optional (near_known != 0): how many sources j have a first lag
       max(1, floor(1 + (base_j + off_min) - s_uniform) + 1) (fp32, in that order) below 4 and
       below 2. The offset-stacked backward splits the sources by first lag; given these counts
       (e.g. from the forward's own host read) it runs without a host synchronisation,
       otherwise (near_known == 0, as a zeroed struct has it) it reads the first lags back from
       the device once per call. Counts that do not match the device's make every output NaN. */
    int32_t near_known, near_lt4, near_lt2;
} delrec_syn_bwd_args;

/* Plain multi-step LIF layer (no recurrence). */
typedef struct {
    int32_t T, B, N;
    const float* x;
    delrec_lif lif;
    float* y;
    float* u;
} delrec_lif_fwd_args;

typedef struct {
    int32_t T, B, N;
    const float* gy;
    const float* u;
    const float* y;
    delrec_lif lif;
    float* dx;
} delrec_lif_bwd_args;

/* Linear layer on spike inputs: out[t][b][m] = bias[m] + sum_k y[t][b][k] * W[m*K + k],
 * the spikes y given as the scans' spike bits. Replaces torch.nn.Linear applied to a
 * recurrent layer's spike output in the SNN_* stacks (reference networks.py:140-181, the
 * Linear that follows each recurrent layer in the Sequential). W is read in fp32 and
 * applied as bf16 hi + mid + lo (about 2^-25 relative per weight, fp32 accumulation). Workspace:
 * delrec_query_workspace(DELREC_WS_SPIKE_LINEAR, T, B, K, M, 0). */
typedef struct {
    int32_t T, B, K, M;
    const uint32_t* bits;        /* (B, ceil(T/32), K) spike words                        */
    const float* W;              /* (M, K) fp32                                           */
    const float* bias;           /* (M) or NULL                                           */
    float* out;                  /* out (T, B, M) fp32                                    */
    void* workspace;
    size_t workspace_bytes;
} delrec_spike_linear_args;

/* Weight gradient of that Linear from the same spike bits: dW[m*K + k] = sum_{t,b}
 * g[t][b][m] * y[t][b][k] (the reference computes it as the torch.nn.Linear backward,
 * g^T x on the fp32 spikes). g is applied as bf16 hi + mid + lo (about 2^-25 relative per
 * term, fp32 accumulation). Workspace: delrec_query_workspace(DELREC_WS_SPIKE_LINEAR_DW, T,
 * B, K, M, 0): g's three bf16 planes (6 bytes per element of g, steps padded to 32) and, when
 * the output tiles alone do not fill the GPU twice over, the splits' partial dW. */
typedef struct {
    int32_t T, B, K, M;
    const uint32_t* bits;        /* (B, ceil(T/32), K) spike words                        */
    const float* g;              /* (T, B, M) gradient of the Linear's output             */
    float* dW;                   /* out (M, K)                                            */
    void* workspace;
    size_t workspace_bytes;
} delrec_spike_linear_dw_args;

/* The loss end of the SNN_* stacks, fused: the readout's output (T, B, C) reduced over time
 * -- DELREC_READOUT_SUM (reference utils.py calc_loss_SSC), _MEAN (calc_loss_HAR,
 * calc_loss_AL) or _MAX (calc_loss_SHD, first maximum) -- optionally after a non-spiking
 * leaky integrator (the SHD readout LIF with threshold 1e8, networks_shd.py:187-199:
 * integrator 1 v = decay * v + x, 2 v = v + (x - v) / tau, decay_input), then
 * torch.nn.CrossEntropyLoss (mean over the batch). Writes the loss, its gradient with
 * respect to the readout's output and optionally the reduced readout (B, C). Workspace: B
 * floats. */
enum { DELREC_READOUT_SUM = 0, DELREC_READOUT_MEAN = 1, DELREC_READOUT_MAX = 2 };
typedef struct {
    int32_t T, B, C;
    const float* logits;         /* (T, B, C)                                              */
    const int64_t* labels;       /* (B) class indices                                      */
    int32_t reduce;              /* DELREC_READOUT_*                                       */
    int32_t integrator;          /* 0 none, 1 leaky (decay_input False), 2 (decay_input)   */
    float tau;                   /* integrator time constant; decay = float(1 - 1/tau)     */
    float* out;                  /* out (B, C) reduced readout, or NULL                    */
    float* dlogits;              /* out (T, B, C) d loss / d logits                        */
    float* loss;                 /* out (1) mean cross-entropy                             */
    void* workspace;
    size_t workspace_bytes;
} delrec_readout_ce_args;

/* Workspace kinds for delrec_query_workspace; flags bit 0: weights are bf16; synaptic
 * kinds: bit 1: hybrid delays (d == NULL), bits 8..15: ceil(2 * s_max) on the float32 s_max
 * the entry point receives (s_uniform for the hybrid), capped at 255 -- the most lags of
 * non-zero weight per connection, which picks the scan form (and its workspace); hybrid:
 * bit 2: d_min >= s_uniform - 1, bits 16..23: off_count (the fields of the entry point's
 * arguments, which also pick the scan form). */
enum { DELREC_WS_AXONAL_FWD = 1, DELREC_WS_AXONAL_BWD = 2, DELREC_WS_SYN_FWD = 3,
       DELREC_WS_SYN_BWD = 4, DELREC_WS_SPIKE_LINEAR = 5 /* N = K inputs, L = M outputs */,
       DELREC_WS_SPIKE_LINEAR_DW = 6 /* N = K inputs, L = M outputs */,
       DELREC_WS_READOUT_CE = 7 /* N = C classes, L = 1 */ };

int delrec_axonal_fwd(const delrec_axonal_fwd_args* a, void* stream);
int delrec_axonal_bwd(const delrec_axonal_bwd_args* a, void* stream);
/* delrec_axonal_bwd without a caller workspace: no counterpart in the reference. For
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results as delrec_axonal_bwd;
 * a->workspace / workspace_bytes are ignored. Scratch is a 64 MiB array of the library's own
 * device memory, one per GPU, held until the process ends (looked up on the first call on a
 * device); sizes whose workspace (delrec_query_workspace, DELREC_WS_AXONAL_BWD) exceeds it
 * return DELREC_ERR_SCRATCH. Calls on one GPU share that array: calls that overlap on one
 * GPU (other streams, other threads) race and must not be issued. Allocates nothing. */
int delrec_axonal_bwd_noalloc(const delrec_axonal_bwd_args* a, void* stream);
int delrec_syn_fwd(const delrec_syn_fwd_args* a, void* stream);
/* The hybrid's offset-stacked backward (off_count > 0, rings beyond LDS) splits the sources
 * by first lag: without the caller's counts (near_known == 0) it reads the first lags back
 * to the host once per call, which synchronises the stream before it launches its scan.
 * Every other path is fully asynchronous. */
int delrec_syn_bwd(const delrec_syn_bwd_args* a, void* stream);
int delrec_spike_linear_fwd(const delrec_spike_linear_args* a, void* stream);
int delrec_spike_linear_dw(const delrec_spike_linear_dw_args* a, void* stream);
/* The same Linear's input gradient dy = g W (the reference: the torch.nn.Linear backward, an
 * fp32 GEMM) as one bf16 GEMM with fp32 accumulation and output: this splits the rows of g
 * (rows x M fp32, rows = T B) into out (rows x 3M bf16) = [hi | lo | hi], hi = bf16(x), lo =
 * bf16(x - hi), for the caller to multiply by W stacked [W_hi; W_hi; W_lo] (3M x K), which
 * sums g_hi W_hi + g_lo W_hi + g_hi W_lo (about 2^-16 relative per product). No counterpart
 * in the reference. */
int delrec_spike_linear_dx_split(const float* g, int64_t rows, int32_t M, void* out, void* stream);
int delrec_readout_ce(const delrec_readout_ce_args* a, void* stream);
int delrec_lif_fwd(const delrec_lif_fwd_args* a, void* stream);
int delrec_lif_bwd(const delrec_lif_bwd_args* a, void* stream);

/* dd[i*N+j] = W[i*N+j] * sum_{l=1}^{Lm-1} C[(i*N+j)*Lm + l] * sign(l-1-d)[|l-1-d| <= s]/s^2
 * with s = 1 + sigma: the reference's closed-form delay gradient test hook. */
int delrec_delay_grad(const float* C, const float* W, const float* d, float sigma,
                      int32_t N, int32_t Lm, float* dd, void* stream);

/* Host read of a device maximum without waiting for the stream. The reference sizes the
 * delay window from max d on the host, L = ceil(1 + max d + max s) + 1 read with .item()
 * (triton_kernels/delays.py:26, from recdel_base.py:381), which waits for all work queued
 * before it; here only the backward needs L. delrec_max_post queues one small kernel on
 * `stream` that writes max(x[0 .. n)) (NaN when an element is NaN) with a ticket into one
 * of DELREC_MAX_SLOTS slots of coherent pinned host memory, as a single 8-byte store, and
 * returns the ticket. delrec_max_take waits for that ticket's slot: DELREC_OK with *out
 * set; DELREC_ERR_STALE when later posts have reused the slot (read the maximum again);
 * DELREC_ERR_PENDING when it has not arrived within timeout_ms. Thread-safe. */
enum { DELREC_MAX_SLOTS = 256 };
int delrec_max_post(const float* x, int32_t n, uint32_t* ticket, void* stream);
int delrec_max_take(uint32_t ticket, float* out, int32_t timeout_ms);

/* Bytes of scratch the given entry point needs for these sizes and flags. */
int delrec_query_workspace(int32_t kind, int32_t T, int32_t B, int32_t N, int32_t L,
                           int32_t flags, size_t* bytes);

/* Benchmark hook, with no counterpart in the reference (its profiler times whole layer
 * calls): delrec_scan_timing(n) with n > 0 brackets the time-scan kernel of the next n
 * axonal / synaptic forward and backward calls with HIP events recorded on the caller's
 * stream; n == 0 switches it off. delrec_scan_timing_read waits for those events and
 * writes each launch's duration in ms and its DELREC_WS_* kind (at most `capacity`); it
 * returns the number of launches recorded, or a negative status. Single-threaded use. */
int delrec_scan_timing(int32_t capacity);
int delrec_scan_timing_read(float* ms, int32_t* kinds, int32_t capacity);

/* Benchmark hook, with no counterpart in the reference: the achievable MFMA rate. Launches
 * on `stream` a loop of independent matrix instructions from registers only (kind 0: bf16
 * v_mfma_f32_16x16x32_bf16, kind 1: fp32 v_mfma_f32_16x16x4_f32), `iters` iterations on two
 * workgroups of 8 waves per CU, and writes the flops that launch issues to *flops; the
 * caller times it (events on the same stream). sink: device scratch of at least
 * 1024 floats per CU (DELREC_ERR_WORKSPACE otherwise). */
int delrec_peak_mfma(int32_t kind, int32_t iters, float* sink, size_t sink_bytes, double* flops, void* stream);

const char* delrec_strerror(int status);
/* "delrec-mi355x <DELREC_ABI_VERSION> (gfx950)": a binding checks it before use (the
 * argument structs change between versions). */
#define DELREC_ABI_VERSION "0.5.0"
const char* delrec_version(void);

#ifdef __cplusplus
}
#endif
#endif /* DELREC_H */
