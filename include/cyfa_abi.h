/*
 * cyfa_abi.h -- C ABI of the MI355X (gfx950) CyFA attention hot path.
 *
 * One shared library (libcyfa_hip.so) exports these entry points. Callers pass
 * plain device pointers and sizes; the library never allocates device memory
 * on the hot path and enqueues all work on the caller's HIP stream. Return 0 on
 * success or a negative CYFA_ERR_* code; cyfa_last_error() returns a
 * thread-local message for the last failing call on the calling thread.
 *
 * Each entry point names the reference interface it replaces (paths relative
 * to the Chyxx/CyFA-Jittor v0.1.2 tree). In the reference those interfaces are
 * Python functions that emit inline CUDA through Jittor's jt.code operator;
 * here the Python host code (cyclic_flow_attention/ops/chunk.py and
 * ops/fused_recurrent.py) binds these
 * symbols with ctypes.
 *
 * Tensor layouts (row-major, contiguous):
 *   q, k   bf16 [B, T, H, K]        v, o    bf16 [B, T, H, V]
 *   g, delta, beta  f32 [B, T, H]   (g = natural log of the decay alpha)
 *   table  f32 [H, M-1, M]          (readout @ Phi, see cyfa_readout_table)
 *   hk     f32 [B, H, K, M]         hv      f32 [B, H, M, V]   clock f32 [B, H]
 */
#ifndef CYFA_ABI_H
#define CYFA_ABI_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CYFA_ABI_VERSION 11

enum {
    CYFA_OK = 0,
    CYFA_ERR_VALUE = -1,       /* bad shape / argument     -> Python ValueError */
    CYFA_ERR_UNSUPPORTED = -2, /* valid but not implemented -> NotImplementedError */
    CYFA_ERR_ALIGN = -3,       /* pointer misaligned        -> ValueError */
    CYFA_ERR_WORKSPACE = -4,   /* workspace missing / small -> ValueError */
    CYFA_ERR_LAUNCH = -5       /* HIP launch failure        -> RuntimeError */
};

/* Arguments of one chunkwise prefill call. Nullable pointers are marked. */
typedef struct CyfaChunkArgs {
    int B, T, H, K, V, M, C;      /* M = num_slots (128); C = chunk size (64) */
    const void *q, *k, *v;        /* bf16, see layouts above */
    const float *g, *delta, *beta;
    const float *table;           /* f32 [H, M-1, M] */
    const float *q_norm_weight;   /* f32 [K] */
    const float *k_norm_weight;   /* f32 [K] */
    float q_norm_eps, k_norm_eps;
    float scale;                  /* pass-1 scale; the reference default is K^-1/2 */
    const float *h0_k;            /* nullable: initial key state   [B,H,K,M] */
    const float *h0_v;            /* nullable: initial value state [B,H,M,V] */
    const float *clock0;          /* nullable: initial clock       [B,H] */
    void *o;                      /* bf16 output [B,T,H,V] */
    float *hk, *hv, *clock;       /* nullable: final states (all three or none) */
    void *workspace;              /* device scratch, >= cyfa_chunk_workspace_bytes() */
    size_t workspace_bytes;
} CyfaChunkArgs;

/* Chunkwise two-pass CyFA forward: clock scan, write vector, pass-1
 * ScalarGatedLA with the fused slot-softmax readout, pass-2 ScalarGatedLA and
 * the final states. Replaces chunk_cyfa (ops/chunk.py:164-353) together with
 * the kernels it launches: clock_cumsum / clock_total (ops/utils.py:229-348),
 * phase_write (ops/utils.py:543-766), head_rmsnorm / query_rms_stats
 * (ops/qk_norm.py:64-297), head_gates / head_layout (ops/utils.py:351-492),
 * local_log2_cumsum (ops/utils.py:495-520), state_forward
 * (ops/chunk_h.py:10-339), first_readout (ops/chunk_readout.py:624-1136) and
 * output_forward (ops/chunk_o.py:10-613). Zero padding of T to a multiple of
 * C (ops/chunk.py:198-207) is handled inside the kernels. */
int cyfa_chunk_fwd(const CyfaChunkArgs *args, void *hip_stream);

/* Gated output norm of the layer (the o_norm(o * (num_slots - 1), gate) of
 * layers/cyfa.py:349-350, the same arithmetic as cyfa_rms_norm with D = V):
 *   xs = bf16(o * prescale);  o' = bf16(xs * rsqrt(mean(xs^2) + eps) * weight * sigmoid(gate)) */
typedef struct CyfaOutNormArgs {
    const float *weight;          /* f32 [V] */
    const void *gate;             /* bf16 [B,T,H,V] */
    float eps, prescale;
} CyfaOutNormArgs;

/* cyfa_chunk_fwd followed by the layer's gated output norm, applied in the
 * pass-2 epilogue before o is written, so that o' is written once and o never
 * reaches HBM. Replaces chunk_cyfa (ops/chunk.py:164-353) together with the
 * RMSNorm.execute call on its output (layers/cyfa.py:62-135, 349-350). args->o
 * receives o'. */
int cyfa_chunk_fwd_normed(const CyfaChunkArgs *args, const CyfaOutNormArgs *norm, void *hip_stream);

/* Size of the device scratch array behind cyfa_chunk_fwd_noalloc: 80 MiB,
 * enough for the workspace of configurations up to B * H * T = 131072
 * token-heads (e.g. B=8, T=2048, H=4 needs 44.5 MiB; B=1, T=16384, H=8 needs
 * 64 MiB). */
#define CYFA_NOALLOC_SCRATCH_BYTES (80ull << 20)

/* cyfa_chunk_fwd (norm == NULL) or cyfa_chunk_fwd_normed (norm set) that
 * allocates nothing and takes no workspace: args->workspace and
 * args->workspace_bytes are ignored, and the intermediates live in a device
 * array of CYFA_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds
 * until the process ends (its address is resolved on the first call on each
 * device: the device of hip_stream, or the current device for the null
 * stream). For callers that cannot allocate device memory: code under HIP
 * graph capture, serving loops that forbid allocation. No counterpart in the
 * reference. Calls whose workspace would exceed the array return
 * CYFA_ERR_UNSUPPORTED. Every call on one GPU uses that GPU's one array, so
 * calls that overlap on one GPU (different streams, or different threads
 * without ordering) race and give wrong results; calls in one stream are
 * ordered and safe. Every intermediate a call reads is written earlier in the
 * same call, so nothing in the array needs clearing between calls. */
int cyfa_chunk_fwd_noalloc(const CyfaChunkArgs *args, const CyfaOutNormArgs *norm, void *hip_stream);

/* Workspace bytes cyfa_chunk_fwd needs for these dimensions (the reference
 * allocates the equivalent intermediates through Jittor, ops/chunk.py:244-336). */
size_t cyfa_chunk_workspace_bytes(int B, int T, int H, int K, int V, int M, int C);

/* Arguments of one isolated ScalarGatedLA pass. (K, V) is (256, 128), the
 * pass-1 shape, or (128, 256), the pass-2 shape; T is a multiple of 64. */
typedef struct CyfaSlaArgs {
    int B, T, H, K, V;
    const void *q, *k;            /* bf16 [B,H,T,K] */
    const void *v;                /* bf16 [B,H,T,V], or [B,T,H,V] when v_bth */
    const float *g;               /* f32 [B,H,T], natural log of the per-token decay */
    const float *initial;         /* nullable f32 [B,H,K,V] (zero state) */
    float scale;
    int raw_output, output_bth, v_bth;
    void *o;                      /* [B,H,T,V], or [B,T,H,V] when output_bth;
                                     f32 when raw_output, else bf16 */
    float *final_state;           /* nullable f32 [B,H,K,V] */
    void *workspace;              /* device scratch, >= cyfa_scalar_la_workspace_bytes() */
    size_t workspace_bytes;
} CyfaSlaArgs;

/* One chunkwise scalar-gated linear-attention pass,
 *   S_{n+1} = 2^G_last S_n + k^T bf16(2^(G_last - G_s) v),
 *   o_t = scale (2^G_t q_t S_n + sum_{s<=t} bf16(2^(G_t - G_s) q_t.k_s) v_s),
 * G the in-chunk cumulative sum of g in log2 units, S_0 = initial. The output
 * is formed per 128-wide key slice, each slice rounded to bf16 after the scale,
 * and the slices summed (in f32 when raw_output, else rounded once more to
 * bf16). Replaces scalar_la / ScalarAttention (ops/chunk.py:30-79) with
 * state_forward (ops/chunk_h.py:10-339), local_log2_cumsum
 * (ops/utils.py:495-520) and output_forward (ops/chunk_o.py:177-613). */
int cyfa_scalar_la(const CyfaSlaArgs *args, void *hip_stream);

/* Workspace bytes cyfa_scalar_la needs for these dimensions. */
size_t cyfa_scalar_la_workspace_bytes(int B, int T, int H, int K, int V);

/* Arguments of one decode step (T == 1). */
typedef struct CyfaDecodeArgs {
    int B, H, K, V, M;
    const void *q, *k, *v;        /* bf16 [B,1,H,K|V] */
    const float *g, *delta, *beta;/* f32 [B,1,H] */
    const float *table;           /* f32 [H, M-1, M] */
    const float *q_norm_weight, *k_norm_weight;
    float q_norm_eps, k_norm_eps, scale;
    const float *hk_in, *hv_in, *clock_in; /* nullable (all or none): zero state */
    void *o;                      /* bf16 [B,1,H,V] */
    float *hk_out, *hv_out, *clock_out;    /* required; may alias the inputs */
    void *workspace;              /* nullable: >= cyfa_decode_workspace_bytes() bytes, 16-byte aligned */
    size_t workspace_bytes;
} CyfaDecodeArgs;

/* Workspace bytes that let a decode step with B H < 64 split each (b, h)
 * across eight workgroups (32 key-state rows and 32 value-state columns
 * each); 0 when B H >= 64 (one workgroup per (b, h) fills the chip). Without
 * the workspace the step runs one workgroup per (b, h); both forms give
 * bit-identical results. No counterpart in the reference (its decode kernel
 * runs one block per (b, h), ops/fused_recurrent.py:177-185). */
size_t cyfa_decode_workspace_bytes(int B, int H, int K, int V);

/* One fused constant-memory decode step: q/k RMS norm, clock and write
 * vector, key-state update and query, slot readout, value-state update and
 * output, in one HBM-streaming kernel. Replaces fused_recurrent_cyfa and its
 * decode kernel (ops/fused_recurrent.py:10-200). Updating in place
 * (hk_out == hk_in, ...) is allowed. */
int cyfa_decode_step(const CyfaDecodeArgs *args, void *hip_stream);

/* Prefetch ranges of cyfa_decode_layer_step, and the largest B H with which
 * it prefetches them. */
#define CYFA_PREFETCH_RANGES 4
#define CYFA_PREFETCH_MAX_BH 64

/* The rest of the layer's one-token step, for the decode loop (K = V = 256,
 * conv width 4, no conv bias). */
typedef struct CyfaDecodeLayerArgs {
    const void *qkv;              /* bf16 projection rows [B, qkv_row] before the convolution:
                                     q (H K) | k (H K) | v (H V) */
    long long qkv_row;
    const void *conv_cache;       /* nullable bf16 [B, 3, 3 H 256] (zero history) */
    void *conv_cache_out;         /* bf16, same addressing; may be conv_cache (updated in place) */
    long long cache_row, cache_batch;
    const void *conv_weight;      /* bf16 [3 H 256, 4], 8-byte aligned */
    const void *abd;              /* bf16 rows [B, abd_row]: a | b | d (H each), b and d biases added */
    long long abd_row;
    const float *dt_bias, *A_log; /* f32 [H] */
    const void *gate;             /* bf16 rows [B, gate_row]: [H 256], 8-byte aligned; or NULL, and
                                     the gate is formed in the kernel from g0 (below) */
    long long gate_row;
    const float *norm_weight;     /* f32 [256] */
    float norm_eps, norm_prescale;
    /* With gate NULL: gate = bf16(g0 g_weight^T + g_bias), the second projection
       of g_proj (layers/cyfa.py:292-295, 349), with the summation order of
       cyfa_linear_rows, so both ways give the same bits. */
    const void *g0;               /* bf16 rows [B, g0_row]: [256] (the output of g_proj[0]), 16-byte aligned */
    long long g0_row;             /* a multiple of 8 */
    const void *g_weight;         /* bf16 [H 256, 256], 16-byte aligned */
    const void *g_bias;           /* nullable bf16 [H 256] */
    /* Cache prefetch (no reference counterpart; all NULL / 0: no ranges). At
       small batches the step occupies one compute unit per (batch, head), and
       one compute unit's loads reach a small fraction of HBM's rate. With
       B H <= CYFA_PREFETCH_MAX_BH the launch adds workgroups on the idle
       compute units: they first read each step workgroup's own state, readout
       table and g_weight rows into the L2 of the XCD that runs it, then these
       device ranges -- the weights of the projections that follow the step --
       into the caches. The extra workgroups write nothing and no result
       depends on them. The ranges are only read (16-byte aligned, each below
       2^31 bytes). prefetch_span[r]: 0, or the bytes of range r that each
       workgroup of the projection reading it takes, workgroup c the bytes
       [c span, (c + 1) span) (cyfa_linear_rows_span); each piece is then read
       into the L2 of the XCD that workgroup c runs on (workgroups are dealt
       to the eight XCDs by block id, c mod 8). A multiple of 16 below 2^31. */
    const void *prefetch[CYFA_PREFETCH_RANGES];
    unsigned long long prefetch_bytes[CYFA_PREFETCH_RANGES];
    unsigned long long prefetch_span[CYFA_PREFETCH_RANGES];
} CyfaDecodeLayerArgs;

/* cyfa_decode_step with the layer around it in the same kernel: q, k and v
 * from the width-4 causal short convolution of the projection row and the new
 * conv cache (ShortConvolution, layers/cyfa.py:138-233), the gate activations
 * from the a|b|d row (layers/cyfa.py:323-326), and args->o receives the gated
 * output norm o_norm(o * prescale, gate) (layers/cyfa.py:349-350) instead of
 * o. args->q, k, v, g, delta and beta are not read. Replaces those steps of
 * CyclicFlowAttention.execute for a one-token step together with
 * fused_recurrent_cyfa (ops/fused_recurrent.py:10-200). With every output
 * apart from its input (hk, hv, clock and conv cache; no partial overlap)
 * and B H <= 32 the launch runs 4 (B H <= 16) or 2 workgroups per (b, h),
 * each computing the whole step and storing its share: the same bits as the
 * one-workgroup form, which in-place calls keep. */
int cyfa_decode_layer_step(const CyfaDecodeArgs *args, const CyfaDecodeLayerArgs *layer, void *hip_stream);

/* table[h] = readout[h] @ Phi, with Phi the real-DFT slot basis [M-1, M].
 * Replaces _basis + jt.matmul (ops/chunk.py:82-103, 281;
 * ops/fused_recurrent.py:53). readout f32 [H, M-1, M-1]; table f32 [H, M-1, M];
 * M even in [4, 256]. */
int cyfa_readout_table(const float *readout, float *table, int H, int M, void *hip_stream);

/* Element type of q, k, v and o in the general-shape entry points. */
enum { CYFA_DTYPE_BF16 = 0, CYFA_DTYPE_F32 = 1 };

/* Workspace bytes of cyfa_chunk_fwd_general (0 for a non-positive argument):
 * per (b, h, token padded to a multiple of 64) row the normalised rows, the
 * clock, the write vector, both passes' row outputs and the phases, plus the
 * fp32 states before every 64-token chunk of both passes,
 * 4 B H (T/64 + 1)(K M + M V) bytes. C does not change it. */
size_t cyfa_chunk_general_workspace_bytes(int B, int T, int H, int K, int V, int M, int C);

/* The chunkwise forward for shapes outside cyfa_chunk_fwd's (the
 * reference's unfused fallback: _scalar_la, the affine scan over chunks, the
 * modal readout and _rotate, ops/chunk.py:115-161, 285-331 and
 * ops/utils.py:98-226, 779-929): K and V in [1, 1024], M even in [4, 256],
 * C in {16, 32, 64}, B * H <= 65535; q, k, v and o of `dtype` (bf16 or
 * fp32), everything else as for cyfa_chunk_fwd. Computes in fp32; bf16 inputs
 * are rounded to bf16 where the reference casts to the input dtype. Each pass
 * runs chunk-parallel over 64-token chunks whatever C is (C changes no value
 * beyond fp32 summation order): a scan forms the states before every chunk,
 * then every chunk's output is formed from its state and its own rows. */
int cyfa_chunk_fwd_general(const CyfaChunkArgs *args, int dtype, void *hip_stream);

/* One decode step for shapes outside cyfa_decode_step's, up to the
 * reference's decode limits (ops/fused_recurrent.py:45-46): K and V in
 * [1, 1024], M even in [4, 256]; q, k, v and o of `dtype`; states fp32; the
 * workspace fields are ignored. One workgroup per (b, h). fp32 at
 * cyfa_decode_step's shapes (K, V in {128, 256}, M = 128, with its alignment)
 * runs that kernel without its bf16 rounding points. */
int cyfa_decode_step_general(const CyfaDecodeArgs *args, int dtype, void *hip_stream);

/* ---- Backward pass of the chunk op ---- */

/* Cotangents in and gradients out of cyfa_chunk_bwd. Layouts as for
 * CyfaChunkArgs; dq, dk, dv take the operands' dtype, the rest is f32. */
typedef struct CyfaChunkBwdArgs {
    const void *d_o;              /* nullable (zero) cotangent of o [B,T,H,V] */
    const float *d_hk;            /* nullable cotangent of the final key state   [B,H,K,M] */
    const float *d_hv;            /* nullable cotangent of the final value state [B,H,M,V] */
    const float *d_clock;         /* nullable cotangent of the final clock       [B,H] */
    void *dq, *dk, *dv;           /* [B,T,H,K], [B,T,H,K], [B,T,H,V] */
    float *dg, *ddelta, *dbeta;   /* [B,T,H] */
    float *dtable;                /* [H,M-1,M]: gradient of the readout table */
    float *dreadout;              /* nullable [H,M-1,M-1]: dtable @ Phi^T, the readout's gradient */
    float *dq_norm_weight;        /* [K] */
    float *dk_norm_weight;        /* [K] */
    float *dh0_k, *dh0_v, *dclock0; /* gradients of the initial states: all three or none */
    void *workspace;              /* device scratch, >= cyfa_chunk_bwd_workspace_bytes() */
    size_t workspace_bytes;
} CyfaChunkBwdArgs;

/* Workspace bytes of cyfa_chunk_bwd (0 for a non-positive argument): the
 * recomputed fp32 rows (q_hat, k_hat, v, the cotangent of o), the states
 * before every chunk of both passes and their cotangents (fp32,
 * 4 B H (N + 1) K M bytes per stack, N = ceil(T / 64)) and the rows'
 * cotangents (above 128 slots also the logits / probabilities and their
 * cotangents, 2 x 1 KiB per row); about 1.4 GB at B=8, T=2048, H=4,
 * K=V=256, M=128.
 * cyfa_chunk_bwd refuses B H ceil(T / 64) 64 >= 2^21 padded rows (its
 * kernels index rows and chunk states with 32-bit counts). */
size_t cyfa_chunk_bwd_workspace_bytes(int B, int T, int H, int K, int V, int M);

/* Gradients of the chunkwise CyFA op with respect to q, k, v, g, delta, beta,
 * the readout table (and readout), both q/k norm weights and the initial
 * states, given the cotangents of o and of the final states. `fwd` holds the
 * forward call's inputs (its o, hk, hv, clock and workspace fields are not
 * read; its C is ignored: the backward works in 64-token chunks); q, k, v
 * and d_o are of `dtype` (bf16 or fp32). K and V in [1, 1024], M even in
 * [4, 256] (the reference's limit; above 128 slots the readout's adjoint
 * streams the table through tile GEMMs instead of staging it on chip). The
 * forward is recomputed in fp32 without intermediate rounding,
 * so the gradients are those of the op's exact arithmetic. Replaces the
 * autograd adjoints behind chunk_cyfa: ScalarAttention.grad / scalar_grad
 * (ops/chunk.py:51-71, ops/chunk_bwd.py:1008-1041), FirstReadout*.grad
 * (ops/chunk_readout.py:13-621, 776-786, 976-988), PhaseWrite.grad and
 * ClockScan.grad (ops/utils.py:297-299, 589-641, 704-754), HeadRMSNorm.grad
 * (ops/qk_norm.py:241-289) and the table matmul's (ops/chunk.py:281). */
int cyfa_chunk_bwd(const CyfaChunkArgs *fwd, int dtype, const CyfaChunkBwdArgs *bwd, void *hip_stream);

/* ---- Layer-side kernels around the op (layers/cyfa.py, modeling_cyfa.py) ---- */

/* Arguments of one RMSNorm over rows of D bf16 values (D a multiple of 256, at
 * most 2048). The residual add of the surrounding block is fused in front:
 *   s   = residual ? bf16(x + residual) : x           (written to sum_out)
 *   xs  = prescale != 1 ? bf16(s * prescale) : s
 *   out = bf16(xs * rsqrt(mean(xs^2) + eps) * weight * (gate ? sigmoid(gate) : 1)) */
typedef struct CyfaNormArgs {
    int rows, D;
    const void *x;                /* bf16 [rows, D] */
    const void *residual;         /* nullable bf16 [rows, D] */
    void *sum_out;                /* bf16 [rows, D]; required when residual is set */
    const float *weight;          /* f32 [D] */
    const void *gate;             /* nullable bf16 [rows, D] */
    float eps, prescale;
    void *out;                    /* bf16 [rows, D] */
} CyfaNormArgs;

/* Replaces RMSNorm.execute / RMSNorm._inference (layers/cyfa.py:62-135; the
 * gated form is the o_norm(o * (num_slots - 1), gate) of layers/cyfa.py:350)
 * and the residual adds of CyFABlock.execute (modeling_cyfa.py:48-51). */
int cyfa_rms_norm(const CyfaNormArgs *args, void *hip_stream);

/* Row-wise argmax of bf16 rows x[r * ldx .. + n) into out[r] (int64), with
 * torch.argmax's result: the index of the first maximum, NaN counting as the
 * largest value. Replaces the greedy token choice of a decode step
 * (logits.argmax, models/cyfa/modeling_cyfa.py:142-158; generation.py:43).
 * x 16-byte aligned, ldx a multiple of 8, n below 2^30. */
int cyfa_argmax_rows(const void *x, long long ldx, int rows, int n, long long *out, void *hip_stream);

/* Arguments of one projection y = x W^T (+ bias) over at most 64 rows of x
 * (1 <= M <= 64; K a positive multiple of 32). With swiglu set (no bias, N a
 * multiple of 32), the rows of W come in groups of 32: 16 rows of the gate
 * projection, then the matching 16 rows of the up projection, and y [M, N/2]
 * receives the SwiGLU product bf16(g sigmoid(g) u) of the bf16-rounded g and u
 * (GatedMLP, models/cyfa/modeling_cyfa.py:22-27). With residual set, y is the
 * block's residual add around the projection (CyFABlock.execute,
 * models/cyfa/modeling_cyfa.py:48-51). */
#define CYFA_LINEAR_PREFETCH_RANGES 2

typedef struct CyfaLinearArgs {
    int M, N, K;
    const void *x;                /* bf16 [M, K], rows ldx elements apart (ldx >= K, ldx % 8 == 0) */
    long long ldx;
    const void *weight;           /* bf16 [N, K] row-major (torch Linear weight) */
    const void *bias;             /* nullable bf16 [N] */
    void *y;                      /* bf16 [M, N] ([M, N/2] with swiglu), rows ldy elements apart */
    long long ldy;
    int swiglu;
    const void *residual;         /* nullable bf16 [M, N], rows ldr apart: y = bf16(residual + bf16(x W^T + b));
                                     not with swiglu; may be y itself */
    long long ldr;
    /* Cache prefetch (no reference counterpart; all NULL / 0: none): extra
       workgroups of the launch, on the compute units its tiles leave idle,
       read prefetch[r] (prefetch_bytes[r] bytes, 16-byte aligned, below 2^31)
       into the caches for the launch after this one, with prefetch_span[r] as
       in CyfaDecodeLayerArgs (0, or the bytes each workgroup of that launch
       reads, cyfa_linear_rows_span: each piece then lands in the L2 of the XCD
       that reads it). Nothing is written; the projection's result does not
       depend on it. */
    const void *prefetch[CYFA_LINEAR_PREFETCH_RANGES];
    unsigned long long prefetch_bytes[CYFA_LINEAR_PREFETCH_RANGES];
    unsigned long long prefetch_span[CYFA_LINEAR_PREFETCH_RANGES];
} CyfaLinearArgs;

/* Replaces the Linear / BiasLinear projections (layers/cyfa.py:15-58) of the
 * one-token decode step when it has at most 64 rows: the q/k/v, a/b/d, g and
 * o projections of CyclicFlowAttention.execute (layers/cyfa.py:302, 323-326,
 * 349, 351), the GatedMLP projections (models/cyfa/modeling_cyfa.py:13-28) and
 * the lm_head (models/cyfa/modeling_cyfa.py:80, 100). fp32 accumulation, one bf16
 * rounding. */
int cyfa_linear_rows(const CyfaLinearArgs *args, void *hip_stream);

/* The bytes of the weight that each workgroup of a cyfa_linear_rows (norm 0)
 * or cyfa_norm_linear_rows (norm 1: with the norm weight, 2: folded) launch
 * of this shape reads, when the workgroups that read the bytes [c span,
 * (c + 1) span) of the weight all run on XCD c mod 8 (workgroup c alone, or
 * with several row tiles the row tiles of N tile c); 0 when a workgroup reads
 * its weight rows in separate pieces, and for shapes the launchers refuse. A
 * host-side query for the prefetch_span fields of CyfaDecodeLayerArgs and
 * CyfaLinearArgs. No reference counterpart. */
size_t cyfa_linear_rows_span(int M, int N, int K, int swiglu, int norm);

/* The RMS norm in front of a projection (K <= 2048 columns):
 *   s  = residual ? bf16(x + residual) : x        (sum_out receives s)
 *   xs = bf16(s * rsqrt(mean(s^2) + eps) * weight)
 * and the projection reads xs in place of x. With weight NULL the caller has
 * multiplied the norm weight into the projection's weight (W' = bf16(W
 * diag(weight))), and the row scale is applied to the fp32 product instead of
 * the operand: y = bf16(rsqrt(mean(s^2) + eps) (s W'^T) + bias). That moves
 * the bf16 rounding of the normalised input to W' (one rounding of each
 * product term either way) and skips the per-element scaling of xs. */
typedef struct CyfaRowNormArgs {
    const float *weight;          /* f32 [K], 16-byte aligned; NULL: folded into the weight (above) */
    float eps;
    const void *residual;         /* nullable bf16 [M, K], rows ldr elements apart */
    void *sum_out;                /* bf16 [M, K], rows ldr apart; required with residual; aliases no input */
    long long ldr;
} CyfaRowNormArgs;

/* Replaces the pre-norm in front of the first projection of each block of a
 * decode step: attn_norm (with the residual add x + attn(...)) before the q/k/v,
 * g and a/b/d projections, and mlp_norm before the GatedMLP gate/up projection
 * (CyFABlock.execute, models/cyfa/modeling_cyfa.py:48-51; RMSNorm,
 * layers/cyfa.py:62-135). The norm's sum of squares runs in another order than
 * cyfa_rms_norm's, so xs may differ from it in the last bit. */
int cyfa_norm_linear_rows(const CyfaLinearArgs *args, const CyfaRowNormArgs *norm, void *hip_stream);

/* The prefill gate path of CyclicFlowAttention.execute for M token rows x
 * [M, K] (layers/cyfa.py:292-295, 323-326, 349): the g_proj[0] and a|b|d
 * projections, the gate activations and g_proj[1] in one launch:
 *   c  = x [W_g0 | W_a | W_b | W_d]^T          (256 + 3H columns)
 *   g0 = bf16(c[:, :256]),  abd = bf16(c[:, 256:] + abd_bias)
 *   g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), delta = sigmoid(d)
 *   gate = bf16(g0 W_g1^T + b_g1)
 * with fp32 accumulation and the roundings of the separate projections (the
 * summation order differs from a library GEMM's, so a value can differ from
 * theirs in the last bit). K a multiple of 64 up to 2048, 3H <= 32, Dv a
 * multiple of 256 up to 2048, g_proj[0] 256 wide. No reference counterpart as
 * one entry point. */
typedef struct CyfaGatePathArgs {
    int M, K, H, Dv;
    const void *x;                /* bf16 [M, K], rows ldx elements apart, 16-byte aligned */
    long long ldx;                /* a multiple of 8, >= K */
    const void *w1;               /* bf16 [256 + 3H, K]: g_proj[0] rows, then a, b, d rows; 16-byte aligned */
    const void *abd_bias;         /* bf16 [3H] (zero for the a part) */
    const void *w2;               /* bf16 [Dv, 256] g_proj[1] weight, 16-byte aligned */
    const void *b2;               /* nullable bf16 [Dv] g_proj[1] bias */
    const float *dt_bias, *A_log; /* f32 [H] */
    void *gate;                   /* bf16 [M, Dv], rows ldg elements apart, 16-byte aligned */
    long long ldg;                /* a multiple of 8, >= Dv */
    float *g, *beta, *delta;      /* f32 [M, H] */
} CyfaGatePathArgs;

int cyfa_gate_path(const CyfaGatePathArgs *args, void *hip_stream);

/* Arguments of one causal depthwise convolution over time of B x T rows of D
 * bf16 channels (D a multiple of 8, W in 2..4):
 *   y[b,t,c] = bias[c] + sum_{w<W} weight[c,w] * X[b, t + w - (W-1), c],
 * X[b,i] = x[b,i] for i >= 0, else cache[b, W-1+i] (or 0 without a cache).
 * Channel c is written to out[c / split] at column c % split, so one launch
 * can convolve a fused q|k|v projection into three tensors. When cache_out is
 * set it receives the new cache, X[b, T-(W-1) .. T-1] (layers/cyfa.py:172-182);
 * it may be the cache itself when T <= 32. */
typedef struct CyfaConvArgs {
    int B, T, D, W;
    const void *x;                /* bf16, element (b,t,c) at x[(b*T + t)*x_row + c] */
    long long x_row;
    const void *cache;            /* nullable bf16, (b,i,c) at cache[b*cache_batch + i*cache_row + c] */
    long long cache_row, cache_batch;
    const void *weight;           /* bf16 [D, W] */
    const void *bias;             /* nullable bf16 [D] */
    void *out[3];                 /* bf16 [B, T, split] each; D / split of them used */
    int split;
    void *cache_out;              /* nullable bf16, same addressing as cache with cache_out_row / _batch */
    long long cache_out_row, cache_out_batch;
} CyfaConvArgs;

/* Replaces ShortConvolution.execute / _inference (layers/cyfa.py:138-233); the
 * new cache (the last W-1 inputs) stays a view of the input in the caller. */
int cyfa_short_conv(const CyfaConvArgs *args, void *hip_stream);

/* out[r, c] = bf16(g sigmoid(g) u), g = gu[r, c], u = gu[r, F + c]; F a
 * multiple of 8. Replaces the activation of GatedMLP.execute
 * (modeling_cyfa.py:22-27). */
int cyfa_silu_mul(const void *gu, void *out, int rows, int F, void *hip_stream);

/* Gate activations from the fused a|b|d projection abd [rows, 3H] bf16 (rows
 * abd_row elements apart; b and d biases included): g = -exp(A_log)
 * softplus(a + dt_bias), beta = sigmoid(b), delta = sigmoid(d), f32 [rows, H].
 * Replaces layers/cyfa.py:323-326. */
int cyfa_gates(const void *abd, long long abd_row, const float *dt_bias, const float *A_log, float *g, float *beta,
               float *delta, int rows, int H, void *hip_stream);

/* Thread-local message of the last failing call (never NULL). No reference
 * counterpart: Jittor reports kernel errors as C++ exceptions. */
const char *cyfa_last_error(void);

/* CYFA_ABI_VERSION of the loaded library. No reference counterpart. */
int cyfa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CYFA_ABI_H */
