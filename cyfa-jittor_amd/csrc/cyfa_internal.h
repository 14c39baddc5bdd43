// cyfa_internal.h -- kernel parameter blocks and launchers shared between the
// C-ABI layer (cyfa_abi.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace cyfa {

struct DecodeParams {
    int B, H;
    const __bf16 *q, *k, *v;
    const float *g, *delta, *beta, *table, *q_w, *k_w;
    float q_eps, k_eps, scale;
    const float *hk_in, *hv_in, *clock_in;
    __bf16* o;
    float *hk_out, *hv_out, *clock_out;
    int f32;  // the op step with q, k, v and o in fp32 (computed without bf16 rounding)
    // Layer step (decode_step_kernel<.., true>): q, k, v come from the width-4
    // short convolution of the projection row qkv, the gates from abd, and o
    // receives the gated output norm instead of the op's output.
    const __bf16* qkv;       // row b at qkv + b * qkv_row: q (H K) | k (H K) | v (H V)
    long long qkv_row;
    const __bf16* cache_in;  // nullable: [B, 3, 2 H K + H V] rows cache_row, batches cache_batch
    __bf16* cache_out;       // the new cache, same addressing (may be cache_in)
    long long cache_row, cache_batch;
    const __bf16* conv_w;    // [2 H K + H V, 4]
    const __bf16* abd;       // row b at abd + b * abd_row: a (H) | b (H) | d (H)
    long long abd_row;
    const float *dt_bias, *A_log;
    const __bf16* gate;      // row b at gate + b * gate_row: [H V]
    long long gate_row;
    const float* on_w;       // [V]
    float on_eps, on_prescale;
    // gate null: gate = bf16(g0 g1_w^T + g1_b) formed in the kernel, row b of
    // g0 at g0 + b * g0_row ([V]), g1_w [H V, V], g1_b nullable [H V]
    const __bf16* g0;
    long long g0_row;
    const __bf16 *g1_w, *g1_b;
    // Small batches (B H < DECODE_SPLIT_BH): the workspace for the slices'
    // partial raw, [B H, max(K, V) / 32, 128] f32; null: one workgroup per (b, h).
    float* part;
    // Layer step, one-workgroup form: pf_wgs extra workgroups (block ids B H
    // onward) read the ranges pf[r] of pf_bytes[r] bytes (each below 2^31,
    // 16-byte aligned; 0: none) into the caches and exit.
    const void* pf[4];
    unsigned long long pf_bytes[4];
    // 0, or the bytes of range r each workgroup of its consumer reads (the
    // consumer's workgroup c reads [c span, (c + 1) span), on XCD c mod 8)
    unsigned long long pf_span[4];
    int pf_wgs;
    // With pf_wgs > 0: the extra workgroups first read the step workgroups'
    // own inputs (hk, hv, the head's table and g_proj[1] rows) into the L2 of
    // the XCD each step workgroup runs on.
    int self_pf;
    // Layer step, one-workgroup form: step workgroups per (b, h), 1, 2 or 4
    // (more than one only with every output apart from its input: each
    // workgroup reads all of the (b, h)'s inputs and stores its share).
    int wpb;
};

// B H up to which the layer step's extra workgroups prefetch the step
// workgroups' own inputs (each XCD's L2 then holds about 450 KB per step
// workgroup dealt to it, 3.6 MB at 64).
constexpr int DECODE_SELF_PREFETCH_MAX_BH = 64;
// B H up to which the layer step runs 4 (2) step workgroups per (b, h) when
// its outputs are apart from its inputs.
constexpr int DECODE_WPB4_MAX_BH = 16;
constexpr int DECODE_WPB2_MAX_BH = 32;

// B H below which a decode step is split across eight workgroups per (b, h).
constexpr int DECODE_SPLIT_BH = 64;
// Workspace bytes of the split decode step (0 when B H does not split).
size_t decode_workspace_bytes(int B, int H, int K, int V);

// Prefill: T is split into N = ceil(T / 64) chunks and every (batch, head)
// sequence into P segments of L consecutive chunks. Segments run in parallel;
// each forms its start state from the segment-local end states before it.
struct PrefillParams {
    int B, T, H, K, V;
    int N, Tp;  // chunks, padded length N * 64
    int P, L;   // segments per sequence, chunks per segment
    const __bf16 *q, *k, *v;
    const float *g, *delta, *beta;
    const float* table;  // f32 [H, 127, 128]
    const float *q_w, *k_w;
    float q_eps, k_eps, scale;
    float log2_scale;  // log2(scale), formed on the host (exact for powers of two)
    const float *h0_k, *h0_v, *clock0;
    __bf16* o;
    float *hk, *hv, *clock;
    // Optional gated output norm applied to o in the pass-2 epilogue (on_w null: none):
    //   xs = bf16(bf16(o) * on_prescale); o = bf16(xs * rsqrt(mean_V xs^2 + on_eps) * on_w * sigmoid(on_gate))
    const float* on_w;       // f32 [V]
    const __bf16* on_gate;   // bf16 [B, T, H, V]
    float on_eps, on_prescale;
    // workspace
    float* lam;        // [B*H, Tp] reduced clock per token, (lam mod 127) / 127
    float* gam;        // [B*H, Tp] in-chunk inclusive scan of g, log2 units
    _Float16* seg;     // [B*H, P-1, K*128 + 128*V] segment-local end states (register order),
                       // each wave's block scaled by 2^-seg_exp
    int* seg_exp;      // [B*H, P-1, 2, 8] power-of-two exponent per (key / value part, wave)
    float* seg_decay;  // [B*H, P] product of alpha over each segment
    __bf16* omega;     // [B*H, Tp, 128] slot weights between the two passes
    int* tab_exp;      // [B*H] power-of-two exponent e of the head's readout table: max |table| 2^-e < 2^14
    _Float16* tab16;   // [H, 128, 128] table 2^-e in fp16, row 127 zero (written by segment_state)
};

// Isolated ScalarGatedLA, one pass (scalar_la): every operand read from memory.
// (K, V) is (256, 128) or (128, 256); T is a multiple of 64. Segments as in
// the prefill, with one state part per segment.
struct SlaParams {
    int B, T, H, K, V;
    int N, P, L;
    const __bf16 *q, *k, *v;  // q, k [B, H, T, K]; v [B, H, T, V] or [B, T, H, V] (v_bth)
    const float* g;           // [B, H, T] natural-log decay
    const float* h0;          // nullable [B, H, K, V]
    float scale;
    int v_bth, o_bth, raw_output;
    void* o;                  // [B, H, T, V] or [B, T, H, V] (o_bth); f32 if raw_output else bf16
    float* hfinal;            // nullable [B, H, K, V]
    // workspace
    _Float16* seg;     // [B*H, P-1, K*V] segment-local end states (register order)
    int* seg_exp;      // [B*H, P-1, 8]
    float* seg_decay;  // [B*H, P]
};

struct SlaWorkspaceLayout {
    size_t seg, seg_exp, seg_decay, total;
};

SlaWorkspaceLayout sla_workspace_layout(int B, int T, int H, int K, int V);
int launch_scalar_la(const SlaParams& p, hipStream_t stream);

// Layer-side kernels (cyfa_layer.hip).
struct NormParams {
    int rows, D;
    const __bf16 *x, *residual;  // residual nullable
    __bf16* sum_out;             // receives bf16(x + residual) when residual is set
    const float* weight;         // fp32 [D]
    const __bf16* gate;          // nullable, [rows, D]
    float eps, prescale;
    __bf16* out;
};

struct ConvParams {
    int B, T, D, W;
    const __bf16* x;
    long long x_row;             // elements between time rows of x
    const __bf16* cache;         // nullable: [B, W-1, D] view
    long long cache_row, cache_batch;
    const __bf16 *weight, *bias; // [D, W], nullable [D]
    __bf16* out[3];              // channel c -> out[c / split][(b*T + t)*split + c % split]
    int split;
    __bf16* cache_out;           // nullable: the last W-1 rows of X, cache addressing
    long long cache_out_row, cache_out_batch;
};

struct WorkspaceLayout {
    size_t lam, gam, seg, seg_exp, seg_decay, omega, tab_exp, tab16, total;
};

// Largest byte span of one sequence's rows that the kernels' 32-bit buffer
// offsets can address.
constexpr size_t MAX_SPAN_BYTES = 0xffffffffull;

// Compute units of the current device (256 when no device is visible).
int device_cu_count();
void choose_segments(int BH, int N, int* P, int* L);
WorkspaceLayout workspace_layout(int B, int T, int H, int K, int V);

int launch_decode_step(const DecodeParams& p, int K, int V, hipStream_t stream);
int launch_prefill(const PrefillParams& p, hipStream_t stream);
int launch_readout_table(const float* readout, float* table, int H, hipStream_t stream);
// y = x W^T (+ bias) for at most 64 rows of x (the one-token decode step's projections).
constexpr int LINEAR_PREFETCH_RANGES = 2;

struct LinearParams {
    int M, N, K;
    const __bf16* x;     // [M, K], rows ldx elements apart
    long long ldx;
    const __bf16* w;     // [N, K] row-major (torch Linear weight)
    const __bf16* bias;  // nullable [N]
    __bf16* y;           // [M, N], rows ldy elements apart ([M, N / 2] with swiglu)
    long long ldy;
    int swiglu;          // W rows interleaved per 32: 16 gate rows, then the matching 16 up rows;
                         // y = bf16(g sigmoid(g) u) of the bf16-rounded g and u
    const __bf16* add;   // nullable [M, N], rows ld_add apart: y = bf16(add + bf16(x W^T + bias)); no swiglu
    long long ld_add;
    // Optional RMS norm of the x rows before the product (over all K columns):
    //   s = norm_residual ? bf16(x + residual) : x   (norm_sum_out receives s)
    //   the product reads bf16(s * rsqrt(mean(s^2) + norm_eps) * norm_weight),
    //   or, with norm_folded (norm_weight null; the caller has multiplied the
    //   norm weight into w), y = rsqrt(mean(s^2) + norm_eps) (s W^T) + bias
    //   with the row scale applied to the fp32 product
    const float* norm_weight;     // nullable: x is used as given (unless norm_folded)
    int norm_folded;
    const __bf16* norm_residual;  // nullable [M, K], rows ldr elements apart (launch_linear_rows forms s first)
    __bf16* norm_sum_out;         // [M, K], rows ldr apart; set with norm_residual; aliases no input
    long long ldr;
    float norm_eps;
    // Cache prefetch for the launch after this one: the ranges pf[r] (pf_bytes[r]
    // bytes, below 2^31; pf_span[r] as DecodeParams.pf_span) are read by pf_wgs
    // extra workgroups after the tiles
    const void* pf[LINEAR_PREFETCH_RANGES];
    unsigned long long pf_bytes[LINEAR_PREFETCH_RANGES];
    unsigned long long pf_span[LINEAR_PREFETCH_RANGES];
    int pf_wgs;
    int grid_x, grid_y;  // tiles along N (padded to a multiple of 8 when grid_y > 1) and along M; set by the launcher
};

constexpr int LINEAR_NORM_MAX_K = 2048;

// Bytes of W each workgroup of launch_linear_rows reads at this shape when
// workgroup c reads exactly W bytes [c span, (c + 1) span); 0 otherwise
// (norm: 0 none, 1 with the norm weight, 2 folded).
unsigned long long linear_rows_span(int M, int N, int K, bool swiglu, int norm);

// The prefill gate path of a layer for rows of tokens x [M, K]:
//   c = x [W_g0 | W_a | W_b | W_d]^T   (256 + 3H columns)
//   g0 = bf16(c[:, :256]); abd = bf16(c[:, 256:] + abd_bias)
//   g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), delta = sigmoid(d)
//   gate = bf16(g0 W_g1^T + b_g1)      (Dv columns)
struct GatePathParams {
    int M, K, H, Dv;
    const __bf16* x;         // [M, K], rows ldx elements apart
    long long ldx;
    const __bf16* w1;        // [256 + 3H, K]: g_proj[0] rows, then a, b, d rows
    const __bf16* abd_bias;  // [3H] (the a part zero)
    const __bf16* w2;        // [Dv, 256] g_proj[1] weight
    const __bf16* b2;        // nullable [Dv]
    const float *dt_bias, *A_log;  // [H]
    __bf16* gate;            // [M, Dv], rows ldg elements apart
    long long ldg;
    float *g, *beta, *delta;  // [M, H]
};
constexpr int GATE_PATH_G0 = 256;       // g_proj[0] width (head_v_dim) the kernel is built for
constexpr int GATE_PATH_MAX_K = 2048;   // largest hidden size (its k-chunk loop is unrolled to this)
constexpr int GATE_PATH_MAX_DV = 2048;  // largest H * head_v_dim (its column rounds, likewise)

// Largest slot count of the backward pass, and of its readout kernels that
// stage a head's table in LDS; above BWD_TABLE_M the readout and its adjoint
// run as tile GEMMs that stream the table (the "wide" readout).
constexpr int BWD_MAX_M = 256;
constexpr int BWD_TABLE_M = 128;

constexpr int BWD_WIDE_MW = 256;    // columns of the wide readout's per-row buffers

// The general-shape path (cyfa_general.hip): any K, V <= 1024, even M in
// [4, 256], C in {16, 32, 64}, bf16 or fp32 q, k, v. It computes in chunks of
// 64 tokens whatever C is (C changes no value beyond fp32 summation order).
constexpr int GEN_CHUNK = 64;

// One chunkwise ScalarGatedLA pass, chunk-parallel (cyfa_backward.hip): the
// states before every chunk by a scan over the chunks, then every chunk's
// output from its state and its own rows.
//   o_t = scale (e^{G_t} q_t S_n + sum_{s <= t in chunk n} e^{G_t - G_s} (q_t . k_s) v_s)
//   S_{n+1} = e^{G_last} S_n + sum_s k_s^T e^{G_last - G_s} v_s
struct ChunkPassParams {
    const float *q, *k, *v;  // head-major fp32 [B*H, Tp, Kq | Vd], Tp a multiple of 64, rows past T zero
    const float* g;          // [B, T, H] natural-log gate (tokens past T add zero)
    const float* s0;         // nullable [B*H, Kq, Vd]
    float* states;           // workspace [B*H, Tp / 64 + 1, Kq, Vd]
    float* s_final;          // nullable [B*H, Kq, Vd]
    float* out;              // head-major fp32 [B*H, Tp, Vd] (nullable when out_bthd is set)
    void* out_bthd;          // nullable [B, T, H, Vd], bf16 when bf16 else fp32
    int bf16;                // round the output to bf16 (the input dtype's cast)
    int mfma;                // tile products on the matrix cores (split bf16 operands, ~16 bits)
    int sbf16;               // with mfma: states stored as bf16 (the workspace then holds bf16_t)
    int B, T, Tp, H, Kq, Vd;
    float scale;
};

struct GenChunkParams {
    int B, T, H, K, V, M, C, bf16;
    const void *q, *k, *v;
    const float *g, *delta, *beta, *table, *q_w, *k_w;
    float q_eps, k_eps, scale;
    const float *h0_k, *h0_v, *clock0;
    void* o;
    float *hk, *hv, *clock;
    void* workspace;
};

struct GenDecodeParams {
    int B, H, K, V, M;
    const void *q, *k, *v;
    const float *g, *delta, *beta, *table, *q_w, *k_w;
    float q_eps, k_eps, scale;
    const float *hk_in, *hv_in, *clock_in;
    void* o;
    float *hk_out, *hv_out, *clock_out;
};

// The general chunk path's workspace: per (b, h, padded token) row the clock
// (f64), q_hat and k_hat (K), v (V), the write vector, the pass-1 output and
// the slot weights (M each) and the phases' cosines and sines (M / 2 each);
// the states before every chunk of both passes; with M > 128 the readout's
// per-row logits (BWD_WIDE_MW columns); all fp32, each region 256-byte
// aligned, tokens padded to a multiple of GEN_CHUNK. With base == nullptr
// only the size.
struct GenWorkspace {
    double* lam;
    float *qh, *kh, *vh, *w, *cs, *sn, *raw, *wts, *sk, *sv, *lg;
    int Tp;
    size_t bytes;
};

inline GenWorkspace general_workspace(int B, int T, int H, int K, int V, int M, void* base) {
    const size_t Tp = (size_t)(T + GEN_CHUNK - 1) / GEN_CHUNK * GEN_CHUNK, rows = (size_t)B * H * Tp;
    const size_t BH = (size_t)B * H, N1 = Tp / GEN_CHUNK + 1;
    char* p = static_cast<char*>(base);
    size_t off = 0;
    const auto take = [&](size_t bytes) {
        char* r = p ? p + off : nullptr;
        off += (bytes + 255) / 256 * 256;
        return r;
    };
    const auto f = [&](size_t n) { return reinterpret_cast<float*>(take(n * 4)); };
    GenWorkspace w;
    w.Tp = (int)Tp;
    w.lam = reinterpret_cast<double*>(take(rows * 8));
    w.qh = f(rows * K);
    w.kh = f(rows * K);
    w.vh = f(rows * V);
    w.w = f(rows * M);
    w.cs = f(rows * (M / 2));
    w.sn = f(rows * (M / 2));
    w.raw = f(rows * M);
    w.wts = f(rows * M);
    w.sk = f(BH * N1 * K * M);
    w.sv = f(BH * N1 * M * V);
    w.lg = f(M > BWD_TABLE_M ? rows * BWD_WIDE_MW : 0);
    w.bytes = off;
    return w;
}

// The backward pass of the chunk op (cyfa_backward.hip): q, k, v and the
// cotangent d_o are bf16 or fp32 (bf16 != 0 selects bf16), every other
// tensor fp32; K, V <= 1024, an even M <= 128.
struct BwdParams {
    int B, T, H, K, V, M, bf16;
    const void *q, *k, *v, *d_o;  // [B, T, H, K | V]; d_o nullable (zero)
    const float *g, *delta, *beta, *table, *q_w, *k_w;
    float q_eps, k_eps, scale;
    const float *h0_k, *h0_v, *clock0;    // nullable
    const float *d_hk, *d_hv, *d_clock;   // nullable cotangents of the final states
    void *dq, *dk, *dv;                   // [B, T, H, K | V] in the operands' dtype
    float *dg, *ddelta, *dbeta;           // [B, T, H]
    float* dtable;                        // [H, M-1, M]
    float* dreadout;                      // nullable [H, M-1, M-1]
    float *dq_w, *dk_w;                   // [K]
    float *dh0_k, *dh0_v, *dclock0;       // nullable
    void* workspace;
};
// The backward pass's workspace (fp32 unless noted, each region 256-byte
// aligned; rows = B*H*Tp head-major, Tp = T rounded up to 64, N = Tp / 64):
// the recomputed forward (normalised rows and their norm factors, clock,
// write vector and phases, pass-1 output, slot weights, the states before
// every chunk of both passes) and the adjoints (cotangent rows, the state
// cotangents before every chunk, the rows' cotangents of both passes, the
// per-chunk boundary terms of the gate cotangent, per-block partial sums of
// the table and norm-weight cotangents).
struct BwdWorkspace {
    double* lam;
    float *qh, *kh, *rq, *rk, *vh, *w, *cs, *sn, *raw, *wts, *sk, *sv;
    float *dO, *dsk, *dsv, *dwts, *dw2, *dvh, *draw, *dlam, *dqh, *dkh, *dw1, *bnd1, *bnd2, *dtab, *dnq, *dnk;
    float *lg, *dlw, *dlp;  // the wide readout (M > BWD_TABLE_M): logits / p, dp / dl [rows, 256]; clock partials [rows, 4]
    int N, nt1, nt2, ro_blocks, norm_blocks;
    size_t bytes;
};
constexpr int BWD_RO_BLOCK = 32;    // rows per block of the readout kernels
constexpr int BWD_WIDE_SPLIT = 1024;  // token rows per table-cotangent partial of the wide readout
constexpr int BWD_SCAN_ROWS = 32;   // rows of a state-scan tile (its columns: 32)
constexpr int BWD_NORM_ROWS = 64;   // rows per norm-adjoint workgroup

// Blocks of 32 rows per readout workgroup: up to eight (the head's table is
// staged once per workgroup), as long as 512 or more workgroups remain.
inline int bwd_ro_per_wg(int B, int Tp, int H) {
    const int blocks = (B * Tp + BWD_RO_BLOCK - 1) / BWD_RO_BLOCK, per = blocks * H / 512;
    return per < 1 ? 1 : per > 8 ? 8 : per;
}

inline BwdWorkspace bwd_workspace(int B, int T, int H, int K, int V, int M, void* base) {
    const size_t Tp = (size_t)(T + 63) / 64 * 64, rows = (size_t)B * H * Tp, N = Tp / 64;
    char* p = static_cast<char*>(base);
    size_t off = 0;
    const auto take = [&](size_t bytes) {
        char* r = p ? p + off : nullptr;
        off += (bytes + 255) / 256 * 256;
        return r;
    };
    const auto f = [&](size_t n) { return reinterpret_cast<float*>(take(n * 4)); };
    BwdWorkspace w;
    w.N = (int)N;
    w.nt1 = (M + 31) / 32 * ((K + BWD_SCAN_ROWS - 1) / BWD_SCAN_ROWS);  // the state scans' tiles
    w.nt2 = (V + 31) / 32 * ((M + BWD_SCAN_ROWS - 1) / BWD_SCAN_ROWS);
    const bool wide = M > BWD_TABLE_M;
    if (wide) {  // the table cotangent's partials: one per BWD_WIDE_SPLIT token rows of a head
        w.ro_blocks = (int)((B * Tp + BWD_WIDE_SPLIT - 1) / BWD_WIDE_SPLIT);
    } else {
        const int blocks = (int)((B * Tp + BWD_RO_BLOCK - 1) / BWD_RO_BLOCK), per = bwd_ro_per_wg(B, (int)Tp, H);
        w.ro_blocks = (blocks + per - 1) / per;  // readout workgroups per head
    }
    w.norm_blocks = (int)(((size_t)B * T * H + BWD_NORM_ROWS - 1) / BWD_NORM_ROWS);
    const size_t BH = (size_t)B * H;
    w.lam = reinterpret_cast<double*>(take(rows * 8));
    w.qh = f(rows * K);
    w.kh = f(rows * K);
    w.rq = f(rows);
    w.rk = f(rows);
    w.vh = f(rows * V);
    w.w = f(rows * M);
    w.cs = f(rows * (M / 2));
    w.sn = f(rows * (M / 2));
    w.raw = f(rows * M);
    w.wts = f(rows * M);
    w.sk = f(BH * (N + 1) * K * M);
    w.sv = f(BH * (N + 1) * M * V);
    w.dO = f(rows * V);
    w.dsk = f(BH * (N + 1) * K * M);
    w.dsv = f(BH * (N + 1) * M * V);
    w.dwts = f(rows * M);
    w.dw2 = f(rows * M);
    w.dvh = f(rows * V);
    w.draw = f(rows * M);
    w.dlam = f(rows);
    w.dqh = f(rows * K);
    w.dkh = f(rows * K);
    w.dw1 = f(rows * M);
    w.bnd1 = f(BH * w.nt1 * N);
    w.bnd2 = f(BH * w.nt2 * N);
    w.dtab = f((size_t)H * w.ro_blocks * (M - 1) * M);
    w.dnq = f((size_t)w.norm_blocks * K);
    w.dnk = f((size_t)w.norm_blocks * K);
    w.lg = f(wide ? rows * BWD_WIDE_MW : 0);
    w.dlw = f(wide ? rows * BWD_WIDE_MW : 0);
    w.dlp = f(wide ? rows * (BWD_WIDE_MW / 64) : 0);
    w.bytes = off;
    return w;
}

int launch_general_table(const float* readout, float* table, int H, int M, hipStream_t stream);
int launch_general_chunk(const GenChunkParams& p, hipStream_t stream);
int launch_chunk_pass(const ChunkPassParams& p, hipStream_t stream);
// The slot readout of every head-major row (cyfa_backward.hip): z = U(lam) raw,
// p = softmax(table z), weights = U(-lam) table^T p, rounded where the input
// dtype is cast when bf16; split: up to 128 slots, the products as split-bf16
// products on the matrix cores (else fp32 ones); lg: with M > 128 a
// [rows, 256] fp32 workspace.
int launch_chunk_readout(const float* raw, const float* cs, const float* sn, const float* table, float* lg, int B,
                         int Tp, int H, int M, int bf16, int split, float* wts, hipStream_t stream);
// The general path's clock and unrounded fp32 write vector with its phases
// (head-major [B*H, Tp] and [B*H, Tp, M | M/2]), for the backward pass's recompute.
int launch_general_clock_write(const float* delta, const float* clock0, const float* beta, int B, int T, int Tp, int H,
                               int M, double* lam, float* w, float* cs, float* sn, hipStream_t stream);
int launch_chunk_bwd(const BwdParams& p, hipStream_t stream);
int launch_general_decode(const GenDecodeParams& p, int bf16, hipStream_t stream);

int launch_rms_norm(const NormParams& p, hipStream_t stream);
int launch_linear_rows(const LinearParams& p, hipStream_t stream);
int launch_short_conv(const ConvParams& p, hipStream_t stream);
int launch_silu_mul(const __bf16* gu, __bf16* out, int rows, int F, hipStream_t stream);
int launch_argmax_rows(const __bf16* x, long long ldx, int rows, int n, long long* out, hipStream_t stream);
int launch_gate_path(const GatePathParams& p, hipStream_t stream);
int launch_gates(const __bf16* abd, long long abd_row, const float* dt_bias, const float* A_log, float* g, float* beta,
                 float* delta, int rows, int H, hipStream_t stream);

}  // namespace cyfa
