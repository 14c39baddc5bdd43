// cyfa_backward.hip -- the backward pass of the chunkwise CyFA op.
//
// Replaces the autograd adjoints chunk_cyfa (ops/chunk.py:164-353) is built
// from: ScalarAttention.grad / scalar_grad for both ScalarGatedLA passes
// (ops/chunk.py:51-71, ops/chunk_bwd.py:1008-1041: state_backward,
// query_key_adjoint, value_adjoint), the slot-readout adjoint of
// FirstReadout*.grad (ops/chunk_readout.py:13-621, 776-786, 976-988),
// PhaseWrite.grad and ClockScan.grad (ops/utils.py:297-299, 589-641,
// 704-754), HeadRMSNorm.grad (ops/qk_norm.py:241-289) and the gradient of
// table = readout @ Phi (ops/chunk.py:281).
//
// The forward is recomputed in fp32 with no intermediate rounding (the
// general path's kernels, keeping the state before every 64-token chunk of
// both passes), so the gradients are those of the op's exact arithmetic;
// every adjoint accumulates in fp32. Per pass (o = SGLA(q, k, v, g, S0,
// scale), in-chunk cumulative log-decay G):
//   D_n  = e^{G_last} D_{n+1} + scale sum_t e^{G_t} q_t (x) dO_t      (state cotangent, reverse over chunks)
//   dq_t = scale (e^{G_t} S_n dO_t + sum_{s<=t} e^{G_t-G_s} (dO_t.v_s) k_s)
//   dk_s = scale sum_{t>=s} e^{G_t-G_s} (dO_t.v_s) q_t + e^{G_last-G_s} D_{n+1} v_s
//   dv_s = scale sum_{t>=s} e^{G_t-G_s} (q_t.k_s) dO_t + e^{G_last-G_s} D_{n+1}^T k_s
//   dL/dG_t = q_t.dq_t - k_t.dk_t + [t = last] <D_{n+1}, S_{n+1}>,  dg = in-chunk reverse cumsum
// The state cotangents are one sweep per (32-column tile, b, h) that keeps
// its tile of D in LDS; the rows' cotangents are then chunk-parallel, one
// workgroup per (chunk, h, b), with no reduction across workgroups. The
// readout adjoint runs per row (z = U(lam) raw, softmax of table z, u =
// table^T p, weights = U(-lam) u) with the head's table and this
// workgroup's share of the table cotangent on chip; partial sums (table,
// norm weights, per-column-tile boundary terms) are added in a fixed order,
// so the result does not depend on scheduling. fp32 FMA loops over LDS
// tiles, no matrix cores: a first, exact form of the training path.
#include <cmath>

#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

constexpr int BC = 64;           // chunk length of the recompute and the sweeps
constexpr int BW_MAX_D = 1024;   // largest K and V
constexpr int BW_TILE = 32;      // state columns per scan workgroup
constexpr int BW_STAGE = 128;    // columns of a staged row block in the chunk kernel
constexpr double kTwoPiBw = 6.283185307179586;

__device__ __forceinline__ float bw_wave_sum(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

__device__ __forceinline__ float bw_wave_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

template <bool BF>
__device__ __forceinline__ float bw_ld(const void* p, size_t i) {
    if constexpr (BF)
        return (float)reinterpret_cast<const bf16_t*>(p)[i];
    else
        return reinterpret_cast<const float*>(p)[i];
}

template <bool BF>
__device__ __forceinline__ void bw_st(void* p, size_t i, float v) {
    if constexpr (BF)
        reinterpret_cast<bf16_t*>(p)[i] = (bf16_t)v;
    else
        reinterpret_cast<float*>(p)[i] = v;
}

// The in-chunk inclusive cumsum G of the natural-log gate over chunk n of
// (b, h), lane = token (tokens past T add zero); one wave.
__device__ __forceinline__ float chunk_gam(const float* g, int b, int h, int T, int H, int n, int lane) {
    const int t = n * BC + lane;
    float x = t < T ? g[((size_t)b * T + t) * H + h] : 0.f;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    return x;
}

// Rows of x [B, T, H, D] into head-major fp32 [B*H, Tp, D]: with a norm
// weight the normalised row x rs w (ops/qk_norm.py:206-233, unrounded) and rs
// per row; without, x itself; x == nullptr or t >= T gives zeros. One wave per row.
template <bool BF>
__global__ __launch_bounds__(256) void bw_rows_kernel(const void* x, const float* w, float eps, int B, int T, int Tp,
                                                      int H, int D, float* out, float* rs_out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= B * H * Tp) return;
    const int t = row % Tp, bh = row / Tp, b = bh / H, h = bh % H;
    float* dst = out + (size_t)row * D;
    if (!x || t >= T) {
        for (int i = lane; i < D; i += 64) dst[i] = 0.f;
        if (rs_out && lane == 0) rs_out[row] = 0.f;
        return;
    }
    const size_t src = (((size_t)b * T + t) * H + h) * D;
    if (!w) {
        for (int i = lane; i < D; i += 64) dst[i] = bw_ld<BF>(x, src + i);
        return;
    }
    float ss = 0.f;
    for (int i = lane; i < D; i += 64) {
        const float v = bw_ld<BF>(x, src + i);
        ss = fmaf(v, v, ss);
    }
    const float rs = rsqrtf(bw_wave_sum(ss) / (float)D + eps);
    for (int i = lane; i < D; i += 64) dst[i] = bw_ld<BF>(x, src + i) * rs * w[i];
    if (rs_out && lane == 0) rs_out[row] = rs;
}

// State cotangents of one pass: D_N = dS_final (or zero), then for n = N-1 .. 0
// D_n = e^{G_last} D_{n+1} + scale sum_t e^{G_t} q_t (x) dO_t. D_n is kept for
// every n (D_0 is the initial state's cotangent), and bnd[tile][n] = the
// tile's part of <D_{n+1}, S_{n+1}>. Grid (ceil(Vd / 32), H, B), 256 threads;
// the tile's [Kq][32] columns of D stay in LDS.
struct ScanArgs {
    const float* q;         // head-major [B*H, Tp, Kq]
    const float* dO;        // head-major [B*H, Tp, Vd]
    const float* g;         // [B, T, H]
    const float* S;         // [B*H, N+1, Kq, Vd]
    const float* dS_final;  // nullable [B*H, Kq, Vd]
    float* D;               // [B*H, N+1, Kq, Vd]
    float* bnd;             // [B*H, ntile, N]
    float* dS0;             // nullable [B*H, Kq, Vd]
    int B, T, Tp, H, Kq, Vd, N;
    float scale;
};

__global__ __launch_bounds__(256) void bw_scan_kernel(ScanArgs a) {
    __shared__ float sD[BW_MAX_D * BW_TILE];
    __shared__ float sdO[BC][BW_TILE];
    __shared__ float sEq[BC];
    __shared__ float sRed[4];
    __shared__ float sEl;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int tile = blockIdx.x, c0 = tile * BW_TILE, h = blockIdx.y, b = blockIdx.z;
    const int Kq = a.Kq, Vd = a.Vd, N = a.N, nt = gridDim.x;
    const size_t bh = (size_t)b * a.H + h, ssz = (size_t)Kq * Vd;
    const float* S = a.S + bh * (N + 1) * ssz;
    float* D = a.D + bh * (N + 1) * ssz;
    const float* q = a.q + bh * a.Tp * Kq;
    const float* dO = a.dO + bh * a.Tp * Vd;
    for (int e = tid; e < Kq * BW_TILE; e += 256) {
        const int r = e / BW_TILE, c = e % BW_TILE;
        sD[e] = (a.dS_final && c0 + c < Vd) ? a.dS_final[bh * ssz + (size_t)r * Vd + c0 + c] : 0.f;
    }
    for (int n = N - 1; n >= 0; n--) {
        // sD holds D_{n+1}: keep it, and its dot with S_{n+1} over the tile
        float dot = 0.f;
        for (int e = tid; e < Kq * BW_TILE; e += 256) {
            const int r = e / BW_TILE, c = e % BW_TILE;
            if (c0 + c < Vd) {
                const size_t at = (size_t)(n + 1) * ssz + (size_t)r * Vd + c0 + c;
                D[at] = sD[e];
                dot = fmaf(sD[e], S[at], dot);
            }
        }
        dot = bw_wave_sum(dot);
        if (lane == 0) sRed[wv] = dot;
        const int t0 = n * BC;
        for (int e = tid; e < BC * BW_TILE; e += 256) {
            const int t = e / BW_TILE, c = e % BW_TILE;
            sdO[t][c] = c0 + c < Vd ? dO[(size_t)(t0 + t) * Vd + c0 + c] : 0.f;
        }
        if (wv == 0) {
            const float G = chunk_gam(a.g, b, h, a.T, a.H, n, lane);
            sEq[lane] = expf(G);
            if (lane == 63) sEl = expf(G);
        }
        __syncthreads();
        if (tid == 0) a.bnd[(bh * nt + tile) * N + n] = (sRed[0] + sRed[1]) + (sRed[2] + sRed[3]);
        const float el = sEl;
        for (int e = tid; e < Kq * BW_TILE; e += 256) {
            const int r = e / BW_TILE, c = e % BW_TILE;
            float acc = 0.f;
            for (int t = 0; t < BC; t++) acc = fmaf(sEq[t] * q[(size_t)(t0 + t) * Kq + r], sdO[t][c], acc);
            sD[e] = fmaf(el, sD[e], a.scale * acc);
        }
        __syncthreads();
    }
    for (int e = tid; e < Kq * BW_TILE; e += 256) {
        const int r = e / BW_TILE, c = e % BW_TILE;
        if (c0 + c < Vd) {
            D[(size_t)r * Vd + c0 + c] = sD[e];
            if (a.dS0) a.dS0[bh * ssz + (size_t)r * Vd + c0 + c] = sD[e];
        }
    }
}

// Cotangents of one chunk's rows: dq, dk (Kq) and dv (Vd) for its 64 tokens
// from S_n (state before the chunk), D_{n+1} (cotangent after it) and the
// two masked decayed score matrices A (q.k) and B (dO.v). Grid (N, H, B),
// 256 threads. A thread owns one row coordinate (block width 256 / TQ of the
// Kq dims, 256 / TV of the Vd dims) for 64 / T tokens, so every load of S,
// D, k or q feeds as many FMAs as the thread has tokens; the other operand
// is a staged row block read as an LDS broadcast.
struct ChunkGradArgs {
    const float *q, *k, *v, *dO;  // head-major [B*H, Tp, Kq | Vd]
    const float* g;               // [B, T, H]
    const float *S, *D;           // [B*H, N+1, Kq, Vd]
    float *dq, *dk, *dv;          // head-major
    int B, T, Tp, H, Kq, Vd, N;
    float scale;
};

template <int TQ, int TV>
__global__ __launch_bounds__(256) void bw_chunk_kernel(ChunkGradArgs a) {
    __shared__ float sA[BC][BC + 1], sB[BC][BC + 1];
    __shared__ float sX[BC][BW_STAGE];
    __shared__ float sG[BC], sEq[BC], sEl[BC];
    const int tid = threadIdx.x, n = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int Kq = a.Kq, Vd = a.Vd, t0 = n * BC;
    const size_t bh = (size_t)b * a.H + h, ssz = (size_t)Kq * Vd;
    const float* q = a.q + (bh * a.Tp + t0) * Kq;
    const float* k = a.k + (bh * a.Tp + t0) * Kq;
    const float* v = a.v + (bh * a.Tp + t0) * Vd;
    const float* dO = a.dO + (bh * a.Tp + t0) * Vd;
    const float* S = a.S + (bh * (a.N + 1) + n) * ssz;
    const float* D = a.D + (bh * (a.N + 1) + n + 1) * ssz;
    if (tid < 64) sG[tid] = chunk_gam(a.g, b, h, a.T, a.H, n, tid);
    __syncthreads();
    if (tid < 64) {
        sEq[tid] = expf(sG[tid]);
        sEl[tid] = expf(sG[BC - 1] - sG[tid]);
    }
    for (int e = tid; e < BC * BC; e += 256) {
        const int t = e / BC, s = e % BC;
        float x = 0.f, y = 0.f;
        if (s <= t) {
            for (int j = 0; j < Kq; j++) x = fmaf(q[(size_t)t * Kq + j], k[(size_t)s * Kq + j], x);
            for (int j = 0; j < Vd; j++) y = fmaf(dO[(size_t)t * Vd + j], v[(size_t)s * Vd + j], y);
            const float d = expf(sG[t] - sG[s]);
            x *= d;
            y *= d;
        }
        sA[t][s] = x;
        sB[t][s] = y;
    }
    // Stages row block [.][c0, c0 + 128) of a chunk matrix X (row stride ld, width wd) in sX.
    const auto stage = [&](const float* X, int ld, int wd, int c0) {
        __syncthreads();
        for (int e = tid; e < BC * BW_STAGE; e += 256) {
            const int t = e / BW_STAGE, c = e % BW_STAGE;
            sX[t][c] = c0 + c < wd ? X[(size_t)t * ld + c0 + c] : 0.f;
        }
        __syncthreads();
    };
    {
        constexpr int W = 256 / TQ, NT = BC / TQ;
        const int rr = tid % W, tg = tid / W;
        for (int r0 = 0; r0 < Kq; r0 += W) {
            const int r = r0 + rr;
            const bool live = r < Kq;
            float acc[NT];
            // dq: e^{G_t} S_n dO_t, then + sum_s B[t][s] k_s
#pragma unroll
            for (int i = 0; i < NT; i++) acc[i] = 0.f;
            for (int cb = 0; cb < Vd; cb += BW_STAGE) {
                stage(dO, Vd, Vd, cb);
                const int cw = min(BW_STAGE, Vd - cb);
                if (live)
                    for (int c = 0; c < cw; c++) {
                        const float sv = S[(size_t)r * Vd + cb + c];
#pragma unroll
                        for (int i = 0; i < NT; i++) acc[i] = fmaf(sv, sX[tg + TQ * i][c], acc[i]);
                    }
            }
            if (live) {
#pragma unroll
                for (int i = 0; i < NT; i++) acc[i] *= sEq[tg + TQ * i];
                for (int s = 0; s < BC; s++) {
                    const float kv = k[(size_t)s * Kq + r];
#pragma unroll
                    for (int i = 0; i < NT; i++) acc[i] = fmaf(sB[tg + TQ * i][s], kv, acc[i]);
                }
#pragma unroll
                for (int i = 0; i < NT; i++)
                    a.dq[(bh * a.Tp + t0 + tg + TQ * i) * Kq + r] = a.scale * acc[i];
            }
            // dk: e^{G_last - G_s} D_{n+1} v_s, then + scale sum_t B[t][s] q_t
#pragma unroll
            for (int i = 0; i < NT; i++) acc[i] = 0.f;
            for (int cb = 0; cb < Vd; cb += BW_STAGE) {
                stage(v, Vd, Vd, cb);
                const int cw = min(BW_STAGE, Vd - cb);
                if (live)
                    for (int c = 0; c < cw; c++) {
                        const float dv = D[(size_t)r * Vd + cb + c];
#pragma unroll
                        for (int i = 0; i < NT; i++) acc[i] = fmaf(dv, sX[tg + TQ * i][c], acc[i]);
                    }
            }
            if (live) {
#pragma unroll
                for (int i = 0; i < NT; i++) acc[i] *= sEl[tg + TQ * i];
                for (int t = 0; t < BC; t++) {
                    const float qv = a.scale * q[(size_t)t * Kq + r];
#pragma unroll
                    for (int i = 0; i < NT; i++) acc[i] = fmaf(sB[t][tg + TQ * i], qv, acc[i]);
                }
#pragma unroll
                for (int i = 0; i < NT; i++) a.dk[(bh * a.Tp + t0 + tg + TQ * i) * Kq + r] = acc[i];
            }
        }
    }
    {
        constexpr int W = 256 / TV, NT = BC / TV;
        const int cc = tid % W, tg = tid / W;
        for (int c0 = 0; c0 < Vd; c0 += W) {
            const int c = c0 + cc;
            const bool live = c < Vd;
            // dv: e^{G_last - G_s} D_{n+1}^T k_s, then + scale sum_t A[t][s] dO_t
            float acc[NT];
#pragma unroll
            for (int i = 0; i < NT; i++) acc[i] = 0.f;
            for (int rb = 0; rb < Kq; rb += BW_STAGE) {
                stage(k, Kq, Kq, rb);
                const int rw = min(BW_STAGE, Kq - rb);
                if (live)
                    for (int r = 0; r < rw; r++) {
                        const float dv = D[(size_t)(rb + r) * Vd + c];
#pragma unroll
                        for (int i = 0; i < NT; i++) acc[i] = fmaf(dv, sX[tg + TV * i][r], acc[i]);
                    }
            }
            if (live) {
#pragma unroll
                for (int i = 0; i < NT; i++) acc[i] *= sEl[tg + TV * i];
                for (int t = 0; t < BC; t++) {
                    const float ov = a.scale * dO[(size_t)t * Vd + c];
#pragma unroll
                    for (int i = 0; i < NT; i++) acc[i] = fmaf(sA[t][tg + TV * i], ov, acc[i]);
                }
#pragma unroll
                for (int i = 0; i < NT; i++) a.dv[(bh * a.Tp + t0 + tg + TV * i) * Vd + c] = acc[i];
            }
        }
    }
}

// The slot-readout adjoint, per row of one head (z = U(lam) raw, l = table z,
// p = softmax(l), u = table^T p, weights = U(-lam) u):
//   du = U(lam) dweights, dp = table du, dl = p (dp - p.dp), dz = table^T dl,
//   draw = U(-lam) dz, dtable += p du^T + dl z^T, and the clock's share
//   dlam = sum_p kappa_p [dz . dU(lam)/dlam raw + dweights . dU(-lam)/dlam u]
// with kappa_p = 2 pi p / (M - 1). Grid (row blocks, H), 256 threads; the
// head's table (rows padded by one float against bank conflicts) and this
// block's part of dtable (thread e owns entries e + 256 i) stay on chip.
struct ReadoutGradArgs {
    const float *raw, *cs, *sn, *table, *dwts;  // head-major rows; table [H, M-1, M]
    float *draw, *dlam, *dtab;                  // dtab: [H, blocks, (M-1) M]
    int B, Tp, H, M;
};

__global__ __launch_bounds__(256) void bw_readout_kernel(ReadoutGradArgs a) {
    constexpr int NE = ((BWD_MAX_M - 1) * BWD_MAX_M + 255) / 256;
    __shared__ float sTab[(BWD_MAX_M - 1) * (BWD_MAX_M + 1)];
    __shared__ float sz[BWD_MAX_M], sdu[BWD_MAX_M], sp[BWD_MAX_M], sdl[BWD_MAX_M], sdz[BWD_MAX_M], su[BWD_MAX_M];
    __shared__ float sRed[2][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, blk = blockIdx.x, h = blockIdx.y;
    const int M = a.M, R = M - 1, P = M / 2, LD = M + 1, RM = R * M;
    const float* tb = a.table + (size_t)h * RM;
    for (int e = tid; e < RM; e += 256) sTab[(e / M) * LD + e % M] = tb[e];
    float acc[NE];
#pragma unroll
    for (int i = 0; i < NE; i++) acc[i] = 0.f;
    // entry e = tid + 256 i is (r, m); stepping i adds 256 = dr rows and dm columns
    const int dr = 256 / M, dm = 256 % M, r_first = tid / M, m_first = tid % M;
    const float kap = tid < P ? (float)(kTwoPiBw * tid / R) : 0.f;
    const int rows = a.B * a.Tp, rho0 = blk * BWD_RO_ROWS, rho1 = min(rho0 + BWD_RO_ROWS, rows);
    __syncthreads();
    for (int rho = rho0; rho < rho1; rho++) {
        const int b = rho / a.Tp, t = rho % a.Tp;
        const size_t row = ((size_t)b * a.H + h) * a.Tp + t;
        float c = 0.f, s = 0.f, re = 0.f, ro = 0.f, de = 0.f, dd = 0.f;
        if (tid < P) {
            c = a.cs[row * P + tid];
            s = a.sn[row * P + tid];
            re = a.raw[row * M + 2 * tid];
            ro = a.raw[row * M + 2 * tid + 1];
            de = a.dwts[row * M + 2 * tid];
            dd = a.dwts[row * M + 2 * tid + 1];
            sz[2 * tid] = c * re - s * ro;
            sz[2 * tid + 1] = s * re + c * ro;
            sdu[2 * tid] = c * de - s * dd;
            sdu[2 * tid + 1] = s * de + c * dd;
        }
        __syncthreads();
        float l = -INFINITY, dp = 0.f;
        if (tid < R) {
            float x = 0.f, y = 0.f;
            for (int m = 0; m < M; m++) {
                const float tv = sTab[tid * LD + m];
                x = fmaf(tv, sz[m], x);
                y = fmaf(tv, sdu[m], y);
            }
            l = x;
            dp = y;
        }
        const float wmx = bw_wave_max(l);
        if (lane == 0) sRed[0][wv] = wmx;
        __syncthreads();
        const float mx = fmaxf(fmaxf(sRed[0][0], sRed[0][1]), fmaxf(sRed[0][2], sRed[0][3]));
        const float ex = tid < R ? expf(l - mx) : 0.f;
        const float wse = bw_wave_sum(ex);
        if (lane == 0) sRed[1][wv] = wse;
        __syncthreads();
        const float pr = ex / ((sRed[1][0] + sRed[1][1]) + (sRed[1][2] + sRed[1][3]));
        const float wpd = bw_wave_sum(pr * dp);
        __syncthreads();  // sRed[0] read by every thread
        if (lane == 0) sRed[0][wv] = wpd;
        __syncthreads();
        const float pdp = (sRed[0][0] + sRed[0][1]) + (sRed[0][2] + sRed[0][3]);
        if (tid < M) {
            sp[tid] = tid < R ? pr : 0.f;
            sdl[tid] = tid < R ? pr * (dp - pdp) : 0.f;
        }
        __syncthreads();
        if (tid < M) {
            float x = 0.f, y = 0.f;
            for (int r = 0; r < R; r++) {
                const float tv = sTab[r * LD + tid];
                x = fmaf(tv, sdl[r], x);
                y = fmaf(tv, sp[r], y);
            }
            sdz[tid] = x;
            su[tid] = y;
        }
        __syncthreads();
        float dl = 0.f;
        if (tid < P) {
            const float ze = sdz[2 * tid], zo = sdz[2 * tid + 1], ue = su[2 * tid], uo = su[2 * tid + 1];
            a.draw[row * M + 2 * tid] = c * ze + s * zo;
            a.draw[row * M + 2 * tid + 1] = -s * ze + c * zo;
            dl = kap * (ze * (-s * re - c * ro) + zo * (c * re - s * ro) + de * (-s * ue + c * uo) +
                        dd * (-c * ue - s * uo));
        }
        if (wv == 0) {  // P <= 64: the pairs are all in wave 0
            dl = bw_wave_sum(dl);
            if (lane == 0) a.dlam[row] = dl;
        }
        int r = r_first, m = m_first;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            if (r < R) acc[i] = fmaf(sp[r], sdu[m], fmaf(sdl[r], sz[m], acc[i]));
            r += dr;
            m += dm;
            if (m >= M) {
                m -= M;
                r++;
            }
        }
        __syncthreads();  // the row's vectors are replaced next
    }
    float* dst = a.dtab + ((size_t)h * gridDim.x + blk) * RM;
#pragma unroll
    for (int i = 0; i < NE; i++)
        if (tid + 256 * i < RM) dst[tid + 256 * i] = acc[i];
}

// Per token of a chunk (lane = token): the gate cotangent of both passes
// (dL/dG_t = q.dq - k.dk, plus <D_{n+1}, S_{n+1}> at the chunk's last token,
// then the in-chunk reverse cumsum), and the write vector's (w = beta a(lam),
// a[2p] = s_p cos theta_p, a[2p+1] = -s_p sin theta_p, dw = the pass-1 value
// cotangent + the pass-2 key cotangent): dbeta = dw . a, and dlam = beta
// dw . da/dlam + the readout's share. Grid (N, B*H), 64 threads.
struct TokenGradArgs {
    const float *qh, *kh, *dqh, *dkh;    // pass 1 rows [.., K]
    const float *wts, *w, *dwts, *dw2;   // pass 2 query and key rows [.., M]
    const float* dw1;                    // pass-1 value cotangent [.., M]
    const float *cs, *sn;                // [.., M/2]
    const float *bnd1, *bnd2;            // [B*H, nt, N]
    const float* beta;                   // [B, T, H]
    float* dlam;                         // [B*H, Tp]: in, the readout's share; out, the total
    float *dg, *dbeta;                   // [B, T, H]
    int B, T, Tp, H, K, M, N, nt1, nt2;
};

__global__ __launch_bounds__(64) void bw_token_kernel(TokenGradArgs a) {
    const int lane = threadIdx.x, n = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int t = n * BC + lane, K = a.K, M = a.M, P = M / 2, R = M - 1;
    const size_t row = (size_t)bh * a.Tp + t;
    float dG = 0.f;
    for (int j = 0; j < K; j++)
        dG += a.qh[row * K + j] * a.dqh[row * K + j] - a.kh[row * K + j] * a.dkh[row * K + j];
    for (int j = 0; j < M; j++)
        dG += a.wts[row * M + j] * a.dwts[row * M + j] - a.w[row * M + j] * a.dw2[row * M + j];
    if (lane == BC - 1) {
        for (int i = 0; i < a.nt1; i++) dG += a.bnd1[((size_t)bh * a.nt1 + i) * a.N + n];
        for (int i = 0; i < a.nt2; i++) dG += a.bnd2[((size_t)bh * a.nt2 + i) * a.N + n];
    }
    float x = dG;
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_down(x, o);
        if (lane + o < 64) x += y;
    }
    float db = 0.f, dl = 0.f;
    for (int p = 0; p < P; p++) {
        const float c = a.cs[row * P + p], s = a.sn[row * P + p];
        const float we = a.dw1[row * M + 2 * p] + a.dw2[row * M + 2 * p];
        const float wo = a.dw1[row * M + 2 * p + 1] + a.dw2[row * M + 2 * p + 1];
        const float sp = (float)sqrt((p == 0 ? 1.0 : 2.0) / R);
        db = fmaf(sp, we * c - wo * s, db);
        dl = fmaf(sp * (float)(kTwoPiBw * p / R), -we * s - wo * c, dl);
    }
    const float bt = t < a.T ? a.beta[((size_t)b * a.T + t) * a.H + h] : 0.f;
    a.dlam[row] = fmaf(bt, dl, a.dlam[row]);
    if (t < a.T) {
        a.dg[((size_t)b * a.T + t) * a.H + h] = x;
        a.dbeta[((size_t)b * a.T + t) * a.H + h] = db;
    }
}

// ddelta_s = sum_{t >= s} dlam_t + dclock (lam_t = clock0 + sum_{s <= t}
// delta_s; the final clock is clock0 + sum delta), dclock0 = sum_t dlam_t +
// dclock, in double. One wave per (b, h): each lane sums a run of tokens, the
// runs' suffix sums cross the lanes.
__global__ __launch_bounds__(64) void bw_clock_kernel(const float* dlam, const float* d_clock, int B, int T, int Tp,
                                                      int H, float* ddelta, float* dclock0) {
    const int bh = blockIdx.x, b = bh / H, h = bh % H, lane = threadIdx.x;
    const int per = (Tp + 63) / 64, t0 = lane * per, t1 = min(t0 + per, Tp);
    double s = 0.0;
    for (int t = t0; t < t1; t++) s += (double)dlam[(size_t)bh * Tp + t];
    double suf = s;  // sum over this lane's run and every later lane's
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_down(suf, o);
        if (lane + o < 64) suf += y;
    }
    const double extra = d_clock ? (double)d_clock[bh] : 0.0;
    double run = suf - s + extra;  // the later lanes' sum
    for (int t = t1 - 1; t >= t0; t--) {
        run += (double)dlam[(size_t)bh * Tp + t];
        if (t < T) ddelta[((size_t)b * T + t) * H + h] = (float)run;
    }
    if (dclock0 && lane == 0) dclock0[bh] = (float)(suf + extra);
}

// RMS-norm adjoint of rows x [B, T, H, D] (x_hat = x rs w, rs = (mean x^2 +
// eps)^-1/2): dx = rs w dx_hat - rs^3 / D (sum_i x_i w_i dx_hat_i) x, and
// per block the partial dw = sum_rows dx_hat x rs. A workgroup takes 64 rows
// (16 per wave, in order), lanes own coordinates j = lane + 64 jj.
template <bool BF>
__global__ __launch_bounds__(256) void bw_norm_kernel(const void* x, const float* w, const float* rs,
                                                      const float* dxh, int B, int T, int Tp, int H, int D, void* dx,
                                                      float* dw_part) {
    constexpr int NJ = BW_MAX_D / 64;
    __shared__ float sdw[4][BW_MAX_D];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63, blk = blockIdx.x;
    const int total = B * T * H;
    float dwa[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) dwa[jj] = 0.f;
    for (int i = 0; i < BWD_NORM_ROWS / 4; i++) {
        const int row = blk * BWD_NORM_ROWS + wv * (BWD_NORM_ROWS / 4) + i;
        if (row >= total) break;
        const int h = row % H, t = (row / H) % T, b = row / (H * T);
        const size_t hm = ((size_t)b * H + h) * Tp + t;
        const float r = rs[hm];
        float sum = 0.f;
#pragma unroll
        for (int jj = 0; jj < NJ; jj++) {
            const int j = lane + 64 * jj;
            if (j < D) {
                const float xv = bw_ld<BF>(x, (size_t)row * D + j), dv = dxh[hm * D + j];
                sum = fmaf(xv * w[j], dv, sum);
                dwa[jj] = fmaf(dv * xv, r, dwa[jj]);
            }
        }
        const float cr = r * r * r * bw_wave_sum(sum) / (float)D;
#pragma unroll
        for (int jj = 0; jj < NJ; jj++) {
            const int j = lane + 64 * jj;
            if (j < D) {
                const float xv = bw_ld<BF>(x, (size_t)row * D + j);
                bw_st<BF>(dx, (size_t)row * D + j, r * w[j] * dxh[hm * D + j] - cr * xv);
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < NJ; jj++)
        if (lane + 64 * jj < D) sdw[wv][lane + 64 * jj] = dwa[jj];
    __syncthreads();
    for (int j = threadIdx.x; j < D; j += 256)
        dw_part[(size_t)blk * D + j] = (sdw[0][j] + sdw[1][j]) + (sdw[2][j] + sdw[3][j]);
}

// out[i] = sum_b part[b][i] for b in order (n columns, nb partial rows).
__global__ __launch_bounds__(256) void bw_reduce_kernel(const float* part, int nb, size_t n, float* out) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    for (int b = 0; b < nb; b++) s += part[(size_t)b * n + i];
    out[i] = s;
}

// The table cotangent: per head, sum the readout blocks' partials in order.
__global__ __launch_bounds__(256) void bw_table_reduce_kernel(const float* part, int nb, int RM, float* out) {
    const int h = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
    if (e >= RM) return;
    const float* p = part + (size_t)h * nb * RM + e;
    float s = 0.f;
    for (int b = 0; b < nb; b++) s += p[(size_t)b * RM];
    out[(size_t)h * RM + e] = s;
}

// dreadout[h][r][j] = sum_m dtable[h][r][m] Phi[j][m] (table = readout Phi,
// ops/chunk.py:82-103, 281); Phi's angle 2 pi ((pair j) mod R) / R is reduced
// exactly in integers. One block per (h, r), thread j.
__global__ __launch_bounds__(256) void bw_dreadout_kernel(const float* dtable, int M, float* dreadout) {
    const int R = M - 1, hr = blockIdx.x, j = threadIdx.x;
    __shared__ float row[BWD_MAX_M];
    if (j < M) row[j] = dtable[(size_t)hr * M + j];
    __syncthreads();
    if (j >= R) return;
    float acc = 0.f;
    for (int m = 0; m < M; m++) {
        if (m == 1) continue;
        const int pair = m >> 1;
        const float sc = (float)sqrt((pair == 0 ? 1.0 : 2.0) / R);
        float sn, cs;
        sincosf((float)((double)((pair * j) % R) * (kTwoPiBw / R)), &sn, &cs);
        acc = fmaf(row[m], sc * ((m & 1) ? sn : cs), acc);
    }
    dreadout[(size_t)hr * R + j] = acc;
}

// Head-major fp32 [B*H, Tp, D] rows into [B, T, H, D] in the operands' dtype.
template <bool BF>
__global__ __launch_bounds__(256) void bw_pack_kernel(const float* src, int B, int T, int Tp, int H, int D, void* dst) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, n = (size_t)B * T * H * D;
    if (i >= n) return;
    const int j = (int)(i % D);
    const size_t row = i / D;
    const int h = (int)(row % H), t = (int)((row / H) % T), b = (int)(row / ((size_t)H * T));
    bw_st<BF>(dst, i, src[(((size_t)b * H + h) * Tp + t) * D + j]);
}

int token_groups(int width) { return width > 128 ? 1 : width > 64 ? 2 : 4; }

template <int TQ>
void launch_chunk_grad_tv(const ChunkGradArgs& a, int tv, dim3 grid, hipStream_t stream) {
    if (tv == 1)
        hipLaunchKernelGGL((bw_chunk_kernel<TQ, 1>), grid, dim3(256), 0, stream, a);
    else if (tv == 2)
        hipLaunchKernelGGL((bw_chunk_kernel<TQ, 2>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((bw_chunk_kernel<TQ, 4>), grid, dim3(256), 0, stream, a);
}

void launch_chunk_grad(const ChunkGradArgs& a, hipStream_t stream) {
    const dim3 grid(a.N, a.H, a.B);
    const int tq = token_groups(a.Kq), tv = token_groups(a.Vd);
    if (tq == 1)
        launch_chunk_grad_tv<1>(a, tv, grid, stream);
    else if (tq == 2)
        launch_chunk_grad_tv<2>(a, tv, grid, stream);
    else
        launch_chunk_grad_tv<4>(a, tv, grid, stream);
}

}  // namespace

int launch_chunk_bwd(const BwdParams& p, hipStream_t stream) {
    const int B = p.B, T = p.T, H = p.H, K = p.K, V = p.V, M = p.M;
    if (B < 1 || T < 1 || H < 1 || K < 1 || K > BW_MAX_D || V < 1 || V > BW_MAX_D || M < 4 || M > BWD_MAX_M || M % 2)
        return -1;
    const int Tp = (T + BC - 1) / BC * BC;
    const BwdWorkspace ws = bwd_workspace(B, T, H, K, V, M, p.workspace);
    const int N = ws.N;
    const size_t rows = (size_t)B * H * Tp;
    const dim3 blk(256), rb((unsigned)((rows + 3) / 4));
    const bool bf = p.bf16 != 0;
    // the normalised rows, v and the output cotangent, head-major fp32
#define CYFA_BW_ROWS(BFV)                                                                                           \
    hipLaunchKernelGGL(bw_rows_kernel<BFV>, rb, blk, 0, stream, p.q, p.q_w, p.q_eps, B, T, Tp, H, K, ws.qh, ws.rq); \
    hipLaunchKernelGGL(bw_rows_kernel<BFV>, rb, blk, 0, stream, p.k, p.k_w, p.k_eps, B, T, Tp, H, K, ws.kh, ws.rk); \
    hipLaunchKernelGGL(bw_rows_kernel<BFV>, rb, blk, 0, stream, p.v, (const float*)nullptr, 0.f, B, T, Tp, H, V,   \
                       ws.vh, (float*)nullptr);                                                                    \
    hipLaunchKernelGGL(bw_rows_kernel<BFV>, rb, blk, 0, stream, p.d_o, (const float*)nullptr, 0.f, B, T, Tp, H, V, \
                       ws.dO, (float*)nullptr);
    if (bf) {
        CYFA_BW_ROWS(true)
    } else {
        CYFA_BW_ROWS(false)
    }
#undef CYFA_BW_ROWS
    // the forward, recomputed in fp32, keeping the states before every chunk
    GenRecomputeParams r{};
    r.B = B;
    r.T = T;
    r.Tp = Tp;
    r.H = H;
    r.K = K;
    r.V = V;
    r.M = M;
    r.qh = ws.qh;
    r.kh = ws.kh;
    r.vh = ws.vh;
    r.g = p.g;
    r.delta = p.delta;
    r.beta = p.beta;
    r.table = p.table;
    r.clock0 = p.clock0;
    r.h0_k = p.h0_k;
    r.h0_v = p.h0_v;
    r.scale = p.scale;
    r.lam = ws.lam;
    r.w = ws.w;
    r.cs = ws.cs;
    r.sn = ws.sn;
    r.raw = ws.raw;
    r.wts = ws.wts;
    r.sk = ws.sk;
    r.sv = ws.sv;
    r.o = ws.dvh;  // overwritten by the pass-2 value cotangent below
    if (launch_general_recompute(r, stream) != 0) return -1;
    // pass 2: state cotangents, then the rows' (slot weights, write vector, v)
    ScanArgs s2{};
    s2.q = ws.wts;
    s2.dO = ws.dO;
    s2.g = p.g;
    s2.S = ws.sv;
    s2.dS_final = p.d_hv;
    s2.D = ws.dsv;
    s2.bnd = ws.bnd2;
    s2.dS0 = p.dh0_v;
    s2.B = B;
    s2.T = T;
    s2.Tp = Tp;
    s2.H = H;
    s2.Kq = M;
    s2.Vd = V;
    s2.N = N;
    s2.scale = 1.f;
    hipLaunchKernelGGL(bw_scan_kernel, dim3(ws.nt2, H, B), blk, 0, stream, s2);
    ChunkGradArgs c2{};
    c2.q = ws.wts;
    c2.k = ws.w;
    c2.v = ws.vh;
    c2.dO = ws.dO;
    c2.g = p.g;
    c2.S = ws.sv;
    c2.D = ws.dsv;
    c2.dq = ws.dwts;
    c2.dk = ws.dw2;
    c2.dv = ws.dvh;
    c2.B = B;
    c2.T = T;
    c2.Tp = Tp;
    c2.H = H;
    c2.Kq = M;
    c2.Vd = V;
    c2.N = N;
    c2.scale = 1.f;
    launch_chunk_grad(c2, stream);
    // the readout: the pass-1 output's cotangent, the clock's share and the table's
    ReadoutGradArgs ro{};
    ro.raw = ws.raw;
    ro.cs = ws.cs;
    ro.sn = ws.sn;
    ro.table = p.table;
    ro.dwts = ws.dwts;
    ro.draw = ws.draw;
    ro.dlam = ws.dlam;
    ro.dtab = ws.dtab;
    ro.B = B;
    ro.Tp = Tp;
    ro.H = H;
    ro.M = M;
    hipLaunchKernelGGL(bw_readout_kernel, dim3(ws.ro_blocks, H), blk, 0, stream, ro);
    // pass 1, with the pass-1 output's cotangent as dO
    ScanArgs s1 = s2;
    s1.q = ws.qh;
    s1.dO = ws.draw;
    s1.S = ws.sk;
    s1.dS_final = p.d_hk;
    s1.D = ws.dsk;
    s1.bnd = ws.bnd1;
    s1.dS0 = p.dh0_k;
    s1.Kq = K;
    s1.Vd = M;
    s1.scale = p.scale;
    hipLaunchKernelGGL(bw_scan_kernel, dim3(ws.nt1, H, B), blk, 0, stream, s1);
    ChunkGradArgs c1 = c2;
    c1.q = ws.qh;
    c1.k = ws.kh;
    c1.v = ws.w;
    c1.dO = ws.draw;
    c1.S = ws.sk;
    c1.D = ws.dsk;
    c1.dq = ws.dqh;
    c1.dk = ws.dkh;
    c1.dv = ws.dw1;
    c1.Kq = K;
    c1.Vd = M;
    c1.scale = p.scale;
    launch_chunk_grad(c1, stream);
    // gates, write vector and clock
    TokenGradArgs tg{};
    tg.qh = ws.qh;
    tg.kh = ws.kh;
    tg.dqh = ws.dqh;
    tg.dkh = ws.dkh;
    tg.wts = ws.wts;
    tg.w = ws.w;
    tg.dwts = ws.dwts;
    tg.dw2 = ws.dw2;
    tg.dw1 = ws.dw1;
    tg.cs = ws.cs;
    tg.sn = ws.sn;
    tg.bnd1 = ws.bnd1;
    tg.bnd2 = ws.bnd2;
    tg.beta = p.beta;
    tg.dlam = ws.dlam;
    tg.dg = p.dg;
    tg.dbeta = p.dbeta;
    tg.B = B;
    tg.T = T;
    tg.Tp = Tp;
    tg.H = H;
    tg.K = K;
    tg.M = M;
    tg.N = N;
    tg.nt1 = ws.nt1;
    tg.nt2 = ws.nt2;
    hipLaunchKernelGGL(bw_token_kernel, dim3(N, B * H), dim3(64), 0, stream, tg);
    hipLaunchKernelGGL(bw_clock_kernel, dim3(B * H), dim3(64), 0, stream, ws.dlam, p.d_clock, B, T, Tp, H, p.ddelta,
                       p.dclock0);
    // the q/k norms, their weights, v's layout
    const dim3 nb(ws.norm_blocks);
    if (bf) {
        hipLaunchKernelGGL(bw_norm_kernel<true>, nb, blk, 0, stream, p.q, p.q_w, ws.rq, ws.dqh, B, T, Tp, H, K, p.dq,
                           ws.dnq);
        hipLaunchKernelGGL(bw_norm_kernel<true>, nb, blk, 0, stream, p.k, p.k_w, ws.rk, ws.dkh, B, T, Tp, H, K, p.dk,
                           ws.dnk);
    } else {
        hipLaunchKernelGGL(bw_norm_kernel<false>, nb, blk, 0, stream, p.q, p.q_w, ws.rq, ws.dqh, B, T, Tp, H, K, p.dq,
                           ws.dnq);
        hipLaunchKernelGGL(bw_norm_kernel<false>, nb, blk, 0, stream, p.k, p.k_w, ws.rk, ws.dkh, B, T, Tp, H, K, p.dk,
                           ws.dnk);
    }
    const dim3 kb((unsigned)((K + 255) / 256));
    hipLaunchKernelGGL(bw_reduce_kernel, kb, blk, 0, stream, ws.dnq, ws.norm_blocks, (size_t)K, p.dq_w);
    hipLaunchKernelGGL(bw_reduce_kernel, kb, blk, 0, stream, ws.dnk, ws.norm_blocks, (size_t)K, p.dk_w);
    const size_t nv = (size_t)B * T * H * V;
    const dim3 vb((unsigned)((nv + 255) / 256));
    if (bf)
        hipLaunchKernelGGL(bw_pack_kernel<true>, vb, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    else
        hipLaunchKernelGGL(bw_pack_kernel<false>, vb, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    const int RM = (M - 1) * M;
    hipLaunchKernelGGL(bw_table_reduce_kernel, dim3((RM + 255) / 256, H), blk, 0, stream, ws.dtab, ws.ro_blocks, RM,
                       p.dtable);
    if (p.dreadout)
        hipLaunchKernelGGL(bw_dreadout_kernel, dim3(H * (M - 1)), blk, 0, stream, p.dtable, M, p.dreadout);
    return 0;
}

}  // namespace cyfa
