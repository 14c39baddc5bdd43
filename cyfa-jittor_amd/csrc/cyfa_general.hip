// cyfa_general.hip -- the general-shape path of the CyFA op: the reference's
// unfused fallback (ops/chunk.py:115-161, 285-331 with ops/utils.py:98-226,
// 779-929), taken for every shape outside the tuned kernels (K = V = 256,
// M = 128, C = 64 in prefill; K, V in {128, 256}, M = 128 in decode), and the
// decode limits of ops/fused_recurrent.py:45-46 (K, V <= 1024, M <= 256).
// No model configuration reaches it, so it is plain code rather than fast
// code: fp32 FMA loops over LDS tiles, no MFMA. q, k, v are bf16 or fp32.
// With bf16 inputs the values are rounded to bf16 where the reference casts
// to the input dtype (q_hat, k_hat, the write vector, the pass-1 output, z,
// the table, p, the slot weights and o); scores, states and decayed values
// stay fp32, as the reference's fp32 path computes them. With fp32 inputs
// nothing is rounded.
#include <cmath>

#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

constexpr double kTwoPi = 6.283185307179586;

template <bool BF>
__device__ __forceinline__ float gen_ld(const void* p, size_t i) {
    if constexpr (BF)
        return (float)reinterpret_cast<const bf16_t*>(p)[i];
    else
        return reinterpret_cast<const float*>(p)[i];
}

template <bool BF>
__device__ __forceinline__ void gen_st(void* p, size_t i, float v) {
    if constexpr (BF)
        reinterpret_cast<bf16_t*>(p)[i] = (bf16_t)v;
    else
        reinterpret_cast<float*>(p)[i] = v;
}

// The cast to the input dtype.
template <bool BF>
__device__ __forceinline__ float gen_rnd(float v) {
    if constexpr (BF)
        return (float)(bf16_t)v;
    else
        return v;
}

__device__ __forceinline__ float gen_wave_sum(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

__device__ __forceinline__ float gen_wave_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

// Cosine and sine of pair p's clock phase: the integer range reduction of
// ops/utils.py:649-661 (wi = floor(lam) mod R; coord = (wi p mod R) +
// frac(lam) p, wrapped into (-R/2, R/2]; theta = 2 pi coord / R), in double.
__device__ __forceinline__ void gen_phase(double lam, int p, int R, float& c, float& s) {
    const double whole = floor(lam);
    const double frac = lam - whole;
    long long wi = (long long)whole % R;
    if (wi < 0) wi += R;
    double coord = (double)((wi * p) % R) + frac * p;
    if (coord > 0.5 * R) coord -= R;
    sincosf((float)(coord * (kTwoPi / R)), &s, &c);
}

// s_p of the write vector and the basis: R^-1/2 for pair 0, (2/R)^1/2 after.
__device__ __forceinline__ float gen_pair_scale(int p, int R) {
    return (float)sqrt((p == 0 ? 1.0 : 2.0) / R);
}

// table[h][r][m] = sum_j readout[h][r][j] Phi[j][m] for any even M (the
// basis of ops/chunk.py:82-103 with the angle 2 pi ((pair j) mod R) / R
// reduced exactly in integers: the R angles' sine and cosine are formed once
// per block in LDS and indexed by k = (pair j) mod R, stepped by pair per j).
// One block per (h, r), one thread per m.
__global__ __launch_bounds__(256) void gen_table_kernel(const float* readout, float* table, int M) {
    const int R = M - 1, hr = blockIdx.x, m = threadIdx.x;
    __shared__ float row[256], cos_k[256], sin_k[256];
    for (int j = m; j < R; j += blockDim.x) {
        row[j] = readout[(size_t)hr * R + j];
        sincosf((float)((double)j * (kTwoPi / R)), &sin_k[j], &cos_k[j]);
    }
    __syncthreads();
    if (m >= M) return;
    float acc = 0.f;
    if (m != 1) {
        const int pair = m >> 1;
        const float sc = gen_pair_scale(pair, R);
        const float* basis = (m & 1) ? sin_k : cos_k;
        int k = 0;  // (pair * j) mod R
        for (int j = 0; j < R; j++) {
            acc = fmaf(row[j], sc * basis[k], acc);
            k += pair;
            k = k >= R ? k - R : k;
        }
    }
    table[(size_t)hr * M + m] = acc;
}

// One (b, t, h) row per wave into head-major fp32 [B, H, Tp, D]: with a norm
// weight, x_hat = x rsqrt(mean x^2 + eps) w cast to the input dtype
// (ops/qk_norm.py:206-233); without, x itself. Rows t >= T are zero.
template <bool BF>
__global__ __launch_bounds__(256) void gen_rows_kernel(const void* x, const float* w, float eps, int B, int T, int Tp,
                                                       int H, int D, float* out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= B * Tp * H) return;
    const int h = row % H, t = (row / H) % Tp, b = row / (H * Tp);
    float* dst = out + (((size_t)b * H + h) * Tp + t) * D;
    if (t >= T) {
        for (int i = lane; i < D; i += 64) dst[i] = 0.f;
        return;
    }
    const size_t src = (((size_t)b * T + t) * H + h) * D;
    if (!w) {
        for (int i = lane; i < D; i += 64) dst[i] = gen_ld<BF>(x, src + i);
        return;
    }
    float ss = 0.f;
    for (int i = lane; i < D; i += 64) {
        const float v = gen_ld<BF>(x, src + i);
        ss = fmaf(v, v, ss);
    }
    ss = gen_wave_sum(ss);
    const float rs = rsqrtf(ss / (float)D + eps);
    for (int i = lane; i < D; i += 64) dst[i] = gen_rnd<BF>(gen_ld<BF>(x, src + i) * rs * w[i]);
}

// The clock lam_t = clock0 + sum_{s <= t} delta_s (ops/utils.py:229-348), in
// double, one wave per (b, h): each lane sums a run of tokens, the runs'
// prefix sums cross the lanes, then each lane writes its run. Padded tokens
// add nothing; the final clock is lam at the last padded token.
__global__ __launch_bounds__(64) void gen_clock_kernel(const float* delta, const float* clock0, int B, int T, int Tp,
                                                       int H, double* lam, float* clock_out) {
    const int bh = blockIdx.x, b = bh / H, h = bh % H, lane = threadIdx.x;
    const int per = (Tp + 63) / 64, t0 = lane * per, t1 = min(t0 + per, Tp);
    const auto dl = [&](int t) { return t < T ? (double)delta[((size_t)b * T + t) * H + h] : 0.0; };
    double s = 0.0;
    for (int t = t0; t < t1; t++) s += dl(t);
    double pre = s;
    for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(pre, o);
        if (lane >= o) pre += y;
    }
    double run = (clock0 ? (double)clock0[bh] : 0.0) + pre - s;
    for (int t = t0; t < t1; t++) {
        run += dl(t);
        lam[(size_t)bh * Tp + t] = run;
    }
    if (clock_out && lane == 63) clock_out[bh] = (float)run;
}

// The write vector w[2p] = beta s_p cos(theta_p), w[2p+1] = -beta s_p
// sin(theta_p) (ops/chunk.py:265-279), cast to the input dtype, and the
// phases' cosines and sines for the readout; one thread per (row, pair).
template <bool BF>
__global__ __launch_bounds__(256) void gen_write_kernel(const double* lam, const float* beta, int B, int T, int Tp,
                                                        int H, int M, float* w, float* cs, float* sn) {
    const int P = M / 2;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)B * H * Tp * P) return;
    const int p = (int)(i % P);
    const size_t row = i / P;
    const int t = (int)(row % Tp), bh = (int)(row / Tp), b = bh / H, h = bh % H;
    float c, s;
    gen_phase(lam[row], p, M - 1, c, s);
    const float bt = t < T ? beta[((size_t)b * T + t) * H + h] : 0.f;
    const float sp = gen_pair_scale(p, M - 1);
    w[row * M + 2 * p] = gen_rnd<BF>(bt * sp * c);
    w[row * M + 2 * p + 1] = gen_rnd<BF>(-bt * sp * s);
    cs[row * P + p] = c;
    sn[row * P + p] = s;
}

constexpr int GEN_MAX_K = 1024;

// The slot readout of one row (ops/utils.py:779-882): z = U(lam) raw cast to
// the input dtype; logits_r = sum_m z_m table[r][m] (r < R, the table cast
// too); p = softmax(logits) cast; u = p table; weights = U(-lam) u cast.
// Runs on one wave; z and p go through LDS region `zs`, `ps` (M floats each).
template <bool BF>
__device__ __forceinline__ void gen_readout_row(const float* raw, const float* cs, const float* sn,
                                                const float* tb, int M, float* zs, float* ps, float* wout, int lane) {
    const int P = M / 2, R = M - 1;
    for (int pr = lane; pr < P; pr += 64) {
        const float c = cs[pr], s = sn[pr], e = raw[2 * pr], o = raw[2 * pr + 1];
        zs[2 * pr] = gen_rnd<BF>(c * e - s * o);
        zs[2 * pr + 1] = gen_rnd<BF>(s * e + c * o);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float lg[4], mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = lane + 64 * j;
        lg[j] = -INFINITY;
        if (r < R) {
            float acc = 0.f;
            for (int m = 0; m < M; m++) acc = fmaf(zs[m], gen_rnd<BF>(tb[(size_t)r * M + m]), acc);
            lg[j] = acc;
            mx = fmaxf(mx, acc);
        }
    }
    mx = gen_wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        lg[j] = lane + 64 * j < R ? expf(lg[j] - mx) : 0.f;
        sum += lg[j];
    }
    sum = gen_wave_sum(sum);
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (lane + 64 * j < R) ps[lane + 64 * j] = gen_rnd<BF>(lg[j] / sum);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int pr = lane; pr < P; pr += 64) {
        float ue = 0.f, uo = 0.f;
        for (int r = 0; r < R; r++) {
            ue = fmaf(ps[r], gen_rnd<BF>(tb[(size_t)r * M + 2 * pr]), ue);
            uo = fmaf(ps[r], gen_rnd<BF>(tb[(size_t)r * M + 2 * pr + 1]), uo);
        }
        const float c = cs[pr], s = sn[pr];
        wout[2 * pr] = gen_rnd<BF>(c * ue + s * uo);
        wout[2 * pr + 1] = gen_rnd<BF>(-s * ue + c * uo);
    }
}

// One column of a state update, row by row: out[r ld] = alpha in[r ld] +
// add(r) for r < rows (in == nullptr: a zero state), and use(r, value) in row
// order. The rows are read in blocks of GEN_ROWS, the next block's loads
// issued before the current block's stores: in and out may be the same
// buffer (an in-place step), so the compiler cannot move a load above an
// earlier store itself, and row-at-a-time code waits a full memory latency
// per row. Every element is read before it is written, by the same thread.
constexpr int GEN_ROWS = 16;

template <class Add, class Use>
__device__ __forceinline__ void gen_state_rows(const float* in, float* out, int ld, int rows, float alpha, Add add,
                                               Use use) {
    float cur[GEN_ROWS], nxt[GEN_ROWS];
    const auto fetch = [&](int r0, float (&dst)[GEN_ROWS]) {
#pragma unroll
        for (int i = 0; i < GEN_ROWS; i++) dst[i] = in && r0 + i < rows ? in[(size_t)(r0 + i) * ld] : 0.f;
    };
    fetch(0, cur);
    for (int r0 = 0; r0 < rows; r0 += GEN_ROWS) {
        if (r0 + GEN_ROWS < rows) fetch(r0 + GEN_ROWS, nxt);
#pragma unroll
        for (int i = 0; i < GEN_ROWS; i++) {
            const int r = r0 + i;
            if (r < rows) {
                const float hv = alpha * cur[i] + add(r);
                out[(size_t)r * ld] = hv;
                use(r, hv);
            }
        }
#pragma unroll
        for (int i = 0; i < GEN_ROWS; i++) cur[i] = nxt[i];
    }
}

// One decode step of any shape (ops/fused_recurrent.py:10-200 with the
// oracle's order): q_hat = cast(q rs w) scale, k_hat = cast(k rs w);
// lam = clock + delta; hk' = e^g hk + k_hat (x) w; raw = hk'^T q_hat;
// readout; hv' = e^g hv + w (x) v; o = cast(hv'^T weights). One workgroup per
// (b, h), 256 threads; the states stream through registers.
template <bool BF>
__global__ __launch_bounds__(256) void gen_decode_kernel(GenDecodeParams p) {
    __shared__ float sq[GEN_MAX_K], sk[GEN_MAX_K], sv[GEN_MAX_K];
    __shared__ float sw[256], scs[128], ssn[128], sraw[256], swt[256], sz[256], spr[256];
    __shared__ float sred[2][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, bh = blockIdx.x, h = bh % p.H;
    const int K = p.K, V = p.V, M = p.M, P = M / 2, R = M - 1;
    const size_t xq = (size_t)bh * K, xv = (size_t)bh * V;
    // the two row norms: sums of squares over the block
    float ssq = 0.f, ssk = 0.f;
    for (int i = tid; i < K; i += 256) {
        const float a = gen_ld<BF>(p.q, xq + i), c = gen_ld<BF>(p.k, xq + i);
        ssq = fmaf(a, a, ssq);
        ssk = fmaf(c, c, ssk);
    }
    ssq = gen_wave_sum(ssq);
    ssk = gen_wave_sum(ssk);
    if (lane == 0) {
        sred[0][wv] = ssq;
        sred[1][wv] = ssk;
    }
    __syncthreads();
    const float tq = (sred[0][0] + sred[0][1]) + (sred[0][2] + sred[0][3]);
    const float tk = (sred[1][0] + sred[1][1]) + (sred[1][2] + sred[1][3]);
    const float rq = rsqrtf(tq / (float)K + p.q_eps), rk = rsqrtf(tk / (float)K + p.k_eps);
    for (int i = tid; i < K; i += 256) {
        sq[i] = gen_rnd<BF>(gen_ld<BF>(p.q, xq + i) * rq * p.q_w[i]) * p.scale;
        sk[i] = gen_rnd<BF>(gen_ld<BF>(p.k, xq + i) * rk * p.k_w[i]);
    }
    for (int i = tid; i < V; i += 256) sv[i] = gen_ld<BF>(p.v, xv + i);
    const double lam = (p.clock_in ? (double)p.clock_in[bh] : 0.0) + (double)p.delta[bh];
    const float alpha = expf(p.g[bh]), beta = p.beta[bh];
    for (int pr = tid; pr < P; pr += 256) {
        float c, s;
        gen_phase(lam, pr, R, c, s);
        scs[pr] = c;
        ssn[pr] = s;
        const float sp = gen_pair_scale(pr, R);
        sw[2 * pr] = gen_rnd<BF>(beta * sp * c);
        sw[2 * pr + 1] = gen_rnd<BF>(-beta * sp * s);
    }
    __syncthreads();
    // hk' and raw: thread m walks the key rows of column m
    for (int m = tid; m < M; m += 256) {
        float acc = 0.f;
        const float wm = sw[m];
        gen_state_rows(p.hk_in ? p.hk_in + (size_t)bh * K * M + m : nullptr, p.hk_out + (size_t)bh * K * M + m, M, K,
                       alpha, [&](int r) { return sk[r] * wm; }, [&](int r, float hv) { acc = fmaf(hv, sq[r], acc); });
        sraw[m] = acc;
    }
    __syncthreads();
    if (wv == 0) gen_readout_row<BF>(sraw, scs, ssn, p.table + (size_t)h * R * M, M, sz, spr, swt, lane);
    __syncthreads();
    // hv' and o: thread j walks the slot rows of value column j
    for (int j = tid; j < V; j += 256) {
        float acc = 0.f;
        const float vj = sv[j];
        gen_state_rows(p.hv_in ? p.hv_in + (size_t)bh * M * V + j : nullptr, p.hv_out + (size_t)bh * M * V + j, V, M,
                       alpha, [&](int m) { return sw[m] * vj; }, [&](int m, float hv) { acc = fmaf(hv, swt[m], acc); });
        gen_st<BF>(p.o, xv + j, acc);
    }
    if (tid == 0) p.clock_out[bh] = (float)lam;
}

}  // namespace

int launch_general_table(const float* readout, float* table, int H, int M, hipStream_t stream) {
    if (M < 4 || M > 256 || M % 2) return -1;
    hipLaunchKernelGGL(gen_table_kernel, dim3(H * (M - 1)), dim3(256), 0, stream, readout, table, M);
    return 0;
}

// The chunk path: rows (q_hat, k_hat, v), the clock, the write vector, then
// pass 1, the readout and pass 2 (ops/chunk.py:136-161, 285-331), each pass
// chunk-parallel (launch_chunk_pass: the states before every chunk by a scan,
// then every chunk's output on tile products), in the workspace laid out by
// general_workspace. bf16 inputs are cast where the reference casts to the
// input dtype (q_hat, k_hat, w, the pass-1 output, the readout's z, table, p
// and weights, o); fp32 inputs are not rounded.
int launch_general_chunk(const GenChunkParams& g, hipStream_t stream) {
    const int B = g.B, T = g.T, H = g.H, K = g.K, V = g.V, M = g.M, C = g.C;
    if (K < 1 || K > GEN_MAX_K || V < 1 || V > GEN_MAX_K || M < 4 || M > 256 || M % 2 ||
        !(C == 16 || C == 32 || C == 64))
        return -1;
    const GenWorkspace ws = general_workspace(B, T, H, K, V, M, g.workspace);
    const int Tp = ws.Tp;
    const size_t rows = (size_t)B * H * Tp;
    const dim3 rb((unsigned)((rows + 3) / 4)), blk(256);
    if (g.bf16) {
        hipLaunchKernelGGL(gen_rows_kernel<true>, rb, blk, 0, stream, g.q, g.q_w, g.q_eps, B, T, Tp, H, K, ws.qh);
        hipLaunchKernelGGL(gen_rows_kernel<true>, rb, blk, 0, stream, g.k, g.k_w, g.k_eps, B, T, Tp, H, K, ws.kh);
        hipLaunchKernelGGL(gen_rows_kernel<true>, rb, blk, 0, stream, g.v, nullptr, 0.f, B, T, Tp, H, V, ws.vh);
    } else {
        hipLaunchKernelGGL(gen_rows_kernel<false>, rb, blk, 0, stream, g.q, g.q_w, g.q_eps, B, T, Tp, H, K, ws.qh);
        hipLaunchKernelGGL(gen_rows_kernel<false>, rb, blk, 0, stream, g.k, g.k_w, g.k_eps, B, T, Tp, H, K, ws.kh);
        hipLaunchKernelGGL(gen_rows_kernel<false>, rb, blk, 0, stream, g.v, nullptr, 0.f, B, T, Tp, H, V, ws.vh);
    }
    hipLaunchKernelGGL(gen_clock_kernel, dim3(B * H), dim3(64), 0, stream, g.delta, g.clock0, B, T, Tp, H, ws.lam,
                       g.clock);
    const size_t pairs = rows * (M / 2);
    const dim3 wb((unsigned)((pairs + 255) / 256));
    if (g.bf16)
        hipLaunchKernelGGL(gen_write_kernel<true>, wb, blk, 0, stream, ws.lam, g.beta, B, T, Tp, H, M, ws.w, ws.cs, ws.sn);
    else
        hipLaunchKernelGGL(gen_write_kernel<false>, wb, blk, 0, stream, ws.lam, g.beta, B, T, Tp, H, M, ws.w, ws.cs, ws.sn);
    // pass 1: raw = sgla(q_hat, k_hat, w), head-major, cast like the input;
    // bf16 inputs take the tile products on the matrix cores (their operands
    // are bf16 values, the states and scores split into two bf16 parts)
    ChunkPassParams p1{};
    p1.q = ws.qh;
    p1.k = ws.kh;
    p1.v = ws.w;
    p1.g = g.g;
    p1.s0 = g.h0_k;
    p1.states = ws.sk;
    p1.s_final = g.hk;
    p1.out = ws.raw;
    p1.bf16 = g.bf16;
    p1.mfma = g.bf16;
    p1.B = B;
    p1.T = T;
    p1.Tp = Tp;
    p1.H = H;
    p1.Kq = K;
    p1.Vd = M;
    p1.scale = g.scale;
    if (launch_chunk_pass(p1, stream) != 0) return -1;
    if (launch_chunk_readout(ws.raw, ws.cs, ws.sn, g.table, ws.lg, B, Tp, H, M, g.bf16, g.bf16, ws.wts, stream) != 0) return -1;
    // pass 2: o = sgla(weights, w, v), written as [B, T, H, V] in the input dtype
    ChunkPassParams p2 = p1;
    p2.q = ws.wts;
    p2.k = ws.w;
    p2.v = ws.vh;
    p2.s0 = g.h0_v;
    p2.states = ws.sv;
    p2.s_final = g.hv;
    p2.out = nullptr;
    p2.out_bthd = g.o;
    p2.Kq = M;
    p2.Vd = V;
    p2.scale = 1.f;
    return launch_chunk_pass(p2, stream);
}

int launch_general_clock_write(const float* delta, const float* clock0, const float* beta, int B, int T, int Tp, int H,
                               int M, double* lam, float* w, float* cs, float* sn, hipStream_t stream) {
    if (M < 4 || M > 256 || M % 2) return -1;
    hipLaunchKernelGGL(gen_clock_kernel, dim3(B * H), dim3(64), 0, stream, delta, clock0, B, T, Tp, H, lam,
                       (float*)nullptr);
    const size_t pairs = (size_t)B * H * Tp * (M / 2);
    hipLaunchKernelGGL(gen_write_kernel<false>, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, stream, lam, beta,
                       B, T, Tp, H, M, w, cs, sn);
    return 0;
}

int launch_general_decode(const GenDecodeParams& p, int bf16, hipStream_t stream) {
    if (p.K < 1 || p.K > GEN_MAX_K || p.V < 1 || p.V > GEN_MAX_K || p.M < 4 || p.M > 256 || p.M % 2) return -1;
    if (bf16)
        hipLaunchKernelGGL(gen_decode_kernel<true>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(gen_decode_kernel<false>, dim3(p.B * p.H), dim3(256), 0, stream, p);
    return 0;
}

}  // namespace cyfa
