// cyfa_prefill.hip -- chunkwise two-pass CyFA prefill for gfx950 (K = V = 256, M = 128).
//
// Pipeline for one call (all kernels on the caller's stream):
//   1. clock_kernel      lam_t = clock0 + sum_{s<=t} delta_s, final clock.
//   2. segment_state     (only when a sequence is split into P > 1 segments)
//                        segment-local end states of both passes from a zero
//                        start, and the product of alpha over each segment.
//   3. carry_kernel      affine carry over segments: S_in[j+1] = a_j S_in[j] + U_j.
//   4. pass1_kernel      per segment, sweep its 64-token chunks with the fp32 key
//                        state [256 x 128] held in registers: raw = scale (2^G q S
//                        + P w), P = mask 2^(G_t-G_s) q k^T; state update
//                        S = 2^G_last S + k^T bf16(2^(G_last-G_s) w); fused slot
//                        readout epilogue -> slot weights (bf16).
//   5. pass2_kernel      the same sweep for the value state [128 x 256] with
//                        query = slot weights, key = w, value = v -> o (bf16).
// All GEMM-shaped work runs on v_mfma_f32_16x16x32_{bf16,f16} with fp32
// accumulation; 64-token chunks are staged in LDS. The sweep keeps each
// segment's state on chip from the first to the last chunk; only segment
// boundary states (one per L chunks) touch HBM.
//
// Lane conventions of the 16x16x32 MFMA (wave64, lane l, lr = l & 15, lg = l >> 4):
//   A[row][k]: row = lr, k = 8 lg + j (j = 0..7)     B[k][col]: col = lr, k = 8 lg + j
//   C[row][col]: col = lr, row = 4 lg + i (i = 0..3)
// A state block pair held as C (rows 32 ks .. 32 ks + 31) is used directly as the
// B operand of the query product by pairing element j < 4 with row 32 ks + 4 lg + j
// and j >= 4 with row 32 ks + 16 + 4 lg + (j - 4); the query fragment is read
// with the same k order.
#include <stdlib.h>

#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

constexpr int KD = 256;             // key / query dim of pass 1
constexpr int VD = 256;             // value dim of pass 2
constexpr int SEG_K = KD * kSlots;  // key-state elements
constexpr int SEG_V = kSlots * VD;  // value-state elements
constexpr int SEG = SEG_K + SEG_V;

constexpr int QS = KD + 8;    // row stride (elements) of a 64 x 256 bf16 tile
constexpr int TS = 64 + 8;    // row stride of a [rows x 64 tokens] bf16 tile
constexpr int ZS = 128 + 8;   // row stride of a 64 x 128 16-bit tile / table
constexpr int RS = 128 + 4;   // row stride of a 64 x 128 fp32 tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ size_t tok_index(const PrefillParams& p, int b, int t, int h) {
    return ((size_t)b * p.T + t) * p.H + h;
}

// Gates of chunk [t0, t0 + 64) into LDS: clock, beta and the in-chunk
// inclusive cumsum of g in log2 units (ops/utils.py:495-520). Wave 0 only.
__device__ __forceinline__ void stage_gates(const PrefillParams& p, int b, int h, int bh, int t0,
                                            float* sLam, float* sBeta, float* sGam) {
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int t = t0 + tid;
        float g = 0.f, be = 0.f;
        if (t < p.T) {
            const size_t i = tok_index(p, b, t, h);
            g = p.g[i];
            be = p.beta[i];
        }
        float x = g;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (tid >= o) x += y;
        }
        sGam[tid] = x * kLog2e;
        sBeta[tid] = be;
        sLam[tid] = p.lam[(size_t)bh * p.Tp + t];
    }
}

// Load row t of a [B, T, H, 256] bf16 tensor in A/B-fragment order (8 k-steps
// of 32) and RMS-normalise it: x_hat = bf16(x rsqrt(mean x^2 + eps) w)
// (ops/qk_norm.py:64-107, 206-233). Rows past T are zero. The four lanes
// sharing lr hold the whole row; their partial sums are combined by shuffles.
__device__ __forceinline__ void load_norm_row(const PrefillParams& p, const bf16_t* x, const float* wn, float eps,
                                              int b, int h, int t, bf16x8 frag[8]) {
    const int lg = (threadIdx.x & 63) >> 4;
    float v[8][8];
    float ss = 0.f;
    const bool valid = t < p.T;
    const bf16_t* row = x + tok_index(p, b, valid ? t : 0, h) * KD;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        if (valid) {
            load_bf16x8(row + 32 * ks + 8 * lg, v[ks]);
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[ks][j] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) ss = fmaf(v[ks][j], v[ks][j], ss);
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const float rs = rsqrtf(ss * (1.f / KD) + eps);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const float4 w0 = *reinterpret_cast<const float4*>(wn + 32 * ks + 8 * lg);
        const float4 w1 = *reinterpret_cast<const float4*>(wn + 32 * ks + 8 * lg + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int j = 0; j < 8; j++) frag[ks][j] = (bf16_t)(v[ks][j] * rs * wv[j]);
    }
}

// Write-vector element w[s][m] (ops/utils.py:664-702), rounded to bf16.
__device__ __forceinline__ bf16_t write_elem(float lam, float beta, int m) {
    float sn, cs;
    const int pair = m >> 1;
    phase_sincos(lam, pair, sn, cs);
    const float a = beta * pair_scale(pair);
    return (bf16_t)((m & 1) ? -a * sn : a * cs);
}

__device__ __forceinline__ bf16x8 cat4(const bf16x4& lo, const bf16x4& hi) {
    bf16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

// Query fragment for the state product, in the k order of a C-block pair.
__device__ __forceinline__ bf16x8 load_query_perm(const bf16_t* row_ks, int lg) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row_ks + 4 * lg);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(row_ks + 16 + 4 * lg);
    return cat4(lo, hi);
}

__device__ __forceinline__ bf16x8 state_as_b(const f32x4& top, const f32x4& bottom) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[i] = (bf16_t)top[i];
        r[4 + i] = (bf16_t)bottom[i];
    }
    return r;
}

// ---------------------------------------------------------------------------
// 1. Clock scan.
__global__ __launch_bounds__(256) void clock_kernel(PrefillParams p) {
    const int bh = blockIdx.x, b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ float s_tot[4];
    double carry = p.clock0 ? (double)p.clock0[bh] : 0.0;
    for (int t0 = 0; t0 < p.Tp; t0 += 1024) {
        float d[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = t0 + 4 * tid + j;
            d[j] = t < p.T ? p.delta[tok_index(p, b, t, h)] : 0.f;
        }
        const float s1 = d[0] + d[1], s2 = s1 + d[2], s3 = s2 + d[3];
        const float pre[4] = {d[0], s1, s2, s3};
        float x = s3;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) s_tot[wave] = x;
        __syncthreads();
        float before = 0.f;
        for (int w = 0; w < wave; w++) before += s_tot[w];
        const float tile = s_tot[0] + s_tot[1] + s_tot[2] + s_tot[3];
        const float excl = before + x - s3;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = t0 + 4 * tid + j;
            if (t < p.Tp) p.lam[(size_t)bh * p.Tp + t] = (float)(carry + (double)(excl + pre[j]));
        }
        carry += (double)tile;
        __syncthreads();
    }
    if (p.clock && tid == 0) p.clock[bh] = (float)carry;
}

// ---------------------------------------------------------------------------
// 2. Segment-local end states (zero start). grid = (B*H*(P-1), 2): y = pass.
constexpr int SEGK_LDS = KD * TS * 2;               // sKt
constexpr int SEGV_LDS = kSlots * TS * 2 + VD * TS * 2;  // sWt + sVt
constexpr int SEG_LDS = (SEGK_LDS > SEGV_LDS ? SEGK_LDS : SEGV_LDS) + 3 * 64 * 4;

__global__ __launch_bounds__(256) void segment_state_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[SEG_LDS];
    const int P1 = p.P - 1;
    const int bh = blockIdx.x / P1, j = blockIdx.x % P1, pass = blockIdx.y;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    float* sLam = reinterpret_cast<float*>(smem + SEG_LDS - 3 * 64 * 4);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    float* out = p.seg + ((size_t)bh * p.P + j) * SEG;
    float logdecay = 0.f;

    if (pass == 0) {
        bf16_t* sKt = reinterpret_cast<bf16_t*>(smem);
        f32x4 acc[16][2];
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++) acc[db][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int n = n0; n < n1; n++) {
            const int t0 = n * 64;
            stage_gates(p, b, h, bh, t0, sLam, sBeta, sGam);
            bf16x8 kf[8];
            load_norm_row(p, p.k, p.k_w, p.k_eps, b, h, t0 + 16 * w + lr, kf);
#pragma unroll
            for (int ks = 0; ks < 8; ks++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++) sKt[(32 * ks + 8 * lg + jj) * TS + 16 * w + lr] = kf[ks][jj];
            __syncthreads();
            const float last = sGam[63];
            logdecay += last;
            bf16x8 wt[2][2];
#pragma unroll
            for (int ss = 0; ss < 2; ss++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) {
                    const int m = 32 * w + 16 * mb + lr;
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) {
                        const int s = 32 * ss + 8 * lg + jj;
                        const float wv = (float)write_elem(sLam[s], sBeta[s], m);
                        wt[ss][mb][jj] = (bf16_t)(wv * exp2f(last - sGam[s]));
                    }
                }
            const float dec = exp2f(last);
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) acc[db][mb] *= dec;
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int ss = 0; ss < 2; ss++) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(sKt + (16 * db + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                    for (int mb = 0; mb < 2; mb++) acc[db][mb] = mfma_bf16(a, wt[ss][mb], acc[db][mb]);
                }
            __syncthreads();
        }
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++) out[(16 * db + 4 * lg + i) * kSlots + 32 * w + 16 * mb + lr] = acc[db][mb][i];
        if (tid == 0) p.seg_decay[bh * p.P + j] = exp2f(logdecay);
    } else {
        bf16_t* sWt = reinterpret_cast<bf16_t*>(smem);
        bf16_t* sVt = sWt + kSlots * TS;
        f32x4 acc[8][4];
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int n = n0; n < n1; n++) {
            const int t0 = n * 64;
            stage_gates(p, b, h, bh, t0, sLam, sBeta, sGam);
            __syncthreads();
            // w^T [128 x 64] for all slots: 4096 pairs / 256 threads.
#pragma unroll 4
            for (int it = 0; it < 16; it++) {
                const int idx = tid + 256 * it, s = idx >> 6, pr = idx & 63;
                float we, wo;
                write_pair(sLam[s], sBeta[s], pr, we, wo);
                sWt[(2 * pr) * TS + s] = (bf16_t)we;
                sWt[(2 * pr + 1) * TS + s] = (bf16_t)wo;
            }
            // v^T for this wave's 64 value columns.
#pragma unroll
            for (int it = 0; it < 8; it++) {
                const int q = lane + 64 * it, s = q >> 3, c8 = (q & 7) * 8;
                const int t = t0 + s;
                bf16x8 vv;
                if (t < p.T) {
                    vv = *reinterpret_cast<const bf16x8*>(p.v + tok_index(p, b, t, h) * VD + 64 * w + c8);
                } else {
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) vv[jj] = (bf16_t)0.f;
                }
#pragma unroll
                for (int jj = 0; jj < 8; jj++) sVt[(64 * w + c8 + jj) * TS + s] = vv[jj];
            }
            __syncthreads();
            const float last = sGam[63];
            const float dec = exp2f(last);
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++) acc[mb][cb] *= dec;
#pragma unroll
            for (int ss = 0; ss < 2; ss++) {
                float f[8];
#pragma unroll
                for (int jj = 0; jj < 8; jj++) f[jj] = exp2f(last - sGam[32 * ss + 8 * lg + jj]);
                bf16x8 vt[4];
#pragma unroll
                for (int cb = 0; cb < 4; cb++) {
                    const bf16x8 raw = *reinterpret_cast<const bf16x8*>(sVt + (64 * w + 16 * cb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) vt[cb][jj] = (bf16_t)((float)raw[jj] * f[jj]);
                }
#pragma unroll
                for (int mb = 0; mb < 8; mb++) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(sWt + (16 * mb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) acc[mb][cb] = mfma_bf16(a, vt[cb], acc[mb][cb]);
                }
            }
            __syncthreads();
        }
        float* outv = out + SEG_K;
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) outv[(16 * mb + 4 * lg + i) * VD + 64 * w + 16 * cb + lr] = acc[mb][cb][i];
    }
}

// ---------------------------------------------------------------------------
// 3. Carry over segments, in place: slot j receives the start state of
// segment j. grid = (B*H, SEG / 1024).
__global__ __launch_bounds__(256) void carry_kernel(PrefillParams p) {
    const int bh = blockIdx.x;
    const int e = (blockIdx.y * 256 + threadIdx.x) * 4;
    float4 S = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e < SEG_K) {
        if (p.h0_k) S = *reinterpret_cast<const float4*>(p.h0_k + (size_t)bh * SEG_K + e);
    } else {
        if (p.h0_v) S = *reinterpret_cast<const float4*>(p.h0_v + (size_t)bh * SEG_V + (e - SEG_K));
    }
    for (int j = 0; j < p.P; j++) {
        float4* slot = reinterpret_cast<float4*>(p.seg + ((size_t)bh * p.P + j) * SEG + e);
        if (j + 1 < p.P) {
            const float4 U = *slot;
            const float a = p.seg_decay[bh * p.P + j];
            *slot = S;
            S.x = fmaf(a, S.x, U.x);
            S.y = fmaf(a, S.y, U.y);
            S.z = fmaf(a, S.z, U.z);
            S.w = fmaf(a, S.w, U.w);
        } else {
            *slot = S;
        }
    }
}

// ---------------------------------------------------------------------------
// 4. Pass 1 (key state) + fused slot readout. grid = B*H*P, 256 threads.
constexpr int P1_Q = 0;                         // bf16 [64][QS] q_hat; later z, then p (f16 [64][ZS])
constexpr int P1_KT = P1_Q + 64 * QS * 2;       // bf16 [256][TS] k_hat^T; later raw f32 [64][RS], then omega staging
constexpr int P1_P = P1_KT + KD * TS * 2;       // bf16 [64][TS] masked scores
constexpr int P1_TAB = P1_P + 64 * TS * 2;      // f16 [128][ZS] table rows r
constexpr int P1_TABT = P1_TAB + 128 * ZS * 2;  // f16 [128][ZS] table^T rows m
constexpr int P1_G = P1_TABT + 128 * ZS * 2;    // f32 [3][64] gates
constexpr int P1_LDS = P1_G + 3 * 64 * 4;
static_assert(64 * RS * 4 <= KD * TS * 2, "raw tile must fit in the k^T tile");
static_assert(64 * ZS * 2 <= 64 * QS * 2, "z/p must fit in the q tile");
static_assert(P1_LDS <= 160 * 1024, "pass-1 LDS exceeds gfx950 LDS");

__global__ __launch_bounds__(256) void pass1_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P1_LDS];
    bf16_t* sQ = reinterpret_cast<bf16_t*>(smem + P1_Q);
    f16_t* sZ = reinterpret_cast<f16_t*>(smem + P1_Q);                       // z, then p
    bf16_t* sOm = reinterpret_cast<bf16_t*>(smem + P1_KT);                   // omega staging (raw is dead by then)
    bf16_t* sKt = reinterpret_cast<bf16_t*>(smem + P1_KT);
    float* sRaw = reinterpret_cast<float*>(smem + P1_KT);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P1_P);
    f16_t* sTab = reinterpret_cast<f16_t*>(smem + P1_TAB);
    f16_t* sTabT = reinterpret_cast<f16_t*>(smem + P1_TABT);
    float* sLam = reinterpret_cast<float*>(smem + P1_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;

    const int bh = blockIdx.x / p.P, j = blockIdx.x % p.P;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);

    // Readout table of head h in fp16, both orientations; row / column 127 zero.
    {
        const float* tb = p.table + (size_t)h * kActive * kSlots;
        for (int idx = tid; idx < 128 * 128; idx += 256) {
            const int r = idx >> 7, m = idx & 127;
            const f16_t v = (f16_t)(r < kActive ? tb[r * kSlots + m] : 0.f);
            sTab[r * ZS + m] = v;
            sTabT[m * ZS + r] = v;
        }
    }

    // Segment start state: acc[db][mb] holds S[16 db + 4 lg + i][32 w + 16 mb + lr].
    f32x4 acc[16][2];
    {
        const float* s0 = p.P > 1 ? p.seg + ((size_t)bh * p.P + j) * SEG
                                  : (p.h0_k ? p.h0_k + (size_t)bh * SEG_K : nullptr);
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[db][mb][i] = s0 ? s0[(16 * db + 4 * lg + i) * kSlots + 32 * w + 16 * mb + lr] : 0.f;
    }

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        stage_gates(p, b, h, bh, t0, sLam, sBeta, sGam);
        // q_hat rows of this wave -> LDS (row-major); k_hat rows -> registers + LDS (transposed).
        {
            bf16x8 qf[8];
            load_norm_row(p, p.q, p.q_w, p.q_eps, b, h, t0 + 16 * w + lr, qf);
#pragma unroll
            for (int ks = 0; ks < 8; ks++)
                *reinterpret_cast<bf16x8*>(sQ + (16 * w + lr) * QS + 32 * ks + 8 * lg) = qf[ks];
        }
        bf16x8 kf[8];
        load_norm_row(p, p.k, p.k_w, p.k_eps, b, h, t0 + 16 * w + lr, kf);
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int jj = 0; jj < 8; jj++) sKt[(32 * ks + 8 * lg + jj) * TS + 16 * w + lr] = kf[ks][jj];
        __syncthreads();

        const float last = sGam[63];
        // Write vector (B operand, this wave's 32 slot columns), raw and decayed.
        bf16x8 wf[2][2], wt[2][2];
#pragma unroll
        for (int ss = 0; ss < 2; ss++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const int m = 32 * w + 16 * mb + lr;
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const int s = 32 * ss + 8 * lg + jj;
                    const bf16_t wb = write_elem(sLam[s], sBeta[s], m);
                    wf[ss][mb][jj] = wb;
                    wt[ss][mb][jj] = (bf16_t)((float)wb * exp2f(last - sGam[s]));
                }
            }

        // Scores for key columns s in [16 w, 16 w + 16), all 64 query rows.
        {
            f32x4 sc[4];
#pragma unroll
            for (int tb = 0; tb < 4; tb++) sc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 8; ks++)
#pragma unroll
                for (int tb = 0; tb < 4; tb++) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(sQ + (16 * tb + lr) * QS + 32 * ks + 8 * lg);
                    sc[tb] = mfma_bf16(a, kf[ks], sc[tb]);
                }
            const int s = 16 * w + lr;
            const float gs = sGam[s];
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * tb + 4 * lg + i;
                    const float v = s <= t ? sc[tb][i] * exp2f(sGam[t] - gs) : 0.f;
                    sP[t * TS + s] = (bf16_t)v;
                }
        }
        __syncthreads();

        // raw = scale (2^G_t q S_n + P w) for this wave's 32 slot columns.
        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++) out[tb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            bf16x8 bs[2];
#pragma unroll
            for (int mb = 0; mb < 2; mb++) bs[mb] = state_as_b(acc[2 * ks][mb], acc[2 * ks + 1][mb]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = load_query_perm(sQ + (16 * tb + lr) * QS + 32 * ks, lg);
#pragma unroll
                for (int mb = 0; mb < 2; mb++) out[tb][mb] = mfma_bf16(a, bs[mb], out[tb][mb]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float f = exp2f(sGam[16 * tb + 4 * lg + i]);
#pragma unroll
                for (int mb = 0; mb < 2; mb++) out[tb][mb][i] *= f;
            }
#pragma unroll
        for (int ss = 0; ss < 2; ss++)
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(sP + (16 * tb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                for (int mb = 0; mb < 2; mb++) out[tb][mb] = mfma_bf16(a, wf[ss][mb], out[tb][mb]);
            }

        // State update: S = 2^G_last S + k_hat^T bf16(2^(G_last - G_s) w).
        {
            const float dec = exp2f(last);
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++) acc[db][mb] *= dec;
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int ss = 0; ss < 2; ss++) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(sKt + (16 * db + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                    for (int mb = 0; mb < 2; mb++) acc[db][mb] = mfma_bf16(a, wt[ss][mb], acc[db][mb]);
                }
        }
        __syncthreads();  // k^T and q tiles are dead from here on

#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    sRaw[(16 * tb + 4 * lg + i) * RS + 32 * w + 16 * mb + lr] = out[tb][mb][i] * p.scale;
        __syncthreads();

        // Readout (ops/chunk_readout.py:797-909): z = U(lam) raw in fp16.
#pragma unroll 4
        for (int it = 0; it < 16; it++) {
            const int idx = tid + 256 * it, t = idx >> 6, pr = idx & 63;
            const float e = sRaw[t * RS + 2 * pr], o = sRaw[t * RS + 2 * pr + 1];
            float sn, cs;
            phase_sincos(sLam[t], pr, sn, cs);
            sZ[t * ZS + 2 * pr] = (f16_t)(cs * e - sn * o);
            sZ[t * ZS + 2 * pr + 1] = (f16_t)(sn * e + cs * o);
        }
        __syncthreads();
        // logits = z table^T for this wave's 16 rows; softmax over the 127 active slots.
        {
            f32x4 lgt[8];
#pragma unroll
            for (int rb = 0; rb < 8; rb++) lgt[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(sZ + (16 * w + lr) * ZS + 32 * ks + 8 * lg);
#pragma unroll
                for (int rb = 0; rb < 8; rb++) {
                    const f16x8 bt = *reinterpret_cast<const f16x8*>(sTab + (16 * rb + lr) * ZS + 32 * ks + 8 * lg);
                    lgt[rb] = mfma_f16(a, bt, lgt[rb]);
                }
            }
            __syncthreads();  // every wave has consumed its z rows before p overwrites them
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float mx = -INFINITY;
#pragma unroll
                for (int rb = 0; rb < 8; rb++)
                    if (16 * rb + lr < kActive) mx = fmaxf(mx, lgt[rb][i]);
                mx = wave_max<16>(mx);
                float e[8], sum = 0.f;
#pragma unroll
                for (int rb = 0; rb < 8; rb++) {
                    e[rb] = 16 * rb + lr < kActive ? __expf(lgt[rb][i] - mx) : 0.f;
                    sum += e[rb];
                }
                sum = wave_sum<16>(sum);
                const float inv = 1.f / sum;
                const int t = 16 * w + 4 * lg + i;
#pragma unroll
                for (int rb = 0; rb < 8; rb++) sZ[t * ZS + 16 * rb + lr] = (f16_t)(e[rb] * inv);
            }
        }
        __syncthreads();
        // u = p table, weights = U(-lam) u -> bf16.
        {
            f32x4 uu[8];
#pragma unroll
            for (int mb = 0; mb < 8; mb++) uu[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int rs = 0; rs < 4; rs++) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(sZ + (16 * w + lr) * ZS + 32 * rs + 8 * lg);
#pragma unroll
                for (int mb = 0; mb < 8; mb++) {
                    const f16x8 bt = *reinterpret_cast<const f16x8*>(sTabT + (16 * mb + lr) * ZS + 32 * rs + 8 * lg);
                    uu[mb] = mfma_f16(a, bt, uu[mb]);
                }
            }
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * w + 4 * lg + i, m = 16 * mb + lr;
                    const float mine = uu[mb][i];
                    const float other = __shfl_xor(mine, 1);
                    float sn, cs;
                    phase_sincos(sLam[t], m >> 1, sn, cs);
                    const float e = (m & 1) ? other : mine, o = (m & 1) ? mine : other;
                    const float om = (m & 1) ? (-sn * e + cs * o) : (cs * e + sn * o);
                    sOm[t * ZS + m] = (bf16_t)om;
                }
        }
        __syncthreads();
        {
            bf16_t* dst = p.omega + ((size_t)bh * p.Tp + t0) * kSlots;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int idx = tid + 256 * it, r = idx >> 4, c8 = (idx & 15) * 8;
                *reinterpret_cast<bf16x8*>(dst + r * kSlots + c8) = *reinterpret_cast<const bf16x8*>(sOm + r * ZS + c8);
            }
        }
        __syncthreads();
    }

    if (j == p.P - 1 && p.hk) {
        float* dst = p.hk + (size_t)bh * SEG_K;
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[(16 * db + 4 * lg + i) * kSlots + 32 * w + 16 * mb + lr] = acc[db][mb][i];
    }
}

// ---------------------------------------------------------------------------
// 5. Pass 2 (value state). grid = B*H*P, 256 threads. Wave w owns value columns
// [64 w, 64 w + 64); acc[mb][cb] holds S[16 mb + 4 lg + i][64 w + 16 cb + lr].
constexpr int P2_OM = 0;                         // bf16 [64][ZS] slot weights (query)
constexpr int P2_WT = P2_OM + 64 * ZS * 2;       // bf16 [128][TS] w^T
constexpr int P2_VT = P2_WT + kSlots * TS * 2;   // bf16 [256][TS] v^T; later o staging [64][QS]
constexpr int P2_P = P2_VT + VD * TS * 2;        // bf16 [64][TS] masked scores
constexpr int P2_G = P2_P + 64 * TS * 2;
constexpr int P2_LDS = P2_G + 3 * 64 * 4;
static_assert(64 * QS * 2 <= VD * TS * 2, "o staging must fit in the v^T tile");

__global__ __launch_bounds__(256) void pass2_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P2_LDS];
    bf16_t* sOmq = reinterpret_cast<bf16_t*>(smem + P2_OM);
    bf16_t* sWt = reinterpret_cast<bf16_t*>(smem + P2_WT);
    bf16_t* sVt = reinterpret_cast<bf16_t*>(smem + P2_VT);
    bf16_t* sO = reinterpret_cast<bf16_t*>(smem + P2_VT);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P2_P);
    float* sLam = reinterpret_cast<float*>(smem + P2_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;

    const int bh = blockIdx.x / p.P, j = blockIdx.x % p.P;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);

    f32x4 acc[8][4];
    {
        const float* s0 = p.P > 1 ? p.seg + ((size_t)bh * p.P + j) * SEG + SEG_K
                                  : (p.h0_v ? p.h0_v + (size_t)bh * SEG_V : nullptr);
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[mb][cb][i] = s0 ? s0[(16 * mb + 4 * lg + i) * VD + 64 * w + 16 * cb + lr] : 0.f;
    }

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        stage_gates(p, b, h, bh, t0, sLam, sBeta, sGam);
        {
            const bf16_t* src = p.omega + ((size_t)bh * p.Tp + t0) * kSlots;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int idx = tid + 256 * it, r = idx >> 4, c8 = (idx & 15) * 8;
                *reinterpret_cast<bf16x8*>(sOmq + r * ZS + c8) = *reinterpret_cast<const bf16x8*>(src + r * kSlots + c8);
            }
        }
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int q = lane + 64 * it, s = q >> 3, c8 = (q & 7) * 8;
            const int t = t0 + s;
            bf16x8 vv;
            if (t < p.T) {
                vv = *reinterpret_cast<const bf16x8*>(p.v + tok_index(p, b, t, h) * VD + 64 * w + c8);
            } else {
#pragma unroll
                for (int jj = 0; jj < 8; jj++) vv[jj] = (bf16_t)0.f;
            }
#pragma unroll
            for (int jj = 0; jj < 8; jj++) sVt[(64 * w + c8 + jj) * TS + s] = vv[jj];
        }
        __syncthreads();
        // Key fragments (the write vector) for key rows s in [16 w, 16 w + 16), and w^T in LDS.
        bf16x8 wq[4];
        {
            const int s = 16 * w + lr;
            const float lam = sLam[s], be = sBeta[s];
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int jj = 0; jj < 8; jj += 2) {
                    const int m = 32 * ks + 8 * lg + jj;
                    float we, wo;
                    write_pair(lam, be, m >> 1, we, wo);
                    wq[ks][jj] = (bf16_t)we;
                    wq[ks][jj + 1] = (bf16_t)wo;
                    sWt[m * TS + s] = wq[ks][jj];
                    sWt[(m + 1) * TS + s] = wq[ks][jj + 1];
                }
        }
        {
            f32x4 sc[4];
#pragma unroll
            for (int tb = 0; tb < 4; tb++) sc[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int tb = 0; tb < 4; tb++) {
                    const bf16x8 a = *reinterpret_cast<const bf16x8*>(sOmq + (16 * tb + lr) * ZS + 32 * ks + 8 * lg);
                    sc[tb] = mfma_bf16(a, wq[ks], sc[tb]);
                }
            const int s = 16 * w + lr;
            const float gs = sGam[s];
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * tb + 4 * lg + i;
                    const float v = s <= t ? sc[tb][i] * exp2f(sGam[t] - gs) : 0.f;
                    sP[t * TS + s] = (bf16_t)v;
                }
        }
        __syncthreads();

        f32x4 out[4][4];
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++) out[tb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            bf16x8 bs[4];
#pragma unroll
            for (int cb = 0; cb < 4; cb++) bs[cb] = state_as_b(acc[2 * ks][cb], acc[2 * ks + 1][cb]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = load_query_perm(sOmq + (16 * tb + lr) * ZS + 32 * ks, lg);
#pragma unroll
                for (int cb = 0; cb < 4; cb++) out[tb][cb] = mfma_bf16(a, bs[cb], out[tb][cb]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float f = exp2f(sGam[16 * tb + 4 * lg + i]);
#pragma unroll
                for (int cb = 0; cb < 4; cb++) out[tb][cb][i] *= f;
            }
        const float last = sGam[63];
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            float f[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++) f[jj] = exp2f(last - sGam[32 * ss + 8 * lg + jj]);
            bf16x8 vb[4], vt[4];
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                vb[cb] = *reinterpret_cast<const bf16x8*>(sVt + (64 * w + 16 * cb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                for (int jj = 0; jj < 8; jj++) vt[cb][jj] = (bf16_t)((float)vb[cb][jj] * f[jj]);
            }
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(sP + (16 * tb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                for (int cb = 0; cb < 4; cb++) out[tb][cb] = mfma_bf16(a, vb[cb], out[tb][cb]);
            }
            if (ss == 0) {
                const float dec = exp2f(last);
#pragma unroll
                for (int mb = 0; mb < 8; mb++)
#pragma unroll
                    for (int cb = 0; cb < 4; cb++) acc[mb][cb] *= dec;
            }
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(sWt + (16 * mb + lr) * TS + 32 * ss + 8 * lg);
#pragma unroll
                for (int cb = 0; cb < 4; cb++) acc[mb][cb] = mfma_bf16(a, vt[cb], acc[mb][cb]);
            }
        }
        __syncthreads();  // v^T is dead; reuse it for the output tile
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    sO[(16 * tb + 4 * lg + i) * QS + 64 * w + 16 * cb + lr] = (bf16_t)out[tb][cb][i];
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int idx = tid + 256 * it, r = idx >> 5, c8 = (idx & 31) * 8;
            const int t = t0 + r;
            if (t < p.T)
                *reinterpret_cast<bf16x8*>(p.o + tok_index(p, b, t, h) * VD + c8) =
                    *reinterpret_cast<const bf16x8*>(sO + r * QS + c8);
        }
        __syncthreads();
    }

    if (j == p.P - 1 && p.hv) {
        float* dst = p.hv + (size_t)bh * SEG_V;
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[(16 * mb + 4 * lg + i) * VD + 64 * w + 16 * cb + lr] = acc[mb][cb][i];
    }
}

// ---------------------------------------------------------------------------
// table[h] = readout[h] @ Phi (ops/chunk.py:82-103, 281). One block per
// (h, r); Phi[j][m] is evaluated on the fly with the exact integer reduction
// (pair * j) mod 127 of its angle.
__global__ __launch_bounds__(128) void readout_table_kernel(const float* readout, float* table) {
    const int hr = blockIdx.x, m = threadIdx.x, pair = m >> 1;
    __shared__ float row[kActive];
    if (m < kActive) row[m] = readout[(size_t)hr * kActive + m];
    __syncthreads();
    float acc = 0.f;
    if (m != 1) {
        const float sc = pair_scale(pair);
        for (int jr = 0; jr < kActive; jr++) {
            float sn, cs;
            sincosf((float)((pair * jr) % kActive) * 0.049473900056532176f, &sn, &cs);
            acc = fmaf(row[jr], sc * ((m & 1) ? sn : cs), acc);
        }
    }
    table[(size_t)hr * kSlots + m] = acc;
}

}  // namespace

void choose_segments(int BH, int N, int* P, int* L) {
    // Aim for about one workgroup per CU (256 CUs) in the sweeps.
    // CYFA_SEGMENT_CHUNKS=<L> fixes the chunks per segment (tests, tuning).
    int target = (256 + BH - 1) / BH;
    if (target < 1) target = 1;
    if (target > N) target = N;
    int l = (N + target - 1) / target;
    if (const char* env = getenv("CYFA_SEGMENT_CHUNKS")) {
        const int forced = atoi(env);
        if (forced > 0) l = forced < N ? forced : N;
    }
    *L = l;
    *P = (N + l - 1) / l;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

WorkspaceLayout workspace_layout(int B, int T, int H, int K, int V) {
    WorkspaceLayout w{};
    const int N = (T + kChunk - 1) / kChunk;
    const int Tp = N * kChunk;
    int P, L;
    choose_segments(B * H, N, &P, &L);
    const size_t BH = (size_t)B * H;
    w.lam = 0;
    w.seg = align256(w.lam + BH * Tp * sizeof(float));
    const size_t seg_bytes = P > 1 ? BH * P * (size_t)(K * kSlots + kSlots * V) * sizeof(float) : 0;
    w.seg_decay = align256(w.seg + seg_bytes);
    w.omega = align256(w.seg_decay + BH * P * sizeof(float));
    w.total = align256(w.omega + BH * Tp * kSlots * 2);
    return w;
}

int launch_prefill(const PrefillParams& p, hipStream_t stream) {
    const int BH = p.B * p.H;
    hipLaunchKernelGGL(clock_kernel, dim3(BH), dim3(256), 0, stream, p);
    if (p.P > 1) {
        hipLaunchKernelGGL(segment_state_kernel, dim3(BH * (p.P - 1), 2), dim3(256), 0, stream, p);
        hipLaunchKernelGGL(carry_kernel, dim3(BH, SEG / 1024), dim3(256), 0, stream, p);
    }
    hipLaunchKernelGGL(pass1_kernel, dim3(BH * p.P), dim3(256), 0, stream, p);
    hipLaunchKernelGGL(pass2_kernel, dim3(BH * p.P), dim3(256), 0, stream, p);
    return 0;
}

int launch_readout_table(const float* readout, float* table, int H, hipStream_t stream) {
    hipLaunchKernelGGL(readout_table_kernel, dim3(H * kActive), dim3(128), 0, stream, readout, table);
    return 0;
}

}  // namespace cyfa
