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
// The sweep kernels run 8 waves (512 threads); each wave holds 1/8 of the fp32
// state as MFMA accumulators, and the global loads of chunk n + 1 are issued
// into registers before chunk n computes. All GEMM-shaped work runs on
// v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation. Every 64-token tile
// (q_hat, k_hat, w, v, slot weights) is staged once in LDS, token-major; the
// operands that contract over tokens are read with the gfx950 LDS transpose
// read. The sweep keeps each segment's state on chip from its first to its
// last chunk; only segment boundary states (one per L chunks) touch HBM.
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

// Row strides (elements) of the LDS tiles. The 16-bit strides are 8 dwords
// modulo the 64 LDS banks, so the four rows a transpose read touches per
// 16-lane block fall on disjoint banks.
constexpr int RS256 = 256 + 16;  // 64 x 256 bf16 tiles
constexpr int RS128 = 128 + 16;  // 64 x 128 16-bit tiles and the 128 x 128 table
constexpr int TS = 64 + 8;       // 64 x 64 score tile
constexpr int FS = 128 + 4;      // 64 x 128 fp32 tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ size_t tok_index(const PrefillParams& p, int b, int t, int h) {
    return ((size_t)b * p.T + t) * p.H + h;
}

// Chunk gates, split into an issue step (global loads into registers, wave 0,
// lane = token) and a commit step (in-chunk scan of g in log2 units,
// ops/utils.py:495-520, and the LDS writes), so that the loads of chunk n + 1
// can be in flight while chunk n computes. LDS per token: sLam = reduced clock
// (lam mod 127) / 127, sBeta, sGam = G_t, sGam[64 + t] = 2^G_t and
// sGam[128 + t] = 2^(G_last - G_t).
struct GateRegs {
    float g, beta, lam;
};

__device__ __forceinline__ GateRegs issue_gates(const PrefillParams& p, int b, int h, int bh, int t0) {
    GateRegs r{0.f, 0.f, 0.f};
    const int tid = threadIdx.x;
    if (tid < 64) {
        const int t = t0 + tid;
        const size_t i = tok_index(p, b, t < p.T ? t : p.T - 1, h);
        r.g = p.g[i];
        r.beta = p.beta[i];
        r.lam = p.lam[(size_t)bh * p.Tp + t];
    }
    return r;
}

__device__ __forceinline__ void commit_gates(const PrefillParams& p, int t0, const GateRegs& r, float* sLam,
                                             float* sBeta, float* sGam) {
    const int tid = threadIdx.x;
    if (tid < 64) {
        const bool valid = t0 + tid < p.T;
        float x = valid ? r.g : 0.f;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (tid >= o) x += y;
        }
        const float gam = x * kLog2e;
        const float last = __shfl(gam, 63, 64);
        sGam[tid] = gam;
        sBeta[tid] = valid ? r.beta : 0.f;
        sLam[tid] = reduced_clock(r.lam);
        sGam[64 + tid] = exp2f(gam);          // 2^G_t
        sGam[128 + tid] = exp2f(last - gam);  // 2^(G_last - G_t)
    }
}

// LDS transpose read (ds_read_b64_tr_b16). Within each 16-lane block of a
// wave, source lane i supplies the address of four consecutive 16-bit
// elements D[i][0..3] and result lane i receives {D[4e + (i >> 2)][i & 3]},
// e = 0..3. load_tr arranges the source addresses so that two such reads
// return the MFMA fragment of the transpose of a row-major tile:
//   lane (lr, lg) element j = X[s0 + 8 lg + j][c0 + lr],   j = 0..7,
// i.e. the A operand A[row = c0 + lr][k = s0 + 8 lg + j] or the B operand
// B[k = s0 + 8 lg + j][col = c0 + lr] of a tile stored token-major.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef s16x4 __attribute__((address_space(3))) lds_s16x4;

__device__ __forceinline__ s16x8 load_tr(const void* X, int ld, int s0, int c0) {
    const int l = threadIdx.x & 63, g = l >> 4, i = l & 15;
    const short* p = reinterpret_cast<const short*>(X) + (s0 + 8 * g + (i >> 2)) * ld + c0 + 4 * (i & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p)));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p + 4 * ld)));
    s16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

__device__ __forceinline__ bf16x8 load_tr_bf16(const bf16_t* X, int ld, int s0, int c0) {
    return __builtin_bit_cast(bf16x8, load_tr(X, ld, s0, c0));
}

__device__ __forceinline__ f16x8 load_tr_f16(const f16_t* X, int ld, int s0, int c0) {
    return __builtin_bit_cast(f16x8, load_tr(X, ld, s0, c0));
}

// Row fragment: lane (lr, lg) gets X[r0 + lr][k0 + 8 lg .. + 8] (A operand, or
// B operand of a product that contracts over X's columns).
template <typename V8, typename T>
__device__ __forceinline__ V8 load_row(const T* X, int ld, int r0, int k0) {
    const int l = threadIdx.x & 63;
    return *reinterpret_cast<const V8*>(X + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// Rows [t0, t0 + 64) of a [B, T, H, 256] bf16 tensor, four 16-byte loads per
// thread of a 512-thread block: row (tid >> 5) + 16 it, columns 8 (tid & 31) .. + 8.
// Rows past T are clamped to T - 1 (and zeroed when stored).
__device__ __forceinline__ void issue_rows(const PrefillParams& p, const bf16_t* x, int b, int h, int t0, bf16x8 raw[4]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int it = 0; it < 4; it++) {
        const int t = t0 + (tid >> 5) + 16 * it;
        raw[it] = *reinterpret_cast<const bf16x8*>(x + tok_index(p, b, t < p.T ? t : p.T - 1, h) * KD + 8 * (tid & 31));
    }
}

// RMS-normalise those rows and store them row-major into dst [64][RS256]:
// x_hat = bf16(x rsqrt(mean x^2 + eps) w) (ops/qk_norm.py:64-107, 206-233).
// A row's 32 chunks live in one half-wave; wn is the weight in LDS.
__device__ __forceinline__ void norm_store_rows(const PrefillParams& p, int t0, const bf16x8 raw[4], const float* wn,
                                                float eps, bf16_t* dst) {
    const int tid = threadIdx.x, c8 = 8 * (tid & 31);
    const float4 w0 = *reinterpret_cast<const float4*>(wn + c8);
    const float4 w1 = *reinterpret_cast<const float4*>(wn + c8 + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int it = 0; it < 4; it++) {
        const int r = (tid >> 5) + 16 * it;
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = (float)raw[it][j];
            ss = fmaf(v, v, ss);
        }
        ss = wave_sum<32>(ss);
        const float rs = t0 + r < p.T ? rsqrtf(ss * (1.f / KD) + eps) : 0.f;
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = (bf16_t)((float)raw[it][j] * rs * wv[j]);
        *reinterpret_cast<bf16x8*>(dst + r * RS256 + c8) = o;
    }
}

// Store rows of v (no normalisation), zero past T.
__device__ __forceinline__ void store_rows(const PrefillParams& p, int t0, const bf16x8 raw[4], bf16_t* dst) {
    const int tid = threadIdx.x, c8 = 8 * (tid & 31);
#pragma unroll
    for (int it = 0; it < 4; it++) {
        const int r = (tid >> 5) + 16 * it;
        bf16x8 o = raw[it];
        if (t0 + r >= p.T) {
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = (bf16_t)0.f;
        }
        *reinterpret_cast<bf16x8*>(dst + r * RS256 + c8) = o;
    }
}

// Slot-weight rows [t0, t0 + 64) of the pass-1 output: two 16-byte loads per thread.
__device__ __forceinline__ void issue_omega(const PrefillParams& p, int bh, int t0, bf16x8 om[2]) {
    const bf16_t* src = p.omega + ((size_t)bh * p.Tp + t0) * kSlots;
#pragma unroll
    for (int it = 0; it < 2; it++) {
        const int idx = threadIdx.x + 512 * it, r = idx >> 4, c8 = (idx & 15) * 8;
        om[it] = *reinterpret_cast<const bf16x8*>(src + r * kSlots + c8);
    }
}

// Write vector of the chunk, w [64 tokens][128] bf16 row-major (ops/utils.py:664-702):
// 4096 pairs over 512 threads.
__device__ __forceinline__ void store_write_rows(const float* sLam, const float* sBeta, bf16_t* dst) {
#pragma unroll
    for (int it = 0; it < 8; it++) {
        const int idx = threadIdx.x + 512 * it, s = idx >> 6, pr = idx & 63;
        float we, wo;
        write_pair(sLam[s], sBeta[s], pr, we, wo);
        bf16_t* d = dst + s * RS128 + 2 * pr;
        d[0] = (bf16_t)we;
        d[1] = (bf16_t)wo;
    }
}

// Write-vector element w[s][m] (ops/utils.py:664-702), rounded to bf16;
// lamr is the token's reduced clock.
__device__ __forceinline__ bf16_t write_elem(float lamr, float beta, int m) { return (bf16_t)write_coord(lamr, beta, m); }

// Masked, decayed score tile for key block sb and query block tb, from an
// accumulated q.k block: P[t][s] = bf16(2^(G_t - G_s) q_t.k_s) for s <= t, else 0
// (ops/chunk_o.py:240-250).
__device__ __forceinline__ void store_scores(const f32x4& sc, int tb, int sb, const float* sGam, bf16_t* sP) {
    const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
    const int s = 16 * sb + lr;
    const float gs = sGam[s];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = 16 * tb + 4 * lg + i;
        const float v = s <= t ? sc[i] * exp2f(sGam[t] - gs) : 0.f;
        sP[t * TS + s] = (bf16_t)v;
    }
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
// 2. Segment-local end states from a zero start. grid = (B*H*(P-1), 2), y = pass;
// 512 threads. Pass 0: wave w owns key-state columns [16 w, 16 w + 16)
// (acc[db] = S[16 db + 4 lg + i][16 w + lr]). Pass 1: wave w owns value-state
// columns [32 w, 32 w + 32) (acc[mb][cb] = S[16 mb + 4 lg + i][32 w + 16 cb + lr]).
constexpr int SG_K = 0;                     // pass 0: bf16 [64][RS256] k_hat rows
constexpr int SG_W = 0;                     // pass 1: bf16 [64][RS128] w rows
constexpr int SG_V = 64 * RS128 * 2;        // pass 1: bf16 [64][RS256] v rows
constexpr int SG_G = SG_V + 64 * RS256 * 2; // f32 [5][64] gates
constexpr int SG_NW = SG_G + 5 * 64 * 4;    // f32 [256] k norm weight
constexpr int SG_LDS = SG_NW + KD * 4;
static_assert(64 * RS256 * 2 <= SG_G, "k tile overlaps the gates");

__global__ __launch_bounds__(512) void segment_state_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[SG_LDS];
    float* sLam = reinterpret_cast<float*>(smem + SG_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    float* sNw = reinterpret_cast<float*>(smem + SG_NW);
    const int P1 = p.P - 1;
    const int bh = blockIdx.x / P1, j = blockIdx.x % P1, pass = blockIdx.y;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    float* out = p.seg + ((size_t)bh * p.P + j) * SEG;
    if (tid < KD) sNw[tid] = p.k_w[tid];

    if (pass == 0) {
        bf16_t* sK = reinterpret_cast<bf16_t*>(smem + SG_K);
        f32x4 acc[16];
#pragma unroll
        for (int db = 0; db < 16; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
        bf16x8 kraw[4];
        issue_rows(p, p.k, b, h, n0 * 64, kraw);
        GateRegs gr = issue_gates(p, b, h, bh, n0 * 64);
        float logdecay = 0.f;
        __syncthreads();
        for (int n = n0; n < n1; n++) {
            const int t0 = n * 64;
            commit_gates(p, t0, gr, sLam, sBeta, sGam);
            norm_store_rows(p, t0, kraw, sNw, p.k_eps, sK);
            if (n + 1 < n1) {
                issue_rows(p, p.k, b, h, t0 + 64, kraw);
                gr = issue_gates(p, b, h, bh, t0 + 64);
            }
            __syncthreads();
            logdecay += sGam[63];
            bf16x8 wt[2];
            {
                const int m = 16 * w + lr;
#pragma unroll
                for (int ss = 0; ss < 2; ss++)
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) {
                        const int s = 32 * ss + 8 * lg + jj;
                        wt[ss][jj] = (bf16_t)((float)write_elem(sLam[s], sBeta[s], m) * sGam[128 + s]);
                    }
            }
            const float dec = sGam[64 + 63];
#pragma unroll
            for (int db = 0; db < 16; db++) acc[db] *= dec;
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int ss = 0; ss < 2; ss++)
                    acc[db] = mfma_bf16(load_tr_bf16(sK, RS256, 32 * ss, 16 * db), wt[ss], acc[db]);
            __syncthreads();
        }
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int i = 0; i < 4; i++) out[(16 * db + 4 * lg + i) * kSlots + 16 * w + lr] = acc[db][i];
        if (tid == 0) p.seg_decay[bh * p.P + j] = exp2f(logdecay);
    } else {
        bf16_t* sW = reinterpret_cast<bf16_t*>(smem + SG_W);
        bf16_t* sV = reinterpret_cast<bf16_t*>(smem + SG_V);
        f32x4 acc[8][2];
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        bf16x8 vraw[4];
        issue_rows(p, p.v, b, h, n0 * 64, vraw);
        GateRegs gr = issue_gates(p, b, h, bh, n0 * 64);
        for (int n = n0; n < n1; n++) {
            const int t0 = n * 64;
            commit_gates(p, t0, gr, sLam, sBeta, sGam);
            store_rows(p, t0, vraw, sV);
            if (n + 1 < n1) {
                issue_rows(p, p.v, b, h, t0 + 64, vraw);
                gr = issue_gates(p, b, h, bh, t0 + 64);
            }
            __syncthreads();
            store_write_rows(sLam, sBeta, sW);
            __syncthreads();
            const float dec = sGam[64 + 63];
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++) acc[mb][cb] *= dec;
#pragma unroll
            for (int ss = 0; ss < 2; ss++) {
                bf16x8 vt[2];
#pragma unroll
                for (int cb = 0; cb < 2; cb++) {
                    const bf16x8 vb = load_tr_bf16(sV, RS256, 32 * ss, 32 * w + 16 * cb);
#pragma unroll
                    for (int jj = 0; jj < 8; jj++) vt[cb][jj] = (bf16_t)((float)vb[jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
                }
#pragma unroll
                for (int mb = 0; mb < 8; mb++) {
                    const bf16x8 a = load_tr_bf16(sW, RS128, 32 * ss, 16 * mb);
#pragma unroll
                    for (int cb = 0; cb < 2; cb++) acc[mb][cb] = mfma_bf16(a, vt[cb], acc[mb][cb]);
                }
            }
            __syncthreads();
        }
        float* outv = out + SEG_K;
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) outv[(16 * mb + 4 * lg + i) * VD + 32 * w + 16 * cb + lr] = acc[mb][cb][i];
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
// 4. Pass 1 (key state) + fused slot readout. grid = B*H*P, 512 threads.
// Wave w owns key-state columns [16 w, 16 w + 16): acc[db] = S[16 db + 4 lg + i][16 w + lr].
// Scores: wave w covers key block sb = w & 3 and query blocks 2 hi, 2 hi + 1
// (hi = w >> 2). Readout: wave w covers query block sb and slot / coordinate
// blocks 4 hi .. 4 hi + 3.
constexpr int P1_Q = 0;                          // bf16 [64][RS256] q_hat rows; later z, then p (f16 [64][RS128])
constexpr int P1_K = P1_Q + 64 * RS256 * 2;      // bf16 [64][RS256] k_hat rows; later raw f32 [64][FS], then weights
constexpr int P1_P = P1_K + 64 * RS256 * 2;      // bf16 [64][TS] masked scores
constexpr int P1_TAB = P1_P + 64 * TS * 2;       // f16 [128][RS128] readout table rows r (row 127 zero)
constexpr int P1_RED = P1_TAB + 128 * RS128 * 2; // f32 [2][64][2] softmax row partials
constexpr int P1_G = P1_RED + 2 * 64 * 2 * 4;    // f32 [5][64] gates
constexpr int P1_NW = P1_G + 5 * 64 * 4;         // f32 [2][256] q and k norm weights
constexpr int P1_LDS = P1_NW + 2 * KD * 4;
static_assert(64 * FS * 4 <= 64 * RS256 * 2, "raw tile must fit in the k tile");
static_assert(P1_LDS <= 160 * 1024, "pass-1 LDS exceeds gfx950 LDS");

__global__ __launch_bounds__(512) void pass1_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P1_LDS];
    bf16_t* sQ = reinterpret_cast<bf16_t*>(smem + P1_Q);
    f16_t* sZ = reinterpret_cast<f16_t*>(smem + P1_Q);
    bf16_t* sK = reinterpret_cast<bf16_t*>(smem + P1_K);
    float* sRaw = reinterpret_cast<float*>(smem + P1_K);
    bf16_t* sOm = reinterpret_cast<bf16_t*>(smem + P1_K);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P1_P);
    f16_t* sTab = reinterpret_cast<f16_t*>(smem + P1_TAB);
    float* sRed = reinterpret_cast<float*>(smem + P1_RED);
    float* sLam = reinterpret_cast<float*>(smem + P1_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    float* sQw = reinterpret_cast<float*>(smem + P1_NW);
    float* sKw = sQw + KD;

    const int bh = blockIdx.x / p.P, j = blockIdx.x % p.P;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int sb = w & 3, hi = w >> 2;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    if (tid < KD) {
        sQw[tid] = p.q_w[tid];
        sKw[tid] = p.k_w[tid];
    }
    {
        const float* tb = p.table + (size_t)h * kActive * kSlots;
        for (int idx = tid; idx < 128 * 128; idx += 512) {
            const int r = idx >> 7, m = idx & 127;
            sTab[r * RS128 + m] = (f16_t)(r < kActive ? tb[r * kSlots + m] : 0.f);
        }
    }
    f32x4 acc[16];
    {
        const float* s0 = p.P > 1 ? p.seg + ((size_t)bh * p.P + j) * SEG
                                  : (p.h0_k ? p.h0_k + (size_t)bh * SEG_K : nullptr);
        if (s0) {
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[db][i] = s0[(16 * db + 4 * lg + i) * kSlots + 16 * w + lr];
        } else {
#pragma unroll
            for (int db = 0; db < 16; db++) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    bf16x8 qraw[4], kraw[4];
    issue_rows(p, p.q, b, h, n0 * 64, qraw);
    issue_rows(p, p.k, b, h, n0 * 64, kraw);
    GateRegs gr = issue_gates(p, b, h, bh, n0 * 64);
    __syncthreads();  // norm weights and table staged

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        commit_gates(p, t0, gr, sLam, sBeta, sGam);
        norm_store_rows(p, t0, qraw, sQw, p.q_eps, sQ);
        norm_store_rows(p, t0, kraw, sKw, p.k_eps, sK);
        if (n + 1 < n1) {
            issue_rows(p, p.q, b, h, t0 + 64, qraw);
            issue_rows(p, p.k, b, h, t0 + 64, kraw);
            gr = issue_gates(p, b, h, bh, t0 + 64);
        }
        __syncthreads();

        // Write vector (B operand) for this wave's 16 slot columns, raw and decayed.
        bf16x8 wf[2], wt[2];
        {
            const int m = 16 * w + lr;
#pragma unroll
            for (int ss = 0; ss < 2; ss++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {
                    const int s = 32 * ss + 8 * lg + jj;
                    const bf16_t wb = write_elem(sLam[s], sBeta[s], m);
                    wf[ss][jj] = wb;
                    wt[ss][jj] = (bf16_t)((float)wb * sGam[128 + s]);
                }
        }
        // Masked, decayed scores P[t][s] for key block sb and query blocks 2 hi, 2 hi + 1.
        {
            f32x4 sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const bf16x8 kb = load_row<bf16x8>(sK, RS256, 16 * sb, 32 * ks);
                sc0 = mfma_bf16(load_row<bf16x8>(sQ, RS256, 32 * hi, 32 * ks), kb, sc0);
                sc1 = mfma_bf16(load_row<bf16x8>(sQ, RS256, 32 * hi + 16, 32 * ks), kb, sc1);
            }
            store_scores(sc0, 2 * hi, sb, sGam, sP);
            store_scores(sc1, 2 * hi + 1, sb, sGam, sP);
        }
        __syncthreads();

        // raw = scale (2^G_t q S_n + P w) for this wave's 16 slot columns.
        f32x4 out[4];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) out[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const bf16x8 bs = state_as_b(acc[2 * ks], acc[2 * ks + 1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
                out[tb] = mfma_bf16(load_query_perm(sQ + (16 * tb + lr) * RS256 + 32 * ks, lg), bs, out[tb]);
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int i = 0; i < 4; i++) out[tb][i] *= sGam[64 + 16 * tb + 4 * lg + i];
#pragma unroll
        for (int ss = 0; ss < 2; ss++)
#pragma unroll
            for (int tb = 0; tb < 4; tb++)
                out[tb] = mfma_bf16(load_row<bf16x8>(sP, TS, 16 * tb, 32 * ss), wf[ss], out[tb]);
        // State update: S = 2^G_last S + k_hat^T bf16(2^(G_last - G_s) w); the
        // k_hat^T fragments come straight from the row-major k tile.
        {
            const float dec = sGam[64 + 63];
#pragma unroll
            for (int db = 0; db < 16; db++) acc[db] *= dec;
#pragma unroll
            for (int db = 0; db < 16; db++)
#pragma unroll
                for (int ss = 0; ss < 2; ss++)
                    acc[db] = mfma_bf16(load_tr_bf16(sK, RS256, 32 * ss, 16 * db), wt[ss], acc[db]);
        }
        __syncthreads();  // q and k tiles are dead from here on
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int i = 0; i < 4; i++) sRaw[(16 * tb + 4 * lg + i) * FS + 16 * w + lr] = out[tb][i] * p.scale;
        __syncthreads();

        // Readout (ops/chunk_readout.py:797-909): z = U(lam) raw, in fp16.
#pragma unroll
        for (int it = 0; it < 8; it++) {
            const int idx = tid + 512 * it, t = idx >> 6, pr = idx & 63;
            const float2 eo = *reinterpret_cast<const float2*>(sRaw + t * FS + 2 * pr);
            float sn, cs;
            pair_sincos(sLam[t], pr, sn, cs);
            f16_t* d = sZ + t * RS128 + 2 * pr;
            d[0] = (f16_t)(cs * eo.x - sn * eo.y);
            d[1] = (f16_t)(sn * eo.x + cs * eo.y);
        }
        __syncthreads();
        // logits = z table^T for query block sb and slots 64 hi .. 64 hi + 63;
        // softmax over the 127 active slots, row max / sum combined across the
        // two waves of a query block through LDS.
        f32x4 lgt[4];
#pragma unroll
        for (int u = 0; u < 4; u++) lgt[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const f16x8 a = load_row<f16x8>(sZ, RS128, 16 * sb, 32 * ks);
#pragma unroll
            for (int u = 0; u < 4; u++) lgt[u] = mfma_f16(a, load_row<f16x8>(sTab, RS128, 16 * (4 * hi + u), 32 * ks), lgt[u]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (16 * (4 * hi + u) + lr < kActive) mx = fmaxf(mx, lgt[u][i]);
            mx = wave_max<16>(mx);
            if (lr == 0) sRed[(16 * sb + 4 * lg + i) * 2 + hi] = mx;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * sb + 4 * lg + i;
            const float mx = fmaxf(sRed[t * 2], sRed[t * 2 + 1]);
            float sum = 0.f;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                lgt[u][i] = 16 * (4 * hi + u) + lr < kActive ? __expf(lgt[u][i] - mx) : 0.f;
                sum += lgt[u][i];
            }
            sum = wave_sum<16>(sum);
            if (lr == 0) sRed[128 + t * 2 + hi] = sum;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * sb + 4 * lg + i;
            const float inv = 1.f / (sRed[128 + t * 2] + sRed[128 + t * 2 + 1]);
#pragma unroll
            for (int u = 0; u < 4; u++) sZ[t * RS128 + 16 * (4 * hi + u) + lr] = (f16_t)(lgt[u][i] * inv);
        }
        __syncthreads();
        // u = p table (table^T fragments by transpose reads), weights = U(-lam) u.
        {
            f32x4 uu[4];
#pragma unroll
            for (int u = 0; u < 4; u++) uu[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int rs = 0; rs < 4; rs++) {
                const f16x8 a = load_row<f16x8>(sZ, RS128, 16 * sb, 32 * rs);
#pragma unroll
                for (int u = 0; u < 4; u++) uu[u] = mfma_f16(a, load_tr_f16(sTab, RS128, 32 * rs, 16 * (4 * hi + u)), uu[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int t = 16 * sb + 4 * lg + i, m = 16 * (4 * hi + u) + lr;
                    const float mine = uu[u][i];
                    const float other = __shfl_xor(mine, 1);
                    float sn, cs;
                    pair_sincos(sLam[t], m >> 1, sn, cs);
                    const float e = (m & 1) ? other : mine, o = (m & 1) ? mine : other;
                    sOm[t * RS128 + m] = (bf16_t)((m & 1) ? (-sn * e + cs * o) : (cs * e + sn * o));
                }
        }
        __syncthreads();
        {
            bf16_t* dst = p.omega + ((size_t)bh * p.Tp + t0) * kSlots;
#pragma unroll
            for (int it = 0; it < 2; it++) {
                const int idx = tid + 512 * it, r = idx >> 4, c8 = (idx & 15) * 8;
                *reinterpret_cast<bf16x8*>(dst + r * kSlots + c8) = *reinterpret_cast<const bf16x8*>(sOm + r * RS128 + c8);
            }
        }
        __syncthreads();
    }

    if (j == p.P - 1 && p.hk) {
        float* dst = p.hk + (size_t)bh * SEG_K;
#pragma unroll
        for (int db = 0; db < 16; db++)
#pragma unroll
            for (int i = 0; i < 4; i++) dst[(16 * db + 4 * lg + i) * kSlots + 16 * w + lr] = acc[db][i];
    }
}

// ---------------------------------------------------------------------------
// 5. Pass 2 (value state). grid = B*H*P, 512 threads. Wave w owns value columns
// [32 w, 32 w + 32): acc[mb][cb] = S[16 mb + 4 lg + i][32 w + 16 cb + lr].
constexpr int P2_OM = 0;                          // bf16 [64][RS128] slot weights (query)
constexpr int P2_W = P2_OM + 64 * RS128 * 2;      // bf16 [64][RS128] w rows (key)
constexpr int P2_V = P2_W + 64 * RS128 * 2;       // bf16 [64][RS256] v rows; later o staging
constexpr int P2_P = P2_V + 64 * RS256 * 2;       // bf16 [64][TS] masked scores
constexpr int P2_G = P2_P + 64 * TS * 2;          // f32 [5][64] gates
constexpr int P2_LDS = P2_G + 5 * 64 * 4;

__global__ __launch_bounds__(512) void pass2_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P2_LDS];
    bf16_t* sOmq = reinterpret_cast<bf16_t*>(smem + P2_OM);
    bf16_t* sW = reinterpret_cast<bf16_t*>(smem + P2_W);
    bf16_t* sV = reinterpret_cast<bf16_t*>(smem + P2_V);
    bf16_t* sO = reinterpret_cast<bf16_t*>(smem + P2_V);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P2_P);
    float* sLam = reinterpret_cast<float*>(smem + P2_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;

    const int bh = blockIdx.x / p.P, j = blockIdx.x % p.P;
    const int b = bh / p.H, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, lr = lane & 15, lg = lane >> 4;
    const int sb = w & 3, hi = w >> 2;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);

    f32x4 acc[8][2];
    {
        const float* s0 = p.P > 1 ? p.seg + ((size_t)bh * p.P + j) * SEG + SEG_K
                                  : (p.h0_v ? p.h0_v + (size_t)bh * SEG_V : nullptr);
        if (s0) {
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[mb][cb][i] = s0[(16 * mb + 4 * lg + i) * VD + 32 * w + 16 * cb + lr];
        } else {
#pragma unroll
            for (int mb = 0; mb < 8; mb++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++) acc[mb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    bf16x8 vraw[4], om[2];
    issue_rows(p, p.v, b, h, n0 * 64, vraw);
    issue_omega(p, bh, n0 * 64, om);
    GateRegs gr = issue_gates(p, b, h, bh, n0 * 64);

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        commit_gates(p, t0, gr, sLam, sBeta, sGam);
#pragma unroll
        for (int it = 0; it < 2; it++) {
            const int idx = tid + 512 * it, r = idx >> 4, c8 = (idx & 15) * 8;
            *reinterpret_cast<bf16x8*>(sOmq + r * RS128 + c8) = om[it];
        }
        store_rows(p, t0, vraw, sV);
        if (n + 1 < n1) {
            issue_rows(p, p.v, b, h, t0 + 64, vraw);
            issue_omega(p, bh, t0 + 64, om);
            gr = issue_gates(p, b, h, bh, t0 + 64);
        }
        __syncthreads();
        store_write_rows(sLam, sBeta, sW);
        __syncthreads();
        {
            f32x4 sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const bf16x8 wb = load_row<bf16x8>(sW, RS128, 16 * sb, 32 * ks);
                sc0 = mfma_bf16(load_row<bf16x8>(sOmq, RS128, 32 * hi, 32 * ks), wb, sc0);
                sc1 = mfma_bf16(load_row<bf16x8>(sOmq, RS128, 32 * hi + 16, 32 * ks), wb, sc1);
            }
            store_scores(sc0, 2 * hi, sb, sGam, sP);
            store_scores(sc1, 2 * hi + 1, sb, sGam, sP);
        }
        __syncthreads();

        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++) out[tb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8 bs0 = state_as_b(acc[2 * ks][0], acc[2 * ks + 1][0]);
            const bf16x8 bs1 = state_as_b(acc[2 * ks][1], acc[2 * ks + 1][1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = load_query_perm(sOmq + (16 * tb + lr) * RS128 + 32 * ks, lg);
                out[tb][0] = mfma_bf16(a, bs0, out[tb][0]);
                out[tb][1] = mfma_bf16(a, bs1, out[tb][1]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float f = sGam[64 + 16 * tb + 4 * lg + i];
                out[tb][0][i] *= f;
                out[tb][1][i] *= f;
            }
        const float dec = sGam[64 + 63];
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++) acc[mb][cb] *= dec;
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            bf16x8 vb[2], vt[2];
#pragma unroll
            for (int cb = 0; cb < 2; cb++) {
                vb[cb] = load_tr_bf16(sV, RS256, 32 * ss, 32 * w + 16 * cb);
#pragma unroll
                for (int jj = 0; jj < 8; jj++) vt[cb][jj] = (bf16_t)((float)vb[cb][jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
            }
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 a = load_row<bf16x8>(sP, TS, 16 * tb, 32 * ss);
                out[tb][0] = mfma_bf16(a, vb[0], out[tb][0]);
                out[tb][1] = mfma_bf16(a, vb[1], out[tb][1]);
            }
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                const bf16x8 a = load_tr_bf16(sW, RS128, 32 * ss, 16 * mb);
                acc[mb][0] = mfma_bf16(a, vt[0], acc[mb][0]);
                acc[mb][1] = mfma_bf16(a, vt[1], acc[mb][1]);
            }
        }
        __syncthreads();  // v is dead; reuse it for the output tile
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    sO[(16 * tb + 4 * lg + i) * RS256 + 32 * w + 16 * cb + lr] = (bf16_t)out[tb][cb][i];
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int idx = tid + 512 * it, r = idx >> 5, c8 = (idx & 31) * 8;
            if (t0 + r < p.T)
                *reinterpret_cast<bf16x8*>(p.o + tok_index(p, b, t0 + r, h) * VD + c8) =
                    *reinterpret_cast<const bf16x8*>(sO + r * RS256 + c8);
        }
        __syncthreads();
    }

    if (j == p.P - 1 && p.hv) {
        float* dst = p.hv + (size_t)bh * SEG_V;
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int cb = 0; cb < 2; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[(16 * mb + 4 * lg + i) * VD + 32 * w + 16 * cb + lr] = acc[mb][cb][i];
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
        hipLaunchKernelGGL(segment_state_kernel, dim3(BH * (p.P - 1), 2), dim3(512), 0, stream, p);
        hipLaunchKernelGGL(carry_kernel, dim3(BH, SEG / 1024), dim3(256), 0, stream, p);
    }
    hipLaunchKernelGGL(pass1_kernel, dim3(BH * p.P), dim3(512), 0, stream, p);
    hipLaunchKernelGGL(pass2_kernel, dim3(BH * p.P), dim3(512), 0, stream, p);
    return 0;
}

int launch_readout_table(const float* readout, float* table, int H, hipStream_t stream) {
    hipLaunchKernelGGL(readout_table_kernel, dim3(H * kActive), dim3(128), 0, stream, readout, table);
    return 0;
}

}  // namespace cyfa
