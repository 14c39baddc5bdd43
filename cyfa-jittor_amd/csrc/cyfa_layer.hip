// cyfa_layer.hip -- the layer-side kernels either side of the CyFA op for gfx950:
// fused residual add + RMSNorm (+ sigmoid gate), the causal depthwise short
// convolution, the gate activations and the SwiGLU product. All are
// HBM-streaming elementwise / row kernels; each reads its inputs once and
// writes its outputs once, in bf16 with fp32 arithmetic.
#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// One wave per row; lane covers columns 4 lane + 256 j.
// (layers/cyfa.py:62-135 and modeling_cyfa.py:48-51)
//   s   = residual ? bf16(x + residual) : x      (sum_out receives s)
//   xs  = prescale != 1 ? bf16(s * prescale) : s
//   out = bf16(xs * rsqrt(mean xs^2 + eps) * weight * (gate ? sigmoid(gate) : 1))
template <int J>
__global__ __launch_bounds__(256) void rms_norm_kernel(NormParams p) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= p.rows) return;
    const size_t base = (size_t)row * p.D;
    // Every load of the row is issued before the first one is used: x, the
    // residual, the weight and the gate.
    bf16x4 xr[J], rr[J], gr[J];
    float4 wr[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int d = 4 * lane + 256 * j;
        xr[j] = *reinterpret_cast<const bf16x4*>(p.x + base + d);
        if (p.residual) rr[j] = *reinterpret_cast<const bf16x4*>(p.residual + base + d);
        wr[j] = *reinterpret_cast<const float4*>(p.weight + d);
        if (p.gate) gr[j] = *reinterpret_cast<const bf16x4*>(p.gate + base + d);
    }
    float v[J][4];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int d = 4 * lane + 256 * j;
        if (p.residual) {
            bf16x4 s;
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = (bf16_t)((float)xr[j][i] + (float)rr[j][i]);
            *reinterpret_cast<bf16x4*>(p.sum_out + base + d) = s;
#pragma unroll
            for (int i = 0; i < 4; i++) v[j][i] = (float)s[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) v[j][i] = (float)xr[j][i];
        }
        if (p.prescale != 1.f) {
#pragma unroll
            for (int i = 0; i < 4; i++) v[j][i] = bf16_round(v[j][i] * p.prescale);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) ss = fmaf(v[j][i], v[j][i], ss);
    }
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss / (float)p.D + p.eps);
#pragma unroll
    for (int j = 0; j < J; j++) {
        const int d = 4 * lane + 256 * j;
        const float4 w = wr[j];
        float y[4] = {v[j][0] * rs * w.x, v[j][1] * rs * w.y, v[j][2] * rs * w.z, v[j][3] * rs * w.w};
        if (p.gate) {
#pragma unroll
            for (int i = 0; i < 4; i++) y[i] *= sigmoidf((float)gr[j][i]);
        }
        *reinterpret_cast<bf16x4*>(p.out + base + d) = bf16x4{(bf16_t)y[0], (bf16_t)y[1], (bf16_t)y[2], (bf16_t)y[3]};
    }
}

// y[m][n] = bias[n] + sum_k x[m][k] W[n][k] for M <= 64 rows (the nn.Linear /
// F.linear calls of the one-token decode step, layers/cyfa.py and
// modeling_cyfa.py). At these shapes a library GEMM tiles M into large blocks
// and leaves most of the chip idle. Here a workgroup of 8 waves computes one
// tile of RT x 16 rows by CT x 16 columns over the whole of K, on
// v_mfma_f32_16x16x32_bf16 (A = x rows, B = W rows read straight from global
// memory: lane (lr, lg) loads 8 consecutive k of row lr). Wave w takes a
// contiguous run of the 32-deep k-steps, so its loads of a row cover whole
// cache lines, with the loads of several steps in flight; the eight partial
// tiles are summed in LDS in wave order. Every output element is therefore
// summed in the same order whatever the tile shape, so the launcher may pick
// the shape per call (launch_linear_rows) without changing a bit of y.
// Rows of x at or past M and rows of W at or past N read as zero (buffer
// bounds).
typedef __amdgpu_buffer_rsrc_t lin_rsrc_t;

__device__ __forceinline__ lin_rsrc_t lin_rsrc(const void* base, size_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ bf16x8 lin_ld(lin_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// k-steps whose loads a wave has in flight together: about 24 loads per lane
__host__ __device__ constexpr int lin_batch(int rt, int ct) { return rt + ct <= 2 ? 12 : rt + ct <= 3 ? 8 : rt + ct <= 4 ? 6 : 4; }

template <int U, int RT, int CT>
__device__ __forceinline__ void lin_issue_w(lin_rsrc_t rw, int s, int s1, uint32_t wrow, uint32_t wstride, int lg,
                                           bf16x8 (&wf)[U][CT]) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (s + u < s1) {
            const uint32_t kb = (uint32_t)(32 * (s + u) + 8 * lg) * 2;
#pragma unroll
            for (int c = 0; c < CT; c++) wf[u][c] = lin_ld(rw, wrow + c * wstride + kb);
        }
    }
}

template <int U, int RT>
__device__ __forceinline__ void lin_issue_x(lin_rsrc_t rx, int s, int s1, uint32_t xrow, uint32_t xstride, int lg,
                                            bf16x8 (&xf)[U][RT]) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (s + u < s1) {
            const uint32_t kb = (uint32_t)(32 * (s + u) + 8 * lg) * 2;
#pragma unroll
            for (int rt = 0; rt < RT; rt++) xf[u][rt] = lin_ld(rx, xrow + rt * xstride + kb);
        }
    }
}

template <int U, int RT, int CT>
__device__ __forceinline__ void lin_mfma(int s, int s1, const bf16x8 (&wf)[U][CT], const bf16x8 (&xf)[U][RT],
                                         f32x4 (&acc)[RT][CT]) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (s + u < s1) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int c = 0; c < CT; c++)
                    acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[u][rt], wf[u][c], acc[rt][c], 0, 0, 0);
        }
    }
}

template <int RT, int CT, bool NORM>
__global__ __launch_bounds__(512) void linear_rows_kernel(LinearParams p) {
    constexpr int TM = 16 * RT, TN = 16 * CT, OUT = TM * TN, R = (OUT + 511) / 512;
    constexpr int U = lin_batch(RT, CT);
    __shared__ float part[8][TM][TN + 1];
    __shared__ float sq[NORM ? 8 : 1][NORM ? TM : 1];
    __shared__ float4 snw[NORM ? LINEAR_NORM_MAX_K / 4 : 1];
    // The wave index comes from a scalar register, so the k-run bounds and
    // every `s + u < s1` test are uniform branches. With a lane-divergent test
    // the compiler left one MFMA of the fused-norm variant to run under an
    // empty exec mask instead of branching around it, and outputs of that
    // build picked up stale operand registers (NaNs on MI355X).
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lr = lane & 15,
              lg = lane >> 4;
    const int n0 = blockIdx.x * TN, m0 = blockIdx.y * TM;
    const int mrows = min(TM, p.M - m0);
    const lin_rsrc_t rx = lin_rsrc(p.x + (size_t)m0 * p.ldx, ((size_t)(mrows - 1) * p.ldx + p.K) * 2);
    const lin_rsrc_t rw = lin_rsrc(p.w + (size_t)n0 * p.K, (size_t)min(TN, p.N - n0) * p.K * 2);
    // the bias and the residual of this thread's outputs, loaded with the operands
    float bias[R], add[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int idx = threadIdx.x + 512 * r, n = n0 + idx % TN, m = idx / TN;
        bias[r] = p.bias && n < p.N ? (float)p.bias[n] : 0.f;
        add[r] = p.add && n < p.N && idx < OUT && m < mrows ? (float)p.add[(size_t)(m0 + m) * p.ld_add + n] : 0.f;
    }
    f32x4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int c = 0; c < CT; c++) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int steps = p.K / 32, per = (steps + 7) / 8;
    const int s0 = min(steps, w * per), s1 = min(steps, s0 + per);
    const uint32_t wrow = (uint32_t)lr * p.K * 2, xrow = (uint32_t)lr * (uint32_t)p.ldx * 2;
    const uint32_t xstride = (uint32_t)(16 * p.ldx * 2), wstride = (uint32_t)(16 * p.K * 2);
    bf16x8 wf[U][CT], xf[U][RT];
    if constexpr (!NORM) {
        for (int s = s0; s < s1; s += U) {
            lin_issue_w<U, RT, CT>(rw, s, s1, wrow, wstride, lg, wf);
            lin_issue_x<U, RT>(rx, s, s1, xrow, xstride, lg, xf);
            lin_mfma<U, RT, CT>(s, s1, wf, xf, acc);
        }
    } else {
        // The row norm (the launcher guarantees one batch: K <= 256 U). Lane
        // (lr, lg) holds 8 columns of row 16 rt + lr per k-step, the same
        // columns in every tile shape. Its sum of squares runs over its
        // k-steps in order, then over the row's four lanes (xor 16, xor 32)
        // and the eight waves in wave order.
        // x (and the residual) first, then the norm weight, then W: loads
        // complete in order, so the norm waits for x alone while W streams in.
        const bool res = p.norm_residual != nullptr;
        lin_issue_x<U, RT>(rx, s0, s1, xrow, xstride, lg, xf);
        bf16x8 rf[U][RT];
        if (res) {
            const lin_rsrc_t rr =
                lin_rsrc(p.norm_residual + (size_t)m0 * p.ldr, ((size_t)(mrows - 1) * p.ldr + p.K) * 2);
            lin_issue_x<U, RT>(rr, s0, s1, (uint32_t)lr * (uint32_t)p.ldr * 2, (uint32_t)(16 * p.ldr * 2), lg, rf);
        }
        const bool has_nw = 4 * (int)threadIdx.x < p.K;  // K <= 2048: one float4 per thread at most
        float4 nwv = float4{0.f, 0.f, 0.f, 0.f};
        if (has_nw) nwv = reinterpret_cast<const float4*>(p.norm_weight)[threadIdx.x];
        lin_issue_w<U, RT, CT>(rw, s0, s1, wrow, wstride, lg, wf);
        if (res) {
            // s = bf16(x + residual); the first column of workgroups writes it out
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < s1) {
#pragma unroll
                    for (int rt = 0; rt < RT; rt++) {
#pragma unroll
                        for (int e = 0; e < 8; e++) xf[u][rt][e] = (bf16_t)((float)xf[u][rt][e] + (float)rf[u][rt][e]);
                        if (blockIdx.x == 0 && 16 * rt + lr < mrows)
                            *reinterpret_cast<bf16x8*>(p.norm_sum_out + (size_t)(m0 + 16 * rt + lr) * p.ldr +
                                                       32 * (s0 + u) + 8 * lg) = xf[u][rt];
                    }
                }
            }
        }
        if (has_nw) snw[threadIdx.x] = nwv;
        float ss[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            ss[rt] = 0.f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < s1) {
#pragma unroll
                    for (int e = 0; e < 8; e++) ss[rt] = fmaf((float)xf[u][rt][e], (float)xf[u][rt][e], ss[rt]);
                }
            }
            ss[rt] += __shfl_xor(ss[rt], 16);
            ss[rt] += __shfl_xor(ss[rt], 32);
            if (lg == 0) sq[w][16 * rt + lr] = ss[rt];
        }
        __syncthreads();
        // bf16(s * rs * weight), as rms_norm_kernel rounds it
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            float t = 0.f;
#pragma unroll
            for (int ww = 0; ww < 8; ww++) t += sq[ww][16 * rt + lr];
            const float rs = rsqrtf(t / (float)p.K + p.norm_eps);
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < s1) {
                    const float4 a = snw[(32 * (s0 + u) + 8 * lg) / 4], b = snw[(32 * (s0 + u) + 8 * lg) / 4 + 1];
                    const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int e = 0; e < 8; e++) xf[u][rt][e] = (bf16_t)((float)xf[u][rt][e] * rs * wv[e]);
                }
            }
        }
        lin_mfma<U, RT, CT>(s0, s1, wf, xf, acc);
    }
    // acc[rt][c][i] = partial y[m0 + 16 rt + 4 lg + i][n0 + 16 c + lr]
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) part[w][16 * rt + 4 * lg + i][16 * c + lr] = acc[rt][c][i];
    __syncthreads();
    if (CT == 2 && p.swiglu) {  // the SwiGLU product of the tile's 16 gate and 16 up columns
        for (int idx = threadIdx.x; idx < TM * 16; idx += 512) {
            const int m = idx >> 4, f = idx & 15;
            float sg = 0.f, su = 0.f;
#pragma unroll
            for (int ww = 0; ww < 8; ww++) {
                sg += part[ww][m][f];
                su += part[ww][m][16 + f];
            }
            const float gf = (float)(bf16_t)sg, uf = (float)(bf16_t)su;
            if (m < mrows && n0 + f < p.N)
                p.y[(size_t)(m0 + m) * p.ldy + n0 / 2 + f] = (bf16_t)(gf * sigmoidf(gf) * uf);
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int idx = threadIdx.x + 512 * r, m = idx / TN, n = idx % TN;
        if (idx < OUT) {
            float s = 0.f;
#pragma unroll
            for (int ww = 0; ww < 8; ww++) s += part[ww][m][n];
            float v = s + bias[r];
            if (p.add) v = (float)(bf16_t)v + add[r];  // the block's residual add, x + bf16(y)
            if (m < mrows && n0 + n < p.N) p.y[(size_t)(m0 + m) * p.ldy + n0 + n] = (bf16_t)v;
        }
    }
}

// Causal depthwise convolution over time (layers/cyfa.py:138-233):
//   y[b, t, c] = bias[c] + sum_{w < W} weight[c, w] * X[b, t + w - (W - 1), c]
// where X[b, i] is x[b, i] for i >= 0, cache[b, W - 1 + i] for i < 0 when a
// cache is given, else 0. Thread = 8 channels x a run of CONV_RUN tokens,
// sliding the W-row window through registers; channel c goes to output
// c / split, column c % split. The thread of the last run writes its window,
// the last W - 1 rows of X, to cache_out (layers/cyfa.py:172-182); with a
// single run it has read its cache rows before, so the update may be in place.
constexpr int CONV_RUN = 32;

template <int W>
__global__ __launch_bounds__(256) void short_conv_kernel(ConvParams p) {
    const int c8 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c8 >= p.D) return;
    const int b = blockIdx.y, t0 = blockIdx.z * CONV_RUN;
    float wt[W][8], bias[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int w = 0; w < W; w++) wt[w][i] = (float)p.weight[(size_t)(c8 + i) * W + w];
        bias[i] = p.bias ? (float)p.bias[c8 + i] : 0.f;
    }
    auto row = [&](int i) -> bf16x8 {
        if (i >= 0) return *reinterpret_cast<const bf16x8*>(p.x + ((size_t)b * p.T + i) * p.x_row + c8);
        if (p.cache)
            return *reinterpret_cast<const bf16x8*>(p.cache + (size_t)b * p.cache_batch + (size_t)(W - 1 + i) * p.cache_row + c8);
        bf16x8 z;
#pragma unroll
        for (int k = 0; k < 8; k++) z[k] = (bf16_t)0.f;
        return z;
    };
    float win[W][8];
#pragma unroll
    for (int w = 0; w < W - 1; w++) {
        const bf16x8 r = row(t0 + w - (W - 1));
#pragma unroll
        for (int i = 0; i < 8; i++) win[w][i] = (float)r[i];
    }
    const int out_i = c8 / p.split, col = c8 % p.split;
    bf16_t* out = p.out[out_i];
    const int t1 = t0 + CONV_RUN < p.T ? t0 + CONV_RUN : p.T;
    // Eight rows at a time: their loads are all in flight before the first is used.
    constexpr int U = 8;
    for (int tb = t0; tb < t1; tb += U) {
        bf16x8 rows[U];
        const bf16_t* src = p.x + ((size_t)b * p.T + tb) * p.x_row + c8;  // rows tb.. are never before the start
        const int n = t1 - tb;
#pragma unroll
        for (int u = 0; u < U; u++)
            rows[u] = *reinterpret_cast<const bf16x8*>(src + (size_t)(u < n ? u : 0) * p.x_row);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (tb + u < t1) {
#pragma unroll
                for (int i = 0; i < 8; i++) win[W - 1][i] = (float)rows[u][i];
                bf16x8 y;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float acc = win[0][i] * wt[0][i];
#pragma unroll
                    for (int w = 1; w < W; w++) acc = fmaf(win[w][i], wt[w][i], acc);
                    y[i] = (bf16_t)(acc + bias[i]);
                }
                *reinterpret_cast<bf16x8*>(out + ((size_t)b * p.T + tb + u) * p.split + col) = y;
#pragma unroll
                for (int w = 0; w < W - 1; w++)
#pragma unroll
                    for (int i = 0; i < 8; i++) win[w][i] = win[w + 1][i];
            }
        }
    }
    if (p.cache_out && t1 == p.T) {
#pragma unroll
        for (int w = 0; w < W - 1; w++) {
            bf16x8 r;
#pragma unroll
            for (int i = 0; i < 8; i++) r[i] = (bf16_t)win[w][i];
            *reinterpret_cast<bf16x8*>(p.cache_out + (size_t)b * p.cache_out_batch + (size_t)w * p.cache_out_row + c8) = r;
        }
    }
}

// SwiGLU product (modeling_cyfa.py:22-27): out = bf16(g sigmoid(g) u) for
// gu = [g | u] rows of 2F bf16.
__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16_t* gu, bf16_t* out, int rows, int F) {
    const size_t i8 = ((size_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i8 >= (size_t)rows * F) return;
    const size_t r = i8 / F, c = i8 % F;
    const bf16x8 g = *reinterpret_cast<const bf16x8*>(gu + r * 2 * F + c);
    const bf16x8 u = *reinterpret_cast<const bf16x8*>(gu + r * 2 * F + F + c);
    bf16x8 y;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float gf = (float)g[i];
        y[i] = (bf16_t)(gf * sigmoidf(gf) * (float)u[i]);
    }
    *reinterpret_cast<bf16x8*>(out + i8) = y;
}

// Row-wise argmax of bf16 logits with torch.argmax's result: the index of the
// first maximum, NaN counting as larger than any number. One workgroup per row;
// each thread keeps the best (value, index) of its strided elements, then the
// workgroup reduces with the same order.
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
    const bool vn = v != v, bn = bv != bv;
    if (vn != bn) return vn;
    if (!vn && v != bv) return v > bv;
    return i < bi;
}

__global__ __launch_bounds__(1024) void argmax_rows_kernel(const bf16_t* x, long long ldx, int n, long long* out) {
    constexpr int NT = 1024, DEPTH = 4;  // four 16-byte loads per thread in flight
    const bf16_t* xr = x + (size_t)blockIdx.x * ldx;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = 0; base < n; base += 8 * NT * DEPTH) {
        bf16x8 v[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
            const int i0 = base + 8 * (threadIdx.x + NT * d);
            if (i0 + 8 <= n) v[d] = *reinterpret_cast<const bf16x8*>(xr + i0);
        }
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
            const int i0 = base + 8 * (threadIdx.x + NT * d);
            if (i0 + 8 <= n) {
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (argmax_better((float)v[d][e], i0 + e, bv, bi)) {
                        bv = (float)v[d][e];
                        bi = i0 + e;
                    }
            } else {
                for (int i = i0; i < n && i < i0 + 8; i++)
                    if (argmax_better((float)xr[i], i, bv, bi)) {
                        bv = (float)xr[i];
                        bi = i;
                    }
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (argmax_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __shared__ float sv[NT / 64];
    __shared__ int si[NT / 64];
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < NT / 64; w++)
            if (argmax_better(sv[w], si[w], bv, bi)) {
                bv = sv[w];
                bi = si[w];
            }
        out[blockIdx.x] = bi;
    }
}

// Gate activations (layers/cyfa.py:323-326) from abd = [a | b | d] rows of 3H
// bf16 (the b / d biases already added): g = -exp(A_log) softplus(a + dt_bias),
// beta = sigmoid(b), delta = sigmoid(d), all fp32 [rows, H].
__global__ __launch_bounds__(256) void gates_kernel(const bf16_t* abd, long long abd_row, const float* dt_bias,
                                                    const float* A_log, float* g, float* beta, float* delta, int rows,
                                                    int H) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * H) return;
    const int r = i / H, h = i % H;
    const bf16_t* row = abd + (size_t)r * abd_row;
    const float a = (float)row[h] + dt_bias[h];
    const float sp = a > 20.f ? a : log1pf(expf(a));
    g[i] = -expf(A_log[h]) * sp;
    beta[i] = sigmoidf((float)row[H + h]);
    delta[i] = sigmoidf((float)row[2 * H + h]);
}

}  // namespace

int launch_rms_norm(const NormParams& p, hipStream_t stream) {
    const dim3 grid((p.rows + 3) / 4), block(256);
    switch (p.D / 256) {
        case 1: hipLaunchKernelGGL(rms_norm_kernel<1>, grid, block, 0, stream, p); break;
        case 2: hipLaunchKernelGGL(rms_norm_kernel<2>, grid, block, 0, stream, p); break;
        case 4: hipLaunchKernelGGL(rms_norm_kernel<4>, grid, block, 0, stream, p); break;
        case 8: hipLaunchKernelGGL(rms_norm_kernel<8>, grid, block, 0, stream, p); break;
        default: return -1;
    }
    return 0;
}

// The tile shape of linear_rows_kernel for one call. Each workgroup reads
// 16 (RT + CT) rows of K (RT x 16 rows of x and CT x 16 rows of W), and at
// these sizes a CU's read rate, not the chip's, is the limit; one workgroup
// fits a CU at a time, so the workgroups past the first 256 run in further
// rounds. Pick the shape with the least bytes read per CU over all rounds
// (on MI355X: 28 -> 35 k tok/s for the 400M decode step at B=64 against a
// fixed 4 x 2 tile). The SwiGLU epilogue needs CT = 2, the 16 gate and 16 up
// columns of one interleaved group; the row norm needs each wave's k-steps in
// one batch of loads (K <= 256 lin_batch). False when no shape qualifies.
static bool linear_tile(int M, int N, bool swiglu, int norm_k, int& rt_out, int& ct_out) {
    static const int shapes[][2] = {{4, 4}, {4, 2}, {2, 4}, {4, 1}, {2, 2}, {1, 4}, {2, 1}, {1, 2}, {1, 1}};
    long long best = -1;
    rt_out = 4;
    ct_out = 2;
    for (const auto& sh : shapes) {
        const int rt = sh[0], ct = sh[1];
        if (swiglu && ct != 2) continue;
        if (norm_k && rt * ct > 8) continue;  // no fused-norm build of the 64 x 64 tile (its registers would spill)
        if (norm_k > 256 * lin_batch(rt, ct)) continue;  // the norm needs all of a row in one batch
        const long long groups = (long long)((M + 16 * rt - 1) / (16 * rt)) * ((N + 16 * ct - 1) / (16 * ct));
        const long long cost = (groups + 255) / 256 * (rt + ct);
        if (best < 0 || cost < best) {
            best = cost;
            rt_out = rt;
            ct_out = ct;
        }
    }
    return best >= 0;
}

int launch_linear_rows(const LinearParams& p, hipStream_t stream) {
    if (p.M < 1 || p.M > 64 || (p.norm_weight && p.K > LINEAR_NORM_MAX_K)) return -1;
    int rt, ct;
    if (!linear_tile(p.M, p.N, p.swiglu != 0, p.norm_weight ? p.K : 0, rt, ct)) return -1;
    const dim3 grid((p.N + 16 * ct - 1) / (16 * ct), (p.M + 16 * rt - 1) / (16 * rt)), block(512);
    const bool norm = p.norm_weight != nullptr;
#define CYFA_LINEAR(RT_, CT_)                                                                                  \
    if (rt == RT_ && ct == CT_) {                                                                              \
        if (norm)                                                                                              \
            hipLaunchKernelGGL((linear_rows_kernel<RT_, CT_, true>), grid, block, 0, stream, p);              \
        else                                                                                                   \
            hipLaunchKernelGGL((linear_rows_kernel<RT_, CT_, false>), grid, block, 0, stream, p);             \
        return 0;                                                                                              \
    }
    if (rt == 4 && ct == 4 && !norm) {  // the lm_head's tile at 64 rows (N = 32000: 500 workgroups)
        hipLaunchKernelGGL((linear_rows_kernel<4, 4, false>), grid, block, 0, stream, p);
        return 0;
    }
    CYFA_LINEAR(4, 2)
    CYFA_LINEAR(2, 4)
    CYFA_LINEAR(4, 1)
    CYFA_LINEAR(2, 2)
    CYFA_LINEAR(1, 4)
    CYFA_LINEAR(2, 1)
    CYFA_LINEAR(1, 2)
    CYFA_LINEAR(1, 1)
#undef CYFA_LINEAR
    return -1;
}

int launch_short_conv(const ConvParams& p, hipStream_t stream) {
    const dim3 grid((p.D / 8 + 255) / 256, p.B, (p.T + CONV_RUN - 1) / CONV_RUN), block(256);
    switch (p.W) {
        case 2: hipLaunchKernelGGL(short_conv_kernel<2>, grid, block, 0, stream, p); break;
        case 3: hipLaunchKernelGGL(short_conv_kernel<3>, grid, block, 0, stream, p); break;
        case 4: hipLaunchKernelGGL(short_conv_kernel<4>, grid, block, 0, stream, p); break;
        default: return -1;
    }
    return 0;
}

int launch_silu_mul(const bf16_t* gu, bf16_t* out, int rows, int F, hipStream_t stream) {
    const size_t n8 = (size_t)rows * F / 8;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream, gu, out, rows, F);
    return 0;
}

int launch_argmax_rows(const bf16_t* x, long long ldx, int rows, int n, long long* out, hipStream_t stream) {
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, stream, x, ldx, n, out);
    return 0;
}

int launch_gates(const bf16_t* abd, long long abd_row, const float* dt_bias, const float* A_log, float* g, float* beta,
                 float* delta, int rows, int H, hipStream_t stream) {
    hipLaunchKernelGGL(gates_kernel, dim3((rows * H + 255) / 256), dim3(256), 0, stream, abd, abd_row, dt_bias, A_log, g,
                       beta, delta, rows, H);
    return 0;
}

}  // namespace cyfa
