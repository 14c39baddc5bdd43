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
// v_mfma_f32_16x16x32_bf16 (A = x rows, B = W rows). Wave w takes a contiguous
// run of the 32-deep k-steps, with the loads of several steps in flight; the
// eight partial tiles are summed in LDS in wave order. Every output element is
// therefore summed in the same order whatever the tile shape, so the launcher
// may pick the shape per call (launch_linear_rows) without changing a bit of y.
//
// Operand loads. An MFMA operand wants lane (lr, lg) to hold 8 consecutive k
// of row lr, so a load in that layout touches 16 rows x 64 bytes; on MI355X
// such loads move data at about half the rate of loads that cover whole
// 128-byte lines (a 64-row x 1024 x 5632 tile read: 8.5 us against 4.9 us).
// So a wave loads each pair of k-steps as whole lines, 8 rows x 128 bytes per
// instruction, writes them to its own LDS region (rows LIN_STRIDE bytes apart,
// so that the 16 rows of an operand read fall in 16 distinct bank groups) and
// reads the operands back in MFMA layout. No other wave touches the region, so
// no barrier is needed: a wave's LDS accesses complete in order.
// Rows of x at or past M and rows of W at or past N read as zero (buffer
// bounds).
typedef __amdgpu_buffer_rsrc_t lin_rsrc_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int LIN_STRIDE = 144;  // staged row: 128 bytes (two k-steps) + 16 bytes of padding

__device__ __forceinline__ float bf16_bits_to_float(unsigned short b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ lin_rsrc_t lin_rsrc(const void* base, size_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// The most k-step pairs whose loads a wave has in flight together, about 24
// loads per lane: P <= lin_pairs(RT, CT).
__host__ __device__ constexpr int lin_pairs(int rt, int ct) { return rt + ct <= 2 ? 6 : rt + ct <= 3 ? 4 : rt + ct <= 4 ? 3 : 2; }

// The offset of a load that must return zero: past the end of every buffer
// the kernel reads (launch_linear_rows keeps each span below 2^31 bytes).
// Loads are predicated through their offset rather than a branch, so that no
// divergent branch sits among the loads: at such a branch the compiler waits
// for every load in flight.
constexpr uint32_t LIN_DEAD = 0x80000000u;

// The loads of k-steps s and s + 1 for G groups of 16 rows (row stride rs
// bytes), as whole lines: instruction i, lane l reads row 8 i + l / 8, the
// 16-byte chunk l % 8 of the row's 128 bytes. Chunks of a step at or past s1
// read zero.
template <int G>
__device__ __forceinline__ void lin_load_pair(lin_rsrc_t r, uint32_t rs, int s, int s1, int lane,
                                              u32x4 (&raw)[2 * G]) {
    const int cl = lane & 7;
    // LIN_DEAD (bit 31) when the chunk's step is at or past s1: the sign bit of
    // s + cl / 4 - s1 is set exactly when the step is live. Written as integer
    // arithmetic; a select here was turned into a divergent branch per load.
    const uint32_t dead = (~(uint32_t)(s + (cl >> 2) - s1)) & LIN_DEAD;
    const uint32_t col = ((uint32_t)(32 * s + 8 * cl) * 2) | dead;
#pragma unroll
    for (int i = 0; i < 2 * G; i++) {
        const uint32_t row = 8 * i + (lane >> 3);
        raw[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, row * rs + col, 0, 0));
    }
}

// Writes the chunks of lin_load_pair to rows [0, 16 G) of a staging region.
template <int G>
__device__ __forceinline__ void lin_stage_pair(char* region, int lane, const u32x4 (&raw)[2 * G]) {
#pragma unroll
    for (int i = 0; i < 2 * G; i++)
        *reinterpret_cast<u32x4*>(region + (8 * i + (lane >> 3)) * LIN_STRIDE + 16 * (lane & 7)) = raw[i];
}

// The MFMA operand of staged step u (0 or 1) for rows 16 g .. 16 g + 15:
// lane (lr, lg) gets row 16 g + lr, k = 8 lg .. 8 lg + 7 of the step.
__device__ __forceinline__ bf16x8 lin_frag(const char* region, int g, int u, int lr, int lg) {
    return *reinterpret_cast<const bf16x8*>(region + (16 * g + lr) * LIN_STRIDE + 16 * (4 * u + lg));
}

// The prefetch workgroups of a projection launch (block ids from `tiles` on,
// nwg of them; this is number wg, on XCD (tiles + wg) mod 8, as workgroups are
// dealt to the XCDs round-robin by block id): the ranges p.pf[r] in order, in
// 8 KiB units (one 16-byte load per thread), eight units in flight. A range
// with a span is read for its consumer, whose workgroups that read the span's
// bytes [c span, (c + 1) span) run on XCD c mod 8: this workgroup reads the
// spans of the consumers on its own XCD, which land in that XCD's L2. A range
// without one is read in units wg, wg + nwg, ... The values go to an empty asm
// statement (the loads must not be dropped); nothing is written.
__device__ __forceinline__ void lin_prefetch(const LinearParams& p, int wg, int nwg, int tiles) {
    const int x = (tiles + wg) & 7, qi = wg >> 3, nx = (nwg - (wg & 7) + 7) >> 3;
#pragma unroll 1
    for (int r = 0; r < LINEAR_PREFETCH_RANGES; r++) {
        const unsigned long long bytes = p.pf_bytes[r];
        if (bytes == 0) continue;
        const lin_rsrc_t rs = lin_rsrc(p.pf[r], (size_t)bytes);  // bytes < 2^31
        const uint32_t span = (uint32_t)p.pf_span[r];
        const uint32_t cpc = (span + 8191) >> 13;  // 8 KiB pieces per consumer span
        const uint32_t ncons = span ? (uint32_t)((bytes + span - 1) / span) : 0u;
        const uint32_t mine = span ? ((uint32_t)x < ncons ? (ncons - (uint32_t)x + 7) >> 3 : 0u) : 0u;
        const uint32_t units = span ? mine * cpc : (uint32_t)((bytes + 8191) >> 13);
        const uint32_t first = span ? (uint32_t)qi : (uint32_t)wg, stride = span ? (uint32_t)nx : (uint32_t)nwg;
#pragma unroll 1
        for (uint32_t u0 = first; u0 < units; u0 += 8u * stride) {
            u32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t u = u0 + (uint32_t)i * stride;
                uint32_t off, live = u < units;
                if (span) {  // piece u % cpc of consumer x + 8 (u / cpc)
                    const uint32_t c = (uint32_t)x + 8u * (u / cpc), in = (u % cpc) * 8192u + (uint32_t)threadIdx.x * 16u;
                    off = c * span + in;
                    live &= in < span;
                } else {
                    off = (u << 13) + (uint32_t)threadIdx.x * 16u;
                }
                v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off | (live ? 0u : LIN_DEAD), 0, 0));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) asm volatile("" ::"v"(v[i]));
        }
    }
}

// A wave's k-run is processed in batches of P pairs of k-steps; every load of
// a batch is issued, unconditionally, before the first is used (a load behind
// a branch, even a uniform one, makes the compiler's wait counts assume the
// worst and wait for loads issued later). The launcher picks P from the run's
// length (linear_pairs), so few loads fall past the run.
// NM: 0 no norm, 1 the row norm with its weight applied to the operand, 2 the
// row norm folded (the weight is in W; the row scale multiplies the product).
template <int RT, int CT, int P, int NM>
__global__ __launch_bounds__(512) void linear_rows_kernel(LinearParams p) {
    constexpr bool NORM = NM != 0;
    constexpr int TM = 16 * RT, TN = 16 * CT, OUT = TM * TN, R = (OUT + 511) / 512;
    constexpr int U = 2 * P;  // k-steps per batch
    static_assert(P >= 1 && P <= lin_pairs(RT, CT), "loads in flight per lane");
    constexpr int STAGE = (TM + TN) * LIN_STRIDE;  // one wave's staging region: x rows, then W rows
    constexpr int PART = 8 * TM * (TN + 1) * 4;    // the eight waves' partial tiles, after the product
    constexpr int LDS = 8 * STAGE > PART ? 8 * STAGE : PART;
    __shared__ __align__(16) char lds[LDS];
    float(*part)[TM][TN + 1] = reinterpret_cast<float(*)[TM][TN + 1]>(lds);
    __shared__ float sq[NORM ? 8 : 1][NORM ? TM : 1];
    __shared__ float4 snw[NM == 1 ? LINEAR_NORM_MAX_K / 4 : 1];
    __shared__ float srs[NM == 2 ? TM : 1];  // folded norm: the row scales
    // The wave index comes from a scalar register, so the k-run bounds and
    // every `s + u < s1` test are uniform branches. With a lane-divergent test
    // the compiler left one MFMA of the fused-norm variant to run under an
    // empty exec mask instead of branching around it, and outputs of that
    // build picked up stale operand registers (NaNs on MI355X).
    // Block ids: the tiles (N tile fastest), then the prefetch workgroups.
    const int tiles = p.grid_x * p.grid_y;
    if ((int)blockIdx.x >= tiles) {
        lin_prefetch(p, (int)blockIdx.x - tiles, (int)gridDim.x - tiles, tiles);
        return;
    }
    const int bx = __builtin_amdgcn_readfirstlane((int)blockIdx.x % p.grid_x),
              by = __builtin_amdgcn_readfirstlane((int)blockIdx.x / p.grid_x);
    const int n0 = bx * TN, m0 = by * TM;
    if (n0 >= p.N) return;  // padding of grid_x
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lr = lane & 15,
              lg = lane >> 4;
    char* const xreg = lds + w * STAGE;
    char* const wreg = xreg + TM * LIN_STRIDE;
    const int mrows = min(TM, p.M - m0);
    const lin_rsrc_t rx = lin_rsrc(p.x + (size_t)m0 * p.ldx, ((size_t)(mrows - 1) * p.ldx + p.K) * 2);
    const lin_rsrc_t rw = lin_rsrc(p.w + (size_t)n0 * p.K, (size_t)min(TN, p.N - n0) * p.K * 2);
    f32x4 acc[RT][CT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int c = 0; c < CT; c++) acc[rt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int steps = p.K / 32, per = (steps + 7) / 8;
    const int s0 = min(steps, w * per), s1 = min(steps, s0 + per);
    const uint32_t xrs = (uint32_t)p.ldx * 2, wrs = (uint32_t)p.K * 2;
    // the bias and the residual of this thread's outputs, loaded first (a null
    // pointer gets an empty buffer: every load of it reads zero)
    const lin_rsrc_t rb = lin_rsrc(p.bias, p.bias ? (size_t)p.N * 2 : 0);
    const lin_rsrc_t ra =
        lin_rsrc(p.add ? p.add + (size_t)m0 * p.ld_add : nullptr, p.add ? ((size_t)(mrows - 1) * p.ld_add + p.N) * 2 : 0);
    float bias[R], add[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int idx = threadIdx.x + 512 * r, n = n0 + idx % TN, m = idx / TN;
        const uint32_t dead = (idx < OUT && m < mrows) ? 0u : LIN_DEAD;
        bias[r] = bf16_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(rb, (uint32_t)n * 2, 0, 0));
        add[r] = bf16_bits_to_float(
            __builtin_amdgcn_raw_buffer_load_b16(ra, ((uint32_t)(m * p.ld_add + n) * 2) | dead, 0, 0));
    }
    if constexpr (!NORM) {
        for (int s = s0; s < s1; s += U) {
            u32x4 rawx[P][2 * RT], raww[P][2 * CT];
#pragma unroll
            for (int h = 0; h < P; h++) {
                lin_load_pair<RT>(rx, xrs, s + 2 * h, s1, lane, rawx[h]);
                lin_load_pair<CT>(rw, wrs, s + 2 * h, s1, lane, raww[h]);
            }
#pragma unroll
            for (int h = 0; h < P; h++) {
                if (s + 2 * h < s1) {
                    lin_stage_pair<RT>(xreg, lane, rawx[h]);
                    lin_stage_pair<CT>(wreg, lane, raww[h]);
#pragma unroll
                    for (int u = 0; u < 2; u++) {
                        if (s + 2 * h + u < s1) {
                            bf16x8 xf[RT], wf[CT];
#pragma unroll
                            for (int rt = 0; rt < RT; rt++) xf[rt] = lin_frag(xreg, rt, u, lr, lg);
#pragma unroll
                            for (int c = 0; c < CT; c++) wf[c] = lin_frag(wreg, c, u, lr, lg);
#pragma unroll
                            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                                for (int c = 0; c < CT; c++)
                                    acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rt], wf[c], acc[rt][c], 0, 0, 0);
                        }
                    }
                }
            }
        }
    } else {
        // The row norm (the launcher guarantees one batch: per <= U). Lane
        // (lr, lg) holds 8 columns of row 16 rt + lr per k-step, the same
        // columns in every tile shape. Its sum of squares runs over its
        // k-steps in order, then over the row's four lanes (xor 16, xor 32)
        // and the eight waves in wave order.
        // x and the norm weight first, then W: loads complete in order, so the
        // norm waits for x while W streams in. With four or more pairs (K =
        // 2048) only the first PW pairs of W are issued here and the rest once
        // x is in registers: all of a wave's run in flight at once takes more
        // than 128 VGPRs, and then one workgroup fits a CU instead of two (at
        // one row, the 1.4B model's gate|up launch of 352 workgroups ran in
        // two rounds on 256 CUs).
        constexpr int PW = P >= 4 ? P / 2 : P;
        u32x4 rawx[P][2 * RT], raww[P][2 * CT];
#pragma unroll
        for (int h = 0; h < P; h++) lin_load_pair<RT>(rx, xrs, s0 + 2 * h, s1, lane, rawx[h]);
        // the norm weight: K <= 2048, one float4 per thread (zero past K)
        float4 nwv = {};
        if constexpr (NM == 1)
            nwv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 lin_rsrc(p.norm_weight, (size_t)p.K * 4), 16 * threadIdx.x, 0, 0));
#pragma unroll
        for (int h = 0; h < PW; h++) lin_load_pair<CT>(rw, wrs, s0 + 2 * h, s1, lane, raww[h]);
        // Every pair is staged, also one past the run (its loads read zero):
        // with the staging under the run's test, the compiler moved the loads
        // of the first pair behind that branch and waited there for every
        // load in flight, W included.
        bf16x8 xf[U][RT];
#pragma unroll
        for (int h = 0; h < P; h++) {
            lin_stage_pair<RT>(xreg, lane, rawx[h]);
#pragma unroll
            for (int u = 0; u < 2; u++)
                if (s0 + 2 * h + u < s1)
#pragma unroll
                    for (int rt = 0; rt < RT; rt++) xf[2 * h + u][rt] = lin_frag(xreg, rt, u, lr, lg);
        }
#pragma unroll
        for (int h = PW; h < P; h++) lin_load_pair<CT>(rw, wrs, s0 + 2 * h, s1, lane, raww[h]);
        if constexpr (NM == 1) snw[threadIdx.x] = nwv;
        float ss[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            ss[rt] = 0.f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < s1) {
                    if constexpr (NM == 1) {
#pragma unroll
                        for (int e = 0; e < 8; e++) ss[rt] = fmaf((float)xf[u][rt][e], (float)xf[u][rt][e], ss[rt]);
                    } else {  // bf16 pairs on the dot product
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const bf16x2 x2 = {xf[u][rt][2 * e], xf[u][rt][2 * e + 1]};
                            ss[rt] = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, ss[rt], false);
                        }
                    }
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
            if constexpr (NM == 2) {  // the operand stays s; the scale goes to the epilogue
                if (w == 0 && lg == 0) srs[16 * rt + lr] = rs;
                continue;
            }
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
#pragma unroll
        for (int h = 0; h < P; h++) {
            if (s0 + 2 * h < s1) {
                lin_stage_pair<CT>(wreg, lane, raww[h]);
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    if (s0 + 2 * h + u < s1) {
                        bf16x8 wf[CT];
#pragma unroll
                        for (int c = 0; c < CT; c++) wf[c] = lin_frag(wreg, c, u, lr, lg);
#pragma unroll
                        for (int rt = 0; rt < RT; rt++)
#pragma unroll
                            for (int c = 0; c < CT; c++)
                                acc[rt][c] =
                                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[2 * h + u][rt], wf[c], acc[rt][c], 0, 0, 0);
                    }
                }
            }
        }
    }
    __syncthreads();  // the partial tiles overwrite the staging regions
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
            const float sc = NM == 2 ? srs[m] : 1.f;
            const float gf = (float)(bf16_t)(sg * sc), uf = (float)(bf16_t)(su * sc);
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
            if constexpr (NM == 2) s *= srs[m];
            float v = s + bias[r];
            if (p.add) v = (float)(bf16_t)v + add[r];  // the block's residual add, x + bf16(y)
            if (m < mrows && n0 + n < p.N) p.y[(size_t)(m0 + m) * p.ldy + n0 + n] = (bf16_t)v;
        }
    }
}

// ---------------------------------------------------------------------------
// One-row projections (M == 1, K >= 512: the projections of a B = 1 decode
// step) with linear_rows_kernel's epilogues: the fused pre-norm (NM 1), the
// SwiGLU pairing of interleaved gate and up rows, the bias and the residual
// add. For one row the MFMA kernel uses one of the sixteen rows of each
// operand block and stages every byte of W through LDS; here each wave
// streams RW rows of W from memory with 16-byte loads and forms the dot
// products on v_dot2_f32_bf16. Lane l covers elements 512 c + 8 l .. + 7 of
// chunk c. W is read once, with the non-temporal hint, so that its stream does
// not displace the cache lines other kernels are about to reuse (the decode
// step's prefetched state and weights, x). The workgroup's four waves share
// one copy of x (normalised with the norm) in LDS, so each compute unit's
// memory pipeline carries x once per workgroup rather than once per wave.
// Every load is issued at once, x first, then the norm weight, then all of W
// (D chunks per row: 4 for K <= 2048, always with the norm, 12 up to K =
// 6144), so that the norm waits for x alone while W streams in. Each row's
// sum runs over the chunks
// in order on the lane, then across the wave in wave_sum's fixed order: an
// order other than linear_rows_kernel's, which can move an output across a
// bf16 rounding boundary; every launch of a given shape takes the same path.
template <int RW, int NM, bool SWIGLU, int D>
__global__ __launch_bounds__(256) void gemv_row_kernel(LinearParams p) {
    static_assert(!SWIGLU || RW % 2 == 0, "SwiGLU pairs gate and up rows");
    static_assert(NM == 0 || D == 4, "the norm needs the whole row in one batch (K <= 2048)");
    constexpr int F = SWIGLU ? RW / 2 : RW;  // outputs per wave
    constexpr int XP = D / 4;                // x pieces of 8 elements per thread (K <= 512 D = 2048 XP)
    __shared__ bf16x8 s_x[64 * D];           // the row (normalised with NM 1), piece e = elements 8 e ..
    __shared__ float s_ss[4];
    const int tid = threadIdx.x, lane = tid & 63, wl = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = blockIdx.x * 4 + wl;
    const int K = p.K, N = p.N, nch = (K + 511) / 512;  // nch <= D: one batch
    // this wave's W rows: SWIGLU, F gate rows 32 g + f0 .. and the matching up
    // rows 32 g + 16 + f0 .. of group g (16 outputs per group)
    int rows[RW];
    const int per_group = 16 / F, g = wave / per_group, f0 = (wave % per_group) * F;
    if constexpr (SWIGLU) {
#pragma unroll
        for (int i = 0; i < F; i++) {
            rows[i] = 32 * g + f0 + i;
            rows[F + i] = 32 * g + 16 + f0 + i;
        }
    } else {
#pragma unroll
        for (int i = 0; i < RW; i++) rows[i] = RW * wave + i;
    }
    lin_rsrc_t rw[RW];
#pragma unroll
    for (int i = 0; i < RW; i++)
        rw[i] = lin_rsrc(rows[i] < N ? p.w + (size_t)rows[i] * K : nullptr, rows[i] < N ? (size_t)K * 2 : 0);
    const lin_rsrc_t rx = lin_rsrc(p.x, (size_t)K * 2);
    const lin_rsrc_t rn = lin_rsrc(NM == 1 ? p.norm_weight : nullptr, NM == 1 ? (size_t)K * 4 : 0);
    // chunk c's 16-byte piece of this lane, or LIN_DEAD past K (K % 8 == 0:
    // a lane's eight elements are all inside or all outside)
    const auto piece = [&](int c) {
        const int k = 512 * c + 8 * lane;
        return ((uint32_t)k * 2) | (c < nch && k < K ? 0u : LIN_DEAD);
    };
    // lane i < RW: the bias and the residual of row RW wave + i, loaded first
    // (a null pointer gets an empty buffer: its loads read zero)
    float bias_l = 0.f, add_l = 0.f;
    if constexpr (!SWIGLU) {
        const int r = RW * wave + lane;
        const uint32_t off = ((uint32_t)r * 2) | (lane < RW && r < N ? 0u : LIN_DEAD);
        bias_l = bf16_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(lin_rsrc(p.bias, p.bias ? (size_t)N * 2 : 0), off, 0, 0));
        add_l = bf16_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(lin_rsrc(p.add, p.add ? (size_t)N * 2 : 0), off, 0, 0));
    }
    // The workgroup's four waves share one copy of the row in LDS: thread t
    // loads pieces t + 256 i (and their norm weights), then W is issued.
    bf16x8 xp[XP];
    float4 na[NM == 1 ? XP : 1], nb[NM == 1 ? XP : 1];
#pragma unroll
    for (int i = 0; i < XP; i++) {
        const int e = tid + 256 * i;
        const uint32_t dead = 8 * e < K ? 0u : LIN_DEAD;
        xp[i] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rx, ((uint32_t)e * 16) | dead, 0, 0));
        if constexpr (NM == 1) {
            na[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rn, ((uint32_t)e * 32) | dead, 0, 0));
            nb[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rn, ((uint32_t)e * 32 + 16) | dead, 0, 0));
        }
    }
    u32x4 wv[D][RW];
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int i = 0; i < RW; i++)
            wv[d][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw[i], piece(d), 0, 2));
    // every load is issued before any is used: without the barrier the
    // scheduler interleaves loads and uses to save registers and keeps only a
    // few loads in flight
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NM == 1) {
        // rsqrt(mean x^2 + eps) over the row: each thread's pieces in order,
        // the wave's lanes (wave_sum), then the four waves in order; then
        // bf16(x rs w), as the separate norm rounds it
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < XP; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bf16x2 x2 = {xp[i][2 * e], xp[i][2 * e + 1]};
                ss = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, ss, false);
            }
        ss = wave_sum(ss);
        if (lane == 0) s_ss[wl] = ss;
        __syncthreads();
        const float rs = rsqrtf((((s_ss[0] + s_ss[1]) + s_ss[2]) + s_ss[3]) / (float)K + p.norm_eps);
#pragma unroll
        for (int i = 0; i < XP; i++) {
            const float wn[8] = {na[i].x, na[i].y, na[i].z, na[i].w, nb[i].x, nb[i].y, nb[i].z, nb[i].w};
#pragma unroll
            for (int e = 0; e < 8; e++) xp[i][e] = (bf16_t)((float)xp[i][e] * rs * wn[e]);
        }
    }
#pragma unroll
    for (int i = 0; i < XP; i++) s_x[tid + 256 * i] = xp[i];
    __syncthreads();
    float acc[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) acc[i] = 0.f;
#pragma unroll
    for (int d = 0; d < D; d++) {
        const bf16x8 xs = s_x[64 * d + lane];
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const bf16x8 wr = __builtin_bit_cast(bf16x8, wv[d][i]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bf16x2 a2 = {xs[2 * e], xs[2 * e + 1]}, b2 = {wr[2 * e], wr[2 * e + 1]};
                acc[i] = __builtin_amdgcn_fdot2_f32_bf16(a2, b2, acc[i], false);
            }
        }
    }
    float tot[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) tot[i] = wave_sum(acc[i]);
    if constexpr (SWIGLU) {
#pragma unroll
        for (int i = 0; i < F; i++) {
            if (lane == i && rows[i] < N) {
                const float gf = (float)(bf16_t)tot[i], uf = (float)(bf16_t)tot[F + i];
                p.y[16 * g + f0 + i] = (bf16_t)(gf * sigmoidf(gf) * uf);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            if (lane == i && rows[i] < N) {
                float v = tot[i] + bias_l;
                if (p.add) v = (float)(bf16_t)v + add_l;  // the block's residual add, x + bf16(y)
                p.y[rows[i]] = (bf16_t)v;
            }
        }
    }
}

// Whether a call takes the one-row form: one row, 512 <= K <= 6144 (K = 256,
// g_proj[1]'s, stays on the tile kernel, whose summation order the decode
// kernel's in-kernel gate repeats), not the folded norm.
static bool gemv_applies(int M, int N, int K, bool swiglu, bool folded) {
    return M == 1 && K >= 512 && K <= 12 * 512 && !folded && (!swiglu || N % 32 == 0);
}

// Workgroups of the one-row form with RW rows per wave (four waves each).
static unsigned gemv_workgroups(int N, bool swiglu, int rw) {
    const long long waves = swiglu ? (long long)(N / 32) * (16 / (rw / 2)) : (N + rw - 1) / rw;
    return (unsigned)((waves + 3) / 4);
}

// RW for a call: the most rows per wave that still give 256 or more
// workgroups (SwiGLU: always 4, a gate and an up pair per output pair).
static int gemv_rows_per_wave(int N, bool swiglu) {
    if (swiglu || gemv_workgroups(N, false, 4) >= 256) return 4;
    return gemv_workgroups(N, false, 2) >= 256 ? 2 : 1;
}

// The one-row form for a call; D chunks per batch.
template <int NM, bool SWIGLU, int D>
static void launch_gemv(const LinearParams& p, hipStream_t stream) {
    const int rw = gemv_rows_per_wave(p.N, SWIGLU);
    const dim3 grid(gemv_workgroups(p.N, SWIGLU, rw)), block(256);
    if (rw == 4) {
        hipLaunchKernelGGL((gemv_row_kernel<4, NM, SWIGLU, D>), grid, block, 0, stream, p);
    } else if constexpr (!SWIGLU) {
        if (rw == 2)
            hipLaunchKernelGGL((gemv_row_kernel<2, NM, false, D>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((gemv_row_kernel<1, NM, false, D>), grid, block, 0, stream, p);
    }
}

// ---------------------------------------------------------------------------
// Prefill gate path (layers/cyfa.py:292-295, 323-326, 349): the layer's
// g_proj[0], a|b|d projections, gate activations and g_proj[1] for 64 token
// rows per workgroup, 512 threads, in place of four launches that each read
// the rows again. Every operand streams in chunks of 64 k (one 128-byte line
// per row) as whole-line loads into a ring of three register sets, three
// chunks ahead; chunk c + 1 is written to one of two LDS buffers while chunk c
// is multiplied from the other, with one barrier per chunk. In LDS, 16-byte
// piece p of row r sits at piece p ^ (r & 7) of the row, so that the sixteen
// rows of an MFMA operand read spread over the banks.
// Stage 1 forms c = x [W_g0 | W_abd]^T: wave w owns g_proj[0] columns
// 32 w .. + 31 of all 64 rows (eight accumulator blocks) and, for w < 4 AB,
// abd block w >> 2 of row block w & 3. g0 is rounded to bf16 and passed
// through LDS into registers, the A operand of every stage-2 product.
// Stage 2 forms gate = g0 W_g1^T + b in rounds of 256 columns (wave w: round
// columns 32 w .. + 31); each wave writes its tile through its own LDS region
// as 16-byte pieces. Rows of x at or past M read as zero (buffer bounds) and
// are not stored. Every product accumulates in fp32 over k in order and is
// rounded to bf16 once, as the separate projections round it; the gates use
// gates_kernel's formula on the rounded a|b|d values.
// The chunk sequences are written out (gp_unrolled): each ring slot is a
// fixed set of registers, and no loop back edge remains (around one the
// compiler waits for every load in flight).
constexpr int GP_ROWS = 64;
constexpr int GP_ROUND = 256;  // gate columns per stage-2 round
constexpr int GP_MAX_CHUNKS = GATE_PATH_MAX_K / 64;
constexpr int GP_MAX_Q = 4 * (GATE_PATH_MAX_DV / GP_ROUND);  // stage-2 chunks: 4 per round

template <int AB>
struct GpLayout {
    static constexpr int NW1 = GATE_PATH_G0 + 16 * AB;   // stage-1 weight rows
    static constexpr int NWL = (NW1 + 63) / 64;          // weight loads per thread per chunk (8 rows per wave load)
    static constexpr int BUF = (GP_ROWS + 64 * NWL) * 128;  // one stage-1 buffer: x rows, then weight rows
    static_assert(GP_ROUND * 128 <= BUF && GP_ROWS * GATE_PATH_G0 * 2 <= BUF, "stage 2 fits a buffer");
};
constexpr int GP_OT = 8 * 16 * 64;  // per-wave output tiles: 16 rows x 32 columns of bf16
static_assert(2 * GpLayout<2>::BUF + GP_OT + GATE_PATH_MAX_DV * 2 <= 160 * 1024, "gate-path LDS");

// The MFMA operand piece of row R, k-step h of the chunk: k = 32 h + 8 lg .. + 7.
__device__ __forceinline__ bf16x8 gp_frag(const char* buf, int R, int h, int lg) {
    return *reinterpret_cast<const bf16x8*>(buf + R * 128 + 16 * ((4 * h + lg) ^ (R & 7)));
}

// f(integral_constant<int, i>) for i = C .. n - 1 (n <= MAX), written out.
template <int C, int MAX, typename F>
__device__ __forceinline__ void gp_unrolled(int n, F&& f) {
    if constexpr (C < MAX) {
        if (C >= n) return;
        f(std::integral_constant<int, C>{});
        gp_unrolled<C + 1, MAX>(n, f);
    }
}

template <int AB>
__global__ __launch_bounds__(512) void gate_path_kernel(GatePathParams p) {
    using L = GpLayout<AB>;
    constexpr int NWL = L::NWL;
    __shared__ __align__(16) char buf[2][L::BUF];
    __shared__ __align__(16) char sot[GP_OT];
    __shared__ __align__(16) bf16_t sbias[GATE_PATH_MAX_DV];  // 512 threads x 4
    static_assert(GATE_PATH_MAX_DV == 4 * 512, "one 8-byte bias load per thread");
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6), lr = lane & 15,
              lg = lane >> 4;
    const int m0 = blockIdx.x * GP_ROWS, mrows = min(GP_ROWS, p.M - m0);
    const int H = p.H, N1 = GATE_PATH_G0 + 3 * H;
    const lin_rsrc_t rx = lin_rsrc(p.x + (size_t)m0 * p.ldx, ((size_t)(mrows - 1) * p.ldx + p.K) * 2);
    const lin_rsrc_t rw1 = lin_rsrc(p.w1, (size_t)N1 * p.K * 2);  // rows past N1 read zero
    const lin_rsrc_t rw2 = lin_rsrc(p.w2, (size_t)p.Dv * GATE_PATH_G0 * 2);
    const uint32_t xrs = (uint32_t)p.ldx * 2, krs = (uint32_t)p.K * 2;
    // a load lane's row within its group of eight, the piece it fetches and
    // where that piece goes in LDS
    const int r8 = lane >> 3, pl = lane & 7, ps = 16 * (pl ^ r8);

    // the gate inputs of this thread's abd column and the g_proj[1] bias (into
    // LDS; past Dv: zero), loaded first
    const int ab_rb = w & 3, ab_cb = w >> 2;
    const lin_rsrc_t rab = lin_rsrc(p.abd_bias, (size_t)3 * H * 2);
    const int acol = 16 * ab_cb + lr, ah = acol % H, akind = acol / H;
    const float abias = bf16_bits_to_float(__builtin_amdgcn_raw_buffer_load_b16(rab, (uint32_t)acol * 2, 0, 0));
    const float adt = p.dt_bias[ah], aal = p.A_log[ah];  // ah < H for every lane
    {
        const lin_rsrc_t rb2 = lin_rsrc(p.b2, p.b2 ? (size_t)p.Dv * 2 : 0);
        *reinterpret_cast<u32x2*>(sbias + 4 * tid) =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rb2, 8 * tid, 0, 0));
    }

    // ---- stage 1: c = x [W_g0 | W_abd]^T ----
    const int nc = p.K / 64;
    u32x4 r1[3][1 + NWL];  // ring: x piece, then the weight pieces (rows 64 i + 8 w + r8)
    const auto issue1 = [&](int c, u32x4 (&r)[1 + NWL]) {
        const uint32_t dead = ((uint32_t)(c - nc) & LIN_DEAD) ^ LIN_DEAD;  // chunks past K read zero
        const uint32_t col = ((uint32_t)c * 128 + 16 * pl) | dead;
        r[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(8 * w + r8) * xrs + col, 0, 0));
#pragma unroll
        for (int i = 0; i < NWL; i++)
            r[1 + i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw1, (uint32_t)(64 * i + 8 * w + r8) * krs + col, 0, 0));
    };
    const auto store1 = [&](char* b, const u32x4 (&r)[1 + NWL]) {
        *reinterpret_cast<u32x4*>(b + (8 * w + r8) * 128 + ps) = r[0];
#pragma unroll
        for (int i = 0; i < NWL; i++) *reinterpret_cast<u32x4*>(b + (GP_ROWS + 64 * i + 8 * w + r8) * 128 + ps) = r[1 + i];
    };
    f32x4 acc[4][2], accab = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int rb = 0; rb < 4; rb++) acc[rb][0] = acc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    issue1(0, r1[0]);
    issue1(1, r1[1]);
    issue1(2, r1[2]);
    store1(buf[0], r1[0]);
    issue1(3, r1[0]);
    gp_unrolled<0, GP_MAX_CHUNKS>(nc, [&](auto cc) {
        constexpr int c = decltype(cc)::value;
        __syncthreads();  // chunk c is in buf[c & 1]; buf[(c + 1) & 1] is read by no one
        const char* b = buf[c & 1];
        store1(buf[(c + 1) & 1], r1[(c + 1) % 3]);
        issue1(c + 4, r1[(c + 1) % 3]);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            bf16x8 xf[4], wf[2];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) xf[rb] = gp_frag(b, 16 * rb + lr, h, lg);
#pragma unroll
            for (int cb = 0; cb < 2; cb++) wf[cb] = gp_frag(b, GP_ROWS + 32 * w + 16 * cb + lr, h, lg);
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[rb], wf[cb], acc[rb][cb], 0, 0, 0);
            if (w < 4 * AB) {  // uniform; LDS reads only
                const bf16x8 xa = gp_frag(b, 16 * ab_rb + lr, h, lg);
                const bf16x8 wa = gp_frag(b, GP_ROWS + GATE_PATH_G0 + 16 * ab_cb + lr, h, lg);
                accab = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, wa, accab, 0, 0, 0);
            }
        }
    });

    // ---- stage 2: gate = g0 W_g1^T + b, 256 columns per round ----
    const int nq = 4 * (p.Dv / GP_ROUND);  // chunk q: round q >> 2, k chunk q & 3
    u32x4 r2[3][4];  // ring: W_g1 rows 256 (q >> 2) + 64 i + 8 w + r8 (rounds past Dv read zero)
    const auto issue2 = [&](int q, u32x4 (&r)[4]) {
        const int n0 = GP_ROUND * (q >> 2);
        const uint32_t dead = ((uint32_t)(n0 - p.Dv) & LIN_DEAD) ^ LIN_DEAD;
        const uint32_t col = ((uint32_t)(q & 3) * 128 + 16 * pl) | dead;
#pragma unroll
        for (int i = 0; i < 4; i++)
            r[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rw2, (uint32_t)(n0 + 64 * i + 8 * w + r8) * (GATE_PATH_G0 * 2) + col, 0, 0));
    };
    const auto store2 = [&](char* b, const u32x4 (&r)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4*>(b + (64 * i + 8 * w + r8) * 128 + ps) = r[i];
    };
    issue2(0, r2[0]);
    issue2(1, r2[1]);
    issue2(2, r2[2]);
    __syncthreads();  // every wave is done with the stage-1 buffers
    // g0 in bf16 into buf[1] (row r: 512 bytes, four lines of 64 k)
    char* g0b = buf[1];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int row = 16 * rb + 4 * lg + i, col = 32 * w + 16 * cb + lr;
                *reinterpret_cast<bf16_t*>(g0b + row * 512 + (col >> 6) * 128 + 16 * (((col >> 3) & 7) ^ (row & 7)) +
                                           2 * (col & 7)) = (bf16_t)acc[rb][cb][i];
            }
    // the gates of the abd block: lane column 16 ab_cb + lr, rows 16 ab_rb + 4 lg + i
    if (w < 4 * AB && acol < 3 * H) {
        float* dst = akind == 0 ? p.g : akind == 1 ? p.beta : p.delta;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = 16 * ab_rb + 4 * lg + i;
            const float v = (float)(bf16_t)(accab[i] + abias);
            if (row < mrows) dst[(size_t)(m0 + row) * H + ah] = akind == 0 ? decay_gate(v + adt, aal) : sigmoidf(v);
        }
    }
    store2(buf[0], r2[0]);
    issue2(3, r2[0]);
    __syncthreads();  // g0 and the first W_g1 chunk in LDS
    // gf[rb][ks] = g0[16 rb + lr][32 ks + 8 lg .. + 7]
    bf16x8 gf[4][GATE_PATH_G0 / 32];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int ks = 0; ks < GATE_PATH_G0 / 32; ks++) {
            const int R = 16 * rb + lr;
            gf[rb][ks] =
                *reinterpret_cast<const bf16x8*>(g0b + R * 512 + (ks >> 1) * 128 + 16 * ((4 * (ks & 1) + lg) ^ (R & 7)));
        }
    f32x4 acc2[4][2];
    char* ot = sot + w * 1024;
    gp_unrolled<0, GP_MAX_Q>(nq, [&](auto qq) {
        constexpr int q = decltype(qq)::value, kq = q & 3;
        // chunk q is in buf[q & 1]; buf[(q + 1) & 1] (for q = 0: g0) is read by no one
        if constexpr (q > 0) __syncthreads();
        const char* b = buf[q & 1];
        if constexpr (q == 0) {
            __syncthreads();  // every wave holds its g0 operands
        }
        store2(buf[(q + 1) & 1], r2[(q + 1) % 3]);
        issue2(q + 4, r2[(q + 1) % 3]);
        if constexpr (kq == 0) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++) acc2[rb][0] = acc2[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            bf16x8 wf[2];
#pragma unroll
            for (int cb = 0; cb < 2; cb++) wf[cb] = gp_frag(b, 32 * w + 16 * cb + lr, h, lg);
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
                    acc2[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gf[rb][2 * kq + h], wf[cb], acc2[rb][cb], 0, 0, 0);
        }
        if constexpr (kq == 3) {  // the round's 64 x 32 tile, 16 rows at a time through the wave's LDS region
            constexpr int rd = q >> 2;
            const int n0 = GP_ROUND * rd + 32 * w;
            float bias[2];
#pragma unroll
            for (int cb = 0; cb < 2; cb++) bias[cb] = (float)sbias[n0 + 16 * cb + lr];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) {
#pragma unroll
                for (int cb = 0; cb < 2; cb++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        *reinterpret_cast<bf16_t*>(ot + (4 * lg + i) * 64 + 2 * (16 * cb + lr)) =
                            (bf16_t)(acc2[rb][cb][i] + bias[cb]);
                // a wave's LDS accesses complete in order; the compiler keeps these in order too
                asm volatile("" ::: "memory");
                const int row = 16 * rb + (lane >> 2);
                const u32x4 v = *reinterpret_cast<const u32x4*>(ot + (lane >> 2) * 64 + 16 * (lane & 3));
                asm volatile("" ::: "memory");
                if (row < mrows) *reinterpret_cast<u32x4*>(p.gate + (size_t)(m0 + row) * p.ldg + n0 + 8 * (lane & 3)) = v;
            }
        }
    });
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
    // The row as a buffer: a chunk of 8 not wholly inside it is loaded at the
    // LIN_DEAD offset (zeros, its elements are read one by one below), so the
    // loads sit behind no branch and all of them are in flight together.
    const lin_rsrc_t r = lin_rsrc(xr, (size_t)n * 2);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int base = 0; base < n; base += 8 * NT * DEPTH) {
        bf16x8 v[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; d++) {
            const int i0 = base + 8 * (threadIdx.x + NT * d);
            const uint32_t dead = i0 + 8 <= n ? 0u : LIN_DEAD;
            v[d] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, ((uint32_t)i0 * 2) | dead, 0, 0));
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
    // The wave's best (value, index): the comparison is associative and
    // commutative, so any reduction order gives the same pair. DPP within rows
    // of 16 lanes, then the four rows through v_readlane (no LDS round trips).
    const auto take = [&](float ov, int oi) {
        if (argmax_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    };
    take(dpp_mov<0xB1>(bv), __builtin_amdgcn_mov_dpp(bi, 0xB1, 0xF, 0xF, true));
    take(dpp_mov<0x4E>(bv), __builtin_amdgcn_mov_dpp(bi, 0x4E, 0xF, 0xF, true));
    take(dpp_mov<0x141>(bv), __builtin_amdgcn_mov_dpp(bi, 0x141, 0xF, 0xF, true));
    take(dpp_mov<0x140>(bv), __builtin_amdgcn_mov_dpp(bi, 0x140, 0xF, 0xF, true));
#pragma unroll
    for (int r = 1; r < 4; r++) take(lane_value(bv, 16 * r), __builtin_amdgcn_readlane(bi, 16 * r));
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
    g[i] = decay_gate((float)row[h] + dt_bias[h], A_log[h]);
    beta[i] = sigmoidf((float)row[H + h]);
    delta[i] = sigmoidf((float)row[2 * H + h]);
}

// s = bf16(x + residual) for the fused norm's rows (M rows of K columns, K a
// multiple of 32), written to s rows ldr apart; one thread per 8 columns.
__global__ __launch_bounds__(256) void add_rows_kernel(const bf16_t* x, long long ldx, const bf16_t* r, long long ldr,
                                                       bf16_t* s, int K) {
    const int c = 8 * (blockIdx.x * 256 + threadIdx.x), m = blockIdx.y;
    if (c >= K) return;
    const bf16x8 xv = *reinterpret_cast<const bf16x8*>(x + (size_t)m * ldx + c);
    const bf16x8 rv = *reinterpret_cast<const bf16x8*>(r + (size_t)m * ldr + c);
    bf16x8 sv;
#pragma unroll
    for (int e = 0; e < 8; e++) sv[e] = (bf16_t)((float)xv[e] + (float)rv[e]);
    *reinterpret_cast<bf16x8*>(s + (size_t)m * ldr + c) = sv;
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

// linear_rows_kernel<RT, CT, P, NM> for P pairs per batch, rounded up to
// an instantiated count (1, 2, 3, 4, 6) within the shape's limit.
template <int RT, int CT, int NM>
static void launch_rows(const LinearParams& p, int pairs, dim3 grid, hipStream_t stream) {
    constexpr int cap = lin_pairs(RT, CT);
    const dim3 block(512);
    if (pairs <= 1) {
        hipLaunchKernelGGL((linear_rows_kernel<RT, CT, 1, NM>), grid, block, 0, stream, p);
    } else if (pairs == 2 || cap == 2) {
        hipLaunchKernelGGL((linear_rows_kernel<RT, CT, 2, NM>), grid, block, 0, stream, p);
    } else if constexpr (cap >= 3) {
        if (pairs == 3 || cap == 3) {
            hipLaunchKernelGGL((linear_rows_kernel<RT, CT, 3, NM>), grid, block, 0, stream, p);
        } else if constexpr (cap >= 4) {
            if (pairs == 4 || cap == 4)
                hipLaunchKernelGGL((linear_rows_kernel<RT, CT, 4, NM>), grid, block, 0, stream, p);
            else if constexpr (cap >= 6)
                hipLaunchKernelGGL((linear_rows_kernel<RT, CT, 6, NM>), grid, block, 0, stream, p);
        }
    }
}

// The tile shape of linear_rows_kernel for one call. Each workgroup reads
// 16 (RT + CT) rows of K (RT x 16 rows of x and CT x 16 rows of W), and at
// these sizes a CU's read rate, not the chip's, is the limit; one workgroup
// fits a CU at a time, so the workgroups past the first 256 run in further
// rounds. Pick the shape with the least bytes read per CU over all rounds
// (on MI355X: 28 -> 35 k tok/s for the 400M decode step at B=64 against a
// fixed 4 x 2 tile). The SwiGLU epilogue needs CT = 2, the 16 gate and 16 up
// columns of one interleaved group; the row norm needs each wave's k-steps in
// one batch of loads (K <= 512 lin_pairs). False when no shape qualifies.
static bool linear_tile(int M, int N, bool swiglu, int norm_k, int& rt_out, int& ct_out) {
    static const int shapes[][2] = {{4, 4}, {4, 2}, {2, 4}, {4, 1}, {2, 2}, {1, 4}, {2, 1}, {1, 2}, {1, 1}};
    long long best = -1;
    rt_out = 4;
    ct_out = 2;
    for (const auto& sh : shapes) {
        const int rt = sh[0], ct = sh[1];
        if (swiglu && ct != 2) continue;
        if (norm_k && rt * ct > 8) continue;  // no fused-norm build of the 64 x 64 tile (its registers would spill)
        if (norm_k > 512 * lin_pairs(rt, ct)) continue;  // the norm needs all of a row in one batch
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

unsigned long long linear_rows_span(int M, int N, int K, bool swiglu, int norm) {
    if (M < 1 || M > 64 || N < 1 || K < 32 || K % 32 || (norm && K > LINEAR_NORM_MAX_K) || (swiglu && N % 32))
        return 0;
    if (gemv_applies(M, N, K, swiglu, norm == 2))  // wave w reads rows RW w ..; SwiGLU's rows come in pieces
        return swiglu ? 0 : 4ull * gemv_rows_per_wave(N, false) * K * 2;
    int rt, ct;
    if (!linear_tile(M, N, swiglu, norm ? K : 0, rt, ct)) return 0;
    // the workgroups of N tile x read W rows 16 ct x ..; they run on XCD x mod 8
    // (block ids x + grid_x y, grid_x a multiple of 8 when there are several row tiles)
    return 16ull * ct * K * 2;
}

// Prefetch workgroups of a projection launch: one per this many bytes of the
// ranges, or every compute unit the tiles leave idle if that is more. Measured
// on MI355X (400M decode steps, graphed; gate|up reading down's weight, down
// the next layer's input weight, o_proj gate|up's): B = 64 43.2 k -> 44.0 k
// tok/s, B = 48 34.4 k -> 35.3 k, B = 32 25.4 k -> 26.4 k; 32 KiB per
// workgroup gave the same, 16 KiB less (43.3 k at B = 64).
constexpr unsigned long long LINEAR_PF_BYTES_PER_WG = 64 << 10;

int launch_linear_rows(const LinearParams& p_in, hipStream_t stream) {
    LinearParams p = p_in;
    const bool norm = p.norm_weight != nullptr || p.norm_folded;
    if (p.M < 1 || p.M > 64 || (norm && p.K > LINEAR_NORM_MAX_K)) return -1;
    // every buffer the kernel reads spans less than LIN_DEAD bytes (so that
    // offset reads zero) and every in-buffer offset fits 32 bits
    const auto span = [&](long long ld, long long cols) { return ((unsigned long long)(p.M - 1) * ld + cols) * 2; };
    if (p.K > (1 << 20) || span(p.ldx, p.K) >= LIN_DEAD || (p.add && span(p.ld_add, p.N) >= LIN_DEAD) ||
        (p.norm_residual && span(p.ldr, p.K) >= LIN_DEAD) || (p.bias && (unsigned long long)p.N * 2 >= LIN_DEAD))
        return -1;
    if (norm && p.norm_residual) {
        // s = bf16(x + residual) first, into norm_sum_out; the norm and the
        // product then read s as x
        hipLaunchKernelGGL(add_rows_kernel, dim3((p.K / 8 + 255) / 256, p.M), dim3(256), 0, stream, p.x, p.ldx,
                           p.norm_residual, p.ldr, p.norm_sum_out, p.K);
        p.x = p.norm_sum_out;
        p.ldx = p.ldr;
        p.norm_residual = nullptr;
        p.norm_sum_out = nullptr;
    }
    if (gemv_applies(p.M, p.N, p.K, p.swiglu != 0, p.norm_folded != 0)) {
        // one batch of chunks for every K up to 6144 (the norm's K <= 2048)
        const bool short_k = p.K <= 4 * 512;
        if (p.swiglu) {
            if (norm)
                launch_gemv<1, true, 4>(p, stream);
            else if (short_k)
                launch_gemv<0, true, 4>(p, stream);
            else
                launch_gemv<0, true, 12>(p, stream);
        } else if (norm) {
            launch_gemv<1, false, 4>(p, stream);
        } else if (short_k) {
            launch_gemv<0, false, 4>(p, stream);
        } else {
            launch_gemv<0, false, 12>(p, stream);
        }
        return 0;
    }
    int rt, ct;
    if (!linear_tile(p.M, p.N, p.swiglu != 0, norm ? p.K : 0, rt, ct)) return -1;
    p.grid_x = (p.N + 16 * ct - 1) / (16 * ct);
    p.grid_y = (p.M + 16 * rt - 1) / (16 * rt);
    // with several row tiles, grid_x a multiple of 8, so that every workgroup
    // of N tile c runs on XCD c mod 8 (linear_rows_span)
    if (p.grid_y > 1) p.grid_x = (p.grid_x + 7) / 8 * 8;
    const int tiles = p.grid_x * p.grid_y;
    p.pf_wgs = 0;
    if (p.pf_bytes[0] || p.pf_bytes[1]) {
        // every idle compute unit, and at least one workgroup per 64 KiB
        const int idle = device_cu_count() - tiles;
        const unsigned long long units = (p.pf_bytes[0] + p.pf_bytes[1] + LINEAR_PF_BYTES_PER_WG - 1) / LINEAR_PF_BYTES_PER_WG;
        const int want = (int)(units < 512 ? units : 512);
        p.pf_wgs = idle > want ? idle : want;
    }
    const dim3 grid(tiles + p.pf_wgs);
    // k-step pairs per batch: the whole of a wave's run when the shape allows it
    const int per = (p.K / 32 + 7) / 8, pairs = min((per + 1) / 2, lin_pairs(rt, ct));
#define CYFA_LINEAR(RT_, CT_)                                                                                  \
    if (rt == RT_ && ct == CT_) {                                                                              \
        if (p.norm_folded)                                                                                     \
            launch_rows<RT_, CT_, 2>(p, pairs, grid, stream);                                                  \
        else if (norm)                                                                                         \
            launch_rows<RT_, CT_, 1>(p, pairs, grid, stream);                                                  \
        else                                                                                                   \
            launch_rows<RT_, CT_, 0>(p, pairs, grid, stream);                                                  \
        return 0;                                                                                              \
    }
    if (rt == 4 && ct == 4 && !norm) {  // the lm_head's tile at 64 rows (N = 32000: 500 workgroups)
        launch_rows<4, 4, 0>(p, pairs, grid, stream);
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
    if ((unsigned long long)n * 2 >= LIN_DEAD) return -1;  // a row's byte offsets stay below the dead offset
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, stream, x, ldx, n, out);
    return 0;
}

int launch_gate_path(const GatePathParams& p, hipStream_t stream) {
    const int ab = (3 * p.H + 15) / 16;
    if (p.M < 1 || p.K < 64 || p.K % 64 || p.K > GATE_PATH_MAX_K || p.H < 1 || ab > 2 || p.Dv < GP_ROUND ||
        p.Dv % GP_ROUND || p.Dv > GATE_PATH_MAX_DV)
        return -1;
    // every buffer the kernel reads spans less than 2^31 bytes (32-bit offsets, LIN_DEAD unused here)
    const unsigned long long xspan = ((unsigned long long)(min(p.M, GP_ROWS) - 1) * p.ldx + p.K) * 2;
    if ((unsigned long long)(GATE_PATH_G0 + 3 * p.H) * p.K * 2 >= LIN_DEAD || xspan >= LIN_DEAD ||
        (unsigned long long)p.Dv * GATE_PATH_G0 * 2 >= LIN_DEAD)
        return -1;
    const dim3 grid((p.M + GP_ROWS - 1) / GP_ROWS), block(512);
    if (ab == 1)
        hipLaunchKernelGGL(gate_path_kernel<1>, grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL(gate_path_kernel<2>, grid, block, 0, stream, p);
    return 0;
}

int launch_gates(const bf16_t* abd, long long abd_row, const float* dt_bias, const float* A_log, float* g, float* beta,
                 float* delta, int rows, int H, hipStream_t stream) {
    hipLaunchKernelGGL(gates_kernel, dim3((rows * H + 255) / 256), dim3(256), 0, stream, abd, abd_row, dt_bias, A_log, g,
                       beta, delta, rows, H);
    return 0;
}

}  // namespace cyfa
