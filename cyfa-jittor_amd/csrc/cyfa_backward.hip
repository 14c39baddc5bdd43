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
// general path's clock, write vector and readout; the states before every
// 64-token chunk of both passes and the pass-1 output from the kernels
// below), so the gradients are those of the op's exact arithmetic; every
// adjoint accumulates in fp32. Per pass (o = SGLA(q, k, v, g, S0, scale),
// in-chunk cumulative log-decay G):
//   D_n  = e^{G_last} D_{n+1} + scale sum_t e^{G_t} q_t (x) dO_t      (state cotangent, reverse over chunks)
//   dq_t = scale (e^{G_t} S_n dO_t + sum_{s<=t} e^{G_t-G_s} (dO_t.v_s) k_s)
//   dk_s = scale sum_{t>=s} e^{G_t-G_s} (dO_t.v_s) q_t + e^{G_last-G_s} D_{n+1} v_s
//   dv_s = scale sum_{t>=s} e^{G_t-G_s} (q_t.k_s) dO_t + e^{G_last-G_s} D_{n+1}^T k_s
//   dL/dG_t = q_t.dq_t - k_t.dk_t + [t = last] <D_{n+1}, S_{n+1}>,  dg = in-chunk reverse cumsum
// The states and their cotangents are one sweep per (state tile, b, h) that
// keeps its tile in registers; outputs and the rows' cotangents are then
// chunk-parallel, one workgroup per (chunk, h, b), with no reduction across
// workgroups. The readout adjoint runs per block of rows (z = U(lam) raw,
// softmax of table z, u = table^T p, weights = U(-lam) u) with the head's
// table and this workgroup's share of the table cotangent on chip (up to 128
// slots; above, as tile GEMMs that stream the table); partial sums (table,
// norm weights, per-tile boundary terms) are added in a fixed order, so the
// result does not depend on scheduling. With bf16 operands the scans' and
// chunk kernels' products and the recomputed readout's run on the matrix
// cores with every fp32 operand split into two bf16 parts (about 16 mantissa
// bits); with fp32 operands they are fp32 FMA loops, exact to fp32 rounding.
#include <cmath>
#include <type_traits>

#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int BC = 64;           // chunk length of the recompute and the sweeps
constexpr int BW_MAX_D = 1024;   // largest K and V
constexpr int BW_TILE = 32;      // state columns per scan workgroup
constexpr double kTwoPiBw = 6.283185307179586;

// Whole-wave sum and max in every lane, on DPP moves and v_readlane (the
// fixed order of wave_sum / wave_max); every call site has the whole wave
// active. (With __shfl_xor each step was an LDS round trip.)
__device__ __forceinline__ float bw_wave_sum(float x) { return wave_sum<64>(x); }

__device__ __forceinline__ float bw_wave_max(float x) { return wave_max<64>(x); }

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
// Inclusive sum over the wave's 64 lanes on DPP moves: shifts by 1, 2, 4 and
// 8 within rows of 16, then row 15's sum broadcast into the next row, and row
// 31's into the upper half (every lane active). (__shfl_up made each step an
// LDS round trip on the scans' serial path.)
template <int CTRL>
__device__ __forceinline__ float bw_dpp_shift(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float bw_wave_scan(float x) {
    x += bw_dpp_shift<0x111>(x);
    x += bw_dpp_shift<0x112>(x);
    x += bw_dpp_shift<0x114>(x);
    x += bw_dpp_shift<0x118>(x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x143, 0xC, 0xF, false));
    return x;
}

__device__ __forceinline__ float chunk_gam(const float* g, int b, int h, int T, int H, int n, int lane) {
    const int t = n * BC + lane;
    return bw_wave_scan(t < T ? g[((size_t)b * T + t) * H + h] : 0.f);
}

// Rows of x [B, T, H, D] into head-major fp32 [B*H, Tp, D]: with a norm
// weight the normalised row x rs w (ops/qk_norm.py:206-233, unrounded) and rs
// per row; without, x itself; x == nullptr or t >= T gives zeros. One wave per row.
// O: the rows' element type (bf16_t only without w: a bf16 x's layout change).
template <bool BF, class O = float>
__global__ __launch_bounds__(256) void bw_rows_kernel(const void* x, const float* w, float eps, int B, int T, int Tp,
                                                      int H, int D, O* out, float* rs_out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= B * H * Tp) return;
    const int t = row % Tp, bh = row / Tp, b = bh / H, h = bh % H;
    O* dst = out + (size_t)row * D;
    if (!x || t >= T) {
        for (int i = lane; i < D; i += 64) dst[i] = (O)0.f;
        if (rs_out && lane == 0) rs_out[row] = 0.f;
        return;
    }
    const size_t src = (((size_t)b * T + t) * H + h) * D;
    if (D == 256 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0) {
        // the tuned head size (16-byte aligned rows): four consecutive
        // elements per lane, one pass over x
        float v[4];
        if constexpr (BF) {
            const bf16x4 xv = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16_t*>(x) + src + 4 * lane);
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = (float)xv[e];
        } else {
            const float4 xv = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + src + 4 * lane);
            v[0] = xv.x, v[1] = xv.y, v[2] = xv.z, v[3] = xv.w;
        }
        float4 o = {v[0], v[1], v[2], v[3]};
        if (w) {
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 4; e++) ss = fmaf(v[e], v[e], ss);
            const float rs = rsqrtf(bw_wave_sum(ss) / (float)D + eps);
            const float4 wv = *reinterpret_cast<const float4*>(w + 4 * lane);
            o = float4{v[0] * rs * wv.x, v[1] * rs * wv.y, v[2] * rs * wv.z, v[3] * rs * wv.w};
            if (rs_out && lane == 0) rs_out[row] = rs;
        }
        if constexpr (std::is_same_v<O, bf16_t>)
            *reinterpret_cast<bf16x4*>(dst + 4 * lane) = bf16x4{(bf16_t)o.x, (bf16_t)o.y, (bf16_t)o.z, (bf16_t)o.w};
        else
            *reinterpret_cast<float4*>(dst + 4 * lane) = o;
        return;
    }
    if (!w) {
        for (int i = lane; i < D; i += 64) dst[i] = (O)bw_ld<BF>(x, src + i);
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

// Global accesses of the backward kernels go through buffer resources over
// regions below 2^31 bytes (a chunk's rows, one state), each out-of-range
// element predicated through its offset: no branch among the loads, at which
// the compiler would wait for every load in flight.
typedef __amdgpu_buffer_rsrc_t bw_rsrc_t;
constexpr uint32_t BW_DEAD = 0x80000000u;  // past every region below (each < 2^31 bytes)

__device__ __forceinline__ bw_rsrc_t bw_rsrc(const float* base, size_t elems) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)(uint32_t)(elems * 4), 0x00020000);
}
__device__ __forceinline__ bw_rsrc_t bw_rsrc(const bf16_t* base, size_t elems) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, (int)(uint32_t)(elems * 2), 0x00020000);
}

// A buffer store that the range check drops when dead is set.
__device__ __forceinline__ void bw_store(bw_rsrc_t r, uint32_t off, bool live, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off | (live ? 0u : BW_DEAD), 0, 0);
}
__device__ __forceinline__ float bw_load(bw_rsrc_t r, uint32_t off, bool live) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off | (live ? 0u : BW_DEAD), 0, 0));
}
// The same for one bf16 element (off in bytes): stored rounded, loaded widened.
__device__ __forceinline__ void bw_store_h(bw_rsrc_t r, uint32_t off, bool live, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16_t)v), r, off | (live ? 0u : BW_DEAD), 0,
                                          0);
}
__device__ __forceinline__ float bw_load_h(bw_rsrc_t r, uint32_t off, bool live) {
    const unsigned short u = __builtin_amdgcn_raw_buffer_load_b16(r, off | (live ? 0u : BW_DEAD), 0, 0);
    return __builtin_bit_cast(float, (uint32_t)u << 16);
}
__device__ __forceinline__ f32x4 bf16x4_bits_to_f32x4(uint32_t w0, uint32_t w1) {
    return f32x4{__builtin_bit_cast(float, w0 << 16), __builtin_bit_cast(float, w0 & 0xffff0000u),
                 __builtin_bit_cast(float, w1 << 16), __builtin_bit_cast(float, w1 & 0xffff0000u)};
}

// The chunk-to-chunk scan of one pass over a [Kq, Vd] matrix X, one
// SCAN_ROWS x 32 tile per workgroup (grid (ceil(Vd / 32), ceil(Kq /
// SCAN_ROWS), B*H), 256 threads, each holding SCAN_RPT x 4 elements of X in
// registers; every element's recurrence is independent of the others):
//   X <- e^{G_last} X + sum_t f_t a_t (x) b_t     (a rank-64 update per chunk)
// Forward (BWD false): the states, n = 0 .. N-1, X_0 = x0 (or zero),
//   f_t = e^{G_last - G_t}, a = k, b = v; xs[n] = the state before chunk n,
//   xs[N] the final state.
// Backward (BWD true): the state cotangents, n = N-1 .. 0, X_N = x0 (the
//   final state's cotangent, or zero), f_t = scale e^{G_t}, a = q, b = dO;
//   xs[n+1] = the cotangent after chunk n, xs[0] (and x_out) the initial
//   state's; bnd[tile][n] = the tile's part of <xs[n+1], S[n+1]>.
// Per chunk the f-scaled rows of a and the columns of b are staged in LDS
// (two broadcast reads of a and one float4 of b per token feed eight FMAs).
constexpr int SCAN_ROWS = BWD_SCAN_ROWS;    // rows of a scan tile
constexpr int SCAN_RPT = SCAN_ROWS / 32;    // rows per thread (8 threads across the 32 columns)
struct StateScanArgs {
    const float *a, *b;  // head-major [B*H, Tp, Kq] and [B*H, Tp, Vd]
    const float* g;      // [B, T, H]
    const float* x0;     // nullable [B*H, Kq, Vd]
    float* xs;           // [B*H, N+1, Kq, Vd]
    const float* S;      // backward: the forward states [B*H, N+1, Kq, Vd]
    float* bnd;          // backward: [B*H, ntiles, N], ntiles = ceil(Vd / 32) ceil(Kq / 64)
    float* x_out;        // nullable [B*H, Kq, Vd]
    int B, T, Tp, H, Kq, Vd, N;
    float scale;
    int sbf;             // matrix-core form: xs and S hold bf16 (bf16_t) states
    int bbf;             // matrix-core form: b holds bf16 (bf16_t) rows
};

template <bool BWD>
__global__ __launch_bounds__(256) void bw_state_scan_kernel(StateScanArgs p) {
    __shared__ float sA[BC][SCAN_ROWS + 4];
    __shared__ __align__(16) float sB[BC][BW_TILE];
    __shared__ float sF[BC];
    __shared__ float sRed[4];
    __shared__ float sEl;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int c0 = blockIdx.x * BW_TILE, r0 = blockIdx.y * SCAN_ROWS, bhi = blockIdx.z;
    const int b = bhi / p.H, h = bhi % p.H, tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int nt = gridDim.x * gridDim.y;
    const int Kq = p.Kq, Vd = p.Vd, N = p.N;
    const size_t bh = bhi, ssz = (size_t)Kq * Vd;
    float* xs = p.xs + bh * (N + 1) * ssz;
    const float* A = p.a + bh * p.Tp * Kq;
    const float* Bm = p.b + bh * p.Tp * Vd;
    // this thread's block: rows r0 + rr .. + SCAN_RPT; columns c0 + cc .. + 3
    const int rr = SCAN_RPT * (tid >> 3), cc = 4 * (tid & 7);
    // Every global access below goes through a buffer resource, predicated
    // through its offset (no branch among the loads); the states per chunk.
    bool ok[SCAN_RPT][4];
    uint32_t off[SCAN_RPT][4];  // byte offset of this thread's elements in a [Kq, Vd] state
    float x[SCAN_RPT][4];
    const bw_rsrc_t rx0 = bw_rsrc(p.x0 ? p.x0 + bh * ssz : nullptr, p.x0 ? ssz : 0);
#pragma unroll
    for (int i = 0; i < SCAN_RPT; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            ok[i][j] = r0 + rr + i < Kq && c0 + cc + j < Vd;
            off[i][j] = ((uint32_t)(r0 + rr + i) * (uint32_t)Vd + (uint32_t)(c0 + cc + j)) * 4u;
            x[i][j] = bw_load(rx0, off[i][j], ok[i][j]);  // zero without x0 (empty buffer)
        }
    // backward: the forward state S[n] of this thread's block, loaded a chunk
    // ahead (with the rows and columns below) for the boundary term <X, S[n]>
    float sv[SCAN_RPT][4] = {};
    const auto fetch_state = [&](int n) {
        const bw_rsrc_t rs = bw_rsrc(p.S + (bh * (N + 1) + n) * ssz, ssz);
#pragma unroll
        for (int i = 0; i < SCAN_RPT; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) sv[i][j] = bw_load(rs, off[i][j], ok[i][j]);
    };
    const auto keep = [&](int n) {  // xs[n] = X; returns the block's part of <X, S[n]> (backward)
        const bw_rsrc_t rs = bw_rsrc(xs + (size_t)n * ssz, ssz);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < SCAN_RPT; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bw_store(rs, off[i][j], ok[i][j], x[i][j]);
                if constexpr (BWD) dot = fmaf(x[i][j], sv[i][j], dot);  // sv is zero where !ok
            }
        return dot;
    };
    // The next chunk's rows of a, columns of b and gate are loaded into
    // registers while the current chunk's FMAs run.
    constexpr int NA = BC * SCAN_ROWS / 256, NB = BC * BW_TILE / 256;
    float ra[NA], rb[NB], rg = 0.f;
    // (the host keeps B T H below 2^21: the gate's offsets fit 32 bits)
    const bw_rsrc_t rgt = bw_rsrc(p.g, (size_t)p.B * p.T * p.H);
    const auto fetch = [&](int n) {
        const int t0 = n * BC;
        const bw_rsrc_t rA = bw_rsrc(A + (size_t)t0 * Kq, (size_t)BC * Kq), rBm = bw_rsrc(Bm + (size_t)t0 * Vd, (size_t)BC * Vd);
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int e = tid + 256 * i, t = e / SCAN_ROWS, r = e % SCAN_ROWS;
            ra[i] = bw_load(rA, ((uint32_t)t * (uint32_t)Kq + (uint32_t)(r0 + r)) * 4u, r0 + r < Kq);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int e = tid + 256 * i, t = e / BW_TILE, c = e % BW_TILE;
            rb[i] = bw_load(rBm, ((uint32_t)t * (uint32_t)Vd + (uint32_t)(c0 + c)) * 4u, c0 + c < Vd);
        }
        // (every wave loads the gate; wave 0 uses it)
        rg = bw_load(rgt, (((uint32_t)b * (uint32_t)p.T + (uint32_t)(t0 + lane)) * (uint32_t)p.H + (uint32_t)h) * 4u,
                     t0 + lane < p.T);
    };
    fetch(BWD ? N - 1 : 0);
    if constexpr (BWD) fetch_state(N);
    for (int step = 0; step < N; step++) {
        const int n = BWD ? N - 1 - step : step;
        const float dot = keep(BWD ? n + 1 : n);
        __syncthreads();  // the previous chunk's tiles are done with
        if constexpr (BWD) {
            const float wsum = bw_wave_sum(dot);
            if (lane == 0) sRed[wv] = wsum;
        }
        if (wv == 0) {  // G: the in-chunk inclusive cumsum of the prefetched gate
            const float G = bw_wave_scan(rg);
            const float Gl = lane_value(G, 63);
            sF[lane] = BWD ? p.scale * expf(G) : expf(Gl - G);
            if (lane == 0) sEl = expf(Gl);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int e = tid + 256 * i;
            sB[e / BW_TILE][e % BW_TILE] = rb[i];
        }
        __syncthreads();  // sF is read below
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int e = tid + 256 * i, t = e / SCAN_ROWS;
            sA[t][e % SCAN_ROWS] = sF[t] * ra[i];
        }
        __syncthreads();
        if (step + 1 < N) fetch(BWD ? n - 1 : n + 1);
        if constexpr (BWD) fetch_state(n);  // for the next step's keep(n)
        if constexpr (BWD) {
            if (tid == 0) p.bnd[(bh * nt + tile) * N + n] = (sRed[0] + sRed[1]) + (sRed[2] + sRed[3]);
        }
        float acc[SCAN_RPT][4] = {};
        for (int t = 0; t < BC; t++) {
            const float4 bv = *reinterpret_cast<const float4*>(&sB[t][cc]);
#pragma unroll
            for (int i = 0; i < SCAN_RPT; i++) {
                const float av = sA[t][rr + i];
                acc[i][0] = fmaf(av, bv.x, acc[i][0]);
                acc[i][1] = fmaf(av, bv.y, acc[i][1]);
                acc[i][2] = fmaf(av, bv.z, acc[i][2]);
                acc[i][3] = fmaf(av, bv.w, acc[i][3]);
            }
        }
        const float el = sEl;
#pragma unroll
        for (int i = 0; i < SCAN_RPT; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) x[i][j] = fmaf(el, x[i][j], acc[i][j]);
    }
    keep(BWD ? 0 : N);
    const bw_rsrc_t rxo = bw_rsrc(p.x_out ? p.x_out + bh * ssz : nullptr, p.x_out ? ssz : 0);
#pragma unroll
    for (int i = 0; i < SCAN_RPT; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) bw_store(rxo, off[i][j], ok[i][j], x[i][j]);  // dropped without x_out
}

// The same scan for bf16 operands on the matrix cores: the rank-64 update
// X += A^T B over the chunk's 64 tokens as split-bf16 products on
// v_mfma_f32_16x16x32_bf16 (each fp32 operand as a bf16 high part and a bf16
// remainder, lo_a hi_b + hi_a lo_b + hi_a hi_b: about 16 mantissa bits, as in
// the chunk kernels' tile GEMMs). A workgroup takes a 32 T2 x 32 T2 tile,
// wave w its 16 T2 x 16 T2 quarter (w >> 1, w & 1) as T2 x T2 accumulator
// blocks: lane (lr, lg) of block (ib, jb) has rows 16 T2 (w >> 1) + 16 ib +
// 4 lg + i, column 16 T2 (w & 1) + 16 jb + lr. The larger tile reads each
// chunk's rows of a and b from fewer workgroups (the scans are bound by those
// reads: every column tile reads the rows of a again, every row tile the
// columns of b). Per chunk, thread (r, q) = (tid % 32 T2, tid / 32 T2) loads
// tokens 8 T2 q .. + 8 T2 of row r of a and of column r of b and stages them
// transposed (row = state coordinate, 64 tokens along the row), so that every
// operand fragment is one 16-byte LDS read. The boundary terms go to bnd per
// 32 x 32 tile, as the FMA form's: with T2 = 2 one per wave, with T2 = 1 one
// per workgroup.
constexpr int SCAN_LDT = BC + 8;  // staged row: 64 tokens + 8 of padding (bf16)

__device__ __forceinline__ void split_bf16x8(const float* v, bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int x = 0; x < 8; x++) {
        hi[x] = (bf16_t)v[x];
        lo[x] = (bf16_t)(v[x] - (float)hi[x]);
    }
}

template <bool BWD, int T2, bool SB, bool BB>
__global__ __launch_bounds__(T2 == 2 ? 512 : 256) void bw_state_scan_mf_kernel(StateScanArgs p) {
    using SE = std::conditional_t<SB, bf16_t, float>;  // the stored states' element
    using BE = std::conditional_t<BB, bf16_t, float>;  // b's element
    static_assert(SCAN_ROWS == 32 && BW_TILE == 32 && (T2 == 1 || T2 == 2), "32 x 32 bnd tiles");
    constexpr int TS = 32 * T2;     // tile side
    // Waves: 8 for 64 x 64 tiles (one workgroup per CU at configuration 3's
    // shapes, so that two waves share each SIMD), 4 for 32 x 32; wave w holds
    // the 16 x 16 T2 block of rows 16 (w / 2) and columns 16 T2 (w % 2).
    constexpr int NTH = T2 == 2 ? 512 : 256, NWV = NTH / 64, IB = 1;
    constexpr int TPT = BC / (NTH / TS);  // tokens per staging thread
    __shared__ __align__(16) bf16_t sAh[TS][SCAN_LDT], sAl[TS][SCAN_LDT];
    __shared__ __align__(16) bf16_t sBh[TS][SCAN_LDT], sBl[TS][SCAN_LDT];
    __shared__ float sF[BC];
    __shared__ float sRed[NWV];
    __shared__ float sEl;
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int c0 = blockIdx.x * TS, r0 = blockIdx.y * TS, bhi = blockIdx.z;
    const int b = bhi / p.H, h = bhi % p.H;
    const int Kq = p.Kq, Vd = p.Vd, N = p.N;
    // bnd tiles of 32 x 32: nx across Vd, ny down Kq; this workgroup's (T2 = 1)
    // or this wave's and its partner's, wave w ^ 2 (T2 = 2)
    const int nx = (Vd + 31) / 32, ny = (Kq + 31) / 32, nt = nx * ny;
    const int ty = T2 == 1 ? (int)blockIdx.y : 2 * (int)blockIdx.y + (wv >> 2);
    const int tx = T2 == 1 ? (int)blockIdx.x : 2 * (int)blockIdx.x + (wv & 1);
    const size_t bh = bhi, ssz = (size_t)Kq * Vd;
    SE* xs = reinterpret_cast<SE*>(p.xs) + bh * (N + 1) * ssz;
    const SE* Sx = reinterpret_cast<const SE*>(p.S);
    const float* A = p.a + bh * p.Tp * Kq;
    const BE* Bm = reinterpret_cast<const BE*>(p.b) + bh * p.Tp * Vd;
    const int wr = 16 * IB * (wv >> 1), wc = 16 * T2 * (wv & 1);  // the wave's block
    bool ok[IB][T2][4];
    uint32_t off[IB][T2][4];
    f32x4 x[IB][T2];
    const bw_rsrc_t rx0 = bw_rsrc(p.x0 ? p.x0 + bh * ssz : nullptr, p.x0 ? ssz : 0);
#pragma unroll
    for (int ib = 0; ib < IB; ib++)
#pragma unroll
        for (int jb = 0; jb < T2; jb++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int xr = r0 + wr + 16 * ib + 4 * lg + i, xc = c0 + wc + 16 * jb + lr;
                ok[ib][jb][i] = xr < Kq && xc < Vd;
                off[ib][jb][i] = ((uint32_t)xr * (uint32_t)Vd + (uint32_t)xc) * 4u;
                x[ib][jb][i] = bw_load(rx0, off[ib][jb][i], ok[ib][jb][i]);
            }
    float sv[IB][T2][4] = {};
    const auto fetch_state = [&](int n) {
        const bw_rsrc_t rs = bw_rsrc(Sx + (bh * (N + 1) + n) * ssz, ssz);
#pragma unroll
        for (int ib = 0; ib < IB; ib++)
#pragma unroll
            for (int jb = 0; jb < T2; jb++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    sv[ib][jb][i] = SB ? bw_load_h(rs, off[ib][jb][i] / 2u, ok[ib][jb][i])
                                       : bw_load(rs, off[ib][jb][i], ok[ib][jb][i]);
    };
    const auto keep = [&](int n) {  // xs[n] = X; returns the lane's part of <X, S[n]> (backward)
        const bw_rsrc_t rs = bw_rsrc(xs + (size_t)n * ssz, ssz);
        float dot = 0.f;
#pragma unroll
        for (int ib = 0; ib < IB; ib++)
#pragma unroll
            for (int jb = 0; jb < T2; jb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if constexpr (SB)
                        bw_store_h(rs, off[ib][jb][i] / 2u, ok[ib][jb][i], x[ib][jb][i]);
                    else
                        bw_store(rs, off[ib][jb][i], ok[ib][jb][i], x[ib][jb][i]);
                    if constexpr (BWD) dot = fmaf(x[ib][jb][i], sv[ib][jb][i], dot);
                }
        return dot;
    };
    const int sr = tid % TS, sq = tid / TS;  // staging: row / column sr, tokens TPT sq ..
    const bw_rsrc_t rgt = bw_rsrc(p.g, (size_t)p.B * p.T * p.H);  // B T H < 2^21 (host)
    // chunk n's rows of a, columns of b and gate into (ra, rb, rg)
    const auto fetch = [&](int n, float* ra, float* rb, float& rg) {
        const int t0 = n * BC;
        const bw_rsrc_t rA = bw_rsrc(A + (size_t)t0 * Kq, (size_t)BC * Kq), rBm = bw_rsrc(Bm + (size_t)t0 * Vd, (size_t)BC * Vd);
#pragma unroll
        for (int i = 0; i < TPT; i++) {
            const uint32_t t = TPT * sq + i;
            ra[i] = bw_load(rA, (t * (uint32_t)Kq + (uint32_t)(r0 + sr)) * 4u, r0 + sr < Kq);
            rb[i] = BB ? bw_load_h(rBm, (t * (uint32_t)Vd + (uint32_t)(c0 + sr)) * 2u, c0 + sr < Vd)
                       : bw_load(rBm, (t * (uint32_t)Vd + (uint32_t)(c0 + sr)) * 4u, c0 + sr < Vd);
        }
        rg = bw_load(rgt, (((uint32_t)b * (uint32_t)p.T + (uint32_t)(t0 + lane)) * (uint32_t)p.H + (uint32_t)h) * 4u,
                     t0 + lane < p.T);
    };
    const auto chunk_of = [&](int step) { return BWD ? N - 1 - step : step; };
    // One chunk step from the registers (ra, rb, rg), which then receive the
    // next chunk. (Two register sets, with the chunk two steps on in flight,
    // were slower: 83 -> 93 us for the forward scan at configuration 3; the
    // scan is bound by each compute unit's reads, not by their latency.)
    const auto run_step = [&](int step, float* ra, float* rb, float& rg) {
        const int n = chunk_of(step);
        const float dot = keep(BWD ? n + 1 : n);
        __syncthreads();  // the previous chunk's operands are done with
        float wsum = 0.f;
        if constexpr (BWD) {
            wsum = bw_wave_sum(dot);
            if (lane == 0) sRed[wv] = wsum;
        }
        if (wv == 0) {  // G: the in-chunk inclusive cumsum of the prefetched gate
            const float G = bw_wave_scan(rg);
            const float Gl = lane_value(G, 63);
            sF[lane] = BWD ? p.scale * expf(G) : expf(Gl - G);
            if (lane == 0) sEl = expf(Gl);
        }
#pragma unroll
        for (int u = 0; u < TPT / 8; u++) {
            bf16x8 hi, lo;
            split_bf16x8(rb + 8 * u, hi, lo);
            *reinterpret_cast<bf16x8*>(&sBh[sr][TPT * sq + 8 * u]) = hi;
            *reinterpret_cast<bf16x8*>(&sBl[sr][TPT * sq + 8 * u]) = lo;
        }
        __syncthreads();  // sF is read below
#pragma unroll
        for (int u = 0; u < TPT / 8; u++) {
            float fa[8];
#pragma unroll
            for (int i = 0; i < 8; i++) fa[i] = sF[TPT * sq + 8 * u + i] * ra[8 * u + i];
            bf16x8 hi, lo;
            split_bf16x8(fa, hi, lo);
            *reinterpret_cast<bf16x8*>(&sAh[sr][TPT * sq + 8 * u]) = hi;
            *reinterpret_cast<bf16x8*>(&sAl[sr][TPT * sq + 8 * u]) = lo;
        }
        __syncthreads();
        if (step + 1 < N) fetch(chunk_of(step + 1), ra, rb, rg);
        if constexpr (BWD) fetch_state(n);  // for the next step's keep(n)
        if constexpr (BWD) {
            if (T2 == 1 && tid == 0)
                p.bnd[(bh * nt + ty * nx + tx) * N + n] = (sRed[0] + sRed[1]) + (sRed[2] + sRed[3]);
            if (T2 == 2 && lane == 0 && (wv & 2) == 0 && ty < ny && tx < nx)  // the tile's two waves
                p.bnd[(bh * nt + ty * nx + tx) * N + n] = sRed[wv] + sRed[wv + 2];
        }
        const float el = sEl;
#pragma unroll
        for (int ib = 0; ib < IB; ib++)
#pragma unroll
            for (int jb = 0; jb < T2; jb++)
#pragma unroll
                for (int i = 0; i < 4; i++) x[ib][jb][i] *= el;
#pragma unroll
        for (int s = 0; s < BC / 32; s++) {
            bf16x8 ah[IB], al[IB], bh8[T2], bl8[T2];
#pragma unroll
            for (int ib = 0; ib < IB; ib++) {
                ah[ib] = *reinterpret_cast<const bf16x8*>(&sAh[wr + 16 * ib + lr][32 * s + 8 * lg]);
                al[ib] = *reinterpret_cast<const bf16x8*>(&sAl[wr + 16 * ib + lr][32 * s + 8 * lg]);
            }
#pragma unroll
            for (int jb = 0; jb < T2; jb++) {
                bh8[jb] = *reinterpret_cast<const bf16x8*>(&sBh[wc + 16 * jb + lr][32 * s + 8 * lg]);
                bl8[jb] = *reinterpret_cast<const bf16x8*>(&sBl[wc + 16 * jb + lr][32 * s + 8 * lg]);
            }
#pragma unroll
            for (int ib = 0; ib < IB; ib++)
#pragma unroll
                for (int jb = 0; jb < T2; jb++) {
                    x[ib][jb] = mfma_bf16(al[ib], bh8[jb], x[ib][jb]);
                    x[ib][jb] = mfma_bf16(ah[ib], bl8[jb], x[ib][jb]);
                    x[ib][jb] = mfma_bf16(ah[ib], bh8[jb], x[ib][jb]);
                }
        }
    };
    float ra[TPT], rb[TPT], rg;
    fetch(chunk_of(0), ra, rb, rg);
    if constexpr (BWD) fetch_state(N);
    for (int step = 0; step < N; step++) run_step(step, ra, rb, rg);
    keep(BWD ? 0 : N);
    const bw_rsrc_t rxo = bw_rsrc(p.x_out ? p.x_out + bh * ssz : nullptr, p.x_out ? ssz : 0);
#pragma unroll
    for (int ib = 0; ib < IB; ib++)
#pragma unroll
        for (int jb = 0; jb < T2; jb++)
#pragma unroll
            for (int i = 0; i < 4; i++) bw_store(rxo, off[ib][jb][i], ok[ib][jb][i], x[ib][jb][i]);  // dropped without x_out
}

// Launches the scan over a [Kq, Vd] state (grid: the FMA form's 32 x 32
// tiles): the matrix-core form for bf16 operands, with 64 x 64 tiles when
// they still give a workgroup per compute unit.
template <bool BWD, int T2>
void launch_scan_mf(const StateScanArgs& a, dim3 grid, hipStream_t stream) {
    const dim3 blk(T2 == 2 ? 512 : 256);
    if (a.sbf && a.bbf)
        hipLaunchKernelGGL((bw_state_scan_mf_kernel<BWD, T2, true, true>), grid, blk, 0, stream, a);
    else if (a.sbf)
        hipLaunchKernelGGL((bw_state_scan_mf_kernel<BWD, T2, true, false>), grid, blk, 0, stream, a);
    else if (a.bbf)
        hipLaunchKernelGGL((bw_state_scan_mf_kernel<BWD, T2, false, true>), grid, blk, 0, stream, a);
    else
        hipLaunchKernelGGL((bw_state_scan_mf_kernel<BWD, T2, false, false>), grid, blk, 0, stream, a);
}

template <bool BWD>
void launch_state_scan(const StateScanArgs& a, bool mfma, hipStream_t stream) {
    const dim3 g32((a.Vd + 31) / 32, (a.Kq + 31) / 32, a.B * a.H), g64((a.Vd + 63) / 64, (a.Kq + 63) / 64, a.B * a.H);
    if (!mfma)
        hipLaunchKernelGGL(bw_state_scan_kernel<BWD>, g32, dim3(256), 0, stream, a);
    else if ((long long)g64.x * g64.y * g64.z >= device_cu_count())
        launch_scan_mf<BWD, 2>(a, g64, stream);
    else
        launch_scan_mf<BWD, 1>(a, g32, stream);
}

// Tile GEMMs of the chunk kernels: a 64 x 64 output tile (rows = the chunk's
// tokens, columns = 64 coordinates), acc[a][b] per thread at (TileMap<MF>::row,
// TileMap<MF>::col), accumulated over a contraction of Kd in k-blocks of 32
// staged through LDS, the next k-block's operands prefetched into registers
// while the current one is multiplied. fa(i, kk) and fb(kk, j) read the
// operands; B_KCONTIG says whether fb is contiguous along kk (else along j).
//  - MF false (fp32 operands): fp32 FMA, a 4 x 4 block per thread (rows
//    4 (tid / 16) .., columns 4 (tid % 16) ..), A staged transposed so a
//    thread's four rows are one float4.
//  - MF true (bf16 operands): matrix cores at near-fp32 accuracy: each fp32
//    operand is split into hi = bf16(x) and lo = bf16(x - hi), staged in LDS,
//    and a.b formed as lo_a hi_b + hi_a lo_b + hi_a hi_b on
//    v_mfma_f32_16x16x32_bf16 with fp32 accumulation (about 16 mantissa
//    bits; the dropped lo_a lo_b is 2^-16 relative): wave w forms rows 16 w
//    .. + 16 as four 16 x 16 blocks, acc[nb][i] = tile[16 w + 4 (lane / 16) +
//    i][16 nb + lane % 16]. The kernels are bound by the staging, not the
//    matrix cores, so the three products cost about what one does.
constexpr int GT_K = 32, GT_LD = 68;  // fp32 staging: [32][68] per operand
constexpr int MT_LD = 40;             // bf16 staging: [64][40] per operand (32 k + 8 pad)
constexpr int STAGE_BYTES = 4 * BC * MT_LD * 2;  // >= the fp32 staging's 2 * GT_K * GT_LD * 4
constexpr int STAGE2_BYTES = 6 * BC * MT_LD * 2;  // tile_gemm_mf<2>: A and two B blocks, hi and lo
static_assert(STAGE_BYTES >= 2 * GT_K * GT_LD * 4, "staging must hold either form");

template <bool MF>
struct TileMap {
    __device__ static int row(int a, int b) {
        if constexpr (MF)
            return 16 * (threadIdx.x >> 6) + 4 * ((threadIdx.x & 63) >> 4) + b;
        else
            return 4 * (threadIdx.x >> 4) + a;
    }
    __device__ static int col(int a, int b) {
        if constexpr (MF)
            return 16 * a + (threadIdx.x & 15);
        else
            return 4 * (threadIdx.x & 15) + b;
    }
};

// Global operands of tile_gemm, read through a buffer resource over the
// operand's region with every out-of-range element predicated to zero through
// its offset (so the next k-block's loads overlap the current one's products).
//  RowsK: element (m, kk) = base[m ld + kk] for m < nm, kk < nk (the A
//         operand, m = the tile row, and a B operand contiguous along kk,
//         m = the tile column).
//  RowsJ: element (kk, j) = base[kk ld + j] for kk < nk, j < nj (a B operand
//         contiguous along j).
struct RowsK {
    bw_rsrc_t r;
    uint32_t ld;
    int nm, nk;
    __device__ RowsK(const float* base, int ld_, int nm_, int nk_)
        : r(bw_rsrc(base, nm_ > 0 ? (size_t)(nm_ - 1) * ld_ + nk_ : 0)), ld((uint32_t)ld_), nm(nm_), nk(nk_) {}
    __device__ float load(int m, int kk) const {
        const uint32_t dead = (m < nm && kk < nk) ? 0u : BW_DEAD;
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ((uint32_t)m * ld + (uint32_t)kk) * 4u | dead, 0, 0));
    }
};

// RowsK with 16-byte loads of four consecutive kk: the caller guarantees a
// 16-byte aligned base and ld, nk multiples of 4. In tile_gemm's matrix-core
// staging, lane (r, kg) then loads kk = k0 + 4 kg .. + 3 and k0 + 16 + 4 kg ..
// + 3, so that each load instruction covers 64 contiguous bytes of 16 rows
// (with one 4-byte load per kk, eight instructions each touched 16 lines).
struct RowsK4 : RowsK {
    __device__ RowsK4(const float* base, int ld_, int nm_, int nk_) : RowsK(base, ld_, nm_, nk_) {}
    __device__ f32x4 load4(int m, int kk0) const {
        const uint32_t dead = (m < nm && kk0 < nk) ? 0u : BW_DEAD;
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, ((uint32_t)m * ld + (uint32_t)kk0) * 4u | dead, 0, 0));
    }
};

struct RowsJ {
    bw_rsrc_t r;
    uint32_t ld;
    int nk, nj;
    __device__ RowsJ(const float* base, int ld_, int nk_, int nj_)
        : r(bw_rsrc(base, nk_ > 0 ? (size_t)(nk_ - 1) * ld_ + nj_ : 0)), ld((uint32_t)ld_), nk(nk_), nj(nj_) {}
    __device__ float load(int kk, int j) const {
        const uint32_t dead = (kk < nk && j < nj) ? 0u : BW_DEAD;
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, ((uint32_t)kk * ld + (uint32_t)j) * 4u | dead, 0, 0));
    }
};

// RowsJ with 16-byte loads of four consecutive j (16-byte aligned base, ld and
// nj multiples of 4). In tile_gemm's matrix-core staging, lane (jq, kp) =
// (tid % 16, tid / 16) loads j = 4 jq .. + 3 of rows kk = k0 + 2 kp and
// k0 + 2 kp + 1 (each load instruction covers whole 256-byte row segments)
// and writes the pairs (kk, kk + 1) of its four columns as 4-byte LDS stores.
struct RowsJ4 : RowsJ {
    __device__ RowsJ4(const float* base, int ld_, int nk_, int nj_) : RowsJ(base, ld_, nk_, nj_) {}
    __device__ f32x4 load4(int kk, int j0) const {
        const uint32_t dead = (kk < nk && j0 < nj) ? 0u : BW_DEAD;
        return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, ((uint32_t)kk * ld + (uint32_t)j0) * 4u | dead, 0, 0));
    }
};

// RowsK, RowsK4, RowsJ and RowsJ4 over bf16 elements (the stored states and
// state cotangents of bf16 calls): two-byte loads, and load4's four
// consecutive elements in one 8-byte load (16-byte aligned base, ld and the
// extent multiples of 4). The values widen to fp32 exactly.
struct RowsKh : RowsK {
    __device__ RowsKh(const bf16_t* base, int ld_, int nm_, int nk_) : RowsK(nullptr, ld_, nm_, nk_) {
        r = bw_rsrc(base, nm_ > 0 ? (size_t)(nm_ - 1) * ld_ + nk_ : 0);
    }
    __device__ float load(int m, int kk) const {
        return bw_load_h(r, ((uint32_t)m * ld + (uint32_t)kk) * 2u, m < nm && kk < nk);
    }
};
struct RowsK4h : RowsK4 {
    __device__ RowsK4h(const bf16_t* base, int ld_, int nm_, int nk_) : RowsK4(nullptr, ld_, nm_, nk_) {
        r = bw_rsrc(base, nm_ > 0 ? (size_t)(nm_ - 1) * ld_ + nk_ : 0);
    }
    __device__ float load(int m, int kk) const {
        return bw_load_h(r, ((uint32_t)m * ld + (uint32_t)kk) * 2u, m < nm && kk < nk);
    }
    __device__ f32x4 load4(int m, int kk0) const {
        const uint32_t dead = (m < nm && kk0 < nk) ? 0u : BW_DEAD;
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, ((uint32_t)m * ld + (uint32_t)kk0) * 2u | dead, 0, 0);
        return bf16x4_bits_to_f32x4(w[0], w[1]);
    }
};
struct RowsJh : RowsJ {
    __device__ RowsJh(const bf16_t* base, int ld_, int nk_, int nj_) : RowsJ(nullptr, ld_, nk_, nj_) {
        r = bw_rsrc(base, nk_ > 0 ? (size_t)(nk_ - 1) * ld_ + nj_ : 0);
    }
    __device__ float load(int kk, int j) const {
        return bw_load_h(r, ((uint32_t)kk * ld + (uint32_t)j) * 2u, kk < nk && j < nj);
    }
};
struct RowsJ4h : RowsJ4 {
    __device__ RowsJ4h(const bf16_t* base, int ld_, int nk_, int nj_) : RowsJ4(nullptr, ld_, nk_, nj_) {
        r = bw_rsrc(base, nk_ > 0 ? (size_t)(nk_ - 1) * ld_ + nj_ : 0);
    }
    __device__ float load(int kk, int j) const {
        return bw_load_h(r, ((uint32_t)kk * ld + (uint32_t)j) * 2u, kk < nk && j < nj);
    }
    __device__ f32x4 load4(int kk, int j0) const {
        const uint32_t dead = (kk < nk && j0 < nj) ? 0u : BW_DEAD;
        const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, ((uint32_t)kk * ld + (uint32_t)j0) * 2u | dead, 0, 0);
        return bf16x4_bits_to_f32x4(w[0], w[1]);
    }
};

// The state operands' row types: fp32, or bf16 with SB.
template <bool SB, bool V4>
using StateRowsK = std::conditional_t<SB, std::conditional_t<V4, RowsK4h, RowsKh>, std::conditional_t<V4, RowsK4, RowsK>>;
template <bool SB, bool V4>
using StateRowsJ = std::conditional_t<SB, std::conditional_t<V4, RowsJ4h, RowsJh>, std::conditional_t<V4, RowsJ4, RowsJ>>;

// Element (i, kk) of A and (kk, j) of B, for a global operand or a callable
// (LDS operands: read only at kk < Kd, contractions of BC tokens).
template <class FA>
__device__ __forceinline__ float opA(const FA& fa, int i, int kk, int Kd) {
    if constexpr (std::is_base_of_v<RowsK, FA>)
        return fa.load(i, kk);
    else
        return kk < Kd ? fa(i, kk) : 0.f;
}
template <class FB>
__device__ __forceinline__ float opB(const FB& fb, int kk, int j, int Kd) {
    if constexpr (std::is_base_of_v<RowsK, FB>)
        return fb.load(j, kk);
    else if constexpr (std::is_base_of_v<RowsJ, FB>)
        return fb.load(kk, j);
    else
        return kk < Kd ? fb(kk, j) : 0.f;
}

// The matrix-core form of tile_gemm (above) for an output of 64 rows by
// 64 NT columns in one pass over the contraction: A is staged once per
// k-block and multiplied against NT B tiles, so that a row block feeding
// several output tiles is read once (NT = 2 halves those reads against two
// passes). acc[nb][i] = tile[16 w + 4 (lane / 16) + i][16 nb + lane % 16],
// nb < 4 NT; the staging area holds (2 + 2 NT) 64-row blocks.
template <int NT, class FA, class FB>
__device__ __forceinline__ void tile_gemm_mf(FA fa, FB fb, int Kd, unsigned char* stage, float acc[4 * NT][4]) {
    const int tid = threadIdx.x;
    {
        bf16_t* sah = reinterpret_cast<bf16_t*>(stage);  // hi and lo parts of A (64 rows) and of B (64 NT rows)
        bf16_t* sal = sah + BC * MT_LD;
        bf16_t* sbh = sal + BC * MT_LD;
        bf16_t* sbl = sbh + NT * BC * MT_LD;
        const int l = tid & 63, w = tid >> 6, lr = l & 15, lg = l >> 4;
        const int r = tid >> 2, kg = tid & 3;  // staging: row r, k-group kg (8 k)
        // RowsK4 operands: lane (r, kg) holds kk = k0 + 4 kg .. + 3 and
        // k0 + 16 + 4 kg .. + 3; the others kk = k0 + 8 kg .. + 7
        constexpr bool VA = std::is_base_of_v<RowsK4, FA>, VB = std::is_base_of_v<RowsK4, FB>;
        constexpr bool JB = std::is_base_of_v<RowsJ4, FB>;  // B: lane (jq, kp) as in RowsJ4
        const int jq = tid & 15, kp = tid >> 4;
        float ra[8], rb[NT][8];
        const auto fetch = [&](int k0) {
            if constexpr (VA) {
                const f32x4 lo4 = fa.load4(r, k0 + 4 * kg), hi4 = fa.load4(r, k0 + 16 + 4 * kg);
#pragma unroll
                for (int x = 0; x < 4; x++) ra[x] = lo4[x], ra[4 + x] = hi4[x];
            } else {
#pragma unroll
                for (int x = 0; x < 8; x++) ra[x] = opA(fa, r, k0 + 8 * kg + x, Kd);
            }
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {  // B's columns 64 nt ..
                if constexpr (VB) {
                    const f32x4 lo4 = fb.load4(64 * nt + r, k0 + 4 * kg), hi4 = fb.load4(64 * nt + r, k0 + 16 + 4 * kg);
#pragma unroll
                    for (int x = 0; x < 4; x++) rb[nt][x] = lo4[x], rb[nt][4 + x] = hi4[x];
                } else if constexpr (JB) {  // rb[c] = B(k0 + 2 kp, 4 jq + c), rb[4 + c] = B(k0 + 2 kp + 1, 4 jq + c)
                    const f32x4 r0 = fb.load4(k0 + 2 * kp, 64 * nt + 4 * jq), r1 = fb.load4(k0 + 2 * kp + 1, 64 * nt + 4 * jq);
#pragma unroll
                    for (int x = 0; x < 4; x++) rb[nt][x] = r0[x], rb[nt][4 + x] = r1[x];
                } else {
#pragma unroll
                    for (int x = 0; x < 8; x++) rb[nt][x] = opB(fb, k0 + 8 * kg + x, 64 * nt + r, Kd);
                }
            }
        };
        // writes the 8 staged values of one operand in its lane order
        const auto put = [&](bf16_t* base, bool split4, const bf16x8& v) {
            if (split4) {
                *reinterpret_cast<bf16x4*>(base + r * MT_LD + 4 * kg) = bf16x4{v[0], v[1], v[2], v[3]};
                *reinterpret_cast<bf16x4*>(base + r * MT_LD + 16 + 4 * kg) = bf16x4{v[4], v[5], v[6], v[7]};
            } else {
                *reinterpret_cast<bf16x8*>(base + r * MT_LD + 8 * kg) = v;
            }
        };
        fetch(0);
        for (int k0 = 0; k0 < Kd; k0 += GT_K) {
            __syncthreads();  // the staging tiles are free
            bf16x8 vah, val;
#pragma unroll
            for (int x = 0; x < 8; x++) {
                vah[x] = (bf16_t)ra[x];
                val[x] = (bf16_t)(ra[x] - (float)vah[x]);
            }
            put(sah, VA, vah);
            put(sal, VA, val);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                bf16x8 vbh, vbl;
#pragma unroll
                for (int x = 0; x < 8; x++) {
                    vbh[x] = (bf16_t)rb[nt][x];
                    vbl[x] = (bf16_t)(rb[nt][x] - (float)vbh[x]);
                }
                bf16_t* bh0 = sbh + 64 * nt * MT_LD;
                bf16_t* bl0 = sbl + 64 * nt * MT_LD;
                if constexpr (JB) {  // column 4 jq + c: the pair (k0 + 2 kp, + 1) as one 4-byte store
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        *reinterpret_cast<bf16x2*>(bh0 + (4 * jq + c) * MT_LD + 2 * kp) = bf16x2{vbh[c], vbh[4 + c]};
                        *reinterpret_cast<bf16x2*>(bl0 + (4 * jq + c) * MT_LD + 2 * kp) = bf16x2{vbl[c], vbl[4 + c]};
                    }
                } else {
                    put(bh0, VB, vbh);
                    put(bl0, VB, vbl);
                }
            }
            __syncthreads();
            if (k0 + GT_K < Kd) fetch(k0 + GT_K);
            const int ao = (16 * w + lr) * MT_LD + 8 * lg;
            const bf16x8 ah = *reinterpret_cast<const bf16x8*>(sah + ao);
            const bf16x8 al = *reinterpret_cast<const bf16x8*>(sal + ao);
#pragma unroll
            for (int nb = 0; nb < 4 * NT; nb++) {
                const int bo = (16 * nb + lr) * MT_LD + 8 * lg;
                const bf16x8 bh = *reinterpret_cast<const bf16x8*>(sbh + bo);
                const bf16x8 bl = *reinterpret_cast<const bf16x8*>(sbl + bo);
                f32x4 c = {acc[nb][0], acc[nb][1], acc[nb][2], acc[nb][3]};
                c = mfma_bf16(al, bh, c);
                c = mfma_bf16(ah, bl, c);
                c = mfma_bf16(ah, bh, c);
#pragma unroll
                for (int i = 0; i < 4; i++) acc[nb][i] = c[i];
            }
        }
    }
}

template <bool MF, bool B_KCONTIG, class FA, class FB>
__device__ __forceinline__ void tile_gemm(FA fa, FB fb, int Kd, unsigned char* stage, float acc[4][4]) {
    static_assert(!std::is_base_of_v<RowsK, FB> || B_KCONTIG, "RowsK: B contiguous along kk");
    static_assert(!std::is_base_of_v<RowsJ, FB> || !B_KCONTIG, "RowsJ: B contiguous along j");
    const int tid = threadIdx.x;
    if constexpr (!MF) {
        float(*sa)[GT_LD] = reinterpret_cast<float(*)[GT_LD]>(stage);
        float(*sb)[GT_LD] = reinterpret_cast<float(*)[GT_LD]>(stage + GT_K * GT_LD * 4);
        constexpr int NE = BC * GT_K / 256;  // staged elements of each operand per thread
        const int ti = 4 * (tid >> 4), tj = 4 * (tid & 15);
        float ra[NE], rb[NE];
        const auto fetch = [&](int k0) {
#pragma unroll
            for (int x = 0; x < NE; x++) {
                const int e = tid + 256 * x;
                const int ka = e % GT_K, i = e / GT_K;
                ra[x] = opA(fa, i, k0 + ka, Kd);
                const int kb = B_KCONTIG ? e % GT_K : e / BC, j = B_KCONTIG ? e / GT_K : e % BC;
                rb[x] = opB(fb, k0 + kb, j, Kd);
            }
        };
        fetch(0);
        for (int k0 = 0; k0 < Kd; k0 += GT_K) {
            __syncthreads();  // the staging tiles are free
#pragma unroll
            for (int x = 0; x < NE; x++) {
                const int e = tid + 256 * x;
                sa[e % GT_K][e / GT_K] = ra[x];
                if (B_KCONTIG)
                    sb[e % GT_K][e / GT_K] = rb[x];
                else
                    sb[e / BC][e % BC] = rb[x];
            }
            __syncthreads();
            if (k0 + GT_K < Kd) fetch(k0 + GT_K);
#pragma unroll 8
            for (int kk = 0; kk < GT_K; kk++) {
                const float4 av = *reinterpret_cast<const float4*>(&sa[kk][ti]);
                const float4 bv = *reinterpret_cast<const float4*>(&sb[kk][tj]);
                const float ar[4] = {av.x, av.y, av.z, av.w}, br[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = fmaf(ar[i], br[j], acc[i][j]);
            }
        }
    } else {
        tile_gemm_mf<1>(fa, fb, Kd, stage, acc);
    }
}

// acc[a][b] *= f(row of (a, b)); NA = 4 NT for a matrix-core tile of 64 NT
// columns.
template <bool MF, int NA = 4, class F>
__device__ __forceinline__ void tile_scale_rows(float acc[NA][4], F f) {
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] *= f(TileMap<MF>::row(a, b));
}

// Writes this thread's part of a 64 x 16 NA tile (columns d0 ..) into
// head-major rows dst [.., D], times a scale.
template <bool MF, int NA = 4>
__device__ __forceinline__ void tile_store(float acc[NA][4], float* dst, int D, int d0, float scale) {
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int t = TileMap<MF>::row(a, b), c = d0 + TileMap<MF>::col(a, b);
            if (c < D) dst[(size_t)t * D + c] = scale * acc[a][b];
        }
}

// tile_gemm over 64 NT output columns: NT = 2 only on the matrix cores.
template <bool MF, bool B_KCONTIG, int NT, class FA, class FB>
__device__ __forceinline__ void tile_gemm_nt(FA fa, FB fb, int Kd, unsigned char* stage, float acc[4 * NT][4]) {
    if constexpr (NT == 1) {
        tile_gemm<MF, B_KCONTIG>(fa, fb, Kd, stage, acc);
    } else {
        static_assert(MF && NT == 2, "wide tiles on the matrix cores");
        tile_gemm_mf<NT>(fa, fb, Kd, stage, acc);
    }
}

// Masked, decayed scores of one chunk into P: P[t][s] = [s <= t] e^{G_t - G_s}
// sum_j X_t[j] Y_s[j] (X, Y: the chunk's 64 rows, D wide), as one tile GEMM.
template <bool MF, bool V4, class E>
__device__ __forceinline__ void chunk_scores(const E* X, const E* Y, int D, const float* sG, unsigned char* stage,
                                             float (*P)[BC + 1]) {
    using RK = StateRowsK<std::is_same_v<E, bf16_t>, V4>;  // fp32 or bf16 rows
    float acc[4][4] = {};
    tile_gemm<MF, true>(RK(X, D, BC, D), RK(Y, D, BC, D), D, stage, acc);
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int t = TileMap<MF>::row(a, b), s = TileMap<MF>::col(a, b);
            P[t][s] = s <= t ? acc[a][b] * expf(sG[t] - sG[s]) : 0.f;
        }
}

// The output of one pass, chunk-parallel (grid (N, H, B), 256 threads):
// o_t = scale (e^{G_t} q_t S_n + sum_{s<=t} A[t][s] v_s), A the masked
// decayed q.k scores, per 64-wide output tile as two tile GEMMs. The
// backward's recompute writes pass 1 head-major and unrounded; the general
// forward rounds to bf16 for bf16 inputs and writes pass 2 as [B, T, H, Vd].
struct OutArgs {
    const float *q, *k, *v;  // head-major [B*H, Tp, Kq | Vd]
    const float* g;
    const float* S;          // [B*H, N+1, Kq, Vd]: fp32, or bf16_t with sbf
    float* out;              // head-major [B*H, Tp, Vd], used when out_bthd is null
    void* out_bthd;          // nullable [B, T, H, Vd], bf16 when bf16 else fp32
    int bf16;                // round to bf16
    int B, T, Tp, H, Kq, Vd, N;
    float scale;
    int sbf;                 // matrix-core form: S holds bf16 states
};

template <bool MF, bool V4, bool SB>
__global__ __launch_bounds__(256) void bw_out_kernel(OutArgs a) {
    using RK = std::conditional_t<V4, RowsK4, RowsK>;  // 16-byte row loads when aligned
    using RJ = std::conditional_t<V4, RowsJ4, RowsJ>;
    using SJ = StateRowsJ<SB, V4>;
    using SE = std::conditional_t<SB, bf16_t, float>;
    __shared__ float sA[BC][BC + 1];
    // (output tiles of 64 columns: two at a time read q once instead of twice
    // but measured slower here, 80 -> 84 us at configuration 3)
    constexpr int NT = 1, NA = 4 * NT;
    __shared__ __align__(16) unsigned char sStage[NT == 2 ? STAGE2_BYTES : STAGE_BYTES];
    __shared__ float sG[BC], sEq[BC];
    const int tid = threadIdx.x, n = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int Kq = a.Kq, Vd = a.Vd, t0 = n * BC;
    const size_t bh = (size_t)b * a.H + h, ssz = (size_t)Kq * Vd;
    const float* q = a.q + (bh * a.Tp + t0) * Kq;
    const float* k = a.k + (bh * a.Tp + t0) * Kq;
    const float* v = a.v + (bh * a.Tp + t0) * Vd;
    const SE* S = reinterpret_cast<const SE*>(a.S) + (bh * (a.N + 1) + n) * ssz;
    if (tid < 64) {
        sG[tid] = chunk_gam(a.g, b, h, a.T, a.H, n, tid);
        sEq[tid] = expf(sG[tid]);
    }
    chunk_scores<MF, V4>(q, k, Kq, sG, sStage, sA);
    float* out = a.out + (bh * a.Tp + t0) * Vd;
    for (int d0 = 0; d0 < Vd; d0 += BC * NT) {
        float acc[NA][4] = {};
        tile_gemm_nt<MF, false, NT>(RK(q, Kq, BC, Kq), SJ(S + d0, Vd, Kq, Vd - d0), Kq, sStage, acc);
        tile_scale_rows<MF, NA>(acc, [&](int t) { return sEq[t]; });
        tile_gemm_nt<MF, false, NT>([&](int i, int kk) { return sA[i][kk]; }, RJ(v + d0, Vd, BC, Vd - d0), BC,
                                    sStage, acc);
        if (!a.out_bthd) {
            if (a.bf16) {
#pragma unroll
                for (int i = 0; i < NA; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[i][j] = (float)(bf16_t)(a.scale * acc[i][j]);
                tile_store<MF, NA>(acc, out, Vd, d0, 1.f);
            } else {
                tile_store<MF, NA>(acc, out, Vd, d0, a.scale);
            }
            continue;
        }
#pragma unroll
        for (int i = 0; i < NA; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = t0 + TileMap<MF>::row(i, j), c = d0 + TileMap<MF>::col(i, j);
                if (c >= Vd || t >= a.T) continue;
                const size_t e = (((size_t)b * a.T + t) * a.H + h) * Vd + c;
                if (a.bf16)
                    reinterpret_cast<bf16_t*>(a.out_bthd)[e] = (bf16_t)(a.scale * acc[i][j]);
                else
                    reinterpret_cast<float*>(a.out_bthd)[e] = a.scale * acc[i][j];
            }
    }
}

// Cotangents of one chunk's rows: dq, dk (Kq) and dv (Vd) for its 64 tokens
// from S_n (state before the chunk), D_{n+1} (cotangent after it) and the
// two masked decayed score matrices A (q.k) and B (dO.v), each output tile
// (64 tokens x 64 coordinates) as two tile GEMMs. Grid (N, H, B), 256 threads.
struct ChunkGradArgs {
    const float *q, *k, *v, *dO;  // head-major [B*H, Tp, Kq | Vd]
    const float* g;               // [B, T, H]
    const float *S, *D;           // [B*H, N+1, Kq, Vd]: fp32, or bf16_t with sbf
    float *dq, *dk, *dv;          // head-major
    int B, T, Tp, H, Kq, Vd, N;
    float scale;
    int sbf;                      // matrix-core form: S and D hold bf16 states
    int rbf;                      // matrix-core form: v and dO hold bf16 rows
};

template <bool MF, bool V4, bool SB, bool RB>
__global__ __launch_bounds__(256) void bw_chunk_kernel(ChunkGradArgs a) {
    using RK = std::conditional_t<V4, RowsK4, RowsK>;  // 16-byte row loads when aligned
    using RJ = std::conditional_t<V4, RowsJ4, RowsJ>;
    using SK = StateRowsK<SB, V4>;  // the states' rows
    using SJ = StateRowsJ<SB, V4>;
    using SE = std::conditional_t<SB, bf16_t, float>;
    using VK = StateRowsK<RB, V4>;  // v's and dO's rows
    using VJ = StateRowsJ<RB, V4>;
    using VE = std::conditional_t<RB, bf16_t, float>;
    __shared__ float sA[BC][BC + 1], sB[BC][BC + 1];
    // Output tiles of 64 NT columns: on the matrix cores two at a time, so that
    // each row block a product reads (dO, v, k, and the other operands' rows)
    // is read once per pair of tiles (the kernel reads HBM at its rate: 222 ->
    // 184 us at configuration 3)
    constexpr int NT = MF && V4 ? 2 : 1, NA = 4 * NT;
    __shared__ __align__(16) unsigned char sStage[NT == 2 ? STAGE2_BYTES : STAGE_BYTES];
    // (the row factors e^{G_t} and e^{G_last - G_t} are formed where used)
    __shared__ float sG[BC];
    const int tid = threadIdx.x, n = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int Kq = a.Kq, Vd = a.Vd, t0 = n * BC;
    const size_t bh = (size_t)b * a.H + h, ssz = (size_t)Kq * Vd;
    const float* q = a.q + (bh * a.Tp + t0) * Kq;
    const float* k = a.k + (bh * a.Tp + t0) * Kq;
    const VE* v = reinterpret_cast<const VE*>(a.v) + (bh * a.Tp + t0) * Vd;
    const VE* dO = reinterpret_cast<const VE*>(a.dO) + (bh * a.Tp + t0) * Vd;
    const SE* S = reinterpret_cast<const SE*>(a.S) + (bh * (a.N + 1) + n) * ssz;
    const SE* D = reinterpret_cast<const SE*>(a.D) + (bh * (a.N + 1) + n + 1) * ssz;
    if (tid < 64) {
        const float G = chunk_gam(a.g, b, h, a.T, a.H, n, tid);
        sG[tid] = G;
    }
    chunk_scores<MF, V4>(q, k, Kq, sG, sStage, sA);
    chunk_scores<MF, V4>(dO, v, Vd, sG, sStage, sB);
    const float sc = a.scale;
    for (int d0 = 0; d0 < Kq; d0 += BC * NT) {
        // dq = scale (e^{G_t} dO_t S_n^T + B k)
        float acc[NA][4] = {};
        tile_gemm_nt<MF, true, NT>(VK(dO, Vd, BC, Vd), SK(S + (size_t)d0 * Vd, Vd, Kq - d0, Vd), Vd, sStage, acc);
        tile_scale_rows<MF, NA>(acc, [&](int t) { return expf(sG[t]); });
        tile_gemm_nt<MF, false, NT>([&](int i, int kk) { return sB[i][kk]; }, RJ(k + d0, Kq, BC, Kq - d0), BC, sStage,
                             acc);
        tile_store<MF, NA>(acc, a.dq + (bh * a.Tp + t0) * Kq, Kq, d0, sc);
        // dk = e^{G_last - G_s} v_s D_{n+1}^T + scale B^T q
#pragma unroll
        for (int x = 0; x < NA; x++)
#pragma unroll
            for (int y = 0; y < 4; y++) acc[x][y] = 0.f;
        tile_gemm_nt<MF, true, NT>(VK(v, Vd, BC, Vd), SK(D + (size_t)d0 * Vd, Vd, Kq - d0, Vd), Vd, sStage, acc);
        tile_scale_rows<MF, NA>(acc, [&](int t) { return expf(sG[BC - 1] - sG[t]); });
        tile_gemm_nt<MF, false, NT>([&](int i, int kk) { return sc * sB[kk][i]; }, RJ(q + d0, Kq, BC, Kq - d0), BC,
                             sStage, acc);
        tile_store<MF, NA>(acc, a.dk + (bh * a.Tp + t0) * Kq, Kq, d0, 1.f);
    }
    for (int d0 = 0; d0 < Vd; d0 += BC * NT) {
        // dv = e^{G_last - G_s} k_s D_{n+1} + scale A^T dO
        float acc[NA][4] = {};
        tile_gemm_nt<MF, false, NT>(RK(k, Kq, BC, Kq), SJ(D + d0, Vd, Kq, Vd - d0), Kq, sStage, acc);
        tile_scale_rows<MF, NA>(acc, [&](int t) { return expf(sG[BC - 1] - sG[t]); });
        tile_gemm_nt<MF, false, NT>([&](int i, int kk) { return sc * sA[kk][i]; }, VJ(dO + d0, Vd, BC, Vd - d0), BC,
                             sStage, acc);
        tile_store<MF, NA>(acc, a.dv + (bh * a.Tp + t0) * Vd, Vd, d0, 1.f);
    }
}

// The slot readout for blocks of 32 rows of one head: z = U(lam) raw,
// l = z table^T, p = softmax(l), u = p table, weights = U(-lam) u; the two
// products as small GEMMs against the staged table on the fp32 matrix cores
// (mfma4 below). BF
// rounds z, the table, p and the weights to bf16 (the general forward's casts
// to a bf16 input dtype, ops/utils.py:779-882); the backward's recompute is
// unrounded. Grid (ceil(B Tp / (32 per_wg)), H), RO_FWD_THREADS threads: a
// workgroup stages the table once and takes per_wg blocks; the LDS holds one
// workgroup per CU, and its waves put several on each SIMD.
template <bool BF>
__device__ __forceinline__ float bw_rnd(float x) {
    if constexpr (BF)
        return (float)(bf16_t)x;
    else
        return x;
}

constexpr int RO_LD = BWD_TABLE_M + 4;  // staged table and row rows, 16-byte aligned
constexpr int RO_FWD_THREADS = 1024;

typedef float f32x4v __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x4_f32 (fp32 operands, fp32 accumulation): lane l holds
// A[l % 16][l / 16] and B[l / 16][l % 16] of a 16 x 4 by 4 x 16 step and rows
// 4 (l / 16) .. + 3 of column l % 16 of the 16 x 16 result.
__device__ __forceinline__ f32x4v mfma4(float a, float b, f32x4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <bool BF>
__global__ __launch_bounds__(RO_FWD_THREADS) void bw_fwd_readout_kernel(const float* raw, const float* cs, const float* sn,
                                                             const float* table, int B, int Tp, int H, int M,
                                                             int per_wg, float* wts) {
    constexpr int TM = BWD_TABLE_M, LD = RO_LD, RB = 32, NT = RO_FWD_THREADS, NW = NT / 64, CPW = 16 / NW;
    static_assert(TM == 128 && (NW == 8 || NW == 16), "eight 16-wide tiles of slots, two of rows");
    __shared__ float sTab[TM * LD];  // rows R .. 127 and columns M .. 127 zero
    __shared__ float sZ[RB][LD], sP[RB][LD];
    __shared__ float sCs[RB][TM / 2], sSn[RB][TM / 2];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, h = blockIdx.y;
    const int lr = lane & 15, lk = lane >> 4;
    const int R = M - 1, P = M / 2, rows = B * Tp;
    for (int e = tid; e < TM * LD; e += NT) {
        const int r = e / LD, m = e % LD;
        sTab[e] = (r < R && m < M) ? bw_rnd<BF>(table[((size_t)h * R + r) * M + m]) : 0.f;
    }
    const auto row_of = [&](int rho) { return ((size_t)(rho / Tp) * H + h) * Tp + rho % Tp; };
    // wave wv: row tile it = wv & 1, column tiles CPW (wv >> 1) .. + CPW - 1 (of r, then of m)
    const int it = wv & 1, ct0 = CPW * (wv >> 1);
    // A block's inputs, element x of this thread = (row i, pair pr) = e / 64,
    // e % 64, e = tid + NT x: loaded one block ahead through buffer
    // resources (rows < 2^21, M <= 128: offsets below 2^30), predicated
    // through the offset, so that no block waits for its own loads.
    constexpr int NX = RB * (TM / 2) / NT;
    const int b_end = min(rows, (int)(blockIdx.x + 1) * per_wg * RB);
    const bw_rsrc_t rcs = bw_rsrc(cs, (size_t)rows * H * P), rsn = bw_rsrc(sn, (size_t)rows * H * P),
                    rraw = bw_rsrc(raw, (size_t)rows * H * M);  // every head's rows
    float nc[NX], ns[NX], nre[NX], nro[NX];
    const auto load_block = [&](int b0) {
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2), rho = b0 + i;
            const bool live = rho < b_end && pr < P;
            const uint32_t row = live ? (uint32_t)row_of(rho) : 0u;
            nc[x] = bw_load(rcs, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            ns[x] = bw_load(rsn, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            nre[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr) * 4u, live);
            nro[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr + 1u) * 4u, live);
        }
    };
    const int b_first = blockIdx.x * per_wg * RB;
    load_block(b_first);
    for (int b0 = b_first; b0 < b_end; b0 += RB) {
        __syncthreads();  // the table is staged; the previous block's tiles are done with
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2);
            const bool live = b0 + i < b_end && pr < P;
            const float c = live ? nc[x] : 1.f, s = ns[x];
            sCs[i][pr] = c;
            sSn[i][pr] = s;
            sZ[i][2 * pr] = bw_rnd<BF>(c * nre[x] - s * nro[x]);  // zero where !live
            sZ[i][2 * pr + 1] = bw_rnd<BF>(s * nre[x] + c * nro[x]);
        }
        load_block(b0 + RB);  // the next block (past the end: dead loads)
        __syncthreads();
        {  // logits l[i][r] = sum_m z[i][m] table[r][m]
            f32x4v acc[CPW];
#pragma unroll
            for (int t = 0; t < CPW; t++) acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
            for (int k0 = 0; k0 < TM; k0 += 4) {
                const float az = sZ[16 * it + lr][k0 + lk];
#pragma unroll
                for (int t = 0; t < CPW; t++) acc[t] = mfma4(az, sTab[(16 * (ct0 + t) + lr) * LD + k0 + lk], acc[t]);
            }
#pragma unroll
            for (int t = 0; t < CPW; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) sP[16 * it + 4 * lk + q][16 * (ct0 + t) + lr] = acc[t][q];
        }
        __syncthreads();
        for (int i = wv; i < RB; i += NW) {
            const float l0 = lane < R ? sP[i][lane] : -INFINITY, l1 = lane + 64 < R ? sP[i][lane + 64] : -INFINITY;
            const float mx = bw_wave_max(fmaxf(l0, l1));
            const float e0 = lane < R ? expf(l0 - mx) : 0.f, e1 = lane + 64 < R ? expf(l1 - mx) : 0.f;
            const float inv = 1.f / bw_wave_sum(e0 + e1);
            sP[i][lane] = bw_rnd<BF>(e0 * inv);
            sP[i][lane + 64] = bw_rnd<BF>(e1 * inv);
        }
        __syncthreads();
        // u[i][m] = sum_r p[i][r] table[r][m] (p and the table zero at r >= R); the
        // weights' pair (2 pr, 2 pr + 1) sits in lanes (lr, lr ^ 1), swapped in by
        // quad_perm [1,0,3,2]
        f32x4v acc[CPW];
#pragma unroll
        for (int t = 0; t < CPW; t++) acc[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < TM; k0 += 4) {
            const float ap = sP[16 * it + lr][k0 + lk];
#pragma unroll
            for (int t = 0; t < CPW; t++) acc[t] = mfma4(ap, sTab[(k0 + lk) * LD + 16 * (ct0 + t) + lr], acc[t]);
        }
        const bool odd = (lr & 1) != 0;
#pragma unroll
        for (int t = 0; t < CPW; t++) {
            const int m = 16 * (ct0 + t) + lr, pr = m >> 1;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float un = acc[t][q], ux = dpp_mov<0xB1>(un);
                const float ue = odd ? ux : un, uo = odd ? un : ux;
                const int i = 16 * it + 4 * lk + q, rho = b0 + i;
                if (rho < rows && pr < P) {
                    const float c = sCs[i][pr], s = sSn[i][pr];
                    wts[row_of(rho) * M + m] = bw_rnd<BF>(odd ? -s * ue + c * uo : c * ue + s * uo);
                }
            }
        }
    }
}

// The same readout with its two products as split-bf16 products on
// v_mfma_f32_16x16x32_bf16 (every fp32 operand as a bf16 high part and a bf16
// remainder, lo_a hi_b + hi_a lo_b + hi_a hi_b: about 16 mantissa bits; with
// BF the operands are bf16 values and the products exact), for calls whose
// tile products run on the matrix cores. The table sits in LDS once as its
// two bf16 parts, row-major [r][m]: the logits read its rows as B fragments,
// u gathers its columns. Wave w takes row tile w & 1 and the slot tiles
// CPW (w >> 1) .. + CPW - 1 of both products (CPW = 16 / waves); the softmax
// reductions on DPP moves.
constexpr int RO_LDB = BWD_TABLE_M + 8;  // bf16 rows of the split table and row blocks
// One workgroup per CU fits the LDS; its waves put several on each SIMD, so
// that one wave's LDS reads and softmax overlap another's products.
constexpr int RO_MF_THREADS = 1024;

// lane (lr, lg) gets X[r0 + lr][k0 + 8 lg .. + 7] of a row-major bf16 tile
__device__ __forceinline__ bf16x8 ro_row(const bf16_t* X, int r0, int k0) {
    const int l = threadIdx.x & 63;
    return *reinterpret_cast<const bf16x8*>(X + (r0 + (l & 15)) * RO_LDB + k0 + 8 * (l >> 4));
}

// lane (lr, lg) gets X[s0 + 8 lg + j][c0 + lr], j = 0..7, of a row-major bf16
// tile (a B fragment of the transpose), as eight 2-byte LDS reads
__device__ __forceinline__ bf16x8 ro_col(const bf16_t* X, int s0, int c0) {
    const int l = threadIdx.x & 63;
    const bf16_t* p = X + (s0 + 8 * (l >> 4)) * RO_LDB + c0 + (l & 15);
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = p[e * RO_LDB];
    return r;
}

__device__ __forceinline__ void split_store(bf16_t* hi, bf16_t* lo, int idx, float v) {
    const bf16_t h = (bf16_t)v;
    hi[idx] = h;
    lo[idx] = (bf16_t)(v - (float)h);
}

template <bool BF>
__global__ __launch_bounds__(RO_MF_THREADS) void bw_fwd_readout_mf_kernel(const float* raw, const float* cs, const float* sn,
                                                                const float* table, int B, int Tp, int H, int M,
                                                                int per_wg, float* wts) {
    constexpr int TM = BWD_TABLE_M, LB = RO_LDB, RB = 32, NT = RO_MF_THREADS, NW = NT / 64, CPW = 16 / NW;
    static_assert(TM == 128 && RB == 32 && (NW == 8 || NW == 16), "eight 16-wide tiles of slots, two of rows");
    __shared__ __align__(16) bf16_t sTh[TM * LB], sTl[TM * LB];  // rows R .. 127 and columns M .. 127 zero
    __shared__ __align__(16) bf16_t sZh[RB * LB], sZl[RB * LB], sPh[RB * LB], sPl[RB * LB];
    __shared__ float sL[RB][TM + 4];
    __shared__ float sCs[RB][TM / 2], sSn[RB][TM / 2];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, h = blockIdx.y;
    const int lr = lane & 15;
    const int R = M - 1, P = M / 2, rows = B * Tp;
    for (int e = tid; e < TM * TM; e += NT) {
        const int r = e / TM, m = e % TM;
        split_store(sTh, sTl, r * LB + m, (r < R && m < M) ? bw_rnd<BF>(table[((size_t)h * R + r) * M + m]) : 0.f);
    }
    const auto row_of = [&](int rho) { return ((size_t)(rho / Tp) * H + h) * Tp + rho % Tp; };
    const int it = wv & 1, ct0 = CPW * (wv >> 1);
    constexpr int NX = RB * (TM / 2) / NT;
    const int b_end = min(rows, (int)(blockIdx.x + 1) * per_wg * RB);
    const bw_rsrc_t rcs = bw_rsrc(cs, (size_t)rows * H * P), rsn = bw_rsrc(sn, (size_t)rows * H * P),
                    rraw = bw_rsrc(raw, (size_t)rows * H * M);  // every head's rows
    float nc[NX], ns[NX], nre[NX], nro[NX];
    const auto load_block = [&](int b0) {
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2), rho = b0 + i;
            const bool live = rho < b_end && pr < P;
            const uint32_t row = live ? (uint32_t)row_of(rho) : 0u;
            nc[x] = bw_load(rcs, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            ns[x] = bw_load(rsn, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            nre[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr) * 4u, live);
            nro[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr + 1u) * 4u, live);
        }
    };
    const int b_first = blockIdx.x * per_wg * RB;
    load_block(b_first);
    for (int b0 = b_first; b0 < b_end; b0 += RB) {
        __syncthreads();  // the table is staged; the previous block's tiles are done with
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2);
            const bool live = b0 + i < b_end && pr < P;
            const float c = live ? nc[x] : 1.f, s = ns[x];
            sCs[i][pr] = c;
            sSn[i][pr] = s;
            split_store(sZh, sZl, i * LB + 2 * pr, bw_rnd<BF>(c * nre[x] - s * nro[x]));  // zero where !live
            split_store(sZh, sZl, i * LB + 2 * pr + 1, bw_rnd<BF>(s * nre[x] + c * nro[x]));
        }
        load_block(b0 + RB);  // the next block (past the end: dead loads)
        __syncthreads();
        {  // logits l[i][r] = sum_m z[i][m] table[r][m]
            f32x4 acc[CPW];
#pragma unroll
            for (int t = 0; t < CPW; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k0 = 0; k0 < TM; k0 += 32) {
                const bf16x8 ah = ro_row(sZh, 16 * it, k0), al = ro_row(sZl, 16 * it, k0);
#pragma unroll
                for (int t = 0; t < CPW; t++) {
                    const bf16x8 bh = ro_row(sTh, 16 * (ct0 + t), k0), bl = ro_row(sTl, 16 * (ct0 + t), k0);
                    acc[t] = mfma_bf16(al, bh, acc[t]);
                    acc[t] = mfma_bf16(ah, bl, acc[t]);
                    acc[t] = mfma_bf16(ah, bh, acc[t]);
                }
            }
            const int lg = lane >> 4;
#pragma unroll
            for (int t = 0; t < CPW; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) sL[16 * it + 4 * lg + q][16 * (ct0 + t) + lr] = acc[t][q];
        }
        __syncthreads();
        for (int i = wv; i < RB; i += NW) {
            const float l0 = lane < R ? sL[i][lane] : -INFINITY, l1 = lane + 64 < R ? sL[i][lane + 64] : -INFINITY;
            const float mx = bw_wave_max(fmaxf(l0, l1));
            const float e0 = lane < R ? expf(l0 - mx) : 0.f, e1 = lane + 64 < R ? expf(l1 - mx) : 0.f;
            const float inv = 1.f / bw_wave_sum(e0 + e1);
            split_store(sPh, sPl, i * LB + lane, bw_rnd<BF>(e0 * inv));
            split_store(sPh, sPl, i * LB + lane + 64, bw_rnd<BF>(e1 * inv));
        }
        __syncthreads();
        // u[i][m] = sum_r p[i][r] table[r][m] (p and the table zero at r >= R); the
        // weights' pair (2 pr, 2 pr + 1) sits in lanes (lr, lr ^ 1), swapped in by
        // quad_perm [1,0,3,2]
        f32x4 acc[CPW];
#pragma unroll
        for (int t = 0; t < CPW; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < TM; k0 += 32) {
            const bf16x8 ah = ro_row(sPh, 16 * it, k0), al = ro_row(sPl, 16 * it, k0);
#pragma unroll
            for (int t = 0; t < CPW; t++) {
                const bf16x8 bh = ro_col(sTh, k0, 16 * (ct0 + t)), bl = ro_col(sTl, k0, 16 * (ct0 + t));
                acc[t] = mfma_bf16(al, bh, acc[t]);
                acc[t] = mfma_bf16(ah, bl, acc[t]);
                acc[t] = mfma_bf16(ah, bh, acc[t]);
            }
        }
        const bool odd = (lr & 1) != 0;
        const int lk = lane >> 4;
#pragma unroll
        for (int t = 0; t < CPW; t++) {
            const int m = 16 * (ct0 + t) + lr, pr = m >> 1;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float un = acc[t][q], ux = dpp_mov<0xB1>(un);
                const float ue = odd ? ux : un, uo = odd ? un : ux;
                const int i = 16 * it + 4 * lk + q, rho = b0 + i;
                if (rho < b_end && pr < P) {
                    const float c = sCs[i][pr], s = sSn[i][pr];
                    wts[row_of(rho) * M + m] = bw_rnd<BF>(odd ? -s * ue + c * uo : c * ue + s * uo);
                }
            }
        }
    }
}

// The slot-readout adjoint for blocks of 32 rows of one head (z = U(lam) raw,
// l = table z, p = softmax(l), u = table^T p, weights = U(-lam) u):
//   du = U(lam) dweights, dp = table du, dl = p (dp - p.dp), dz = table^T dl,
//   draw = U(-lam) dz, dtable += p du^T + dl z^T, and the clock's share
//   dlam = sum_p kappa_p [dz . dU(lam)/dlam raw + dweights . dU(-lam)/dlam u]
// with kappa_p = 2 pi p / (M - 1). Every product over the block is a small
// GEMM against the head's table (staged once in LDS, rows RO_LD floats apart)
// on the fp32 matrix cores, v_mfma_f32_16x16x4_f32 (fp32 operands, fp32
// accumulation): lane l holds A[l % 16][l / 16] and B[l / 16][l % 16] of a
// 16 x 4 by 4 x 16 step and rows 4 (l / 16) .. + 3 of column l % 16 of the
// 16 x 16 result. Grid (workgroups per head, H), RO_ADJ_THREADS threads: a
// workgroup takes per_wg blocks of 32 rows (bwd_ro_per_wg) and keeps its part
// of dtable in the accumulators (wave w owns the 16 x 16 tiles (r, m) of
// columns m in 16 (w % 8) .. + 15 and rows r in 16 DRT (w / 8) .. + 16 DRT - 1,
// DRT = 64 / waves). The LDS holds one workgroup per CU; its waves put
// several on each SIMD, so that one wave's LDS reads overlap another's
// matrix-core steps.
constexpr int RO_BLK = BWD_RO_BLOCK;
constexpr int RO_ADJ_THREADS = 1024;
struct ReadoutGradArgs {
    const float *raw, *cs, *sn, *table, *dwts;  // head-major rows; table [H, M-1, M]
    float *draw, *dlam, *dtab;                  // dtab: [H, workgroups, (M-1) M]
    int B, Tp, H, M;
    int per_wg;                                 // blocks of 32 rows per workgroup
};

__global__ __launch_bounds__(RO_ADJ_THREADS) void bw_readout_kernel(ReadoutGradArgs a) {
    constexpr int TM = BWD_TABLE_M, LD = RO_LD, NT = RO_ADJ_THREADS, NW = NT / 64;
    constexpr int CPW = 16 / NW, DRT = 64 / NW;  // slot tiles per wave in the block products; dtable row tiles
    static_assert(NW == 8 || NW == 16, "two row tiles x eight slot tiles over the waves; eight dtable column tiles");
    static_assert(RO_BLK == 32 && TM == 128, "two 16-row tiles of rows, eight 16-wide tiles of slots");
    __shared__ float sTab[TM * LD];  // rows R .. 127 and columns M .. 127 zero
    __shared__ float sZ[RO_BLK][LD], sDU[RO_BLK][LD], sP[RO_BLK][LD], sDL[RO_BLK][LD];
    __shared__ float sCs[RO_BLK][TM / 2], sSn[RO_BLK][TM / 2];
    __shared__ float sLam[RO_BLK][NW / 2];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, blk = blockIdx.x, h = blockIdx.y;
    const int lr = lane & 15, lk = lane >> 4;  // operand row / column and k of this lane
    const int M = a.M, R = M - 1, P = M / 2, RM = R * M;
    for (int e = tid; e < TM * LD; e += NT) {  // the table, zero beyond R x M
        const int r = e / LD, m = e % LD;
        sTab[e] = (r < R && m < M) ? a.table[((size_t)h * R + r) * M + m] : 0.f;
    }
    // GEMMs over the block: wave wv takes row tile it = wv & 1 and the column
    // tiles CPW (wv >> 1) .. + CPW - 1 of the logits (r) and of dz, u (m)
    const int it = wv & 1, ct0 = CPW * (wv >> 1), dm = wv & 7, dr0 = DRT * (wv >> 3);
    f32x4v dacc[DRT];  // dtable tiles (r tile dr0 + rt, m tile dm)
#pragma unroll
    for (int rt = 0; rt < DRT; rt++) dacc[rt] = f32x4v{0.f, 0.f, 0.f, 0.f};
    const int rows = a.B * a.Tp;
    // A block's inputs, element x of this thread = (row i, pair pr) = e / 64,
    // e % 64, e = tid + NT x: loaded one block ahead through buffer
    // resources (rows < 2^21, M <= 128: offsets below 2^30), predicated
    // through the offset, so that no block waits for its own loads.
    constexpr int NX = RO_BLK * (TM / 2) / NT;
    const int b_end = min(rows, (blk + 1) * a.per_wg * RO_BLK);
    const bw_rsrc_t rcs = bw_rsrc(a.cs, (size_t)rows * a.H * P), rsn = bw_rsrc(a.sn, (size_t)rows * a.H * P),
                    rraw = bw_rsrc(a.raw, (size_t)rows * a.H * M), rdw = bw_rsrc(a.dwts, (size_t)rows * a.H * M);
    float nc[NX], ns[NX], nre[NX], nro[NX], nde[NX], ndd[NX];
    const auto load_block = [&](int b0) {
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2), rho = b0 + i;
            const bool live = rho < b_end && pr < P;
            const uint32_t row = live ? (uint32_t)(((rho / a.Tp) * a.H + h) * a.Tp + rho % a.Tp) : 0u;
            nc[x] = bw_load(rcs, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            ns[x] = bw_load(rsn, (row * (uint32_t)P + (uint32_t)pr) * 4u, live);
            nre[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr) * 4u, live);
            nro[x] = bw_load(rraw, (row * (uint32_t)M + 2u * (uint32_t)pr + 1u) * 4u, live);
            nde[x] = bw_load(rdw, (row * (uint32_t)M + 2u * (uint32_t)pr) * 4u, live);
            ndd[x] = bw_load(rdw, (row * (uint32_t)M + 2u * (uint32_t)pr + 1u) * 4u, live);
        }
    };
    const int b_first = blk * a.per_wg * RO_BLK;
    load_block(b_first);
    for (int b0 = b_first; b0 < b_end; b0 += RO_BLK) {
        __syncthreads();  // the previous block's tiles are done with
        // z = U(lam) raw and du = U(lam) dweights
#pragma unroll
        for (int x = 0; x < NX; x++) {
            const int e = tid + NT * x, i = e / (TM / 2), pr = e % (TM / 2);
            const bool live = b0 + i < b_end && pr < P;
            const float c = live ? nc[x] : 1.f, s = ns[x];  // zero inputs where !live
            sCs[i][pr] = c;
            sSn[i][pr] = s;
            sZ[i][2 * pr] = c * nre[x] - s * nro[x];
            sZ[i][2 * pr + 1] = s * nre[x] + c * nro[x];
            sDU[i][2 * pr] = c * nde[x] - s * ndd[x];
            sDU[i][2 * pr + 1] = s * nde[x] + c * ndd[x];
        }
        load_block(b0 + RO_BLK);  // the next block (past the end: dead loads)
        __syncthreads();
        // logits l[i][r] = sum_m z[i][m] table[r][m] and dp[i][r] = sum_m du[i][m] table[r][m]
        {
            f32x4v accl[CPW], accd[CPW];
#pragma unroll
            for (int t = 0; t < CPW; t++) accl[t] = accd[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
            for (int k0 = 0; k0 < TM; k0 += 4) {
                const float az = sZ[16 * it + lr][k0 + lk], ad = sDU[16 * it + lr][k0 + lk];
#pragma unroll
                for (int t = 0; t < CPW; t++) {
                    const float bt = sTab[(16 * (ct0 + t) + lr) * LD + k0 + lk];
                    accl[t] = mfma4(az, bt, accl[t]);
                    accd[t] = mfma4(ad, bt, accd[t]);
                }
            }
#pragma unroll
            for (int t = 0; t < CPW; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    sP[16 * it + 4 * lk + q][16 * (ct0 + t) + lr] = accl[t][q];
                    sDL[16 * it + 4 * lk + q][16 * (ct0 + t) + lr] = accd[t][q];
                }
        }
        __syncthreads();
        // softmax and dl per row: wave wv takes rows wv, wv + NW, ...; lanes take slots lane, lane + 64
        for (int i = wv; i < RO_BLK; i += NW) {
            const float l0 = lane < R ? sP[i][lane] : -INFINITY, l1 = lane + 64 < R ? sP[i][lane + 64] : -INFINITY;
            const float mx = bw_wave_max(fmaxf(l0, l1));
            const float e0 = lane < R ? expf(l0 - mx) : 0.f, e1 = lane + 64 < R ? expf(l1 - mx) : 0.f;
            const float inv = 1.f / bw_wave_sum(e0 + e1);
            const float p0 = e0 * inv, p1 = e1 * inv;
            const float d0 = sDL[i][lane], d1 = sDL[i][lane + 64];
            const float pdp = bw_wave_sum(p0 * d0 + p1 * d1);
            sP[i][lane] = p0;
            sP[i][lane + 64] = p1;
            sDL[i][lane] = p0 * (d0 - pdp);
            sDL[i][lane + 64] = p1 * (d1 - pdp);
        }
        __syncthreads();
        // dz[i][m] = sum_r dl[i][r] table[r][m] and u[i][m] = sum_r p[i][r] table[r][m]
        // (p and dl are zero at r >= R, as is the table); then draw and the clock's share
        {
            f32x4v accz[CPW], accu[CPW];
#pragma unroll
            for (int t = 0; t < CPW; t++) accz[t] = accu[t] = f32x4v{0.f, 0.f, 0.f, 0.f};
            for (int k0 = 0; k0 < TM; k0 += 4) {
                const float al = sDL[16 * it + lr][k0 + lk], ap = sP[16 * it + lr][k0 + lk];
#pragma unroll
                for (int t = 0; t < CPW; t++) {
                    const float bt = sTab[(k0 + lk) * LD + 16 * (ct0 + t) + lr];
                    accz[t] = mfma4(al, bt, accz[t]);
                    accu[t] = mfma4(ap, bt, accu[t]);
                }
            }
            // lane holds rows i = 16 it + 4 lk + q of column m = 16 (ct0 + t) + lr; the pair
            // (2 pr, 2 pr + 1) sits in lanes (lr, lr ^ 1), swapped in by quad_perm [1,0,3,2].
            // With z = U(lam) raw and du = U(lam) dweights, the clock's share
            // kappa_p [dz . dU(lam)/dlam raw + dweights . dU(-lam)/dlam u] is
            // kappa_p [(z_e dz_o - z_o dz_e) + (du_e u_o - du_o u_e)] (a rotation keeps
            // the 2-d cross product); the even lane of a pair forms it.
            const bool odd = (lr & 1) != 0;
            float dl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < CPW; t++) {
                const int m = 16 * (ct0 + t) + lr, pr = m >> 1;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float gz = accz[t][q], gx = dpp_mov<0xB1>(gz);
                    const float gu = accu[t][q], ux = dpp_mov<0xB1>(gu);
                    const float ge = odd ? gx : gz, go = odd ? gz : gx, ue = odd ? ux : gu, uo = odd ? gu : ux;
                    const int i = 16 * it + 4 * lk + q, rho = b0 + i;
                    if (rho < rows && pr < P) {
                        const size_t row = ((size_t)(rho / a.Tp) * a.H + h) * a.Tp + rho % a.Tp;
                        const float c = sCs[i][pr], s = sSn[i][pr];
                        a.draw[row * M + m] = odd ? -s * ge + c * go : c * ge + s * go;
                        if (!odd) {
                            const float ze = sZ[i][2 * pr], zo = sZ[i][2 * pr + 1];
                            const float de = sDU[i][2 * pr], dd = sDU[i][2 * pr + 1];
                            dl[q] += (float)(kTwoPiBw * pr / R) * ((ze * go - zo * ge) + (de * uo - dd * ue));
                        }
                    }
                }
            }
            // the row's share over this wave's 16 lanes (its column tiles summed above,
            // in tile order), then the waves of the row tile in wave order
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float v = wave_sum<16>(dl[q]);
                if (lr == 0) sLam[16 * it + 4 * lk + q][wv >> 1] = v;
            }
        }
        __syncthreads();
        if (tid < RO_BLK && b0 + tid < rows) {  // the clock's share per row
            const int rho = b0 + tid;
            float v = sLam[tid][0];
#pragma unroll
            for (int j = 1; j < NW / 2; j++) v += sLam[tid][j];
            a.dlam[((size_t)(rho / a.Tp) * a.H + h) * a.Tp + rho % a.Tp] = v;
        }
        // dtable[r][m] += sum_i p[i][r] du[i][m] + dl[i][r] z[i][m] over the block's rows
        for (int k0 = 0; k0 < RO_BLK; k0 += 4) {
            const float bu = sDU[k0 + lk][16 * dm + lr], bz = sZ[k0 + lk][16 * dm + lr];
#pragma unroll
            for (int rt = 0; rt < DRT; rt++) {
                const float ap = sP[k0 + lk][16 * (dr0 + rt) + lr], al = sDL[k0 + lk][16 * (dr0 + rt) + lr];
                dacc[rt] = mfma4(ap, bu, dacc[rt]);
                dacc[rt] = mfma4(al, bz, dacc[rt]);
            }
        }
    }
    // lane holds dtable rows 16 (dr0 + rt) + 4 lk + q of column 16 dm + lr
    float* dst = a.dtab + ((size_t)h * gridDim.x + blk) * RM;
#pragma unroll
    for (int rt = 0; rt < DRT; rt++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int r = 16 * (dr0 + rt) + 4 * lk + q, m = 16 * dm + lr;
            if (r < R && m < M) dst[r * M + m] = dacc[rt][q];
        }
}

// The readout and its adjoint for 128 < M <= 256 slots, where a head's table
// (up to 255 x 256 fp32) does not fit in LDS beside the row blocks: every
// product is a 64 x 64 fp32 tile GEMM (tile_gemm<false>) that streams the
// table from memory, and the softmax and its adjoint run per row between
// them. Token rows rho of head h are the B Tp rows (b, h, t), rho = b Tp + t,
// at head-major row ((b H + h) Tp + t); X_lam(rho)[m] is U(lam) x (pairs
// rotated by the row's phases, as z = U(lam) raw and du = U(lam) dweights).
// Per-row intermediates have MW = 256 columns.
constexpr int BW_WIDE_MW = BWD_WIDE_MW;        // columns of the wide path's per-row buffers
constexpr int BW_WIDE_SPLIT = BWD_WIDE_SPLIT;  // token rows per dtable partial
constexpr int BW_WIDE_CT = BW_WIDE_MW / BC;    // column tiles of a row (the clock's partials)

struct WideArgs {
    const float *raw, *cs, *sn, *table, *dwts;  // head-major rows; table [H, M-1, M]
    float *lg, *dl;                             // [B H Tp, MW]: logits then p; dp then dl
    float *wts, *draw, *dlp, *dlam;             // dlp [B H Tp, BW_WIDE_CT]: the clock's partials
    float* dtab;                                // [H, splits, (M-1) M]
    int B, Tp, H, M, splits;
    int bf;                                     // forward: round z, the table, p and the weights to bf16
};

__device__ __forceinline__ float wide_rnd(const WideArgs& a, float x) { return a.bf ? (float)(bf16_t)x : x; }

__device__ __forceinline__ size_t wide_row(const WideArgs& a, int h, int rho) {
    return ((size_t)(rho / a.Tp) * a.H + h) * a.Tp + rho % a.Tp;
}

// Element m of U(lam) x for head-major row `row` (x = raw or dweights).
__device__ __forceinline__ float wide_rot(const WideArgs& a, const float* x, size_t row, int m) {
    const int P = a.M / 2, pr = m >> 1;
    const float c = a.cs[row * P + pr], s = a.sn[row * P + pr];
    const float e = x[row * a.M + 2 * pr], o = x[row * a.M + 2 * pr + 1];
    return (m & 1) ? s * e + c * o : c * e - s * o;
}

// out[row][r] = sum_m X_lam(rho)[m] table[h][r][m] for a 64-row block and 64
// table rows (X = raw: the logits into lg; X = dweights: dp into dl).
// Grid (ceil(B Tp / 64), ceil((M - 1) / 64), H).
template <bool ADJ>
__global__ __launch_bounds__(256) void bw_wide_logits_kernel(WideArgs a) {
    __shared__ __align__(16) unsigned char sStage[STAGE_BYTES];
    const int rho0 = blockIdx.x * BC, r0 = blockIdx.y * BC, h = blockIdx.z;
    const int M = a.M, R = M - 1, rows = a.B * a.Tp;
    const float* x = ADJ ? a.dwts : a.raw;
    const float* tb = a.table + (size_t)h * R * M;
    float acc[4][4] = {};
    tile_gemm<false, true>(
        [&](int i, int m) {
            return rho0 + i < rows ? wide_rnd(a, wide_rot(a, x, wide_row(a, h, rho0 + i), m)) : 0.f;
        },
        [&](int m, int j) { return r0 + j < R ? wide_rnd(a, tb[(size_t)(r0 + j) * M + m]) : 0.f; }, M, sStage, acc);
    float* out = ADJ ? a.dl : a.lg;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rho = rho0 + TileMap<false>::row(i, 0);
        if (rho >= rows) continue;
        const size_t row = wide_row(a, h, rho);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r0 + TileMap<false>::col(i, j);
            if (r < R) out[row * BW_WIDE_MW + r] = acc[i][j];
        }
    }
}

// Per row, one wave: p = softmax(logits) over the R = M - 1 slots into lg;
// ADJ: dl = p (dp - p.dp) into dl (p already in lg). Grid ceil(B H Tp / 4).
template <bool ADJ>
__global__ __launch_bounds__(256) void bw_wide_softmax_kernel(WideArgs a) {
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, R = a.M - 1;
    if (row >= (size_t)a.B * a.H * a.Tp) return;
    float* lg = a.lg + row * BW_WIDE_MW;
    float v[4];
    if (!ADJ) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = lane + 64 * i;
            v[i] = r < R ? lg[r] : -INFINITY;
            mx = fmaxf(mx, v[i]);
        }
        mx = bw_wave_max(mx);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[i] = lane + 64 * i < R ? expf(v[i] - mx) : 0.f;
            sum += v[i];
        }
        const float inv = 1.f / bw_wave_sum(sum);
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i < R) lg[lane + 64 * i] = wide_rnd(a, v[i] * inv);
    } else {
        float* dl = a.dl + row * BW_WIDE_MW;
        float pv[4], pdp = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = lane + 64 * i;
            pv[i] = r < R ? lg[r] : 0.f;
            v[i] = r < R ? dl[r] : 0.f;
            pdp += pv[i] * v[i];
        }
        pdp = bw_wave_sum(pdp);
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i < R) dl[lane + 64 * i] = pv[i] * (v[i] - pdp);
    }
}

// u = p table for a 64-row block and 64 columns (m0 ..), then
//   forward: weights = U(-lam) u into wts;
//   ADJ: dz = dl table as well; draw = U(-lam) dz, and the clock's share of
//   the block's pairs, kappa_p [(z_e dz_o - z_o dz_e) + (du_e u_o - du_o u_e)],
//   summed over the tile's pairs in column order into dlp[row][m0 / 64].
// Grid (ceil(B Tp / 64), ceil(M / 64), H).
template <bool ADJ>
__global__ __launch_bounds__(256) void bw_wide_u_kernel(WideArgs a) {
    __shared__ __align__(16) unsigned char sStage[STAGE_BYTES];
    __shared__ float sPart[BC][17];
    const int tid = threadIdx.x, rho0 = blockIdx.x * BC, m0 = blockIdx.y * BC, h = blockIdx.z;
    const int M = a.M, R = M - 1, P = M / 2, rows = a.B * a.Tp;
    const float* tb = a.table + (size_t)h * R * M;
    const auto tab = [&](int r, int j) { return m0 + j < M ? wide_rnd(a, tb[(size_t)r * M + m0 + j]) : 0.f; };
    float u[4][4] = {}, dz[4][4] = {};
    tile_gemm<false, false>(
        [&](int i, int r) { return rho0 + i < rows ? a.lg[wide_row(a, h, rho0 + i) * BW_WIDE_MW + r] : 0.f; }, tab, R,
        sStage, u);
    if (ADJ)
        tile_gemm<false, false>(
            [&](int i, int r) { return rho0 + i < rows ? a.dl[wide_row(a, h, rho0 + i) * BW_WIDE_MW + r] : 0.f; },
            tab, R, sStage, dz);
    const int cg = tid & 15;  // this thread's four columns m0 + 4 cg ..: pairs (m0 + 4 cg) / 2 and + 1
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int ri = TileMap<false>::row(i, 0), rho = rho0 + ri;
        float dls = 0.f;
        if (rho < rows) {
            const size_t row = wide_row(a, h, rho);
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                const int m = m0 + TileMap<false>::col(i, j), pr = m >> 1;
                if (pr >= P) continue;
                const float c = a.cs[row * P + pr], s = a.sn[row * P + pr];
                if (!ADJ) {
                    a.wts[row * M + m] = wide_rnd(a, c * u[i][j] + s * u[i][j + 1]);
                    a.wts[row * M + m + 1] = wide_rnd(a, -s * u[i][j] + c * u[i][j + 1]);
                } else {
                    const float ge = dz[i][j], go = dz[i][j + 1], ue = u[i][j], uo = u[i][j + 1];
                    a.draw[row * M + m] = c * ge + s * go;
                    a.draw[row * M + m + 1] = -s * ge + c * go;
                    const float ze = wide_rot(a, a.raw, row, m), zo = wide_rot(a, a.raw, row, m + 1);
                    const float de = wide_rot(a, a.dwts, row, m), dd = wide_rot(a, a.dwts, row, m + 1);
                    dls += (float)(kTwoPiBw * pr / R) * ((ze * go - zo * ge) + (de * uo - dd * ue));
                }
            }
        }
        if (ADJ) sPart[ri][cg] = dls;
    }
    if (ADJ) {
        __syncthreads();
        if (tid < BC && rho0 + tid < rows) {
            float t = 0.f;
            for (int g = 0; g < 16; g++) t += sPart[tid][g];
            a.dlp[wide_row(a, h, rho0 + tid) * BW_WIDE_CT + blockIdx.y] = t;
        }
    }
}

// The readout's share of the clock cotangent: the column tiles' partials in
// order. One thread per head-major row.
__global__ __launch_bounds__(256) void bw_wide_dlam_kernel(WideArgs a) {
    const size_t row = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (row >= (size_t)a.B * a.H * a.Tp) return;
    const int nt = (a.M + BC - 1) / BC;
    float t = 0.f;
    for (int c = 0; c < nt; c++) t += a.dlp[row * BW_WIDE_CT + c];
    a.dlam[row] = t;
}

// dtable[h][r][m] partial over token rows [split BW_WIDE_SPLIT, + BW_WIDE_SPLIT):
// sum_rho p[rho][r] du[rho][m] + dl[rho][r] z[rho][m], for 64 table rows and
// 64 columns. Grid (ceil((M - 1) / 64), ceil(M / 64), H splits).
__global__ __launch_bounds__(256) void bw_wide_dtable_kernel(WideArgs a) {
    __shared__ __align__(16) unsigned char sStage[STAGE_BYTES];
    const int r0 = blockIdx.x * BC, m0 = blockIdx.y * BC, h = blockIdx.z / a.splits, sp = blockIdx.z % a.splits;
    const int M = a.M, R = M - 1, rows = a.B * a.Tp, k0 = sp * BW_WIDE_SPLIT;
    const int Kd = min(BW_WIDE_SPLIT, rows - k0);
    float acc[4][4] = {};
    tile_gemm<false, false>(
        [&](int i, int k) { return r0 + i < R ? a.lg[wide_row(a, h, k0 + k) * BW_WIDE_MW + r0 + i] : 0.f; },
        [&](int k, int j) { return m0 + j < M ? wide_rot(a, a.dwts, wide_row(a, h, k0 + k), m0 + j) : 0.f; }, Kd,
        sStage, acc);
    tile_gemm<false, false>(
        [&](int i, int k) { return r0 + i < R ? a.dl[wide_row(a, h, k0 + k) * BW_WIDE_MW + r0 + i] : 0.f; },
        [&](int k, int j) { return m0 + j < M ? wide_rot(a, a.raw, wide_row(a, h, k0 + k), m0 + j) : 0.f; }, Kd,
        sStage, acc);
    float* dst = a.dtab + ((size_t)h * a.splits + sp) * R * M;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = r0 + TileMap<false>::row(i, j), m = m0 + TileMap<false>::col(i, j);
            if (r < R && m < M) dst[(size_t)r * M + m] = acc[i][j];
        }
}

// Per chunk of (b, h): the gate cotangent of both passes (dL/dG_t = q.dq -
// k.dk, plus <D_{n+1}, S_{n+1}> at the chunk's last token, then the in-chunk
// reverse cumsum), and the write vector's (w = beta a(lam), a[2p] = s_p cos
// theta_p, a[2p+1] = -s_p sin theta_p, dw = the pass-1 value cotangent + the
// pass-2 key cotangent): dbeta = dw . a, and dlam = beta dw . da/dlam + the
// readout's share. Grid (N, B*H), 256 threads: wave w forms tokens w, w + 4,
// .. (two at a time) with its lanes across the row (coalesced 16- and 8-byte
// loads), then wave 0 scans.
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

template <bool V4>
__global__ __launch_bounds__(256) void bw_token_kernel(TokenGradArgs a) {
    __shared__ float sdG[BC], sdB[BC], sdL[BC];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
    const int K = a.K, M = a.M, P = M / 2, R = M - 1;
    // the write vector's per-pair factors: sqrt(1/R) for p = 0, sqrt(2/R) after;
    // the phase derivative's 2 pi p / R for the lane's pairs p = lane, lane + 64
    const float sp0 = (float)sqrt(1.0 / R), sp1 = (float)sqrt(2.0 / R);
    const float kp[2] = {(float)(kTwoPiBw * lane / R), (float)(kTwoPiBw * (lane + 64) / R)};
    // Wave wv forms the rows wv + 8 u and wv + 8 u + 4 together, so that both
    // rows' loads are in flight at once. The lane reads four consecutive
    // elements of the K-rows with V4 (K % 4 == 0), one otherwise, and the
    // pair (2 p, 2 p + 1) of the M-rows.
    for (int i0 = wv; i0 < BC; i0 += 8) {
        size_t row[2];
        float dG[2], db[2], dl[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            row[u] = (size_t)bh * a.Tp + n * BC + i0 + 4 * u;
            dG[u] = db[u] = dl[u] = 0.f;
        }
        if constexpr (!V4) {
            for (int j = lane; j < K; j += 64)
#pragma unroll
                for (int u = 0; u < 2; u++)
                    dG[u] += a.qh[row[u] * K + j] * a.dqh[row[u] * K + j] - a.kh[row[u] * K + j] * a.dkh[row[u] * K + j];
        }
        for (int j = 4 * lane; V4 && j < K; j += 256) {
            float4 q[2], dq[2], k[2], dk[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                q[u] = *reinterpret_cast<const float4*>(a.qh + row[u] * K + j);
                dq[u] = *reinterpret_cast<const float4*>(a.dqh + row[u] * K + j);
                k[u] = *reinterpret_cast<const float4*>(a.kh + row[u] * K + j);
                dk[u] = *reinterpret_cast<const float4*>(a.dkh + row[u] * K + j);
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
                dG[u] += (q[u].x * dq[u].x + q[u].y * dq[u].y + q[u].z * dq[u].z + q[u].w * dq[u].w) -
                         (k[u].x * dk[u].x + k[u].y * dk[u].y + k[u].z * dk[u].z + k[u].w * dk[u].w);
        }
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int p = lane + 64 * c;
            if (p >= P) break;
            float2 wt[2], dwt[2], w[2], d2[2], d1[2];
            float cs[2], sn[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const size_t e = row[u] * M + 2 * p;
                wt[u] = *reinterpret_cast<const float2*>(a.wts + e);
                dwt[u] = *reinterpret_cast<const float2*>(a.dwts + e);
                w[u] = *reinterpret_cast<const float2*>(a.w + e);
                d2[u] = *reinterpret_cast<const float2*>(a.dw2 + e);
                d1[u] = *reinterpret_cast<const float2*>(a.dw1 + e);
                cs[u] = a.cs[row[u] * P + p];
                sn[u] = a.sn[row[u] * P + p];
            }
            const float sp = p == 0 ? sp0 : sp1;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                dG[u] += (wt[u].x * dwt[u].x + wt[u].y * dwt[u].y) - (w[u].x * d2[u].x + w[u].y * d2[u].y);
                const float we = d1[u].x + d2[u].x, wo = d1[u].y + d2[u].y;
                db[u] = fmaf(sp, we * cs[u] - wo * sn[u], db[u]);
                dl[u] = fmaf(sp * kp[c], -we * sn[u] - wo * cs[u], dl[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float g = bw_wave_sum(dG[u]), bb = bw_wave_sum(db[u]), ll = bw_wave_sum(dl[u]);
            if (lane == 0) {
                sdG[i0 + 4 * u] = g;
                sdB[i0 + 4 * u] = bb;
                sdL[i0 + 4 * u] = ll;
            }
        }
    }
    __syncthreads();
    if (wv != 0) return;
    const int t = n * BC + lane;
    const size_t row = (size_t)bh * a.Tp + t;
    float x = sdG[lane];
    if (lane == BC - 1) {
        for (int i = 0; i < a.nt1; i++) x += a.bnd1[((size_t)bh * a.nt1 + i) * a.N + n];
        for (int i = 0; i < a.nt2; i++) x += a.bnd2[((size_t)bh * a.nt2 + i) * a.N + n];
    }
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_down(x, o);
        if (lane + o < 64) x += y;
    }
    const float bt = t < a.T ? a.beta[((size_t)b * a.T + t) * a.H + h] : 0.f;
    a.dlam[row] = fmaf(bt, sdL[lane], a.dlam[row]);
    if (t < a.T) {
        a.dg[((size_t)b * a.T + t) * a.H + h] = x;
        a.dbeta[((size_t)b * a.T + t) * a.H + h] = sdB[lane];
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
template <bool BF, int NJ>
__global__ __launch_bounds__(256) void bw_norm_kernel(const void* x, const float* w, const float* rs,
                                                      const float* dxh, int B, int T, int Tp, int H, int D, void* dx,
                                                      float* dw_part) {
    // Lane l holds columns l + 64 jj (jj < NJ, NJ 64 >= D); the global
    // accesses go through buffer resources over one row, columns past D
    // predicated through the offset (no branch among the loads), and a wave
    // takes its rows in groups of RB: every load of a group is issued before
    // the first row's arithmetic, so the group waits for memory once.
    constexpr int ES = BF ? 2 : 4;
    constexpr int RPW = BWD_NORM_ROWS / 4;                   // rows per wave
    constexpr int RB = 32 / NJ < RPW ? (32 / NJ > 0 ? 32 / NJ : 1) : RPW;
    static_assert(RPW % RB == 0, "whole groups");
    __shared__ float sdw[4][NJ * 64];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, blk = blockIdx.x;
    const int total = B * T * H;
    float dwa[NJ], wj[NJ];
    const bw_rsrc_t rw = bw_rsrc(w, (size_t)D);
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) {
        dwa[jj] = 0.f;
        wj[jj] = bw_load(rw, (uint32_t)(lane + 64 * jj) * 4u, lane + 64 * jj < D);
    }
    const int row0 = blk * BWD_NORM_ROWS + wv * RPW;
    for (int g = 0; g < RPW; g += RB) {
        float xv[RB][NJ], dv[RB][NJ], r[RB];
        bool live[RB];
#pragma unroll
        for (int k = 0; k < RB; k++) {
            const int row = row0 + g + k;
            live[k] = row < total;
            // (the row and its coordinates through readfirstlane: in vector
            // registers, every buffer access built on them would become a
            // waterfall loop)
            const int rr = __builtin_amdgcn_readfirstlane(live[k] ? row : 0);
            const int h = __builtin_amdgcn_readfirstlane(rr % H), t = __builtin_amdgcn_readfirstlane((rr / H) % T),
                      b = __builtin_amdgcn_readfirstlane(rr / (H * T));
            const size_t hm = ((size_t)b * H + h) * Tp + t;
            const bw_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char*>(reinterpret_cast<const char*>(x)) + (size_t)rr * D * ES, (short)0, live[k] ? D * ES : 0,
                0x00020000);
            const bw_rsrc_t rd = bw_rsrc(dxh + hm * D, live[k] ? (size_t)D : 0);
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                const int j = lane + 64 * jj;
                const uint32_t dead = j < D ? 0u : BW_DEAD;
                if constexpr (BF)
                    xv[k][jj] = (float)__builtin_bit_cast(
                        bf16_t, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rx, ((uint32_t)j * 2u) | dead, 0, 0));
                else
                    xv[k][jj] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, ((uint32_t)j * 4u) | dead, 0, 0));
                dv[k][jj] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, ((uint32_t)j * 4u) | dead, 0, 0));
            }
            r[k] = bw_load(bw_rsrc(rs + hm, 1), 0u, live[k]);
        }
#pragma unroll
        for (int k = 0; k < RB; k++) {
            const int row = row0 + g + k;
            float sum = 0.f;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                sum = fmaf(xv[k][jj] * wj[jj], dv[k][jj], sum);
                dwa[jj] = fmaf(dv[k][jj] * xv[k][jj], r[k], dwa[jj]);  // zero for a row past the end
            }
            const float cr = r[k] * r[k] * r[k] * bw_wave_sum(sum) / (float)D;
            const bw_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<char*>(dx) + (size_t)(live[k] ? row : 0) * D * ES,
                                                                   (short)0, live[k] ? D * ES : 0, 0x00020000);
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                const int j = lane + 64 * jj;
                const uint32_t dead = j < D ? 0u : BW_DEAD;
                const float o = r[k] * wj[jj] * dv[k][jj] - cr * xv[k][jj];
                if constexpr (BF)
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16_t)o), ro,
                                                          ((uint32_t)j * 2u) | dead, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, o), ro, ((uint32_t)j * 4u) | dead, 0, 0);
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) sdw[wv][lane + 64 * jj] = dwa[jj];
    __syncthreads();
    for (int j = threadIdx.x; j < D; j += 256)
        dw_part[(size_t)blk * D + j] = (sdw[0][j] + sdw[1][j]) + (sdw[2][j] + sdw[3][j]);
}

// bw_norm_kernel for D columns: NJ the power of two with 64 NJ >= D.
template <bool BF>
void launch_norm_adjoint(dim3 nb, const void* x, const float* w, const float* rs, const float* dxh, int B, int T,
                         int Tp, int H, int D, void* dx, float* dw_part, hipStream_t stream) {
    const dim3 blk(256);
#define CYFA_BW_NORM(NJ_) \
    hipLaunchKernelGGL((bw_norm_kernel<BF, NJ_>), nb, blk, 0, stream, x, w, rs, dxh, B, T, Tp, H, D, dx, dw_part)
    if (D <= 64)
        CYFA_BW_NORM(1);
    else if (D <= 128)
        CYFA_BW_NORM(2);
    else if (D <= 256)
        CYFA_BW_NORM(4);
    else if (D <= 512)
        CYFA_BW_NORM(8);
    else
        CYFA_BW_NORM(16);
#undef CYFA_BW_NORM
}

// out[i] = sum over the nb partial rows of part[.][i]: one wave per column,
// lane l adding rows l, l + 64, .. in order, then the wave's fixed-order sum.
__global__ __launch_bounds__(256) void bw_reduce_kernel(const float* part, int nb, size_t n, float* out) {
    const size_t i = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= n) return;
    float s = 0.f;
    for (int b = lane; b < nb; b += 64) s += part[(size_t)b * n + i];
    s = bw_wave_sum(s);
    if (lane == 0) out[i] = s;
}

// The table cotangent: per head, sum the readout blocks' partials in order.
__global__ __launch_bounds__(256) void bw_table_reduce_kernel(const float* part, int nb, int RM, float* out) {
    const int h = blockIdx.y, e = blockIdx.x * 256 + threadIdx.x;
    if (e >= RM) return;
    const float* p = part + (size_t)h * nb * RM + e;
    float s = 0.f;
    int b = 0;
    for (; b + 16 <= nb; b += 16) {  // sixteen loads in flight, then the sums in order
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = p[(size_t)(b + i) * RM];
#pragma unroll
        for (int i = 0; i < 16; i++) s += v[i];
    }
    for (; b < nb; b++) s += p[(size_t)b * RM];
    out[(size_t)h * RM + e] = s;
}

// dreadout[h][r][j] = sum_m dtable[h][r][m] Phi[j][m] (table = readout Phi,
// ops/chunk.py:82-103, 281); Phi's angle 2 pi ((pair j) mod R) / R is reduced
// exactly in integers. One block per (h, r), thread j.
// The R angles' sine and cosine are formed once per block in LDS and indexed
// by the exact integer reduction (pair j) mod R, stepped by j per pair: the
// same values as a sincosf per term.
__global__ __launch_bounds__(256) void bw_dreadout_kernel(const float* dtable, int M, float* dreadout) {
    const int R = M - 1, hr = blockIdx.x, j = threadIdx.x;
    __shared__ float row[BWD_MAX_M], sin_k[BWD_MAX_M], cos_k[BWD_MAX_M];
    if (j < M) row[j] = dtable[(size_t)hr * M + j];
    if (j < R) sincosf((float)((double)j * (kTwoPiBw / R)), &sin_k[j], &cos_k[j]);
    __syncthreads();
    if (j >= R) return;
    float acc = 0.f;
    int k = 0;  // (pair j) mod R
    for (int pair = 0; pair < M / 2; pair++) {
        const float sc = (float)sqrt((pair == 0 ? 1.0 : 2.0) / R);
        acc = fmaf(row[2 * pair], sc * cos_k[k], acc);
        if (pair > 0) acc = fmaf(row[2 * pair + 1], sc * sin_k[k], acc);  // column 1 is not a basis vector
        k += j;
        k = k >= R ? k - R : k;
    }
    dreadout[(size_t)hr * R + j] = acc;
}

// Head-major fp32 [B*H, Tp, D] rows into [B, T, H, D] in the operands' dtype.
template <bool BF>
__global__ __launch_bounds__(256) void bw_pack_kernel(const float* src, int B, int T, int Tp, int H, int D, void* dst) {
    // four consecutive elements per thread (D % 4 == 0, the launcher checks;
    // a row's four never straddle two rows)
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4, n = (size_t)B * T * H * D;
    if (i >= n) return;
    const int j = (int)(i % D);
    const size_t row = i / D;
    const int h = (int)(row % H), t = (int)((row / H) % T), b = (int)(row / ((size_t)H * T));
    const float4 v = *reinterpret_cast<const float4*>(src + (((size_t)b * H + h) * Tp + t) * D + j);
    if constexpr (BF) {
        const bf16x4 o = {(bf16_t)v.x, (bf16_t)v.y, (bf16_t)v.z, (bf16_t)v.w};
        *reinterpret_cast<bf16x4*>(reinterpret_cast<bf16_t*>(dst) + i) = o;
    } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(dst) + i) = v;
    }
}

// The same, one element per thread (any D, any alignment of dst).
template <bool BF>
__global__ __launch_bounds__(256) void bw_pack1_kernel(const float* src, int B, int T, int Tp, int H, int D, void* dst) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, n = (size_t)B * T * H * D;
    if (i >= n) return;
    const int j = (int)(i % D);
    const size_t row = i / D;
    const int h = (int)(row % H), t = (int)((row / H) % T), b = (int)(row / ((size_t)H * T));
    bw_st<BF>(dst, i, src[(((size_t)b * H + h) * Tp + t) * D + j]);
}

void launch_chunk_grad(const ChunkGradArgs& a, bool mfma, hipStream_t stream) {
    // rows and states 16-byte aligned (workspace buffers, rows of Kq and Vd floats)
    const bool v4 = a.Kq % 4 == 0 && a.Vd % 4 == 0;
    const dim3 grid(a.N, a.H, a.B);
    // (the flags pair as the backward sets them: sbf for bf16 calls, rbf for pass 2's)
    if (mfma && v4 && a.rbf)
        hipLaunchKernelGGL((bw_chunk_kernel<true, true, true, true>), grid, dim3(256), 0, stream, a);
    else if (mfma && v4)
        hipLaunchKernelGGL((a.sbf ? bw_chunk_kernel<true, true, true, false> : bw_chunk_kernel<true, true, false, false>),
                           grid, dim3(256), 0, stream, a);
    else if (mfma && a.rbf)
        hipLaunchKernelGGL((bw_chunk_kernel<true, false, true, true>), grid, dim3(256), 0, stream, a);
    else if (mfma)
        hipLaunchKernelGGL((a.sbf ? bw_chunk_kernel<true, false, true, false> : bw_chunk_kernel<true, false, false, false>),
                           grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((bw_chunk_kernel<false, false, false, false>), grid, dim3(256), 0, stream, a);
}

}  // namespace

int launch_chunk_pass(const ChunkPassParams& p, hipStream_t stream) {
    if (p.B < 1 || p.H < 1 || p.T < 1 || p.Tp < p.T || p.Tp % BC || p.Kq < 1 || p.Kq > BW_MAX_D || p.Vd < 1 ||
        p.Vd > BW_MAX_D || (!p.out && !p.out_bthd) || !p.states)
        return -1;
    const int N = p.Tp / BC;
    StateScanArgs sa{};
    sa.a = p.k;
    sa.b = p.v;
    sa.g = p.g;
    sa.x0 = p.s0;
    sa.xs = p.states;
    sa.x_out = p.s_final;
    sa.B = p.B;
    sa.T = p.T;
    sa.Tp = p.Tp;
    sa.H = p.H;
    sa.Kq = p.Kq;
    sa.Vd = p.Vd;
    sa.N = N;
    sa.scale = 1.f;
    sa.sbf = p.mfma && p.sbf16;
    launch_state_scan<false>(sa, p.mfma, stream);
    OutArgs oa{};
    oa.q = p.q;
    oa.k = p.k;
    oa.v = p.v;
    oa.g = p.g;
    oa.S = p.states;
    oa.out = p.out;
    oa.out_bthd = p.out_bthd;
    oa.bf16 = p.bf16;
    oa.B = p.B;
    oa.T = p.T;
    oa.Tp = p.Tp;
    oa.H = p.H;
    oa.Kq = p.Kq;
    oa.Vd = p.Vd;
    oa.N = N;
    oa.scale = p.scale;
    oa.sbf = p.mfma && p.sbf16;
    // rows and states 16-byte aligned (workspace buffers, rows of Kq and Vd floats)
    const bool v4 = p.Kq % 4 == 0 && p.Vd % 4 == 0;
    const dim3 og(N, p.H, p.B);
    if (p.mfma && v4)
        hipLaunchKernelGGL((oa.sbf ? bw_out_kernel<true, true, true> : bw_out_kernel<true, true, false>), og, dim3(256),
                           0, stream, oa);
    else if (p.mfma)
        hipLaunchKernelGGL((oa.sbf ? bw_out_kernel<true, false, true> : bw_out_kernel<true, false, false>), og,
                           dim3(256), 0, stream, oa);
    else
        hipLaunchKernelGGL((bw_out_kernel<false, false, false>), og, dim3(256), 0, stream, oa);
    return 0;
}

int launch_chunk_readout(const float* raw, const float* cs, const float* sn, const float* table, float* lg, int B,
                         int Tp, int H, int M, int bf16, int split, float* wts, hipStream_t stream) {
    if (B < 1 || H < 1 || Tp < 1 || Tp % BC || M < 4 || M > BWD_MAX_M || M % 2) return -1;
    const dim3 blk(256);
    if (M > BWD_TABLE_M) {  // logits, softmax, then the weights, streaming the table
        if (!lg) return -1;
        WideArgs wa{};
        wa.raw = raw;
        wa.cs = cs;
        wa.sn = sn;
        wa.table = table;
        wa.lg = lg;
        wa.wts = wts;
        wa.B = B;
        wa.Tp = Tp;
        wa.H = H;
        wa.M = M;
        wa.bf = bf16;
        const int rows_h = B * Tp;
        const size_t rows = (size_t)rows_h * H;
        hipLaunchKernelGGL(bw_wide_logits_kernel<false>, dim3((rows_h + BC - 1) / BC, (M - 1 + BC - 1) / BC, H), blk,
                           0, stream, wa);
        hipLaunchKernelGGL(bw_wide_softmax_kernel<false>, dim3((unsigned)((rows + 3) / 4)), blk, 0, stream, wa);
        hipLaunchKernelGGL(bw_wide_u_kernel<false>, dim3((rows_h + BC - 1) / BC, (M + BC - 1) / BC, H), blk, 0,
                           stream, wa);
        return 0;
    }
    const int per = bwd_ro_per_wg(B, Tp, H), blocks = (B * Tp + BWD_RO_BLOCK - 1) / BWD_RO_BLOCK;
    const dim3 grid((blocks + per - 1) / per, H);
    if (split && bf16)
        hipLaunchKernelGGL(bw_fwd_readout_mf_kernel<true>, grid, dim3(RO_MF_THREADS), 0, stream, raw, cs, sn, table, B, Tp, H, M, per,
                           wts);
    else if (split)
        hipLaunchKernelGGL(bw_fwd_readout_mf_kernel<false>, grid, dim3(RO_MF_THREADS), 0, stream, raw, cs, sn, table, B, Tp, H, M, per,
                           wts);
    else if (bf16)
        hipLaunchKernelGGL(bw_fwd_readout_kernel<true>, grid, dim3(RO_FWD_THREADS), 0, stream, raw, cs, sn, table, B, Tp, H, M, per,
                           wts);
    else
        hipLaunchKernelGGL(bw_fwd_readout_kernel<false>, grid, dim3(RO_FWD_THREADS), 0, stream, raw, cs, sn, table, B, Tp, H, M, per,
                           wts);
    return 0;
}

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
    hipLaunchKernelGGL((bw_rows_kernel<BFV, RowT>), rb, blk, 0, stream, p.v, (const float*)nullptr, 0.f, B, T, Tp, H, \
                       V, reinterpret_cast<RowT*>(ws.vh), (float*)nullptr);                                        \
    hipLaunchKernelGGL((bw_rows_kernel<BFV, RowT>), rb, blk, 0, stream, p.d_o, (const float*)nullptr, 0.f, B, T, Tp, H, \
                       V, reinterpret_cast<RowT*>(ws.dO), (float*)nullptr);
    // v and dO of bf16 calls stay bf16 in the head-major rows (exact): the
    // pass-2 scans and chunk kernels read half the bytes.
    if (bf) {
        using RowT = bf16_t;
        CYFA_BW_ROWS(true)
    } else {
        using RowT = float;
        CYFA_BW_ROWS(false)
    }
#undef CYFA_BW_ROWS
    // the forward, recomputed in fp32: clock, write vector, the states before
    // every chunk of both passes, the pass-1 output and the slot weights
    if (launch_general_clock_write(p.delta, p.clock0, p.beta, B, T, Tp, H, M, ws.lam, ws.w, ws.cs, ws.sn, stream) != 0)
        return -1;
    // The stored states and state cotangents of bf16 calls are bf16, as the
    // reference stores its chunk states and their cotangents (the recurrence
    // itself runs in fp32 registers; ops/chunk_h.py:212-214, 329-331).
    StateScanArgs f1{};
    f1.sbf = bf;
    f1.a = ws.kh;
    f1.b = ws.w;
    f1.g = p.g;
    f1.x0 = p.h0_k;
    f1.xs = ws.sk;
    f1.B = B;
    f1.T = T;
    f1.Tp = Tp;
    f1.H = H;
    f1.Kq = K;
    f1.Vd = M;
    f1.N = N;
    f1.scale = 1.f;
    ChunkPassParams p1{};
    p1.q = ws.qh;
    p1.k = ws.kh;
    p1.v = ws.w;
    p1.g = p.g;
    p1.s0 = p.h0_k;
    p1.states = ws.sk;
    p1.out = ws.raw;
    p1.mfma = bf;
    p1.sbf16 = bf;
    p1.B = B;
    p1.T = T;
    p1.Tp = Tp;
    p1.H = H;
    p1.Kq = K;
    p1.Vd = M;
    p1.scale = p.scale;
    if (launch_chunk_pass(p1, stream) != 0 ||
        launch_chunk_readout(ws.raw, ws.cs, ws.sn, p.table, ws.lg, B, Tp, H, M, 0, bf, ws.wts, stream) != 0)
        return -1;
    const int ro_per_wg = bwd_ro_per_wg(B, Tp, H);
    const bool wide = M > BWD_TABLE_M;
    WideArgs wa{};
    wa.raw = ws.raw;
    wa.cs = ws.cs;
    wa.sn = ws.sn;
    wa.table = p.table;
    wa.dwts = ws.dwts;
    wa.lg = ws.lg;
    wa.dl = ws.dlw;
    wa.wts = ws.wts;
    wa.draw = ws.draw;
    wa.dlp = ws.dlp;
    wa.dlam = ws.dlam;
    wa.dtab = ws.dtab;
    wa.B = B;
    wa.Tp = Tp;
    wa.H = H;
    wa.M = M;
    wa.splits = ws.ro_blocks;
    const int rows_h = B * Tp;
    const dim3 g_logits((rows_h + BC - 1) / BC, (M - 1 + BC - 1) / BC, H), g_u((rows_h + BC - 1) / BC, (M + BC - 1) / BC, H);
    const dim3 g_rows((unsigned)((rows + 3) / 4));
    StateScanArgs f2 = f1;
    f2.a = ws.w;
    f2.b = ws.vh;
    f2.x0 = p.h0_v;
    f2.xs = ws.sv;
    f2.bbf = bf;  // v's rows
    f2.Kq = M;
    f2.Vd = V;
    launch_state_scan<false>(f2, bf, stream);
    // pass 2: state cotangents, then the rows' (slot weights, write vector, v)
    StateScanArgs s2 = f2;
    s2.a = ws.wts;
    s2.b = ws.dO;
    s2.x0 = p.d_hv;
    s2.xs = ws.dsv;
    s2.S = ws.sv;
    s2.bnd = ws.bnd2;
    s2.x_out = p.dh0_v;
    launch_state_scan<true>(s2, bf, stream);
    ChunkGradArgs c2{};
    c2.sbf = bf;
    c2.rbf = bf;  // v's and dO's rows
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
    launch_chunk_grad(c2, bf, stream);
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
    ro.per_wg = ro_per_wg;
    if (wide) {  // dp, dl, then dz with draw and the clock's share, and the table cotangent's partials
        hipLaunchKernelGGL(bw_wide_logits_kernel<true>, g_logits, blk, 0, stream, wa);
        hipLaunchKernelGGL(bw_wide_softmax_kernel<true>, g_rows, blk, 0, stream, wa);
        hipLaunchKernelGGL(bw_wide_u_kernel<true>, g_u, blk, 0, stream, wa);
        hipLaunchKernelGGL(bw_wide_dlam_kernel, dim3((unsigned)((rows + 255) / 256)), blk, 0, stream, wa);
        hipLaunchKernelGGL(bw_wide_dtable_kernel, dim3((M - 1 + BC - 1) / BC, (M + BC - 1) / BC, H * ws.ro_blocks), blk, 0,
                           stream, wa);
    } else {
        hipLaunchKernelGGL(bw_readout_kernel, dim3(ws.ro_blocks, H), dim3(RO_ADJ_THREADS), 0, stream, ro);
    }
    // pass 1, with the pass-1 output's cotangent as dO
    StateScanArgs s1 = f1;
    s1.a = ws.qh;
    s1.b = ws.draw;
    s1.x0 = p.d_hk;
    s1.xs = ws.dsk;
    s1.S = ws.sk;
    s1.bnd = ws.bnd1;
    s1.x_out = p.dh0_k;
    s1.scale = p.scale;
    launch_state_scan<true>(s1, bf, stream);
    ChunkGradArgs c1 = c2;
    c1.rbf = 0;  // pass 1's rows (the write vector, draw) are fp32
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
    launch_chunk_grad(c1, bf, stream);
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
    if (K % 4 == 0)
        hipLaunchKernelGGL(bw_token_kernel<true>, dim3(N, B * H), blk, 0, stream, tg);
    else
        hipLaunchKernelGGL(bw_token_kernel<false>, dim3(N, B * H), blk, 0, stream, tg);
    hipLaunchKernelGGL(bw_clock_kernel, dim3(B * H), dim3(64), 0, stream, ws.dlam, p.d_clock, B, T, Tp, H, p.ddelta,
                       p.dclock0);
    // the q/k norms, their weights, v's layout
    const dim3 nb(ws.norm_blocks);
    if (bf) {
        launch_norm_adjoint<true>(nb, p.q, p.q_w, ws.rq, ws.dqh, B, T, Tp, H, K, p.dq, ws.dnq, stream);
        launch_norm_adjoint<true>(nb, p.k, p.k_w, ws.rk, ws.dkh, B, T, Tp, H, K, p.dk, ws.dnk, stream);
    } else {
        launch_norm_adjoint<false>(nb, p.q, p.q_w, ws.rq, ws.dqh, B, T, Tp, H, K, p.dq, ws.dnq, stream);
        launch_norm_adjoint<false>(nb, p.k, p.k_w, ws.rk, ws.dkh, B, T, Tp, H, K, p.dk, ws.dnk, stream);
    }
    const dim3 kb((unsigned)((K + 3) / 4));
    hipLaunchKernelGGL(bw_reduce_kernel, kb, blk, 0, stream, ws.dnq, ws.norm_blocks, (size_t)K, p.dq_w);
    hipLaunchKernelGGL(bw_reduce_kernel, kb, blk, 0, stream, ws.dnk, ws.norm_blocks, (size_t)K, p.dk_w);
    const size_t nv = (size_t)B * T * H * V;
    const dim3 vb((unsigned)((nv + 255) / 256)), vb4((unsigned)((nv / 4 + 255) / 256));
    const bool pack4 = V % 4 == 0 && ((uintptr_t)p.dv & (bf ? 7 : 15)) == 0;
    if (bf && pack4)
        hipLaunchKernelGGL(bw_pack_kernel<true>, vb4, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    else if (pack4)
        hipLaunchKernelGGL(bw_pack_kernel<false>, vb4, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    else if (bf)
        hipLaunchKernelGGL(bw_pack1_kernel<true>, vb, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    else
        hipLaunchKernelGGL(bw_pack1_kernel<false>, vb, blk, 0, stream, ws.dvh, B, T, Tp, H, V, p.dv);
    const int RM = (M - 1) * M;
    hipLaunchKernelGGL(bw_table_reduce_kernel, dim3((RM + 255) / 256, H), blk, 0, stream, ws.dtab, ws.ro_blocks, RM,
                       p.dtable);
    if (p.dreadout)
        hipLaunchKernelGGL(bw_dreadout_kernel, dim3(H * (M - 1)), blk, 0, stream, p.dtable, M, p.dreadout);
    return 0;
}

}  // namespace cyfa
