// cyfa_decode.hip -- fused constant-memory CyFA decode step for gfx950.
//
// The step is HBM-bound: it streams the fp32 key state hk [K, M] and value
// state hv [M, V] in and out once (512 KiB per (b, h) for K = V = 256).
//
// Math (ops/fused_recurrent.py:57-188): q_hat = bf16(q rs_q w_q) * scale,
// k_hat = bf16(k rs_k w_k); lam = clock + delta; alpha = e^g;
// w = bf16(beta U(-lam) b); hk' = alpha hk + k_hat (x) w; raw = hk'^T q_hat;
// z = U(lam) raw; p = softmax(table z); u = table^T p; weights = U(-lam) u;
// hv' = alpha hv + w (x) v; o = bf16(hv'^T weights).
// The readout is evaluated in fp32 (the reference rounds z, the table and p
// to bf16 here); the write vector and the normalised q/k keep the reference's
// bf16 rounding so decode and the chunkwise prefill see identical operands.
//
// Two launch forms with bit-identical results:
//  * one 1024-thread workgroup per (b, h) (decode_step_kernel), when B H fills
//    the chip (B H >= 64): both state streams are issued at entry and both
//    updated states are written before the slot readout runs;
//  * small batches (B H < 64, e.g. B = 1): eight workgroups per (b, h)
//    (decode_split_a_kernel), each updating 32 rows of hk and 32 columns of
//    hv (128-byte line-aligned slices), and writing its slice's partial sums
//    of raw; then one workgroup per (b, h) (decode_split_b_kernel) sums the
//    partials, runs the readout and forms o from the updated hv.
// raw is always reduced in the same order: per 32-row slice s, each of 256
// threads accumulates its four rows, the eight 32-thread groups are summed in
// group order, and the slices in slice order; o is formed with the same
// thread mapping in both forms.
#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

__device__ __forceinline__ void stream_store(float4* p, const float4& v) {
    __builtin_nontemporal_store(__builtin_bit_cast(f32x4, v), reinterpret_cast<f32x4*>(p));
}

namespace {

constexpr int SLICE = 32;  // hk rows / hv columns per slice

// Loads. Every load of a kernel is issued before the first is used, small
// inputs first: loads complete in order, so the prologue waits for those
// alone while the state streams are in flight. Loads go through buffer
// resources and are predicated through their offset, never a branch: at a
// branch among loads (even a uniform one) the compiler waits for every load
// in flight. DEAD is an offset past the end of every buffer read here
// (launch_decode_step keeps each span below 2^31 bytes), so its load returns
// zero; a null base gets an empty buffer, whose every load returns zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t DEAD = 0x80000000u;

__device__ __forceinline__ rsrc_t buf(const void* base, size_t bytes) {
    const uint32_t n = base == nullptr ? 0u : bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// DEAD unless a < b (integer arithmetic: a select here can become a branch)
__device__ __forceinline__ uint32_t dead_unless_below(int a, int b) { return (~(uint32_t)(a - b)) & DEAD; }

__device__ __forceinline__ float ld_bf16(rsrc_t r, uint32_t off) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0) << 16);
}
__device__ __forceinline__ float ld_f32(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ bf16x4 ld_bf16x4(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ float4 ld_f32x4(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// The states are touched exactly once per step: non-temporal loads and stores
// keep them from displacing reusable lines in the caches (about 20% faster
// at B = 64 with the state streaming from HBM).
__device__ __forceinline__ float4 stream_load(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}

// Element i of row `row` (n elements per row) of q, k or v: bf16, or fp32
// (F32; the pointer then holds fp32 data).
template <bool F32>
__device__ __forceinline__ float ld_in(const __bf16* base, size_t row, int n, int i, uint32_t dead) {
    if constexpr (F32)
        return ld_f32(buf(reinterpret_cast<const float*>(base) + row * n, (size_t)n * 4), ((uint32_t)i * 4) | dead);
    else
        return ld_bf16(buf(base + row * n, (size_t)n * 2), ((uint32_t)i * 2) | dead);
}

// The one-token inputs of (b, h): q and k channel c (< K) or v channel c (< V)
// of this head. LAYER: from the width-4 causal short convolution of the
// projection row (layers/cyfa.py:138-233, the arithmetic of short_conv_kernel);
// otherwise read from q, k, v. The convolution window (cache rows 0-2, then x)
// and the weights of a channel are loaded by load_conv, used by conv_out.
struct ConvIn {
    float win[4], wt[4];
};

// The buffers of batch row b's conv inputs: the cache rows (empty without a
// cache), the projection row and the conv weights; D = 2 H K + H V channels.
struct ConvSrc {
    rsrc_t cache, qkv, w;
    uint32_t row;  // cache row stride, bytes
};

__device__ __forceinline__ ConvSrc conv_src(const DecodeParams& p, int b, int D) {
    ConvSrc c;
    c.cache = buf(p.cache_in ? p.cache_in + (size_t)b * p.cache_batch : nullptr, ((size_t)2 * p.cache_row + D) * 2);
    c.qkv = buf(p.qkv + (size_t)b * p.qkv_row, (size_t)D * 2);
    c.w = buf(p.conv_w, (size_t)D * 8);
    c.row = (uint32_t)p.cache_row * 2;
    return c;
}

// Channel ch's window and weights (all zero when dead is DEAD).
__device__ __forceinline__ ConvIn load_conv(const ConvSrc& src, int ch, uint32_t dead) {
    ConvIn c;
#pragma unroll
    for (int w = 0; w < 3; w++) c.win[w] = ld_bf16(src.cache, (w * src.row + (uint32_t)ch * 2) | dead);
    c.win[3] = ld_bf16(src.qkv, ((uint32_t)ch * 2) | dead);
    const bf16x4 wt = ld_bf16x4(src.w, ((uint32_t)ch * 8) | dead);  // one 8-byte load
#pragma unroll
    for (int w = 0; w < 4; w++) c.wt[w] = (float)wt[w];
    return c;
}

__device__ __forceinline__ float conv_out(const ConvIn& c) {
    float acc = c.win[0] * c.wt[0];
#pragma unroll
    for (int w = 1; w < 4; w++) acc = fmaf(c.win[w], c.wt[w], acc);
    return bf16_round(acc);
}

// The new conv cache of a channel: the last three rows of its window, through
// the cache_out rows of batch row b (a store at a DEAD offset is dropped; the
// stores are predicated like the loads, since a store behind a branch makes
// later wait counts assume it was not issued and wait for loads past it).
__device__ __forceinline__ rsrc_t conv_out_rows(const DecodeParams& p, int b, int D) {
    return buf(p.cache_out + (size_t)b * p.cache_batch, ((size_t)2 * p.cache_row + D) * 2);
}

__device__ __forceinline__ void store_conv_cache(rsrc_t out, uint32_t row, int ch, uint32_t dead, const ConvIn& c) {
#pragma unroll
    for (int w = 0; w < 3; w++)
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16_t)c.win[w + 1]), out,
                                              (w * row + (uint32_t)ch * 2) | dead, 0, 0);
}

// Gate inputs of (b, h): LAYER, the a, b, d projections (the activations
// follow in gate_values); otherwise g, delta, beta themselves.
struct GateIn {
    float x0, x1, x2, dt_bias, A_log, clock;  // clock: the incoming clock (0 without a state)
};

template <bool LAYER>
__device__ __forceinline__ GateIn load_gate_inputs(const DecodeParams& p, int bh) {
    GateIn gi;
    const int b = bh / p.H, h = bh % p.H;
    if (LAYER) {
        const rsrc_t r = buf(p.abd + (size_t)b * p.abd_row, (size_t)3 * p.H * 2);
        gi.x0 = ld_bf16(r, (uint32_t)h * 2);
        gi.x1 = ld_bf16(r, (uint32_t)(p.H + h) * 2);
        gi.x2 = ld_bf16(r, (uint32_t)(2 * p.H + h) * 2);
        gi.dt_bias = ld_f32(buf(p.dt_bias, (size_t)p.H * 4), (uint32_t)h * 4);
        gi.A_log = ld_f32(buf(p.A_log, (size_t)p.H * 4), (uint32_t)h * 4);
    } else {
        gi.x0 = ld_f32(buf(p.g, (size_t)(bh + 1) * 4), (uint32_t)bh * 4);
        gi.x1 = ld_f32(buf(p.delta, (size_t)(bh + 1) * 4), (uint32_t)bh * 4);
        gi.x2 = ld_f32(buf(p.beta, (size_t)(bh + 1) * 4), (uint32_t)bh * 4);
        gi.dt_bias = gi.A_log = 0.f;
    }
    gi.clock = ld_f32(buf(p.hk_in != nullptr ? p.clock_in : nullptr, (size_t)(bh + 1) * 4), (uint32_t)bh * 4);
    return gi;
}

// Gate activations (layers/cyfa.py:323-326, as gates_kernel) or the given gates.
template <bool LAYER>
__device__ __forceinline__ void gate_values(const DecodeParams& p, int bh, const GateIn& gi, float& g, float& delta,
                                            float& beta) {
    if (LAYER) {
        g = decay_gate(gi.x0 + gi.dt_bias, gi.A_log);
        beta = sigmoidf(gi.x1);
        delta = sigmoidf(gi.x2);
    } else {
        g = gi.x0;
        delta = gi.x1;
        beta = gi.x2;
    }
}

// Wave 0's norm weight and gate for the output norm (LAYER): four
// consecutive values per lane, as rms_norm_kernel<1> holds them.
template <int V, bool LAYER>
__device__ __forceinline__ void load_norm_inputs(const DecodeParams& p, int bh, float4* on_w4, bf16x4* on_g4) {
    constexpr int OJ = (V + 255) / 256;
    if (LAYER) {
        const int lane = threadIdx.x & 63;
        const uint32_t dead = dead_unless_below(threadIdx.x >> 6, 1);
        const rsrc_t rn = buf(p.on_w, (size_t)V * 4);
        const rsrc_t rg = buf(p.gate + (size_t)(bh / p.H) * p.gate_row + (size_t)(bh % p.H) * V, (size_t)V * 2);
#pragma unroll
        for (int j = 0; j < OJ; j++) {
            on_w4[j] = ld_f32x4(rn, ((uint32_t)(4 * lane + 256 * j) * 4) | dead);
            on_g4[j] = ld_bf16x4(rg, ((uint32_t)(4 * lane + 256 * j) * 2) | dead);
        }
    }
}

// The head's readout table, [kActive, kSlots] f32, 4 float4 per thread of a
// 1024-thread workgroup (zero past its end); staged in LDS by stage_table.
constexpr int TQ = kActive * kSlots / 4;
static_assert(TQ > 3 * 1024 && TQ <= 4 * 1024, "table staging covers the table");

__device__ __forceinline__ void load_table(const DecodeParams& p, int h, float4 (&tab)[4]) {
    const rsrc_t r = buf(p.table + (size_t)h * kActive * kSlots, (size_t)kActive * kSlots * 4);
#pragma unroll
    for (int i = 0; i < 4; i++) tab[i] = ld_f32x4(r, (uint32_t)(threadIdx.x + 1024 * i) * 16);
}

__device__ __forceinline__ void stage_table(float* s_tab, const float4 (&tab)[4]) {
    float4* st4 = reinterpret_cast<float4*>(s_tab);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 3; i++) st4[tid + 1024 * i] = tab[i];
    if (tid + 3 * 1024 < TQ) st4[tid + 3 * 1024] = tab[3];
}

// The gate of (b, h) as the second projection of g_proj (layers/cyfa.py:
// 292-295, 349) when the caller passes g0 instead of the gate: gate = bf16(g0 W^T +
// bias) for the head's V = 256 columns, in linear_rows_kernel's summation
// order for K = 256 (eight 32-deep k-steps, one per wave there): each k-step
// on one v_mfma_f32_16x16x32_bf16 from zero, with g0 in row 0 of A and the
// other rows zero; the eight partials summed in k-step order, then the bias.
// Wave c (0..15) forms columns 16 c .. 16 c + 15; lane (lr, lg) holds W row
// 16 c + lr, k = 32 s + 8 lg .. 32 s + 8 lg + 7 of step s.
struct GateW {
    bf16x8 w[8];
    float bias;
};

// live false: the wave's rows read zero (another step workgroup of the
// (b, h) forms those columns).
__device__ __forceinline__ GateW load_gate_weights(const DecodeParams& p, int h, bool live = true) {
    constexpr int V = 256;
    const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, lr = lane & 15, lg = lane >> 4;
    const rsrc_t r = buf(p.g1_w && live ? p.g1_w + ((size_t)h * V + 16 * c) * V : nullptr, (size_t)16 * V * 2);
    GateW g;
#pragma unroll
    for (int st = 0; st < 8; st++)
        g.w[st] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(lr * V + 32 * st + 8 * lg) * 2, 0, 0));
    g.bias = ld_bf16(buf(p.g1_b ? p.g1_b + (size_t)h * V : nullptr, (size_t)V * 2), (uint32_t)(16 * c + lr) * 2);
    return g;
}

// g0 of batch row b, 16 bytes per thread for threads 0..31 (zero elsewhere).
__device__ __forceinline__ bf16x8 load_g0(const DecodeParams& p, int b) {
    const rsrc_t r = buf(p.g0 ? p.g0 + (size_t)b * p.g0_row : nullptr, 512);
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                          r, ((uint32_t)threadIdx.x * 16) | dead_unless_below(threadIdx.x, 32), 0, 0));
}

// s_gate[16 c + lr] = the gate's column 16 c + lr, bf16-rounded (s_g0: g0 as 32 bf16x8).
__device__ __forceinline__ void gate_columns(const bf16x8* s_g0, const GateW& g, float* s_gate) {
    const int lane = threadIdx.x & 63, c = threadIdx.x >> 6, lr = lane & 15, lg = lane >> 4;
    float tot = 0.f;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        const bf16x8 a = lr == 0 ? s_g0[4 * st + lg] : bf16x8{};
        const f32x4 acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, g.w[st], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        tot += acc[0];  // row 0 of the tile (lanes lg = 0)
    }
    if (lg == 0) s_gate[16 * c + lr] = bf16_round(tot + g.bias);
}

// Write vector w (ops/utils.py:664-702) and the phase of every pair into LDS;
// threads 0..63 (one pair each). bf16 inputs: w rounded to bf16, the phase on
// the hardware sine/cosine of the once-reduced clock. F32 (fp32 inputs, which
// the reference computes without rounding): w unrounded, the phase from the
// reference's integer range reduction of the clock and the full-precision
// sincosf.
template <bool F32 = false>
__device__ __forceinline__ void write_vector_lds(float lam, float beta, float* s_w, float* s_c, float* s_s) {
    const int tid = threadIdx.x;
    if (tid < kPairs) {
        float s, c;
        if constexpr (F32)
            sincosf(clock_phase(lam, tid), &s, &c);
        else
            pair_sincos(reduced_clock(lam), tid, s, c);
        const float a = beta * pair_scale(tid);
        s_w[2 * tid] = F32 ? a * c : bf16_round(a * c);
        s_w[2 * tid + 1] = F32 ? -a * s : bf16_round(-a * s);
        s_c[tid] = c;
        s_s[tid] = s;
    }
}

// Key-state slice s for the 256 "slice threads" vt: float4 j (0..3) of thread
// vt is element (row 32 s + vt / 32 + 8 j, columns 4 (vt % 32) ..) of hk, i.e.
// float4 index 1024 s + vt + 256 j. Updates and stores the four float4 and
// accumulates the thread's partial raw in row order j.
// With `out` set (several step workgroups per (b, h)) the float4 go through
// that buffer resource instead, at a DEAD offset (dropped) unless `dead` is 0.
__device__ __forceinline__ float4 key_slice_update(const float4 (&hk)[4], float4* hk_out, int s, int vt, float decay,
                                                   const float* s_k, const float* s_q, const float* s_w,
                                                   const rsrc_t* out = nullptr, uint32_t dead = 0) {
    const int m4 = (vt & 31) * 4;
    const float w0 = s_w[m4], w1 = s_w[m4 + 1], w2 = s_w[m4 + 2], w3 = s_w[m4 + 3];
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int d = SLICE * s + (vt >> 5) + 8 * j;
        const float kd = s_k[d], qd = s_q[d];
        float4 n = hk[j];
        n.x = fmaf(n.x, decay, kd * w0);
        n.y = fmaf(n.y, decay, kd * w1);
        n.z = fmaf(n.z, decay, kd * w2);
        n.w = fmaf(n.w, decay, kd * w3);
        if (out)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(f32x4, n), *out,
                                                   ((uint32_t)(1024 * s + vt + 256 * j) * 16) | dead, 0, 2);
        else
            stream_store(hk_out + 1024 * s + vt + 256 * j, n);
        a.x = fmaf(n.x, qd, a.x);
        a.y = fmaf(n.y, qd, a.y);
        a.z = fmaf(n.z, qd, a.z);
        a.w = fmaf(n.w, qd, a.w);
    }
    return a;
}

// part[g][m] (g = vt / 32): a slice's eight group partials -> its partial raw
// of slot m, summed in group order.
__device__ __forceinline__ float slice_partial(const float* part, int m) {
    float r = part[m];
#pragma unroll
    for (int g = 1; g < 8; g++) r += part[g * kSlots + m];
    return r;
}

// Slot readout from raw (ops/fused_recurrent.py:114-175), fp32, 1024 threads;
// the table of the head is in LDS. Leaves the weights in s_om.
__device__ __forceinline__ void readout_1024(const float* s_raw, const float* s_c, const float* s_s, const float* tb,
                                             float* s_z, float* s_p, float (*s_part)[256], float* s_om) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < kPairs) {
        const float c = s_c[tid], s = s_s[tid];
        const float e = s_raw[2 * tid], o = s_raw[2 * tid + 1];
        s_z[2 * tid] = c * e - s * o;
        s_z[2 * tid + 1] = s * e + c * o;
    }
    __syncthreads();
    {
        const int r = tid >> 3, part = tid & 7;
        float lg = 0.f;
        if (r < kActive) {
            const float4* row = reinterpret_cast<const float4*>(tb + r * kSlots + part * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 t = row[i];
                const int m = part * 16 + 4 * i;
                lg += t.x * s_z[m] + t.y * s_z[m + 1] + t.z * s_z[m + 2] + t.w * s_z[m + 3];
            }
        }
        lg += dpp_mov<0xB1>(lg);   // xor 1
        lg += dpp_mov<0x4E>(lg);   // xor 2
        lg += dpp_mov<0x141>(lg);  // the other quad of the octet (quads are uniform by now)
        if (part == 0) s_p[r] = r < kActive ? lg : -INFINITY;
    }
    __syncthreads();
    if (wave == 0) {
        const float a = s_p[lane], b = s_p[lane + 64];
        const float mx = wave_max(fmaxf(a, b));
        const float ea = expf(a - mx);
        const float eb = (lane + 64 < kActive) ? expf(b - mx) : 0.f;
        const float inv = 1.f / wave_sum(ea + eb);
        s_p[lane] = ea * inv;
        s_p[lane + 64] = eb * inv;
    }
    __syncthreads();
    {
        const int m = tid & (kSlots - 1), part = tid >> 7;  // 8 parts of 16 slots
        float u = 0.f;
        const int r1 = part * 16 + 16 < kActive ? part * 16 + 16 : kActive;
        for (int r = part * 16; r < r1; r++) u = fmaf(s_p[r], tb[r * kSlots + m], u);
        s_part[part][m] = u;
    }
    __syncthreads();
    if (tid < kPairs) {
        float ue = 0.f, uo = 0.f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            ue += s_part[q][2 * tid];
            uo += s_part[q][2 * tid + 1];
        }
        const float c = s_c[tid], s = s_s[tid];
        s_om[2 * tid] = c * ue + s * uo;
        s_om[2 * tid + 1] = -s * ue + c * uo;
    }
    __syncthreads();
}

// o = hv'^T weights with 1024 threads: thread tid covers value columns
// 4 (tid % VQ) .. and rows tid / VQ + VROWS j of hv' (hv_r), then the waves'
// partials are summed in wave order. LAYER: the gated output norm
// o_norm(o * prescale, gate) (layers/cyfa.py:349-350, as rms_norm_kernel<1>:
// wave 0 holds four consecutive values per lane) before o is stored.
// S step workgroups per (b, h): workgroup sp stores columns [sp V / S, (sp + 1) V / S).
template <int V, bool LAYER, bool F32 = false, int S = 1>
__device__ __forceinline__ void output_1024(const DecodeParams& p, int bh, const float4* hv_r, const float* s_om,
                                            float (*s_part)[256], float* s_v, const float4* on_w4,
                                            const bf16x4* on_g4, const float* s_gate, int sp = 0) {
    constexpr int NT = 1024, VQ = V / 4, VROWS = NT / VQ, VJ = kSlots / VROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    {
        const int v4 = (tid % VQ) * 4, r0 = tid / VQ;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int j = 0; j < VJ; j++) {
            const float om = s_om[r0 + VROWS * j];
            a0 = fmaf(hv_r[j].x, om, a0);
            a1 = fmaf(hv_r[j].y, om, a1);
            a2 = fmaf(hv_r[j].z, om, a2);
            a3 = fmaf(hv_r[j].w, om, a3);
        }
        if (VQ == 32) {  // two rows of the sweep share a wave
            a0 += __shfl_xor(a0, 32);
            a1 += __shfl_xor(a1, 32);
            a2 += __shfl_xor(a2, 32);
            a3 += __shfl_xor(a3, 32);
        }
        if (VQ == 64 || lane < 32) {
            s_part[wave][v4] = a0;
            s_part[wave][v4 + 1] = a1;
            s_part[wave][v4 + 2] = a2;
            s_part[wave][v4 + 3] = a3;
        }
    }
    __syncthreads();
    if (!LAYER) {
        if (tid < V) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NT / 64; w++) s += s_part[w][tid];
            if constexpr (F32)
                reinterpret_cast<float*>(p.o)[(size_t)bh * V + tid] = s;
            else
                p.o[(size_t)bh * V + tid] = (bf16_t)s;
        }
        return;
    }
    if (tid < V) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; w++) s += s_part[w][tid];
        s_v[tid] = (float)(bf16_t)s;  // o as the op would store it
    }
    __syncthreads();
    if (wave == 0) {
        constexpr int J = (V + 255) / 256;
        float xs[J][4];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < J; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float x = s_v[4 * lane + 256 * j + i];
                if (p.on_prescale != 1.f) x = bf16_round(x * p.on_prescale);
                xs[j][i] = x;
                ss = fmaf(x, x, ss);
            }
        ss = wave_sum(ss);
        const float rs = rsqrtf(ss / (float)V + p.on_eps);
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int d0 = 4 * lane + 256 * j;
            const float4 w = on_w4[j];
            const bf16x4 g4 = on_g4[j];
            const float wa[4] = {w.x, w.y, w.z, w.w};
            bf16x4 y;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float gv = s_gate ? s_gate[d0 + i] : (float)g4[i];  // formed in the kernel, or given
                y[i] = (bf16_t)(xs[j][i] * rs * wa[i] * sigmoidf(gv));
            }
            if (S == 1 || d0 * S / V == sp) *reinterpret_cast<bf16x4*>(p.o + (size_t)bh * V + d0) = y;
        }
    }
}

// q/k RMS norms (ops/fused_recurrent.py:62-89) from each thread's raw q, k
// channel (threads < K) and its norm weights qw, kw (loaded with the other
// small inputs), into s_q (scaled) and s_k; NW waves. Rounded to bf16 unless
// F32 (fp32 inputs).
template <int K, int NW, bool F32 = false>
__device__ __forceinline__ void qk_norms(const DecodeParams& p, float qv, float kv, float qw, float kw,
                                         float (*s_red)[NW], float* s_q, float* s_k) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0 && wave < K / 64) {
        s_red[0][wave] = sq;
        s_red[1][wave] = sk;
    }
    __syncthreads();
    float tq = 0.f, tk = 0.f;
#pragma unroll
    for (int i = 0; i < K / 64; i++) {
        tq += s_red[0][i];
        tk += s_red[1][i];
    }
    if (tid < K) {
        const float rq = rsqrtf(tq / K + p.q_eps), rk = rsqrtf(tk / K + p.k_eps);
        s_q[tid] = (F32 ? qv * rq * qw : bf16_round(qv * rq * qw)) * p.scale;
        s_k[tid] = F32 ? kv * rk * kw : bf16_round(kv * rk * kw);
    }
}

// The prefetch workgroups of the layer step (block ids B H onward, `nwg` of
// them after the nstep step workgroups; this is number `wg`, on XCD
// (nstep + wg) mod 8 as workgroups are dealt
// to the XCDs round-robin by block id): the ranges p.pf[r], range after
// range, so that the first range is in the caches first, eight 16 KiB units
// (one 16-byte load per thread) in flight per workgroup. A range with a span
// is read for its consumer: the consumer's workgroup c reads the span's bytes
// [c span, (c + 1) span) on XCD c mod 8, so this workgroup reads, in 16 KiB
// pieces, the spans of the consumer workgroups on its own XCD, which land in
// that XCD's L2; a range without one is read in units u = wg, wg + nwg, ...
// The values are consumed by an empty asm statement (the loads must not be
// dropped) and nothing is written. Loads past a range's end or a span's end
// read zero or are skipped (the dead offset).
__device__ __forceinline__ void prefetch_ranges(const DecodeParams& p, int wg, int nwg, int nstep) {
    const int x = (nstep + wg) & 7, qi = wg >> 3, nx = (nwg - (wg & 7) + 7) >> 3;
#pragma unroll 1
    for (int r = 0; r < 4; r++) {
        const unsigned long long bytes = p.pf_bytes[r];
        if (bytes == 0) continue;
        const rsrc_t rs = buf(p.pf[r], (size_t)bytes);  // bytes < 2^31: no 32-bit overflow below
        const uint32_t span = (uint32_t)p.pf_span[r];
        // units of this workgroup: u = first, first + stride, ... < units
        const uint32_t cpc = (span + 16383) >> 14;  // 16 KiB pieces per consumer span
        const uint32_t ncons = span ? (uint32_t)((bytes + span - 1) / span) : 0u;
        const uint32_t mine = span ? ((uint32_t)x < ncons ? (ncons - (uint32_t)x + 7) >> 3 : 0u) : 0u;
        const uint32_t units = span ? mine * cpc : (uint32_t)((bytes + 16383) >> 14);
        const uint32_t first = span ? (uint32_t)qi : (uint32_t)wg, stride = span ? (uint32_t)nx : (uint32_t)nwg;
#pragma unroll 1
        for (uint32_t u0 = first; u0 < units; u0 += 8u * stride) {
            f32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t u = u0 + (uint32_t)i * stride;
                uint32_t off, live = u < units;
                if (span) {  // piece j of consumer x + 8 (u / cpc)
                    const uint32_t c = (uint32_t)x + 8u * (u / cpc), in = (u % cpc) * 16384u + (uint32_t)threadIdx.x * 16u;
                    off = c * span + in;
                    live &= in < span;
                } else {
                    off = (u << 14) + (uint32_t)threadIdx.x * 16u;
                }
                v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off | (live ? 0u : DEAD), 0, 0));
            }
#pragma unroll
            for (int i = 0; i < 8; i++) asm volatile("" ::"v"(v[i]));
        }
    }
}

// The step workgroups' own inputs, read by the extra workgroups into the L2
// of the XCD each step workgroup runs on (workgroups are dealt to the eight
// XCDs round-robin by block id: step workgroup i on XCD i mod 8, extra
// workgroup q on XCD (nstep + q) mod 8, nstep = B H S step workgroups, S per
// (b, h); step workgroup i serves (b, h) = i mod B H, part i / B H). A step
// workgroup pulls about 450 KB through one compute unit, whose memory
// pipeline bounds it to a small fraction of the chip's rate; from its XCD's
// L2 the loads return sooner. Per step workgroup, 20 + 8 / S units of 16 KiB
// in the order the step reads them: hk (8), the head's table (4), hv (8), the
// part's g_proj[1] rows (8 / S); unit k of the XCD's j-th step workgroup is
// number k m + j of the XCD's list (m step workgroups on the XCD), taken by
// its extra workgroups in turn, eight units in flight. Loads past an input's
// end or of a null input read zero.
template <int K, int V>
__device__ __forceinline__ void prefetch_own_inputs(const DecodeParams& p, int q, int nwg, int S) {
    const int BH = p.B * p.H, nstep = BH * S, NU = 20 + 8 / S, x = (nstep + q) & 7;
    const int m = x < nstep ? (nstep - x + 7) >> 3 : 0;  // step workgroups x, x + 8, .. on this XCD
    const int qi = q >> 3, nx = (nwg - (q & 7) + 7) >> 3;
    const int units = NU * m;
#pragma unroll 1
    for (int u0 = qi; u0 < units; u0 += 8 * nx) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int u = u0 + i * nx, mm = m > 0 ? m : 1, k = u / mm, wi = x + 8 * (u - k * mm);
            const int bh = wi % BH, part = wi / BH, h = bh % p.H;
            const char* base = nullptr;
            size_t bytes = 0;
            if (u < units) {
                if (k < 8) {
                    base = p.hk_in ? reinterpret_cast<const char*>(p.hk_in + (size_t)bh * K * kSlots) + (size_t)k * 16384 : nullptr;
                    bytes = 16384;
                } else if (k < 12) {
                    base = reinterpret_cast<const char*>(p.table + (size_t)h * kActive * kSlots) + (size_t)(k - 8) * 16384;
                    bytes = (size_t)kActive * kSlots * 4 - (size_t)(k - 8) * 16384;
                } else if (k < 20) {
                    base = p.hv_in ? reinterpret_cast<const char*>(p.hv_in + (size_t)bh * kSlots * V) + (size_t)(k - 12) * 16384 : nullptr;
                    bytes = 16384;
                } else {
                    base = p.g1_w ? reinterpret_cast<const char*>(p.g1_w + (size_t)h * V * V) +
                                        (size_t)(part * 8 / S + k - 20) * 16384
                                  : nullptr;
                    bytes = 16384;
                }
            }
            v[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(buf(base, base ? bytes : 0),
                                                                                    (uint32_t)threadIdx.x * 16u, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < 8; i++) asm volatile("" ::"v"(v[i]));
    }
}

// The one-workgroup form. LAYER: the layer's one-token step around the op in
// the same kernel: q, k and v from the short convolution and the new conv
// cache, the gate activations from the a|b|d row, and o through the gated
// output norm. Phases: every load issued (small inputs, then hk, then hv);
// prologue (conv, gates, write vector, q/k norms) while the states stream in;
// key-state update as hk arrives; the slot readout while hv arrives; then the
// value-state update and o.
// S: step workgroups per (b, h) (LAYER only, outputs apart from inputs): each
// computes the whole step and stores its share of hk' (slices), hv' (rows) and
// o (columns, with the gate columns it forms); workgroup 0 of the (b, h) also
// the conv cache and the clock.
template <int K, int V, bool LAYER, bool F32 = false, int S = 1>
__global__ __launch_bounds__(1024) void decode_step_kernel(DecodeParams p) {
    constexpr int NT = 1024;
    constexpr int NS = K / SLICE;   // key-state slices
    constexpr int RK = NS / 4;      // slices per thread (four 256-thread groups)
    constexpr int VQ = V / 4;       // float4 per hv row
    constexpr int VROWS = NT / VQ;  // hv rows covered per sweep
    constexpr int VJ = kSlots / VROWS;
    constexpr int NW = NT / 64;
    constexpr int OJ = (V + 255) / 256;
    static_assert(S == 1 || (LAYER && !F32 && K == 256 && V == 256), "several workgroups per (b, h): the layer step");
    const int BH = p.B * p.H;
    if (LAYER && (int)blockIdx.x >= BH * S) {  // a prefetch workgroup (the whole workgroup exits here)
        if (p.self_pf) prefetch_own_inputs<K, V>(p, (int)blockIdx.x - BH * S, p.pf_wgs, S);
        prefetch_ranges(p, (int)blockIdx.x - BH * S, p.pf_wgs, BH * S);
        return;
    }
    const int bh = S == 1 ? (int)blockIdx.x : (int)blockIdx.x % BH, sp = S == 1 ? 0 : (int)blockIdx.x / BH;
    const int h = bh % p.H, b = bh / p.H, tid = threadIdx.x, vt = tid & 255;

    __shared__ float s_q[K], s_k[K], s_w[kSlots], s_raw[kSlots], s_z[kSlots];
    __shared__ float s_p[kSlots], s_om[kSlots], s_c[kPairs], s_s[kPairs];
    __shared__ float s_part[NW][256];
    __shared__ float s_kpart[NS][8][kSlots];  // key-state slice partials of raw, per 32-thread group
    __shared__ float s_red[2][NW];
    __shared__ float s_v[NT];  // v channel tid (tid < V); o in output_1024
    __shared__ __align__(16) float s_tab[kActive * kSlots];  // this head's readout table
    __shared__ bf16x8 s_g0[LAYER ? 32 : 1];                   // g0 (the gate formed in the kernel)
    __shared__ float s_gate[LAYER ? V : 1];

    const bool has_state = p.hk_in != nullptr;
    const bool own_gate = LAYER && p.g1_w != nullptr;
    float4* hk_out = reinterpret_cast<float4*>(p.hk_out + (size_t)bh * K * kSlots);
    float4* hv_out = reinterpret_cast<float4*>(p.hv_out + (size_t)bh * kSlots * V);

    // Small inputs: this thread's q and k channel tid and v channel tid (or
    // the conv windows they come from), the gates, the q/k norm weights, the
    // output norm inputs and the table.
    const uint32_t dk = dead_unless_below(tid, K), dv = dead_unless_below(tid, V);
    ConvIn cq{}, ck{}, cv{};
    float qv = 0.f, kv = 0.f, vv = 0.f;
    if (LAYER) {
        const int HK = p.H * K;
        const ConvSrc src = conv_src(p, b, 2 * HK + p.H * V);
        cq = load_conv(src, h * K + tid, dk);
        ck = load_conv(src, HK + h * K + tid, dk);
        cv = load_conv(src, 2 * HK + h * V + tid, dv);
    } else {
        qv = ld_in<F32>(p.q, bh, K, tid, dk);
        kv = ld_in<F32>(p.k, bh, K, tid, dk);
        vv = ld_in<F32>(p.v, bh, V, tid, dv);
    }
    const GateIn gi = load_gate_inputs<LAYER>(p, bh);
    const float qw = ld_f32(buf(p.q_w, (size_t)K * 4), ((uint32_t)tid * 4) | dk);
    const float kw = ld_f32(buf(p.k_w, (size_t)K * 4), ((uint32_t)tid * 4) | dk);
    float4 on_w4[OJ];
    bf16x4 on_g4[OJ];
    load_norm_inputs<V, LAYER>(p, bh, on_w4, on_g4);
    float4 tab[4];
    load_table(p, h, tab);
    const bf16x8 g0v = LAYER ? load_g0(p, b) : bf16x8{};

    // The key-state stream: slices (tid >> 8) + 4 r, four float4 of slice
    // thread vt each.
    const rsrc_t rk = buf(has_state ? p.hk_in + (size_t)bh * K * kSlots : nullptr, (size_t)K * kSlots * 4);
    float4 hk_r[RK][4];
#pragma unroll
    for (int r = 0; r < RK; r++)
#pragma unroll
        for (int j = 0; j < 4; j++) hk_r[r][j] = stream_load(rk, (uint32_t)(1024 * ((tid >> 8) + 4 * r) + vt + 256 * j) * 16);

    // Prologue.
    if (LAYER) {
        qv = conv_out(cq);
        kv = conv_out(ck);
        vv = conv_out(cv);
        const rsrc_t co = conv_out_rows(p, b, 2 * p.H * K + p.H * V);
        const uint32_t row = (uint32_t)p.cache_row * 2, sd = sp == 0 ? 0u : DEAD;
        store_conv_cache(co, row, h * K + tid, dk | sd, cq);
        store_conv_cache(co, row, p.H * K + h * K + tid, dk | sd, ck);
        store_conv_cache(co, row, 2 * p.H * K + h * V + tid, dv | sd, cv);
    }
    s_v[tid] = vv;  // every thread: a store behind tid < V let the compiler sink cv's loads below the states'
    if (LAYER && tid < 32) s_g0[tid] = g0v;
    float g_in, delta_in, beta_in;
    gate_values<LAYER>(p, bh, gi, g_in, delta_in, beta_in);
    stage_table(s_tab, tab);
    const float lam = gi.clock + delta_in;
    const float decay = expf(g_in);
    write_vector_lds<F32>(lam, beta_in, s_w, s_c, s_s);
    qk_norms<K, NW, F32>(p, qv, kv, qw, kw, s_red, s_q, s_k);
    __syncthreads();
    if (tid == 0 && sp == 0) p.clock_out[bh] = lam;  // after every thread has read clock_in

    // The value-state stream, float4 tid + NT j, issued once the small
    // inputs' registers are free; it is first needed after the readout.
    const rsrc_t rv = buf(has_state ? p.hv_in + (size_t)bh * kSlots * V : nullptr, (size_t)kSlots * V * 4);
    float4 hv_r[VJ];
#pragma unroll
    for (int j = 0; j < VJ; j++) hv_r[j] = stream_load(rv, (uint32_t)(tid + NT * j) * 16);

    // Key state: hk' = alpha hk + k_hat (x) w ; raw = hk'^T q_hat, by slices
    // (with S > 1, slice s stored by part s S / NS).
    const rsrc_t hk_o = buf(p.hk_out + (size_t)bh * K * kSlots, (size_t)K * kSlots * 4);
#pragma unroll
    for (int r = 0; r < RK; r++) {
        const int s = (tid >> 8) + 4 * r;
        const float4 a = key_slice_update(hk_r[r], hk_out, s, vt, decay, s_k, s_q, s_w, S == 1 ? nullptr : &hk_o,
                                          s * S / NS == sp ? 0u : DEAD);
        float* pt = &s_kpart[s][vt >> 5][(vt & 31) * 4];
        pt[0] = a.x;
        pt[1] = a.y;
        pt[2] = a.z;
        pt[3] = a.w;
    }
    // the gate projection's weights (L2-resident), in the key state's registers;
    // issued with the value state they would not fit beside it
    GateW gw{};
    if (LAYER) gw = load_gate_weights(p, h, S == 1 || (int)(tid >> 6) * S / NW == sp);
    __syncthreads();
    if (tid < kSlots) {
        float r = slice_partial(&s_kpart[0][0][0], tid);
#pragma unroll
        for (int s = 1; s < NS; s++) r += slice_partial(&s_kpart[s][0][0], tid);
        s_raw[tid] = r;
    }
    __syncthreads();
    readout_1024(s_raw, s_c, s_s, s_tab, s_z, s_p, s_part, s_om);

    // Value state: hv' = alpha hv + w (x) v, written now; kept in hv_r for o.
    {
        const int v4 = (tid % VQ) * 4, r0 = tid / VQ;
        const float v0 = s_v[v4], v1 = s_v[v4 + 1], v2 = s_v[v4 + 2], v3 = s_v[v4 + 3];
#pragma unroll
        for (int j = 0; j < VJ; j++) {
            const float wm = s_w[r0 + VROWS * j];
            float4 n = hv_r[j];
            n.x = fmaf(n.x, decay, wm * v0);
            n.y = fmaf(n.y, decay, wm * v1);
            n.z = fmaf(n.z, decay, wm * v2);
            n.w = fmaf(n.w, decay, wm * v3);
            if constexpr (S == 1) {
                stream_store(hv_out + tid + NT * j, n);
            } else {  // rows of sweep j stored by part j S / VJ
                const rsrc_t hv_o = buf(p.hv_out + (size_t)bh * kSlots * V, (size_t)kSlots * V * 4);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(f32x4, n), hv_o,
                                                       ((uint32_t)(tid + NT * j) * 16) | (j * S / VJ == sp ? 0u : DEAD), 0, 2);
            }
            hv_r[j] = n;
        }
    }
    if (own_gate) gate_columns(s_g0, gw, s_gate);
    output_1024<V, LAYER, F32, S>(p, bh, hv_r, s_om, s_part, s_v, on_w4, on_g4, own_gate ? s_gate : nullptr, sp);
}

// Small-batch form, part A: grid (NSL, B H), 256 threads; workgroup s updates
// key-state slice s (rows 32 s ..) and value-state slice s (columns 32 s ..)
// and writes its slice's partial raw to part_out[(bh NSL + s) 128 + m]. The
// conv cache and the clock are left to part B, which runs after every
// workgroup of part A has read them.
template <int K, int V, bool LAYER>
__global__ __launch_bounds__(256) void decode_split_a_kernel(DecodeParams p) {
    constexpr int NT = 256, NW = NT / 64;
    constexpr int NSL = (K > V ? K : V) / SLICE;
    constexpr int VQ = V / 4;
    const int s = blockIdx.x, bh = blockIdx.y, h = bh % p.H, b = bh / p.H, tid = threadIdx.x;
    __shared__ float s_q[K], s_k[K], s_w[kSlots], s_c[kPairs], s_s[kPairs];
    __shared__ float s_kpart[8][kSlots];
    __shared__ float s_v[NT];  // v channel 32 s + tid (tid < 32)
    __shared__ float s_red[2][NW];

    const bool key = s < K / SLICE, val = s < V / SLICE;
    const bool has_state = p.hk_in != nullptr;
    float4* hk_out = reinterpret_cast<float4*>(p.hk_out + (size_t)bh * K * kSlots);
    float4* hv_out = reinterpret_cast<float4*>(p.hv_out + (size_t)bh * kSlots * V);

    // small inputs first (q, k channel tid; v channel 32 s + tid), then the slices
    const uint32_t dk = dead_unless_below(tid, K), dv = val ? dead_unless_below(tid, SLICE) : DEAD;
    ConvIn cq{}, ck{}, cv{};
    float qv = 0.f, kv = 0.f, vv = 0.f;
    if (LAYER) {
        const int HK = p.H * K;
        const ConvSrc src = conv_src(p, b, 2 * HK + p.H * V);
        cq = load_conv(src, h * K + tid, dk);
        ck = load_conv(src, HK + h * K + tid, dk);
        cv = load_conv(src, 2 * HK + h * V + SLICE * s + tid, dv);
    } else {
        qv = ld_in<false>(p.q, bh, K, tid, dk);
        kv = ld_in<false>(p.k, bh, K, tid, dk);
        vv = ld_in<false>(p.v, bh, V, SLICE * s + tid, dv);
    }
    const GateIn gi = load_gate_inputs<LAYER>(p, bh);
    const float qw = ld_f32(buf(p.q_w, (size_t)K * 4), ((uint32_t)tid * 4) | dk);
    const float kw = ld_f32(buf(p.k_w, (size_t)K * 4), ((uint32_t)tid * 4) | dk);
    // This workgroup's slices of both states: hk float4 1024 s + tid + 256 j;
    // hv row tid / 8 + 32 j, columns 32 s + 4 (tid % 8) ...
    const rsrc_t rk = buf(has_state && key ? p.hk_in + (size_t)bh * K * kSlots : nullptr, (size_t)K * kSlots * 4);
    const rsrc_t rv = buf(has_state && val ? p.hv_in + (size_t)bh * kSlots * V : nullptr, (size_t)kSlots * V * 4);
    float4 hk_r[4], hv_r[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        hk_r[j] = stream_load(rk, (uint32_t)(1024 * s + tid + 256 * j) * 16);
        hv_r[j] = stream_load(rv, (uint32_t)(((tid >> 3) + 32 * j) * VQ + 8 * s + (tid & 7)) * 16);
    }
    if (LAYER) {
        qv = conv_out(cq);
        kv = conv_out(ck);
        vv = conv_out(cv);
    }
    s_v[tid] = vv;  // every thread (see decode_step_kernel)
    float g_in, delta_in, beta_in;
    gate_values<LAYER>(p, bh, gi, g_in, delta_in, beta_in);
    const float lam = gi.clock + delta_in;
    const float decay = expf(g_in);
    write_vector_lds(lam, beta_in, s_w, s_c, s_s);
    qk_norms<K, NW>(p, qv, kv, qw, kw, s_red, s_q, s_k);
    __syncthreads();
    if (key) {
        const float4 a = key_slice_update(hk_r, hk_out, s, tid, decay, s_k, s_q, s_w);
        float* pt = &s_kpart[tid >> 5][(tid & 31) * 4];
        pt[0] = a.x;
        pt[1] = a.y;
        pt[2] = a.z;
        pt[3] = a.w;
    }
    if (val) {
        const int c = 4 * (tid & 7);
        const float v0 = s_v[c], v1 = s_v[c + 1], v2 = s_v[c + 2], v3 = s_v[c + 3];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int m = (tid >> 3) + 32 * j;
            const float wm = s_w[m];
            float4 n = hv_r[j];
            n.x = fmaf(n.x, decay, wm * v0);
            n.y = fmaf(n.y, decay, wm * v1);
            n.z = fmaf(n.z, decay, wm * v2);
            n.w = fmaf(n.w, decay, wm * v3);
            stream_store(hv_out + (size_t)m * VQ + 8 * s + (tid & 7), n);
        }
    }
    __syncthreads();
    if (key && tid < kSlots) p.part[((size_t)bh * NSL + s) * kSlots + tid] = slice_partial(&s_kpart[0][0], tid);
}

// Small-batch form, part B: one 1024-thread workgroup per (b, h): raw from the
// slices' partials (slice order), the readout, o from the updated value state
// (read back, L2-resident), the conv cache and the clock.
template <int K, int V, bool LAYER>
__global__ __launch_bounds__(1024) void decode_split_b_kernel(DecodeParams p) {
    constexpr int NT = 1024;
    constexpr int NS = K / SLICE, NSL = (K > V ? K : V) / SLICE;
    constexpr int VQ = V / 4, VROWS = NT / VQ, VJ = kSlots / VROWS;
    constexpr int NW = NT / 64;
    constexpr int OJ = (V + 255) / 256;
    const int bh = blockIdx.x, h = bh % p.H, b = bh / p.H, tid = threadIdx.x;
    __shared__ float s_raw[kSlots], s_z[kSlots], s_p[kSlots], s_om[kSlots], s_c[kPairs], s_s[kPairs], s_w[kSlots];
    __shared__ float s_part[NW][256];
    __shared__ float s_v[LAYER ? V : 1];
    __shared__ __align__(16) float s_tab[kActive * kSlots];
    __shared__ bf16x8 s_g0[LAYER ? 32 : 1];
    __shared__ float s_gate[LAYER ? V : 1];

    const bool own_gate = LAYER && p.g1_w != nullptr;
    float4 on_w4[OJ];
    bf16x4 on_g4[OJ];
    load_norm_inputs<V, LAYER>(p, bh, on_w4, on_g4);
    const bf16x8 g0v = LAYER ? load_g0(p, b) : bf16x8{};
    GateW gw{};
    if (LAYER) gw = load_gate_weights(p, h);
    const GateIn gi = load_gate_inputs<LAYER>(p, bh);
    // the slices' partials of raw (threads < 128, slice order)
    const rsrc_t rp = buf(p.part + (size_t)bh * NSL * kSlots, (size_t)NSL * kSlots * 4);
    const uint32_t dm = dead_unless_below(tid, kSlots);
    float part_r[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) part_r[s] = ld_f32(rp, ((uint32_t)(s * kSlots + tid) * 4) | dm);
    // The conv cache of this head's channels: the last three rows of each
    // window (each channel read and written by one thread, so an in-place
    // update needs no ordering between threads).
    const int HK = p.H * K;
    const int ch = tid < K ? h * K + tid : tid < 2 * K ? HK + h * K + (tid - K) : 2 * HK + h * V + (tid - 2 * K);
    float win[3] = {0.f, 0.f, 0.f};
    if (LAYER) {
        const ConvSrc src = conv_src(p, b, 2 * HK + p.H * V);
        const uint32_t dc = dead_unless_below(tid, 2 * K + V);
#pragma unroll
        for (int w = 1; w < 3; w++) win[w - 1] = ld_bf16(src.cache, (w * src.row + (uint32_t)ch * 2) | dc);
        win[2] = ld_bf16(src.qkv, ((uint32_t)ch * 2) | dc);
    }
    float4 tab[4];
    load_table(p, h, tab);
    const rsrc_t rv = buf(p.hv_out + (size_t)bh * kSlots * V, (size_t)kSlots * V * 4);
    float4 hv_r[VJ];
#pragma unroll
    for (int j = 0; j < VJ; j++) hv_r[j] = ld_f32x4(rv, (uint32_t)(tid + NT * j) * 16);
    if (tid < kSlots) {
        float r = part_r[0];
#pragma unroll
        for (int s = 1; s < NS; s++) r += part_r[s];
        s_raw[tid] = r;
    }
    if (LAYER && tid < 2 * K + V) {
#pragma unroll
        for (int w = 0; w < 3; w++)
            p.cache_out[(size_t)b * p.cache_batch + (size_t)w * p.cache_row + ch] = (bf16_t)win[w];
    }
    float g_in, delta_in, beta_in;
    gate_values<LAYER>(p, bh, gi, g_in, delta_in, beta_in);
    (void)g_in;
    const float lam = gi.clock + delta_in;
    write_vector_lds(lam, beta_in, s_w, s_c, s_s);
    stage_table(s_tab, tab);
    if (LAYER && tid < 32) s_g0[tid] = g0v;
    __syncthreads();
    if (tid == 0) p.clock_out[bh] = lam;  // after every thread has read clock_in
    readout_1024(s_raw, s_c, s_s, s_tab, s_z, s_p, s_part, s_om);
    if (own_gate) gate_columns(s_g0, gw, s_gate);
    output_1024<V, LAYER>(p, bh, hv_r, s_om, s_part, s_v, on_w4, on_g4, own_gate ? s_gate : nullptr);
}

template <int K, int V, bool LAYER>
void launch(const DecodeParams& p, hipStream_t stream) {
    const int BH = p.B * p.H;
    if (p.part && BH < DECODE_SPLIT_BH) {
        constexpr int NSL = (K > V ? K : V) / SLICE;
        hipLaunchKernelGGL((decode_split_a_kernel<K, V, LAYER>), dim3(NSL, BH), dim3(256), 0, stream, p);
        hipLaunchKernelGGL((decode_split_b_kernel<K, V, LAYER>), dim3(BH), dim3(1024), 0, stream, p);
    } else {
        // the layer step's prefetch workgroups follow the B H S step workgroups
        // (dispatched after them, so they take the idle compute units)
        const int extra = LAYER ? p.pf_wgs : 0;
        if constexpr (LAYER && K == 256 && V == 256) {
            if (p.wpb == 4) {
                hipLaunchKernelGGL((decode_step_kernel<K, V, true, false, 4>), dim3(4 * BH + extra), dim3(1024), 0, stream, p);
                return;
            }
            if (p.wpb == 2) {
                hipLaunchKernelGGL((decode_step_kernel<K, V, true, false, 2>), dim3(2 * BH + extra), dim3(1024), 0, stream, p);
                return;
            }
        }
        hipLaunchKernelGGL((decode_step_kernel<K, V, LAYER>), dim3(BH + extra), dim3(1024), 0, stream, p);
    }
}

// The op step; fp32 inputs always take the one-workgroup form.
template <int K, int V>
void launch_op(const DecodeParams& p, hipStream_t stream) {
    if (p.f32)
        hipLaunchKernelGGL((decode_step_kernel<K, V, false, true>), dim3(p.B * p.H), dim3(1024), 0, stream, p);
    else
        launch<K, V, false>(p, stream);
}

}  // namespace

size_t decode_workspace_bytes(int B, int H, int K, int V) {
    if (B <= 0 || H <= 0 || (long long)B * H >= DECODE_SPLIT_BH) return 0;
    return (size_t)B * H * ((K > V ? K : V) / SLICE) * kSlots * sizeof(float);
}

int launch_decode_step(const DecodeParams& p, int K, int V, hipStream_t stream) {
    if (p.qkv) {  // the layer step: K = V = 256 and bf16 only
        if (K != 256 || V != 256 || p.f32) return -1;
        // every buffer the kernels read spans less than DEAD bytes
        const long long D = (long long)p.H * (2 * K + V);
        if (p.cache_in && (p.cache_row < 0 || (2 * p.cache_row + D) * 2 >= (long long)DEAD)) return -1;
        if (D * 8 >= (long long)DEAD) return -1;
        launch<256, 256, true>(p, stream);
    } else if (K == 256 && V == 256)
        launch_op<256, 256>(p, stream);
    else if (K == 128 && V == 128)
        launch_op<128, 128>(p, stream);
    else if (K == 256 && V == 128)
        launch_op<256, 128>(p, stream);
    else if (K == 128 && V == 256)
        launch_op<128, 256>(p, stream);
    else
        return -1;
    return 0;
}

}  // namespace cyfa
