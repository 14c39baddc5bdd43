// cyfa_decode.hip -- fused constant-memory CyFA decode step for gfx950.
//
// One 1024-thread workgroup per (batch, head). The step is HBM-bound: it
// streams the fp32 key state hk [K, M] and value state hv [M, V] in and out
// once (512 KiB per (b, h) for K = V = 256). Both states are issued as
// coalesced float4 loads at kernel entry. Both updated states are written
// before the slot readout runs (the value-state update does not depend on the
// readout; the updated hv stays in registers for o = hv'^T weights), so the
// write stream drains while the readout computes.
//
// Math (ops/fused_recurrent.py:57-188): q_hat = bf16(q rs_q w_q) * scale,
// k_hat = bf16(k rs_k w_k); lam = clock + delta; alpha = e^g;
// w = bf16(beta U(-lam) b); hk' = alpha hk + k_hat (x) w; raw = hk'^T q_hat;
// z = U(lam) raw; p = softmax(table z); u = table^T p; weights = U(-lam) u;
// hv' = alpha hv + w (x) v; o = bf16(hv'^T weights).
// The readout is evaluated in fp32 (the reference rounds z, the table and p
// to bf16 here); the write vector and the normalised q/k keep the reference's
// bf16 rounding so decode and the chunkwise prefill see identical operands.
#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

// The states are touched exactly once per step: non-temporal loads and stores
// keep them from displacing reusable lines in the caches (about 20% faster
// at B = 64 with the state streaming from HBM).
__device__ __forceinline__ float4 stream_load(const float4* p) {
    return __builtin_bit_cast(float4, __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p)));
}

__device__ __forceinline__ void stream_store(float4* p, const float4& v) {
    __builtin_nontemporal_store(__builtin_bit_cast(f32x4, v), reinterpret_cast<f32x4*>(p));
}

// LAYER: the layer's one-token step around the op in the same kernel. The
// width-4 causal short convolution of the projection row (layers/cyfa.py:138-233,
// the arithmetic of short_conv_kernel) gives this head's q, k and v and the new
// conv cache; the gate activations (layers/cyfa.py:323-326, as gates_kernel)
// come from the a|b|d row; and o goes through the gated output norm
// o_norm(o * prescale, gate) (layers/cyfa.py:349-350, as rms_norm_kernel<1>:
// wave 0 holds four consecutive values per lane) before it is stored.
template <int K, int V, bool LAYER>
__global__ __launch_bounds__(1024) void decode_step_kernel(DecodeParams p) {
    constexpr int NT = 1024;
    constexpr int KJ = K / 32;      // float4 of hk per thread (row has 32 float4)
    constexpr int VQ = V / 4;       // float4 per hv row
    constexpr int VROWS = NT / VQ;  // hv rows covered per sweep
    constexpr int VJ = kSlots / VROWS;
    constexpr int NW = NT / 64;
    const int bh = blockIdx.x, h = bh % p.H, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;

    __shared__ float s_q[K], s_k[K], s_w[kSlots], s_raw[kSlots], s_z[kSlots];
    __shared__ float s_p[kSlots], s_om[kSlots], s_c[kPairs], s_s[kPairs];
    __shared__ float s_part[NW][V > kSlots ? V : kSlots];
    __shared__ float s_red[2][NW];
    __shared__ float s_v[LAYER ? V : 1];
    __shared__ __align__(16) float s_tab[kActive * kSlots];  // this head's readout table

    const bool has_state = p.hk_in != nullptr;
    const float4* hk_in = reinterpret_cast<const float4*>(p.hk_in + (size_t)bh * K * kSlots);
    const float4* hv_in = reinterpret_cast<const float4*>(p.hv_in + (size_t)bh * kSlots * V);
    float4* hk_out = reinterpret_cast<float4*>(p.hk_out + (size_t)bh * K * kSlots);
    float4* hv_out = reinterpret_cast<float4*>(p.hv_out + (size_t)bh * kSlots * V);

    // Layer step: the short-convolution inputs of this thread's channels (the
    // q and k channel tid, the v channel tid) are loaded ahead of the state
    // streams, so they arrive first. win[c][0..2] = cache rows, win[c][3] = x.
    float cwin[3][4], cwt[3][4];
    if (LAYER) {
        const int b = bh / p.H, HK = p.H * K;
        const int ch[3] = {h * K + tid, HK + h * K + tid, 2 * HK + h * V + tid};
#pragma unroll
        for (int c = 0; c < 3; c++) {
            if (tid < (c < 2 ? K : V)) {
#pragma unroll
                for (int w = 0; w < 3; w++)
                    cwin[c][w] = p.cache_in ? (float)p.cache_in[(size_t)b * p.cache_batch + (size_t)w * p.cache_row + ch[c]]
                                            : 0.f;
                cwin[c][3] = (float)p.qkv[(size_t)b * p.qkv_row + ch[c]];
                const bf16x4 wt = *reinterpret_cast<const bf16x4*>(p.conv_w + (size_t)ch[c] * 4);  // one 8-byte load
#pragma unroll
                for (int w = 0; w < 4; w++) cwt[c][w] = (float)wt[w];
            }
        }
    }

    // Layer step: wave 0's norm weight and gate for the output norm at the
    // end, loaded now so that their latency is not the kernel's last step.
    constexpr int OJ = (V + 255) / 256;  // four consecutive values per lane and 256-wide block
    float4 on_w4[OJ];
    bf16x4 on_g4[OJ];
    if (LAYER && wave == 0) {
        const bf16_t* gt = p.gate + (size_t)(bh / p.H) * p.gate_row + (size_t)h * V;
#pragma unroll
        for (int j = 0; j < OJ; j++) {
            on_w4[j] = *reinterpret_cast<const float4*>(p.on_w + 4 * lane + 256 * j);
            on_g4[j] = *reinterpret_cast<const bf16x4*>(gt + 4 * lane + 256 * j);
        }
    }

    // The readout table (L2-resident, 64 KB per head) is read into registers
    // ahead of the state streams and staged in LDS during the prologue, so the
    // readout after the state writes finds it on chip.
    constexpr int TQ = kActive * kSlots / 4;  // float4 of the table: 3 per thread, 4 for the first 992
    static_assert(NT == 1024 && TQ > 3 * NT && TQ <= 4 * NT, "table staging covers the table");
    const float4* tb4 = reinterpret_cast<const float4*>(p.table + (size_t)h * kActive * kSlots);
    const float4 tab0 = tb4[tid], tab1 = tb4[tid + NT], tab2 = tb4[tid + 2 * NT];
    const float4 tab3 = tid + 3 * NT < TQ ? tb4[tid + 3 * NT] : float4{0.f, 0.f, 0.f, 0.f};

    // Issue both state streams; everything below overlaps with them.
    float4 hk_r[KJ], hv_r[VJ];
    if (has_state) {
#pragma unroll
        for (int j = 0; j < KJ; j++) hk_r[j] = stream_load(hk_in + tid + NT * j);
#pragma unroll
        for (int j = 0; j < VJ; j++) hv_r[j] = stream_load(hv_in + tid + NT * j);
    } else {
#pragma unroll
        for (int j = 0; j < KJ; j++) hk_r[j] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < VJ; j++) hv_r[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    // q/k RMS statistics (ops/fused_recurrent.py:62-89).
    float qv = 0.f, kv = 0.f;
    float g_in, delta_in, beta_in;
    if (LAYER) {
        const int b = bh / p.H;
        const int HK = p.H * K;
        // The arithmetic of short_conv_kernel; the new cache is the last three rows of the window.
        auto conv = [&](int c, int ch) -> float {
            float acc = cwin[c][0] * cwt[c][0];
#pragma unroll
            for (int w = 1; w < 4; w++) acc = fmaf(cwin[c][w], cwt[c][w], acc);
#pragma unroll
            for (int w = 0; w < 3; w++)
                p.cache_out[(size_t)b * p.cache_batch + (size_t)w * p.cache_row + ch] = (bf16_t)cwin[c][w + 1];
            return bf16_round(acc);
        };
        if (tid < K) {
            qv = conv(0, h * K + tid);
            kv = conv(1, HK + h * K + tid);
        }
        if (tid < V) s_v[tid] = conv(2, 2 * HK + h * V + tid);
        const bf16_t* row = p.abd + (size_t)b * p.abd_row;
        const float a = (float)row[h] + p.dt_bias[h];
        const float sp = a > 20.f ? a : log1pf(expf(a));
        g_in = -expf(p.A_log[h]) * sp;
        beta_in = sigmoidf((float)row[p.H + h]);
        delta_in = sigmoidf((float)row[2 * p.H + h]);
    } else {
        if (tid < K) {
            qv = (float)p.q[(size_t)bh * K + tid];
            kv = (float)p.k[(size_t)bh * K + tid];
        }
        g_in = p.g[bh];
        delta_in = p.delta[bh];
        beta_in = p.beta[bh];
    }
    const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0 && wave < K / 64) {
        s_red[0][wave] = sq;
        s_red[1][wave] = sk;
    }
    {
        float4* st4 = reinterpret_cast<float4*>(s_tab);
        st4[tid] = tab0;
        st4[tid + NT] = tab1;
        st4[tid + 2 * NT] = tab2;
        if (tid + 3 * NT < TQ) st4[tid + 3 * NT] = tab3;
    }
    const float clock = has_state ? p.clock_in[bh] : 0.f;
    const float lam = clock + delta_in;
    const float decay = expf(g_in);
    const float beta = beta_in;
    if (tid < kPairs) {
        float s, c;
        pair_sincos(reduced_clock(lam), tid, s, c);
        const float a = beta * pair_scale(tid);
        s_w[2 * tid] = bf16_round(a * c);
        s_w[2 * tid + 1] = bf16_round(-a * s);
        s_c[tid] = c;
        s_s[tid] = s;
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
        s_q[tid] = bf16_round(qv * rq * p.q_w[tid]) * p.scale;
        s_k[tid] = bf16_round(kv * rk * p.k_w[tid]);
    }
    __syncthreads();
    if (tid == 0) p.clock_out[bh] = lam;  // after every thread has read clock_in

    // Key state: hk' = alpha hk + k_hat (x) w ; raw = hk'^T q_hat.
    {
        const int m4 = (tid & 31) * 4;
        const float w0 = s_w[m4], w1 = s_w[m4 + 1], w2 = s_w[m4 + 2], w3 = s_w[m4 + 3];
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int d = (tid >> 5) + 32 * j;
            const float kd = s_k[d], qd = s_q[d];
            float4 n = hk_r[j];
            n.x = fmaf(n.x, decay, kd * w0);
            n.y = fmaf(n.y, decay, kd * w1);
            n.z = fmaf(n.z, decay, kd * w2);
            n.w = fmaf(n.w, decay, kd * w3);
            stream_store(hk_out + tid + NT * j, n);
            a0 = fmaf(n.x, qd, a0);
            a1 = fmaf(n.y, qd, a1);
            a2 = fmaf(n.z, qd, a2);
            a3 = fmaf(n.w, qd, a3);
        }
        a0 += __shfl_xor(a0, 32);
        a1 += __shfl_xor(a1, 32);
        a2 += __shfl_xor(a2, 32);
        a3 += __shfl_xor(a3, 32);
        if (lane < 32) {
            s_part[wave][m4] = a0;
            s_part[wave][m4 + 1] = a1;
            s_part[wave][m4 + 2] = a2;
            s_part[wave][m4 + 3] = a3;
        }
    }
    // Value state: hv' = alpha hv + w (x) v, written now; kept in hv_r for o.
    {
        const int v4 = (tid % VQ) * 4, r0 = tid / VQ;
        float v0, v1, v2, v3;
        if (LAYER) {
            v0 = s_v[v4];
            v1 = s_v[v4 + 1];
            v2 = s_v[v4 + 2];
            v3 = s_v[v4 + 3];
        } else {
            const bf16x4 vb = *reinterpret_cast<const bf16x4*>(p.v + (size_t)bh * V + v4);
            v0 = (float)vb[0];
            v1 = (float)vb[1];
            v2 = (float)vb[2];
            v3 = (float)vb[3];
        }
#pragma unroll
        for (int j = 0; j < VJ; j++) {
            const float wm = s_w[r0 + VROWS * j];
            float4 n = hv_r[j];
            n.x = fmaf(n.x, decay, wm * v0);
            n.y = fmaf(n.y, decay, wm * v1);
            n.z = fmaf(n.z, decay, wm * v2);
            n.w = fmaf(n.w, decay, wm * v3);
            stream_store(hv_out + tid + NT * j, n);
            hv_r[j] = n;
        }
    }
    __syncthreads();
    if (tid < kSlots) {
        float r = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) r += s_part[w][tid];
        s_raw[tid] = r;
    }
    __syncthreads();

    // Slot readout (ops/fused_recurrent.py:114-175), fp32.
    if (tid < kPairs) {
        const float c = s_c[tid], s = s_s[tid];
        const float e = s_raw[2 * tid], o = s_raw[2 * tid + 1];
        s_z[2 * tid] = c * e - s * o;
        s_z[2 * tid + 1] = s * e + c * o;
    }
    __syncthreads();
    const float* tb = s_tab;
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
        lg += __shfl_xor(lg, 1);
        lg += __shfl_xor(lg, 2);
        lg += __shfl_xor(lg, 4);
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

    // o = hv'^T weights, from the updated value state kept in registers.
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
            for (int w = 0; w < NW; w++) s += s_part[w][tid];
            p.o[(size_t)bh * V + tid] = (bf16_t)s;
        }
        return;
    }
    if (tid < V) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) s += s_part[w][tid];
        s_v[tid] = (float)(bf16_t)s;  // o as the op would store it
    }
    __syncthreads();
    if (wave == 0) {
        constexpr int J = OJ;
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
            for (int i = 0; i < 4; i++) y[i] = (bf16_t)(xs[j][i] * rs * wa[i] * sigmoidf((float)g4[i]));
            *reinterpret_cast<bf16x4*>(p.o + (size_t)bh * V + d0) = y;
        }
    }
}

int launch_decode_step(const DecodeParams& p, int K, int V, hipStream_t stream) {
    dim3 grid(p.B * p.H), block(1024);
    if (p.qkv) {  // the layer step: K = V = 256 only
        if (K != 256 || V != 256) return -1;
        hipLaunchKernelGGL((decode_step_kernel<256, 256, true>), grid, block, 0, stream, p);
    } else if (K == 256 && V == 256)
        hipLaunchKernelGGL((decode_step_kernel<256, 256, false>), grid, block, 0, stream, p);
    else if (K == 128 && V == 128)
        hipLaunchKernelGGL((decode_step_kernel<128, 128, false>), grid, block, 0, stream, p);
    else if (K == 256 && V == 128)
        hipLaunchKernelGGL((decode_step_kernel<256, 128, false>), grid, block, 0, stream, p);
    else if (K == 128 && V == 256)
        hipLaunchKernelGGL((decode_step_kernel<128, 256, false>), grid, block, 0, stream, p);
    else
        return -1;
    return 0;
}

}  // namespace cyfa
