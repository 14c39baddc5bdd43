// cyfa_device.h -- device-side helpers shared by the CyFA gfx950 kernels.
//
// Vector types for the CDNA4 MFMA builtins, bf16/fp16 conversions (hardware
// round-to-nearest-even conversions on gfx950), the integer range-reduced
// clock phase and wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cyfa {

constexpr int kSlots = 128;   // stored slot coordinates M
constexpr int kActive = 127;  // active slots R = M - 1
constexpr int kPairs = 64;    // Fourier pairs M / 2
constexpr int kChunk = 64;    // tokens per chunk
constexpr int kMaxSegments = 8192;  // segments per sequence in a prefill sweep

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_round(float x) { return (float)(bf16_t)x; }

// Load 8 consecutive bf16 (16 bytes, 16-byte aligned) and widen to fp32.
__device__ __forceinline__ void load_bf16x8(const bf16_t* p, float out[8]) {
    bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; i++) out[i] = (float)v[i];
}

// Clock phase of Fourier pair `pair` at clock lam, with the integer range
// reduction of the reference (ops/utils.py:649-661):
//   wi = floor(lam) mod R (non-negative); coord = ((wi * pair) mod R) + frac(lam) * pair,
//   wrapped into (-R/2, R/2]; theta = coord * 2 pi / R.
// The integer part keeps |theta| <= pi exact for any clock value, so the phase
// stays accurate when lam grows to 1e4 and beyond.
__device__ __forceinline__ float clock_phase(float lam, int pair) {
    const float whole = floorf(lam);
    const float frac = lam - whole;
    int wi = (int)whole % kActive;
    if (wi < 0) wi += kActive;
    float coord = (float)((wi * pair) % kActive) + frac * (float)pair;
    if (coord > 0.5f * kActive) coord -= (float)kActive;
    return coord * 0.049473900056532176f;  // 2 pi / 127
}

// The same reduced phase in revolutions (coord / R, in (-1/2, 1/2]) evaluated
// with the hardware sine/cosine (v_sin_f32 / v_cos_f32 take revolutions).
// The argument is already reduced exactly, so no further range reduction is
// needed.
__device__ __forceinline__ void phase_sincos(float lam, int pair, float& s, float& c) {
    const float whole = floorf(lam);
    const float frac = lam - whole;
    int wi = (int)whole % kActive;
    if (wi < 0) wi += kActive;
    float coord = (float)((wi * pair) % kActive) + frac * (float)pair;
    if (coord > 0.5f * kActive) coord -= (float)kActive;
    const float rev = coord * (1.0f / kActive);
    s = __builtin_amdgcn_sinf(rev);
    c = __builtin_amdgcn_cosf(rev);
}

// Clock reduced once per token: lam' = (lam mod R) / R. The phase of pair p
// in revolutions is then p * lam' (the same angle, modulo 2 pi, as the
// reference's integer reduction above; p * lam' < 64 revolutions so one fp32
// product keeps the angle to ~2.5e-5 rad), and the sine / cosine of pair p
// cost one multiply and one transcendental each. lam - R floor(lam / R) is
// formed with one fma, which is exact (the result is a multiple of lam's ulp
// below 2 R); the quotient estimate may be off by one, which the two
// corrections undo.
__device__ __forceinline__ float reduced_clock(float lam) {
    const float q = floorf(lam * (1.0f / kActive));
    float r = fmaf(-(float)kActive, q, lam);
    r = r < 0.f ? r + (float)kActive : r;
    r = r >= (float)kActive ? r - (float)kActive : r;
    return r * (1.0f / kActive);
}

// 2^x with the hardware exponential (v_exp_f32); results below the normal
// range flush to zero, which is what every caller wants for decay factors.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void pair_sincos(float lamr, int pair, float& s, float& c) {
    const float rev = (float)pair * lamr;
    s = __builtin_amdgcn_sinf(rev);
    c = __builtin_amdgcn_cosf(rev);
}

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// s_p of the real-DFT basis: (1/R)^1/2 for pair 0, (2/R)^1/2 otherwise.
__device__ __forceinline__ float pair_scale(int pair) {
    return pair == 0 ? 0.088735650941611332f : 0.12549115289319523f;
}

// Write-vector pair (w[2p], w[2p+1]) = beta s_p (cos theta_p, -sin theta_p)
// (ops/utils.py:664-702), before rounding; lamr = reduced_clock(lam).
__device__ __forceinline__ void write_pair(float lamr, float beta, int pair, float& we, float& wo) {
    float s, c;
    pair_sincos(lamr, pair, s, c);
    const float a = beta * pair_scale(pair);
    we = a * c;
    wo = -a * s;
}

// Write-vector element m alone: beta s_p cos(theta_p) for even m,
// -beta s_p sin(theta_p) for odd m (one transcendental).
__device__ __forceinline__ float write_coord(float lamr, float beta, int m) {
    const int pair = m >> 1;
    const float rev = (float)pair * lamr;
    const float a = beta * pair_scale(pair);
    return (m & 1) ? -a * __builtin_amdgcn_sinf(rev) : a * __builtin_amdgcn_cosf(rev);
}

// 1 / (1 + e^-x) with the hardware exponential and reciprocal (v_exp_f32,
// v_rcp_f32, each within 1 ulp): a relative error of a few 1e-7, far below the
// bf16 rounding of every result it feeds. Saturates to 0 / 1 for large |x|.
__device__ __forceinline__ float sigmoidf(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// The decay gate g = -exp(A_log) softplus(a + dt_bias) (layers/cyfa.py:323), of
// x = a + dt_bias; softplus switches to the identity above 20 as F.softplus does.
__device__ __forceinline__ float decay_gate(float x, float A_log) {
    const float sp = x > 20.f ? x : log1pf(expf(x));
    return -expf(A_log) * sp;
}

// Wave reductions on the VALU. __shfl_xor is a ds_bpermute, an LDS round trip
// per step (about 30 of them sat on the decode step's serial path): here DPP
// moves reduce within rows of 16 lanes and v_readlane gathers the rows.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_value(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Sum (max) over aligned groups of W lanes, in every lane of the group; every
// lane of the wave must be active. Fixed order: pairs (quad_perm [1,0,3,2]),
// quads ([2,3,0,1]), octets (row_half_mirror), rows of 16 (row_mirror) - after
// each step every lane of a group holds the same value, so a mirror reads the
// value the matching xor lane holds - then rows (0 + 1) and (2 + 3), then
// their sum.
template <int W = 64>
__device__ __forceinline__ float wave_sum(float x) {
    static_assert(W == 16 || W == 32 || W == 64, "group of 16, 32 or 64 lanes");
    x += dpp_mov<0xB1>(x);
    x += dpp_mov<0x4E>(x);
    x += dpp_mov<0x141>(x);
    x += dpp_mov<0x140>(x);
    if (W == 16) return x;
    const float lo = lane_value(x, 0) + lane_value(x, 16), hi = lane_value(x, 32) + lane_value(x, 48);
    if (W == 32) return (threadIdx.x & 32) ? hi : lo;
    return lo + hi;
}

template <int W = 64>
__device__ __forceinline__ float wave_max(float x) {
    static_assert(W == 16 || W == 32 || W == 64, "group of 16, 32 or 64 lanes");
    x = fmaxf(x, dpp_mov<0xB1>(x));
    x = fmaxf(x, dpp_mov<0x4E>(x));
    x = fmaxf(x, dpp_mov<0x141>(x));
    x = fmaxf(x, dpp_mov<0x140>(x));
    if (W == 16) return x;
    const float lo = fmaxf(lane_value(x, 0), lane_value(x, 16)), hi = fmaxf(lane_value(x, 32), lane_value(x, 48));
    if (W == 32) return (threadIdx.x & 32) ? hi : lo;
    return fmaxf(lo, hi);
}

}  // namespace cyfa
