// cyfa_prefill.hip -- chunkwise two-pass CyFA prefill for gfx950 (K = V = 256, M = 128).
//
// Pipeline for one call (all kernels on the caller's stream):
//   1. segment_state    the clock lam_t = clock0 + sum_{s<=t} delta_s and the
//                       in-chunk decay scan of every token, the final clock,
//                       and (when a sequence is split into P > 1 segments)
//                       the segment-local end states E_j of both passes from
//                       a zero start and the product a_j of alpha over each
//                       segment.
//   2. pass1_kernel     per segment: start from the carried state
//                       S_j = sum_{i<j} (prod_{i<l<j} a_l) E_i + (prod_{l<j} a_l) h0,
//                       then sweep the segment's 64-token chunks with the
//                       fp32 key state [256 x 128] held in registers; each
//                       chunk's pass-1 output (2^G q S + P w per 128-wide key
//                       half, bf16) goes through LDS into the slot readout
//                       z = U(lam) raw; p = softmax(table z); u = table^T p;
//                       slot weights bf16(U(-lam) u) (ops/chunk_readout.py:797-909),
//                       which are written for pass 2.
//   3. pass2_kernel     per segment: the same carry and sweep for the value state
//                       [128 x 256] with query = slot weights, key = w,
//                       value = v -> o (bf16).
// The pass-1 output is formed as two 128-wide key slices, each scaled and
// rounded to bf16, and summed, as the reference does (ops/chunk_o.py:240-250,
// 369-374). A sweep workgroup has 8 waves, one per 32 state columns of a
// 128-row half (pass 1) or per 32 value columns (pass 2); each wave holds its
// 128 x 32 block of the fp32 state (64 registers per lane) from the first to
// the last chunk of the segment. Each 64-token chunk is loaded from HBM once,
// normalised once and staged once in LDS, token-major; every fragment a wave
// reads from LDS feeds two MFMAs (its two 16-column blocks). All GEMM-shaped
// work runs on v_mfma_f32_16x16x32_{bf16,f16} with fp32 accumulation, and
// operands that contract over tokens use the gfx950 LDS transpose read. Only
// segment boundary states (one per L chunks) touch HBM.
//
// Lane conventions of the 16x16x32 MFMA (wave64, lane l, lr = l & 15, lg = l >> 4):
//   A[row][k]: row = lr, k = 8 lg + j (j = 0..7)     B[k][col]: col = lr, k = 8 lg + j
//   C[row][col]: col = lr, row = 4 lg + i (i = 0..3)
// A pair of state blocks held as C (rows 32 ks .. 32 ks + 31) serves directly as
// the A operand of a product that contracts over those rows, with element j < 4
// taken from row 32 ks + 4 lg + j and j >= 4 from row 32 ks + 16 + 4 lg + (j - 4);
// the other operand is read in the same k order. The sweeps compute their
// outputs transposed (output coordinate = C row, token = C column), so each lane
// ends with four consecutive output coordinates of one token.
#include <stdlib.h>

#include <type_traits>

#include "cyfa_device.h"
#include "cyfa_internal.h"

namespace cyfa {

namespace {

constexpr int KD = 256;             // key / query dim of pass 1
constexpr int VD = 256;             // value dim of pass 2
constexpr int HALF = 128;           // key / value columns per sweep workgroup
constexpr int SEG_K = KD * kSlots;  // key-state elements
constexpr int SEG_V = kSlots * VD;  // value-state elements
constexpr int SEG = SEG_K + SEG_V;

// LDS tile layouts. Element (r, e) of a tile sits at Tile<LD, XA>::off(r, e):
// rows LD elements apart, and in rows with bit 3 set the 16-byte unit index
// e >> 3 is XORed with XA. The layouts were chosen by measuring
// SQ_LDS_BANK_CONFLICT on gfx950 for each access pattern of the sweeps:
//   padded rows (LD = 256 + 16, 128 + 16)  row reads and staging stores
//                                          conflict-free; transpose reads 2-way
//   LD = 256 + 32 / 128 + 32 with XA = 2   row reads, transpose reads and
//                                          staging stores conflict-free
template <int LD, int XA>
struct Tile {
    static constexpr int ld = LD;
    static constexpr int bytes = 64 * LD * 2;  // 64 rows of 16-bit elements
    static_assert(XA < 4, "the XOR stays inside a 32-element block");
    // The XOR only touches the unit index within a 32-element block, so
    // whole blocks (e & ~31) add as plain offsets.
    __device__ static __forceinline__ int off(int r, int e) {
        return r * LD + (e & ~31) + (((((e & 31) >> 3) ^ (XA * ((r >> 3) & 1)))) << 3) + (e & 7);
    }
};
using TileQ = Tile<256 + 16, 0>;  // q_hat: row reads only
using TileF = Tile<256 + 32, 2>;  // k_hat, v: row and transpose reads
using TileW = Tile<128 + 32, 2>;  // w: row and transpose reads
using TileO = Tile<128 + 16, 0>;  // slot weights: row reads only
using TileP = Tile<64 + 8, 2>;    // 64 x 64 masked scores
constexpr int RS = 128 + 16;      // readout table rows
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ size_t tok_index(const PrefillParams& p, int b, int t, int h) {
    return ((size_t)b * p.T + t) * p.H + h;
}

// Keeps the scheduler from hoisting the LDS fragment loads of later MFMA steps
// above this point (which would raise register pressure past the 128-register
// budget of two workgroups per CU).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Sweep and segment-state grids are (H, B, segments): the coordinates come
// straight from the block ids. (A quotient such as blockIdx.x / P is formed in
// vector registers, and the buffer resources derived from it would then be
// wrapped in a waterfall loop at every access.)
struct SegCoord {
    int bh, j, b, h;
};

__device__ __forceinline__ SegCoord seg_coord(int H, int j) {
    const int b = blockIdx.y, h = blockIdx.x;
    return {b * H + h, j, b, h};
}

// Global memory in the sweeps goes through buffer instructions: a 128-bit
// resource per stream in scalar registers and one 32-bit byte offset per lane,
// which keeps the address arithmetic out of the vector register budget.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, size_t bytes) {
    const uint32_t n = bytes > 0xffffffffull ? 0xffffffffu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ bf16x8 ld_b128(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float ld_f32(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ bf16x4 ld_b64(rsrc_t r, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(r, off, soff, 0));
}

__device__ __forceinline__ void st_b64(rsrc_t r, uint32_t off, uint32_t soff, bf16x4 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, soff, 0);
}

// The streams of one (batch, head) sequence: q, k, v, o rows of 512 bytes
// H * 512 bytes apart, beta H * 4 bytes apart, the per-token reduced clock
// and decay scan of the workspace contiguous.
struct Seq {
    rsrc_t q, k, v, o, beta, delta, g, lam, gam;
    uint32_t row16, row4;
};

// The 256-wide rows (b, t, h), t < T, of a [B, T, H, 256] bf16 tensor, row t at byte t * H * 512.
__device__ __forceinline__ rsrc_t rows_rsrc(const PrefillParams& p, int b, int h, const bf16_t* x) {
    const size_t first = (size_t)b * p.T * p.H + h;     // token row of (b, 0, h)
    const size_t span = ((size_t)(p.T - 1) * p.H + 1);  // rows up to (b, T - 1, h)
    return make_rsrc(x + first * 256, span * 256 * 2);
}

__device__ __forceinline__ Seq make_seq(const PrefillParams& p, int b, int h, int bh) {
    const size_t first = (size_t)b * p.T * p.H + h;
    const size_t span = ((size_t)(p.T - 1) * p.H + 1);
    Seq s;
    s.q = rows_rsrc(p, b, h, p.q);
    s.k = rows_rsrc(p, b, h, p.k);
    s.v = rows_rsrc(p, b, h, p.v);
    s.o = rows_rsrc(p, b, h, p.o);
    s.beta = make_rsrc(p.beta + first, span * 4);
    s.delta = make_rsrc(p.delta + first, span * 4);
    s.g = make_rsrc(p.g + first, span * 4);
    s.lam = make_rsrc(p.lam + (size_t)bh * p.Tp, (size_t)p.Tp * 4);
    s.gam = make_rsrc(p.gam + (size_t)bh * p.Tp, (size_t)p.Tp * 4);
    s.row16 = (uint32_t)p.H * KD * 2;
    s.row4 = (uint32_t)p.H * 4;
    return s;
}

// Segment states in the workspace are kept in the register order of the
// sweeps: the eight values that lane `lane` of wave w holds as accumulator
// blocks (x, 0) and (x, 1) sit at element offset frag_offset(w, x, lane) (16
// bytes per lane), so a wave loads or stores a block pair as one contiguous
// 1 KiB run. Element 4 c + i of the run holds (see load_tr_perm for the row
// order)
//   key state   S[128 (w >> 2) + state_row(x, lg, i)][32 (w & 3) + 16 c + lr]
//   value state S[state_row(x, lg, i)][32 w + 16 c + lr].
// The key state fills [0, SEG_K), the value state [SEG_K, SEG).
__host__ __device__ constexpr int frag_offset(int w, int x, int lane) { return ((w * 8 + x) * 64 + lane) * 8; }

// Row (within a 128-row half) of element i of state block x in a lane of row
// group lg.
__host__ __device__ constexpr int state_row(int x, int lg, int i) { return 32 * (x >> 1) + 8 * lg + 4 * (x & 1) + i; }

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over the 8 lanes of an aligned octet: quad_perm [1,0,3,2], [2,3,0,1],
// then row_half_mirror (lane i of the octet reads lane 7 - i).
__device__ __forceinline__ float octet_sum(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    return x;
}

// Chunk gates, loaded by every wave with lane = token (issue) and staged in
// LDS by wave 0 (commit). The clock kernel has already formed the reduced
// clock lamr_t and the in-chunk decay scan G_t (log2 units, ops/utils.py:495-520).
// LDS per token: sLam = lamr, sBeta, sGam = G_t, sGam[64 + t] = 2^G_t,
// sGam[128 + t] = 2^(G_last - G_t).
struct GateRegs {
    float beta, lamr, gam;
};

__device__ __forceinline__ GateRegs issue_gates(const Seq& sq, int T, int t0) {
    const int t = t0 + (threadIdx.x & 63);
    GateRegs r;
    r.beta = ld_f32(sq.beta, (uint32_t)(t < T ? t : T - 1) * sq.row4);
    r.lamr = ld_f32(sq.lam, (uint32_t)t * 4);
    r.gam = ld_f32(sq.gam, (uint32_t)t * 4);
    return r;
}

__device__ __forceinline__ float chunk_last_gam(const GateRegs& r) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, r.gam), 63));
}

// inv: 1 / sigma of the state after this chunk's update (see StateScale).
// Written by the wave whose index is `leader`.
__device__ __forceinline__ void commit_gates(int T, int t0, const GateRegs& r, float* sLam, float* sBeta, float* sGam,
                                             float inv, int leader = 0) {
    const int lane = threadIdx.x & 63;
    if (wave_id() == leader) {
        const float last = chunk_last_gam(r);
        sGam[lane] = r.gam;
        sBeta[lane] = t0 + lane < T ? r.beta : 0.f;
        sLam[lane] = r.lamr;
        sGam[64 + lane] = fast_exp2(r.gam);                // 2^G_t
        sGam[128 + lane] = fast_exp2(last - r.gam) * inv;  // 2^(G_last - G_t) / sigma'
    }
}

// The sweeps hold the fp32 state as S = sigma * acc with sigma uniform over the
// workgroup. The chunk update S' = 2^G_last S + A^T bf16(2^(G_last - G_s) B)
// becomes acc' = acc + A^T bf16(2^(G_last - G_s) / sigma' B) with
// sigma' = 2^G_last sigma: the decay costs one scalar product per chunk instead
// of a multiply per accumulator, and sigma folds into the per-token factors
// that already scale the update's values and the inter-chunk output. When
// sigma' would fall below 2^-64 it is multiplied into acc instead and reset to
// 1 (so |acc| stays within 2^64 |S|).
struct StateScale {
    float sig = 1.f;   // sigma of the state the chunk starts from
    float next = 1.f;  // sigma after the chunk's update
    float fold = 1.f;  // multiplied into acc before the update (1 unless renormalising)
    __device__ __forceinline__ void begin_chunk(float last_gam) {
        const float s = sig * fast_exp2(last_gam);
        const bool renorm = s < 0x1p-64f;
        fold = renorm ? s : 1.f;
        next = renorm ? 1.f : s;
    }
    __device__ __forceinline__ float inv() const { return 1.f / next; }
};

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

__device__ __forceinline__ s16x8 tr_pair(const short* p, int ld) {
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p)));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p + 4 * ld)));
    s16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

// s0 is a multiple of 8, so rows r and r + 4 of a lane share the XOR of r >> 3.
template <class L>
__device__ __forceinline__ bf16x8 load_tr(const bf16_t* X, int s0, int c0) {
    const int l = threadIdx.x & 63, g = l >> 4, i = l & 15;
    const short* p = reinterpret_cast<const short*>(X) + L::off(s0 + 8 * g + (i >> 2), c0 + 4 * (i & 3));
    return __builtin_bit_cast(bf16x8, tr_pair(p, L::ld));
}

// The same read with the columns of a 32-column block taken in the order
//   lane (lr, lg) element j = X[s0 + 8 lg + j][c0 + 8 (lr >> 2) + 4 h + (lr & 3)]
// (c0 a multiple of 32, h = 0, 1). As the A operand of the state update it
// leaves the C rows 4 lg + i of state block 2 b + h holding key (or slot)
// index 32 b + 8 lg + 4 h + i, so that a C-block pair is the A operand of the
// product over those indices in their natural order: element j of lane lg is
// index 32 b + 8 lg + j, and the other operand is a plain row fragment.
template <class L>
__device__ __forceinline__ bf16x8 load_tr_perm(const bf16_t* X, int s0, int c0, int h) {
    const int l = threadIdx.x & 63, g = l >> 4, i = l & 15;
    const short* p = reinterpret_cast<const short*>(X) + L::off(s0 + 8 * g + (i >> 2), c0 + 8 * (i & 3) + 4 * h);
    return __builtin_bit_cast(bf16x8, tr_pair(p, L::ld));
}

// Transpose read of a row-major f16 tile with the rows of a 32-row block taken
// in the k order of a C-block pair:
//   lane (lr, lg) element j = X[r0 + 4 lg + j][c0 + lr]             (j < 4)
//                             X[r0 + 16 + 4 lg + (j - 4)][c0 + lr]  (j >= 4)
// i.e. the A operand A[row = c0 + lr][k] of a product whose other operand is a
// C-block pair (rows r0 .. r0 + 31) used directly as the B operand.
__device__ __forceinline__ f16x8 load_tr_pair_f16(const f16_t* X, int ld, int r0, int c0) {
    const int l = threadIdx.x & 63, g = l >> 4, i = l & 15;
    const short* p = reinterpret_cast<const short*>(X) + (r0 + 4 * g + (i >> 2)) * ld + c0 + 4 * (i & 3);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p)));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(const_cast<short*>(p + 16 * ld)));
    s16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return __builtin_bit_cast(f16x8, r);
}

// Row fragment: lane (lr, lg) gets X[r0 + lr][k0 + 8 lg .. + 8] (A operand, or
// B operand of a product that contracts over X's columns); k0 a multiple of 8.
template <class L, typename V8 = bf16x8, typename T>
__device__ __forceinline__ V8 load_row(const T* X, int r0, int k0) {
    const int l = threadIdx.x & 63;
    return *reinterpret_cast<const V8*>(X + L::off(r0 + (l & 15), k0 + 8 * (l >> 4)));
}

template <typename V8, typename T>
__device__ __forceinline__ V8 load_row_ld(const T* X, int ld, int r0, int k0) {
    const int l = threadIdx.x & 63;
    return *reinterpret_cast<const V8*>(X + (r0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// Full 256-wide rows [t0, t0 + 64) of a [B, T, H, 256] bf16 tensor for a
// 512-thread block: thread tid holds row tid >> 3, columns 64 q + 8 c .. + 8 in
// raw[q] (q = 0..3, c = tid & 7). Rows past T are clamped to T - 1 (zeroed when
// stored).
__device__ __forceinline__ void issue_rows_stride(rsrc_t x, uint32_t row_bytes, int T, int t0, bf16x8 raw[4]) {
    const int t = t0 + (threadIdx.x >> 3);
    const uint32_t off = (uint32_t)(t < T ? t : T - 1) * row_bytes + 16 * (threadIdx.x & 7);
#pragma unroll
    for (int q = 0; q < 4; q++) raw[q] = ld_b128(x, off + 128 * q);
}

__device__ __forceinline__ void issue_rows(const Seq& sq, rsrc_t x, int T, int t0, bf16x8 raw[4]) {
    issue_rows_stride(x, sq.row16, T, t0, raw);
}

// x_hat = bf16(x rsqrt(mean x^2 + eps) w) over the full row (ops/qk_norm.py:64-107,
// 206-233), stored into the tile dst (zero past T). wn is the norm weight in
// LDS. The sum of squares uses the bf16 dot product (two elements per
// instruction, fp32 accumulation) and the 8 threads of a row meet by DPP.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <class L>
__device__ __forceinline__ void norm_store_rows(const PrefillParams& p, int t0, const bf16x8 raw[4], const float* wn,
                                                float eps, bf16_t* dst) {
    const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bf16x2 x2 = {raw[q][2 * j], raw[q][2 * j + 1]};
            ss = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, ss, false);
        }
    float4 wq[4][2];  // all weight reads in flight at once
#pragma unroll
    for (int q = 0; q < 4; q++) {
        wq[q][0] = *reinterpret_cast<const float4*>(wn + 64 * q + 8 * c);
        wq[q][1] = *reinterpret_cast<const float4*>(wn + 64 * q + 8 * c + 4);
    }
    ss = octet_sum(ss);
    const float rs = t0 + r < p.T ? rsqrtf(ss * (1.f / KD) + eps) : 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float wv[8] = {wq[q][0].x, wq[q][0].y, wq[q][0].z, wq[q][0].w,
                             wq[q][1].x, wq[q][1].y, wq[q][1].z, wq[q][1].w};
        bf16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = (bf16_t)((float)raw[q][j] * (rs * wv[j]));
        *reinterpret_cast<bf16x8*>(dst + L::off(r, 64 * q + 8 * c)) = o;
    }
}

// Store 64 x 256 rows held with the issue_rows mapping into the tile dst; rows
// at or past `valid` are zeroed.
template <class L>
__device__ __forceinline__ void store_rows(const bf16x8 raw[4], int valid, bf16_t* dst) {
    const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        bf16x8 o = raw[q];
        if (r >= valid) {
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = (bf16_t)0.f;
        }
        *reinterpret_cast<bf16x8*>(dst + L::off(r, 64 * q + 8 * c)) = o;
    }
}

// The same rows for a 256-thread group: thread u (0..255) holds row u >> 2,
// columns 64 (u & 3) + 8 j .. + 8 in raw[j] (j = 0..7).
__device__ __forceinline__ void issue_rows_q(const Seq& sq, rsrc_t x, int T, int t0, int u, bf16x8 raw[8]) {
    const int t = t0 + (u >> 2);
    const uint32_t off = (uint32_t)(t < T ? t : T - 1) * sq.row16 + 128 * (u & 3);
#pragma unroll
    for (int j = 0; j < 8; j++) raw[j] = ld_b128(x, off + 16 * j);
}

// norm_store_rows for that mapping (the 4 threads of a row meet by DPP).
template <class L>
__device__ __forceinline__ void norm_store_rows_q(const PrefillParams& p, int t0, int u, const bf16x8 raw[8],
                                                  const float* wn, float eps, bf16_t* dst) {
    const int r = u >> 2, c0 = 64 * (u & 3);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const bf16x2 x2 = {raw[j][2 * e], raw[j][2 * e + 1]};
            ss = __builtin_amdgcn_fdot2_f32_bf16(x2, x2, ss, false);
        }
    ss += dpp<0xB1>(ss);
    ss += dpp<0x4E>(ss);
    const float rs = t0 + r < p.T ? rsqrtf(ss * (1.f / KD) + eps) : 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++) {  // weights read four groups at a time
        float4 wq[4][2];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            wq[j][0] = *reinterpret_cast<const float4*>(wn + c0 + 32 * h + 8 * j);
            wq[j][1] = *reinterpret_cast<const float4*>(wn + c0 + 32 * h + 8 * j + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float wv[8] = {wq[j][0].x, wq[j][0].y, wq[j][0].z, wq[j][0].w,
                                 wq[j][1].x, wq[j][1].y, wq[j][1].z, wq[j][1].w};
            bf16x8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = (bf16_t)((float)raw[4 * h + j][e] * (rs * wv[e]));
            *reinterpret_cast<bf16x8*>(dst + L::off(r, c0 + 32 * h + 8 * j)) = o;
        }
    }
}

// 128-wide rows [t0, t0 + 64) (row r at byte r * row_bytes): thread tid holds
// row tid >> 3, columns 8 c + 64 it .. + 8 in raw[it] (c = tid & 7).
__device__ __forceinline__ void issue_half_rows(rsrc_t x, uint32_t row_bytes, int t0, bf16x8 raw[2]) {
    const uint32_t off = (uint32_t)(t0 + (threadIdx.x >> 3)) * row_bytes + 16 * (threadIdx.x & 7);
#pragma unroll
    for (int it = 0; it < 2; it++) raw[it] = ld_b128(x, off + 128 * it);
}

// Slot-weight rows of the readout output (256-byte rows).
__device__ __forceinline__ void issue_omega(rsrc_t om_rows, int t0, bf16x8 om[2]) {
    issue_half_rows(om_rows, kSlots * 2, t0, om);
}

// Store 64 x 128 rows held with that mapping into the tile dst (layout L);
// rows at or past `valid` are zeroed.
template <class L = TileO>
__device__ __forceinline__ void store_half_rows(const bf16x8 raw[2], int valid, bf16_t* dst) {
    const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
#pragma unroll
    for (int it = 0; it < 2; it++) {
        bf16x8 o = raw[it];
        if (r >= valid) {
#pragma unroll
            for (int j = 0; j < 8; j++) o[j] = (bf16_t)0.f;
        }
        *reinterpret_cast<bf16x8*>(dst + L::off(r, 8 * c + 64 * it)) = o;
    }
}

// Write vector of the chunk, w [64 tokens][128] bf16 row-major (ops/utils.py:664-702),
// from the gate registers: lane = token, wave w covers pairs 8 w .. 8 w + 7.
// The hardware gives (cos, sin) of pair 8 w and of pair 1; the next pairs
// follow by complex multiplication, i.e. rotation by theta (seven steps add
// about 1e-6 to a result rounded to bf16).
// NW waves share the tile (wave g of the group covers pairs 64 / NW g ..).
template <class L, int NW = 8>
__device__ __forceinline__ void store_write_tile(const GateRegs& gr, int valid, bf16_t* dst, int g) {
    constexpr int NP = 64 / NW;  // pairs per wave
    const int lane = threadIdx.x & 63;
    const float beta = lane < valid ? gr.beta : 0.f;
    float s1, c1, sn, cs;
    pair_sincos(gr.lamr, 1, s1, c1);
    pair_sincos(gr.lamr, NP * g, sn, cs);
#pragma unroll
    for (int h = 0; h < NP / 8; h++) {
        bf16x8 o[2];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const float a = beta * pair_scale(NP * g + 8 * h + q);
            o[q >> 2][2 * (q & 3)] = (bf16_t)(a * cs);
            o[q >> 2][2 * (q & 3) + 1] = (bf16_t)(-a * sn);
            const float cn = cs * c1 - sn * s1;
            sn = sn * c1 + cs * s1;
            cs = cn;
        }
        *reinterpret_cast<bf16x8*>(dst + L::off(lane, 2 * NP * g + 16 * h)) = o[0];
        *reinterpret_cast<bf16x8*>(dst + L::off(lane, 2 * NP * g + 16 * h + 8)) = o[1];
    }
}

template <class L>
__device__ __forceinline__ void store_write_tile(const GateRegs& gr, int valid, bf16_t* dst) {
    store_write_tile<L, 8>(gr, valid, dst, wave_id());
}

// The 10 causal 16 x 16 score blocks (query block tb >= key block sb): wave w
// takes blocks w and w + 8.
__device__ __forceinline__ void score_block(int blk, int& tb, int& sb) {
    tb = blk < 1 ? 0 : blk < 3 ? 1 : blk < 6 ? 2 : 3;
    sb = blk - tb * (tb + 1) / 2;
}

// Block blk (query block tb >= key block sb) of the masked, decayed scores of
// a query tile X and key tile Y (columns xc / yc onward, 128-wide
// contraction), into the TileP tile sP:
// P[t][s] = bf16(2^(G_t - G_s) c x_t . y_s) for s <= t, else 0 (ops/chunk_o.py:240-250),
// c = 2^log2_scale the output scale of the pass (exact for the default
// scale 1/16: scaling a bf16 value by a power of two commutes with rounding).
// The block is computed transposed (C rows = keys, columns = queries), so a
// lane holds four consecutive keys of one query and writes them in one store.
template <class LX, class LY>
__device__ __forceinline__ void score_tile(const bf16_t* X, int xc, const bf16_t* Y, int yc, int blk, const float* sGam,
                                           float log2_scale, bf16_t* sP) {
    const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
    int tb, sb;
    score_block(blk, tb, sb);
    bf16x8 a[4], b[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        a[ks] = load_row<LY>(Y, 16 * sb, yc + 32 * ks);
        b[ks] = load_row<LX>(X, 16 * tb, xc + 32 * ks);
    }
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ks++) sc = mfma_bf16(a[ks], b[ks], sc);
    const int t = 16 * tb + lr, s0 = 16 * sb + 4 * lg;
    const float gt = sGam[t] + log2_scale;
    const float4 gs = *reinterpret_cast<const float4*>(sGam + s0);
    const float gsv[4] = {gs.x, gs.y, gs.z, gs.w};
    bf16x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float v = sc[i] * fast_exp2(gt - gsv[i]);
        o[i] = (bf16_t)(s0 + i <= t ? v : 0.f);
    }
    *reinterpret_cast<bf16x4*>(sP + TileP::off(t, s0)) = o;
}

__device__ __forceinline__ void zero_scores(bf16_t* sP, int tiles) {
    for (int idx = threadIdx.x; idx < tiles * TileP::bytes / 4; idx += blockDim.x) reinterpret_cast<uint32_t*>(sP)[idx] = 0u;
}

// A C-block pair of the fp32 state as a bf16 operand (the reference emits the
// per-chunk states in bf16, ops/chunk_h.py:238-327).
__device__ __forceinline__ bf16x8 state_frag(const f32x4& top, const f32x4& bottom) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        r[i] = (bf16_t)top[i];
        r[4 + i] = (bf16_t)bottom[i];
    }
    return r;
}

__device__ __forceinline__ bf16x4 to_bf16x4(const f32x4& x, float s) {
    return bf16x4{(bf16_t)(x[0] * s), (bf16_t)(x[1] * s), (bf16_t)(x[2] * s), (bf16_t)(x[3] * s)};
}

// ---------------------------------------------------------------------------
// Clock and in-chunk decay scan (ops/utils.py:229-348, 495-520):
//   lam[t] = reduced_clock(clock0 + sum_{s<=t} delta_s)
//   gam[t] = log2(e) sum_{chunk start <= s <= t} g_s
// They are formed inside segment_state: every workgroup starts from the
// clock before its first chunk (a double sum over the earlier tokens) and
// carries it in double from chunk to chunk; the state workgroups scan each
// chunk with lane = token, and one extra workgroup per sequence covers the
// last segment (all of the sequence when P = 1) and writes the final clock.
template <int CTRL>
__device__ __forceinline__ float dpp_shift(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// clock0 + sum_{s < t_end} delta_s, summed in double by the workgroup (512
// threads) in a fixed order, so every workgroup of a sequence gets the same bits.
// clock0 + sum of delta over tokens [0, t_end) of sequence sq, in double:
// each thread adds tokens tid, tid + 512, .. in order, then the wave and
// workgroup sums. The first four tokens' loads per thread go out before
// issue_after(), the caller's own loads, so the sum does not wait for those
// (vector loads complete in issue order); tokens past t_end load zero.
template <typename F>
__device__ __forceinline__ double clock_before(const PrefillParams& p, const Seq& sq, int bh, int t_end,
                                               F&& issue_after) {
    __shared__ double part[8];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int te = min(t_end, p.T);
    float d[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int t = tid + 512 * k;
        d[k] = ld_f32(sq.delta, ((uint32_t)t * sq.row4) | ((uint32_t)((t - te) >> 31 ^ -1) & 0x80000000u));
    }
    issue_after();
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < 4; k++) acc += (double)d[k];  // zero past te
    for (int t = tid + 2048; t < te; t += 512) acc += (double)ld_f32(sq.delta, (uint32_t)t * sq.row4);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) part[w] = acc;
    __syncthreads();
    double tot = p.clock0 ? (double)p.clock0[bh] : 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) tot += part[i];
    __syncthreads();
    return tot;
}

// Raw gate inputs of one chunk, lane = token (loads only; see finish_gates).
struct GateIn {
    float d, g, beta;
};

__device__ __forceinline__ GateIn load_gate_inputs(const Seq& sq, int T, int t0) {
    const int t = t0 + (threadIdx.x & 63);
    const uint32_t off = (uint32_t)(t < T ? t : T - 1) * sq.row4;
    GateIn r;
    r.d = t < T ? ld_f32(sq.delta, off) : 0.f;
    r.g = t < T ? ld_f32(sq.g, off) : 0.f;
    r.beta = ld_f32(sq.beta, off);
    return r;
}

// Inclusive scan over the 64 lanes of a wave by DPP: row_shr 1, 2, 4, 8 within
// each 16-lane row, then row_bcast 15 (rows 1, 3) and row_bcast 31 (rows 2, 3).
__device__ __forceinline__ float wave_scan(float x) {
    x += dpp_shift<0x111>(x);
    x += dpp_shift<0x112>(x);
    x += dpp_shift<0x114>(x);
    x += dpp_shift<0x118>(x);
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x142, 0xA, 0xF, false));
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x143, 0xC, 0xF, false));
    return x;
}

// Inclusive scans over the chunk's 64 lanes; clock advances by the chunk's sum of delta.
__device__ __forceinline__ GateRegs finish_gates(const GateIn& r, double& clock) {
    const float sd = wave_scan(r.d), sg = wave_scan(r.g);
    GateRegs out;
    out.beta = r.beta;
    out.lamr = reduced_clock((float)(clock + (double)sd));
    out.gam = sg * kLog2e;
    clock += (double)__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sd), 63));
    return out;
}

// The clock of tokens [t_begin, Tp) from the clock `carry` before t_begin
// (t_begin a multiple of 64), 2048 tokens per step, four consecutive tokens
// per thread; writes lam / gam and the final clock. The 16 threads of a
// 64-token chunk form one DPP row.
__device__ __forceinline__ void clock_scan(const PrefillParams& p, int bh, int b, int h, int t_begin, double carry) {
    constexpr int NW = 8;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ float s_tot[NW];
    for (int t0 = t_begin; t0 < p.Tp; t0 += 4 * 512) {
        float d[4], gg[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = t0 + 4 * tid + j;
            const bool valid = t < p.T;
            d[j] = valid ? p.delta[tok_index(p, b, t, h)] : 0.f;
            gg[j] = valid ? p.g[tok_index(p, b, t, h)] : 0.f;
        }
        const float s1 = d[0] + d[1], s2 = s1 + d[2], s3 = s2 + d[3];
        const float pre[4] = {d[0], s1, s2, s3};
        float x = s3;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        // in-chunk inclusive scan of g over the row's 16 threads (row_shr 1, 2, 4, 8)
        const float g1 = gg[0] + gg[1], g2 = g1 + gg[2], g3 = g2 + gg[3];
        float xs = g3;
        xs += dpp_shift<0x111>(xs);
        xs += dpp_shift<0x112>(xs);
        xs += dpp_shift<0x114>(xs);
        xs += dpp_shift<0x118>(xs);
        const float gex = xs - g3;
        const float gpre[4] = {gg[0], g1, g2, g3};
        if (lane == 63) s_tot[wave] = x;
        __syncthreads();
        float before = 0.f, tile = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            before += w < wave ? s_tot[w] : 0.f;
            tile += s_tot[w];
        }
        const float excl = before + x - s3;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int t = t0 + 4 * tid + j;
            if (t < p.Tp) {
                p.lam[(size_t)bh * p.Tp + t] = reduced_clock((float)(carry + (double)(excl + pre[j])));
                p.gam[(size_t)bh * p.Tp + t] = (gex + gpre[j]) * kLog2e;
            }
        }
        carry += (double)tile;
        __syncthreads();
    }
    if (p.clock && tid == 0) p.clock[bh] = (float)carry;
}

// One chunk's update of a segment sweep's state block: acc += A^T bf16(2^(G_last
// - G_s) / sigma' B) for the 64 tokens staged in LDS (A rows from column a_col
// of tile sArow, B columns from column b_col of tile sBcol, both token-major;
// sGam[128 + s] = 2^(G_last - G_s) / sigma').
// bt[c][jj] = B[32 ss + 8 lg + jj][b_col + 16 c + lr], scaled.
template <class LA, class LB>
__device__ __forceinline__ void chunk_state_update(const bf16_t* sArow, int a_col, const bf16_t* sBcol, int b_col,
                                                   const float* sGam, f32x4 acc[8][2]) {
    const int lg = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int ss = 0; ss < 2; ss++) {
        bf16x8 bt[2];
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const bf16x8 f = load_tr<LB>(sBcol, 32 * ss, b_col + 16 * c);
#pragma unroll
            for (int jj = 0; jj < 8; jj++) bt[c][jj] = (bf16_t)((float)f[jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
        }
        sched_fence();
#pragma unroll
        for (int x = 0; x < 8; x++) {
            const bf16x8 af = load_tr_perm<LA>(sArow, 32 * ss, a_col + 32 * (x >> 1), x & 1);
            acc[x][0] = mfma_bf16(af, bt[0], acc[x][0]);
            acc[x][1] = mfma_bf16(af, bt[1], acc[x][1]);
            if (x & 1) sched_fence();
        }
    }
}

// Segment-local end state E = sigma acc of this wave's block, in fp16 at
// out + frag_offset(w, .., lane), scaled by 2^-e so that the wave's largest |E|
// is below 2^15 (fp16 keeps 11 bits, four times finer than the bf16 rounding
// the state gets before each inter-chunk product); e goes to exp_out[w].
__device__ __forceinline__ void store_segment_state(const f32x4 acc[8][2], float sig, _Float16* out, int* exp_out) {
    const int lane = threadIdx.x & 63, w = wave_id();
    float m = 0.f;
#pragma unroll
    for (int x = 0; x < 8; x++)
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) m = fmaxf(m, fabsf(acc[x][c][i]));
    m = wave_max(m) * sig;
    int e = 0;
    if (m > 0.f && m < INFINITY) {
        frexpf(m, &e);  // m < 2^e
        e -= 15;
    }
    const float f = ldexpf(sig, -e);
#pragma unroll
    for (int x = 0; x < 8; x++) {
        f16x8 v;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) v[4 * c + i] = (f16_t)(acc[x][c][i] * f);
        *reinterpret_cast<f16x8*>(out + frag_offset(w, x, lane)) = v;
    }
    if (lane == 0) exp_out[w] = e;
}

// ---------------------------------------------------------------------------
// 1. Segment-local end states from a zero start, both parts in one workgroup:
// the gates, the clock and the write-vector tile are formed once for the key
// state S_K += k_hat^T w' and the value state S_V += w^T v'. grid = (H, B, P),
// 512 threads (blockIdx.z: see segment_state_kernel); state blocks as in
// frag_offset: key state rows 128 y .., y = w >> 2, columns 32 (w & 3) ..;
// value state columns 32 w ...
constexpr int SG_K = 0;                     // k_hat, TileF
constexpr int SG_V = SG_K + TileF::bytes;  // v, TileF
constexpr int SG_W = SG_V + TileF::bytes;  // w, TileW
constexpr int SG_G = SG_W + TileW::bytes;  // f32 [5][64] gates
constexpr int SG_NW = SG_G + 5 * 64 * 4;   // f32 [256] k norm weight
constexpr int SG_LDS = SG_NW + KD * 4;
static_assert(SG_LDS <= 160 * 1024, "segment-state workgroup must fit in one CU's LDS");

__device__ __forceinline__ void segment_state_body(const PrefillParams& p, int bh, int j, int b, int h,
                                                   unsigned char* smem) {
    bf16_t* sK = reinterpret_cast<bf16_t*>(smem + SG_K);
    bf16_t* sV = reinterpret_cast<bf16_t*>(smem + SG_V);
    bf16_t* sW = reinterpret_cast<bf16_t*>(smem + SG_W);
    float* sLam = reinterpret_cast<float*>(smem + SG_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    float* sNw = reinterpret_cast<float*>(smem + SG_NW);
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    f32x4 acck[8][2], accv[8][2];
#pragma unroll
    for (int x = 0; x < 8; x++) acck[x][0] = acck[x][1] = accv[x][0] = accv[x][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const Seq sq = make_seq(p, b, h, bh);
    GateIn gin;
    bf16x8 kraw[4], vraw[4];
    float kwv;
    // the clock prefix's loads first, then the first chunk's (see clock_before)
    double clock = clock_before(p, sq, bh, n0 * 64, [&] {
        gin = load_gate_inputs(sq, p.T, n0 * 64);
        issue_rows(sq, sq.k, p.T, n0 * 64, kraw);
        issue_rows(sq, sq.v, p.T, n0 * 64, vraw);
        kwv = p.k_w[tid & (KD - 1)];
    });
    if (tid < KD) sNw[tid] = kwv;
    float logdecay = 0.f;
    StateScale sc;
    __syncthreads();
    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        const GateRegs gr = finish_gates(gin, clock);
        if (w == 0) {  // the clock and decay scan for the sweeps
            p.lam[(size_t)bh * p.Tp + t0 + lane] = gr.lamr;
            p.gam[(size_t)bh * p.Tp + t0 + lane] = gr.gam;
        }
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, t0, gr, sLam, sBeta, sGam, sc.inv());
        store_write_tile<TileW>(gr, p.T - t0, sW);
        norm_store_rows<TileF>(p, t0, kraw, sNw, p.k_eps, sK);
        store_rows<TileF>(vraw, p.T - t0, sV);
        __syncthreads();
        if (n + 1 < n1) {
            issue_rows(sq, sq.k, p.T, t0 + 64, kraw);
            issue_rows(sq, sq.v, p.T, t0 + 64, vraw);
            gin = load_gate_inputs(sq, p.T, t0 + 64);
        }
        logdecay += sGam[63];
        if (sc.fold != 1.f) {
#pragma unroll
            for (int x = 0; x < 8; x++) {
                acck[x][0] *= sc.fold;
                acck[x][1] *= sc.fold;
                accv[x][0] *= sc.fold;
                accv[x][1] *= sc.fold;
            }
        }
        chunk_state_update<TileF, TileW>(sK, HALF * (w >> 2), sW, 32 * (w & 3), sGam, acck);
        chunk_state_update<TileW, TileF>(sW, 0, sV, 32 * w, sGam, accv);
        sc.sig = sc.next;
        __syncthreads();
    }
    const size_t slot = (size_t)bh * (p.P - 1) + j;
    store_segment_state(acck, sc.sig, p.seg + slot * SEG, p.seg_exp + slot * 2 * 8);
    store_segment_state(accv, sc.sig, p.seg + slot * SEG + SEG_K, p.seg_exp + (slot * 2 + 1) * 8);
    if (tid == 0) p.seg_decay[bh * p.P + j] = exp2f(logdecay);
}

// Power-of-two exponent e of head h's readout table with max |table| 2^-e in
// [2^13, 2^14) (0 for an all-zero or non-finite table), and the table in fp16
// as table 2^-e (workgroups of batch 0), which pass 1 stages: any finite table
// keeps fp16's full precision and range.
__device__ __forceinline__ void table_exponent(const PrefillParams& p, int h, int bh) {
    __shared__ float part[8];
    const int tid = threadIdx.x;
    const float4* tb4 = reinterpret_cast<const float4*>(p.table + (size_t)h * kActive * kSlots);
    constexpr int NQ = kActive * kSlots / 4;
    float m = 0.f;
    for (int i = tid; i < NQ; i += 512) {
        const float4 t = tb4[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
    }
    m = wave_max(m);
    if ((tid & 63) == 0) part[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        float mx = part[0];
#pragma unroll
        for (int i = 1; i < 8; i++) mx = fmaxf(mx, part[i]);
        int e = 0;
        if (mx > 0.f && mx < INFINITY) {
            frexpf(mx, &e);  // mx < 2^e
            e -= 14;
        }
        p.tab_exp[bh] = e;
        part[0] = ldexpf(1.f, -e);
    }
    __syncthreads();
    // The fp16 table of head h, for every sequence's pass 1 (the exponent
    // depends on the head only).
    if (blockIdx.y == 0) {
        const float ts = part[0];
        const float* tb = p.table + (size_t)h * kActive * kSlots;
        f16_t* dst = p.tab16 + (size_t)h * kSlots * kSlots;
        for (int i = tid; i < kSlots * kSlots / 4; i += 512) {
            const int r = i >> 5;
            const float4 t = r < kActive ? *reinterpret_cast<const float4*>(tb + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            *reinterpret_cast<f16x4*>(dst + 4 * i) = f16x4{(f16_t)(t.x * ts), (f16_t)(t.y * ts), (f16_t)(t.z * ts), (f16_t)(t.w * ts)};
        }
    }
}

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void segment_state_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[SG_LDS];
    // Workgroups are dispatched in block order; the later segments, whose
    // clock prefix (clock_before) is longest, go first: z = 0 is the clock of
    // the last segment, then segments P - 2 down to 0.
    const int z = blockIdx.z;
    if (z == 0) {  // clock of the last segment and the table's exponent
        const SegCoord cd = seg_coord(p.H, p.P - 1);
        const Seq sq = make_seq(p, cd.b, cd.h, cd.bh);
        const int t_begin = (p.P - 1) * p.L * 64;
        const double carry = clock_before(p, sq, cd.bh, t_begin, [] {});
        table_exponent(p, cd.h, cd.bh);
        clock_scan(p, cd.bh, cd.b, cd.h, t_begin, carry);
        return;
    }
    const SegCoord cd = seg_coord(p.H, p.P - 1 - z);
    segment_state_body(p, cd.bh, cd.j, cd.b, cd.h, smem);
}

// ---------------------------------------------------------------------------
// Start state of segment j, in register order (the affine carry over
// segments S_{i+1} = a_i S_i + E_i, unrolled):
//   S_j = sum_{i<j} (prod_{i<l<j} a_l) E_i + (prod_{l<j} a_l) h0.
// part selects the key (0) or value (1) part of the stored states; h0 is
// row-major and nullable, h0_index(x, c, i) gives the element of acc[x][c][i].
// The segment workgroups of one sequence have block ids H * B apart; when
// H * B is a multiple of 8 they are dealt to the same XCD, and most E_i reads
// hit that XCD's L2.
// seg: E_0 of this sequence and part (E_i at seg + i * seg_stride elements);
// seg_exp: its wave exponents (E_i's at seg_exp + i * exp_stride); decay: a_0.
//
// The E_i go through the vector memory pipeline at one 1 KiB wave load per
// 16 cycles of the CU, so the sum issues exactly the loads it uses: blocks of
// at most SE_BLOCK states, each straight-line code (a compile-time count) with
// SE_DEPTH states in flight. The first block's loads go out before the
// caller's first-chunk loads (issue_first), so that adding E_{j-1} does not
// wait for those; vector loads complete in issue order.
constexpr int SE_DEPTH = 3;
constexpr int SE_BLOCK = 8;
constexpr uint32_t SE_DEAD = 0x80000000u;

struct StartStates {
    rsrc_t e, exps, decays;  // E_0 .. E_{j-1}; their exponents (exp_stride apart); a_0 ..
    uint32_t lane_off, stride_b, exp_stride_b;
    __device__ __forceinline__ uint32_t off(int i, int x) const { return lane_off + 1024u * x + (uint32_t)i * stride_b; }
};

// acc += (running decay product) 2^e_i E_i for i = i0, i0 - 1, .., i0 - NE + 1,
// in that order; `a` carries the product of the decays already passed.
template <int NE, int DEPTH, typename F>
__device__ __forceinline__ void add_states(const StartStates& st, int i0, float& a, f32x4 acc[8][2], F&& after_first) {
    constexpr int D = NE < DEPTH ? NE : DEPTH;
    const int lane = threadIdx.x & 63;
    // lane l < NE: exponent and decay of E_{i0 - l}
    const int le = i0 - lane;
    const uint32_t dm = ((uint32_t)(le | (NE - 1 - lane)) >> 31) * SE_DEAD;
    const int expv = (int)__builtin_amdgcn_raw_buffer_load_b32(st.exps, ((uint32_t)le * st.exp_stride_b) | dm, 0, 0);
    const int decv = (int)__builtin_amdgcn_raw_buffer_load_b32(st.decays, ((uint32_t)le * 4) | dm, 0, 0);
    f16x8 v[D][8];
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int x = 0; x < 8; x++)
            v[d][x] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(st.e, st.off(i0 - d, x), 0, 0));
    after_first();
#pragma unroll
    for (int d = 0; d < NE; d++) {
        const float ai = ldexpf(a, __builtin_amdgcn_readlane(expv, d));
#pragma unroll
        for (int x = 0; x < 8; x++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int q = 0; q < 4; q++) acc[x][c][q] = fmaf(ai, (float)v[d % D][x][4 * c + q], acc[x][c][q]);
        a *= __builtin_bit_cast(float, __builtin_amdgcn_readlane(decv, d));
        if (d + D < NE) {
#pragma unroll
            for (int x = 0; x < 8; x++)
                v[d % D][x] =
                    __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(st.e, st.off(i0 - d - D, x), 0, 0));
        }
    }
}

// issue_first() is called exactly once, after the first states' loads.
// DEPTH: states in flight (SE_DEPTH unless the caller's registers are short).
template <int DEPTH = SE_DEPTH, typename H0Index, typename Issue>
__device__ __forceinline__ void load_start_state(const _Float16* seg, size_t seg_stride, const int* seg_exp,
                                                 int exp_stride, const float* decay, int j, const float* h0,
                                                 H0Index h0_index, f32x4 acc[8][2], Issue&& issue_first) {
    const int lane = threadIdx.x & 63, w = wave_id();
#pragma unroll
    for (int x = 0; x < 8; x++) acc[x][0] = acc[x][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    float a = 1.f;
    if (j == 0) {
        issue_first();
    } else {
        // Host side: P <= kMaxSegments keeps j seg_stride 2 below 2^31.
        StartStates st;
        st.e = make_rsrc(seg, (size_t)j * seg_stride * 2);
        st.exps = make_rsrc(seg_exp + w, (size_t)j * exp_stride * 4);
        st.decays = make_rsrc(decay, (size_t)j * 4);
        st.lane_off = (uint32_t)frag_offset(w, 0, lane) * 2;
        st.stride_b = (uint32_t)seg_stride * 2;
        st.exp_stride_b = (uint32_t)exp_stride * 4;
        // The first block takes the remainder, so the later ones are full.
        const int r = (j - 1) % SE_BLOCK + 1;
        switch (r) {
            case 1: add_states<1, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 2: add_states<2, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 3: add_states<3, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 4: add_states<4, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 5: add_states<5, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 6: add_states<6, DEPTH>(st, j - 1, a, acc, issue_first); break;
            case 7: add_states<7, DEPTH>(st, j - 1, a, acc, issue_first); break;
            default: add_states<8, DEPTH>(st, j - 1, a, acc, issue_first); break;
        }
        static_assert(SE_BLOCK == 8, "the cases above cover 1 .. SE_BLOCK");
        for (int i0 = j - 1 - r; i0 >= 0; i0 -= SE_BLOCK) add_states<SE_BLOCK, DEPTH>(st, i0, a, acc, [] {});
    }
    if (h0) {
#pragma unroll
        for (int x = 0; x < 8; x++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int q = 0; q < 4; q++) acc[x][c][q] = fmaf(a, h0[h0_index(x, c, q)], acc[x][c][q]);
    }
}

// The same for the two parts of a prefill call's segment states.
template <int DEPTH = SE_DEPTH, typename H0Index, typename Issue>
__device__ __forceinline__ void load_start_state(const PrefillParams& p, int bh, int j, int part, const float* h0,
                                                 H0Index h0_index, f32x4 acc[8][2], Issue&& issue_first) {
    load_start_state<DEPTH>(p.seg + (size_t)bh * (p.P - 1) * SEG + part * SEG_K, SEG,
                     p.seg_exp + (size_t)bh * (p.P - 1) * 16 + part * 8, 16, p.seg_decay + bh * p.P, j, h0, h0_index,
                     acc, issue_first);
}

// ---------------------------------------------------------------------------
// Slot readout of 16 tokens (ops/chunk_readout.py:797-909), fp16 MFMA with
// fp32 accumulation; lane (lr, lg) works on token lr. The two 128-wide key
// halves of the pass-1 output (bf16, rows RR apart) come from LDS, the table
// (f16 [128][RS], row 127 zero, staged as table 2^-et) too.
//   z_t = U(lam_t) (raw0_t + raw1_t) 2^-ez_t          (B operand, registers)
//   L^T[r][t] = table[r] . z_t                       (C rows r = 16 rb + 4 lg + i)
//   p_t = softmax over r < 127 of L^T[:, t] 2^(et + ez_t)
//                                                    (in registers + 2 shuffles)
//   u^T[m][t] = sum_r table[r][m] p_t[r]             (p_t as the B operand straight
//                                                     from the C layout)
//   weights_t = bf16(U(-lam_t) u_t 2^et)             (four consecutive m per store)
// ez_t is a power of two per token with max |z_t| 2^-ez_t < 2^15, so the fp16
// operand never overflows however large the pass-1 output grows (coherent
// keys over long contexts); the scales are undone on the fp32 logits and on
// the weights, and powers of two commute with every rounding in between.
constexpr int RR = 128 + 8;  // row stride of the pass-1 output tiles in LDS

__device__ __forceinline__ void readout_tokens(const bf16_t* sR0, const bf16_t* sR1, const f16_t* sTab, float lamr,
                                               float tab_scale, bf16_t* dst) {
    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    // Phases: the hardware gives (cos, sin) of pairs 1, 8, 16 and of the
    // lane's first pair of each group; the others follow by rotation (complex
    // multiplication), at most six steps for z and eight for the weights,
    // each adding about 1e-7 to values that are rounded to fp16 / bf16.
    float s1, c1, s16, c16;
    pair_sincos(lamr, 1, s1, c1);
    pair_sincos(lamr, 16, s16, c16);
    float zs[4], zc[4];  // pairs 4 lg + q, then 16 ks + 4 lg + q
    pair_sincos(lamr, 4 * lg, zs[0], zc[0]);
    // raw0 + raw1, element 2 q (+1) of fragment ks = coordinate 32 ks + 8 lg + 2 q (+1)
    float re[4][4], ro[4][4];
    float m = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const bf16x8 ra = *reinterpret_cast<const bf16x8*>(sR0 + lr * RR + 32 * ks + 8 * lg);
        const bf16x8 rb = *reinterpret_cast<const bf16x8*>(sR1 + lr * RR + 32 * ks + 8 * lg);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            re[ks][q] = (float)ra[2 * q] + (float)rb[2 * q];
            ro[ks][q] = (float)ra[2 * q + 1] + (float)rb[2 * q + 1];
            m = fmaxf(m, fmaxf(fabsf(re[ks][q]), fabsf(ro[ks][q])));
        }
    }
    // The token's largest raw coordinate (its 128 values are spread over the
    // four row groups); a rotated pair is at most sqrt(2) times larger.
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    int ez = 0;
    if (m > 0.f && m < INFINITY) {
        frexpf(m, &ez);  // m < 2^ez
        ez -= 14;
    }
    const float zscale = ldexpf(1.f, -ez);
    zs[0] *= zscale;
    zc[0] *= zscale;
#pragma unroll
    for (int q = 1; q < 4; q++) {
        zc[q] = zc[q - 1] * c1 - zs[q - 1] * s1;
        zs[q] = zs[q - 1] * c1 + zc[q - 1] * s1;
    }
    // z fragments: element j = z_t[32 ks + 8 lg + j] 2^-ez.
    f16x8 zf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float e = re[ks][q], o = ro[ks][q];
            const float sn = zs[q], cs = zc[q];
            zf[ks][2 * q] = (f16_t)(cs * e - sn * o);
            zf[ks][2 * q + 1] = (f16_t)(sn * e + cs * o);
            if (ks < 3) {
                zc[q] = cs * c16 - sn * s16;
                zs[q] = sn * c16 + cs * s16;
            }
        }
    }
    f32x4 L[8];
#pragma unroll
    for (int rb8 = 0; rb8 < 8; rb8++) L[rb8] = f32x4{0.f, 0.f, 0.f, 0.f};
    sched_fence();
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
        for (int rb8 = 0; rb8 < 8; rb8++)
            L[rb8] = mfma_f16(load_row_ld<f16x8>(sTab, RS, 16 * rb8, 32 * ks), zf[ks], L[rb8]);
        sched_fence();
    }
    if (lg == 3) L[7][3] = -INFINITY;  // slot r = 127 is not active
    float mx = -INFINITY;
#pragma unroll
    for (int rb8 = 0; rb8 < 8; rb8++)
#pragma unroll
        for (int i = 0; i < 4; i++) mx = fmaxf(mx, L[rb8][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // e^(logit - max) with logit = L 2^(et + ez): one exponential per slot
    const float lsc = kLog2e * tab_scale * ldexpf(1.f, ez);
    float sum = 0.f;
#pragma unroll
    for (int rb8 = 0; rb8 < 8; rb8++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            L[rb8][i] = fast_exp2((L[rb8][i] - mx) * lsc);
            sum += L[rb8][i];
        }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const float inv = 1.f / sum;
    f16x8 pf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pf[ks][i] = (f16_t)(L[2 * ks][i] * inv);
            pf[ks][4 + i] = (f16_t)(L[2 * ks + 1][i] * inv);
        }
    f32x4 U[8];
#pragma unroll
    for (int mb = 0; mb < 8; mb++) U[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    sched_fence();
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
        for (int mb = 0; mb < 8; mb++) U[mb] = mfma_f16(load_tr_pair_f16(sTab, RS, 32 * ks, 16 * mb), pf[ks], U[mb]);
        sched_fence();
    }
    // Lane holds u_t[16 mb + 4 lg + i] 2^-et: pairs 8 mb + 2 lg + q, q = 0, 1.
    float s8, c8, ws[2], wc[2];
    pair_sincos(lamr, 8, s8, c8);
    pair_sincos(lamr, 2 * lg, ws[0], wc[0]);
    ws[0] *= tab_scale;
    wc[0] *= tab_scale;
    wc[1] = wc[0] * c1 - ws[0] * s1;
    ws[1] = ws[0] * c1 + wc[0] * s1;
#pragma unroll
    for (int mb = 0; mb < 8; mb++) {
        bf16x4 o;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const float sn = ws[q], cs = wc[q];
            const float ue = U[mb][2 * q], uo = U[mb][2 * q + 1];
            o[2 * q] = (bf16_t)(cs * ue + sn * uo);
            o[2 * q + 1] = (bf16_t)(cs * uo - sn * ue);
            if (mb < 7) {
                wc[q] = cs * c8 - sn * s8;
                ws[q] = sn * c8 + cs * s8;
            }
        }
        *reinterpret_cast<bf16x4*>(dst + 16 * mb + 4 * lg) = o;
    }
}

// ---------------------------------------------------------------------------
// 2. Pass 1 (key state) and the slot readout, one segment per workgroup.
// grid = (H, B, P), 512 threads.
// Wave w works on key half y = w >> 2 and state columns [32 mq, 32 mq + 32),
// mq = w & 3: acc[kb][c] = S[128 y + state_row(kb, lg, i)][32 mq + 16 c + lr],
// and the same 32 output coordinates of half y:
// out[tb][c] = raw_y^T[32 mq + 16 c + 4 lg + i][16 tb + lr].
constexpr int P1_Q = 0;                        // q_hat, TileQ
constexpr int P1_K = P1_Q + TileQ::bytes;      // k_hat, TileF
constexpr int P1_W = P1_K + TileF::bytes;      // w, TileW
constexpr int P1_P = P1_W + TileW::bytes;      // masked scores of each half, 2 x TileP
constexpr int P1_G = P1_P + 2 * TileP::bytes;  // f32 [5][64] gates
constexpr int P1_NW = P1_G + 5 * 64 * 4;      // f32 [2][256] q and k norm weights
constexpr int P1_T = P1_NW + 2 * KD * 4;       // f16 [128][RS] readout table of the head (row 127 zero)
constexpr int P1_LDS = P1_T + 128 * RS * 2;
static_assert(2 * 64 * RR * 2 <= TileQ::bytes, "the two pass-1 output tiles fit in the q_hat tile");
static_assert(P1_LDS <= 160 * 1024, "pass-1 workgroup must fit in one CU's LDS");

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void pass1_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P1_LDS];
    bf16_t* sQ = reinterpret_cast<bf16_t*>(smem + P1_Q);
    bf16_t* sK = reinterpret_cast<bf16_t*>(smem + P1_K);
    bf16_t* sW = reinterpret_cast<bf16_t*>(smem + P1_W);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P1_P);
    float* sLam = reinterpret_cast<float*>(smem + P1_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    float* sQw = reinterpret_cast<float*>(smem + P1_NW);
    float* sKw = sQw + KD;
    f16_t* sTab = reinterpret_cast<f16_t*>(smem + P1_T);
    // After the scores and the inter-chunk product the q_hat tile is free; it
    // then holds the chunk's pass-1 output of both key halves for the readout.
    bf16_t* sR0 = sQ;
    bf16_t* sR1 = sQ + 64 * RR;

    const SegCoord cd = seg_coord(p.H, blockIdx.z);
    const int bh = cd.bh, j = cd.j, b = cd.b, h = cd.h;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), lr = lane & 15, lg = lane >> 4;
    const int y = w >> 2, mq = w & 3;
    const float log2_scale = p.log2_scale;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    const Seq sq = make_seq(p, b, h, bh);
    // Staging is split between the halves: every wave normalises its share of
    // q at the top of a chunk; the waves of the second half (u = tid - 256)
    // load and stage k_hat, the write-vector tile and the gates of the next
    // chunk while the first half runs the chunk's slot readout.
    const int u = tid - 256;
    // The table is staged in fp16 as table 2^-et (segment_state wrote it and
    // et: max |table| 2^-et < 2^14); the readout undoes the factor.
    const int et = p.tab_exp[bh];
    const float tab_scale = ldexpf(1.f, et);
    // The first chunk's loads follow the start state's first loads (see
    // load_start_state). kraw holds k rows in the second half and the table's
    // rows in the first: the same eight loads per lane, with no branch among
    // them (a branch would make the waits for the start state cover them).
    bf16x8 qraw[4], kraw[8];
    GateRegs gr;
    float qw, kw;
    f32x4 acc[8][2];
    load_start_state<2>(p, bh, j, 0, p.h0_k ? p.h0_k + (size_t)bh * SEG_K : nullptr,
                     [&](int kb, int c, int i) { return (HALF * y + state_row(kb, lg, i)) * kSlots + 32 * mq + 16 * c + lr; },
                     acc, [&] {
                         issue_rows(sq, sq.q, p.T, n0 * 64, qraw);
                         const int t = min(n0 * 64 + (u >> 2), p.T - 1);
                         const rsrc_t src = y ? sq.k : make_rsrc(p.tab16 + (size_t)h * kSlots * kSlots, kSlots * kSlots * 2);
                         const uint32_t base = y ? (uint32_t)t * sq.row16 + 128 * (u & 3) : 16 * tid;
                         const uint32_t step = y ? 16 : 4096;
#pragma unroll
                         for (int i = 0; i < 8; i++) kraw[i] = ld_b128(src, base + step * i);
                         gr = issue_gates(sq, p.T, n0 * 64);
                         qw = p.q_w[tid & (KD - 1)];
                         kw = p.k_w[tid & (KD - 1)];
                     });
    if (tid < KD) {
        sQw[tid] = qw;
        sKw[tid] = kw;
    }
    if (y == 0) {  // table rows 16 i + (tid >> 4), columns 8 (tid & 15) ..
#pragma unroll
        for (int i = 0; i < 8; i++)
            *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16_t*>(sTab) + (16 * i + (tid >> 4)) * RS + 8 * (tid & 15)) = kraw[i];
    }
    zero_scores(sP, 2);  // the two blocks above the diagonal that the intra product reads stay zero
    bf16_t* sPy = sP + y * (TileP::bytes / 2);
    StateScale sc;
    __syncthreads();  // norm weights and table staged, score tiles zeroed
    if (y == 1) {
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, n0 * 64, gr, sLam, sBeta, sGam, sc.inv(), 4);
        store_write_tile<TileW, 4>(gr, p.T - n0 * 64, sW, mq);
        norm_store_rows_q<TileF>(p, n0 * 64, u, kraw, sKw, p.k_eps, sK);
    }

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        norm_store_rows<TileQ>(p, t0, qraw, sQw, p.q_eps, sQ);
        __syncthreads();
        // The second half has taken this chunk's scale step while staging it.
        if (y == 0) sc.begin_chunk(sGam[63]);
        // The next chunk's loads are spread over the phases (q here, k and the
        // gates after the scores) so that no wave waits at a barrier for the
        // CU's memory pipeline to accept them.
        if (n + 1 < n1) issue_rows(sq, sq.q, p.T, t0 + 64, qraw);

        // Masked, decayed scores of this half's key slice: blocks mq, mq + 4 (and mq + 8).
        score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq, sGam, log2_scale, sPy);
        score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq + 4, sGam, log2_scale, sPy);
        if (mq < 2) score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq + 8, sGam, log2_scale, sPy);
        // raw_y^T = 2^G_t S_n^T q_t over this half's key rows.
        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) out[tb][0] = out[tb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8 a0 = state_frag(acc[2 * ks][0], acc[2 * ks + 1][0]);
            const bf16x8 a1 = state_frag(acc[2 * ks][1], acc[2 * ks + 1][1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 bq = load_row<TileQ>(sQ, 16 * tb, HALF * y + 32 * ks);
                out[tb][0] = mfma_bf16(a0, bq, out[tb][0]);
                out[tb][1] = mfma_bf16(a1, bq, out[tb][1]);
            }
        }
        const float osc = p.scale * sc.sig;
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const float f = sGam[64 + 16 * tb + lr] * osc;
            out[tb][0] *= f;
            out[tb][1] *= f;
        }
        __syncthreads();  // scores complete

        // raw_y^T += w^T P_y^T (P carries the scale); the blocks of P above the diagonal are zero.
        // wf[c][ss][jj] = w[32 ss + 8 lg + jj][32 mq + 16 c + lr].
        bf16x8 wf[2][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int ss = 0; ss < 2; ss++) wf[c][ss] = load_tr<TileW>(sW, 32 * ss, 32 * mq + 16 * c);
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int ss = 0; ss <= (tb >> 1); ss++) {
                const bf16x8 pf = load_row<TileP>(sPy, 16 * tb, 32 * ss);
                out[tb][0] = mfma_bf16(wf[0][ss], pf, out[tb][0]);
                out[tb][1] = mfma_bf16(wf[1][ss], pf, out[tb][1]);
            }
        // The half's output, rounded to bf16 (ops/chunk_o.py:369-374), into LDS.
        bf16_t* sRy = y == 0 ? sR0 : sR1;
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
                *reinterpret_cast<bf16x4*>(sRy + (16 * tb + lr) * RR + 32 * mq + 16 * c + 4 * lg) = to_bf16x4(out[tb][c], 1.f);
        // State update: S = 2^G_last S + k_hat^T bf16(2^(G_last - G_s) w), as
        // acc += k_hat^T bf16(2^(G_last - G_s) / sigma' w).
        if (sc.fold != 1.f) {
#pragma unroll
            for (int kb = 0; kb < 8; kb++) {
                acc[kb][0] *= sc.fold;
                acc[kb][1] *= sc.fold;
            }
        }
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            bf16x8 wt[2];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    wt[c][jj] = (bf16_t)((float)wf[c][ss][jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
#pragma unroll
            for (int kb = 0; kb < 8; kb++) {
                const bf16x8 kf = load_tr_perm<TileF>(sK, 32 * ss, HALF * y + 32 * (kb >> 1), kb & 1);
                acc[kb][0] = mfma_bf16(kf, wt[0], acc[kb][0]);
                acc[kb][1] = mfma_bf16(kf, wt[1], acc[kb][1]);
            }
        }
        sc.sig = sc.next;
        const float lamr = sLam[16 * mq + lr];
        __syncthreads();  // output tiles complete; k_hat, w and the gates of this chunk are done with
        if (y == 0) {
            // Slot readout of the chunk: wave mq takes tokens 16 mq .. 16 mq + 15.
            readout_tokens(sR0 + 16 * mq * RR, sR1 + 16 * mq * RR, sTab, lamr, tab_scale,
                           p.omega + ((size_t)bh * p.Tp + t0 + 16 * mq + lr) * kSlots);
        } else if (n + 1 < n1) {
            // The readout outlasts these loads; their latency is hidden behind it.
            issue_rows_q(sq, sq.k, p.T, t0 + 64, u, kraw);
            gr = issue_gates(sq, p.T, t0 + 64);
            sc.begin_chunk(chunk_last_gam(gr));
            commit_gates(p.T, t0 + 64, gr, sLam, sBeta, sGam, sc.inv(), 4);
            store_write_tile<TileW, 4>(gr, p.T - t0 - 64, sW, mq);
            norm_store_rows_q<TileF>(p, t0 + 64, u, kraw, sKw, p.k_eps, sK);
        }
        __syncthreads();  // tiles are overwritten by the next chunk
    }

    if (j == p.P - 1 && p.hk) {
        float* dst = p.hk + (size_t)bh * SEG_K;
#pragma unroll
        for (int kb = 0; kb < 8; kb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    dst[(HALF * y + state_row(kb, lg, i)) * kSlots + 32 * mq + 16 * c + lr] = acc[kb][c][i] * sc.sig;
    }
}

// ---------------------------------------------------------------------------
// 3. Pass 2 (value state), one segment per workgroup. grid = (H, B, P), 512
// threads. Wave w owns value columns [32 w, 32 w + 32):
// acc[mb][c] = S[state_row(mb, lg, i)][32 w + 16 c + lr], and the same 32 output
// coordinates: out[tb][c] = o^T[32 w + 16 c + 4 lg + i][16 tb + lr].
constexpr int P2_OM = 0;                     // slot weights (query), TileO
constexpr int P2_W = P2_OM + TileO::bytes;   // w (key), TileW
constexpr int P2_V = P2_W + TileW::bytes;    // v, TileF
constexpr int P2_P = P2_V + TileF::bytes;    // masked scores, TileP
constexpr int P2_G = P2_P + TileP::bytes;    // f32 [5][64] gates
constexpr int P2_N = P2_G + 5 * 64 * 4;      // output norm: f32 [64][8] partial sums of squares, f32 [256] weight
constexpr int P2_LDS = P2_N + (64 * 8 + VD) * 4;
static_assert(P2_LDS <= 160 * 1024, "pass-2 workgroup must fit in one CU's LDS");

// NORM: the gated output norm (on_w, on_gate) is applied before o is stored.
// Each lane's eight coordinates of a token are rounded and scaled (xs), their
// squares summed over the lane's row group and written per wave to LDS; the
// per-token totals are read back after the chunk's last barrier, where the
// normalised, gated output is stored.
template <bool NORM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void pass2_kernel(PrefillParams p) {
    __shared__ __align__(16) unsigned char smem[P2_LDS];
    bf16_t* sOm = reinterpret_cast<bf16_t*>(smem + P2_OM);
    bf16_t* sW = reinterpret_cast<bf16_t*>(smem + P2_W);
    bf16_t* sV = reinterpret_cast<bf16_t*>(smem + P2_V);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P2_P);
    float* sLam = reinterpret_cast<float*>(smem + P2_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    float* sNs = reinterpret_cast<float*>(smem + P2_N);  // [token][wave]
    float* sNw = sNs + 64 * 8;

    const SegCoord cd = seg_coord(p.H, blockIdx.z);
    const int bh = cd.bh, j = cd.j, b = cd.b, h = cd.h;
    const int lane = threadIdx.x & 63, w = wave_id(), lr = lane & 15, lg = lane >> 4;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    const Seq sq = make_seq(p, b, h, bh);
    const rsrc_t rom = make_rsrc(p.omega + (size_t)bh * p.Tp * kSlots, (size_t)p.Tp * kSlots * 2);
    const uint32_t o_lane = (uint32_t)lr * sq.row16 + 2 * (32 * w + 4 * lg);
    // The first chunk's loads follow the start state's first loads.
    bf16x8 vraw[4], om[2];
    GateRegs gr;
    float nw = 0.f;
    f32x4 acc[8][2];
    load_start_state(p, bh, j, 1, p.h0_v ? p.h0_v + (size_t)bh * SEG_V : nullptr,
                     [&](int mb, int c, int i) { return state_row(mb, lg, i) * VD + 32 * w + 16 * c + lr; }, acc,
                     [&] {
                         issue_rows(sq, sq.v, p.T, n0 * 64, vraw);
                         issue_omega(rom, n0 * 64, om);
                         gr = issue_gates(sq, p.T, n0 * 64);
                         if (NORM) nw = p.on_w[threadIdx.x & (VD - 1)];
                     });
    if (NORM && threadIdx.x < VD) sNw[threadIdx.x] = nw;
    zero_scores(sP, 1);
    StateScale sc;

    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, t0, gr, sLam, sBeta, sGam, sc.inv());
        store_write_tile<TileW>(gr, p.T - t0, sW);
        store_half_rows(om, 64, sOm);
        store_rows<TileF>(vraw, p.T - t0, sV);
        __syncthreads();
        // NORM: this chunk's gate for the lane's output coordinates, issued
        // before the next chunk's loads, so that waiting for it in the
        // epilogue does not wait for them (loads complete in order).
        // Rows past T are clamped to T - 1 inside the per-lane offset: the
        // buffer's range check covers the lane offset only, not the scalar
        // offset, so a row index never goes into the scalar offset of a load.
        bf16x4 gate[4][2];
        if constexpr (NORM) {
            const rsrc_t rg = rows_rsrc(p, b, h, p.on_gate);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const int tg = min(t0 + 16 * tb + lr, p.T - 1);
                const uint32_t off = (uint32_t)tg * sq.row16 + 2 * (32 * w + 4 * lg);
#pragma unroll
                for (int c = 0; c < 2; c++) gate[tb][c] = ld_b64(rg, off + 32 * c, 0);
            }
        }
        // The next chunk's loads are spread over the phases (see pass 1).
        if (n + 1 < n1) issue_omega(rom, t0 + 64, om);

        score_tile<TileO, TileW>(sOm, 0, sW, 0, w, sGam, 0.f, sP);
        if (w < 2) score_tile<TileO, TileW>(sOm, 0, sW, 0, w + 8, sGam, 0.f, sP);
        // o^T = 2^G_t S_n^T weights_t.
        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) out[tb][0] = out[tb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8 a0 = state_frag(acc[2 * ks][0], acc[2 * ks + 1][0]);
            const bf16x8 a1 = state_frag(acc[2 * ks][1], acc[2 * ks + 1][1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 bo = load_row<TileO>(sOm, 16 * tb, 32 * ks);
                out[tb][0] = mfma_bf16(a0, bo, out[tb][0]);
                out[tb][1] = mfma_bf16(a1, bo, out[tb][1]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const float f = sGam[64 + 16 * tb + lr] * sc.sig;
            out[tb][0] *= f;
            out[tb][1] *= f;
        }
        __syncthreads();  // scores complete
        if (n + 1 < n1) {
            issue_rows(sq, sq.v, p.T, t0 + 64, vraw);
            gr = issue_gates(sq, p.T, t0 + 64);
        }

        // o^T += v^T P^T. vb[c][ss][jj] = v[32 ss + 8 lg + jj][32 w + 16 c + lr].
        bf16x8 vb[2][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int ss = 0; ss < 2; ss++) vb[c][ss] = load_tr<TileF>(sV, 32 * ss, 32 * w + 16 * c);
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int ss = 0; ss <= (tb >> 1); ss++) {
                const bf16x8 pf = load_row<TileP>(sP, 16 * tb, 32 * ss);
                out[tb][0] = mfma_bf16(vb[0][ss], pf, out[tb][0]);
                out[tb][1] = mfma_bf16(vb[1][ss], pf, out[tb][1]);
            }
        bf16x4 xs[4][2];  // NORM: bf16(bf16(o) * prescale)
        if constexpr (NORM) {
            float ss[4];
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                ss[tb] = 0.f;
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const bf16x4 o4 = to_bf16x4(out[tb][c], 1.f);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        xs[tb][c][i] = (bf16_t)((float)o4[i] * p.on_prescale);
                        const float x = (float)xs[tb][c][i];
                        ss[tb] = fmaf(x, x, ss[tb]);
                    }
                }
            }
            // the four tiles' exchanges issued together (their latencies overlap)
            float sh[4];
#pragma unroll
            for (int tb = 0; tb < 4; tb++) sh[tb] = __shfl_xor(ss[tb], 16);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) ss[tb] += sh[tb];
#pragma unroll
            for (int tb = 0; tb < 4; tb++) sh[tb] = __shfl_xor(ss[tb], 32);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                ss[tb] += sh[tb];
                if (lg == 0) sNs[(16 * tb + lr) * 8 + w] = ss[tb];
            }
        } else {
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                if (t0 + 16 * tb + lr < p.T) {
#pragma unroll
                    for (int c = 0; c < 2; c++)
                        st_b64(sq.o, o_lane + 32 * c, (uint32_t)(t0 + 16 * tb) * sq.row16, to_bf16x4(out[tb][c], 1.f));
                }
            }
        }
        // State update: S = 2^G_last S + w^T bf16(2^(G_last - G_s) v), as
        // acc += w^T bf16(2^(G_last - G_s) / sigma' v).
        if (sc.fold != 1.f) {
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                acc[mb][0] *= sc.fold;
                acc[mb][1] *= sc.fold;
            }
        }
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            bf16x8 vt[2];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    vt[c][jj] = (bf16_t)((float)vb[c][ss][jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                const bf16x8 wk = load_tr_perm<TileW>(sW, 32 * ss, 32 * (mb >> 1), mb & 1);
                acc[mb][0] = mfma_bf16(wk, vt[0], acc[mb][0]);
                acc[mb][1] = mfma_bf16(wk, vt[1], acc[mb][1]);
            }
        }
        sc.sig = sc.next;
        __syncthreads();
        if constexpr (NORM) {
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const float4 s0 = *reinterpret_cast<const float4*>(sNs + (16 * tb + lr) * 8);
                const float4 s1 = *reinterpret_cast<const float4*>(sNs + (16 * tb + lr) * 8 + 4);
                const float tot = ((s0.x + s0.y) + (s0.z + s0.w)) + ((s1.x + s1.y) + (s1.z + s1.w));
                const float rs = rsqrtf(tot * (1.f / VD) + p.on_eps);
                if (t0 + 16 * tb + lr < p.T) {
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        const float4 wv = *reinterpret_cast<const float4*>(sNw + 32 * w + 16 * c + 4 * lg);
                        const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
                        bf16x4 y;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            y[i] = (bf16_t)((float)xs[tb][c][i] * rs * wa[i] * sigmoidf((float)gate[tb][c][i]));
                        st_b64(sq.o, o_lane + 32 * c, (uint32_t)(t0 + 16 * tb) * sq.row16, y);
                    }
                }
            }
        }
    }

    if (j == p.P - 1 && p.hv) {
        float* dst = p.hv + (size_t)bh * SEG_V;
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[state_row(mb, lg, i) * VD + 32 * w + 16 * c + lr] = acc[mb][c][i] * sc.sig;
    }
}

// ---------------------------------------------------------------------------
// table[h] = readout[h] @ Phi (ops/chunk.py:82-103, 281). One block per
// (h, r); Phi[j][m] is taken from the 127 angles 2 pi k / 127 (sine and
// cosine formed once per block in LDS) at the exact integer reduction
// k = (pair * j) mod 127 of its angle, stepped by pair per j.
__global__ __launch_bounds__(128) void readout_table_kernel(const float* readout, float* table) {
    const int hr = blockIdx.x, m = threadIdx.x, pair = m >> 1;
    __shared__ float row[kActive], cos_k[kActive], sin_k[kActive];
    if (m < kActive) {
        row[m] = readout[(size_t)hr * kActive + m];
        sincosf((float)m * 0.049473900056532176f, &sin_k[m], &cos_k[m]);
    }
    __syncthreads();
    float acc = 0.f;
    if (m != 1) {
        const float sc = pair_scale(pair);
        const float* basis = (m & 1) ? sin_k : cos_k;
        int k = 0;  // (pair * jr) mod 127
        for (int jr = 0; jr < kActive; jr++) {
            acc = fmaf(row[jr], sc * basis[k], acc);
            k += pair;
            k = k >= kActive ? k - kActive : k;
        }
    }
    table[(size_t)hr * kSlots + m] = acc;
}

// ---------------------------------------------------------------------------
// 4. Isolated ScalarGatedLA: one pass of scalar_la (ops/chunk.py:30-79 over
// state_forward, ops/chunk_h.py:10-339, and output_forward, ops/chunk_o.py:177-613)
//   S_{n+1} = 2^G_last S_n + k^T bf16(2^(G_last - G_s) v)
//   o_t = scale (2^G_t q_t S_n + sum_{s <= t} bf16(2^(G_t - G_s) q_t . k_s) v_s)
// with q, k, v and g read from memory and the in-chunk decay scan G formed on
// the fly. Shape A: K = 256, V = 128 (the pass-1 shape; the output is formed
// per 128-wide key slice, each slice scaled and rounded to bf16, and the slices
// summed, as the reference's raw output accumulates them, ops/chunk_o.py:240-250);
// shape B: K = 128, V = 256 (the pass-2 shape). Segments as in the prefill:
// segment-local end states, then one sweep per segment from its carried start.

// The streams of one (batch, head) sequence; row strides in bytes.
struct SlaSeq {
    rsrc_t q, k, v, o, g;
    uint32_t rk, rv, ro;
};

__device__ __forceinline__ SlaSeq make_sla_seq(const SlaParams& p, int b, int h) {
    const size_t bh = (size_t)b * p.H + h;
    const size_t bth = (size_t)b * p.T * p.H + h;        // row (b, 0, h) of a [B, T, H, .] tensor
    const size_t span = (size_t)(p.T - 1) * p.H + 1;     // its rows up to (b, T - 1, h)
    SlaSeq s;
    s.q = make_rsrc(p.q + bh * p.T * p.K, (size_t)p.T * p.K * 2);
    s.k = make_rsrc(p.k + bh * p.T * p.K, (size_t)p.T * p.K * 2);
    s.rk = p.K * 2;
    s.v = p.v_bth ? make_rsrc(p.v + bth * p.V, span * p.V * 2) : make_rsrc(p.v + bh * p.T * p.V, (size_t)p.T * p.V * 2);
    s.rv = (p.v_bth ? p.H : 1) * p.V * 2;
    const size_t osz = p.raw_output ? 4 : 2;
    char* o = reinterpret_cast<char*>(p.o);
    s.o = p.o_bth ? make_rsrc(o + bth * p.V * osz, span * p.V * osz) : make_rsrc(o + bh * p.T * p.V * osz, (size_t)p.T * p.V * osz);
    s.ro = (p.o_bth ? p.H : 1) * p.V * (uint32_t)osz;
    s.g = make_rsrc(p.g + bh * p.T, (size_t)p.T * 4);
    return s;
}

// G_t = log2(e) * (in-chunk inclusive sum of g) from the raw gate, lane = token
// (ops/utils.py:495-520).
__device__ __forceinline__ GateRegs sla_gates(float graw) {
    GateRegs r;
    r.beta = 0.f;
    r.lamr = 0.f;
    r.gam = wave_scan(graw) * kLog2e;
    return r;
}

__device__ __forceinline__ void st_b128(rsrc_t r, uint32_t off, uint32_t soff, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, soff, 0);
}

// Segment-local end states, grid (H, B, P - 1), 512 threads; the state blocks of
// the waves as in the prefill's key (shape A) or value (shape B) part.
constexpr int SLS_F = 0;                      // the 256-wide operand, TileF
constexpr int SLS_H = SLS_F + TileF::bytes;  // the 128-wide operand, TileW
constexpr int SLS_G = SLS_H + TileW::bytes;  // f32 [5][64] gates
constexpr int SLS_LDS = SLS_G + 5 * 64 * 4;
static_assert(2 * SLS_LDS <= 160 * 1024, "two scalar_la segment workgroups must fit in one CU's LDS");

template <bool SA>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void sla_segment_kernel(SlaParams p) {
    __shared__ __align__(16) unsigned char smem[SLS_LDS];
    bf16_t* sF = reinterpret_cast<bf16_t*>(smem + SLS_F);  // the 256-wide operand: k (A) or v (B), TileF
    bf16_t* sH = reinterpret_cast<bf16_t*>(smem + SLS_H);  // the 128-wide operand: v (A) or k (B), TileW
    float* sLam = reinterpret_cast<float*>(smem + SLS_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    using LA = typename std::conditional<SA, TileF, TileW>::type;
    using LB = typename std::conditional<SA, TileW, TileF>::type;
    const bf16_t* sArow = SA ? sF : sH;
    const bf16_t* sBcol = SA ? sH : sF;
    const int h = blockIdx.x, b = blockIdx.y, j = blockIdx.z, bh = b * p.H + h;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    const int a_col = SA ? HALF * (w >> 2) : 0;
    const int b_col = SA ? 32 * (w & 3) : 32 * w;
    const SlaSeq sq = make_sla_seq(p, b, h);
    const rsrc_t xf = SA ? sq.k : sq.v, xh = SA ? sq.v : sq.k;
    const uint32_t rf = SA ? sq.rk : sq.rv, rh = SA ? sq.rv : sq.rk;
    f32x4 acc[8][2];
#pragma unroll
    for (int x = 0; x < 8; x++) acc[x][0] = acc[x][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 fraw[4], hraw[2];
    issue_rows_stride(xf, rf, p.T, n0 * 64, fraw);
    issue_half_rows(xh, rh, n0 * 64, hraw);
    float graw = ld_f32(sq.g, (uint32_t)(n0 * 64 + lane) * 4);
    float logdecay = 0.f;
    StateScale sc;
    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        const GateRegs gr = sla_gates(graw);
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, t0, gr, sLam, sBeta, sGam, sc.inv());
        store_rows<TileF>(fraw, 64, sF);
        store_half_rows<TileW>(hraw, 64, sH);
        __syncthreads();
        if (n + 1 < n1) {
            issue_rows_stride(xf, rf, p.T, t0 + 64, fraw);
            issue_half_rows(xh, rh, t0 + 64, hraw);
            graw = ld_f32(sq.g, (uint32_t)(t0 + 64 + lane) * 4);
        }
        logdecay += sGam[63];
        if (sc.fold != 1.f) {
#pragma unroll
            for (int x = 0; x < 8; x++) {
                acc[x][0] *= sc.fold;
                acc[x][1] *= sc.fold;
            }
        }
        chunk_state_update<LA, LB>(sArow, a_col, sBcol, b_col, sGam, acc);
        sc.sig = sc.next;
        __syncthreads();
    }
    const size_t slot = (size_t)bh * (p.P - 1) + j;
    store_segment_state(acc, sc.sig, p.seg + slot * (KD * HALF), p.seg_exp + slot * 8);
    if (tid == 0) p.seg_decay[bh * p.P + j] = exp2f(logdecay);
}

// Start state of segment j of a scalar_la sequence (one part per segment).
template <typename H0Index>
__device__ __forceinline__ void sla_start_state(const SlaParams& p, int bh, int j, H0Index h0_index, f32x4 acc[8][2]) {
    load_start_state(p.seg + (size_t)bh * (p.P - 1) * (KD * HALF), KD * HALF, p.seg_exp + (size_t)bh * (p.P - 1) * 8, 8,
                     p.seg_decay + bh * p.P, j, p.h0 ? p.h0 + (size_t)bh * (KD * HALF) : nullptr, h0_index, acc, [] {});
}

// Shape A sweep (K = 256, V = 128), grid (H, B, P), 512 threads. Wave w works
// on key slice y = w >> 2 and state columns [32 mq, 32 mq + 32), mq = w & 3, as
// pass 1 does; each slice's output, bf16(scale x), goes through LDS and the
// two slices are summed per token.
constexpr int SA_Q = 0;                        // q, TileQ
constexpr int SA_K = SA_Q + TileQ::bytes;      // k, TileF
constexpr int SA_V = SA_K + TileF::bytes;      // v, TileW
constexpr int SA_P = SA_V + TileW::bytes;      // masked scores of each slice, 2 x TileP
constexpr int SA_G = SA_P + 2 * TileP::bytes;  // f32 [5][64] gates
constexpr int SA_LDS = SA_G + 5 * 64 * 4;
static_assert(SA_LDS <= 160 * 1024, "scalar_la workgroup must fit in one CU's LDS");

__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void sla_sweep_a_kernel(SlaParams p) {
    __shared__ __align__(16) unsigned char smem[SA_LDS];
    bf16_t* sQ = reinterpret_cast<bf16_t*>(smem + SA_Q);
    bf16_t* sK = reinterpret_cast<bf16_t*>(smem + SA_K);
    bf16_t* sW = reinterpret_cast<bf16_t*>(smem + SA_V);
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + SA_P);
    float* sLam = reinterpret_cast<float*>(smem + SA_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    bf16_t* sR0 = sQ;  // the slices' outputs, after the q tile is done with
    bf16_t* sR1 = sQ + 64 * RR;
    const int h = blockIdx.x, b = blockIdx.y, j = blockIdx.z, bh = b * p.H + h;
    const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), lr = lane & 15, lg = lane >> 4;
    const int y = w >> 2, mq = w & 3;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    const SlaSeq sq = make_sla_seq(p, b, h);
    bf16x8 qraw[4], kraw[4], vraw[2];
    issue_rows_stride(sq.q, sq.rk, p.T, n0 * 64, qraw);
    issue_rows_stride(sq.k, sq.rk, p.T, n0 * 64, kraw);
    issue_half_rows(sq.v, sq.rv, n0 * 64, vraw);
    float graw = ld_f32(sq.g, (uint32_t)(n0 * 64 + lane) * 4);
    zero_scores(sP, 2);
    bf16_t* sPy = sP + y * (TileP::bytes / 2);
    f32x4 acc[8][2];
    sla_start_state(p, bh, j,
                    [&](int kb, int c, int i) { return (HALF * y + state_row(kb, lg, i)) * HALF + 32 * mq + 16 * c + lr; },
                    acc);
    StateScale sc;
    // combine mapping: token r, columns [16 cq, 16 cq + 16)
    const int r = tid >> 3, cq = tid & 7;
    const bool raw = p.raw_output != 0;
    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        const GateRegs gr = sla_gates(graw);
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, t0, gr, sLam, sBeta, sGam, sc.inv());
        store_rows<TileQ>(qraw, 64, sQ);
        store_rows<TileF>(kraw, 64, sK);
        store_half_rows<TileW>(vraw, 64, sW);
        __syncthreads();
        if (n + 1 < n1) {
            issue_rows_stride(sq.q, sq.rk, p.T, t0 + 64, qraw);
            graw = ld_f32(sq.g, (uint32_t)(t0 + 64 + lane) * 4);
        }
        // Masked, decayed scores of this slice (unscaled): blocks mq, mq + 4 (and mq + 8).
        score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq, sGam, 0.f, sPy);
        score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq + 4, sGam, 0.f, sPy);
        if (mq < 2) score_tile<TileQ, TileF>(sQ, HALF * y, sK, HALF * y, mq + 8, sGam, 0.f, sPy);
        // x_y^T = 2^G_t S_n^T q_t over this slice's key rows.
        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) out[tb][0] = out[tb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8 a0 = state_frag(acc[2 * ks][0], acc[2 * ks + 1][0]);
            const bf16x8 a1 = state_frag(acc[2 * ks][1], acc[2 * ks + 1][1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 bq = load_row<TileQ>(sQ, 16 * tb, HALF * y + 32 * ks);
                out[tb][0] = mfma_bf16(a0, bq, out[tb][0]);
                out[tb][1] = mfma_bf16(a1, bq, out[tb][1]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const float f = sGam[64 + 16 * tb + lr] * sc.sig;
            out[tb][0] *= f;
            out[tb][1] *= f;
        }
        __syncthreads();  // scores complete, q tile done with
        if (n + 1 < n1) {
            issue_rows_stride(sq.k, sq.rk, p.T, t0 + 64, kraw);
            issue_half_rows(sq.v, sq.rv, t0 + 64, vraw);
        }
        // x_y^T += v^T P_y^T; wf[c][ss][jj] = v[32 ss + 8 lg + jj][32 mq + 16 c + lr].
        bf16x8 wf[2][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int ss = 0; ss < 2; ss++) wf[c][ss] = load_tr<TileW>(sW, 32 * ss, 32 * mq + 16 * c);
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int ss = 0; ss <= (tb >> 1); ss++) {
                const bf16x8 pf = load_row<TileP>(sPy, 16 * tb, 32 * ss);
                out[tb][0] = mfma_bf16(wf[0][ss], pf, out[tb][0]);
                out[tb][1] = mfma_bf16(wf[1][ss], pf, out[tb][1]);
            }
        bf16_t* sRy = y == 0 ? sR0 : sR1;
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
                *reinterpret_cast<bf16x4*>(sRy + (16 * tb + lr) * RR + 32 * mq + 16 * c + 4 * lg) =
                    to_bf16x4(out[tb][c], p.scale);
        // S = 2^G_last S + k^T bf16(2^(G_last - G_s) v), as acc += k^T bf16(2^(G_last - G_s) / sigma' v).
        if (sc.fold != 1.f) {
#pragma unroll
            for (int kb = 0; kb < 8; kb++) {
                acc[kb][0] *= sc.fold;
                acc[kb][1] *= sc.fold;
            }
        }
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            bf16x8 wt[2];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    wt[c][jj] = (bf16_t)((float)wf[c][ss][jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
#pragma unroll
            for (int kb = 0; kb < 8; kb++) {
                const bf16x8 kf = load_tr_perm<TileF>(sK, 32 * ss, HALF * y + 32 * (kb >> 1), kb & 1);
                acc[kb][0] = mfma_bf16(kf, wt[0], acc[kb][0]);
                acc[kb][1] = mfma_bf16(kf, wt[1], acc[kb][1]);
            }
        }
        sc.sig = sc.next;
        __syncthreads();  // both slices' outputs complete
        {
            float x[16];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(sR0 + r * RR + 16 * cq + 8 * hh);
                const bf16x8 c2 = *reinterpret_cast<const bf16x8*>(sR1 + r * RR + 16 * cq + 8 * hh);
#pragma unroll
                for (int e = 0; e < 8; e++) x[8 * hh + e] = (float)a[e] + (float)c2[e];
            }
            const uint32_t soff = (uint32_t)(t0 + r) * sq.ro;
            if (raw) {
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++)
                    st_b128(sq.o, 4 * (16 * cq + 4 * q4), soff, f32x4{x[4 * q4], x[4 * q4 + 1], x[4 * q4 + 2], x[4 * q4 + 3]});
            } else {
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    bf16x8 o8;
#pragma unroll
                    for (int e = 0; e < 8; e++) o8[e] = (bf16_t)x[8 * hh + e];
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o8), sq.o, 2 * (16 * cq + 8 * hh), soff, 0);
                }
            }
        }
        __syncthreads();  // tiles are overwritten by the next chunk
    }
    if (j == p.P - 1 && p.hfinal) {
        float* dst = p.hfinal + (size_t)bh * (KD * HALF);
#pragma unroll
        for (int kb = 0; kb < 8; kb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    dst[(HALF * y + state_row(kb, lg, i)) * HALF + 32 * mq + 16 * c + lr] = acc[kb][c][i] * sc.sig;
    }
}

// Shape B sweep (K = 128, V = 256), grid (H, B, P), 512 threads; wave w owns
// value columns [32 w, 32 w + 32) as pass 2 does.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void sla_sweep_b_kernel(SlaParams p) {
    __shared__ __align__(16) unsigned char smem[P2_N];
    bf16_t* sQh = reinterpret_cast<bf16_t*>(smem + P2_OM);  // q, TileO
    bf16_t* sK = reinterpret_cast<bf16_t*>(smem + P2_W);    // k, TileW
    bf16_t* sV = reinterpret_cast<bf16_t*>(smem + P2_V);    // v, TileF
    bf16_t* sP = reinterpret_cast<bf16_t*>(smem + P2_P);
    float* sLam = reinterpret_cast<float*>(smem + P2_G);
    float* sBeta = sLam + 64;
    float* sGam = sBeta + 64;
    const int h = blockIdx.x, b = blockIdx.y, j = blockIdx.z, bh = b * p.H + h;
    const int lane = threadIdx.x & 63, w = wave_id(), lr = lane & 15, lg = lane >> 4;
    const int n0 = j * p.L, n1 = min(n0 + p.L, p.N);
    const SlaSeq sq = make_sla_seq(p, b, h);
    const bool raw = p.raw_output != 0;
    const uint32_t osz = raw ? 4 : 2;
    const uint32_t o_lane = (uint32_t)lr * sq.ro + osz * (32 * w + 4 * lg);
    bf16x8 vraw[4], qraw[2], kraw[2];
    issue_rows_stride(sq.v, sq.rv, p.T, n0 * 64, vraw);
    issue_half_rows(sq.q, sq.rk, n0 * 64, qraw);
    issue_half_rows(sq.k, sq.rk, n0 * 64, kraw);
    float graw = ld_f32(sq.g, (uint32_t)(n0 * 64 + lane) * 4);
    zero_scores(sP, 1);
    f32x4 acc[8][2];
    sla_start_state(p, bh, j, [&](int mb, int c, int i) { return state_row(mb, lg, i) * VD + 32 * w + 16 * c + lr; },
                    acc);
    StateScale sc;
    for (int n = n0; n < n1; n++) {
        const int t0 = n * 64;
        const GateRegs gr = sla_gates(graw);
        sc.begin_chunk(chunk_last_gam(gr));
        commit_gates(p.T, t0, gr, sLam, sBeta, sGam, sc.inv());
        store_half_rows<TileO>(qraw, 64, sQh);
        store_half_rows<TileW>(kraw, 64, sK);
        store_rows<TileF>(vraw, 64, sV);
        __syncthreads();
        if (n + 1 < n1) {
            issue_half_rows(sq.q, sq.rk, t0 + 64, qraw);
            issue_half_rows(sq.k, sq.rk, t0 + 64, kraw);
            graw = ld_f32(sq.g, (uint32_t)(t0 + 64 + lane) * 4);
        }
        score_tile<TileO, TileW>(sQh, 0, sK, 0, w, sGam, 0.f, sP);
        if (w < 2) score_tile<TileO, TileW>(sQh, 0, sK, 0, w + 8, sGam, 0.f, sP);
        // o^T = 2^G_t S_n^T q_t.
        f32x4 out[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; tb++) out[tb][0] = out[tb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const bf16x8 a0 = state_frag(acc[2 * ks][0], acc[2 * ks + 1][0]);
            const bf16x8 a1 = state_frag(acc[2 * ks][1], acc[2 * ks + 1][1]);
#pragma unroll
            for (int tb = 0; tb < 4; tb++) {
                const bf16x8 bo = load_row<TileO>(sQh, 16 * tb, 32 * ks);
                out[tb][0] = mfma_bf16(a0, bo, out[tb][0]);
                out[tb][1] = mfma_bf16(a1, bo, out[tb][1]);
            }
        }
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const float f = sGam[64 + 16 * tb + lr] * sc.sig;
            out[tb][0] *= f;
            out[tb][1] *= f;
        }
        __syncthreads();  // scores complete
        if (n + 1 < n1) issue_rows_stride(sq.v, sq.rv, p.T, t0 + 64, vraw);
        // o^T += v^T P^T. vb[c][ss][jj] = v[32 ss + 8 lg + jj][32 w + 16 c + lr].
        bf16x8 vb[2][2];
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int ss = 0; ss < 2; ss++) vb[c][ss] = load_tr<TileF>(sV, 32 * ss, 32 * w + 16 * c);
#pragma unroll
        for (int tb = 0; tb < 4; tb++)
#pragma unroll
            for (int ss = 0; ss <= (tb >> 1); ss++) {
                const bf16x8 pf = load_row<TileP>(sP, 16 * tb, 32 * ss);
                out[tb][0] = mfma_bf16(vb[0][ss], pf, out[tb][0]);
                out[tb][1] = mfma_bf16(vb[1][ss], pf, out[tb][1]);
            }
#pragma unroll
        for (int tb = 0; tb < 4; tb++) {
            const uint32_t soff = (uint32_t)(t0 + 16 * tb) * sq.ro;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const bf16x4 o4 = to_bf16x4(out[tb][c], p.scale);
                if (raw)
                    st_b128(sq.o, o_lane + osz * 16 * c, soff, f32x4{(float)o4[0], (float)o4[1], (float)o4[2], (float)o4[3]});
                else
                    st_b64(sq.o, o_lane + osz * 16 * c, soff, o4);
            }
        }
        // S = 2^G_last S + k^T bf16(2^(G_last - G_s) v), as acc += k^T bf16(2^(G_last - G_s) / sigma' v).
        if (sc.fold != 1.f) {
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                acc[mb][0] *= sc.fold;
                acc[mb][1] *= sc.fold;
            }
        }
#pragma unroll
        for (int ss = 0; ss < 2; ss++) {
            bf16x8 vt[2];
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int jj = 0; jj < 8; jj++)
                    vt[c][jj] = (bf16_t)((float)vb[c][ss][jj] * sGam[128 + 32 * ss + 8 * lg + jj]);
#pragma unroll
            for (int mb = 0; mb < 8; mb++) {
                const bf16x8 kk = load_tr_perm<TileW>(sK, 32 * ss, 32 * (mb >> 1), mb & 1);
                acc[mb][0] = mfma_bf16(kk, vt[0], acc[mb][0]);
                acc[mb][1] = mfma_bf16(kk, vt[1], acc[mb][1]);
            }
        }
        sc.sig = sc.next;
        __syncthreads();
    }
    if (j == p.P - 1 && p.hfinal) {
        float* dst = p.hfinal + (size_t)bh * (HALF * VD);
#pragma unroll
        for (int mb = 0; mb < 8; mb++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) dst[state_row(mb, lg, i) * VD + 32 * w + 16 * c + lr] = acc[mb][c][i] * sc.sig;
    }
}

}  // namespace

int device_cu_count() {
    constexpr int kMaxDevices = 64;
    static int cached[kMaxDevices];  // 0 = not queried yet; every writer stores the same value
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();  // no device: clear the error, use the MI355X count
        return 256;
    }
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

void choose_segments(int BH, int N, int* P, int* L) {
    // One sweep workgroup per segment: aim for one workgroup per CU.
    // CYFA_SEGMENT_CHUNKS=<L> fixes the chunks per segment (tests, tuning).
    const int cus = device_cu_count();
    int target = (cus + BH - 1) / BH;
    if (target < 1) target = 1;
    if (target > N) target = N;
    int l = (N + target - 1) / target;
    if (const char* env = getenv("CYFA_SEGMENT_CHUNKS")) {
        const int forced = atoi(env);
        if (forced > 0) l = forced < N ? forced : N;
    }
    // At most kMaxSegments segments: the sweeps address the stored segment
    // states of a sequence with 32-bit offsets below 2^31.
    if ((N + l - 1) / l > kMaxSegments) l = (N + kMaxSegments - 1) / kMaxSegments;
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
    w.gam = align256(w.lam + BH * Tp * sizeof(float));
    w.seg = align256(w.gam + BH * Tp * sizeof(float));
    const size_t nseg = P > 1 ? BH * (P - 1) : 0;
    w.seg_exp = align256(w.seg + nseg * (size_t)(K * kSlots + kSlots * V) * sizeof(_Float16));
    w.seg_decay = align256(w.seg_exp + nseg * 16 * sizeof(int));
    w.omega = align256(w.seg_decay + BH * P * sizeof(float));
    w.tab_exp = align256(w.omega + BH * Tp * kSlots * 2);
    w.tab16 = align256(w.tab_exp + BH * sizeof(int));
    w.total = align256(w.tab16 + (size_t)H * kSlots * kSlots * sizeof(_Float16));
    return w;
}

int launch_prefill(const PrefillParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(segment_state_kernel, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    hipLaunchKernelGGL(pass1_kernel, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    if (p.on_w)
        hipLaunchKernelGGL(pass2_kernel<true>, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    else
        hipLaunchKernelGGL(pass2_kernel<false>, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    return 0;
}

SlaWorkspaceLayout sla_workspace_layout(int B, int T, int H, int K, int V) {
    SlaWorkspaceLayout w;
    const int N = (T + kChunk - 1) / kChunk;
    int P, L;
    choose_segments(B * H, N, &P, &L);
    const size_t BH = (size_t)B * H;
    const size_t nseg = P > 1 ? BH * (P - 1) : 0;
    w.seg = 0;
    w.seg_exp = align256(w.seg + nseg * (size_t)K * V * sizeof(_Float16));
    w.seg_decay = align256(w.seg_exp + nseg * 8 * sizeof(int));
    w.total = align256(w.seg_decay + BH * P * sizeof(float));
    return w;
}

int launch_scalar_la(const SlaParams& p, hipStream_t stream) {
    const bool a = p.K == KD;
    if (p.P > 1) {
        if (a)
            hipLaunchKernelGGL(sla_segment_kernel<true>, dim3(p.H, p.B, p.P - 1), dim3(512), 0, stream, p);
        else
            hipLaunchKernelGGL(sla_segment_kernel<false>, dim3(p.H, p.B, p.P - 1), dim3(512), 0, stream, p);
    }
    if (a)
        hipLaunchKernelGGL(sla_sweep_a_kernel, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    else
        hipLaunchKernelGGL(sla_sweep_b_kernel, dim3(p.H, p.B, p.P), dim3(512), 0, stream, p);
    return 0;
}

int launch_readout_table(const float* readout, float* table, int H, hipStream_t stream) {
    hipLaunchKernelGGL(readout_table_kernel, dim3(H * kActive), dim3(128), 0, stream, readout, table);
    return 0;
}

}  // namespace cyfa
