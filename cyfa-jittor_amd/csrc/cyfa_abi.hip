// cyfa_abi.hip -- extern "C" entry points of libcyfa_hip.so (declared in
// include/cyfa_abi.h). Validates arguments, maps them onto the kernel
// parameter blocks and launches on the caller's stream. No device memory is
// allocated here; the caller supplies every buffer, including the workspace.
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "cyfa_abi.h"
#include "cyfa_internal.h"

// Scratch of cyfa_chunk_fwd_noalloc: a device array each GPU holds from the
// library's load until the process ends. In host code `scratch` names a
// host-side stand-in, not device memory; its device address is resolved once
// per device with hipGetSymbolAddress (scratch_base) and only that address
// is handed to kernels.
static __device__ __align__(256) unsigned char scratch[CYFA_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return code;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(CYFA_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return CYFA_OK;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_base[kMaxDevices];  // device address of `scratch` per device, resolved on first use

// Device address of the scratch array on the device the launch stream belongs
// to (the current device for the null stream), resolved once per device with
// that device current (made current for the call and restored after it when
// the caller's current device is another one).
int scratch_base(hipStream_t stream, void** out, const char* what) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur < 0) {
        (void)hipGetLastError();
        return fail(CYFA_ERR_LAUNCH, "%s: no current HIP device", what);
    }
    int dev = cur;
    if (stream) {
        hipDevice_t d = -1;
        if (hipStreamGetDevice(stream, &d) != hipSuccess || d < 0) {
            (void)hipGetLastError();
            return fail(CYFA_ERR_LAUNCH, "%s: the stream's device is unknown", what);
        }
        dev = (int)d;
    }
    if (dev >= kMaxDevices) return fail(CYFA_ERR_LAUNCH, "%s: device %d beyond %d", what, dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_base[dev]) {
        if (dev != cur && hipSetDevice(dev) != hipSuccess) {
            (void)hipGetLastError();
            return fail(CYFA_ERR_LAUNCH, "%s: cannot make device %d current", what, dev);
        }
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(CYFA_ERR_LAUNCH, "%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", what,
                        dev, hipGetErrorString(e));
        }
        g_scratch_base[dev] = p;
    }
    *out = g_scratch_base[dev];
    return CYFA_OK;
}

}  // namespace

extern "C" {

int cyfa_abi_version(void) { return CYFA_ABI_VERSION; }

const char* cyfa_last_error(void) { return g_error; }

size_t cyfa_chunk_workspace_bytes(int B, int T, int H, int K, int V, int M, int C) {
    (void)M;
    (void)C;
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0) return 0;
    return cyfa::workspace_layout(B, T, H, K, V).total;
}

int cyfa_readout_table(const float* readout, float* table, int H, int M, void* hip_stream) {
    if (M < 4 || M > 256 || M % 2)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_readout_table: num_slots must be even and in [4, 256], got %d", M);
    if (H <= 0) return fail(CYFA_ERR_VALUE, "cyfa_readout_table: H must be positive, got %d", H);
    if (!readout || !table) return fail(CYFA_ERR_VALUE, "cyfa_readout_table: null pointer");
    if (M != 128) {  // the general path's table (any even M)
        if (cyfa::launch_general_table(readout, table, H, M, (hipStream_t)hip_stream) != 0)
            return fail(CYFA_ERR_UNSUPPORTED, "cyfa_readout_table: launch refused");
        return check_launch("cyfa_readout_table");
    }
    if (cyfa::launch_readout_table(readout, table, H, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_readout_table: launch refused");
    return check_launch("cyfa_readout_table");
}

namespace {

// f32: q, k, v and o are fp32 (cyfa_decode_step_general at the tuned shapes):
// the same kernels without the bf16 rounding points, one workgroup per (b, h).
int decode_step(const CyfaDecodeArgs* a, const CyfaDecodeLayerArgs* ly, void* hip_stream, bool f32 = false) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_decode_step: null args");
    if (a->M != 128) return fail(CYFA_ERR_UNSUPPORTED, "cyfa_decode_step: num_slots must be 128, got %d", a->M);
    if (!((a->K == 128 || a->K == 256) && (a->V == 128 || a->V == 256)))
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_decode_step: head dims K=%d V=%d not in {128, 256}", a->K, a->V);
    if (a->B <= 0 || a->H <= 0) return fail(CYFA_ERR_VALUE, "cyfa_decode_step: B=%d H=%d must be positive", a->B, a->H);
    if ((!ly && (!a->q || !a->k || !a->v || !a->g || !a->delta || !a->beta)) || !a->table || !a->q_norm_weight ||
        !a->k_norm_weight || !a->o || !a->hk_out || !a->hv_out || !a->clock_out)
        return fail(CYFA_ERR_VALUE, "cyfa_decode_step: null required pointer");
    if (ly) {
        if (a->K != 256 || a->V != 256)
            return fail(CYFA_ERR_UNSUPPORTED, "cyfa_decode_layer_step: head dims K=%d V=%d, the layer step needs 256",
                        a->K, a->V);
        if (!ly->qkv || !ly->conv_cache_out || !ly->conv_weight || !ly->abd || !ly->dt_bias || !ly->A_log ||
            !ly->norm_weight || (!ly->gate && (!ly->g0 || !ly->g_weight)))
            return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: null required pointer");
        const long long D = 3LL * a->H * 256;
        if (ly->qkv_row < D || ly->abd_row < 3LL * a->H || ly->cache_row < D || ly->cache_batch < 3 * ly->cache_row ||
            (ly->gate && (ly->gate_row < (long long)a->H * 256 || ly->gate_row % 4)) ||
            (!ly->gate && (ly->g0_row < 256 || ly->g0_row % 8)))
            return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: row strides too small or misaligned");
        if (!aligned(ly->gate, 8) || !aligned(ly->conv_weight, 8) || !aligned(ly->norm_weight, 16) ||
            (!ly->gate && (!aligned(ly->g0, 16) || !aligned(ly->g_weight, 16))))
            return fail(CYFA_ERR_ALIGN,
                        "cyfa_decode_layer_step: gate and conv_weight need 8-byte, norm_weight, g0 and g_weight "
                        "16-byte alignment");
        if (!(ly->norm_eps >= 0.f) || !isfinite(ly->norm_prescale))
            return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: norm_eps=%g prescale=%g", (double)ly->norm_eps,
                        (double)ly->norm_prescale);
    }
    const bool has_in = a->hk_in != nullptr;
    if (has_in != (a->hv_in != nullptr) || has_in != (a->clock_in != nullptr))
        return fail(CYFA_ERR_VALUE, "cyfa_decode_step: hk_in, hv_in and clock_in must be all set or all null");
    if ((!ly && !aligned(a->v, 8)) || !aligned(a->table, 16) || !aligned(a->hk_out, 16) || !aligned(a->hv_out, 16) ||
        (has_in && (!aligned(a->hk_in, 16) || !aligned(a->hv_in, 16))))
        return fail(CYFA_ERR_ALIGN, "cyfa_decode_step: states/table need 16-byte and v 8-byte alignment");
    cyfa::DecodeParams p{};
    p.B = a->B;
    p.H = a->H;
    p.q = (const __bf16*)a->q;
    p.k = (const __bf16*)a->k;
    p.v = (const __bf16*)a->v;
    p.g = a->g;
    p.delta = a->delta;
    p.beta = a->beta;
    p.table = a->table;
    p.q_w = a->q_norm_weight;
    p.k_w = a->k_norm_weight;
    p.q_eps = a->q_norm_eps;
    p.k_eps = a->k_norm_eps;
    p.scale = a->scale;
    p.hk_in = a->hk_in;
    p.hv_in = a->hv_in;
    p.clock_in = a->clock_in;
    p.o = (__bf16*)a->o;
    p.hk_out = a->hk_out;
    p.hv_out = a->hv_out;
    p.clock_out = a->clock_out;
    p.f32 = f32 ? 1 : 0;
    const size_t ws = cyfa::decode_workspace_bytes(a->B, a->H, a->K, a->V);
    if (!f32 && ws && a->workspace && a->workspace_bytes >= ws) {
        if (!aligned(a->workspace, 16)) return fail(CYFA_ERR_ALIGN, "cyfa_decode_step: workspace needs 16-byte alignment");
        p.part = (float*)a->workspace;
    }
    if (ly) {
        p.qkv = (const __bf16*)ly->qkv;
        p.qkv_row = ly->qkv_row;
        p.cache_in = (const __bf16*)ly->conv_cache;
        p.cache_out = (__bf16*)ly->conv_cache_out;
        p.cache_row = ly->cache_row;
        p.cache_batch = ly->cache_batch;
        p.conv_w = (const __bf16*)ly->conv_weight;
        p.abd = (const __bf16*)ly->abd;
        p.abd_row = ly->abd_row;
        p.dt_bias = ly->dt_bias;
        p.A_log = ly->A_log;
        p.gate = (const __bf16*)ly->gate;
        p.gate_row = ly->gate_row;
        if (!ly->gate) {
            p.g0 = (const __bf16*)ly->g0;
            p.g0_row = ly->g0_row;
            p.g1_w = (const __bf16*)ly->g_weight;
            p.g1_b = (const __bf16*)ly->g_bias;
        }
        p.on_w = ly->norm_weight;
        p.on_eps = ly->norm_eps;
        p.on_prescale = ly->norm_prescale;
        // Prefetch: at most CYFA_PREFETCH_MAX_BH step workgroups, the
        // one-workgroup form, and workgroups on the compute units it leaves idle.
        unsigned long long pf_total = 0;
        for (int r = 0; r < CYFA_PREFETCH_RANGES; r++) {
            const unsigned long long n = ly->prefetch_bytes[r];
            if (n == 0) continue;
            if (!ly->prefetch[r] || n >= (1ull << 31))
                return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: prefetch range %d: null or %llu bytes (below 2^31)",
                            r, n);
            if (!aligned(ly->prefetch[r], 16))
                return fail(CYFA_ERR_ALIGN, "cyfa_decode_layer_step: prefetch range %d needs 16-byte alignment", r);
            const unsigned long long span = ly->prefetch_span[r];
            if (span % 16 != 0 || span >= (1ull << 31))
                return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: prefetch range %d: span %llu (a multiple of 16 "
                            "below 2^31)", r, span);
            pf_total += n;
        }
        const long long bh = (long long)a->B * a->H;
        // Several step workgroups per (b, h) at small batches, each storing its
        // share: only with every output apart from its input (in place, one
        // workgroup's stores could reach another's loads)
        const bool apart = p.hk_out != p.hk_in && p.hv_out != p.hv_in && p.clock_out != p.clock_in &&
                           (!p.cache_in || (const void*)p.cache_in != (const void*)p.cache_out);
        p.wpb = apart && !p.part ? (bh <= cyfa::DECODE_WPB4_MAX_BH ? 4 : bh <= cyfa::DECODE_WPB2_MAX_BH ? 2 : 1) : 1;
        const long long steps = bh * p.wpb;
        const int idle = cyfa::device_cu_count() - (int)(steps < 1 << 20 ? steps : 1 << 20);
        p.self_pf = bh <= cyfa::DECODE_SELF_PREFETCH_MAX_BH && !p.part && idle > 0;
        if ((pf_total || p.self_pf) && bh <= CYFA_PREFETCH_MAX_BH && !p.part && idle > 0) {
            for (int r = 0; r < CYFA_PREFETCH_RANGES; r++) {
                p.pf[r] = ly->prefetch[r];
                p.pf_bytes[r] = ly->prefetch_bytes[r];
                p.pf_span[r] = ly->prefetch_span[r];
            }
            // every idle compute unit for the self-prefetch (each XCD gets its share)
            const unsigned long long units = p.self_pf ? (unsigned long long)idle : (pf_total + 16383) >> 14;
            p.pf_wgs = (int)(units < (unsigned long long)idle ? units : (unsigned long long)idle);
        }
    }
    if (cyfa::launch_decode_step(p, a->K, a->V, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_decode_step: no kernel for K=%d V=%d", a->K, a->V);
    return check_launch(ly ? "cyfa_decode_layer_step" : "cyfa_decode_step");
}

}  // namespace

int cyfa_decode_step(const CyfaDecodeArgs* a, void* hip_stream) { return decode_step(a, nullptr, hip_stream); }

size_t cyfa_decode_workspace_bytes(int B, int H, int K, int V) {
    if (!((K == 128 || K == 256) && (V == 128 || V == 256))) return 0;
    return cyfa::decode_workspace_bytes(B, H, K, V);
}

int cyfa_decode_layer_step(const CyfaDecodeArgs* a, const CyfaDecodeLayerArgs* layer, void* hip_stream) {
    if (!layer) return fail(CYFA_ERR_VALUE, "cyfa_decode_layer_step: null layer args");
    return decode_step(a, layer, hip_stream);
}

namespace {

// use_scratch: the workspace is the device's scratch array (args->workspace
// and args->workspace_bytes are ignored).
int chunk_fwd(const CyfaChunkArgs* a, const CyfaOutNormArgs* on, void* hip_stream, bool use_scratch = false) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: null args");
    if (a->M != 128) return fail(CYFA_ERR_UNSUPPORTED, "cyfa_chunk_fwd: num_slots must be 128, got %d", a->M);
    if (a->C != 64) return fail(CYFA_ERR_UNSUPPORTED, "cyfa_chunk_fwd: chunk_size must be 64, got %d", a->C);
    if (a->K != 256 || a->V != 256)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_chunk_fwd: head dims K=%d V=%d, the prefill kernels need 256", a->K,
                    a->V);
    if (a->B <= 0 || a->T <= 0 || a->H <= 0)
        return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: B=%d T=%d H=%d must be positive", a->B, a->T, a->H);
    if (!a->q || !a->k || !a->v || !a->g || !a->delta || !a->beta || !a->table || !a->q_norm_weight ||
        !a->k_norm_weight || !a->o)
        return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: null required pointer");
    // The kernels address a sequence's rows with 32-bit byte offsets.
    if ((size_t)a->T * a->H * a->K * 2 > cyfa::MAX_SPAN_BYTES)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_chunk_fwd: T * H * K * 2 = %zu bytes per sequence exceeds 2^32 - 1",
                    (size_t)a->T * a->H * a->K * 2);
    if (!(a->scale > 0.f) || !isfinite(a->scale))
        return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: scale must be positive and finite, got %g", (double)a->scale);
    const bool has_h0 = a->h0_k != nullptr;
    if (has_h0 != (a->h0_v != nullptr) || has_h0 != (a->clock0 != nullptr))
        return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: h0_k, h0_v and clock0 must be all set or all null");
    const bool has_out = a->hk != nullptr;
    if (has_out != (a->hv != nullptr) || has_out != (a->clock != nullptr))
        return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd: hk, hv and clock must be all set or all null");
    if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->o, 16) ||
        !aligned(a->q_norm_weight, 16) || !aligned(a->k_norm_weight, 16) ||
        (has_h0 && (!aligned(a->h0_k, 16) || !aligned(a->h0_v, 16))))
        return fail(CYFA_ERR_ALIGN, "cyfa_chunk_fwd: q/k/v/o, norm weights and states need 16-byte alignment");
    const cyfa::WorkspaceLayout ws = cyfa::workspace_layout(a->B, a->T, a->H, a->K, a->V);
    void* workspace = a->workspace;
    if (use_scratch) {
        if (ws.total > CYFA_NOALLOC_SCRATCH_BYTES)
            return fail(CYFA_ERR_UNSUPPORTED,
                        "cyfa_chunk_fwd_noalloc: B=%d T=%d H=%d needs %zu bytes of scratch; the array holds %llu "
                        "(call cyfa_chunk_fwd with a workspace instead)",
                        a->B, a->T, a->H, ws.total, (unsigned long long)CYFA_NOALLOC_SCRATCH_BYTES);
    } else {
        if (!workspace || a->workspace_bytes < ws.total)
            return fail(CYFA_ERR_WORKSPACE, "cyfa_chunk_fwd: workspace of %zu bytes needed, got %zu", ws.total,
                        workspace ? a->workspace_bytes : (size_t)0);
        if (!aligned(workspace, 256)) return fail(CYFA_ERR_ALIGN, "cyfa_chunk_fwd: workspace needs 256-byte alignment");
    }
    if (on) {
        if (!on->weight || !on->gate) return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd_normed: null weight or gate");
        if (!aligned(on->weight, 16) || !aligned(on->gate, 16))
            return fail(CYFA_ERR_ALIGN, "cyfa_chunk_fwd_normed: weight and gate need 16-byte alignment");
        if (!(on->eps >= 0.f) || !isfinite(on->eps) || !isfinite(on->prescale))
            return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd_normed: eps=%g prescale=%g", (double)on->eps,
                        (double)on->prescale);
    }

    cyfa::PrefillParams p{};
    p.B = a->B;
    p.T = a->T;
    p.H = a->H;
    p.K = a->K;
    p.V = a->V;
    p.N = (a->T + 63) / 64;
    p.Tp = p.N * 64;
    cyfa::choose_segments(p.B * p.H, p.N, &p.P, &p.L);
    p.q = (const __bf16*)a->q;
    p.k = (const __bf16*)a->k;
    p.v = (const __bf16*)a->v;
    p.g = a->g;
    p.delta = a->delta;
    p.beta = a->beta;
    p.table = a->table;
    p.q_w = a->q_norm_weight;
    p.k_w = a->k_norm_weight;
    p.q_eps = a->q_norm_eps;
    p.k_eps = a->k_norm_eps;
    p.scale = a->scale;
    p.log2_scale = log2f(a->scale);
    p.h0_k = a->h0_k;
    p.h0_v = a->h0_v;
    p.clock0 = a->clock0;
    p.o = (__bf16*)a->o;
    p.hk = a->hk;
    p.hv = a->hv;
    p.clock = a->clock;
    p.on_w = on ? on->weight : nullptr;
    p.on_gate = on ? (const __bf16*)on->gate : nullptr;
    p.on_eps = on ? on->eps : 0.f;
    p.on_prescale = on ? on->prescale : 1.f;
    if (use_scratch) {
        if (int rc = scratch_base((hipStream_t)hip_stream, &workspace, "cyfa_chunk_fwd_noalloc")) return rc;
    }
    char* base = (char*)workspace;
    p.lam = (float*)(base + ws.lam);
    p.gam = (float*)(base + ws.gam);
    p.seg = (_Float16*)(base + ws.seg);
    p.seg_exp = (int*)(base + ws.seg_exp);
    p.seg_decay = (float*)(base + ws.seg_decay);
    p.omega = (__bf16*)(base + ws.omega);
    p.tab_exp = (int*)(base + ws.tab_exp);
    p.tab16 = (_Float16*)(base + ws.tab16);
    if (cyfa::launch_prefill(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_chunk_fwd: launch refused");
    return check_launch(on ? "cyfa_chunk_fwd_normed" : "cyfa_chunk_fwd");
}

}  // namespace

int cyfa_chunk_fwd(const CyfaChunkArgs* a, void* hip_stream) { return chunk_fwd(a, nullptr, hip_stream); }

int cyfa_chunk_fwd_normed(const CyfaChunkArgs* a, const CyfaOutNormArgs* norm, void* hip_stream) {
    if (!norm) return fail(CYFA_ERR_VALUE, "cyfa_chunk_fwd_normed: null norm args");
    return chunk_fwd(a, norm, hip_stream);
}

int cyfa_chunk_fwd_noalloc(const CyfaChunkArgs* a, const CyfaOutNormArgs* norm, void* hip_stream) {
    return chunk_fwd(a, norm, hip_stream, true);
}

size_t cyfa_scalar_la_workspace_bytes(int B, int T, int H, int K, int V) {
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0) return 0;
    return cyfa::sla_workspace_layout(B, T, H, K, V).total;
}

int cyfa_scalar_la(const CyfaSlaArgs* a, void* hip_stream) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_scalar_la: null args");
    if (!((a->K == 256 && a->V == 128) || (a->K == 128 && a->V == 256)))
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_scalar_la: (K, V) = (%d, %d), supported are (256, 128) and (128, 256)",
                    a->K, a->V);
    if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->T % 64 != 0)
        return fail(CYFA_ERR_VALUE, "cyfa_scalar_la: B=%d H=%d must be positive and T=%d a positive multiple of 64",
                    a->B, a->H, a->T);
    if (!a->q || !a->k || !a->v || !a->g || !a->o) return fail(CYFA_ERR_VALUE, "cyfa_scalar_la: null required pointer");
    {  // the kernels address a sequence's rows with 32-bit byte offsets
        const size_t T = (size_t)a->T, osz = a->raw_output ? 4 : 2;
        const size_t span_k = T * a->K * 2;
        const size_t span_v = T * (a->v_bth ? a->H : 1) * a->V * 2;
        const size_t span_o = T * (a->output_bth ? a->H : 1) * a->V * osz;
        const size_t span = span_k > span_v ? (span_k > span_o ? span_k : span_o) : (span_v > span_o ? span_v : span_o);
        if (span > cyfa::MAX_SPAN_BYTES)
            return fail(CYFA_ERR_UNSUPPORTED, "cyfa_scalar_la: a sequence spans %zu bytes, above 2^32 - 1", span);
    }
    if (!isfinite(a->scale)) return fail(CYFA_ERR_VALUE, "cyfa_scalar_la: scale must be finite, got %g", (double)a->scale);
    if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->o, 16))
        return fail(CYFA_ERR_ALIGN, "cyfa_scalar_la: q/k/v/o need 16-byte alignment");
    if (!aligned(a->g, 4) || (a->initial && !aligned(a->initial, 4)) || (a->final_state && !aligned(a->final_state, 4)))
        return fail(CYFA_ERR_ALIGN, "cyfa_scalar_la: g and the states need 4-byte alignment");
    const cyfa::SlaWorkspaceLayout ws = cyfa::sla_workspace_layout(a->B, a->T, a->H, a->K, a->V);
    if (!a->workspace || a->workspace_bytes < ws.total)
        return fail(CYFA_ERR_WORKSPACE, "cyfa_scalar_la: workspace of %zu bytes needed, got %zu", ws.total,
                    a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned(a->workspace, 256)) return fail(CYFA_ERR_ALIGN, "cyfa_scalar_la: workspace needs 256-byte alignment");
    cyfa::SlaParams p{};
    p.B = a->B;
    p.T = a->T;
    p.H = a->H;
    p.K = a->K;
    p.V = a->V;
    p.N = a->T / 64;
    cyfa::choose_segments(p.B * p.H, p.N, &p.P, &p.L);
    p.q = (const __bf16*)a->q;
    p.k = (const __bf16*)a->k;
    p.v = (const __bf16*)a->v;
    p.g = a->g;
    p.h0 = a->initial;
    p.scale = a->scale;
    p.v_bth = a->v_bth != 0;
    p.o_bth = a->output_bth != 0;
    p.raw_output = a->raw_output != 0;
    p.o = a->o;
    p.hfinal = a->final_state;
    char* base = (char*)a->workspace;
    p.seg = (_Float16*)(base + ws.seg);
    p.seg_exp = (int*)(base + ws.seg_exp);
    p.seg_decay = (float*)(base + ws.seg_decay);
    if (cyfa::launch_scalar_la(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_scalar_la: launch refused");
    return check_launch("cyfa_scalar_la");
}

static int linear_params(const CyfaLinearArgs* a, const char* name, cyfa::LinearParams& p) {
    if (!a) return fail(CYFA_ERR_VALUE, "%s: null args", name);
    if (a->M < 1 || a->M > 64 || a->N < 1 || a->K < 32 || a->K % 32 != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: M=%d N=%d K=%d (needs 1 <= M <= 64, K a multiple of 32)", name, a->M,
                    a->N, a->K);
    if (!a->x || !a->weight || !a->y) return fail(CYFA_ERR_VALUE, "%s: null required pointer", name);
    if (a->swiglu && (a->bias || a->N % 32 != 0))
        return fail(CYFA_ERR_VALUE, "%s: swiglu needs N a multiple of 32 and no bias", name);
    if (a->ldx < a->K || a->ldx % 8 != 0 || a->ldy < (a->swiglu ? a->N / 2 : a->N))
        return fail(CYFA_ERR_VALUE, "%s: ldx=%lld ldy=%lld", name, a->ldx, a->ldy);
    if (!aligned(a->x, 16) || !aligned(a->weight, 16) || !aligned(a->y, 2) || (a->bias && !aligned(a->bias, 2)))
        return fail(CYFA_ERR_ALIGN, "%s: x and weight need 16-byte alignment", name);
    if (a->residual && (a->swiglu || a->ldr < a->N || !aligned(a->residual, 2)))
        return fail(CYFA_ERR_VALUE, "%s: residual needs no swiglu and ldr >= N (ldr=%lld)", name, a->ldr);
    p = cyfa::LinearParams{};
    p.M = a->M;
    p.N = a->N;
    p.K = a->K;
    p.x = (const __bf16*)a->x;
    p.ldx = a->ldx;
    p.w = (const __bf16*)a->weight;
    p.bias = (const __bf16*)a->bias;
    p.y = (__bf16*)a->y;
    p.ldy = a->ldy;
    p.swiglu = a->swiglu != 0;
    p.add = (const __bf16*)a->residual;
    p.ld_add = a->ldr;
    static_assert(CYFA_LINEAR_PREFETCH_RANGES == cyfa::LINEAR_PREFETCH_RANGES, "prefetch ranges");
    for (int r = 0; r < CYFA_LINEAR_PREFETCH_RANGES; r++) {
        const unsigned long long n = a->prefetch_bytes[r], span = a->prefetch_span[r];
        if (n == 0) continue;
        if (!a->prefetch[r] || n >= (1ull << 31))
            return fail(CYFA_ERR_VALUE, "%s: prefetch range %d: null or %llu bytes (below 2^31)", name, r, n);
        if (!aligned(a->prefetch[r], 16))
            return fail(CYFA_ERR_ALIGN, "%s: prefetch range %d needs 16-byte alignment", name, r);
        if (span % 16 != 0 || span >= (1ull << 31))
            return fail(CYFA_ERR_VALUE, "%s: prefetch range %d: span %llu (a multiple of 16 below 2^31)", name, r,
                        span);
        p.pf[r] = a->prefetch[r];
        p.pf_bytes[r] = n;
        p.pf_span[r] = span;
    }
    return CYFA_OK;
}


int cyfa_linear_rows(const CyfaLinearArgs* a, void* hip_stream) {
    cyfa::LinearParams p;
    if (int rc = linear_params(a, "cyfa_linear_rows", p)) return rc;
    if (cyfa::launch_linear_rows(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_linear_rows: no tile for M=%d N=%d K=%d", a->M, a->N, a->K);
    return check_launch("cyfa_linear_rows");
}

size_t cyfa_linear_rows_span(int M, int N, int K, int swiglu, int norm) {
    return norm < 0 || norm > 2 ? 0 : cyfa::linear_rows_span(M, N, K, swiglu != 0, norm);
}

int cyfa_norm_linear_rows(const CyfaLinearArgs* a, const CyfaRowNormArgs* n, void* hip_stream) {
    cyfa::LinearParams p;
    if (int rc = linear_params(a, "cyfa_norm_linear_rows", p)) return rc;
    if (!n) return fail(CYFA_ERR_VALUE, "cyfa_norm_linear_rows: null norm args");
    if (a->K > cyfa::LINEAR_NORM_MAX_K)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_norm_linear_rows: K=%d above %d", a->K, cyfa::LINEAR_NORM_MAX_K);
    if (n->weight && !aligned(n->weight, 16))
        return fail(CYFA_ERR_ALIGN, "cyfa_norm_linear_rows: norm weight needs 16-byte alignment");
    if (n->residual) {
        if (!n->sum_out) return fail(CYFA_ERR_VALUE, "cyfa_norm_linear_rows: residual without sum_out");
        if (n->ldr < a->K || n->ldr % 8 != 0)
            return fail(CYFA_ERR_VALUE, "cyfa_norm_linear_rows: ldr=%lld", n->ldr);
        if (!aligned(n->residual, 16) || !aligned(n->sum_out, 16))
            return fail(CYFA_ERR_ALIGN, "cyfa_norm_linear_rows: residual and sum_out need 16-byte alignment");
    }
    p.norm_weight = n->weight;
    p.norm_folded = n->weight ? 0 : 1;  // NULL: the norm weight is folded into the projection's weight
    p.norm_eps = n->eps;
    p.norm_residual = (const __bf16*)n->residual;
    p.norm_sum_out = n->residual ? (__bf16*)n->sum_out : nullptr;
    p.ldr = n->ldr;
    if (cyfa::launch_linear_rows(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_norm_linear_rows: no tile for M=%d N=%d K=%d", a->M, a->N, a->K);
    return check_launch("cyfa_norm_linear_rows");
}

int cyfa_rms_norm(const CyfaNormArgs* a, void* hip_stream) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_rms_norm: null args");
    if (a->rows < 0 || a->D <= 0) return fail(CYFA_ERR_VALUE, "cyfa_rms_norm: rows=%d D=%d", a->rows, a->D);
    if (a->D % 256 != 0 || a->D > 2048 || (a->D / 256 & (a->D / 256 - 1)) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_rms_norm: D=%d must be 256, 512, 1024 or 2048", a->D);
    if (!a->x || !a->weight || !a->out || (a->residual && !a->sum_out))
        return fail(CYFA_ERR_VALUE, "cyfa_rms_norm: null required pointer");
    if (!aligned(a->x, 8) || !aligned(a->out, 8) || !aligned(a->weight, 16) || (a->residual && !aligned(a->residual, 8)) ||
        (a->sum_out && !aligned(a->sum_out, 8)) || (a->gate && !aligned(a->gate, 8)))
        return fail(CYFA_ERR_ALIGN, "cyfa_rms_norm: bf16 rows need 8-byte and the weight 16-byte alignment");
    if (a->rows == 0) return CYFA_OK;
    cyfa::NormParams p;
    p.rows = a->rows;
    p.D = a->D;
    p.x = (const __bf16*)a->x;
    p.residual = (const __bf16*)a->residual;
    p.sum_out = (__bf16*)a->sum_out;
    p.weight = a->weight;
    p.gate = (const __bf16*)a->gate;
    p.eps = a->eps;
    p.prescale = a->prescale;
    p.out = (__bf16*)a->out;
    if (cyfa::launch_rms_norm(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_rms_norm: D=%d", a->D);
    return check_launch("cyfa_rms_norm");
}

int cyfa_short_conv(const CyfaConvArgs* a, void* hip_stream) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_short_conv: null args");
    if (a->B < 0 || a->T < 0 || a->D <= 0 || a->split <= 0)
        return fail(CYFA_ERR_VALUE, "cyfa_short_conv: B=%d T=%d D=%d split=%d", a->B, a->T, a->D, a->split);
    if (a->W < 2 || a->W > 4) return fail(CYFA_ERR_UNSUPPORTED, "cyfa_short_conv: width %d not in 2..4", a->W);
    if (a->D % 8 != 0 || a->split % 8 != 0 || a->D % a->split != 0 || a->D / a->split > 3)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_short_conv: D=%d split=%d (multiples of 8, at most 3 outputs)", a->D,
                    a->split);
    if (!a->x || !a->weight) return fail(CYFA_ERR_VALUE, "cyfa_short_conv: null required pointer");
    for (int i = 0; i < a->D / a->split; i++)
        if (!a->out[i] || !aligned(a->out[i], 16)) return fail(CYFA_ERR_ALIGN, "cyfa_short_conv: output %d null or misaligned", i);
    if (!aligned(a->x, 16) || a->x_row % 8 != 0 || (a->cache && (!aligned(a->cache, 16) || a->cache_row % 8 || a->cache_batch % 8)) ||
        (a->cache_out && (!aligned(a->cache_out, 16) || a->cache_out_row % 8 || a->cache_out_batch % 8)))
        return fail(CYFA_ERR_ALIGN, "cyfa_short_conv: inputs need 16-byte aligned rows");
    if (a->cache_out && a->cache_out == a->cache && a->T > 32)
        return fail(CYFA_ERR_VALUE, "cyfa_short_conv: in-place cache update needs T <= 32, got %d", a->T);
    if (a->B == 0 || a->T == 0) return CYFA_OK;
    cyfa::ConvParams p;
    p.B = a->B;
    p.T = a->T;
    p.D = a->D;
    p.W = a->W;
    p.x = (const __bf16*)a->x;
    p.x_row = a->x_row;
    p.cache = (const __bf16*)a->cache;
    p.cache_row = a->cache_row;
    p.cache_batch = a->cache_batch;
    p.weight = (const __bf16*)a->weight;
    p.bias = (const __bf16*)a->bias;
    for (int i = 0; i < 3; i++) p.out[i] = (__bf16*)a->out[i];
    p.split = a->split;
    p.cache_out = (__bf16*)a->cache_out;
    p.cache_out_row = a->cache_out_row;
    p.cache_out_batch = a->cache_out_batch;
    if (cyfa::launch_short_conv(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_short_conv: W=%d", a->W);
    return check_launch("cyfa_short_conv");
}

int cyfa_silu_mul(const void* gu, void* out, int rows, int F, void* hip_stream) {
    if (!gu || !out || rows < 0 || F <= 0) return fail(CYFA_ERR_VALUE, "cyfa_silu_mul: bad arguments");
    if (F % 8 != 0) return fail(CYFA_ERR_UNSUPPORTED, "cyfa_silu_mul: F=%d must be a multiple of 8", F);
    if (!aligned(gu, 16) || !aligned(out, 16)) return fail(CYFA_ERR_ALIGN, "cyfa_silu_mul: 16-byte alignment needed");
    if (rows == 0) return CYFA_OK;
    if (cyfa::launch_silu_mul((const __bf16*)gu, (__bf16*)out, rows, F, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_silu_mul: launch refused");
    return check_launch("cyfa_silu_mul");
}

int cyfa_argmax_rows(const void* x, long long ldx, int rows, int n, long long* out, void* hip_stream) {
    if (!x || !out || rows < 0 || n <= 0 || ldx < n || ldx % 8 != 0)
        return fail(CYFA_ERR_VALUE, "cyfa_argmax_rows: rows=%d n=%d ldx=%lld", rows, n, ldx);
    if (!aligned(x, 16) || !aligned(out, 8)) return fail(CYFA_ERR_ALIGN, "cyfa_argmax_rows: x needs 16-byte alignment");
    if (rows == 0) return CYFA_OK;
    if (cyfa::launch_argmax_rows((const __bf16*)x, ldx, rows, n, out, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_argmax_rows: launch refused");
    return check_launch("cyfa_argmax_rows");
}

int cyfa_gate_path(const CyfaGatePathArgs* a, void* hip_stream) {
    if (!a) return fail(CYFA_ERR_VALUE, "cyfa_gate_path: null args");
    if (a->M < 0 || a->K <= 0 || a->H <= 0 || a->Dv <= 0 || a->ldx < a->K || a->ldg < a->Dv)
        return fail(CYFA_ERR_VALUE, "cyfa_gate_path: M=%d K=%d H=%d Dv=%d ldx=%lld ldg=%lld", a->M, a->K, a->H, a->Dv,
                    a->ldx, a->ldg);
    if (a->K % 64 || a->K > cyfa::GATE_PATH_MAX_K || 3 * a->H > 32 || a->Dv % 256 || a->Dv > cyfa::GATE_PATH_MAX_DV)
        return fail(CYFA_ERR_UNSUPPORTED,
                    "cyfa_gate_path: K=%d (a multiple of 64, <= %d), H=%d (3H <= 32), Dv=%d (a multiple of 256, <= %d)",
                    a->K, cyfa::GATE_PATH_MAX_K, a->H, a->Dv, cyfa::GATE_PATH_MAX_DV);
    if (!a->x || !a->w1 || !a->abd_bias || !a->w2 || !a->dt_bias || !a->A_log || !a->gate || !a->g || !a->beta ||
        !a->delta)
        return fail(CYFA_ERR_VALUE, "cyfa_gate_path: null required pointer");
    if (a->ldx % 8 || a->ldg % 8) return fail(CYFA_ERR_VALUE, "cyfa_gate_path: ldx, ldg must be multiples of 8");
    if (!aligned(a->x, 16) || !aligned(a->w1, 16) || !aligned(a->w2, 16) || !aligned(a->gate, 16))
        return fail(CYFA_ERR_ALIGN, "cyfa_gate_path: x, w1, w2 and gate need 16-byte alignment");
    if (a->M == 0) return CYFA_OK;
    cyfa::GatePathParams p;
    p.M = a->M;
    p.K = a->K;
    p.H = a->H;
    p.Dv = a->Dv;
    p.x = (const __bf16*)a->x;
    p.ldx = a->ldx;
    p.w1 = (const __bf16*)a->w1;
    p.abd_bias = (const __bf16*)a->abd_bias;
    p.w2 = (const __bf16*)a->w2;
    p.b2 = (const __bf16*)a->b2;
    p.dt_bias = a->dt_bias;
    p.A_log = a->A_log;
    p.gate = (__bf16*)a->gate;
    p.ldg = a->ldg;
    p.g = a->g;
    p.beta = a->beta;
    p.delta = a->delta;
    if (cyfa::launch_gate_path(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_gate_path: shape refused");
    return check_launch("cyfa_gate_path");
}

int cyfa_gates(const void* abd, long long abd_row, const float* dt_bias, const float* A_log, float* g, float* beta,
               float* delta, int rows, int H, void* hip_stream) {
    if (!abd || !dt_bias || !A_log || !g || !beta || !delta || rows < 0 || H <= 0 || abd_row < 3LL * H)
        return fail(CYFA_ERR_VALUE, "cyfa_gates: bad arguments");
    if (rows == 0) return CYFA_OK;
    if (cyfa::launch_gates((const __bf16*)abd, abd_row, dt_bias, A_log, g, beta, delta, rows, H, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "cyfa_gates: launch refused");
    return check_launch("cyfa_gates");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The general-shape path (cyfa_general.hip).

size_t cyfa_chunk_general_workspace_bytes(int B, int T, int H, int K, int V, int M, int C) {
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || M <= 0 || C <= 0) return 0;
    return cyfa::general_workspace(B, T, H, K, V, M, nullptr).bytes;
}

namespace {

// Shape limits of the general path, shared by the chunk and decode entries.
int general_shape(const char* fn, int B, int H, int K, int V, int M, int dtype) {
    if (dtype != CYFA_DTYPE_BF16 && dtype != CYFA_DTYPE_F32)
        return fail(CYFA_ERR_VALUE, "%s: dtype must be CYFA_DTYPE_BF16 or CYFA_DTYPE_F32, got %d", fn, dtype);
    if (B <= 0 || H <= 0) return fail(CYFA_ERR_VALUE, "%s: B=%d H=%d must be positive", fn, B, H);
    if (K < 1 || K > 1024 || V < 1 || V > 1024)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: head dims K=%d V=%d must lie in [1, 1024]", fn, K, V);
    if (M < 4 || M > 256 || M % 2)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: num_slots must be even and in [4, 256], got %d", fn, M);
    return 0;
}

}  // namespace

int cyfa_chunk_fwd_general(const CyfaChunkArgs* a, int dtype, void* hip_stream) {
    const char* fn = "cyfa_chunk_fwd_general";
    if (!a) return fail(CYFA_ERR_VALUE, "%s: null args", fn);
    if (int rc = general_shape(fn, a->B, a->H, a->K, a->V, a->M, dtype)) return rc;
    if (a->T <= 0) return fail(CYFA_ERR_VALUE, "%s: T=%d must be positive", fn, a->T);
    if (!(a->C == 16 || a->C == 32 || a->C == 64))
        return fail(CYFA_ERR_UNSUPPORTED, "%s: chunk_size must be 16, 32 or 64, got %d", fn, a->C);
    if (!a->q || !a->k || !a->v || !a->g || !a->delta || !a->beta || !a->table || !a->q_norm_weight ||
        !a->k_norm_weight || !a->o)
        return fail(CYFA_ERR_VALUE, "%s: null required pointer", fn);
    if (!(a->scale > 0.f) || !isfinite(a->scale))
        return fail(CYFA_ERR_VALUE, "%s: scale must be positive and finite, got %g", fn, (double)a->scale);
    const bool has_h0 = a->h0_k != nullptr;
    if (has_h0 != (a->h0_v != nullptr) || has_h0 != (a->clock0 != nullptr))
        return fail(CYFA_ERR_VALUE, "%s: h0_k, h0_v and clock0 must be all set or all null", fn);
    const bool has_out = a->hk != nullptr;
    if (has_out != (a->hv != nullptr) || has_out != (a->clock != nullptr))
        return fail(CYFA_ERR_VALUE, "%s: hk, hv and clock must be all set or all null", fn);
    // the kernels index rows (b, h, padded t) and their elements with 32-bit
    // counts, and the state scans take one grid row per (b, h)
    const size_t Tp = (size_t)(a->T + cyfa::GEN_CHUNK - 1) / cyfa::GEN_CHUNK * cyfa::GEN_CHUNK;
    const size_t rows = (size_t)a->B * a->H * Tp;
    if (rows * 256 >= ((size_t)1 << 31))
        return fail(CYFA_ERR_UNSUPPORTED, "%s: B * H * padded T = %zu rows is too many", fn, rows);
    if ((size_t)a->B * a->H > 65535)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: B * H = %zu is above 65535", fn, (size_t)a->B * a->H);
    const size_t need = cyfa::general_workspace(a->B, a->T, a->H, a->K, a->V, a->M, nullptr).bytes;
    if (!a->workspace || a->workspace_bytes < need)
        return fail(CYFA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", fn, need,
                    a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned(a->workspace, 256)) return fail(CYFA_ERR_ALIGN, "%s: workspace needs 256-byte alignment", fn);
    cyfa::GenChunkParams g{};
    g.B = a->B;
    g.T = a->T;
    g.H = a->H;
    g.K = a->K;
    g.V = a->V;
    g.M = a->M;
    g.C = a->C;
    g.bf16 = dtype == CYFA_DTYPE_BF16;
    g.q = a->q;
    g.k = a->k;
    g.v = a->v;
    g.g = a->g;
    g.delta = a->delta;
    g.beta = a->beta;
    g.table = a->table;
    g.q_w = a->q_norm_weight;
    g.k_w = a->k_norm_weight;
    g.q_eps = a->q_norm_eps;
    g.k_eps = a->k_norm_eps;
    g.scale = a->scale;
    g.h0_k = a->h0_k;
    g.h0_v = a->h0_v;
    g.clock0 = a->clock0;
    g.o = a->o;
    g.hk = a->hk;
    g.hv = a->hv;
    g.clock = a->clock;
    g.workspace = a->workspace;
    if (cyfa::launch_general_chunk(g, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: launch refused", fn);
    return check_launch(fn);
}

int cyfa_decode_step_general(const CyfaDecodeArgs* a, int dtype, void* hip_stream) {
    const char* fn = "cyfa_decode_step_general";
    if (!a) return fail(CYFA_ERR_VALUE, "%s: null args", fn);
    if (int rc = general_shape(fn, a->B, a->H, a->K, a->V, a->M, dtype)) return rc;
    if (!a->q || !a->k || !a->v || !a->g || !a->delta || !a->beta || !a->table || !a->q_norm_weight ||
        !a->k_norm_weight || !a->o || !a->hk_out || !a->hv_out || !a->clock_out)
        return fail(CYFA_ERR_VALUE, "%s: null required pointer", fn);
    const bool has_in = a->hk_in != nullptr;
    if (has_in != (a->hv_in != nullptr) || has_in != (a->clock_in != nullptr))
        return fail(CYFA_ERR_VALUE, "%s: hk_in, hv_in and clock_in must be all set or all null", fn);
    if (!isfinite(a->scale)) return fail(CYFA_ERR_VALUE, "%s: scale must be finite", fn);
    // fp32 at the tuned kernel's shapes: that kernel, without its bf16 rounding
    // (its alignment needs met; the workspace fields stay ignored)
    if (dtype == CYFA_DTYPE_F32 && a->M == 128 && (a->K == 128 || a->K == 256) && (a->V == 128 || a->V == 256) &&
        aligned(a->v, 8) && aligned(a->table, 16) && aligned(a->hk_out, 16) && aligned(a->hv_out, 16) &&
        (!has_in || (aligned(a->hk_in, 16) && aligned(a->hv_in, 16))))
        return decode_step(a, nullptr, hip_stream, true);
    cyfa::GenDecodeParams p{};
    p.B = a->B;
    p.H = a->H;
    p.K = a->K;
    p.V = a->V;
    p.M = a->M;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.g = a->g;
    p.delta = a->delta;
    p.beta = a->beta;
    p.table = a->table;
    p.q_w = a->q_norm_weight;
    p.k_w = a->k_norm_weight;
    p.q_eps = a->q_norm_eps;
    p.k_eps = a->k_norm_eps;
    p.scale = a->scale;
    p.hk_in = a->hk_in;
    p.hv_in = a->hv_in;
    p.clock_in = a->clock_in;
    p.o = a->o;
    p.hk_out = a->hk_out;
    p.hv_out = a->hv_out;
    p.clock_out = a->clock_out;
    if (cyfa::launch_general_decode(p, dtype == CYFA_DTYPE_BF16, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: launch refused", fn);
    return check_launch(fn);
}

// ---------------------------------------------------------------------------
// The backward pass of the chunk op (cyfa_backward.hip).

size_t cyfa_chunk_bwd_workspace_bytes(int B, int T, int H, int K, int V, int M) {
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || M <= 0) return 0;
    return cyfa::bwd_workspace(B, T, H, K, V, M, nullptr).bytes;
}

int cyfa_chunk_bwd(const CyfaChunkArgs* a, int dtype, const CyfaChunkBwdArgs* d, void* hip_stream) {
    const char* fn = "cyfa_chunk_bwd";
    if (!a || !d) return fail(CYFA_ERR_VALUE, "%s: null args", fn);
    if (dtype != CYFA_DTYPE_BF16 && dtype != CYFA_DTYPE_F32)
        return fail(CYFA_ERR_VALUE, "%s: dtype must be CYFA_DTYPE_BF16 or CYFA_DTYPE_F32, got %d", fn, dtype);
    if (a->B <= 0 || a->T <= 0 || a->H <= 0)
        return fail(CYFA_ERR_VALUE, "%s: B=%d T=%d H=%d must be positive", fn, a->B, a->T, a->H);
    if (a->K < 1 || a->K > 1024 || a->V < 1 || a->V > 1024)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: head dims K=%d V=%d must lie in [1, 1024]", fn, a->K, a->V);
    if (a->M < 4 || a->M > cyfa::BWD_MAX_M || a->M % 2)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: num_slots must be even and in [4, %d], got %d", fn, cyfa::BWD_MAX_M,
                    a->M);
    if (!a->q || !a->k || !a->v || !a->g || !a->delta || !a->beta || !a->table || !a->q_norm_weight ||
        !a->k_norm_weight)
        return fail(CYFA_ERR_VALUE, "%s: null required forward input", fn);
    if (!d->dq || !d->dk || !d->dv || !d->dg || !d->ddelta || !d->dbeta || !d->dtable || !d->dq_norm_weight ||
        !d->dk_norm_weight)
        return fail(CYFA_ERR_VALUE, "%s: null required gradient output", fn);
    if (!(a->scale > 0.f) || !isfinite(a->scale))
        return fail(CYFA_ERR_VALUE, "%s: scale must be positive and finite, got %g", fn, (double)a->scale);
    const bool has_h0 = a->h0_k != nullptr;
    if (has_h0 != (a->h0_v != nullptr) || has_h0 != (a->clock0 != nullptr))
        return fail(CYFA_ERR_VALUE, "%s: h0_k, h0_v and clock0 must be all set or all null", fn);
    const bool has_dh0 = d->dh0_k != nullptr;
    if (has_dh0 != (d->dh0_v != nullptr) || has_dh0 != (d->dclock0 != nullptr))
        return fail(CYFA_ERR_VALUE, "%s: dh0_k, dh0_v and dclock0 must be all set or all null", fn);
    // the kernels index (b, h, padded t) rows and chunk states with 32-bit counts per row
    const size_t Tp = (size_t)(a->T + 63) / 64 * 64, rows = (size_t)a->B * a->H * Tp;
    if (rows * 1024 >= ((size_t)1 << 31))
        return fail(CYFA_ERR_UNSUPPORTED, "%s: B * H * padded T = %zu rows is too many", fn, rows);
    const size_t need = cyfa::bwd_workspace(a->B, a->T, a->H, a->K, a->V, a->M, nullptr).bytes;
    if (!d->workspace || d->workspace_bytes < need)
        return fail(CYFA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", fn, need,
                    d->workspace ? d->workspace_bytes : (size_t)0);
    if (!aligned(d->workspace, 256)) return fail(CYFA_ERR_ALIGN, "%s: workspace needs 256-byte alignment", fn);
    cyfa::BwdParams p{};
    p.B = a->B;
    p.T = a->T;
    p.H = a->H;
    p.K = a->K;
    p.V = a->V;
    p.M = a->M;
    p.bf16 = dtype == CYFA_DTYPE_BF16;
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
    p.d_o = d->d_o;
    p.g = a->g;
    p.delta = a->delta;
    p.beta = a->beta;
    p.table = a->table;
    p.q_w = a->q_norm_weight;
    p.k_w = a->k_norm_weight;
    p.q_eps = a->q_norm_eps;
    p.k_eps = a->k_norm_eps;
    p.scale = a->scale;
    p.h0_k = a->h0_k;
    p.h0_v = a->h0_v;
    p.clock0 = a->clock0;
    p.d_hk = d->d_hk;
    p.d_hv = d->d_hv;
    p.d_clock = d->d_clock;
    p.dq = d->dq;
    p.dk = d->dk;
    p.dv = d->dv;
    p.dg = d->dg;
    p.ddelta = d->ddelta;
    p.dbeta = d->dbeta;
    p.dtable = d->dtable;
    p.dreadout = d->dreadout;
    p.dq_w = d->dq_norm_weight;
    p.dk_w = d->dk_norm_weight;
    p.dh0_k = d->dh0_k;
    p.dh0_v = d->dh0_v;
    p.dclock0 = d->dclock0;
    p.workspace = d->workspace;
    if (cyfa::launch_chunk_bwd(p, (hipStream_t)hip_stream) != 0)
        return fail(CYFA_ERR_UNSUPPORTED, "%s: launch refused", fn);
    return check_launch(fn);
}
