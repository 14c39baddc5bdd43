"""Constant-state autoregressive CyFA decoding on the gfx950 HIP path.

Keeps the reference's signature, checks and return convention
(ops/fused_recurrent.py:10-200 of Chyxx/CyFA-Jittor v0.1.2). One call runs one
fused HBM-streaming kernel of libcyfa_hip.so: ``cyfa_decode_step`` at the tuned
shapes, ``cyfa_decode_step_general`` at any other.
"""

import torch

from .. import _native
from .chunk import _operand_dtype
from .utils import check_table, readout_table


def fused_recurrent_cyfa(
    q,
    k,
    v,
    g,
    delta,
    beta,
    readout,
    q_norm_weight,
    k_norm_weight,
    q_norm_eps=1e-6,
    k_norm_eps=1e-6,
    scale=None,
    initial_state=None,
    output_final_state=False,
    cu_seqlens=None,
    *,
    table=None,
    inplace=False,
    split=False,
):
    """Decode one token using constant-size key, value and clock states.

    Uses the same input layout and return convention as chunk_cyfa (q, k, v
    of bf16, fp16 or fp32; o in their dtype). bf16 operands with K, V in
    {128, 256} and 128 slots run the tuned kernel; fp16 and fp32 operands
    and every other shape up to K, V <= 1024 and 256 slots run the general
    step (cyfa_decode_step_general: bf16 operands rounded where the
    reference casts, fp16 and fp32 in fp32 without intermediate rounding, as
    the reference's kernel computes in the input dtype). The new
    states are returned as new tensors; ``inplace=True`` (an extension) updates
    the given initial_state tensors instead and returns them. ``table`` (an
    extension) passes a precomputed readout @ Phi to skip rebuilding it.
    ``split`` (an extension): with B H < 64 the step runs on eight
    workgroups per (batch, head) in two launches instead of one workgroup per
    (batch, head) in one. Both give bit-identical results; on MI355X the
    one-workgroup form is 1-3 us faster at every B H < 64 measured, so it is
    the default.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    M = readout.shape[-1] + 1
    tracked = (q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight)
    if initial_state is not None:
        tracked = tracked + tuple(initial_state)
    if torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in tracked):
        raise ValueError(
            "fused_recurrent_cyfa is inference-only; use torch.no_grad() or chunk_cyfa for gradients"
        )
    if T != 1 or cu_seqlens is not None:
        raise NotImplementedError("native fused decode currently needs dense T=1")
    if M > 256 or K > 1024 or V > 1024:
        raise ValueError("decode shape exceeds block limits")
    out_dtype = _operand_dtype("fused_recurrent_cyfa", q, k, v)
    state_in = tuple(initial_state) if initial_state is not None else ()
    dev = _native.require_device(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, table, *state_in)
    # bf16 operands at the tuned kernel's shapes; everything else takes the
    # general step, in bf16 for bf16 operands and in fp32 for fp16 and fp32 ones
    io_dtype = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
    fast = K in (128, 256) and V in (128, 256) and M == 128 and io_dtype == torch.bfloat16
    q, k, v = (x.to(io_dtype).contiguous() for x in (q, k, v))
    g, delta, beta = (x.to(torch.float32).contiguous() for x in (g, delta, beta))
    qw = q_norm_weight.to(torch.float32).contiguous()
    kw = k_norm_weight.to(torch.float32).contiguous()
    if table is None:
        table = readout_table(readout)
    else:
        check_table(table, H, M)
    if initial_state is not None:
        hk_in, hv_in, c_in = initial_state
        if tuple(hk_in.shape) != (B, H, K, M) or tuple(hv_in.shape) != (B, H, M, V) or tuple(c_in.shape) != (B, H):
            raise ValueError("initial_state must be (hk [B,H,K,M], hv [B,H,M,V], clock [B,H])")
        if inplace:
            for x in (hk_in, hv_in, c_in):
                if x.dtype != torch.float32 or not x.is_contiguous():
                    raise ValueError("inplace decode needs contiguous fp32 state tensors")
        else:
            hk_in, hv_in, c_in = (x.to(torch.float32).contiguous() for x in (hk_in, hv_in, c_in))
    else:
        hk_in = hv_in = c_in = None
    if inplace and initial_state is not None:
        hk_out, hv_out, c_out = hk_in, hv_in, c_in
    else:
        hk_out = torch.empty(B, H, K, M, dtype=torch.float32, device=dev)
        hv_out = torch.empty(B, H, M, V, dtype=torch.float32, device=dev)
        c_out = torch.empty(B, H, dtype=torch.float32, device=dev)
    o = torch.empty(B, 1, H, V, dtype=io_dtype, device=dev)
    workspace = _native.decode_workspace(B, H, K, V, dev) if split and fast else None  # alive until the launch
    args = _native.CyfaDecodeArgs(
        B=B, H=H, K=K, V=V, M=M,
        workspace=_native.ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel(),
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
        g=g.data_ptr(), delta=delta.data_ptr(), beta=beta.data_ptr(),
        table=table.data_ptr(), q_norm_weight=qw.data_ptr(), k_norm_weight=kw.data_ptr(),
        q_norm_eps=float(q_norm_eps), k_norm_eps=float(k_norm_eps),
        scale=float(K**-0.5 if scale is None else scale),
        hk_in=_native.ptr(hk_in), hv_in=_native.ptr(hv_in), clock_in=_native.ptr(c_in),
        o=o.data_ptr(), hk_out=hk_out.data_ptr(), hv_out=hv_out.data_ptr(), clock_out=c_out.data_ptr(),
    )
    if fast:
        _native.decode_step(args, dev)
    else:
        _native.decode_step_general(args, _native.general_dtype(q), dev)
    if out_dtype != io_dtype:
        o = o.to(out_dtype)
    return o, ((hk_out, hv_out, c_out) if output_final_state else None)


def decode_layer_step(qkv, conv_cache, conv_cache_out, conv_weight, abd, dt_bias, A_log, gate, norm_weight, norm_eps,
                      norm_prescale, table, q_norm_weight, k_norm_weight, q_norm_eps, k_norm_eps, num_heads,
                      initial_state=None, output_final_state=False, inplace=False, split=False, g_proj=None,
                      prefetch=(), out_state=None):
    """The layer's one-token step around the op in one kernel (cyfa_decode_layer_step).

    qkv [B, 1, 3 H 256] is the projection before the short convolution (rows
    may be strided), conv_cache / conv_cache_out [B, 3, 3 H 256] the conv
    history in and out (conv_cache may be None; conv_cache_out may be
    conv_cache), conv_weight [3 H 256, 4], abd [B, 1, 3H] the a|b|d projection
    with its biases, gate [B, 1, H 256]. Returns (o', states) with o' the gated
    output norm o_norm(o * norm_prescale, gate) of the op's output, [B, 1, H, 256],
    and the states as fused_recurrent_cyfa returns them. ``split``: as in
    fused_recurrent_cyfa. ``g_proj`` (with gate None): (g0 [B, 1, 256], weight
    [H 256, 256], bias [H 256] or None), and the kernel forms the gate as
    linear(g0, weight, bias) - the second projection of g_proj - with the same
    bits as _native.linear. ``prefetch``: up to four contiguous device tensors
    (the weights of the projections that follow the step), each alone or as
    (tensor, span) with span from _native.linear_rows_span for the projection
    that reads it, that the launch reads into the device's caches on the
    compute units the step leaves idle, when B H <= _native.PREFETCH_MAX_BH
    and the one-workgroup form runs (a tensor with a span lands in the L2 of
    the XCD whose workgroup will read each piece); nothing depends on their
    values. ``out_state``: (hk, hv, clock) tensors that receive the new
    states (contiguous fp32, apart from the inputs) instead of new ones; with
    every output apart from its input (the states and the conv cache) and
    B H <= 32 the kernel runs several workgroups per (b, h), the same bits.
    """
    B = qkv.shape[0]
    H, K, V, M = num_heads, 256, 256, table.shape[-1]
    state_in = tuple(initial_state) if initial_state is not None else ()
    if (gate is None) == (g_proj is None):
        raise ValueError("decode_layer_step: pass exactly one of gate and g_proj")
    g0, g_w, g_b = g_proj if g_proj is not None else (None, None, None)
    dev = _native.require_device(qkv, conv_cache, conv_cache_out, conv_weight, abd, dt_bias, A_log, gate, norm_weight,
                                 table, q_norm_weight, k_norm_weight, g0, g_w, g_b, *state_in)
    D = 2 * H * K + H * V
    if qkv.shape[-1] != D or qkv.stride(-1) != 1 or conv_weight.shape != (D, 4) or not conv_weight.is_contiguous():
        raise ValueError("decode_layer_step: qkv must have 3 H 256 unit-stride columns and conv_weight [3 H 256, 4]")
    tensors = (("qkv", qkv), ("abd", abd), ("conv_weight", conv_weight), ("conv_cache_out", conv_cache_out))
    tensors += (("gate", gate),) if gate is not None else (("g0", g0), ("g_proj weight", g_w))
    tensors += (("g_proj bias", g_b),) if g_b is not None else ()
    for name, x in tensors:
        if x.dtype != torch.bfloat16 or x.stride(-1) != 1:
            raise ValueError(f"decode_layer_step: {name} must be bfloat16 with unit last-dim stride")
    if abd.shape[-1] != 3 * H or (gate is not None and gate.shape[-1] != H * V):
        raise ValueError(f"decode_layer_step: abd needs {3 * H} and gate {H * V} columns")
    if g_proj is not None:
        if g0.shape[-1] != V or g0.numel() != B * V or g_w.shape != (H * V, V) or (g_b is not None and g_b.shape != (H * V,)):
            raise ValueError(f"decode_layer_step: g_proj needs g0 [{B}, 1, {V}], weight [{H * V}, {V}], bias [{H * V}]")
        g0 = g0.reshape(B, V)  # a view for the layer's column slice of the input projection
        if g0.stride(1) != 1 or g0.stride(0) % 8 or g0.data_ptr() % 16:
            g0 = g0.contiguous()
        g_w = g_w.detach().contiguous()
        g_b = None if g_b is None else g_b.detach().contiguous()
    if conv_cache_out.dim() != 3 or tuple(conv_cache_out.shape) != (B, 3, D):
        raise ValueError(f"decode_layer_step: conv_cache_out must be [{B}, 3, {D}]")
    check_table(table, H, M)
    if conv_cache is not None and (conv_cache.dtype != torch.bfloat16 or conv_cache.shape != conv_cache_out.shape):
        raise ValueError("decode_layer_step: conv_cache must be bfloat16 of conv_cache_out's shape")
    if conv_cache is not None and conv_cache.stride() != conv_cache_out.stride():
        raise ValueError("decode_layer_step: conv_cache and conv_cache_out must share their layout")
    qw = q_norm_weight.to(torch.float32).contiguous()
    kw = k_norm_weight.to(torch.float32).contiguous()
    db = dt_bias.detach().to(torch.float32).contiguous()
    al = A_log.detach().to(torch.float32).contiguous()
    nw = norm_weight.detach().to(torch.float32).contiguous()
    if initial_state is not None:
        hk_in, hv_in, c_in = initial_state
        if tuple(hk_in.shape) != (B, H, K, M) or tuple(hv_in.shape) != (B, H, M, V) or tuple(c_in.shape) != (B, H):
            raise ValueError("initial_state must be (hk [B,H,K,M], hv [B,H,M,V], clock [B,H])")
        if inplace:
            for x in (hk_in, hv_in, c_in):
                if x.dtype != torch.float32 or not x.is_contiguous():
                    raise ValueError("inplace decode needs contiguous fp32 state tensors")
        else:
            hk_in, hv_in, c_in = (x.to(torch.float32).contiguous() for x in (hk_in, hv_in, c_in))
    else:
        hk_in = hv_in = c_in = None
    if out_state is not None:
        hk_out, hv_out, c_out = out_state
        if (tuple(hk_out.shape) != (B, H, K, M) or tuple(hv_out.shape) != (B, H, M, V) or tuple(c_out.shape) != (B, H)
                or any(x.dtype != torch.float32 or not x.is_contiguous() or x.device != dev
                       for x in (hk_out, hv_out, c_out))):
            raise ValueError("decode_layer_step: out_state must be contiguous fp32 (hk [B,H,K,M], hv [B,H,M,V], "
                             "clock [B,H]) on the step's device")
    elif inplace and initial_state is not None:
        hk_out, hv_out, c_out = hk_in, hv_in, c_in
    else:
        hk_out = torch.empty(B, H, K, M, dtype=torch.float32, device=dev)
        hv_out = torch.empty(B, H, M, V, dtype=torch.float32, device=dev)
        c_out = torch.empty(B, H, dtype=torch.float32, device=dev)
    o = torch.empty(B, 1, H, V, dtype=torch.bfloat16, device=dev)
    workspace = _native.decode_workspace(B, H, K, V, dev) if split else None  # alive until the launch
    args = _native.CyfaDecodeArgs(
        B=B, H=H, K=K, V=V, M=M, table=table.data_ptr(),
        workspace=_native.ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel(), q_norm_weight=qw.data_ptr(), k_norm_weight=kw.data_ptr(),
        q_norm_eps=float(q_norm_eps), k_norm_eps=float(k_norm_eps), scale=float(K ** -0.5),
        hk_in=_native.ptr(hk_in), hv_in=_native.ptr(hv_in), clock_in=_native.ptr(c_in),
        o=o.data_ptr(), hk_out=hk_out.data_ptr(), hv_out=hv_out.data_ptr(), clock_out=c_out.data_ptr(),
    )
    layer = _native.CyfaDecodeLayerArgs(
        qkv=qkv.data_ptr(), qkv_row=qkv.stride(0), conv_cache=_native.ptr(conv_cache),
        conv_cache_out=conv_cache_out.data_ptr(), cache_row=conv_cache_out.stride(1),
        cache_batch=conv_cache_out.stride(0), conv_weight=conv_weight.data_ptr(), abd=abd.data_ptr(),
        abd_row=abd.stride(0), dt_bias=db.data_ptr(), A_log=al.data_ptr(), gate=_native.ptr(gate),
        gate_row=0 if gate is None else gate.stride(0), norm_weight=nw.data_ptr(), norm_eps=float(norm_eps),
        norm_prescale=float(norm_prescale), g0=_native.ptr(g0), g0_row=0 if g0 is None else g0.stride(0),
        g_weight=_native.ptr(g_w), g_bias=_native.ptr(g_b),
    )
    if len(prefetch) > _native.PREFETCH_RANGES:
        raise ValueError(f"decode_layer_step: at most {_native.PREFETCH_RANGES} prefetch tensors")
    for i, item in enumerate(prefetch):
        t, span = item if isinstance(item, tuple) else (item, 0)
        if not t.is_contiguous() or t.device != qkv.device:
            raise ValueError("decode_layer_step: prefetch tensors must be contiguous, on the step's device")
        layer.prefetch[i] = t.data_ptr()
        layer.prefetch_bytes[i] = t.numel() * t.element_size()
        layer.prefetch_span[i] = int(span)
    _native.decode_layer_step(args, layer, dev)
    return o, ((hk_out, hv_out, c_out) if output_final_state else None)
