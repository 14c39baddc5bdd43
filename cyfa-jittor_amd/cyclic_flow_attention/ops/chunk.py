"""Chunkwise CyFA prefill on the gfx950 HIP path.

Keeps the reference's signature, argument meaning and error behaviour
(ops/chunk.py:164-353 of Chyxx/CyFA-Jittor v0.1.2); the whole computation --
q/k RMS norm, clock scan, write vector, both ScalarGatedLA passes, the fused
slot readout and the final states -- runs inside ``cyfa_chunk_fwd`` of
libcyfa_hip.so. With inputs that require a gradient the op is an autograd
function whose backward is ``cyfa_chunk_bwd`` (the reference's adjoints:
ops/chunk.py:51-71, ops/chunk_bwd.py, ops/chunk_readout.py:13-621,
ops/utils.py:589-754, ops/qk_norm.py:241-289).
"""

import torch

from .. import _native
from .utils import check_forward_only, check_table, readout_table


def chunk_cyfa(
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
    checkpoint_level=0,
    chunk_size=64,
    *,
    table=None,
    output_norm=None,
    no_alloc=False,
):
    """Chunkwise Cyclic Flow Attention.

    Inputs q, k and v use [batch, time, heads, channels]; g, delta and beta use
    [batch, time, heads]. The readout has [heads, slots-1, slots-1]. Returns
    the output ([batch, time, heads, V], in q's dtype) and, when requested,
    (key_state [B,H,K,M], value_state [B,H,M,V], clock [B,H]), all fp32.
    bf16 q, k, v with K = V = 256, 128 slots and chunk_size 64 run the tuned
    kernels, as the reference takes its fused bf16 kernels only for bf16
    inputs (ops/chunk.py:209-223, 257-264). Every other call -- fp16 or fp32
    operands at any shape, or any other shape (K, V <= 1024, an even slot
    count up to 256, chunk_size 16, 32 or 64) -- runs the general path,
    cyfa_chunk_fwd_general, which computes in fp32: fp16 and fp32 operands
    without intermediate rounding, bf16 operands rounded where the reference
    casts to the input dtype, like the reference's unfused fallback
    (ops/chunk.py:285-331).
    ``table`` (keyword only, not in the reference signature) is a precomputed
    readout @ Phi [H, M-1, M] fp32; when None it is formed from ``readout``.
    ``output_norm`` (keyword only, an extension) is ``(weight [V], gate
    [B, T, H, V] bf16, eps, prescale)``: the layer's gated output norm
    bf16(xs rsqrt(mean xs^2 + eps) weight sigmoid(gate)), xs = bf16(o prescale),
    is then applied inside the kernels and its result returned in place of o.
    ``no_alloc`` (keyword only, an extension) runs cyfa_chunk_fwd_noalloc: the
    intermediates live in the library's per-device scratch array instead of
    a workspace allocated here (calls on one GPU must not overlap).

    When grad mode is on and q, k, v, g, delta, beta, the readout, a norm
    weight or an initial state requires a gradient, the call is recorded for
    autograd: the forward runs as above and the backward (cyfa_chunk_bwd)
    returns the gradients of all of them (slot counts up to 256; ``table``,
    ``output_norm`` and ``no_alloc`` are inference-only).
    """
    if cu_seqlens is not None:
        raise NotImplementedError("packed layout requires native segment dispatch")
    if checkpoint_level != 0:
        raise NotImplementedError("only saved-activation training is implemented")
    state_in = tuple(initial_state) if initial_state is not None else ()
    tracked = (q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight) + state_in
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tracked):
        if table is not None or output_norm is not None or no_alloc:
            raise NotImplementedError("chunk_cyfa: table, output_norm and no_alloc are inference-only; "
                                      "call it under torch.no_grad() or drop them")
        M = readout.shape[-1] + 1
        if M > BWD_MAX_SLOTS:
            raise NotImplementedError(f"chunk_cyfa: the backward pass supports up to {BWD_MAX_SLOTS} slots, got {M}")
        B, T, H = q.shape[:3]
        rows = B * H * ((T + 63) // 64 * 64)
        if rows * 1024 >= 1 << 31:  # cyfa_chunk_bwd's 32-bit row indexing: refuse before the forward runs
            raise NotImplementedError(f"chunk_cyfa: the backward pass supports B * H * padded T below "
                                      f"{(1 << 31) // 1024} rows, got {rows}")
        h0k, h0v, c0 = state_in if state_in else (None, None, None)
        o, hk, hv, clock = _ChunkCyFA.apply(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, h0k, h0v,
                                            c0, float(q_norm_eps), float(k_norm_eps), scale, int(chunk_size))
        return o, ((hk, hv, clock) if output_final_state else None)
    return _chunk_forward(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, q_norm_eps, k_norm_eps,
                          scale, initial_state, output_final_state, chunk_size, table, output_norm, no_alloc)


# Largest slot count of the backward pass (the reference's decode limit,
# ops/fused_recurrent.py:45-46; up to 128 slots the readout adjoint keeps the
# head's table on chip, above it streams the table through tile GEMMs).
BWD_MAX_SLOTS = 256


def _chunk_forward(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, q_norm_eps, k_norm_eps, scale,
                   initial_state, output_final_state, chunk_size, table, output_norm, no_alloc):
    """The forward op: the tuned kernels at K = V = 256, 128 slots and chunk
    size 64, the general path at every other shape (see chunk_cyfa)."""
    state_in = tuple(initial_state) if initial_state is not None else ()
    B, T, H, K = q.shape
    V = v.shape[-1]
    M = readout.shape[-1] + 1
    if tuple(k.shape) != (B, T, H, K) or tuple(v.shape[:3]) != (B, T, H):
        raise ValueError(f"q/k/v shapes disagree: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    for name, x in (("g", g), ("delta", delta), ("beta", beta)):
        if tuple(x.shape) != (B, T, H):
            raise ValueError(f"{name} must have shape {(B, T, H)}, got {tuple(x.shape)}")
    out_dtype = _operand_dtype("chunk_cyfa", q, k, v)
    dev = _native.require_device(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, table, *state_in)
    # bf16 operands at the tuned kernels' shape; everything else takes the
    # general path, in bf16 for bf16 operands and in fp32 for fp16 and fp32 ones
    io_dtype = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float32
    fast = K == 256 and V == 256 and M == 128 and chunk_size == 64 and io_dtype == torch.bfloat16
    if not fast and (output_norm is not None or no_alloc):
        raise NotImplementedError("output_norm and no_alloc need bf16 q, k, v with K = V = 256, 128 slots and "
                                  "chunk_size 64")
    q, k, v = (x.to(io_dtype).contiguous() for x in (q, k, v))
    g, delta, beta = (x.to(torch.float32).contiguous() for x in (g, delta, beta))
    qw = q_norm_weight.to(torch.float32).contiguous()
    kw = k_norm_weight.to(torch.float32).contiguous()
    if table is None:
        table = readout_table(readout)
    else:
        check_table(table, H, M)
    if initial_state is not None:
        h0k, h0v, c0 = (x.to(torch.float32).contiguous() for x in initial_state)
        if tuple(h0k.shape) != (B, H, K, M) or tuple(h0v.shape) != (B, H, M, V) or tuple(c0.shape) != (B, H):
            raise ValueError("initial_state must be (hk [B,H,K,M], hv [B,H,M,V], clock [B,H])")
    else:
        h0k = h0v = c0 = None
    o = torch.empty(B, T, H, V, dtype=io_dtype, device=dev)
    if output_final_state:
        hk = torch.empty(B, H, K, M, dtype=torch.float32, device=dev)
        hv = torch.empty(B, H, M, V, dtype=torch.float32, device=dev)
        clock = torch.empty(B, H, dtype=torch.float32, device=dev)
    else:
        hk = hv = clock = None
    if no_alloc:
        ws_bytes, workspace = 0, None
    else:
        ws_bytes = (_native.chunk_workspace_bytes(B, T, H, K, V, M, chunk_size) if fast else
                    _native.chunk_general_workspace_bytes(B, T, H, K, V, M, chunk_size))
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)  # alive until the launch
    args = _native.CyfaChunkArgs(
        B=B, T=T, H=H, K=K, V=V, M=M, C=chunk_size,
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(),
        g=g.data_ptr(), delta=delta.data_ptr(), beta=beta.data_ptr(),
        table=table.data_ptr(), q_norm_weight=qw.data_ptr(), k_norm_weight=kw.data_ptr(),
        q_norm_eps=float(q_norm_eps), k_norm_eps=float(k_norm_eps),
        scale=float(K**-0.5 if scale is None else scale),
        h0_k=_native.ptr(h0k), h0_v=_native.ptr(h0v), clock0=_native.ptr(c0),
        o=o.data_ptr(), hk=_native.ptr(hk), hv=_native.ptr(hv), clock=_native.ptr(clock),
        workspace=_native.ptr(workspace), workspace_bytes=ws_bytes,
    )
    if not fast:
        _native.chunk_fwd_general(args, _native.general_dtype(q), dev)
    elif output_norm is None:
        if no_alloc:
            _native.chunk_fwd_noalloc(args, None, dev)
        else:
            _native.chunk_fwd(args, dev)
    else:
        on_w, on_gate, on_eps, on_prescale = output_norm
        on_w = on_w.detach().to(torch.float32).contiguous()
        if tuple(on_w.shape) != (V,):
            raise ValueError(f"output_norm weight must have shape ({V},), got {tuple(on_w.shape)}")
        on_gate = on_gate.reshape(B, T, H, V)
        if on_gate.dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise NotImplementedError(f"output_norm gate must be a float tensor, got {on_gate.dtype}")
        on_gate = on_gate.to(torch.bfloat16).contiguous()
        _native.require_device(on_w, on_gate)
        norm = _native.CyfaOutNormArgs(weight=on_w.data_ptr(), gate=on_gate.data_ptr(), eps=float(on_eps),
                                       prescale=float(on_prescale))
        if no_alloc:
            _native.chunk_fwd_noalloc(args, norm, dev)
        else:
            _native.chunk_fwd_normed(args, norm, dev)
    if out_dtype != io_dtype:
        o = o.to(out_dtype)
    return o, ((hk, hv, clock) if output_final_state else None)


class _ChunkCyFA(torch.autograd.Function):
    """chunk_cyfa as an autograd function: the HIP forward, and the
    gradients of every floating input from cyfa_chunk_bwd, which recomputes
    the forward in fp32 from the saved inputs (so nothing but the inputs is
    kept between the passes). Replaces the reference's jt.Function adjoints
    behind chunk_cyfa (ops/chunk.py:51-71; ops/chunk_readout.py:776-786,
    976-988; ops/utils.py:297-299, 589-641, 704-754; ops/qk_norm.py:241-289)."""

    @staticmethod
    def forward(ctx, q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, h0k, h0v, c0, q_eps, k_eps,
                scale, chunk_size):
        init = (h0k, h0v, c0) if h0k is not None else None
        o, (hk, hv, clock) = _chunk_forward(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, q_eps,
                                            k_eps, scale, init, True, chunk_size, None, None, False)
        ctx.save_for_backward(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, h0k, h0v, c0)
        ctx.eps = (q_eps, k_eps)
        ctx.scale = scale
        ctx.set_materialize_grads(False)
        return o, hk, hv, clock

    @staticmethod
    def backward(ctx, d_o, d_hk, d_hv, d_clock):
        q, k, v, g, delta, beta, readout, q_w, k_w, h0k, h0v, c0 = ctx.saved_tensors
        B, T, H, K = q.shape
        V = v.shape[-1]
        M = readout.shape[-1] + 1
        dev = q.device
        io = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
        f32 = torch.float32

        def c(x, dt=f32):
            return None if x is None else x.detach().to(dt).contiguous()

        qc, kc, vc = c(q, io), c(k, io), c(v, io)
        gc, dc, bc, qwc, kwc = c(g), c(delta), c(beta), c(q_w), c(k_w)
        table = readout_table(readout.detach())
        has_h0 = h0k is not None
        h0kc, h0vc, c0c = c(h0k), c(h0v), c(c0)
        d_oc = c(d_o, io)
        d_hkc, d_hvc, d_clc = c(d_hk), c(d_hv), c(d_clock)

        def empty(shape, dt=f32):
            return torch.empty(shape, dtype=dt, device=dev)

        dq, dk, dv = empty((B, T, H, K), io), empty((B, T, H, K), io), empty((B, T, H, V), io)
        dg, ddelta, dbeta = empty((B, T, H)), empty((B, T, H)), empty((B, T, H))
        dtable, dreadout = empty((H, M - 1, M)), empty((H, M - 1, M - 1))
        dqw, dkw = empty((K,)), empty((K,))
        dh0k = dh0v = dc0 = None
        if has_h0:
            dh0k, dh0v, dc0 = empty((B, H, K, M)), empty((B, H, M, V)), empty((B, H))
        ws_bytes = _native.chunk_bwd_workspace_bytes(B, T, H, K, V, M)
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        q_eps, k_eps = ctx.eps
        args = _native.CyfaChunkArgs(
            B=B, T=T, H=H, K=K, V=V, M=M, C=64,
            q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(),
            g=gc.data_ptr(), delta=dc.data_ptr(), beta=bc.data_ptr(),
            table=table.data_ptr(), q_norm_weight=qwc.data_ptr(), k_norm_weight=kwc.data_ptr(),
            q_norm_eps=float(q_eps), k_norm_eps=float(k_eps),
            scale=float(K**-0.5 if ctx.scale is None else ctx.scale),
            h0_k=_native.ptr(h0kc), h0_v=_native.ptr(h0vc), clock0=_native.ptr(c0c),
        )
        grads = _native.CyfaChunkBwdArgs(
            d_o=_native.ptr(d_oc), d_hk=_native.ptr(d_hkc), d_hv=_native.ptr(d_hvc), d_clock=_native.ptr(d_clc),
            dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
            dg=dg.data_ptr(), ddelta=ddelta.data_ptr(), dbeta=dbeta.data_ptr(),
            dtable=dtable.data_ptr(), dreadout=dreadout.data_ptr(),
            dq_norm_weight=dqw.data_ptr(), dk_norm_weight=dkw.data_ptr(),
            dh0_k=_native.ptr(dh0k), dh0_v=_native.ptr(dh0v), dclock0=_native.ptr(dc0),
            workspace=workspace.data_ptr(), workspace_bytes=ws_bytes,
        )
        _native.chunk_bwd(args, _native.general_dtype(qc), grads, dev)

        def like(grad, x):
            return None if x is None or grad is None else grad.to(x.dtype)

        return (like(dq, q), like(dk, k), like(dv, v), like(dg, g), like(ddelta, delta), like(dbeta, beta),
                like(dreadout, readout), like(dqw, q_w), like(dkw, k_w), like(dh0k, h0k), like(dh0v, h0v),
                like(dc0, c0), None, None, None, None)


def _operand_dtype(what, *xs):
    """The dtype of q, k, v (one float dtype). bf16 operands run the bf16
    kernels; fp32 and fp16 operands run the general path in fp32 without
    intermediate rounding (the reference's scalar path for non-bf16 inputs,
    ops/chunk.py:285-331) and the output is returned in the input dtype."""
    dt = xs[0].dtype
    if any(x.dtype != dt for x in xs) or dt not in (torch.bfloat16, torch.float16, torch.float32):
        raise NotImplementedError(f"{what}: q, k, v must share one of bf16, fp16, fp32; got "
                                  + ", ".join(str(x.dtype) for x in xs))
    return dt


def scalar_la(q, k, v, g, initial, scale=1.0, raw_output=False, output_bth=False, v_bth=False):
    """One chunkwise scalar-gated linear-attention pass (ops/chunk.py:74-79 of
    the reference, ``ScalarAttention`` at ops/chunk.py:30-71), on the HIP path.

    q, k [B, H, T, K] bf16; v [B, H, T, V] bf16 ([B, T, H, V] when ``v_bth``);
    g [B, H, T] natural-log decay; initial [B, H, K, V] fp32 or None (zero
    state). (K, V) is (256, 128) or (128, 256) and T a multiple of 64. Returns
    (o, final): o is [B, H, T, V] ([B, T, H, V] when ``output_bth``), fp32 when
    ``raw_output`` (the sum of the per-128-wide-key-slice outputs, each rounded
    to bf16 after the scale) and bf16 otherwise; final is the fp32 state.
    Forward only.
    """
    state_in = (initial,) if initial is not None else ()
    check_forward_only("scalar_la", (q, k, v, g) + state_in)
    if q.dim() != 4 or k.shape != q.shape:
        raise ValueError(f"q and k must be [B, H, T, K] of one shape, got {tuple(q.shape)} {tuple(k.shape)}")
    B, H, T, K = q.shape
    V = v.shape[-1]
    want_v = (B, T, H, V) if v_bth else (B, H, T, V)
    if tuple(v.shape) != want_v:
        raise ValueError(f"v must have shape {want_v}, got {tuple(v.shape)}")
    if tuple(g.shape) != (B, H, T):
        raise ValueError(f"g must have shape {(B, H, T)}, got {tuple(g.shape)}")
    if T % 64 != 0:
        raise ValueError(f"scalar_la needs T to be a multiple of 64, got {T}")
    for name, x in (("q", q), ("k", k), ("v", v)):
        if x.dtype != torch.bfloat16:
            raise NotImplementedError(f"scalar_la computes in bfloat16; {name} is {x.dtype}")
    dev = _native.require_device(q, k, v, g, *state_in)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    g = g.to(torch.float32).contiguous()
    h0 = None
    if initial is not None:
        h0 = initial.to(torch.float32).contiguous()
        if tuple(h0.shape) != (B, H, K, V):
            raise ValueError(f"initial must have shape {(B, H, K, V)}, got {tuple(h0.shape)}")
    shape = (B, T, H, V) if output_bth else (B, H, T, V)
    o = torch.empty(shape, dtype=torch.float32 if raw_output else torch.bfloat16, device=dev)
    final = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    ws_bytes = _native.scalar_la_workspace_bytes(B, T, H, K, V)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    args = _native.CyfaSlaArgs(
        B=B, T=T, H=H, K=K, V=V, q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), g=g.data_ptr(),
        initial=_native.ptr(h0), scale=float(scale), raw_output=int(bool(raw_output)),
        output_bth=int(bool(output_bth)), v_bth=int(bool(v_bth)), o=o.data_ptr(), final_state=final.data_ptr(),
        workspace=workspace.data_ptr(), workspace_bytes=ws_bytes,
    )
    _native.scalar_la(args, dev)
    return o, final
