"""CPU restatement of the CyFA layer, block and causal LM -- TEST INFRASTRUCTURE ONLY.

Functions take a flat state dict keyed by the reference's PyTorch-compatible
parameter names (layers/cyfa.py:268-297, models/cyfa/modeling_cyfa.py:59-133)
so that the product model and the oracle consume identical weights.

``mode="exact"`` computes in float64 with no bfloat16 casts; ``mode="mirror"``
computes in float32 and casts to bfloat16 wherever the reference's bf16
inference path does (``.cast(x.dtype)`` points of layers/cyfa.py and
modeling_cyfa.py). ``op_mode`` (default: ``mode``) sets the mode of the
attention op alone: ``mode="mirror", op_mode="exact"`` is the reference's bf16
layer plumbing around an exact (float64) CyFA op, the fp32-or-better
reference a bf16 layer is compared with (a float64 plumbing would round the
clock increments differently from any bf16 layer and let the clock drift).
"""

import math

import torch

from . import cyfa_oracle as ops


def _dt(mode):
    return torch.float64 if mode == "exact" else torch.float32


def _cast(x, mode):
    return x.to(torch.bfloat16).to(torch.float32) if mode == "mirror" else x


def linear(x, weight, bias=None, mode="exact"):
    """Linear / BiasLinear (layers/cyfa.py:15-59): fp32 accumulation (+bias), then cast."""
    dt = _dt(mode)
    y = x.to(dt) @ weight.to(dt).T
    if bias is not None:
        y = y + bias.to(dt)
    return _cast(y, mode)


def rms_norm(x, weight, eps, gate=None, mode="exact"):
    """RMSNorm with optional sigmoid gate (layers/cyfa.py:62-135)."""
    dt = _dt(mode)
    xf = x.to(dt)
    y = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps) * weight.to(dt)
    if gate is not None:
        y = y * torch.sigmoid(gate.to(dt))
    return _cast(y, mode)


def short_conv(x, weight, bias=None, cache=None, lengths=None, mode="exact"):
    """Causal depthwise convolution, no activation (layers/cyfa.py:138-233).

    x [B,T,D]; weight [D,1,W]; cache [B,W-1,D] (previous pre-conv inputs).
    Returns (y [B,T,D], new_cache [B,W-1,D]).
    """
    dt = _dt(mode)
    B, T, D = x.shape
    W = weight.shape[-1]
    history = x if cache is None else torch.cat([cache.to(x.dtype), x], dim=1)
    offset = W - 1 if cache is None else 0
    hist = history.to(dt)
    S = hist.shape[1]
    y = torch.zeros(B, T, D, dtype=dt)
    wf = weight.to(dt)[:, 0, :]
    for i in range(W):
        idx = torch.arange(T) + i - offset
        valid = (idx >= 0) & (idx < S)
        window = torch.zeros(B, T, D, dtype=dt)
        window[:, valid] = hist[:, idx[valid]]
        y = y + window * wf[:, i]
    if bias is not None:
        y = y + bias.to(dt)
    if W == 1:
        new_cache = history[:, :0]
    elif lengths is None and S >= W - 1:
        new_cache = history[:, -(W - 1):]
    else:
        ends = torch.full((B,), T, dtype=torch.int64) if lengths is None else lengths.to(torch.int64)
        pos = ends[:, None] - offset + torch.arange(W - 1)[None, :]
        gathered = history[torch.arange(B)[:, None], pos.clamp(min=0)]
        new_cache = torch.where((pos >= 0)[..., None], gathered, torch.zeros((), dtype=history.dtype))
    return _cast(y, mode), new_cache


def gate_activations(a, b, d, dt_bias, A_log, mode="exact"):
    """Gate activations of layers/cyfa.py:323-326 from the three projections
    (a, b, d: [..., H], the b and d biases included):
    g = -exp(A_log) softplus(a + dt_bias) (natural log of the decay),
    beta = sigmoid(b), delta = sigmoid(d). Returns (g, beta, delta)."""
    dt = _dt(mode)
    g = -torch.exp(A_log.to(dt)) * torch.nn.functional.softplus(a.to(dt) + dt_bias.to(dt))
    return g, torch.sigmoid(b.to(dt)), torch.sigmoid(d.to(dt))


def layer_gates(p, pre, xin, mode="exact"):
    """(g, delta, beta) of the layer for the normed input xin: the a, b and d
    projections (layers/cyfa.py:323-326; a_proj has no bias, b_proj and
    d_proj have one) through gate_activations. The d projection reads a
    detached xin (layers/cyfa.py:325, ``self.d_proj(x.detach())``): delta
    trains d_proj but sends no gradient into xin or anything before it."""
    a = linear(xin, p[pre + "a_proj.weight"], mode=mode)
    b = linear(xin, p[pre + "b_proj.weight"], p[pre + "b_proj.bias"], mode)
    d = linear(xin.detach(), p[pre + "d_proj.weight"], p[pre + "d_proj.bias"], mode)
    g, beta, delta = gate_activations(a, b, d, p[pre + "dt_bias"], p[pre + "A_log"], mode)
    return g, delta, beta


def attention_layer(p, pre, x, cfg, cache=None, use_cache=False, attention_mask=None, mode="exact",
                    chunk_size=64, op_mode=None, cast_output=True):
    """CyclicFlowAttention.execute (layers/cyfa.py:299-357).

    p: state dict; pre: name prefix such as "model.layers.0.attn.";
    cfg: dict with hidden_size, num_heads, head_dim, num_slots, norm_eps.
    cast_output=False leaves the layer output (o_proj) in the working precision.
    """
    dt = _dt(mode)
    B, T, _ = x.shape
    H = cfg["num_heads"]
    Dk = int(cfg["head_dim"] * cfg.get("expand_k", 1.0))
    Dv = int(cfg["head_dim"] * cfg.get("expand_v", 1.0))
    eps = cfg.get("norm_eps", 1e-6)
    xin = _cast(x.to(dt), mode)
    q = linear(xin, p[pre + "q_proj.weight"], mode=mode)
    k = linear(xin, p[pre + "k_proj.weight"], mode=mode)
    v = linear(xin, p[pre + "v_proj.weight"], mode=mode)
    lengths = None
    if attention_mask is not None:
        m = attention_mask.to(dt)[..., None]
        q, k, v = q * m, k * m, v * m
        lengths = attention_mask.to(torch.int64).sum(1)
    conv_cache = (None, None, None) if cache is None else cache.get("conv_state", (None, None, None))
    if cfg.get("use_short_conv", True):
        q, cq = short_conv(q, p[pre + "q_conv1d.weight"], p.get(pre + "q_conv1d.bias"), conv_cache[0], lengths, mode)
        k, ck = short_conv(k, p[pre + "k_conv1d.weight"], p.get(pre + "k_conv1d.bias"), conv_cache[1], lengths, mode)
        v, cv = short_conv(v, p[pre + "v_conv1d.weight"], p.get(pre + "v_conv1d.bias"), conv_cache[2], lengths, mode)
    else:
        cq = ck = cv = None
    q = q.reshape(B, T, H, Dk)
    k = k.reshape(B, T, H, Dk)
    v = v.reshape(B, T, H, Dv)
    g, delta, beta = layer_gates(p, pre, xin, mode)
    if attention_mask is not None:
        valid = attention_mask.to(torch.bool)[..., None]
        zero = torch.zeros((), dtype=dt)
        g, delta, beta = (torch.where(valid, t, zero) for t in (g, delta, beta))
    kwargs = dict(
        q=q, k=k, v=v, g=g, delta=delta, beta=beta,
        readout=p[pre + "readout"],
        q_norm_weight=p[pre + "q_norm.weight"].float(),
        k_norm_weight=p[pre + "k_norm.weight"].float(),
        q_norm_eps=eps, k_norm_eps=eps,
        initial_state=None if cache is None else cache["recurrent_state"],
        output_final_state=use_cache,
        mode=op_mode or mode,
    )
    if T == 1 and cache is not None:
        o, state = ops.fused_recurrent_cyfa(**kwargs)
    else:
        o, state = ops.chunk_cyfa(**kwargs, chunk_size=chunk_size)
    gate = linear(linear(xin, p[pre + "g_proj.0.weight"], mode=mode), p[pre + "g_proj.1.weight"],
                  p[pre + "g_proj.1.bias"], mode).reshape(B, T, H, Dv)
    scaled = _cast(o.to(dt) * (cfg["num_slots"] - 1), mode)
    o = rms_norm(scaled, p[pre + "o_norm.weight"], eps, gate, mode).reshape(B, T, H * Dv)
    y = linear(o, p[pre + "o_proj.weight"], mode=mode if cast_output else "exact")
    new_cache = {"recurrent_state": state, "conv_state": (cq, ck, cv)} if use_cache else None
    return y, new_cache


def mlp_intermediate(cfg):
    """SwiGLU width (models/cyfa/modeling_cyfa.py:13-17)."""
    if cfg.get("intermediate_size"):
        return cfg["intermediate_size"]
    return 256 * math.ceil(int(cfg["hidden_size"] * cfg.get("hidden_ratio", 4.0) * 2 / 3) / 256)


def gated_mlp(p, pre, x, mode="exact"):
    """GatedMLP (models/cyfa/modeling_cyfa.py:13-27)."""
    dt = _dt(mode)
    g = linear(x, p[pre + "gate_proj.weight"], mode=mode).to(dt)
    u = linear(x, p[pre + "up_proj.weight"], mode=mode).to(dt)
    return linear(_cast(g * torch.sigmoid(g) * u, mode), p[pre + "down_proj.weight"], mode=mode)


def causal_lm(p, cfg, input_ids, cache=None, use_cache=False, attention_mask=None, mode="exact",
              chunk_size=64, op_mode=None, last_logits_only=False, progress=None):
    """CyclicFlowAttentionForCausalLM.execute without the loss
    (models/cyfa/modeling_cyfa.py:49-108). Returns (logits, cache).
    ``last_logits_only`` returns the logits of the last position only
    ([B, 1, vocab]; the final norm and lm_head act per row, so these equal the
    last row of the full logits); ``progress(i)`` is called after layer i."""
    dt = _dt(mode)
    eps = cfg.get("norm_eps", 1e-6)
    x = p["model.embeddings.weight"].to(dt)[input_ids]
    new = []
    for i in range(cfg["num_hidden_layers"]):
        pre = f"model.layers.{i}."
        h = rms_norm(x, p[pre + "attn_norm.weight"], eps, mode=mode)
        y, c = attention_layer(p, pre + "attn.", h, cfg, None if cache is None else cache[i], use_cache,
                               attention_mask, mode, chunk_size, op_mode)
        r = _cast(x + y, mode)
        x = _cast(r + gated_mlp(p, pre + "mlp.", rms_norm(r, p[pre + "mlp_norm.weight"], eps, mode=mode), mode),
                  mode)
        new.append(c)
        if progress is not None:
            progress(i)
    if last_logits_only:
        x = x[:, -1:]
    hidden = rms_norm(x, p["model.norm.weight"], eps, mode=mode)
    logits = linear(hidden, p["lm_head.weight"], mode=mode)
    return logits, (new if use_cache else None)
