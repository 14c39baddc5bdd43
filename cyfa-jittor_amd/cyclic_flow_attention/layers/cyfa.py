"""Cyclic Flow Attention layer (PyTorch-ROCm host code around the HIP op).

Mirrors layers/cyfa.py:236-357 of Chyxx/CyFA-Jittor v0.1.2: constructor
arguments, parameter names (torch-checkpoint compatible), the
``y, cache = layer(x)`` contract and the cache layout
{"recurrent_state": (hk, hv, clock), "conv_state": (cq, ck, cv)}.
Projections run as torch (hipBLASLt) GEMMs in bf16 with fp32 accumulation,
except calls of at most 64 rows (decode steps) on the fused path, which run
on the HIP kernel behind ``_native.linear``; the attention itself is
``ops.chunk_cyfa`` (prefill) or ``ops.fused_recurrent_cyfa`` (one-token
decode), both HIP kernels.

Like the reference, which switches to its inference kernels for bf16 CUDA
tensors without gradients (layers/cyfa.py:66-73, 148-155), bf16 GPU inference
takes a fused path: one q|k|v projection and one short-convolution launch
for the three tensors, one a|b|d projection with a fused gate kernel, and the
gated o_norm inside the prefill's last kernel. Decode steps of at most 64 rows
form q|k|v, g_proj[0] and a|b|d in one projection launch, and a one-token step
runs the convolution, the gates, the op and the gated o_norm as one HIP kernel.
Other inputs take the general torch path.
"""

import math

import torch
import torch.nn.functional as F
from torch import nn

from .. import _native
from ..ops import chunk_cyfa, fused_recurrent_cyfa
from ..ops.fused_recurrent import decode_layer_step
from ..ops.utils import readout_table

# A one-token step with at least this many (batch, head) workgroups forms
# g_proj[1] inside the decode kernel by default, as does a small-batch step
# that prefetches (see gate_projection_in_kernel).
GATE_IN_KERNEL_MIN_WORKGROUPS = 128
# Bytes of weights a small-batch decode step reads into the caches while its
# decode kernel runs (prefetch_weights): ranges are taken in the order the
# step reads them (o_proj, then the caller's: the MLP's gate|up and down, then
# the next layer's input projection), skipping any that would pass the budget
# except a range marked as a prefix (the next layer's input weight), of which
# the leading part that fits is read; a weight whose projection reads one
# contiguous span per workgroup goes with that span, and its pieces land in
# the L2 of the XCD that reads them. Measured on MI355X (graphed steps, 1.4B
# at B=1): o_proj alone 957-970 tok/s, with down (31 MB) 990, with down and
# the first 10-25% of the next input weight 999-1000 (the budget leaves it
# 24%), with half of it 996, with all of it (58 MB) 958 - past what the L2s
# hold until it is read.
# (A prefix item is only taken up to PREFETCH_PREFIX_MAX_BH.)
PREFETCH_BUDGET_BYTES = 36 << 20
# Largest B H whose step takes (a prefix of) the next layer's input weight: from
# B H = 64 the step workgroups' own prefetched inputs fill most of each XCD's
# L2 (400M at B=16: 17.2 k tok/s without the prefix, 16.8 k with it).
PREFETCH_PREFIX_MAX_BH = 16


def inference_fast_path(x):
    """bf16 GPU inference without gradients (the reference's `_inference` condition)."""
    return x.is_cuda and x.dtype == torch.bfloat16 and not torch.is_grad_enabled()


class FusedWeight:
    """Concatenation of parameters along dim 0, rebuilt when any of them changes."""

    def __init__(self):
        self.key = None
        self.value = None

    def get(self, *tensors, build=None):
        """torch.cat(tensors) along dim 0, or build(*tensors) when given."""
        key = tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)
        if key != self.key:
            parts = [t.detach() for t in tensors]
            self.value = build(*parts) if build is not None else torch.cat(parts, dim=0)
            self.key = key
        return self.value


class RMSNorm(nn.Module):
    """RMSNorm with an optional sigmoid gate (layers/cyfa.py:62-135)."""

    def __init__(self, dim, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x, gate=None, *, prescale=1.0, residual=None):
        """norm(x) [* sigmoid(gate)]. Keyword extensions used by the fused
        inference path: ``prescale`` normalises bf16(x * prescale) (the layer's
        o * (num_slots - 1)); ``residual`` first forms s = x + residual and
        returns (s, norm(s))."""
        D = x.shape[-1]
        if (inference_fast_path(x) and D % 256 == 0 and D // 256 in (1, 2, 4, 8)
                and (gate is None or gate.dtype == torch.bfloat16)
                and (residual is None or residual.dtype == torch.bfloat16)):
            return _native.rms_norm(x, self.weight, self.eps, gate, residual, prescale)
        total = None
        if residual is not None:
            x = total = x + residual
        if prescale != 1.0:
            x = x * prescale
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()
        if gate is not None:
            y = y * torch.sigmoid(gate.float())
        y = y.to(x.dtype)
        return y if residual is None else (total, y)

    execute = forward


class ShortConvolution(nn.Module):
    """Causal depthwise convolution without activation (layers/cyfa.py:138-233).

    ``forward(x, cache=None, lengths=None) -> (y, new_cache)``; the cache holds
    the last ``width - 1`` pre-convolution inputs, or the ``width - 1`` inputs
    before each row's ``lengths`` for right-padded batches.
    """

    def __init__(self, dim, width, bias=False):
        super().__init__()
        self.width = width
        self.weight = nn.Parameter(torch.randn(dim, 1, width) * 0.02)
        self.bias = nn.Parameter(torch.zeros(dim)) if bias else None

    def forward(self, x, cache=None, lengths=None):
        B, T, D = x.shape
        W = self.width
        if inference_fast_path(x) and lengths is None and 2 <= W <= 4 and D % 8 == 0:
            y = _native.short_conv(x, self.weight.reshape(D, W).to(x.dtype),
                                   None if self.bias is None else self.bias.to(x.dtype),
                                   None if cache is None else cache.to(x.dtype))[0]
            return y, conv_cache_tail(x, cache, W)
        history = x if cache is None else torch.cat([cache.to(x.dtype), x], dim=1)
        offset = W - 1 if cache is None else 0
        padded = F.pad(history, (0, 0, offset, 0)) if offset else history
        y = F.conv1d(
            padded.transpose(1, 2),
            self.weight.to(x.dtype),
            None if self.bias is None else self.bias.to(x.dtype),
            groups=D,
        ).transpose(1, 2)
        S = history.shape[1]
        if W == 1:
            new_cache = history[:, :0]
        elif lengths is None and S >= W - 1:
            new_cache = history[:, -(W - 1):]
        else:
            ends = torch.full((B,), T, dtype=torch.int64, device=x.device) if lengths is None else lengths.long()
            pos = ends[:, None] - offset + torch.arange(W - 1, device=x.device)[None, :]
            gathered = history[torch.arange(B, device=x.device)[:, None], pos.clamp(min=0)]
            new_cache = torch.where((pos >= 0)[..., None], gathered, torch.zeros((), dtype=x.dtype, device=x.device))
        return y.contiguous(), new_cache

    execute = forward


def shared_conv_cache(conv_state):
    """The [B, W-1, Dq+Dk+Dv] buffer the three conv caches are channel slices
    of, when they are (as the fused path creates them); else None."""
    cq, ck, cv = conv_state
    base = cq._base if cq._base is not None else None
    if base is None or ck._base is not base or cv._base is not base or base.dim() != 3:
        return None
    if cq.data_ptr() != base.data_ptr() or base.stride(-1) != 1:
        return None
    Dq, Dk = cq.shape[-1], ck.shape[-1]
    item = base.element_size()
    if ck.data_ptr() != cq.data_ptr() + Dq * item or cv.data_ptr() != ck.data_ptr() + Dk * item:
        return None
    if base.shape[-1] != Dq + Dk + cv.shape[-1] or base.shape[:2] != cq.shape[:2]:
        return None
    return base


def conv_cache_tail(x, cache, W):
    """The last W - 1 rows of cat(cache, x) over time (layers/cyfa.py:172-174)."""
    B, T, D = x.shape
    if T >= W - 1:
        return x[:, T - (W - 1):].contiguous()
    if cache is None:  # positions before the start read as zeros (layers/cyfa.py:175-182)
        cache = torch.zeros(B, W - 1, D, dtype=x.dtype, device=x.device)
    return torch.cat([cache.to(x.dtype)[:, T:], x], dim=1)


class CyclicFlowAttention(nn.Module):
    """CyFA attention with projections, short convolutions and a gated readout.

    forward returns (hidden_states, cache). The cache contains recurrent
    states and the short-convolution histories when use_cache is enabled.
    """

    def __init__(
        self,
        hidden_size=1024,
        num_heads=4,
        head_dim=256,
        expand_k=1.0,
        expand_v=1.0,
        num_slots=128,
        use_short_conv=True,
        conv_size=4,
        conv_bias=False,
        norm_eps=1e-6,
        chunk_size=64,
        **kwargs,
    ):
        super().__init__()
        self.num_heads = num_heads
        self.head_k_dim = int(head_dim * expand_k)
        self.head_v_dim = int(head_dim * expand_v)
        self.key_dim = num_heads * self.head_k_dim
        self.value_dim = num_heads * self.head_v_dim
        self.num_slots, self.chunk_size = num_slots, chunk_size
        self.q_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.k_proj = nn.Linear(hidden_size, self.key_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, self.value_dim, bias=False)
        self.a_proj = nn.Linear(hidden_size, num_heads, bias=False)
        self.b_proj = nn.Linear(hidden_size, num_heads, bias=True)
        self.d_proj = nn.Linear(hidden_size, num_heads, bias=True)
        # Defaults of layers/cyfa.py:274-284.
        dt = torch.exp(torch.rand(num_heads) * (math.log(0.1) - math.log(0.001)) + math.log(0.001))
        self.dt_bias = nn.Parameter(dt + torch.log(1.0 - torch.exp(-dt)))
        self.A_log = nn.Parameter(torch.log(torch.rand(num_heads) * 16.0 + 1e-3))
        self.readout = nn.Parameter(torch.eye(num_slots - 1).expand(num_heads, -1, -1).clone())
        self.q_norm = RMSNorm(self.head_k_dim, norm_eps)
        self.k_norm = RMSNorm(self.head_k_dim, norm_eps)
        self.use_short_conv = use_short_conv
        if use_short_conv:
            self.q_conv1d = ShortConvolution(self.key_dim, conv_size, conv_bias)
            self.k_conv1d = ShortConvolution(self.key_dim, conv_size, conv_bias)
            self.v_conv1d = ShortConvolution(self.value_dim, conv_size, conv_bias)
        self.g_proj = nn.Sequential(
            nn.Linear(hidden_size, self.head_v_dim, bias=False),
            nn.Linear(self.head_v_dim, self.value_dim, bias=True),
        )
        self.o_norm = RMSNorm(self.head_v_dim, norm_eps)
        self.o_proj = nn.Linear(self.value_dim, hidden_size, bias=False)
        self._table_key = None
        self._table = None
        self._qkv_weight = FusedWeight()
        self._conv_weight = FusedWeight()
        self._abd_weight = FusedWeight()
        self._abd_bias = FusedWeight()
        self._a_bias_zero = None  # a_proj has no bias: zeros in the fused a|b|d bias
        # decode steps: one [q | k | v | g_proj[0] | a | b | d] projection
        self._in_weight = FusedWeight()
        self._in_weight_folded = FusedWeight()
        self._gp_weight = FusedWeight()
        # When set, a decode step with the block's norm fused into the input
        # projection multiplies the norm weight into the projection's weight
        # (cached) and applies the row scale to the product (cyfa_norm_linear_rows
        # with a NULL norm weight): the kernel skips scaling every operand
        # element, and the bf16 rounding of the normalised input moves to the
        # folded weight. With MLPs folded too the 400M step at B=64 runs about
        # 6% faster on MI355X, but the greedy tokens then follow the
        # reference's rounding less closely (one of 130 decidable steps of the
        # configuration-4 check differs), so it is off by default.
        self.fold_prenorm_weight = False
        self._in_bias = FusedWeight()
        self._in_bias_zero = None
        # When set, one-token steps update the cache's recurrent states in place;
        # otherwise new state tensors are returned.
        self.decode_in_place = False
        # When set (a layer cache of the input's layout), one-token steps of the
        # fused path write the new states and conv cache into it: the graphed
        # decode loop alternates two caches, so that no step updates in place
        # and the decode kernel can run several workgroups per (batch, head).
        self.decode_next = None
        # Whether a one-token step forms the gate (g_proj[1]) inside the decode
        # kernel instead of a separate projection launch (same bits either way).
        # On MI355X it saves about 1.4% of the 400M step at B=64 (one launch per
        # layer fewer) but costs the kernel 2.4 us of L2 reads (each workgroup
        # reads its head's 128 KB weight slice), and without the weight in the
        # caches it loses at B=1. None (the default) picks it when the step has
        # at least GATE_IN_KERNEL_MIN_WORKGROUPS (batch, head) workgroups, or
        # when the small-batch prefetch applies, which then reads the gate
        # weight first (400M at B=1: 1025 -> 1035 tok/s; at B=16: 15.2k ->
        # 15.4k; 1.4B at B=1: 711 -> 713).
        self.gate_projection_in_kernel = None
        # Whether a one-token step at small batch (B H <= _native.PREFETCH_MAX_BH)
        # has the decode kernel read o_proj's weight, and the weights forward_block
        # is given (the decode loop passes the block's MLP weights), into the
        # caches on the compute units it leaves idle, within
        # PREFETCH_BUDGET_BYTES. No result changes.
        self.prefetch_weights = True

    def readout_table(self):
        """readout @ Phi, cached while the readout parameter is unchanged."""
        key = (self.readout.data_ptr(), self.readout._version, self.readout.device)
        if self._table_key != key:
            self._table = readout_table(self.readout.detach())
            self._table_key = key
        return self._table

    def _fused_ok(self, x, attention_mask):
        return (inference_fast_path(x) and attention_mask is None and self.use_short_conv
                and 2 <= self.q_conv1d.width <= 4 and self.q_conv1d.bias is None)

    def forward(self, x, cache=None, use_cache=False, attention_mask=None):
        if self._fused_ok(x, attention_mask):
            return self._forward_fused(x, cache, use_cache)
        B, T, _ = x.shape
        H = self.num_heads
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        lengths = None
        if attention_mask is not None:
            # Right padding is neutral for both the recurrence and the convolution.
            mask = attention_mask.unsqueeze(-1).to(q.dtype)
            q, k, v = q * mask, k * mask, v * mask
            lengths = attention_mask.to(torch.int32).sum(1)
        conv_cache = (None, None, None) if cache is None else cache.get("conv_state", (None, None, None))
        if self.use_short_conv:
            q, cq = self.q_conv1d(q, conv_cache[0], lengths)
            k, ck = self.k_conv1d(k, conv_cache[1], lengths)
            v, cv = self.v_conv1d(v, conv_cache[2], lengths)
        else:
            cq = ck = cv = None
        q = q.reshape(B, T, H, self.head_k_dim)
        k = k.reshape(B, T, H, self.head_k_dim)
        v = v.reshape(B, T, H, self.head_v_dim)
        a = self.a_proj(x).float() + self.dt_bias.float()
        g = -self.A_log.float().exp() * F.softplus(a)
        # the clock branch trains d_proj but passes no gradient into x
        # (reference layers/cyfa.py:325: d_proj(x.detach()))
        delta = torch.sigmoid(self.d_proj(x.detach()).float())
        beta = torch.sigmoid(self.b_proj(x).float())
        if attention_mask is not None:
            valid = attention_mask.unsqueeze(-1).bool()
            g, delta, beta = (torch.where(valid, t, torch.zeros_like(t)) for t in (g, delta, beta))
        kwargs = dict(
            q=q,
            k=k,
            v=v,
            g=g,
            delta=delta,
            beta=beta,
            readout=self.readout,
            q_norm_weight=self.q_norm.weight.float(),
            k_norm_weight=self.k_norm.weight.float(),
            q_norm_eps=self.q_norm.eps,
            k_norm_eps=self.k_norm.eps,
            initial_state=None if cache is None else cache["recurrent_state"],
            output_final_state=use_cache,
        )
        if not self.training and T == 1 and not torch.is_grad_enabled():
            o, state = fused_recurrent_cyfa(**kwargs, table=self.readout_table())
        else:
            o, state = chunk_cyfa(**kwargs, chunk_size=self.chunk_size,
                                  table=None if torch.is_grad_enabled() else self.readout_table())
        gate = self.g_proj(x).reshape(B, T, H, self.head_v_dim)
        o = self.o_norm(o * (self.num_slots - 1), gate).reshape(B, T, self.value_dim)
        o = self.o_proj(o)
        new_cache = {"recurrent_state": state, "conv_state": (cq, ck, cv)} if use_cache else None
        return o, new_cache

    def forward_block(self, x, norm, cache=None, use_cache=False, prefetch=()):
        """The attention half of a decoder block, x + self(norm(x), cache,
        use_cache) (CyFABlock.execute, models/cyfa/modeling_cyfa.py:48-51), for
        the decoder's bf16 inference loop. Returns (x + o, new_cache). A decode
        step with at most 64 rows runs the norm inside the input projection and
        the residual add inside o_proj. ``prefetch``: weights of the projections
        that follow (the block's MLP), which a one-token step at small batch
        reads into the caches while its decode kernel runs (decode_layer_step);
        nothing depends on them."""
        if self._fused_ok(x, None):
            return self._forward_fused(x, cache, use_cache, prenorm=norm, prefetch=prefetch)
        o, new_cache = self(norm(x), cache, use_cache)
        return x + o, new_cache

    def step_prefetch_in_decode_kernel(self, x):
        """Whether a one-token step of forward_block(x, ...) reads the weights
        that follow it into the caches inside its decode kernel (small
        batches); at larger batches the projections read the next one's."""
        return self.prefetch_weights and x.numel() // x.shape[-1] * self.num_heads <= _native.PREFETCH_MAX_BH

    def step_input_weight(self, x, norm):
        """The input projection's weight a one-token step of forward_block(x,
        norm) reads first, as a prefetch range for the step before it:
        ((weight, span, True),) - the span each workgroup of the projection
        reads, and True: the leading part that fits the budget may be taken -
        or () when the step runs elsewhere."""
        rows = x.numel() // x.shape[-1]
        if not self._fused_ok(x, None) or rows > _native.LINEAR_ROWS_MAX:
            return ()
        g0 = self.g_proj[0]
        w = self._in_weight.get(self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, g0.weight,
                                self.a_proj.weight, self.b_proj.weight, self.d_proj.weight)
        folded = self.fold_prenorm_weight and x.shape[-1] <= _native.LINEAR_NORM_MAX_K
        if folded:
            w = self._in_weight_folded.get(w, norm.weight, build=_native.fold_norm_weight)
        return ((w, _native.linear_rows_span(rows, w.shape[0], w.shape[1], norm=2 if folded else 1), True),)

    def _forward_fused(self, x, cache, use_cache, prenorm=None, prefetch=()):
        """bf16 inference: the same math as forward with fused launches. With
        ``prenorm`` (the block's norm), x is the block input and the result is
        (x + o, new_cache), as forward_block."""
        B, T, _ = x.shape
        block_in = None
        if prenorm is not None:
            block_in = x
            if B * T > _native.LINEAR_ROWS_MAX:
                x, prenorm = prenorm(x), None
        H, Dk, Dv = self.num_heads, self.key_dim, self.value_dim
        W = self.q_conv1d.width
        g0, g1 = self.g_proj
        if self._a_bias_zero is None or self._a_bias_zero.dtype != self.b_proj.bias.dtype \
                or self._a_bias_zero.device != self.b_proj.bias.device:
            self._a_bias_zero = torch.zeros_like(self.b_proj.bias.detach())
        abd_bias = self._abd_bias.get(self._a_bias_zero, self.b_proj.bias, self.d_proj.bias)
        if B * T <= _native.LINEAR_ROWS_MAX:
            # one launch for the q|k|v, g_proj[0] and a|b|d projections; the
            # outputs are column slices of one buffer with 16-byte aligned rows
            D3, Dg = 2 * Dk + Dv, g0.weight.shape[0]
            if self._in_bias_zero is None or self._in_bias_zero.shape[0] != D3 + Dg \
                    or self._in_bias_zero.dtype != abd_bias.dtype or self._in_bias_zero.device != abd_bias.device:
                self._in_bias_zero = torch.zeros(D3 + Dg, dtype=abd_bias.dtype, device=abd_bias.device)
            w_in = self._in_weight.get(self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, g0.weight,
                                       self.a_proj.weight, self.b_proj.weight, self.d_proj.weight)
            b_in = self._in_bias.get(self._in_bias_zero, abd_bias)
            if prenorm is not None and self.fold_prenorm_weight and x.shape[-1] <= _native.LINEAR_NORM_MAX_K:
                w_f = self._in_weight_folded.get(w_in, prenorm.weight, build=_native.fold_norm_weight)
                _, y_in = _native.norm_linear(x, None, prenorm.eps, w_f, b_in,
                                              out_cols=(D3 + Dg + 3 * H + 7) // 8 * 8)
            elif prenorm is not None:
                _, y_in = _native.norm_linear(x, prenorm.weight, prenorm.eps, w_in, b_in,
                                              out_cols=(D3 + Dg + 3 * H + 7) // 8 * 8)
            else:
                y_in = _native.linear(x, w_in, b_in, out_cols=(D3 + Dg + 3 * H + 7) // 8 * 8)
            qkv, g0_out, abd = y_in[..., :D3], y_in[..., D3:D3 + Dg], y_in[..., D3 + Dg:]
        else:
            qkv = _native.linear(x, self._qkv_weight.get(self.q_proj.weight, self.k_proj.weight, self.v_proj.weight))
            g0_out = abd = None
        conv_cache = None if cache is None else cache.get("conv_state")
        cat_cache = None
        if conv_cache is not None:
            cat_cache = shared_conv_cache(conv_cache)
            if cat_cache is None or cat_cache.dtype != x.dtype:
                cat_cache = torch.cat([c.to(x.dtype) for c in conv_cache], dim=-1)
        # the new caches are channel slices of one buffer the conv kernel writes
        # (the cache itself when a graphed decode step updates in place)
        nxt = self.decode_next if cache is not None and T == 1 else None
        nxt_conv = None if nxt is None else shared_conv_cache(nxt["conv_state"])
        if nxt_conv is not None and (nxt_conv.dtype != x.dtype or tuple(nxt_conv.shape) != (B, W - 1, qkv.shape[-1])):
            nxt_conv = None
        in_place = self.decode_in_place and cat_cache is not None and T <= 32 and nxt is None
        if in_place:
            tail = cat_cache
        elif nxt_conv is not None:
            tail = nxt_conv
        else:
            tail = torch.empty(B, W - 1, qkv.shape[-1], dtype=x.dtype, device=x.device)
        wconv = self._conv_weight.get(self.q_conv1d.weight, self.k_conv1d.weight, self.v_conv1d.weight)
        if (not self.training and T == 1 and W == 4 and self.head_k_dim == 256 and self.head_v_dim == 256
                and all(c.bias is None for c in (self.q_conv1d, self.k_conv1d, self.v_conv1d))
                and (cat_cache is None or cat_cache.stride() == tail.stride())):
            # one-token step: short convolution, gates, the decode op and the
            # gated output norm in one kernel
            if abd is None:
                abd = _native.linear(x, self._abd_weight.get(self.a_proj.weight, self.b_proj.weight,
                                                              self.d_proj.weight), abd_bias)
            if g0_out is None:
                g0_out = _native.linear(x, g0.weight)
            # g_proj[1] inside the kernel (the same bits as _native.linear) when asked and
            # its operands are bf16; otherwise the gate is projected first
            want = self.gate_projection_in_kernel
            small = self.prefetch_weights and B * H <= _native.PREFETCH_MAX_BH
            if want is None:
                want = B * H >= GATE_IN_KERNEL_MIN_WORKGROUPS or small
            in_kernel = (want and g1.weight.dtype == torch.bfloat16
                         and (g1.bias is None or g1.bias.dtype == torch.bfloat16))
            gate = None if in_kernel else _native.linear(g0_out, g1.weight, g1.bias)
            # at small batches the decode kernel leaves most compute units and
            # HBM idle: it reads o_proj's weight and the caller's into the caches
            pf = ()
            if small:
                total = 0
                # (the kernel's extra workgroups read g_proj[1]'s rows into the
                # L2 of each step workgroup themselves); o_proj's weight with
                # the span each of its workgroups reads, so that every piece
                # lands in the L2 of the XCD that reads it
                w_o = self.o_proj.weight
                span_o = _native.linear_rows_span(B * T, w_o.shape[0], w_o.shape[1])
                for item in ((w_o, span_o),) + tuple(prefetch):
                    t, span, prefix = (item + (False,))[:3] if isinstance(item, tuple) else (item, 0, False)
                    n = t.numel() * t.element_size()
                    if len(pf) >= _native.PREFETCH_RANGES or (prefix and B * H > PREFETCH_PREFIX_MAX_BH):
                        break
                    if total + n <= PREFETCH_BUDGET_BYTES:
                        pf, total = pf + ((t, span),), total + n
                    elif prefix and PREFETCH_BUDGET_BYTES - total >= 1 << 20:
                        k = (PREFETCH_BUDGET_BYTES - total) // t.element_size() // 8 * 8
                        pf, total = pf + ((t.reshape(-1)[:k], span),), PREFETCH_BUDGET_BYTES
            o, state = decode_layer_step(
                qkv, cat_cache, tail, wconv.reshape(-1, W).to(x.dtype), abd, self.dt_bias, self.A_log, gate,
                self.o_norm.weight, self.o_norm.eps, float(self.num_slots - 1), self.readout_table(),
                self.q_norm.weight, self.k_norm.weight, self.q_norm.eps, self.k_norm.eps, H,
                initial_state=None if cache is None else cache["recurrent_state"], output_final_state=use_cache,
                inplace=self.decode_in_place and cache is not None and nxt is None,
                g_proj=(g0_out, g1.weight, g1.bias) if in_kernel else None, prefetch=pf,
                out_state=None if nxt is None else nxt["recurrent_state"])
            # at larger batches extra workgroups of o_proj read the weight of
            # the projection after it (the MLP's gate|up) into the caches
            o_pf = () if small else tuple(item[:2] for item in tuple(prefetch)[:1] if isinstance(item, tuple))
            o = _native.linear(o.view(B, T, Dv), self.o_proj.weight, residual=block_in, prefetch=o_pf)
            cq, ck, cv = tail[..., :Dk], tail[..., Dk:2 * Dk], tail[..., 2 * Dk:]
            new_cache = {"recurrent_state": state, "conv_state": (cq, ck, cv)} if use_cache else None
            return o, new_cache
        if Dk == Dv:
            q, k, v = _native.short_conv(qkv, wconv.reshape(-1, W).to(x.dtype), None, cat_cache, split=Dk,
                                         cache_out=tail)
        else:
            (y,) = _native.short_conv(qkv, wconv.reshape(-1, W).to(x.dtype), None, cat_cache, cache_out=tail)
            q, k, v = y[..., :Dk].contiguous(), y[..., Dk:2 * Dk].contiguous(), y[..., 2 * Dk:].contiguous()
        cq, ck, cv = tail[..., :Dk], tail[..., Dk:2 * Dk], tail[..., 2 * Dk:]
        gate = None
        if abd is None and g0_out is None:
            w1 = self._gp_weight.get(g0.weight, self.a_proj.weight, self.b_proj.weight, self.d_proj.weight)
            if _native.gate_path_ok(x, w1, g1.weight, g1.bias, H):
                # g_proj[0], a|b|d, the gates and g_proj[1] in one launch
                gate, g, beta, delta = _native.gate_path(x, w1, abd_bias, g1.weight, g1.bias, self.dt_bias,
                                                         self.A_log, H)
                gate = gate.view(B, T, H, self.head_v_dim)
        if gate is None:
            if abd is None:
                abd = _native.linear(x, self._abd_weight.get(self.a_proj.weight, self.b_proj.weight,
                                                              self.d_proj.weight), abd_bias)
            g, beta, delta = _native.gates(abd, self.dt_bias, self.A_log)
        kwargs = dict(
            q=q.view(B, T, H, self.head_k_dim),
            k=k.view(B, T, H, self.head_k_dim),
            v=v.view(B, T, H, self.head_v_dim),
            g=g,
            delta=delta,
            beta=beta,
            readout=self.readout,
            q_norm_weight=self.q_norm.weight.float(),
            k_norm_weight=self.k_norm.weight.float(),
            q_norm_eps=self.q_norm.eps,
            k_norm_eps=self.k_norm.eps,
            initial_state=None if cache is None else cache["recurrent_state"],
            output_final_state=use_cache,
        )
        if gate is None:
            if g0_out is None:
                g0_out = _native.linear(x, g0.weight)
            gate = _native.linear(g0_out, g1.weight, g1.bias).view(B, T, H, self.head_v_dim)
        if not self.training and T == 1:
            o, state = fused_recurrent_cyfa(**kwargs, table=self.readout_table(),
                                            inplace=self.decode_in_place and cache is not None)
            o = self.o_norm(o, gate, prescale=float(self.num_slots - 1)).view(B, T, Dv)
        else:
            # the gated output norm runs in the prefill's last kernel
            o, state = chunk_cyfa(**kwargs, chunk_size=self.chunk_size, table=self.readout_table(),
                                  output_norm=(self.o_norm.weight, gate, self.o_norm.eps,
                                               float(self.num_slots - 1)))
            o = o.view(B, T, Dv)
        o = _native.linear(o, self.o_proj.weight, residual=block_in)
        new_cache = {"recurrent_state": state, "conv_state": (cq, ck, cv)} if use_cache else None
        return o, new_cache

    execute = forward
