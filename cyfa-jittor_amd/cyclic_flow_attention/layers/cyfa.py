"""Cyclic Flow Attention layer (PyTorch-ROCm host code around the HIP op).

Mirrors layers/cyfa.py:236-357 of Chyxx/CyFA-Jittor v0.1.2: constructor
arguments, parameter names (torch-checkpoint compatible), the
``y, cache = layer(x)`` contract and the cache layout
{"recurrent_state": (hk, hv, clock), "conv_state": (cq, ck, cv)}.
Projections run as torch (hipBLASLt) GEMMs in bf16 with fp32 accumulation;
the attention itself is ``ops.chunk_cyfa`` (prefill) or
``ops.fused_recurrent_cyfa`` (one-token decode), both HIP kernels.
"""

import math

import torch
import torch.nn.functional as F
from torch import nn

from ..ops import chunk_cyfa, fused_recurrent_cyfa
from ..ops.utils import readout_table


class RMSNorm(nn.Module):
    """RMSNorm with an optional sigmoid gate (layers/cyfa.py:62-135)."""

    def __init__(self, dim, eps):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x, gate=None):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight.float()
        if gate is not None:
            y = y * torch.sigmoid(gate.float())
        return y.to(x.dtype)

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

    def readout_table(self):
        """readout @ Phi, cached while the readout parameter is unchanged."""
        key = (self.readout.data_ptr(), self.readout._version, self.readout.device)
        if self._table_key != key:
            self._table = readout_table(self.readout.detach())
            self._table_key = key
        return self._table

    def forward(self, x, cache=None, use_cache=False, attention_mask=None):
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
        delta = torch.sigmoid(self.d_proj(x).float())
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
            o, state = chunk_cyfa(**kwargs, chunk_size=self.chunk_size)
        gate = self.g_proj(x).reshape(B, T, H, self.head_v_dim)
        o = self.o_norm(o * (self.num_slots - 1), gate).reshape(B, T, self.value_dim)
        o = self.o_proj(o)
        new_cache = {"recurrent_state": state, "conv_state": (cq, ck, cv)} if use_cache else None
        return o, new_cache

    execute = forward
