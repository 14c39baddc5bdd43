"""CyFA decoder blocks and causal language model (PyTorch host code).

Mirrors models/cyfa/modeling_cyfa.py:13-133 of Chyxx/CyFA-Jittor v0.1.2:
pre-norm attention + SwiGLU MLP blocks, torch-checkpoint-compatible parameter
names, and the bf16 precision policy of ``to_bfloat16``.
"""

import math

import torch
import torch.nn.functional as F
from torch import nn

from ... import _native
from ...layers.cyfa import CyclicFlowAttention, FusedWeight, RMSNorm, inference_fast_path


def mlp_width(config):
    return config.intermediate_size or 256 * math.ceil(int(config.hidden_size * config.hidden_ratio * 2 / 3) / 256)


class GatedMLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        mid = mlp_width(config)
        self.gate_proj = nn.Linear(config.hidden_size, mid, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, mid, bias=False)
        self.down_proj = nn.Linear(mid, config.hidden_size, bias=False)
        self._gate_up = FusedWeight()
        self._gate_up_il = FusedWeight()
        self._gate_up_folded = FusedWeight()
        # decode steps: mlp_norm's weight multiplied into the gate|up weight
        # (off by default; see CyclicFlowAttention.fold_prenorm_weight)
        self.fold_norm_weight = False

    def forward(self, x):
        rows = x.numel() // x.shape[-1]
        if (inference_fast_path(x) and rows <= _native.LINEAR_ROWS_MAX and self.gate_proj.weight.shape[0] % 16 == 0
                and x.shape[-1] % 32 == 0):
            # decode steps: the SwiGLU product in the gate|up projection's epilogue
            w = self._gate_up_il.get(self.gate_proj.weight, self.up_proj.weight, build=_native.interleave_gate_up)
            return _native.linear(_native.linear_swiglu(x, w), self.down_proj.weight)
        if inference_fast_path(x) and self.gate_proj.weight.shape[0] % 8 == 0:
            # one [gate | up] GEMM and the fused SwiGLU kernel
            gu = _native.linear(x, self._gate_up.get(self.gate_proj.weight, self.up_proj.weight))
            return _native.linear(_native.silu_mul(gu), self.down_proj.weight)
        g = self.gate_proj(x)
        u = self.up_proj(x)
        return self.down_proj((F.silu(g.float()) * u.float()).to(x.dtype))

    def _step_gate_up(self, norm, K):
        """The gate|up weight a decode step reads: interleaved, with the norm
        weight folded in when fold_norm_weight is set."""
        w = self._gate_up_il.get(self.gate_proj.weight, self.up_proj.weight, build=_native.interleave_gate_up)
        if self.fold_norm_weight and K <= _native.LINEAR_NORM_MAX_K:
            w = self._gate_up_folded.get(w, norm.weight, build=_native.fold_norm_weight)
        return w

    def step_weights(self, norm, x):
        """The weights a decode step of forward_block(x, norm) reads, in the
        order it reads them (gate|up, then down), each with the span each
        workgroup of its projection reads (_native.linear_rows_span); () when
        it runs elsewhere."""
        rows = x.numel() // x.shape[-1]
        if (inference_fast_path(x) and rows <= _native.LINEAR_ROWS_MAX and self.gate_proj.weight.shape[0] % 16 == 0
                and x.shape[-1] % 32 == 0):
            K = x.shape[-1]
            w_gu, w_d = self._step_gate_up(norm, K), self.down_proj.weight
            folded = self.fold_norm_weight and K <= _native.LINEAR_NORM_MAX_K
            return ((w_gu, _native.linear_rows_span(rows, w_gu.shape[0], K, swiglu=True, norm=2 if folded else 1)),
                    (w_d, _native.linear_rows_span(rows, w_d.shape[0], w_d.shape[1])))
        return ()

    def forward_block(self, x, norm, prefetch_next=None):
        """The MLP half of a decoder block, x + self(norm(x)). A decode step with
        at most 64 rows runs the norm inside the gate|up projection and the
        residual add inside down_proj. With ``prefetch_next`` ((tensor, span)
        items: the next layer's input weight, or ()), the gate|up launch also
        reads down's weight into the caches and down reads those; nothing
        depends on them."""
        rows = x.numel() // x.shape[-1]
        if (inference_fast_path(x) and rows <= _native.LINEAR_ROWS_MAX and self.gate_proj.weight.shape[0] % 16 == 0
                and x.shape[-1] % 32 == 0):
            K = x.shape[-1]
            w = self._step_gate_up(norm, K)
            w_d = self.down_proj.weight
            gu_pf = d_pf = ()
            if prefetch_next is not None:
                gu_pf = ((w_d, _native.linear_rows_span(rows, w_d.shape[0], w_d.shape[1])),)
                d_pf = tuple(item[:2] for item in prefetch_next)
            if self.fold_norm_weight and K <= _native.LINEAR_NORM_MAX_K:
                _, h = _native.norm_linear(x, None, norm.eps, w, swiglu=True, prefetch=gu_pf)
            else:
                _, h = _native.norm_linear(x, norm.weight, norm.eps, w, swiglu=True, prefetch=gu_pf)
            return _native.linear(h, w_d, residual=x, prefetch=d_pf)
        return x + self(norm(x))


class CyFABlock(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.attn_norm = RMSNorm(config.hidden_size, config.norm_eps)
        self.attn = CyclicFlowAttention(
            hidden_size=config.hidden_size,
            num_heads=config.num_heads,
            head_dim=config.head_dim,
            expand_k=config.expand_k,
            expand_v=config.expand_v,
            num_slots=config.num_slots,
            use_short_conv=config.use_short_conv,
            conv_size=config.conv_size,
            conv_bias=config.conv_bias,
            norm_eps=config.norm_eps,
            chunk_size=config.chunk_size,
        )
        self.mlp_norm = RMSNorm(config.hidden_size, config.norm_eps)
        self.mlp = GatedMLP(config)

    def forward(self, x, cache=None, use_cache=False, attention_mask=None):
        y, cache = self.attn(self.attn_norm(x), cache, use_cache, attention_mask)
        residual = x + y
        return residual + self.mlp(self.mlp_norm(residual)), cache


class CyclicFlowAttentionModel(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.embeddings = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([CyFABlock(config) for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.norm_eps)

    def forward(self, input_ids, cache=None, use_cache=False, attention_mask=None):
        x = self.embeddings(input_ids)
        new = []
        if not inference_fast_path(x):
            for i, layer in enumerate(self.layers):
                x, s = layer(x, None if cache is None else cache[i], use_cache, attention_mask)
                new.append(s)
            return self.norm(x), (new if use_cache else None)
        if x.numel() // x.shape[-1] <= _native.LINEAR_ROWS_MAX and attention_mask is None:
            # bf16 decode steps: each pre-norm runs inside the projection after
            # it, each residual add inside the projection before it (x + y, as
            # CyFABlock.forward, bit for bit)
            # (a small-batch step's decode kernel reads the weights that follow
            # it into the caches: the block's MLP, then the next layer's input
            # projection, the first layer's after the last)
            n = len(self.layers)
            for i, layer in enumerate(self.layers):
                nxt = self.layers[(i + 1) % n]
                nin = nxt.attn.step_input_weight(x, nxt.attn_norm)
                pf = tuple(layer.mlp.step_weights(layer.mlp_norm, x)) + nin
                x, s = layer.attn.forward_block(x, layer.attn_norm, None if cache is None else cache[i], use_cache,
                                                prefetch=pf)
                # (larger batches: each projection reads the next one's weight)
                x = layer.mlp.forward_block(x, layer.mlp_norm,
                                            None if layer.attn.step_prefetch_in_decode_kernel(x) else nin)
                new.append(s)
            return self.norm(x), (new if use_cache else None)
        # bf16 prefill: each residual add runs inside the following norm kernel
        # (x + y and residual + mlp, as CyFABlock.forward, bit for bit)
        pending = None
        for i, layer in enumerate(self.layers):
            h = layer.attn_norm(x) if pending is None else None
            if pending is not None:
                x, h = layer.attn_norm(pending, residual=x)
            y, s = layer.attn(h, None if cache is None else cache[i], use_cache, attention_mask)
            x, m = layer.mlp_norm(y, residual=x)
            pending = layer.mlp(m)
            new.append(s)
        if pending is None:
            return self.norm(x), (new if use_cache else None)
        _, out = self.norm(pending, residual=x)
        return out, (new if use_cache else None)


# Parameters that stay fp32 under to_bfloat16 (modeling_cyfa.py:110-116).
FP32_PARAMETERS = ("norm.weight", "readout", "A_log", "dt_bias")


class CyclicFlowAttentionForCausalLM(nn.Module):
    """CyFA causal language model with Torch-checkpoint-compatible parameter names."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.model = CyclicFlowAttentionModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embeddings.weight

    @classmethod
    def from_pretrained(cls, path):
        """The bf16 model of a local checkpoint directory (config.json and
        *.safetensors, loaded strictly; models/cyfa/modeling_cyfa.py:85-89)."""
        from ...utils import load_model

        return load_model(path)[0]

    def save_pretrained(self, directory, tokenizer=None):
        """config.json and model.safetensors under ``directory`` (and the
        tokenizer's files and special-token ids when one is given;
        models/cyfa/modeling_cyfa.py:91-94)."""
        from ...utils import save_model

        save_model(self, directory, tokenizer)

    def forward(self, input_ids, labels=None, cache=None, use_cache=False, attention_mask=None):
        # The final norm stays a launch of its own: inside the lm_head
        # projection each of its 1000 workgroups would normalise the rows again
        # (48 us on MI355X at B = 64, against 39 us for the two launches).
        hidden, cache = self.model(input_ids, cache, use_cache, attention_mask)
        if inference_fast_path(hidden):
            logits = _native.linear(hidden, self.lm_head.weight)
        else:
            logits = self.lm_head(hidden)
        loss = None
        if labels is not None:
            loss = F.cross_entropy(
                logits[:, :-1].float().reshape(-1, self.config.vocab_size),
                labels[:, 1:].reshape(-1),
                ignore_index=-100,
            )
        return {"logits": logits, "loss": loss, "cache": cache}

    def to_bfloat16(self):
        for name, p in self.named_parameters():
            if not any(s in name for s in FP32_PARAMETERS):
                p.data = p.data.to(torch.bfloat16)
        return self

    @torch.no_grad()
    def graphed_decoder(self, cache, tokens):
        """A GraphedDecodeStep continuing from a prefill cache and the last tokens [B, 1]."""
        return GraphedDecodeStep(self, cache, tokens)

    @torch.no_grad()
    def generate(self, input_ids, max_new_tokens=32, eos_token_id=None):
        """Greedy decoding with the constant-size state (modeling_cyfa.py:142-158).

        The argmax stays on the device; tokens are copied to the host once at
        the end (the reference synchronises every step)."""
        self.eval()
        tokens = [input_ids]
        cache = None
        current = input_ids
        for _ in range(max_new_tokens):
            result = self(current, cache=cache, use_cache=True)
            cache = result["cache"]
            current = result["logits"][:, -1:].argmax(-1)
            tokens.append(current)
            if eos_token_id is not None and bool((current == eos_token_id).all()):
                break
        return torch.cat(tokens, dim=1)


def _clone_cache(c):
    """Copy of one layer's cache; the three conv caches become channel slices
    of one buffer, the layout the fused conv kernel updates in place."""
    conv = torch.cat([t for t in c["conv_state"]], dim=-1)
    sizes = [t.shape[-1] for t in c["conv_state"]]
    views, start = [], 0
    for n in sizes:
        views.append(conv[..., start:start + n])
        start += n
    return {"recurrent_state": tuple(t.clone() for t in c["recurrent_state"]), "conv_state": tuple(views)}


class GraphedDecodeStep:
    """One greedy decode step of the whole model, captured as HIP graphs.

    A step reads the token buffer, runs every layer's one-token path, writes
    the new recurrent states and conv histories, and stores the argmax token
    in the token buffer for the next replay. Two caches alternate: the step
    captured from cache 0 writes cache 1 and the other one back, so that no
    decode kernel updates a state in place (which lets it run several
    workgroups per (batch, head) at small batches; see decode_next on the
    attention layer). ``step()`` replays the graph of the current parity and
    returns the token buffer [B, 1] (valid until the next replay); ``cache``
    is the cache the next step reads, ``logits`` the last step's logits. The
    reference runs the same step as separate launches with a host sync per
    token (generation.py:23-62).
    """

    def __init__(self, model, cache, tokens):
        if not torch.cuda.is_available() or not tokens.is_cuda:
            raise ValueError("graphed decoding needs the model and tokens on a GPU")
        self.model = model
        self.tokens = tokens.detach().clone()
        first = [_clone_cache(c) for c in cache]
        self._caches = (first, [_clone_cache(c) for c in first])
        layers = [blk.attn for blk in model.model.layers]
        self.graphs, self._logits = [], []
        try:
            # one eager step on copies warms up library handles and kernel selection
            scratch = [_clone_cache(c) for c in first]
            for attn, nxt in zip(layers, [_clone_cache(c) for c in first]):
                attn.decode_next = nxt
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                model(self.tokens.clone(), cache=scratch, use_cache=True)
            torch.cuda.current_stream().wait_stream(side)
            del scratch
            for parity in (0, 1):
                src, dst = self._caches[parity], self._caches[1 - parity]
                for attn, nxt in zip(layers, dst):
                    attn.decode_next = nxt
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    out = model(self.tokens, cache=src, use_cache=True)
                    for d, o in zip(dst, out["cache"]):  # layers off the fused path return new tensors
                        for a, b in zip(d["recurrent_state"], o["recurrent_state"]):
                            if a.data_ptr() != b.data_ptr():
                                a.copy_(b)
                        for a, b in zip(d["conv_state"], o["conv_state"]):
                            if a.data_ptr() != b.data_ptr():
                                a.copy_(b)
                    last = out["logits"][:, -1:]
                    if inference_fast_path(last):
                        _native.argmax_rows(last, out=self.tokens)  # straight into the token buffer
                    else:
                        self.tokens.copy_(last.argmax(-1))
                self.graphs.append(graph)
                self._logits.append(out["logits"])
        finally:
            for attn in layers:
                attn.decode_next = None
        self._parity = 0

    @property
    def cache(self):
        """The layer caches the next step reads."""
        return self._caches[self._parity]

    @property
    def logits(self):
        """The logits of the last step (valid until the next replay)."""
        return self._logits[1 - self._parity]

    def step(self):
        self.graphs[self._parity].replay()
        self._parity ^= 1
        return self.tokens
