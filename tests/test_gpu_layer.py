"""GPU parity of the layer-side HIP kernels, the CyclicFlowAttention layer and
the causal LM against the CPU oracle.

Layer and model references use ``oracle.model_oracle`` with ``mode="mirror"``
(fp32 arithmetic with the reference's bf16 casts of layers/cyfa.py and
modeling_cyfa.py) and ``op_mode="exact"`` (the CyFA op in float64): the
reference's own bf16 plumbing around an exact op. The layer output itself is
left unrounded (``cast_output=False``), so the bf16 layer is compared with an
fp32 output. Tolerances are the north star's (tests/tolerance.py): max-abs
2e-2, mean-rel 5e-3.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import model_oracle as MO
from tolerance import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF16_ULP = 2.0 ** -8  # relative spacing of bf16 values


def _bf16_close(got, ref, ulps=2):
    """Elementwise within `ulps` bf16 units of the reference's magnitude."""
    got = got.double().cpu()
    ref = ref.double().cpu()
    tol = ulps * BF16_ULP * ref.abs() + 1e-6
    bad = ((got - ref).abs() > tol).sum().item()
    assert bad == 0, f"{bad} elements off by more than {ulps} bf16 ulps; max diff {(got - ref).abs().max().item()}"


@pytest.mark.parametrize("D,gate,residual,prescale", [(256, True, False, 127.0), (1024, False, True, 1.0),
                                                      (2048, False, False, 1.0), (512, True, True, 1.0)])
def test_rms_norm_kernel(D, gate, residual, prescale):
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(D)
    rows = 300
    x = torch.randn(rows, D, generator=gen).bfloat16()
    w = 1 + 0.1 * torch.randn(D, generator=gen)
    gt = torch.randn(rows, D, generator=gen).bfloat16() if gate else None
    rs = torch.randn(rows, D, generator=gen).bfloat16() if residual else None
    out = _native.rms_norm(x.to(DEV), w.to(DEV), 1e-6, None if gt is None else gt.to(DEV),
                           None if rs is None else rs.to(DEV), prescale)
    s = x.double()
    if rs is not None:
        total, out = out
        s = (x.double() + rs.double()).bfloat16().double()
        assert torch.equal(total.cpu(), s.bfloat16())
    if prescale != 1.0:
        s = (s * prescale).bfloat16().double()
    ref = s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + 1e-6) * w.double()
    if gt is not None:
        ref = ref * torch.sigmoid(gt.double())
    _bf16_close(out, ref)


@pytest.mark.parametrize("B,T,W,split,cache", [(2, 100, 4, 64, False), (3, 1, 4, 64, True), (1, 37, 3, 192, True),
                                               (2, 2, 2, 96, False)])
def test_short_conv_kernel(B, T, W, split, cache):
    from cyclic_flow_attention import _native

    D = 192
    gen = torch.Generator().manual_seed(T + W)
    x = torch.randn(B, T, D, generator=gen).bfloat16()
    w = torch.randn(D, W, generator=gen).bfloat16()
    c = torch.randn(B, W - 1, D, generator=gen).bfloat16() if cache else None
    outs = _native.short_conv(x.to(DEV), w.to(DEV), None, None if c is None else c.to(DEV), split=split)
    got = torch.cat([o.cpu() for o in outs], dim=-1)
    hist = x.double() if c is None else torch.cat([c.double(), x.double()], 1)
    pad = W - 1 if c is None else 0
    ref = F.conv1d(F.pad(hist.transpose(1, 2), (pad, 0)), w.double()[:, None, :], groups=D).transpose(1, 2)
    _bf16_close(got, ref)


def test_silu_mul_and_gate_kernels():
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(3)
    gu = torch.randn(77, 2 * 264, generator=gen).bfloat16()
    got = _native.silu_mul(gu.to(DEV)).cpu()
    g, u = gu.double()[:, :264], gu.double()[:, 264:]
    _bf16_close(got, g * torch.sigmoid(g) * u)
    H = 4
    abd = torch.randn(3, 50, 3 * H, generator=gen).bfloat16()
    dt_bias = torch.randn(H, generator=gen)
    A_log = torch.randn(H, generator=gen)
    gg, beta, delta = (t.cpu().double() for t in _native.gates(abd.to(DEV), dt_bias.to(DEV), A_log.to(DEV)))
    a = abd.double()
    ref_g, ref_beta, ref_delta = MO.gate_activations(a[..., :H], a[..., H:2 * H], a[..., 2 * H:], dt_bias.double(),
                                                     A_log.double())
    torch.testing.assert_close(gg, ref_g, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(beta, ref_beta, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(delta, ref_delta, rtol=1e-5, atol=1e-6)


def _layer(hidden=1024, H=4, seed=0):
    """A seeded bf16 layer with the model's init policy (utils.py:122-129) and its state dict."""
    from cyclic_flow_attention.layers import CyclicFlowAttention

    torch.manual_seed(seed)
    layer = CyclicFlowAttention(hidden_size=hidden, num_heads=H, head_dim=256, num_slots=128).eval()
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith(".weight") and "norm" not in name:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
            elif name.endswith(".bias"):
                p.zero_()
            if not any(s in name for s in ("norm.weight", "readout", "A_log", "dt_bias")):
                p.data = p.data.bfloat16()
    sd = {"attn." + k: v.detach().float() for k, v in layer.state_dict().items()}
    cfg = dict(hidden_size=hidden, num_heads=H, head_dim=256, num_slots=128, norm_eps=1e-6, use_short_conv=True)
    return layer.to(DEV), sd, cfg


def _oracle_layer(sd, cfg, x, cache=None, use_cache=True):
    return MO.attention_layer(sd, "attn.", x.float(), cfg, cache=cache, use_cache=use_cache, mode="mirror",
                              op_mode="exact", cast_output=False)


def test_layer_config1_matches_oracle():
    """Config 1: one layer, B=1, T=2048, hidden 1024, 4 heads x 256, x ~ N(0, 1)."""
    layer, sd, cfg = _layer()
    x = torch.randn(1, 2048, 1024, generator=torch.Generator().manual_seed(0)).bfloat16()
    with torch.no_grad():
        y, cache = layer(x.to(DEV), use_cache=True)
    ry, rcache = _oracle_layer(sd, cfg, x)
    assert y.dtype == torch.bfloat16 and y.shape == (1, 2048, 1024)
    assert_close(y, ry, what="layer y")
    for a, b, n in zip(cache["recurrent_state"], rcache["recurrent_state"], ("hk", "hv", "clock")):
        assert_close(a, b, what=f"layer {n}")
    for a, b in zip(cache["conv_state"], rcache["conv_state"]):
        _bf16_close(a, b)  # projection outputs: GEMM summation orders differ by a rounding


def test_layer_fused_and_general_paths_agree():
    """The fused bf16 inference path and the general torch plumbing (the path
    right-padded batches take) give the same layer output."""
    layer, _, _ = _layer(seed=1)
    x = torch.randn(2, 300, 1024, generator=torch.Generator().manual_seed(1)).bfloat16().to(DEV)
    with torch.no_grad():
        y_fused, c_fused = layer(x, use_cache=True)
        y_gen, c_gen = layer(x, use_cache=True, attention_mask=torch.ones(2, 300, dtype=torch.long, device=DEV))
    assert_close(y_fused, y_gen.float(), what="fused vs general y")
    for a, b in zip(c_fused["conv_state"], c_gen["conv_state"]):
        assert torch.equal(a, b)


def test_layer_prefix_then_decode_matches_oracle():
    layer, sd, cfg = _layer(seed=2)
    x = torch.randn(2, 80, 1024, generator=torch.Generator().manual_seed(2)).bfloat16()
    with torch.no_grad():
        _, cache = layer(x[:, :67].to(DEV), use_cache=True)
        outs = []
        for t in range(67, 80):
            y, cache = layer(x[:, t:t + 1].to(DEV), cache=cache, use_cache=True)
            outs.append(y)
    _, rcache = _oracle_layer(sd, cfg, x[:, :67])
    routs = []
    for t in range(67, 80):
        ry, rcache = _oracle_layer(sd, cfg, x[:, t:t + 1], cache=rcache)
        routs.append(ry)
    assert_close(torch.cat(outs, 1), torch.cat(routs, 1), what="layer decode y")
    for a, b, n in zip(cache["recurrent_state"], rcache["recurrent_state"], ("hk", "hv", "clock")):
        assert_close(a, b, what=f"layer decode {n}")


def _model(name, seed=0, layers=None):
    from cyclic_flow_attention.utils import initialize_model, read_config

    config = read_config(name)
    if layers is not None:
        config.num_hidden_layers = layers
    model = initialize_model(config, std=0.02, seed=seed).to(DEV).eval()
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    cfg = {k: getattr(config, k) for k in config.__dataclass_fields__}
    return model, params, cfg


@pytest.mark.parametrize("name,layers,prompt", [("tiny.json", None, 70), ("cyclic_flow_attention_400m.json", 2, 130)])
def test_greedy_tokens_match_oracle(name, layers, prompt):
    """64 greedy decode steps after a chunkwise prompt. The oracle re-scores
    the GPU's token sequence (teacher forcing); every GPU token must be the
    oracle's argmax wherever the oracle's top-2 logit gap exceeds two bf16
    roundings of the largest logit. Inside that gap bf16 logits cannot decide
    the token (random-init models put about one step in ten there); such
    steps are only counted."""
    model, params, cfg = _model(name, seed=3, layers=layers)
    gen = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg["vocab_size"], (1, prompt), generator=gen)
    with torch.no_grad():
        out = model.generate(ids.to(DEV), max_new_tokens=64).cpu()
    assert out.shape == (1, prompt + 64)
    new = out[0, prompt:]
    logits, cache = MO.causal_lm(params, cfg, ids, use_cache=True, mode="mirror", op_mode="exact")
    last = logits[0, -1]
    ties = 0
    for i in range(64):
        top2 = last.topk(2)
        tok = int(new[i])
        if tok != int(top2.indices[0]):
            gap = float(last[top2.indices[0]] - last[tok])
            assert gap <= 2 * BF16_ULP * float(last.abs().max()), f"step {i}: token {tok} vs oracle {top2.indices[0]}"
            ties += 1
        logits, cache = MO.causal_lm(params, cfg, new[None, i:i + 1], cache=cache, use_cache=True, mode="mirror",
                                     op_mode="exact")
        last = logits[0, -1]
    print(f"{name}: {64 - ties} of 64 greedy tokens equal the oracle's argmax, {ties} near-ties")
    assert ties <= 16, f"{ties} of 64 steps were near-ties"


@pytest.mark.parametrize("name,layers,B", [("tiny.json", None, 2), ("cyclic_flow_attention_400m.json", 2, 4)])
def test_graphed_decode_matches_eager(name, layers, B):
    """Replays of the HIP-graph captured decode step equal eager steps bit for
    bit, replay after replay, with unrelated eager GPU work in between."""
    model, _, cfg = _model(name, seed=5, layers=layers)
    ids = torch.randint(0, cfg["vocab_size"], (B, 70), generator=torch.Generator().manual_seed(6)).to(DEV)
    with torch.no_grad():
        out = model(ids, use_cache=True)
        tok = out["logits"][:, -1:].argmax(-1)
        dec = model.graphed_decoder(out["cache"], tok)
        cache = out["cache"]
        for step in range(6):
            eager = model(tok, cache=cache, use_cache=True)
            cache = eager["cache"]
            tok = eager["logits"][:, -1:].argmax(-1)
            got = dec.step()
            assert torch.equal(dec.logits, eager["logits"]), f"step {step}: logits differ"
            assert torch.equal(got, tok), f"step {step}: tokens differ"
            torch.randn(256, 256, device=DEV).matmul(torch.randn(256, 256, device=DEV))  # unrelated work
            torch.cuda.synchronize()


@pytest.mark.parametrize("M,N,K,bias,ldx", [(1, 3072, 1024, False, 1024), (64, 12, 1024, True, 1024),
                                            (17, 256, 1024, False, 1024), (64, 1024, 256, True, 256),
                                            (33, 1024, 2816, False, 2816), (64, 32000, 1024, False, 1024),
                                            (5, 100, 64, True, 3 * 64), (64, 3340, 1024, True, 1024),
                                            (64, 1024, 2816, False, 2816), (40, 5000, 512, True, 512),
                                            (1, 32000, 2048, False, 2048), (1, 2048, 5632, True, 5632),
                                            (1, 6424, 2048, True, 3 * 2048), (1, 300, 544, True, 544)])
def test_linear_rows_kernel(M, N, K, bias, ldx):
    """cyfa_linear_rows against x W^T + b in float64: one bf16 rounding of an
    fp32 sum (bound: half a bf16 ulp of the result plus the fp32 summation
    error, K 2^-24 sum |x||w|, with a factor of two to spare). The one-row
    cases with K >= 512 run the streaming kernel with four, two and one W rows
    per wave, K a whole number of its 512-element chunks or not."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M * N + K)
    xs = torch.randn(M, ldx, generator=gen).bfloat16()
    x = xs[:, :K]  # rows ldx apart
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16()
    b = torch.randn(N, generator=gen).bfloat16() if bias else None
    with torch.no_grad():
        y = _native.linear(xs.to(DEV)[:, :K], w.to(DEV), None if b is None else b.to(DEV))
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    ref = x.double() @ w.double().T + (0 if b is None else b.double())
    bound = 2 * (BF16_ULP / 2 * ref.abs() + K * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T)) + 1e-30
    err = (y.cpu().double() - ref).abs()
    assert (err <= bound).all(), f"max err {err.max().item()} vs bound {bound[err.argmax() // N, err.argmax() % N].item()}"


@pytest.mark.parametrize("N,K", [(32000, 1024), (3340, 1024), (5000, 512)])
def test_linear_rows_tile_shape_does_not_change_bits(N, K):
    """The launcher picks the workgroup tile per call (64 rows and 2 rows get
    different tiles at these N); every output is the same fixed-order sum in
    any tile, so a row's result does not depend on the other rows. (A single
    row with K >= 512 takes the streaming one-row kernel, whose sums run in
    another order; its accuracy is checked against float64 above.)"""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(N + K)
    x = torch.randn(64, K, generator=gen).bfloat16().to(DEV)
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16().to(DEV)
    b = torch.randn(N, generator=gen).bfloat16().to(DEV)
    with torch.no_grad():
        full = _native.linear(x, w, b)
        rows = [_native.linear(x[m:m + 2], w, b) for m in (0, 17, 62)]
    torch.cuda.synchronize()
    for m, y in zip((0, 17, 62), rows):
        assert torch.equal(y, full[m:m + 2]), f"rows {m}, {m + 1}"


@pytest.mark.parametrize("M,N,K,kind", [(64, 5632, 1024, "swiglu"), (64, 3340, 1024, "norm"),
                                        (64, 1024, 2816, "residual"), (32, 1024, 1024, "residual")])
def test_linear_rows_prefetch_changes_no_bit(M, N, K, kind):
    """The extra workgroups that read other weights into the caches for the
    next launch (one range with the span its workgroups read, one without)
    leave the projection's result unchanged, bit for bit; two calls in a
    row, the second with fewer rows."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M + N + K)
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16().to(DEV)
    nw = (1 + 0.1 * torch.randn(K, generator=gen)).to(DEV)
    nxt = (0.05 * torch.randn(2048, 1024, generator=gen)).bfloat16().to(DEV)
    other = torch.randn(1 << 20, generator=gen).to(DEV)[:777_777]  # 3.1 MB, no span
    pf = ((nxt, _native.linear_rows_span(M, 2048, 1024, norm=1)), other)
    assert pf[0][1] > 0

    def run(x, prefetch):
        if kind == "swiglu":
            return _native.norm_linear(x, nw, 1e-6, w, swiglu=True, prefetch=prefetch)[1]
        if kind == "norm":
            return _native.norm_linear(x, nw, 1e-6, w, prefetch=prefetch)[1]
        return _native.linear(x, w, residual=torch.ones(x.shape[0], N, dtype=torch.bfloat16, device=DEV),
                              prefetch=prefetch)

    for rows in (M, M // 2 + 1):
        x = torch.randn(rows, K, generator=gen).bfloat16().to(DEV)
        with torch.no_grad():
            ref, got = run(x, ()), run(x, pf)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), rows




@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (64, 1024, 2816), (17, 3340, 256)])
def test_linear_rows_residual_add(M, N, K):
    """The residual-add epilogue of cyfa_linear_rows (the block's x + o_proj(o)
    and x + down(h)) equals the projection followed by a bf16 add, bit for bit."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=gen).bfloat16().to(DEV)
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16().to(DEV)
    b = torch.randn(N, generator=gen).bfloat16().to(DEV)
    r = torch.randn(M, N + 8, generator=gen).bfloat16().to(DEV)[:, :N]  # rows N + 8 apart
    with torch.no_grad():
        got = _native.linear(x, w, b, residual=r)
        ref = r + _native.linear(x, w, b)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,residual,swiglu,K", [(1, False, False, 1024), (37, True, False, 1024),
                                                 (64, True, False, 1024), (64, True, True, 1024),
                                                 (5, True, True, 2048), (64, False, False, 512),
                                                 (1, True, False, 2048), (1, True, True, 2048),
                                                 (1, False, True, 1024)])
def test_norm_linear_rows(M, residual, swiglu, K):
    """cyfa_norm_linear_rows (the pre-norm inside the projection): s equals the
    separate residual add bit for bit; y against the norm and the projection
    in float64, with the bound of one bf16 rounding of each normalised input
    and of the result plus the fp32 summation error (factor two to spare); and
    y equals rms_norm followed by linear except where the norm's sum of squares,
    added in another order, moves an input across a bf16 rounding boundary."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M * 7 + K + 3 * residual + swiglu)
    N = 2 * 1408 if swiglu else 3340
    x = torch.randn(M, K, generator=gen).bfloat16()
    r = torch.randn(M, K, generator=gen).bfloat16() if residual else None
    nw = 1.0 + 0.1 * torch.randn(K, generator=gen)
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16()
    b = None if swiglu else torch.randn(N, generator=gen).bfloat16()
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    with torch.no_grad():
        s, y = _native.norm_linear(d(x), d(nw), 1e-6, d(w), d(b), residual=d(r), swiglu=swiglu)
        if residual:
            s_ref, h_ref = _native.rms_norm(d(x), d(nw), 1e-6, residual=d(r))
        else:
            s_ref, h_ref = d(x), _native.rms_norm(d(x), d(nw), 1e-6)
        y_ref = _native.linear_swiglu(h_ref, d(w)) if swiglu else _native.linear(h_ref, d(w), d(b))
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref)
    assert y.shape == y_ref.shape and not y.isnan().any()
    if not swiglu:
        s64 = s.cpu().double()
        h64 = s64 * torch.rsqrt(s64.pow(2).mean(-1, keepdim=True) + 1e-6) * nw.double()
        y64 = h64 @ w.double().T + b.double()
        mag = h64.abs() @ w.double().abs().T
        bound = 2 * (BF16_ULP / 2 * (y64.abs() + mag) + K * 2.0 ** -24 * mag) + 1e-30
        err = (y.cpu().double() - y64).abs()
        assert (err <= bound).all(), f"max err {err.max().item()}"
    # one input moved by an ulp changes about a tenth of its row's outputs
    rows = int((y != y_ref).reshape(M, -1).any(-1).sum())
    assert rows <= max(1, M // 10), f"{rows} of {M} rows differ from rms_norm + linear"


@pytest.mark.parametrize("M,residual,swiglu,K", [(1, False, False, 1024), (37, True, False, 1024),
                                                 (64, False, False, 1024), (64, False, True, 1024),
                                                 (5, True, True, 2048), (64, False, False, 512)])
def test_norm_linear_rows_folded(M, residual, swiglu, K):
    """cyfa_norm_linear_rows with the norm weight folded into the projection's
    weight (NULL norm weight): y = bf16(rs (s W'^T) + bias) with W' =
    bf16(W diag(w)), checked in float64 with the bound of the result's bf16
    rounding plus the fp32 summation error (factor two to spare); with SwiGLU,
    the gate and up values rounded to bf16 as the kernel rounds them, then the
    product; s equals the separate residual add bit for bit."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M * 11 + K + 3 * residual + swiglu)
    N = 2 * 1408 if swiglu else 3340
    x = torch.randn(M, K, generator=gen).bfloat16()
    r = torch.randn(M, K, generator=gen).bfloat16() if residual else None
    nw = 1.0 + 0.1 * torch.randn(K, generator=gen)
    w = (0.05 * torch.randn(N, K, generator=gen)).bfloat16()
    b = None if swiglu else torch.randn(N, generator=gen).bfloat16()
    wf = _native.fold_norm_weight(w, nw)
    assert torch.equal(wf, (w.float() * nw).bfloat16())
    d = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    with torch.no_grad():
        s, y = _native.norm_linear(d(x), None, 1e-6, d(wf), d(b), residual=d(r), swiglu=swiglu)
        s_ref = d(x) if r is None else (d(x).float() + d(r).float()).bfloat16()
    torch.cuda.synchronize()
    assert torch.equal(s, s_ref)
    s64 = s.cpu().double()
    rs = torch.rsqrt(s64.pow(2).mean(-1, keepdim=True) + 1e-6)
    p64 = rs * (s64 @ wf.double().T)
    mag = rs * (s64.abs() @ wf.double().abs().T)
    if not swiglu:
        y64 = p64 + b.double()
        bound = 2 * (BF16_ULP / 2 * (y64.abs() + mag) + K * 2.0 ** -24 * mag) + 1e-30
        err = (y.cpu().double() - y64).abs()
        assert (err <= bound).all(), f"max err {err.max().item()}"
    else:
        # y = bf16(g sigmoid(g) u) of g, u rounded to bf16: propagate each one's
        # rounding and summation error through the product, plus the last rounding
        groups = N // 32
        gi = (32 * torch.arange(groups)[:, None] + torch.arange(16)).reshape(-1)
        g64, u64 = p64[:, gi], p64[:, gi + 16]
        eg = BF16_ULP / 2 * g64.abs() + K * 2.0 ** -24 * mag[:, gi]
        eu = BF16_ULP / 2 * u64.abs() + K * 2.0 ** -24 * mag[:, gi + 16]
        sg = torch.sigmoid(g64)
        y64 = g64 * sg * u64
        dy_dg = (u64 * (sg + g64 * sg * (1 - sg))).abs()
        bound = 2 * (dy_dg * eg + (g64 * sg).abs() * eu + BF16_ULP / 2 * y64.abs()) + 1e-30
        err = (y.cpu().double() - y64).abs()
        assert (err <= bound).all(), f"max err {err.max().item()}"


@pytest.mark.parametrize("B,state,inplace,split,own_gate,H", [
    (3, True, False, True, False, 4), (2, False, False, True, False, 4), (4, True, True, True, False, 4),
    (64, True, True, True, False, 4), (3, True, True, False, False, 4), (1, True, True, True, False, 4),
    (64, True, True, False, True, 4), (3, True, True, True, True, 4), (1, False, False, False, True, 4),
    (17, True, False, False, True, 4),
    # configuration 5's heads (the 1.4B model's single-sequence step), both forms and the in-kernel gate
    (1, True, True, False, False, 8), (1, True, True, True, False, 8), (1, True, True, False, True, 8),
    (16, True, True, False, True, 8)])
def test_decode_layer_step_equals_separate_kernels(B, state, inplace, split, own_gate, H):
    """cyfa_decode_layer_step (short convolution, gates, decode op and gated
    output norm in one kernel, or in the two kernels of the small-batch split)
    against the separate kernels on the same inputs: the same arithmetic in
    the same order, so outputs, states and the new conv cache are
    bit-identical. own_gate: the kernel also forms the gate from g0 (the
    second projection of g_proj), against _native.linear(g0, W, b)."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops import fused_recurrent_cyfa
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    D = 3 * H * 256
    gen = torch.Generator().manual_seed(B + 10 * state + 100 * inplace + 1000 * H)
    qkv_rows = torch.randn(B, 1, D + 40, generator=gen).bfloat16().to(DEV)
    qkv = qkv_rows[..., :D]  # rows D + 40 apart
    cache = (0.5 * torch.randn(B, 3, D, generator=gen)).bfloat16().to(DEV) if state else None
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16().to(DEV)
    abd = torch.randn(B, 1, 3 * H, generator=gen).bfloat16().to(DEV)
    dt_bias, A_log = torch.randn(H, generator=gen).to(DEV), torch.randn(H, generator=gen).to(DEV)
    gate = torch.randn(B, 1, H * 256, generator=gen).bfloat16().to(DEV)
    g0_rows = torch.randn(B, 1, 256 + 24, generator=gen).bfloat16().to(DEV)
    g0 = g0_rows[..., 8:264]  # a column slice, rows 280 apart (as in the layer's input projection)
    g_w = (0.06 * torch.randn(H * 256, 256, generator=gen)).bfloat16().to(DEV)
    g_b = (0.5 * torch.randn(H * 256, generator=gen)).bfloat16().to(DEV)
    if own_gate:
        gate = _native.linear(g0, g_w, g_b)
    nw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    qw, kw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV), (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    readout = (torch.eye(127).expand(H, 127, 127) + 0.05 * torch.randn(H, 127, 127, generator=gen)).to(DEV)
    init = None
    if state:
        init = (0.3 * torch.randn(B, H, 256, 128, generator=gen).to(DEV),
                0.3 * torch.randn(B, H, 128, 256, generator=gen).to(DEV), 50 * torch.rand(B, H, generator=gen).to(DEV))
    table = _native.readout_table(readout)
    with torch.no_grad():
        # separate kernels
        tail_ref = torch.empty(B, 3, D, dtype=torch.bfloat16, device=DEV)
        q, k, v = _native.short_conv(qkv, wconv, None, cache, split=H * 256, cache_out=tail_ref)
        g, beta, delta = _native.gates(abd, dt_bias, A_log)
        o, st = fused_recurrent_cyfa(q.view(B, 1, H, 256), k.view(B, 1, H, 256), v.view(B, 1, H, 256), g, delta, beta,
                                     readout, qw, kw, initial_state=None if init is None else tuple(t.clone() for t in init),
                                     output_final_state=True, table=table)
        ref = _native.rms_norm(o.view(B, 1, H, 256), nw, 1e-6, gate.view(B, 1, H, 256), prescale=127.0)
        # one kernel
        cache_in = None if cache is None else cache.clone()
        tail = cache_in if (inplace and cache_in is not None) else torch.empty(B, 3, D, dtype=torch.bfloat16, device=DEV)
        st_in = None if init is None else tuple(t.clone() for t in init)
        got, st2 = decode_layer_step(qkv, cache_in, tail, wconv, abd, dt_bias, A_log, None if own_gate else gate, nw,
                                     1e-6, 127.0, table, qw, kw, 1e-6, 1e-6, H, initial_state=st_in,
                                     output_final_state=True, inplace=inplace and st_in is not None, split=split,
                                     g_proj=(g0, g_w, g_b) if own_gate else None)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(tail, tail_ref)
    for a, b in zip(st2, st):
        assert torch.equal(a, b)
    if inplace and st_in is not None:
        assert st2[0].data_ptr() == st_in[0].data_ptr()


@pytest.mark.parametrize("B,H", [(1, 8), (4, 4), (16, 4), (64, 4)])
def test_decode_layer_step_prefetch_changes_nothing(B, H):
    """The layer step's cache prefetch (extra workgroups reading device ranges
    at B H <= 64; ignored above) leaves every output bit as it is: o', the
    states and the conv cache equal the step without it. The ranges have odd
    sizes (a partial 16 KiB unit, a 16-byte one), and two are read per
    consumer span (one a whole number of 16 KiB pieces, one not, with a
    partial last span)."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    D = 3 * H * 256
    gen = torch.Generator().manual_seed(77 + B + H)
    qkv = torch.randn(B, 1, D, generator=gen).bfloat16().to(DEV)
    cache = (0.5 * torch.randn(B, 3, D, generator=gen)).bfloat16().to(DEV)
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16().to(DEV)
    abd = torch.randn(B, 1, 3 * H, generator=gen).bfloat16().to(DEV)
    dt_bias, A_log = torch.randn(H, generator=gen).to(DEV), torch.randn(H, generator=gen).to(DEV)
    gate = torch.randn(B, 1, H * 256, generator=gen).bfloat16().to(DEV)
    nw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    qw, kw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV), (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    table = _native.readout_table((torch.eye(127).expand(H, 127, 127)
                                   + 0.05 * torch.randn(H, 127, 127, generator=gen)).contiguous().to(DEV))
    init = (0.3 * torch.randn(B, H, 256, 128, generator=gen).to(DEV),
            0.3 * torch.randn(B, H, 128, 256, generator=gen).to(DEV), 50 * torch.rand(B, H, generator=gen).to(DEV))
    ranges = (torch.randn(4_200_000, device=DEV).bfloat16(),
              torch.randn(250_003, device=DEV), torch.randn(4, device=DEV))
    outs = []
    with torch.no_grad():
        for pf in ((), ((ranges[0], 32768), (ranges[1], 90112), ranges[2])):
            tail = torch.empty(B, 3, D, dtype=torch.bfloat16, device=DEV)
            o, st = decode_layer_step(qkv, cache, tail, wconv, abd, dt_bias, A_log, gate, nw, 1e-6, 127.0, table, qw,
                                      kw, 1e-6, 1e-6, H, initial_state=tuple(t.clone() for t in init),
                                      output_final_state=True, prefetch=pf)
            outs.append((o, st, tail))
    torch.cuda.synchronize()
    (o0, st0, t0), (o1, st1, t1) = outs
    assert torch.equal(o0, o1) and torch.equal(t0, t1)
    for a, b in zip(st0, st1):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H,big", [(1, 8, 16), (4, 4, 32), (16, 4, 32)])
def test_decode_layer_step_small_batch_equals_rows_of_a_large_batch(B, H, big):
    """At B H <= 64 the layer step launches extra workgroups that read every
    step workgroup's state, table and g_proj[1] rows into its XCD's L2 ahead
    of it; above 64 there are none. Each (batch, head) is computed alone in
    either case, so the first B rows of a batch of `big` (B H > 64) equal the
    same rows stepped as a batch of B, bit for bit: o', both states, the
    clock and the conv cache, with the gate formed in the kernel."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    D = 3 * H * 256
    gen = torch.Generator().manual_seed(300 + B + H)
    qkv = torch.randn(big, 1, D, generator=gen).bfloat16().to(DEV)
    cache = (0.5 * torch.randn(big, 3, D, generator=gen)).bfloat16().to(DEV)
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16().to(DEV)
    abd = torch.randn(big, 1, 3 * H, generator=gen).bfloat16().to(DEV)
    dt_bias, A_log = torch.randn(H, generator=gen).to(DEV), torch.randn(H, generator=gen).to(DEV)
    g0 = torch.randn(big, 1, 256, generator=gen).bfloat16().to(DEV)
    g_w = (0.06 * torch.randn(H * 256, 256, generator=gen)).bfloat16().to(DEV)
    g_b = (0.5 * torch.randn(H * 256, generator=gen)).bfloat16().to(DEV)
    nw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    qw, kw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV), (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    table = _native.readout_table((torch.eye(127).expand(H, 127, 127)
                                   + 0.05 * torch.randn(H, 127, 127, generator=gen)).contiguous().to(DEV))
    init = (0.3 * torch.randn(big, H, 256, 128, generator=gen).to(DEV),
            0.3 * torch.randn(big, H, 128, 256, generator=gen).to(DEV), 50 * torch.rand(big, H, generator=gen).to(DEV))
    outs = []
    with torch.no_grad():
        for n in (big, B):
            tail = torch.empty(n, 3, D, dtype=torch.bfloat16, device=DEV)
            o, st = decode_layer_step(qkv[:n], cache[:n], tail, wconv, abd[:n], dt_bias, A_log, None, nw, 1e-6, 127.0,
                                      table, qw, kw, 1e-6, 1e-6, H,
                                      initial_state=tuple(t[:n].clone() for t in init), output_final_state=True,
                                      g_proj=(g0[:n], g_w, g_b))
            outs.append((o, st, tail))
    torch.cuda.synchronize()
    (o0, st0, t0), (o1, st1, t1) = outs
    assert torch.equal(o0[:B], o1) and torch.equal(t0[:B], t1)
    for a, b in zip(st0, st1):
        assert torch.equal(a[:B], b)


@pytest.mark.parametrize("B,H,gate_in_kernel", [(1, 8, True), (1, 4, False), (2, 8, True), (3, 8, False),
                                                 (8, 4, True), (2, 16, True)])
def test_decode_layer_step_split_workgroups_equal_one(B, H, gate_in_kernel):
    """With its outputs apart from its inputs and B H <= 32 the layer step runs
    4 (B H <= 16) or 2 step workgroups per (b, h), each computing the whole
    step and storing its share of hk', hv', o and (workgroup 0) the conv cache
    and the clock; in place it runs one. Both give the same bits: o', both
    states, the clock and the conv cache."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    D = 3 * H * 256
    gen = torch.Generator().manual_seed(500 + 10 * B + H)
    qkv = torch.randn(B, 1, D, generator=gen).bfloat16().to(DEV)
    cache = (0.5 * torch.randn(B, 3, D, generator=gen)).bfloat16().to(DEV)
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16().to(DEV)
    abd = torch.randn(B, 1, 3 * H, generator=gen).bfloat16().to(DEV)
    dt_bias, A_log = torch.randn(H, generator=gen).to(DEV), torch.randn(H, generator=gen).to(DEV)
    nw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    qw, kw = (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV), (1 + 0.1 * torch.randn(256, generator=gen)).to(DEV)
    table = _native.readout_table((torch.eye(127).expand(H, 127, 127)
                                   + 0.05 * torch.randn(H, 127, 127, generator=gen)).contiguous().to(DEV))
    init = (0.3 * torch.randn(B, H, 256, 128, generator=gen).to(DEV),
            0.3 * torch.randn(B, H, 128, 256, generator=gen).to(DEV), 50 * torch.rand(B, H, generator=gen).to(DEV))
    if gate_in_kernel:
        gate, g_proj = None, (torch.randn(B, 1, 256, generator=gen).bfloat16().to(DEV),
                              (0.06 * torch.randn(H * 256, 256, generator=gen)).bfloat16().to(DEV),
                              (0.5 * torch.randn(H * 256, generator=gen)).bfloat16().to(DEV))
    else:
        gate, g_proj = torch.randn(B, 1, H * 256, generator=gen).bfloat16().to(DEV), None
    outs = []
    with torch.no_grad():
        for inplace in (False, True):
            tail = torch.empty(B, 3, D, dtype=torch.bfloat16, device=DEV)
            st_in = tuple(t.clone() for t in init)
            o, st = decode_layer_step(qkv, cache, tail, wconv, abd, dt_bias, A_log, gate, nw, 1e-6, 127.0, table, qw,
                                      kw, 1e-6, 1e-6, H, initial_state=st_in, output_final_state=True,
                                      inplace=inplace, g_proj=g_proj)
            if inplace:
                assert st[0].data_ptr() == st_in[0].data_ptr()
            outs.append((o, st, tail))
    torch.cuda.synchronize()
    (o0, st0, t0), (o1, st1, t1) = outs
    assert torch.equal(o0, o1) and torch.equal(t0, t1)
    for a, b in zip(st0, st1):
        assert torch.equal(a, b)


def test_model_decode_prefetch_changes_nothing():
    """A 400M-shape model (2 layers) decoding at B=2: the decode steps with
    the layers' weight prefetch equal the steps without it, bit for bit."""
    model, _, cfg = _model("cyclic_flow_attention_400m.json", seed=9, layers=2)
    ids = torch.randint(0, cfg["vocab_size"], (2, 70), generator=torch.Generator().manual_seed(10)).to(DEV)
    logits = []
    with torch.no_grad():
        for on in (False, True):
            for blk in model.model.layers:
                blk.attn.prefetch_weights = on
            out = model(ids, use_cache=True)
            cache, tok, run = out["cache"], out["logits"][:, -1:].argmax(-1), []
            for _ in range(4):
                out = model(tok, cache=cache, use_cache=True)
                cache, tok = out["cache"], out["logits"][:, -1:].argmax(-1)
                run.append(out["logits"])
            logits.append(torch.cat(run, 1))
    torch.cuda.synchronize()
    assert torch.equal(logits[0], logits[1])


@pytest.mark.parametrize("M", [1, 37, 64])
def test_linear_swiglu_equals_projection_then_silu_mul(M):
    """The SwiGLU epilogue of cyfa_linear_rows (interleaved gate|up weight)
    equals the [gate | up] projection followed by silu_mul, bit for bit: every
    output column is the same fixed-order sum and the same roundings."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M)
    F_, K = 2816, 1024
    x = torch.randn(M, K, generator=gen).bfloat16().to(DEV)
    wg = (0.05 * torch.randn(F_, K, generator=gen)).bfloat16().to(DEV)
    wu = (0.05 * torch.randn(F_, K, generator=gen)).bfloat16().to(DEV)
    with torch.no_grad():
        ref = _native.silu_mul(_native.linear(x, torch.cat([wg, wu], 0)))
        got = _native.linear_swiglu(x, _native.interleave_gate_up(wg, wu))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_padded_generation_matches_individual_prompts():
    """generate_batch over right-padded prompts gives each prompt's own greedy
    continuation (the reference's tests/test_inference.py:56-65)."""
    from cyclic_flow_attention.generation import generate, generate_batch

    model, _, _ = _model("tiny.json", seed=0)
    prompts = [[10, 20, 30], list(range(4, 67))]
    expected = [generate(model, ids, max_new_tokens=8) for ids in prompts]
    actual = generate_batch(model, prompts, max_new_tokens=8)
    assert actual == expected
    with pytest.raises(ValueError):
        generate_batch(model, [[1], []])


def test_checkpoint_round_trip_and_seeded_sampling(tmp_path):
    """A saved and reloaded model gives the same logits, and sampling with a
    seed repeats (the reference's tests/test_inference.py:20-53)."""
    from cyclic_flow_attention.generation import generate
    from cyclic_flow_attention.utils import load_model, save_model

    model, _, _ = _model("tiny.json", seed=1)
    ids = (torch.arange(65)[None] + 32).to(DEV)
    with torch.no_grad():
        reference = model(ids)["logits"]
    save_model(model, tmp_path)
    loaded, _ = load_model(tmp_path)
    loaded = loaded.to(DEV).eval()
    with torch.no_grad():
        assert torch.equal(loaded(ids)["logits"], reference)
    first = generate(loaded, [32, 33], 4, temperature=0.8, top_p=0.9, seed=5)
    second = generate(loaded, [32, 33], 4, temperature=0.8, top_p=0.9, seed=5)
    assert first == second and len(first) == 4
    with pytest.raises(ValueError):
        generate(loaded, [32], 4, top_p=0.0)


def test_argmax_rows_equals_torch_argmax():
    """cyfa_argmax_rows gives torch.argmax's index: the first of tied maxima,
    NaN largest, an all -inf row at 0, and rows that end off a multiple of 8."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(9)
    x = (torch.randint(-20, 20, (7, 32000), generator=gen) / 4).bfloat16()  # many ties
    x[3, 12345] = float("nan")
    x[4, 77] = float("nan")
    x[4, 5] = float("nan")
    x[5] = float("-inf")
    xd = x.to(DEV)
    got = _native.argmax_rows(xd)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), xd.argmax(-1).cpu())
    y = torch.randn(5, 104, generator=gen).bfloat16().to(DEV)[:, :100]  # rows 104 apart, 100 wide
    assert torch.equal(_native.argmax_rows(y).cpu(), y.argmax(-1).cpu())


def _bf16_ulp(b):
    """Spacing of bf16 values at b (bf16 keeps 8 significant bits)."""
    _, e = torch.frexp(b.abs().clamp_min(2.0 ** -126))
    return torch.ldexp(torch.ones_like(b), e - 8)


def _near_rounding_edge(v64, err):
    """Entries whose float64 value lies within err of a bf16 rounding edge: an
    fp32 sum may round them to the neighbouring bf16 value."""
    b = v64.bfloat16().double()
    return (_bf16_ulp(b) / 2 - (v64 - b).abs()) < err


@pytest.mark.parametrize("M,H,K", [(200, 4, 1024), (64, 4, 1024), (131, 8, 2048)])
def test_gate_path_matches_float64(M, H, K):
    """cyfa_gate_path (g_proj[0], a|b|d, the gate activations and g_proj[1] in
    one launch) against float64 with the kernel's rounding points: g0 and abd
    rounded to bf16 (where the float64 value lies within a statistical bound
    of the fp32 summation error of a rounding edge, either neighbour), the gates of the rounded
    a|b|d, and gate = bf16(g0 W_g1^T + b) within its last rounding plus the
    fp32 summation error and the effect of any such neighbour in g0."""
    from cyclic_flow_attention import _native

    gen = torch.Generator().manual_seed(M + H + K)
    Dv = 256 * H
    x = torch.randn(M, K, generator=gen).bfloat16()
    w1 = (0.03 * torch.randn(256 + 3 * H, K, generator=gen)).bfloat16()
    abd_bias = torch.cat([torch.zeros(H), torch.randn(2 * H, generator=gen)]).bfloat16()
    w2 = (0.05 * torch.randn(Dv, 256, generator=gen)).bfloat16()
    b2 = torch.randn(Dv, generator=gen).bfloat16()
    dt_bias = torch.randn(H, generator=gen)
    A_log = torch.rand(H, generator=gen)
    d = lambda t: t.to(DEV)  # noqa: E731
    with torch.no_grad():
        gate, g, beta, delta = _native.gate_path(d(x), d(w1), d(abd_bias), d(w2), d(b2), d(dt_bias), d(A_log), H)
    torch.cuda.synchronize()
    x64, w164 = x.double(), w1.double()
    c64 = x64 @ w164.T
    # fp32 summation error of the K exact bf16 products: each rounding errs by
    # at most 2^-24 of its running sum, and as independent errors over sums
    # that grow like a random walk they total a standard deviation near
    # 2^-25 * sum|x w|; 8 * 2^-24 * sum|x w| is about 16 of them (the K * 2^-24
    # worst case would mark most entries as near an edge)
    e1 = 8 * 2.0 ** -24 * (x64.abs() @ w164.abs().T)
    g0_64, abd64 = c64[:, :256], c64[:, 256:] + abd_bias.double()
    g0b = g0_64.bfloat16().double()
    near0 = _near_rounding_edge(g0_64, e1[:, :256])
    assert near0.double().mean() < 0.05
    w264 = w2.double()
    p64 = g0b @ w264.T + b2.double()
    mag2 = g0b.abs() @ w264.abs().T
    flip = (near0.double() * _bf16_ulp(g0b)) @ w264.abs().T
    bound = 2 * (BF16_ULP / 2 * (p64.abs() + mag2) + 256 * 2.0 ** -24 * mag2 + flip) + 1e-30
    err = (gate.cpu().double() - p64).abs()
    assert (err <= bound).all(), f"gate: max err {err.max().item()}"
    ab = abd64.bfloat16().double()
    nearab = _near_rounding_edge(abd64, e1[:, 256:] + 2.0 ** -24 * abd64.abs())
    a, b, dd = ab[:, :H], ab[:, H:2 * H], ab[:, 2 * H:]
    g64 = -torch.exp(A_log.double()) * torch.nn.functional.softplus(a + dt_bias.double())
    for got, ref, deriv, nr, name in (
        (g, g64, torch.exp(A_log.double()) * torch.sigmoid(a + dt_bias.double()), nearab[:, :H], "g"),
        (beta, torch.sigmoid(b), torch.sigmoid(b) * (1 - torch.sigmoid(b)), nearab[:, H:2 * H], "beta"),
        (delta, torch.sigmoid(dd), torch.sigmoid(dd) * (1 - torch.sigmoid(dd)), nearab[:, 2 * H:], "delta"),
    ):
        span = _bf16_ulp(ab[:, :H] if name == "g" else (b if name == "beta" else dd))
        tol = 4e-6 * ref.abs() + nr.double() * deriv * span + 1e-7
        e = (got.cpu().double() - ref).abs()
        assert (e <= tol).all(), f"{name}: max err {e.max().item()}"
