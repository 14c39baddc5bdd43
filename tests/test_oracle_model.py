"""Pins of the oracle's layer / block / model plumbing (oracle/model_oracle.py).

Each piece is checked against a library routine that computes the same
textbook operation by another route (torch.nn.functional), or against an
invariant the reference relies on: prefix + continuation equals the full
sequence (tests/test_inference.py:20-34 of the reference), and right padding
is neutral (tests/test_inference.py:56-65).
"""

import math

import torch
import torch.nn.functional as F

from oracle import model_oracle as MO

D64 = torch.float64


def _layer_params(hidden=64, H=1, Dh=32, seed=0):
    """A small random state dict with the reference's parameter names."""
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s, std=0.1: std * torch.randn(*s, dtype=D64, generator=gen)
    pre = "attn."
    p = {
        pre + "q_proj.weight": r(H * Dh, hidden), pre + "k_proj.weight": r(H * Dh, hidden),
        pre + "v_proj.weight": r(H * Dh, hidden), pre + "a_proj.weight": r(H, hidden),
        pre + "b_proj.weight": r(H, hidden), pre + "b_proj.bias": r(H),
        pre + "d_proj.weight": r(H, hidden), pre + "d_proj.bias": r(H),
        pre + "dt_bias": r(H), pre + "A_log": r(H).abs().log(),
        pre + "readout": torch.eye(127, dtype=D64).expand(H, 127, 127) + r(H, 127, 127, std=0.05),
        pre + "q_norm.weight": 1 + r(Dh), pre + "k_norm.weight": 1 + r(Dh),
        pre + "q_conv1d.weight": r(H * Dh, 1, 4, std=0.5), pre + "k_conv1d.weight": r(H * Dh, 1, 4, std=0.5),
        pre + "v_conv1d.weight": r(H * Dh, 1, 4, std=0.5),
        pre + "g_proj.0.weight": r(Dh, hidden), pre + "g_proj.1.weight": r(H * Dh, Dh),
        pre + "g_proj.1.bias": r(H * Dh), pre + "o_norm.weight": 1 + r(Dh),
        pre + "o_proj.weight": r(hidden, H * Dh),
    }
    cfg = dict(hidden_size=hidden, num_heads=H, head_dim=Dh, num_slots=128, norm_eps=1e-6, use_short_conv=True)
    return p, pre, cfg


def test_linear_and_rms_norm_match_library_routines():
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(3, 5, 16, dtype=D64, generator=gen)
    w = torch.randn(8, 16, dtype=D64, generator=gen)
    b = torch.randn(8, dtype=D64, generator=gen)
    torch.testing.assert_close(MO.linear(x, w, b), F.linear(x, w, b))
    nw = torch.rand(16, dtype=D64, generator=gen) + 0.5
    gate = torch.randn(3, 5, 16, dtype=D64, generator=gen)
    ref = F.rms_norm(x, (16,), nw, eps=1e-6) * torch.sigmoid(gate)
    torch.testing.assert_close(MO.rms_norm(x, nw, 1e-6, gate), ref)


def test_short_conv_matches_conv1d_and_continues_from_its_cache():
    gen = torch.Generator().manual_seed(2)
    B, T, D, W = 2, 11, 6, 4
    x = torch.randn(B, T, D, dtype=D64, generator=gen)
    w = torch.randn(D, 1, W, dtype=D64, generator=gen)
    bias = torch.randn(D, dtype=D64, generator=gen)
    y, cache = MO.short_conv(x, w, bias)
    ref = F.conv1d(F.pad(x.transpose(1, 2), (W - 1, 0)), w, bias, groups=D).transpose(1, 2)
    torch.testing.assert_close(y, ref)
    torch.testing.assert_close(cache, x[:, -(W - 1):])
    # split the sequence: the cache carries the history exactly
    y1, c1 = MO.short_conv(x[:, :7], w, bias)
    y2, c2 = MO.short_conv(x[:, 7:], w, bias, cache=c1)
    torch.testing.assert_close(torch.cat([y1, y2], 1), y)
    torch.testing.assert_close(c2, cache)
    # a length-aware cache of right-padded rows equals the cache of the unpadded prefix
    lengths = torch.tensor([T, 5])
    _, cl = MO.short_conv(x, w, bias, lengths=lengths)
    _, c5 = MO.short_conv(x[1:, :5], w, bias)
    torch.testing.assert_close(cl[1:], c5)


def test_attention_layer_prefix_then_decode_equals_full_sequence():
    p, pre, cfg = _layer_params()
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 70, cfg["hidden_size"], dtype=D64, generator=gen)
    full, _ = MO.attention_layer(p, pre, x, cfg, use_cache=True)
    y, cache = MO.attention_layer(p, pre, x[:, :64], cfg, use_cache=True)
    outs = [y]
    for t in range(64, 70):
        y, cache = MO.attention_layer(p, pre, x[:, t:t + 1], cfg, cache=cache, use_cache=True)
        outs.append(y)
    torch.testing.assert_close(torch.cat(outs, 1), full, atol=1e-10, rtol=0)


def test_attention_layer_right_padding_is_neutral():
    p, pre, cfg = _layer_params(seed=4)
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(2, 40, cfg["hidden_size"], dtype=D64, generator=gen)
    mask = torch.ones(2, 40, dtype=torch.long)
    mask[1, 25:] = 0
    y, cache = MO.attention_layer(p, pre, x, cfg, use_cache=True, attention_mask=mask)
    y1, cache1 = MO.attention_layer(p, pre, x[1:, :25], cfg, use_cache=True)
    torch.testing.assert_close(y[1:, :25], y1, atol=1e-10, rtol=0)
    for a, b in zip(cache["recurrent_state"], cache1["recurrent_state"]):
        torch.testing.assert_close(a[1:], b, atol=1e-10, rtol=0)
    for a, b in zip(cache["conv_state"], cache1["conv_state"]):
        torch.testing.assert_close(a[1:], b, atol=0, rtol=0)


def test_causal_lm_prefix_then_decode_equals_full_forward():
    p, pre, cfg = _layer_params(seed=6)
    gen = torch.Generator().manual_seed(7)
    V, hidden = 50, cfg["hidden_size"]
    lm = {"model.layers.0." + k: v for k, v in p.items()}
    lm["model.embeddings.weight"] = torch.randn(V, hidden, dtype=D64, generator=gen)
    lm["model.layers.0.attn_norm.weight"] = 1 + 0.1 * torch.randn(hidden, dtype=D64, generator=gen)
    lm["model.layers.0.mlp_norm.weight"] = 1 + 0.1 * torch.randn(hidden, dtype=D64, generator=gen)
    for name, shape in (("gate_proj", (96, hidden)), ("up_proj", (96, hidden)), ("down_proj", (hidden, 96))):
        lm[f"model.layers.0.mlp.{name}.weight"] = 0.1 * torch.randn(*shape, dtype=D64, generator=gen)
    lm["model.norm.weight"] = torch.ones(hidden, dtype=D64)
    lm["lm_head.weight"] = 0.1 * torch.randn(V, hidden, dtype=D64, generator=gen)
    cfg = dict(cfg, num_hidden_layers=1, vocab_size=V, intermediate_size=96)
    ids = torch.randint(0, V, (1, 68), generator=gen)
    full, _ = MO.causal_lm(lm, cfg, ids)
    logits, cache = MO.causal_lm(lm, cfg, ids[:, :64], use_cache=True)
    outs = [logits]
    for t in range(64, 68):
        logits, cache = MO.causal_lm(lm, cfg, ids[:, t:t + 1], cache=cache, use_cache=True)
        outs.append(logits)
    torch.testing.assert_close(torch.cat(outs, 1), full, atol=1e-10, rtol=0)
    # the last-position form: the final norm and lm_head act per row
    seen = []
    last, _ = MO.causal_lm(lm, cfg, ids, last_logits_only=True, progress=seen.append)
    assert last.shape == (1, 1, V) and seen == [0]
    torch.testing.assert_close(last, full[:, -1:], atol=1e-12, rtol=0)  # one row: another BLAS blocking


def test_gated_mlp_against_a_scalar_loop_and_its_special_cases():
    """GatedMLP (models/cyfa/modeling_cyfa.py:13-27) in exact mode against a
    brute-force float64 loop over scalars with math.exp, on a tiny input, and
    the cases the formula fixes: zero up projection gives zero, a gate of zero
    gives zero (silu(0) = 0), and swapping the gate and up weights changes the
    result (silu is not symmetric)."""
    import math

    gen = torch.Generator().manual_seed(11)
    d, f, rows = 5, 7, 3
    p = {
        "m.gate_proj.weight": torch.randn(f, d, generator=gen, dtype=torch.float64),
        "m.up_proj.weight": torch.randn(f, d, generator=gen, dtype=torch.float64),
        "m.down_proj.weight": torch.randn(d, f, generator=gen, dtype=torch.float64),
    }
    x = torch.randn(rows, d, generator=gen, dtype=torch.float64)
    got = MO.gated_mlp(p, "m.", x, mode="exact").double()
    wg, wu, wd = (p[f"m.{n}_proj.weight"].tolist() for n in ("gate", "up", "down"))
    for r in range(rows):
        xr = x[r].tolist()
        h = []
        for j in range(f):
            g = sum(wg[j][c] * xr[c] for c in range(d))
            u = sum(wu[j][c] * xr[c] for c in range(d))
            h.append(g / (1.0 + math.exp(-g)) * u)
        for o in range(d):
            want = sum(wd[o][j] * h[j] for j in range(f))
            assert abs(got[r, o].item() - want) <= 1e-12 * (1 + abs(want))
    zero_up = dict(p, **{"m.up_proj.weight": torch.zeros(f, d, dtype=torch.float64)})
    assert torch.equal(MO.gated_mlp(zero_up, "m.", x, mode="exact").double(), torch.zeros(rows, d, dtype=torch.float64))
    zero_gate = dict(p, **{"m.gate_proj.weight": torch.zeros(f, d, dtype=torch.float64)})
    assert MO.gated_mlp(zero_gate, "m.", x, mode="exact").abs().max().item() == 0.0
    swapped = dict(p, **{"m.gate_proj.weight": p["m.up_proj.weight"], "m.up_proj.weight": p["m.gate_proj.weight"]})
    assert (MO.gated_mlp(swapped, "m.", x, mode="exact").double() - got).abs().max().item() > 1e-3


def test_gate_activations_special_cases():
    """g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), delta =
    sigmoid(d) (layers/cyfa.py:323-326), pinned by scalar closed forms:
    a = 0 gives -exp(A_log) log(1 + exp(dt_bias)); a -> -inf gives g -> 0-
    (no decay); a large gives -exp(A_log) (a + dt_bias); beta and delta are
    the logistic function of their own projection only."""
    A_log = torch.tensor([0.0, math.log(3.0), -1.5], dtype=D64)
    dt_bias = torch.tensor([0.0, -2.0, 1.25], dtype=D64)
    zero = torch.zeros(1, 3, dtype=D64)
    g, beta, delta = MO.gate_activations(zero, zero, zero, dt_bias, A_log)
    for h in range(3):
        want = -math.exp(float(A_log[h])) * math.log1p(math.exp(float(dt_bias[h])))
        assert abs(float(g[0, h]) - want) < 1e-15
    assert abs(float(g[0, 0]) + math.log(2.0)) < 1e-15  # A_log = dt_bias = 0: -log 2
    torch.testing.assert_close(beta, torch.full_like(beta, 0.5), rtol=0, atol=0)
    big = torch.full((1, 3), 60.0, dtype=D64)
    g_hi, _, _ = MO.gate_activations(big, zero, zero, dt_bias, A_log)
    g_lo, _, _ = MO.gate_activations(-big, zero, zero, dt_bias, A_log)
    for h in range(3):
        assert abs(float(g_hi[0, h]) + math.exp(float(A_log[h])) * (60.0 + float(dt_bias[h]))) < 1e-9
        assert -1e-20 < float(g_lo[0, h]) < 0.0
    b = torch.tensor([[-3.0, 0.7, 9.0]], dtype=D64)
    d = torch.tensor([[2.0, -0.4, -7.5]], dtype=D64)
    _, beta, delta = MO.gate_activations(zero, b, d, dt_bias, A_log)
    for h in range(3):
        assert abs(float(beta[0, h]) - 1 / (1 + math.exp(-float(b[0, h])))) < 1e-15
        assert abs(float(delta[0, h]) - 1 / (1 + math.exp(-float(d[0, h])))) < 1e-15


def test_layer_gates_wire_each_projection_to_its_gate():
    """With zero a/b/d projection weights the layer's gates are constants of
    the biases alone: g from dt_bias and A_log, beta = sigmoid(b_proj.bias),
    delta = sigmoid(d_proj.bias), with distinct biases so that a swapped
    projection or a missing bias fails. A nonzero a_proj then moves g only."""
    p, pre, cfg = _layer_params(H=2)
    H, hidden = 2, cfg["hidden_size"]
    for n in ("a_proj", "b_proj", "d_proj"):
        p[pre + n + ".weight"] = torch.zeros(H, hidden, dtype=D64)
    p[pre + "b_proj.bias"] = torch.tensor([0.3, -1.1], dtype=D64)
    p[pre + "d_proj.bias"] = torch.tensor([-2.2, 0.9], dtype=D64)
    p[pre + "dt_bias"] = torch.tensor([-0.5, 0.75], dtype=D64)
    p[pre + "A_log"] = torch.tensor([0.2, -0.3], dtype=D64)
    x = torch.randn(2, 5, hidden, dtype=D64, generator=torch.Generator().manual_seed(11))
    g, delta, beta = MO.layer_gates(p, pre, x)
    assert g.shape == delta.shape == beta.shape == (2, 5, H)
    for h in range(H):
        want_g = -math.exp(float(p[pre + "A_log"][h])) * math.log1p(math.exp(float(p[pre + "dt_bias"][h])))
        want_b = 1 / (1 + math.exp(-float(p[pre + "b_proj.bias"][h])))
        want_d = 1 / (1 + math.exp(-float(p[pre + "d_proj.bias"][h])))
        assert (g[..., h] - want_g).abs().max() < 1e-15
        assert (beta[..., h] - want_b).abs().max() < 1e-15
        assert (delta[..., h] - want_d).abs().max() < 1e-15
    p[pre + "a_proj.weight"] = torch.randn(H, hidden, dtype=D64, generator=torch.Generator().manual_seed(12))
    g2, delta2, beta2 = MO.layer_gates(p, pre, x)
    assert (g2 - g).abs().max() > 1e-3
    assert torch.equal(delta2, delta) and torch.equal(beta2, beta)
    a = x @ p[pre + "a_proj.weight"].T
    for (bi, t, h) in ((0, 0, 0), (1, 4, 1), (0, 2, 1)):
        z = float(a[bi, t, h]) + float(p[pre + "dt_bias"][h])
        want = -math.exp(float(p[pre + "A_log"][h])) * math.log1p(math.exp(z))
        assert abs(float(g2[bi, t, h]) - want) < 1e-12


def test_attention_layer_output_norm_is_per_head_and_scale_free():
    """The layer normalises o per head before o_proj (layers/cyfa.py:349-350):
    o is linear in v, so scaling one head's v projection leaves the layer's
    output unchanged up to the norm's eps, while the other head's output is
    not rescaled with it (a norm over all heads at once would move both)."""
    p, pre, cfg = _layer_params(hidden=64, H=2, Dh=32, seed=6)
    cfg["norm_eps"] = 1e-15  # (127 o)^2 is about 1e-4 at this scale: eps must not matter
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(1, 50, cfg["hidden_size"], dtype=D64, generator=gen)
    y, _ = MO.attention_layer(p, pre, x, cfg)
    scaled = dict(p)
    w = p[pre + "v_proj.weight"].clone()
    w[:32] *= 10.0  # head 0's value channels
    scaled[pre + "v_proj.weight"] = w
    y10, _ = MO.attention_layer(scaled, pre, x, cfg)
    torch.testing.assert_close(y10, y, atol=1e-9, rtol=1e-7)
    unnormed = dict(p, **{pre + "o_norm.weight": 2 * p[pre + "o_norm.weight"]})
    y2, _ = MO.attention_layer(unnormed, pre, x, cfg)
    torch.testing.assert_close(y2, 2 * y, atol=1e-12, rtol=1e-12)  # the norm weight multiplies, after the norm


def test_attention_layer_gate_is_sigmoid_of_g_proj():
    """The output gate is sigmoid(g_proj(x)) multiplying the normalised o
    before o_proj (layers/cyfa.py:292-295, 349-351): with a zero last g_proj
    weight the gate is sigmoid(bias), and a bias that is one value c across
    channels scales the whole output by sigmoid(c)."""
    p, pre, cfg = _layer_params(seed=8)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(1, 30, cfg["hidden_size"], dtype=D64, generator=gen)
    outs = []
    for c in (0.0, 1.5):
        q = dict(p, **{pre + "g_proj.1.weight": torch.zeros_like(p[pre + "g_proj.1.weight"]),
                       pre + "g_proj.1.bias": torch.full_like(p[pre + "g_proj.1.bias"], c)})
        outs.append(MO.attention_layer(q, pre, x, cfg)[0])
    ratio = (1 / (1 + math.exp(-1.5))) / 0.5
    torch.testing.assert_close(outs[1], ratio * outs[0], atol=1e-12, rtol=1e-12)


def test_clock_branch_sends_no_gradient_into_x():
    """delta = sigmoid(d_proj(x.detach())) (layers/cyfa.py:325): the clock
    branch trains d_proj but passes no gradient into x. With every other path
    from x to the output cut (zero q/k/v, a, b and g_proj[0] weights; q, k, v
    made constant by conv biases, beta and the gate by their biases) the
    output still depends on x through delta -- a perturbation of x moves it --
    yet x.grad is exactly zero while d_proj.weight.grad is not. Without the
    detach x.grad would be the perturbation's slope."""
    p, pre, cfg = _layer_params(hidden=48, H=2, Dh=32, seed=13)
    H, Dh, hidden = 2, 32, 48
    gen = torch.Generator().manual_seed(14)
    for n in ("q_proj", "k_proj", "v_proj"):
        p[pre + n + ".weight"] = torch.zeros(H * Dh, hidden, dtype=D64)
        p[pre + n.replace("_proj", "_conv1d") + ".bias"] = torch.randn(H * Dh, dtype=D64, generator=gen)
    for n in ("a_proj", "b_proj"):
        p[pre + n + ".weight"] = torch.zeros(H, hidden, dtype=D64)
    p[pre + "g_proj.0.weight"] = torch.zeros(Dh, hidden, dtype=D64)
    p[pre + "d_proj.weight"] = (0.5 * torch.randn(H, hidden, dtype=D64, generator=gen)).requires_grad_(True)
    x = torch.randn(1, 40, hidden, dtype=D64, generator=gen).requires_grad_(True)
    y, _ = MO.attention_layer(p, pre, x, cfg)
    y.pow(2).sum().backward()
    assert x.grad is None or torch.count_nonzero(x.grad) == 0
    assert p[pre + "d_proj.weight"].grad.abs().max() > 1e-6
    with torch.no_grad():
        y2, _ = MO.attention_layer(p, pre, x + 0.05 * torch.randn(x.shape, dtype=D64, generator=gen), cfg)
    assert (y2 - y.detach()).abs().max() > 1e-6
