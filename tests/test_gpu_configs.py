"""GPU parity at the configurations the headline numbers are quoted on.

Configuration 3: CyFA-400M (24 layers) prefill of B=8 x T=2048 uniform random
ids. Configuration 4: the same model, B=64, a 2048-token prompt, then greedy
graphed decode steps. Plus the model-level form of the reference's only
consistency test (tests/test_inference.py:20-34: a 64-token chunk prefix and
one decode step against the full 65-token forward, rrms < 0.02).

References (oracle.model_oracle, the same seeded weights):
  O_me  mode="mirror", op_mode="exact": the reference's bf16 layer plumbing
        around a float64 CyFA op (the fp32-or-better reference);
  O_mm  mode="mirror", op_mode="mirror": the reference's own bf16 arithmetic
        for the op as well.

Tolerances. The first layer's states must meet the north-star bar (max-abs
2e-2, mean-rel 5e-3) against O_me. Deeper in a 24-layer random-init model,
bf16 rounding anywhere moves the clock lam = sum(delta) by up to ~0.3 after 24
layers, which rotates the high Fourier pairs of the states by up to a radian:
the reference's own arithmetic (O_mm) then differs from O_me by ~13% mean-rel
on the last layer's states and ~2% on the logits. So the last layer's states
and the logits are required to stay within 1.5x of that spread (the
reference's own rounding budget at the same point), and greedy tokens are
checked by teacher forcing with the steps where O_mm and O_me themselves pick
different tokens, or O_me's top-2 gap is below two bf16 roundings of its
largest logit, counted as undecidable (their count is bounded).
"""

import pytest
import torch

from oracle import cyfa_oracle as O
from oracle import model_oracle as MO
from tolerance import assert_close, metrics

pytestmark = pytest.mark.gpu

DEV = "cuda"
T_PROMPT = 2048
BF16_ULP = 2.0 ** -8
BUDGET_FACTOR = 1.5  # GPU deviation from O_me allowed, relative to O_mm's
# configuration 4's greedy check: 17 of its 130 steps are undecidable on
# MI355X (none mismatched); the bound adds a slack of 7
CFG4_MAX_UNDECIDABLE = 24


def _budget_close(got, ref, spread_ref, what):
    """got within BUDGET_FACTOR of the reference arithmetic's own spread
    (spread_ref vs ref), or within the north-star bar if that is wider."""
    m = metrics(got, ref)
    s = metrics(spread_ref, ref)
    print(f"{what}: gpu {m} / reference rounding {s}")
    assert m["mean_rel"] <= max(5e-3, BUDGET_FACTOR * s["mean_rel"]), f"{what}: {m} vs budget {s}"
    assert m["rrms"] <= max(5e-3, BUDGET_FACTOR * s["rrms"]), f"{what}: {m} vs budget {s}"
    return m


@pytest.fixture(scope="module")
def model400():
    from cyclic_flow_attention.utils import initialize_model, read_config

    config = read_config("cyclic_flow_attention_400m.json")
    model = initialize_model(config, std=0.02, seed=0).to(DEV).eval()
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    cfg = {k: getattr(config, k) for k in config.__dataclass_fields__}
    return model, params, cfg


@pytest.fixture(scope="module")
def prompts(model400):
    """Two 2048-token prompts (rows checked against the oracle) and the oracle's
    prefill of them in both modes."""
    _, params, cfg = model400
    gen = torch.Generator().manual_seed(303)
    ids = torch.randint(0, cfg["vocab_size"], (2, T_PROMPT), generator=gen)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    me = MO.causal_lm(params, cfg, ids, use_cache=True, mode="mirror", op_mode="exact")
    mm = MO.causal_lm(params, cfg, ids, use_cache=True, mode="mirror", op_mode="mirror")
    return ids, me, mm


@pytest.mark.timeout(600)
def test_config3_model_prefill_matches_oracle(model400, prompts):
    """Configuration 3: the 24-layer prefill of B=8 x T=2048 on the GPU; rows 0
    and 7 (the oracle's two prompts) compared with O_me: logits of every
    position, and the first and last layers' final states and clocks."""
    model, _, cfg = model400
    ids2, (lg_me, c_me), (lg_mm, c_mm) = prompts
    gen = torch.Generator().manual_seed(304)
    ids = torch.randint(0, cfg["vocab_size"], (8, T_PROMPT), generator=gen)
    ids[0], ids[7] = ids2[0], ids2[1]
    with torch.no_grad():
        out = model(ids.to(DEV), use_cache=True)
    torch.cuda.synchronize()
    logits = out["logits"][[0, 7]].float().cpu()
    assert out["logits"].shape == (8, T_PROMPT, cfg["vocab_size"]) and out["logits"].dtype == torch.bfloat16
    assert torch.isfinite(logits).all()
    _budget_close(logits, lg_me, lg_mm, "cfg3 logits")
    first = out["cache"][0]["recurrent_state"]
    for i, n in enumerate(("hk", "hv")):
        assert_close(first[i][[0, 7]], c_me[0]["recurrent_state"][i], what=f"cfg3 layer 0 {n}")
    torch.testing.assert_close(first[2][[0, 7]].double().cpu(), c_me[0]["recurrent_state"][2].double(),
                               atol=2e-2, rtol=0, msg="cfg3 layer 0 clock")
    last = out["cache"][-1]["recurrent_state"]
    for i, n in enumerate(("hk", "hv", "clock")):
        _budget_close(last[i][[0, 7]].float().cpu(), c_me[-1]["recurrent_state"][i],
                      c_mm[-1]["recurrent_state"][i], f"cfg3 layer 23 {n}")


@pytest.mark.timeout(600)
def test_config4_graphed_decode_and_greedy_tokens(model400, prompts):
    """Configuration 4: B=64 after a 2048-token chunkwise prompt. Replays of the
    graphed 24-layer step equal eager steps bit for bit for 8 steps; then 64
    greedy graphed steps, with rows 0 and 63 (the oracle's prompts) checked by
    teacher forcing against O_me: every decidable step picks O_me's token,
    the undecidable ones are counted and bounded (17 of 130 observed), and at
    every step the GPU's own logits prefer its token over O_me's by at most
    twice the reference's own rounding noise on that difference."""
    model, params, cfg = model400
    ids2, (lg_me, c_me), (lg_mm, c_mm) = prompts
    B, steps = 64, 64
    gen = torch.Generator().manual_seed(305)
    ids = torch.randint(0, cfg["vocab_size"], (B, T_PROMPT), generator=gen)
    ids[0], ids[B - 1] = ids2[0], ids2[1]
    with torch.no_grad():
        hidden, cache = model.model(ids.to(DEV), use_cache=True)
        first = model.lm_head(hidden[:, -1:])
        tok = first.argmax(-1)
        del hidden
        dec = model.graphed_decoder(cache, tok)
        tokens = [tok[[0, B - 1], 0].cpu()]
        gpu_logits = [first[[0, B - 1], -1].float().cpu()]
        eager_tok = tok
        for step in range(8):
            eager = model(eager_tok, cache=cache, use_cache=True)
            cache = eager["cache"]
            eager_tok = eager["logits"][:, -1:].argmax(-1)
            got = dec.step()
            assert torch.equal(dec.logits, eager["logits"]), f"step {step}: graphed logits differ from eager"
            assert torch.equal(got, eager_tok), f"step {step}: graphed tokens differ from eager"
            tokens.append(got[[0, B - 1], 0].cpu())
            gpu_logits.append(dec.logits[[0, B - 1], -1].float().cpu())
        del cache, eager
        for _ in range(steps - 8):
            tokens.append(dec.step()[[0, B - 1], 0].cpu())
            gpu_logits.append(dec.logits[[0, B - 1], -1].float().cpu())
    torch.cuda.synchronize()
    toks = torch.stack(tokens, 1)  # [2, steps + 1]: the prefill's token, then one per step
    me_last, mm_last = lg_me[:, -1], lg_mm[:, -1]
    cache_me = c_me
    cache_mm = c_mm
    undecidable = mismatched = 0
    for i in range(steps + 1):
        for r in range(2):
            top2 = me_last[r].topk(2)
            gap = float(top2.values[0] - top2.values[1])
            decidable = (int(mm_last[r].argmax()) == int(top2.indices[0])
                         and gap > 2 * BF16_ULP * float(me_last[r].abs().max()))
            # at every step the GPU prefers its token over O_me's by no more than
            # twice the reference's own rounding noise on a logit difference
            noise = 2 * 2 ** 0.5 * float((mm_last[r] - me_last[r]).pow(2).mean().sqrt())
            pref = float(gpu_logits[i][r][int(toks[r, i])] - gpu_logits[i][r][top2.indices[0]])
            assert pref <= noise, f"step {i} row {r}: the GPU prefers token {int(toks[r, i])} by {pref:.4f}"
            if not decidable:
                undecidable += 1
            elif int(toks[r, i]) != int(top2.indices[0]):
                mismatched += 1
                d = mm_last[r] - me_last[r]
                print(f"step {i} row {r}: token {int(toks[r, i])} vs {int(top2.indices[0])}; gap {gap:.4g}, "
                      f"reference rounding moves the gap by {float(d[top2.indices[0]] - d[top2.indices[1]]):.4g}")
        if i == steps:
            break
        feed = toks[:, i:i + 1]
        lg, cache_me = MO.causal_lm(params, cfg, feed, cache=cache_me, use_cache=True, mode="mirror", op_mode="exact")
        lgm, cache_mm = MO.causal_lm(params, cfg, feed, cache=cache_mm, use_cache=True, mode="mirror",
                                     op_mode="mirror")
        me_last, mm_last = lg[:, -1], lgm[:, -1]
    total = 2 * (steps + 1)
    print(f"cfg4 greedy tokens: {total - undecidable - mismatched} of {total} decidable steps match, "
          f"{undecidable} undecidable, {mismatched} mismatched")
    assert mismatched == 0, f"{mismatched} decidable greedy steps differ from the oracle's token"
    assert undecidable <= CFG4_MAX_UNDECIDABLE, f"{undecidable} of {total} steps undecidable"


@pytest.mark.parametrize("name", ["tiny.json", "cyclic_flow_attention_400m.json"])
def test_model_prefix_then_decode_equals_full_forward(name):
    """The reference's consistency test at the model level
    (tests/test_inference.py:20-34): ids 32..96, a 64-token chunkwise prefix
    and one decode step give the last position's logits of the full 65-token
    forward within rrms 0.02, the reference's own bar. Both GPU results are
    also compared with the oracle's full forward (O_me): logits of a
    multi-layer model are within 1.5x of the spread of the reference's own
    bf16 arithmetic (O_mm) at the same point (about 6e-3 mean-rel for the
    tiny model, 2e-2 for the 24-layer model)."""
    from cyclic_flow_attention.utils import initialize_model, read_config

    config = read_config(name)
    model = initialize_model(config, std=0.02, seed=7).to(DEV).eval()
    ids = torch.arange(65)[None] + 32
    with torch.no_grad():
        reference = model(ids.to(DEV))["logits"].float().cpu()
        prefix = model(ids[:, :64].to(DEV), use_cache=True)
        decoded = model(ids[:, 64:].to(DEV), cache=prefix["cache"], use_cache=True)["logits"].float().cpu()
    m = metrics(decoded, reference[:, -1:])
    print(f"{name}: prefix + decode vs full {m}")
    assert m["rrms"] < 0.02, m
    params = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    cfg = {k: getattr(config, k) for k in config.__dataclass_fields__}
    me, _ = MO.causal_lm(params, cfg, ids, mode="mirror", op_mode="exact")
    mm, _ = MO.causal_lm(params, cfg, ids, mode="mirror", op_mode="mirror")
    for got, what in ((reference[:, -1:], "full"), (decoded, "prefix + decode")):
        _budget_close(got, me[:, -1:], mm[:, -1:], f"{name} {what} vs oracle")


@pytest.mark.parametrize("B,H", [(64, 4), (1, 8)])
def test_decode_layer_step_matches_oracle(B, H):
    """decode_layer_step at configuration 4's shape (B=64, H=4: 256
    workgroups) and configuration 5's (B=1, H=8: the 1.4B model's
    single-sequence step) against the oracle's layer arithmetic: short
    convolution and conv cache, gate activations, the exact decode op and the
    gated output norm."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops.fused_recurrent import decode_layer_step

    D = 3 * H * 256
    gen = torch.Generator().manual_seed(64 + B + H)
    qkv = torch.randn(B, 1, D, generator=gen).bfloat16()
    cache = (0.5 * torch.randn(B, 3, D, generator=gen)).bfloat16()
    wconv = (0.3 * torch.randn(D, 4, generator=gen)).bfloat16()
    abd = torch.randn(B, 1, 3 * H, generator=gen).bfloat16()
    dt_bias, A_log = torch.randn(H, generator=gen), torch.randn(H, generator=gen)
    gate = torch.randn(B, 1, H * 256, generator=gen).bfloat16()
    nw = 1 + 0.1 * torch.randn(256, generator=gen)
    qw, kw = 1 + 0.1 * torch.randn(256, generator=gen), 1 + 0.1 * torch.randn(256, generator=gen)
    readout = torch.eye(127).expand(H, 127, 127) + 0.05 * torch.randn(H, 127, 127, generator=gen)
    init = (0.3 * torch.randn(B, H, 256, 128, generator=gen), 0.3 * torch.randn(B, H, 128, 256, generator=gen),
            1e4 * torch.rand(B, H, generator=gen))
    dev = {n: t.to(DEV) for n, t in dict(qkv=qkv, cache=cache, wconv=wconv, abd=abd, dt_bias=dt_bias, A_log=A_log,
                                         gate=gate, nw=nw, qw=qw, kw=kw, readout=readout).items()}
    table = _native.readout_table(dev["readout"])
    tail = torch.empty(B, 3, D, dtype=torch.bfloat16, device=DEV)
    with torch.no_grad():
        got, st = decode_layer_step(dev["qkv"], dev["cache"], tail, dev["wconv"], dev["abd"], dev["dt_bias"],
                                    dev["A_log"], dev["gate"], dev["nw"], 1e-6, 127.0, table, dev["qw"], dev["kw"],
                                    1e-6, 1e-6, H, initial_state=tuple(t.to(DEV) for t in init),
                                    output_final_state=True)
    torch.cuda.synchronize()
    # oracle: mirror plumbing (bf16 conv outputs) around the exact op
    y, new_cache = MO.short_conv(qkv.float(), wconv.float()[:, None, :], cache=cache.float(), mode="mirror")
    q, k, v = (y[..., i * H * 256:(i + 1) * H * 256].reshape(B, 1, H, 256) for i in range(3))
    a = abd.float()
    g, beta, delta = MO.gate_activations(a[..., :H], a[..., H:2 * H], a[..., 2 * H:], dt_bias, A_log, mode="mirror")
    o, rst = O.fused_recurrent_cyfa(q.double(), k.double(), v.double(), g.double(), delta.double(), beta.double(),
                                    readout.double(), qw.double(), kw.double(),
                                    initial_state=tuple(t.double() for t in init), output_final_state=True)
    gate4 = gate.float().reshape(B, 1, H, 256)
    ref = MO.rms_norm((o.float() * 127).bfloat16().float(), nw, 1e-6, gate4, mode="exact")
    # the reference's own arithmetic: the op in mirror mode, then the same norm
    om, _ = O.fused_recurrent_cyfa(q.double(), k.double(), v.double(), g.double(), delta.double(), beta.double(),
                                   readout.double(), qw.double(), kw.double(),
                                   initial_state=tuple(t.double() for t in init), mode="mirror")
    own = metrics(MO.rms_norm((om.float() * 127).bfloat16().float(), nw, 1e-6, gate4, mode="exact"), ref)
    # o' is the normalised head output before o_proj (elements up to ~5, where a
    # bf16 ulp is 0.03): max-abs within the north-star bar or 1.5x the
    # reference's own rounding at this point, mean-rel within 5e-3
    assert_close(got.reshape(B, 1, H, 256), ref, max_abs=max(2e-2, 1.5 * own["max_abs"]),
                 what=f"B{B} H{H} layer step o'")
    for a_, b_, n in zip(st, rst, ("hk", "hv")):
        assert_close(a_, b_, what=f"B{B} H{H} layer step {n}")
    torch.testing.assert_close(st[2].double().cpu(), rst[2], atol=5e-3, rtol=1e-6)
    assert torch.equal(tail.cpu(), new_cache.bfloat16())
