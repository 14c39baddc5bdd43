"""GPU parity of the general-shape path (cyfa_chunk_fwd_general,
cyfa_decode_step_general, the general readout table) against the CPU oracle
in exact float64 mode.

Shapes outside the tuned kernels (K = V = 256, 128 slots, chunk 64 in
prefill; K, V in {128, 256}, 128 slots in decode) take this path, as the
reference's unfused fallback takes them (ops/chunk.py:285-331). Tolerance:
bf16 operands are rounded where the reference casts to the input dtype, so
they meet the north-star bar (max-abs 2e-2, mean-rel 5e-3); fp32 operands
are computed in fp32 without rounding and must agree to max-abs 1e-3 and
mean-rel 1e-4 (fp16 operands likewise, with o, returned in fp16, to
mean-rel 5e-4).
"""

import pytest
import torch

from oracle import cyfa_oracle as O
from tolerance import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"
F32_BAR = dict(max_abs=1e-3, mean_rel=1e-4)
# fp16 operands run in fp32 too; only o is returned in fp16, whose rounding
# (2^-11 relative) alone gives about 1.5e-4 mean-rel
F16_OUT_BAR = dict(max_abs=1e-3, mean_rel=5e-4)


def _inputs(B, T, H, K, V, M, seed, dtype, state):
    gen = torch.Generator().manual_seed(seed)
    R = M - 1
    x = dict(
        q=torch.randn(B, T, H, K, generator=gen),
        k=torch.randn(B, T, H, K, generator=gen),
        v=torch.randn(B, T, H, V, generator=gen),
        g=torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 3),
        delta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        readout=torch.eye(R).expand(H, R, R) + 0.05 * torch.randn(H, R, R, generator=gen),
        q_norm_weight=1 + 0.1 * torch.randn(K, generator=gen),
        k_norm_weight=1 + 0.1 * torch.randn(K, generator=gen),
    )
    for name in ("q", "k", "v"):
        x[name] = x[name].to(dtype)
    init = None
    if state:
        init = (0.3 * torch.randn(B, H, K, M, generator=gen), 0.3 * torch.randn(B, H, M, V, generator=gen),
                50.0 * torch.rand(B, H, generator=gen))
    return x, init


def _oracle_args(x, init):
    xd = {k: v.double() for k, v in x.items()}
    return xd, (None if init is None else tuple(t.double() for t in init))


def _bar(dtype):
    return {} if dtype == torch.bfloat16 else F32_BAR


CHUNK_CASES = [
    # B, T, H, K, V, M, C, dtype, state
    (2, 100, 2, 128, 64, 64, 32, torch.bfloat16, True),
    (1, 130, 2, 384, 128, 128, 64, torch.float32, True),
    (2, 70, 1, 64, 256, 32, 16, torch.bfloat16, False),
    (1, 200, 2, 256, 256, 96, 64, torch.float32, False),
    (1, 64, 3, 256, 128, 128, 64, torch.bfloat16, True),  # V = 128: outside the tuned kernels
    (1, 10, 2, 96, 80, 16, 64, torch.float32, True),      # T shorter than one chunk
    (1, 96, 1, 128, 128, 64, 32, torch.float16, True),    # fp16 operands run in fp32
    (1, 70, 1, 1024, 1024, 256, 32, torch.bfloat16, True),  # the largest head dims and slot count
    (1, 40, 2, 1, 1, 4, 16, torch.float32, True),          # the smallest
    (2, 1, 2, 64, 64, 16, 64, torch.bfloat16, True),       # a one-token sequence
]


@pytest.mark.parametrize("B,T,H,K,V,M,C,dtype,state", CHUNK_CASES)
def test_general_chunk_matches_oracle(B, T, H, K, V, M, C, dtype, state):
    from cyclic_flow_attention.ops import chunk_cyfa

    x, init = _inputs(B, T, H, K, V, M, seed=B * 1000 + T + K + M, dtype=dtype, state=state)
    xg = {k: v.to(DEV) for k, v in x.items()}
    ig = None if init is None else tuple(t.to(DEV) for t in init)
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True, chunk_size=C)
    torch.cuda.synchronize()
    assert o.dtype == dtype and tuple(o.shape) == (B, T, H, V)
    xd, idd = _oracle_args(x, init)
    o_ref, st_ref = O.chunk_cyfa(**xd, initial_state=idd, output_final_state=True, chunk_size=C, mode="exact")
    what = f"general chunk B{B} T{T} H{H} K{K} V{V} M{M} C{C} {dtype}"
    assert_close(o, o_ref, what=f"{what} o", **(F16_OUT_BAR if dtype == torch.float16 else _bar(dtype)))
    assert_close(st[0], st_ref[0], what=f"{what} hk", **_bar(dtype))
    assert_close(st[1], st_ref[1], what=f"{what} hv", **_bar(dtype))
    torch.testing.assert_close(st[2].double().cpu(), st_ref[2], atol=5e-3, rtol=1e-6, msg=f"{what} clock")


DECODE_CASES = [
    # B, H, K, V, M, dtype, state
    (2, 2, 64, 96, 64, torch.bfloat16, True),
    (1, 3, 512, 384, 128, torch.float32, True),
    (2, 1, 1024, 1024, 256, torch.bfloat16, True),
    (3, 2, 128, 128, 32, torch.float32, False),
    # fp32 at the tuned kernel's shapes (K, V in {128, 256}, 128 slots): that
    # kernel without its bf16 rounding points
    (3, 2, 128, 256, 128, torch.float32, True),
    (1, 4, 256, 128, 128, torch.float32, False),
    (64, 4, 256, 256, 128, torch.float32, True),
]


@pytest.mark.parametrize("B,H,K,V,M,dtype,state", DECODE_CASES)
def test_general_decode_matches_oracle(B, H, K, V, M, dtype, state):
    from cyclic_flow_attention.ops import fused_recurrent_cyfa

    x, init = _inputs(B, 1, H, K, V, M, seed=7 + B + K + M, dtype=dtype, state=state)
    xg = {k: v.to(DEV) for k, v in x.items()}
    ig = None if init is None else tuple(t.to(DEV) for t in init)
    with torch.no_grad():
        o, st = fused_recurrent_cyfa(**xg, initial_state=ig, output_final_state=True)
    torch.cuda.synchronize()
    assert o.dtype == dtype and tuple(o.shape) == (B, 1, H, V)
    xd, idd = _oracle_args(x, init)
    o_ref, st_ref = O.fused_recurrent_cyfa(**xd, initial_state=idd, output_final_state=True, mode="exact")
    what = f"general decode B{B} H{H} K{K} V{V} M{M} {dtype}"
    assert_close(o, o_ref, what=f"{what} o", **_bar(dtype))
    assert_close(st[0], st_ref[0], what=f"{what} hk", **_bar(dtype))
    assert_close(st[1], st_ref[1], what=f"{what} hv", **_bar(dtype))
    torch.testing.assert_close(st[2].double().cpu(), st_ref[2], atol=1e-4, rtol=1e-6, msg=f"{what} clock")


@pytest.mark.parametrize("M", [16, 64, 96, 256])
def test_general_readout_table_matches_oracle(M):
    from cyclic_flow_attention.ops.utils import readout_table

    gen = torch.Generator().manual_seed(M)
    R = M - 1
    ro = torch.eye(R).expand(2, R, R) + 0.1 * torch.randn(2, R, R, generator=gen)
    got = readout_table(ro.to(DEV)).cpu().double()
    torch.testing.assert_close(got, O.readout_table(ro.double()), atol=2e-5, rtol=0)


def test_general_prefix_then_decode_continues_the_chunk():
    """A general-shape prefix through chunk_cyfa, then one decode step from
    its final states, equals the last token of chunk_cyfa over the whole
    sequence (the consistency tests/test_inference.py:20-34 checks at the
    model level), in fp32."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    B, T, H, K, V, M = 1, 65, 2, 128, 96, 64
    x, _ = _inputs(B, T, H, K, V, M, seed=5, dtype=torch.float32, state=False)
    xg = {k: v.to(DEV) for k, v in x.items()}
    seq = ("q", "k", "v", "g", "delta", "beta")
    with torch.no_grad():
        full, _ = chunk_cyfa(**xg, chunk_size=32)
        pre = {k: (v[:, :T - 1] if k in seq else v) for k, v in xg.items()}
        _, st = chunk_cyfa(**pre, output_final_state=True, chunk_size=32)
        step = {k: (v[:, T - 1:] if k in seq else v) for k, v in xg.items()}
        last, _ = fused_recurrent_cyfa(**step, initial_state=st)
    torch.cuda.synchronize()
    assert_close(last[:, 0], full[:, T - 1], what="general prefix + decode vs full", **F32_BAR)
