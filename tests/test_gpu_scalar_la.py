"""Isolated ScalarGatedLA pass (ops.chunk.scalar_la, cyfa_scalar_la) against the
oracle's chunkwise pass (oracle.cyfa_oracle.sgla_chunk, float64, no
intermediate rounding) at the two pass shapes; configuration 2 of the
benchmark (B=8, H=4, T=4096) at full size. Tolerances: max-abs 2e-2 and
mean-rel 5e-3 (tests/tolerance.py)."""

import pytest
import torch

from oracle import cyfa_oracle as O
from tolerance import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, H, T, K, V, seed, state):
    """Configuration-2 inputs: q, k, v ~ N(0, 1) bf16 with q and k
    L2-normalised per head; log alpha = logsigmoid(N(3, 1))."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, H, T, K, generator=gen), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, H, T, K, generator=gen), dim=-1)
    v = torch.randn(B, H, T, V, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen) + 3)
    h0 = 0.3 * torch.randn(B, H, K, V, generator=gen) if state else None
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), g, h0


def _run(q, k, v, g, h0, scale, raw, output_bth=False, v_bth=False):
    from cyclic_flow_attention.ops.chunk import scalar_la

    vin = v.transpose(1, 2).contiguous() if v_bth else v
    with torch.no_grad():
        o, final = scalar_la(q.to(DEV), k.to(DEV), vin.to(DEV), g.to(DEV), None if h0 is None else h0.to(DEV), scale,
                             raw, output_bth, v_bth)
    torch.cuda.synchronize()
    if output_bth:
        o = o.transpose(1, 2)
    return o, final


def _oracle(q, k, v, g, h0, scale):
    B, H, T, K = q.shape
    V = v.shape[-1]
    S0 = torch.zeros(B, H, K, V, dtype=torch.float64) if h0 is None else h0.double()
    return O.sgla_chunk(q.double(), k.double(), v.double(), g.double(), S0, scale, mode="exact")


CASES = [
    # B, H, T, K, V, initial state, raw output, output_bth, v_bth, forced chunks per segment
    (1, 1, 64, 256, 128, False, True, False, False, None),
    (2, 2, 512, 256, 128, True, True, False, False, "3"),
    (2, 2, 512, 256, 128, True, False, True, True, "2"),
    (1, 1, 64, 128, 256, False, False, False, False, None),
    (2, 2, 512, 128, 256, True, False, False, False, "3"),
    (2, 2, 512, 128, 256, True, True, True, True, "1"),
]


@pytest.mark.parametrize("B,H,T,K,V,state,raw,obth,vbth,seg", CASES)
def test_scalar_la_matches_oracle(B, H, T, K, V, state, raw, obth, vbth, seg, monkeypatch):
    if seg is not None:
        monkeypatch.setenv("CYFA_SEGMENT_CHUNKS", seg)
    q, k, v, g, h0 = _inputs(B, H, T, K, V, seed=T + K, state=state)
    scale = K ** -0.5 if K == 256 else 1.0
    o, final = _run(q, k, v, g, h0, scale, raw, obth, vbth)
    assert o.dtype == (torch.float32 if raw else torch.bfloat16) and o.shape == (B, H, T, V)
    ro, rfinal = _oracle(q, k, v, g, h0, scale)
    assert_close(o, ro, what=f"scalar_la o K{K} B{B} T{T}")
    assert_close(final, rfinal, what=f"scalar_la final K{K} B{B} T{T}")


@pytest.mark.parametrize("K,V", [(256, 128), (128, 256)])
def test_scalar_la_config2(K, V):
    """Configuration 2 at full size: B=8, H=4, T=4096, zero initial state."""
    q, k, v, g, _ = _inputs(8, 4, 4096, K, V, seed=2, state=False)
    scale = K ** -0.5 if K == 256 else 1.0
    o, final = _run(q, k, v, g, None, scale, raw=K == 256)
    ro, rfinal = _oracle(q, k, v, g, None, scale)
    assert_close(o, ro, what=f"scalar_la config 2 o K{K}")
    assert_close(final, rfinal, what=f"scalar_la config 2 final K{K}")


def test_scalar_la_chunk_equals_token_recurrence():
    """The chunkwise pass and the token-by-token recurrence of the same pass
    (oracle.sgla_recurrent) agree."""
    q, k, v, g, h0 = _inputs(1, 2, 192, 128, 256, seed=7, state=True)
    o, final = _run(q, k, v, g, h0, 1.0, raw=False)
    ro, rfinal = O.sgla_recurrent(q.double(), k.double(), v.double(), g.double(), h0.double(), 1.0)
    assert_close(o, ro, what="scalar_la vs recurrence o")
    assert_close(final, rfinal, what="scalar_la vs recurrence final")
