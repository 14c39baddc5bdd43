"""The gradients the backward pass is checked against are float64 autograd
through the oracle's exact mode. This pins them: autograd agrees with
central finite differences of the oracle's forward (torch.autograd.gradcheck)
for every input of chunk_cyfa -- q, k, v, g, delta, beta, the readout, both
norm weights and the three initial states -- and every output (o and the
final states), on a ragged sequence with more than one chunk. The clock
phase's integer range reduction is continuous in lambda (a step across an
integer moves the angle by a multiple of 2 pi), so finite differences see
the same derivative 2 pi p / R as autograd.
"""

import torch

from oracle import cyfa_oracle as O


def _tiny(seed, M=8, K=4, V=3, T=6, H=1):
    gen = torch.Generator().manual_seed(seed)
    R = M - 1
    x = [
        torch.randn(1, T, H, K, generator=gen),                          # q
        torch.randn(1, T, H, K, generator=gen),                          # k
        torch.randn(1, T, H, V, generator=gen),                          # v
        torch.nn.functional.logsigmoid(torch.randn(1, T, H, generator=gen) + 1),  # g
        torch.sigmoid(torch.randn(1, T, H, generator=gen)),               # delta
        torch.sigmoid(torch.randn(1, T, H, generator=gen)),               # beta
        torch.eye(R).expand(H, R, R) + 0.3 * torch.randn(H, R, R, generator=gen),  # readout
        1 + 0.2 * torch.randn(K, generator=gen),                         # q_norm_weight
        1 + 0.2 * torch.randn(K, generator=gen),                         # k_norm_weight
        0.5 * torch.randn(1, H, K, M, generator=gen),                    # hk0
        0.5 * torch.randn(1, H, M, V, generator=gen),                    # hv0
        3.7 + torch.rand(1, H, generator=gen),                           # clock0
    ]
    return [t.double().requires_grad_(True) for t in x]


def _op(C):
    def f(q, k, v, g, delta, beta, readout, qw, kw, hk0, hv0, c0):
        o, (hk, hv, clock) = O.chunk_cyfa(q, k, v, g, delta, beta, readout, qw, kw, initial_state=(hk0, hv0, c0),
                                          output_final_state=True, chunk_size=C)
        return o, hk, hv, clock

    return f


def test_oracle_gradients_match_finite_differences():
    assert torch.autograd.gradcheck(_op(4), _tiny(0), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_oracle_gradients_match_finite_differences_one_chunk_and_heads():
    assert torch.autograd.gradcheck(_op(8), _tiny(1, M=6, K=3, V=2, T=5, H=2), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_gate_gradient_form():
    """The backward forms dg_t as the in-chunk reverse cumsum of
    q_t.dq_t - k_t.dk_t plus <D_{n+1}, S_{n+1}> at the chunk's last token,
    for o = SGLA(q, k, v, g) with D the cotangent of the state after the
    chunk. The same identity, restated from the oracle's own gradients
    (dq, dk, and dS of the final state), must equal autograd's dg."""
    gen = torch.Generator().manual_seed(3)
    B, H, T, K, V, C = 1, 1, 8, 3, 2, 8  # one chunk
    q, k = torch.randn(B, H, T, K, generator=gen).double(), torch.randn(B, H, T, K, generator=gen).double()
    v = torch.randn(B, H, T, V, generator=gen).double()
    g = torch.nn.functional.logsigmoid(torch.randn(B, H, T, generator=gen)).double()
    S0 = torch.randn(B, H, K, V, generator=gen).double()
    dO = torch.randn(B, H, T, V, generator=gen).double()
    dS = torch.randn(B, H, K, V, generator=gen).double()
    for t in (q, k, v, g, S0):
        t.requires_grad_(True)
    o, S = O.sgla_chunk(q, k, v, g, S0, 0.7, C)
    ((o * dO).sum() + (S * dS).sum()).backward()
    dG = (q * q.grad).sum(-1) - (k * k.grad).sum(-1)
    dG[..., -1] += (dS * S.detach()).sum((-1, -2))
    dg = dG.flip(-1).cumsum(-1).flip(-1)
    assert torch.allclose(dg, g.grad, atol=1e-10, rtol=1e-10)
