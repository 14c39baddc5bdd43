"""Pin of the oracle's two-pass absolute-clock CyFA against the README's
relative-time definition with dense slot transports (oracle/relative_time.py).

The relative-time form uses neither the Fourier basis, nor U(lambda), nor the
write vector, nor the readout table, so agreement to 1e-10 in float64 pins all
of them together, plus the two ScalarGatedLA passes and the readout.
"""

import pytest
import torch

from oracle import cyfa_oracle as O
from oracle.relative_time import relative_time_attention

R = 127


def _inputs(T, K, V, H=1, B=1, seed=0, readout_noise=0.1):
    gen = torch.Generator().manual_seed(seed)
    d = torch.float64
    q = torch.randn(B, T, H, K, dtype=d, generator=gen)
    k = torch.randn(B, T, H, K, dtype=d, generator=gen)
    v = torch.randn(B, T, H, V, dtype=d, generator=gen)
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, dtype=d, generator=gen) + 2)
    delta = torch.sigmoid(torch.randn(B, T, H, dtype=d, generator=gen))
    beta = torch.sigmoid(torch.randn(B, T, H, dtype=d, generator=gen))
    Rm = torch.eye(R, dtype=d)[None] + readout_noise * torch.randn(H, R, R, dtype=d, generator=gen)
    qw = 0.5 + torch.rand(K, dtype=d, generator=gen)
    kw = 0.5 + torch.rand(K, dtype=d, generator=gen)
    return q, k, v, g, delta, beta, Rm, qw, kw


def _brute(q, k, v, g, delta, beta, Rm, qw, kw, b=0, h=0, K0=None, V0=None):
    K = q.shape[-1]
    qh = O.head_rmsnorm(q, qw, 1e-6)[b, :, h] * K**-0.5
    kh = O.head_rmsnorm(k, kw, 1e-6)[b, :, h]
    return relative_time_attention(qh, kh, v[b, :, h], torch.exp(g[b, :, h]), delta[b, :, h], beta[b, :, h],
                                   Rm[h], K0, V0)


@pytest.mark.parametrize("T,K,V,C", [(37, 16, 8, 16), (70, 32, 24, 32), (20, 256, 256, 64)])
def test_two_pass_equals_relative_time(T, K, V, C):
    args = _inputs(T, K, V, H=2, seed=T)
    o, st = O.chunk_cyfa(*args, output_final_state=True, chunk_size=C)
    for h in range(2):
        ob, _, _ = _brute(*args, h=h)
        torch.testing.assert_close(o[0, :, h], ob, atol=1e-10, rtol=0)
    o_rec, st_rec = O.recurrent_cyfa(*args)
    torch.testing.assert_close(o_rec, o, atol=1e-12, rtol=0)
    for a, b in zip(st, st_rec):
        torch.testing.assert_close(a, b, atol=1e-12, rtol=0)


def test_initial_state_maps_from_slot_space():
    """A nonzero slot-space start K0/V0 corresponds to hk = (U(-c0) Phi^T K0)^T."""
    T, K, V = 30, 16, 12
    args = _inputs(T, K, V, seed=11)
    gen = torch.Generator().manual_seed(12)
    K0 = torch.randn(R, K, dtype=torch.float64, generator=gen)
    V0 = torch.randn(R, V, dtype=torch.float64, generator=gen)
    c0 = torch.tensor([[123.37]], dtype=torch.float64)
    phi = O.basis(128)
    c, s = O.phase_cos_sin(c0[0])
    hk = O.rotate((phi.T @ K0).T, c.expand(K, 64), s.expand(K, 64), negative=True)  # [K, M]
    hv = O.rotate((phi.T @ V0).T, c.expand(V, 64), s.expand(V, 64), negative=True).T  # [M, V]
    o, _ = O.chunk_cyfa(*args, initial_state=(hk[None, None], hv[None, None], c0), chunk_size=16)
    ob, _, _ = _brute(*args, K0=K0, V0=V0)
    torch.testing.assert_close(o[0, :, 0], ob, atol=1e-10, rtol=0)


def test_zero_state_output_is_clock_offset_invariant():
    args = _inputs(45, 16, 8, seed=21)
    B, T, H, K = args[0].shape
    zeros = (torch.zeros(B, H, K, 128, dtype=torch.float64), torch.zeros(B, H, 128, 8, dtype=torch.float64))
    o1, _ = O.chunk_cyfa(*args, chunk_size=16)
    o2, _ = O.chunk_cyfa(*args, initial_state=zeros + (torch.full((B, H), 5071.5, dtype=torch.float64),),
                         chunk_size=16)
    torch.testing.assert_close(o1, o2, atol=1e-10, rtol=0)
