"""cyfa_chunk_fwd_noalloc (the op on the library's per-device scratch array)
against cyfa_chunk_fwd / cyfa_chunk_fwd_normed with a caller workspace: the
same kernels on the same inputs, so outputs and states are bit-identical. Two
calls in a row, the second smaller, so the second runs on the array the first
left filled; then an oversize call is refused before any launch."""

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(B, T, H, seed):
    gen = torch.Generator().manual_seed(seed)
    x = dict(
        q=torch.randn(B, T, H, 256, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, 256, generator=gen).bfloat16(),
        v=torch.randn(B, T, H, 256, generator=gen).bfloat16(),
        g=torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 3),
        delta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        readout=torch.eye(127).expand(H, 127, 127) + 0.05 * torch.randn(H, 127, 127, generator=gen),
        q_norm_weight=1 + 0.1 * torch.randn(256, generator=gen),
        k_norm_weight=1 + 0.1 * torch.randn(256, generator=gen),
    )
    init = (0.3 * torch.randn(B, H, 256, 128, generator=gen), 0.3 * torch.randn(B, H, 128, 256, generator=gen),
            50 * torch.rand(B, H, generator=gen))
    norm = ((1 + 0.2 * torch.randn(256, generator=gen)).to(DEV),
            (2 * torch.randn(B, T, H, 256, generator=gen)).bfloat16().to(DEV), 1e-6, 127.0)
    return {n: t.to(DEV) for n, t in x.items()}, tuple(t.to(DEV) for t in init), norm


@pytest.mark.parametrize("normed", [False, True])
def test_noalloc_equals_workspace_entry_point(normed):
    from cyclic_flow_attention.ops import chunk_cyfa

    for B, T, H, seed in ((8, 2048, 4, 1), (2, 333, 2, 2)):  # the second call is smaller
        x, init, norm = _case(B, T, H, seed)
        kw = dict(initial_state=init, output_final_state=True, output_norm=norm if normed else None)
        with torch.no_grad():
            o_ref, st_ref = chunk_cyfa(**x, **kw)
            o, st = chunk_cyfa(**x, **kw, no_alloc=True)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"B{B} T{T} H{H}: outputs differ"
        for a, b in zip(st, st_ref):
            assert torch.equal(a, b), f"B{B} T{T} H{H}: states differ"


def test_noalloc_refuses_oversize_before_launch():
    from cyclic_flow_attention.ops import chunk_cyfa

    B, T, H = 64, 2048, 4  # 132 MiB of intermediates, above the 80 MiB array
    q = torch.zeros(B, T, H, 256, dtype=torch.bfloat16, device=DEV)
    g = torch.zeros(B, T, H, device=DEV)
    x = dict(q=q, k=q, v=q, g=g, delta=g, beta=g, readout=torch.eye(127, device=DEV).expand(H, 127, 127),
             q_norm_weight=torch.ones(256, device=DEV), k_norm_weight=torch.ones(256, device=DEV))
    with pytest.raises(NotImplementedError, match="scratch"):
        with torch.no_grad():
            chunk_cyfa(**x, no_alloc=True)
