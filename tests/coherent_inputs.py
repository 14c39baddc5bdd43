"""Inputs whose pass-1 output exceeds the fp16 range (shared by a CPU check of
the inputs and the GPU range test).

q and k share one direction (with a little noise), the norm weights are 3,
the decay is almost 1 (g = -1e-4) and the clock moves slowly (delta = 2e-3),
so the key state keeps adding coherent k_hat (x) w terms: |raw| grows about
linearly with t and passes 65504 after ~10k tokens (about two thirds of the
tokens of a 16384-token sequence are beyond the fp16 range). The readout is
3e-4 (I + noise): the table's entries (at most ~9e-5) sit at the edge of the
fp16 normal range, and the logits (table . z) stay within a range of ~30, so
the slot softmax is well conditioned and a rounding cannot flip its winner.
"""

import torch


def coherent_inputs(B=1, T=16384, H=1, seed=7):
    gen = torch.Generator().manual_seed(seed)
    d = torch.randn(256, generator=gen)
    x = dict(
        q=(d + 0.05 * torch.randn(B, T, H, 256, generator=gen)).bfloat16(),
        k=(d + 0.05 * torch.randn(B, T, H, 256, generator=gen)).bfloat16(),
        v=torch.randn(B, T, H, 256, generator=gen).bfloat16(),
        g=torch.full((B, T, H), -1e-4),
        delta=torch.full((B, T, H), 2e-3),
        beta=torch.full((B, T, H), 0.9),
        readout=3e-4 * (torch.eye(127).expand(H, 127, 127) + 0.05 * torch.randn(H, 127, 127, generator=gen)),
        q_norm_weight=torch.full((256,), 3.0),
        k_norm_weight=torch.full((256,), 3.0),
    )
    return x


def pass1_output(x):
    """The exact pass-1 output raw [B, H, T, 128] and the rotated readout input z."""
    from oracle import cyfa_oracle as O

    xd = {n: t.double() for n, t in x.items()}
    B, T, H, K = xd["q"].shape
    qh = O.head_rmsnorm(xd["q"], xd["q_norm_weight"], 1e-6).permute(0, 2, 1, 3)
    kh = O.head_rmsnorm(xd["k"], xd["k_norm_weight"], 1e-6).permute(0, 2, 1, 3)
    lam = torch.cumsum(xd["delta"].permute(0, 2, 1), -1)
    w = O.write_vector(lam, xd["beta"].permute(0, 2, 1))
    raw, _ = O.sgla_chunk(qh, kh, w, xd["g"].permute(0, 2, 1), torch.zeros(B, H, K, 128, dtype=torch.float64),
                          K ** -0.5)
    c, s = O.phase_cos_sin(lam)
    return raw, O.rotate(raw, c, s)
