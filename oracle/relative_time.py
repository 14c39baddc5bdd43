"""Relative-time CyFA recurrence with dense slot transports -- TEST INFRASTRUCTURE ONLY.

This is the *definition* of CyFA from the reference README (README.md:32-56),
written without the absolute-clock change of variables that the kernels use:

    K_t = a_t P(d_t) K_{t-1} + b_t e_0 k_t^T        (slot space, [R, K])
    V_t = a_t P(d_t) V_{t-1} + b_t e_0 v_t^T        ([R, V])
    o_t = (R V_t)^T softmax(R K_t q_t)

P(d) is the fractional cyclic shift of R = 127 slots, the band-limited
interpolation kernel  P(d)[r, r'] = (1/R) [1 + 2 sum_{p=1}^{63} cos(2 pi p (r - r' - d) / R)],
which for integer d is exactly the cyclic roll by d. Nothing here uses the
Fourier basis, the U(lambda) rotation, the write vector or the readout table of
``cyfa_oracle``; agreement of the two formulations on random inputs pins all of
those (README.md:58-110 states that the change of variables is exact).
"""

import math

import torch


def shift_matrix(d, R=127):
    """Dense fractional cyclic shift P(d) [R, R] in float64 (closed form)."""
    r = torch.arange(R, dtype=torch.float64)
    diff = r[:, None] - r[None, :] - float(d)
    p = torch.arange(1, (R - 1) // 2 + 1, dtype=torch.float64)
    return (1.0 + 2.0 * torch.cos(2 * math.pi * p * diff[..., None] / R).sum(-1)) / R


def relative_time_attention(q, k, v, alpha, delta, beta, R_mat, K0=None, V0=None):
    """Brute-force relative-time CyFA for one (batch, head) sequence, float64.

    q [T, K] (already normalised and scaled), k [T, K], v [T, V];
    alpha, delta, beta [T]; R_mat [R, R]. K0 [R, K] / V0 [R, V] are the initial
    slot-space memories (zero if None). Returns (o [T, V], K_T, V_T).
    """
    T, Kd = k.shape
    Vd = v.shape[-1]
    R = R_mat.shape[0]
    Km = torch.zeros(R, Kd, dtype=torch.float64) if K0 is None else K0.clone().double()
    Vm = torch.zeros(R, Vd, dtype=torch.float64) if V0 is None else V0.clone().double()
    e0 = torch.zeros(R, dtype=torch.float64)
    e0[0] = 1.0
    out = []
    Rm = R_mat.double()
    for t in range(T):
        P = shift_matrix(float(delta[t]), R)
        a = float(alpha[t])
        b = float(beta[t])
        Km = a * (P @ Km) + b * torch.outer(e0, k[t].double())
        Vm = a * (P @ Vm) + b * torch.outer(e0, v[t].double())
        logits = Rm @ (Km @ q[t].double())
        p = torch.softmax(logits, dim=0)
        out.append((Rm @ Vm).T @ p)
    return torch.stack(out), Km, Vm
