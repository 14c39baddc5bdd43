"""CPU restatement of the CyFA attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use this module, and only as the checker. The product package
never imports it.

Two numeric modes:

* ``mode="exact"``: float64 arithmetic on the given inputs with no intermediate
  rounding. This is the "fp32 reference" the north-star tolerances are quoted
  against (float64 is used so the oracle's own error is negligible).
* ``mode="mirror"``: float32 arithmetic with bfloat16 rounding at the points the
  reference rounds on its large fused path (normalised q/k, write vector,
  decayed values, masked scores, per-128-wide-key-slice pass-1 output, rotated
  readout input, table, probabilities, slot weights, pass-2 output). It
  documents the rounding budget of the reference itself.

Every function cites the reference file:line it restates. Paths are relative to
the reference root (Chyxx/CyFA-Jittor v0.1.2).
"""

import math

import torch

LOG2E = 1.4426950408889634

__all__ = [
    "basis",
    "readout_table",
    "clock_phase",
    "phase_cos_sin",
    "write_vector",
    "rotate",
    "head_rmsnorm",
    "sgla_chunk",
    "sgla_recurrent",
    "slot_readout",
    "chunk_cyfa",
    "fused_recurrent_cyfa",
    "recurrent_cyfa",
]


def _check_mode(mode):
    if mode not in ("exact", "mirror"):
        raise ValueError(f"mode must be 'exact' or 'mirror', got {mode!r}")
    return torch.float64 if mode == "exact" else torch.float32


def _rnd(x, mode):
    """bfloat16 round-to-nearest-even in mirror mode, identity in exact mode."""
    if mode == "mirror":
        return x.to(torch.bfloat16).to(torch.float32)
    return x


def basis(M=128, mode="exact"):
    """Real-DFT slot basis Phi [M-1, M] (ops/chunk.py:82-103).

    Phi[r, 2p] = s_p cos(2 pi p r / R), Phi[r, 2p+1] = s_p sin(2 pi p r / R),
    Phi[:, 1] = 0, s_0 = R^-1/2, s_p = (2/R)^1/2, R = M - 1.
    """
    dt = _check_mode(mode)
    period = M - 1
    col = torch.arange(M)
    row = torch.arange(period, dtype=dt)[:, None]
    pair = (col // 2).to(dt)[None, :]
    if mode == "mirror":
        # float32 products as the reference's __fmul_rn (ops/chunk.py:92-93)
        omega = pair * torch.tensor(2 * math.pi / period, dtype=dt)
        phase = row * omega
    else:
        phase = row * pair * (2 * math.pi / period)
    z = torch.where(col % 2 == 1, torch.sin(phase), torch.cos(phase))
    scale = torch.where(
        col < 2,
        torch.tensor(period**-0.5, dtype=dt),
        torch.tensor((2 / period) ** 0.5, dtype=dt),
    )
    phi = z * scale
    phi[:, 1] = 0
    return phi


def readout_table(readout, mode="exact"):
    """table_h = readout_h @ Phi, [H, M-1, M] (ops/chunk.py:281)."""
    dt = _check_mode(mode)
    M = readout.shape[-1] + 1
    return readout.to(dt) @ basis(M, mode)


def clock_phase(lam, mode="exact", M=128):
    """Integer range-reduced clock phase theta[..., p] (ops/utils.py:649-661).

    wi = floor(lam) mod R (non-negative); coord = ((wi*p) mod R) + frac(lam)*p,
    wrapped into (-R/2, R/2]; theta = coord * 2 pi / R.
    """
    dt = _check_mode(mode)
    R = M - 1
    lam = lam.to(dt)
    whole = torch.floor(lam)
    frac = lam - whole
    wi = torch.remainder(whole.to(torch.int64), R)
    pair = torch.arange(M // 2, dtype=torch.int64)
    coord = torch.remainder(wi[..., None] * pair, R).to(dt) + frac[..., None] * pair.to(dt)
    coord = torch.where(coord > R * 0.5, coord - R, coord)
    if mode == "mirror":
        return coord * torch.tensor(2 * math.pi / R, dtype=dt)
    return coord * (2 * math.pi / R)


def phase_cos_sin(lam, mode="exact", M=128):
    theta = clock_phase(lam, mode, M)
    return torch.cos(theta), torch.sin(theta)


def _pair_scale(M, dt):
    R = M - 1
    pair = torch.arange(M // 2)
    return torch.where(
        pair == 0, torch.tensor((1.0 / R) ** 0.5, dtype=dt), torch.tensor((2.0 / R) ** 0.5, dtype=dt)
    )


def write_vector(lam, beta, mode="exact", M=128):
    """w = beta * U(-lam) b, [..., M] (ops/utils.py:664-702, ops/chunk.py:265-279).

    w[2p] = beta s_p cos(theta_p), w[2p+1] = -beta s_p sin(theta_p).
    """
    dt = _check_mode(mode)
    c, s = phase_cos_sin(lam, mode, M)
    sp = _pair_scale(M, dt)
    b = beta.to(dt)[..., None]
    w = torch.stack([b * sp * c, -b * sp * s], dim=-1).reshape(*c.shape[:-1], M)
    return _rnd(w, mode)


def rotate(x, c, s, negative=False):
    """Pairwise U(lam) x (negative=False) or U(-lam) x (ops/chunk.py:115-124)."""
    pairs = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
    e, o = pairs[..., 0], pairs[..., 1]
    if negative:
        y0, y1 = c * e + s * o, -s * e + c * o
    else:
        y0, y1 = c * e - s * o, s * e + c * o
    return torch.stack([y0, y1], dim=-1).reshape(x.shape)


def head_rmsnorm(x, weight, eps, mode="exact"):
    """x * rsqrt(mean(x^2) + eps) * w over the last dim (ops/qk_norm.py:206-233)."""
    dt = _check_mode(mode)
    xf = x.to(dt)
    rs = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
    return _rnd(xf * rs * weight.to(dt), mode)


def _exp_gate(x, mode):
    # Mirror mode works in log2 units like the kernels (exp2f); exact uses e^x.
    return torch.exp2(x) if mode == "mirror" else torch.exp(x)


def _local_cumsum(g, C, mode):
    """In-chunk inclusive cumsum of the log-gate (ops/utils.py:495-520).

    Mirror mode returns log2 units (x log2 e) as the reference's local_scan.
    """
    B, H, T = g.shape
    gc = g.reshape(B, H, T // C, C).cumsum(-1)
    if mode == "mirror":
        gc = gc * LOG2E
    return gc


def sgla_chunk(q, k, v, g, S0, scale, chunk_size=64, mode="exact", k_slices=1, round_output=False):
    """Chunkwise scalar-gated linear attention, one pass.

    Restates ops/chunk.py:136-161 (_scalar_la) with the reference's state
    convention (ops/chunk_h.py:238-327: S_n is the state *before* chunk n,
    decayed values bf16(v * 2^(G_last - G_s)) accumulated in fp32) and output
    assembly (ops/chunk_o.py:240-250, 369-374: per 128-wide key slice,
    x = scale * (2^G_t q_t S_n + sum_s bf16(mask 2^(G_t-G_s) q_t.k_s) v_s)).

    q, k [B,H,T,K]; v [B,H,T,V]; g [B,H,T] natural-log decay; S0 [B,H,K,V].
    T must be a multiple of chunk_size. ``k_slices`` splits K for the per-slice
    rounding of the reference's pass 1 (mirror mode); ``round_output`` rounds
    each slice's output to bf16. Returns (o [B,H,T,V], S_final [B,H,K,V]).
    """
    dt = _check_mode(mode)
    B, H, T, K = q.shape
    V = v.shape[-1]
    C = chunk_size
    if T % C:
        raise ValueError("sgla_chunk needs T to be a multiple of chunk_size")
    N = T // C
    q = q.to(dt).reshape(B, H, N, C, K)
    k = k.to(dt).reshape(B, H, N, C, K)
    v = v.to(dt).reshape(B, H, N, C, V)
    gc = _local_cumsum(g.to(dt), C, mode)
    S = S0.to(dt).clone()
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool))
    KS = K // k_slices
    out = []
    for n in range(N):
        G = gc[:, :, n]  # [B,H,C]
        last = G[..., -1]
        Sh = _rnd(S, mode)
        qn, kn, vn = q[:, :, n], k[:, :, n], v[:, :, n]
        decay_q = _exp_gate(G, mode)[..., None]
        rel = _exp_gate(G[..., :, None] - G[..., None, :], mode)
        acc = torch.zeros(B, H, C, V, dtype=dt)
        for sl in range(k_slices):
            ks = slice(sl * KS, (sl + 1) * KS)
            inter = (qn[..., ks] @ Sh[..., ks, :]) * decay_q
            sc = qn[..., ks] @ kn[..., ks].transpose(-1, -2)
            sc = _rnd(torch.where(mask, sc * rel, torch.zeros((), dtype=dt)), mode)
            x = (inter + sc @ vn) * scale
            if round_output:
                x = _rnd(x, mode)
            acc = acc + x
        out.append(acc)
        vt = _rnd(vn * _exp_gate(last[..., None] - G, mode)[..., None], mode)
        S = S * _exp_gate(last, mode)[..., None, None] + kn.transpose(-1, -2) @ vt
    return torch.stack(out, dim=2).reshape(B, H, T, V), S


def sgla_recurrent(q, k, v, g, S0, scale, mode="exact"):
    """Token-by-token form of one pass: S_t = a_t S_{t-1} + k_t v_t^T,
    o_t = scale S_t^T q_t (README.md:58-110; ops/fused_recurrent.py:105-111).
    """
    dt = _check_mode(mode)
    B, H, T, K = q.shape
    S = S0.to(dt).clone()
    q, k, v, g = q.to(dt), k.to(dt), v.to(dt), g.to(dt)
    out = []
    for t in range(T):
        S = S * torch.exp(g[:, :, t])[..., None, None] + k[:, :, t, :, None] * v[:, :, t, None, :]
        out.append(scale * torch.einsum("bhk,bhkv->bhv", q[:, :, t], S))
    return torch.stack(out, dim=2), S


def slot_readout(raw, lam, table, mode="exact"):
    """Token-wise slot softmax readout (ops/utils.py:779-882; fused epilogue
    ops/chunk_readout.py:797-909; decode ops/fused_recurrent.py:114-175).

    z = U(lam) raw; logits_r = sum_m z_m table[r, m] (r < R);
    p = softmax(logits); u = p @ table; weights = U(-lam) u.
    raw [B,H,T,M]; lam [B,H,T]; table [H,R,M]. Returns weights [B,H,T,M].
    """
    dt = _check_mode(mode)
    M = raw.shape[-1]
    c, s = phase_cos_sin(lam, mode, M)
    z = _rnd(rotate(raw.to(dt), c, s), mode)
    tb = _rnd(table.to(dt), mode)
    logits = torch.einsum("bhtm,hrm->bhtr", z, tb)
    p = _rnd(torch.softmax(logits, dim=-1), mode)
    u = torch.einsum("bhtr,hrm->bhtm", p, tb)
    return _rnd(rotate(u, c, s, negative=True), mode)


def chunk_cyfa(
    q,
    k,
    v,
    g,
    delta,
    beta,
    readout,
    q_norm_weight,
    k_norm_weight,
    q_norm_eps=1e-6,
    k_norm_eps=1e-6,
    scale=None,
    initial_state=None,
    output_final_state=False,
    chunk_size=64,
    mode="exact",
):
    """Chunkwise two-pass CyFA (ops/chunk.py:164-353).

    q, k, v [B,T,H,D]; g, delta, beta [B,T,H]; readout [H,R,R].
    Returns (o [B,T,H,V], (hk [B,H,K,M], hv [B,H,M,V], clock [B,H]) or None).
    """
    dt = _check_mode(mode)
    B, T, H, K = q.shape
    V = v.shape[-1]
    M = readout.shape[-1] + 1
    C = chunk_size
    pad = (-T) % C
    if pad:  # zero padding is neutral: alpha = 1, delta = 0, beta = 0 (ops/chunk.py:198-207)

        def padt(x):
            z = torch.zeros((B, pad) + tuple(x.shape[2:]), dtype=x.dtype)
            return torch.cat([x, z], dim=1)

        q, k, v, g, delta, beta = map(padt, (q, k, v, g, delta, beta))
    qh = head_rmsnorm(q, q_norm_weight, q_norm_eps, mode).permute(0, 2, 1, 3)
    kh = head_rmsnorm(k, k_norm_weight, k_norm_eps, mode).permute(0, 2, 1, 3)
    vh = v.to(dt).permute(0, 2, 1, 3)
    gh, dh, bh = (x.to(dt).permute(0, 2, 1) for x in (g, delta, beta))
    if initial_state is None:
        hk = torch.zeros(B, H, K, M, dtype=dt)
        hv = torch.zeros(B, H, M, V, dtype=dt)
        clock = None
    else:
        hk, hv, clock = (x.to(dt) for x in initial_state)
    lam = torch.cumsum(dh, dim=-1)  # ops/chunk.py:254-256
    if clock is not None:
        lam = lam + clock[..., None]
    w = write_vector(lam, bh, mode, M)
    table = readout_table(readout, mode)
    sc = K**-0.5 if scale is None else scale
    slices = K // 128 if (mode == "mirror" and K > 128 and K % 128 == 0) else 1
    raw, hkt = sgla_chunk(qh, kh, w, gh, hk, sc, C, mode, k_slices=slices, round_output=(mode == "mirror"))
    weights = slot_readout(raw, lam, table, mode)
    o, hvt = sgla_chunk(weights, w, vh, gh, hv, 1.0, C, mode, round_output=(mode == "mirror"))
    o = o.permute(0, 2, 1, 3)[:, :T]
    state = None
    if output_final_state:
        final_clock = dh.sum(-1)  # ops/chunk.py:348-352
        if clock is not None:
            final_clock = final_clock + clock
        state = (hkt, hvt, final_clock)
    return o, state


def fused_recurrent_cyfa(
    q,
    k,
    v,
    g,
    delta,
    beta,
    readout,
    q_norm_weight,
    k_norm_weight,
    q_norm_eps=1e-6,
    k_norm_eps=1e-6,
    scale=None,
    initial_state=None,
    output_final_state=False,
    mode="exact",
):
    """One decode step (ops/fused_recurrent.py:10-200, kernel 57-188).

    q, k, v [B,1,H,D]; g, delta, beta [B,1,H]. Rounding order of the decode
    kernel: q_hat = bf16(q rs w) then * scale; k_hat = bf16(k rs w);
    lam = clock + delta; hk' = e^g hk + k_hat (x) w; raw = hk'^T q_hat;
    readout; hv' = e^g hv + w (x) v; o = bf16(hv'^T weights).
    """
    dt = _check_mode(mode)
    B, T, H, K = q.shape
    V = v.shape[-1]
    M = readout.shape[-1] + 1
    if T != 1:
        raise NotImplementedError("fused_recurrent_cyfa needs T == 1")
    sc = K**-0.5 if scale is None else scale
    if initial_state is None:
        hk = torch.zeros(B, H, K, M, dtype=dt)
        hv = torch.zeros(B, H, M, V, dtype=dt)
        clock = torch.zeros(B, H, dtype=dt)
    else:
        hk, hv, clock = (x.to(dt) for x in initial_state)
    qh = head_rmsnorm(q[:, 0], q_norm_weight, q_norm_eps, mode) * sc  # [B,H,K]
    kh = head_rmsnorm(k[:, 0], k_norm_weight, k_norm_eps, mode)
    vv = v[:, 0].to(dt)
    lam = clock + delta[:, 0].to(dt)
    decay = torch.exp(g[:, 0].to(dt))[..., None, None]
    w = write_vector(lam, beta[:, 0], mode, M)  # [B,H,M]
    hk2 = hk * decay + kh[..., :, None] * w[..., None, :]
    raw = torch.einsum("bhkm,bhk->bhm", hk2, qh)
    table = readout_table(readout, mode)
    weights = slot_readout(raw[:, :, None], lam[:, :, None], table, mode)[:, :, 0]
    hv2 = hv * decay + w[..., :, None] * vv[..., None, :]
    o = _rnd(torch.einsum("bhmv,bhm->bhv", hv2, weights), mode)
    state = (hk2, hv2, lam) if output_final_state else None
    return o[:, None], state


def recurrent_cyfa(q, k, v, g, delta, beta, readout, q_norm_weight, k_norm_weight, q_norm_eps=1e-6,
                   k_norm_eps=1e-6, scale=None, initial_state=None, mode="exact"):
    """T decode steps in sequence: the token-by-token form of chunk_cyfa."""
    B, T = q.shape[:2]
    state = initial_state
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, state = fused_recurrent_cyfa(
            q[:, sl], k[:, sl], v[:, sl], g[:, sl], delta[:, sl], beta[:, sl], readout,
            q_norm_weight, k_norm_weight, q_norm_eps, k_norm_eps, scale, state, True, mode,
        )
        outs.append(o)
    return torch.cat(outs, dim=1), state
