"""GPU parity of the HIP op path against the CPU oracle (exact float64 mode).

Tolerance (north star, bf16 HIP path vs fp32-or-better reference):
max |a - b| <= 2e-2 and mean|a - b| / mean|b| <= 5e-3, on the op outputs and
the returned fp32 states. Inputs are identical seeded tensors: bf16 q/k/v on
the GPU and the same bf16 values widened to float64 for the oracle.
"""

import os

import pytest
import torch

from oracle import cyfa_oracle as O
from tolerance import assert_close

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, T, H, K=256, V=256, seed=0, state=False, clock_scale=50.0):
    gen = torch.Generator().manual_seed(seed)
    x = dict(
        q=torch.randn(B, T, H, K, generator=gen).bfloat16(),
        k=torch.randn(B, T, H, K, generator=gen).bfloat16(),
        v=torch.randn(B, T, H, V, generator=gen).bfloat16(),
        g=torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 3),
        delta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
        readout=torch.eye(127).expand(H, 127, 127) + 0.05 * torch.randn(H, 127, 127, generator=gen),
        q_norm_weight=1 + 0.1 * torch.randn(K, generator=gen),
        k_norm_weight=1 + 0.1 * torch.randn(K, generator=gen),
    )
    init = None
    if state:
        init = (
            0.3 * torch.randn(B, H, K, 128, generator=gen),
            0.3 * torch.randn(B, H, 128, V, generator=gen),
            clock_scale * torch.rand(B, H, generator=gen),
        )
    return x, init


def _gpu(x, init):
    xg = {k: v.to(DEV) for k, v in x.items()}
    ig = None if init is None else tuple(t.to(DEV) for t in init)
    return xg, ig


def _oracle(x, init):
    xd = {k: v.double() for k, v in x.items()}
    idd = None if init is None else tuple(t.double() for t in init)
    return xd, idd


def _check_states(got, ref, what):
    names = ("hk", "hv", "clock")
    for a, b, n in zip(got, ref, names):
        if n == "clock":
            torch.testing.assert_close(a.double().cpu(), b, atol=5e-3, rtol=1e-6, msg=f"{what} clock")
        else:
            assert_close(a, b, what=f"{what} {n}")


def test_readout_table_matches_oracle():
    from cyclic_flow_attention.ops.utils import readout_table

    gen = torch.Generator().manual_seed(1)
    ro = torch.eye(127).expand(3, 127, 127) + 0.1 * torch.randn(3, 127, 127, generator=gen)
    got = readout_table(ro.to(DEV)).cpu().double()
    torch.testing.assert_close(got, O.readout_table(ro.double()), atol=2e-5, rtol=0)


@pytest.mark.parametrize("B,H,K,V,state", [(3, 2, 256, 256, True), (2, 4, 256, 256, False),
                                           (1, 1, 128, 128, True), (2, 2, 256, 128, True),
                                           (64, 4, 256, 256, True)])  # configuration 4: 256 workgroups
def test_decode_step_matches_oracle(B, H, K, V, state):
    from cyclic_flow_attention.ops import fused_recurrent_cyfa

    x, init = _inputs(B, 1, H, K, V, seed=B * 10 + H, state=state, clock_scale=1e4)
    xg, ig = _gpu(x, init)
    xd, idd = _oracle(x, init)
    with torch.no_grad():
        o, st = fused_recurrent_cyfa(**xg, initial_state=ig, output_final_state=True)
    torch.cuda.synchronize()
    ro, rst = O.fused_recurrent_cyfa(**xd, initial_state=idd, output_final_state=True)
    assert_close(o, ro, what="decode o")
    _check_states(st, rst, "decode")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_step_inplace_equals_out_of_place(dtype):
    """An in-place step (states updated in their own buffers) gives the bits
    of an out-of-place one, for bf16 and for fp32 operands (the tuned kernel's
    fp32 form)."""
    from cyclic_flow_attention.ops import fused_recurrent_cyfa

    x, init = _inputs(2, 1, 2, seed=5, state=True)
    for name in ("q", "k", "v"):
        x[name] = x[name].to(dtype)
    xg, ig = _gpu(x, init)
    with torch.no_grad():
        o1, st1 = fused_recurrent_cyfa(**xg, initial_state=ig, output_final_state=True)
        buf = tuple(t.clone() for t in ig)
        o2, st2 = fused_recurrent_cyfa(**xg, initial_state=buf, output_final_state=True, inplace=True)
    assert st2[0].data_ptr() == buf[0].data_ptr()
    assert torch.equal(o1, o2)
    for a, b in zip(st1, st2):
        assert torch.equal(a, b)


CHUNK_CASES = [
    # B, T, H, initial state, forced chunks per segment (None = heuristic)
    (1, 2048, 4, False, None),   # config-1 shape
    (2, 333, 2, True, None),     # ragged T, many one-chunk segments
    (1, 1, 1, False, None),      # a single token
    (1, 63, 1, True, None),
    (1, 130, 2, True, "1"),
    (1, 512, 2, True, "3"),      # segments of 3 chunks, last one shorter
    (2, 512, 2, True, "100"),    # one segment: no segment-state kernel
    (16, 1024, 4, False, None),  # 64 sequences, 4 chunks per segment
    (8, 2048, 4, True, None),    # configuration 3's attention shape: 8 segments of 4 chunks
    (1, 65536, 2, True, None),   # four times configuration 5's length: 1024 chunks, the clock past 3e4
]


@pytest.mark.parametrize("B,T,H,state,seg", CHUNK_CASES)
def test_chunk_matches_oracle(B, T, H, state, seg, monkeypatch):
    from cyclic_flow_attention.ops import chunk_cyfa

    if seg is not None:
        monkeypatch.setenv("CYFA_SEGMENT_CHUNKS", seg)
    x, init = _inputs(B, T, H, seed=T + B, state=state)
    xg, ig = _gpu(x, init)
    xd, idd = _oracle(x, init)
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
    torch.cuda.synchronize()
    ro, rst = O.chunk_cyfa(**xd, initial_state=idd, output_final_state=True)
    assert o.shape == (B, T, H, 256) and o.dtype == torch.bfloat16
    assert_close(o, ro, what=f"chunk o B{B} T{T} H{H}")
    _check_states(st, rst, "chunk")


@pytest.mark.parametrize("case", ["strong_decay", "extreme_decay", "large_values"])
def test_chunk_state_scale_paths(case, monkeypatch):
    """Paths of the sweeps' state bookkeeping that mild gates never reach.

    strong_decay: about 2^-23 of decay per chunk, so the per-workgroup state
    scale falls below 2^-64 every few chunks and is multiplied into the fp32
    accumulators; extreme_decay: the chunk decay underflows to zero in fp32
    (the state restarts from the chunk's own update, as the oracle's 2^-185
    factor makes it); large_values: value magnitudes of 3e4 drive the
    segment-local value states past the fp16 range, so they are stored with a
    power-of-two scale. Outputs and value states are compared after dividing
    by the value scale (the tolerance is absolute in max-abs)."""
    from cyclic_flow_attention.ops import chunk_cyfa

    monkeypatch.setenv("CYFA_SEGMENT_CHUNKS", "2")
    B, T, H = 2, 640, 2
    x, init = _inputs(B, T, H, seed=31, state=True)
    gen = torch.Generator().manual_seed(32)
    scale = 1.0
    if case == "strong_decay":
        x["g"] = -0.25 - 0.05 * torch.rand(B, T, H, generator=gen)
    elif case == "extreme_decay":
        x["g"] = -3.0 - torch.rand(B, T, H, generator=gen)
    else:
        scale = 3e4
        x["v"] = (x["v"].float() * scale).bfloat16()
        init = (init[0], init[1] * scale, init[2])
    xg, ig = _gpu(x, init)
    xd, idd = _oracle(x, init)
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
    torch.cuda.synchronize()
    ro, rst = O.chunk_cyfa(**xd, initial_state=idd, output_final_state=True)
    assert torch.isfinite(o.float()).all()
    assert_close(o.double().cpu() / scale, ro / scale, what=f"state paths {case} o")
    assert_close(st[0], rst[0], what=f"state paths {case} hk")
    assert_close(st[1].double().cpu() / scale, rst[1] / scale, what=f"state paths {case} hv")


def test_chunk_long_clock_range_reduction():
    """Clock values around 1.2e4 (the config-5 regime) keep their phase accuracy."""
    from cyclic_flow_attention.ops import chunk_cyfa

    x, init = _inputs(1, 1024, 2, seed=77, state=True, clock_scale=0.0)
    init = (init[0], init[1], torch.full((1, 2), 12000.5))
    xg, ig = _gpu(x, init)
    xd, idd = _oracle(x, init)
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
    ro, rst = O.chunk_cyfa(**xd, initial_state=idd, output_final_state=True)
    assert_close(o, ro, what="long clock o")
    _check_states(st, rst, "long clock")


def test_chunk_equals_recurrent_decode_on_gpu():
    """Chunkwise prefill and T single-token decode steps agree (both HIP paths)."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    x, init = _inputs(2, 100, 2, seed=9, state=True)
    xg, ig = _gpu(x, init)
    with torch.no_grad():
        oc, stc = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
        st = ig
        outs = []
        for t in range(100):
            step = {k: (v[:, t:t + 1] if k in ("q", "k", "v", "g", "delta", "beta") else v) for k, v in xg.items()}
            o, st = fused_recurrent_cyfa(**step, initial_state=st, output_final_state=True)
            outs.append(o)
    orr = torch.cat(outs, dim=1)
    assert_close(orr, oc.float(), what="chunk vs recurrent o")
    for a, b, n in zip(st, stc, ("hk", "hv", "clock")):
        assert_close(a, b.double(), what=f"chunk vs recurrent {n}")


def test_prefix_chunk_then_decode():
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    x, _ = _inputs(1, 80, 2, seed=13)
    xg, _ = _gpu(x, None)
    seq = ("q", "k", "v", "g", "delta", "beta")
    with torch.no_grad():
        full, stf = chunk_cyfa(**xg, output_final_state=True)
        pre = {k: (v[:, :64] if k in seq else v) for k, v in xg.items()}
        _, st = chunk_cyfa(**pre, output_final_state=True)
        outs = []
        for t in range(64, 80):
            step = {k: (v[:, t:t + 1] if k in seq else v) for k, v in xg.items()}
            o, st = fused_recurrent_cyfa(**step, initial_state=st, output_final_state=True)
            outs.append(o)
    assert_close(torch.cat(outs, 1), full[:, 64:].float(), what="prefix+decode o")
    for a, b, n in zip(st, stf, ("hk", "hv", "clock")):
        assert_close(a, b.double(), what=f"prefix+decode {n}")


@pytest.mark.parametrize("B,T,H,seg", [(1, 130, 2, "1"), (2, 333, 2, None), (1, 2048, 4, None)])
def test_chunk_output_norm_equals_separate_norm(B, T, H, seg, monkeypatch):
    """The gated output norm in the pass-2 epilogue (cyfa_chunk_fwd_normed)
    against cyfa_chunk_fwd followed by cyfa_rms_norm on the same inputs: the
    same roundings, so results differ only where the per-token sum of squares,
    added in another order, moves a value across a bf16 rounding boundary."""
    from cyclic_flow_attention import _native
    from cyclic_flow_attention.ops import chunk_cyfa

    if seg is not None:
        monkeypatch.setenv("CYFA_SEGMENT_CHUNKS", seg)
    x, init = _inputs(B, T, H, seed=5 * T + B, state=True)
    xg, ig = _gpu(x, init)
    gen = torch.Generator().manual_seed(T)
    gate = (2 * torch.randn(B, T, H, 256, generator=gen)).bfloat16().to(DEV)
    weight = (1 + 0.2 * torch.randn(256, generator=gen)).to(DEV)
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
        ref = _native.rms_norm(o, weight, 1e-6, gate, prescale=127.0)
        on, stn = chunk_cyfa(**xg, initial_state=ig, output_final_state=True,
                             output_norm=(weight, gate, 1e-6, 127.0))
    torch.cuda.synchronize()
    for a, b in zip(st, stn):
        assert torch.equal(a, b)
    a, b = on.float(), ref.float()
    ulp = torch.ldexp(torch.ones_like(b), torch.frexp(b)[1] - 8)  # one bf16 ulp of the reference value
    diff = (a - b).abs()
    assert (diff <= ulp).all(), f"max diff {diff.max().item()}"
    assert (diff > 0).float().mean().item() < 1e-2


def test_config5_long_carry_prefill_then_decode():
    """Configuration 5's attention shape: B=1, H=8, a 16384-token chunkwise
    prefill (the clock reaches about 8200, 32 segments carry the state) followed
    by configuration 5's 512 fused decode steps from the prefill's states, all
    against the oracle on identical inputs: the prefill's o, every decode
    step's o and the states after the last step.

    Between calls the state is the interface's fp32 cache (the clock is an
    fp32 [B, H] tensor and a decode step forms lam = clock + delta in fp32,
    ops/fused_recurrent.py:91 of the reference), so the oracle's clock is
    carried through fp32 as well: at lam ~ 8200 one fp32 rounding is up to
    4.9e-4, and a float64 clock drifts away from any fp32 state by a random
    walk of those roundings (about 9e-3 after 512 steps), which rotates the
    high Fourier pairs of the newest write vectors (7.7e-3 mean-rel on hk)."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    T, steps = 16384, 512
    x, _ = _inputs(1, T + steps, 8, seed=5)
    xg, _ = _gpu(x, None)
    xd, _ = _oracle(x, None)
    seq = ("q", "k", "v", "g", "delta", "beta")
    pre_g = {k: (v[:, :T] if k in seq else v) for k, v in xg.items()}
    pre_d = {k: (v[:, :T] if k in seq else v) for k, v in xd.items()}
    with torch.no_grad():
        o, st = chunk_cyfa(**pre_g, output_final_state=True)
        outs = []
        for t in range(T, T + steps):
            step = {k: (v[:, t:t + 1] if k in seq else v) for k, v in xg.items()}
            od, st = fused_recurrent_cyfa(**step, initial_state=st, output_final_state=True)
            outs.append(od)
    torch.cuda.synchronize()
    ro, rst = O.chunk_cyfa(**pre_d, output_final_state=True)
    assert_close(o, ro, what="config 5 prefill o")
    routs = []
    for t in range(T, T + steps):
        rst = (rst[0], rst[1], rst[2].float().double())  # the fp32 clock of the cache
        step = {k: (v[:, t:t + 1] if k in seq else v) for k, v in xd.items()}
        r1, rst = O.fused_recurrent_cyfa(**step, initial_state=rst, output_final_state=True)
        routs.append(r1)
    assert_close(torch.cat(outs, 1), torch.cat(routs, 1), what="config 5 decode o")
    _check_states(st, rst, "config 5")


def test_readout_range_guard_coherent_long_context():
    """Coherent q/k, alpha ~ 1 and a slowly moving clock over 16384 tokens
    drive the pass-1 output past the fp16 range for about two thirds of the
    tokens (tests/coherent_inputs.py; a CPU test checks that). The fused
    readout scales z per token and the table per head by powers of two, so the
    prefill stays finite and matches the oracle; a decode step continuing from
    its states (fp32 readout) agrees as well. The table's entries (~1e-4) sit
    at the edge of the fp16 normal range, which the per-head table scale
    covers. Outputs are compared relative to their RMS (they grow with T);
    the max-abs bound is the larger of the north-star 2e-2 and 1.5x the
    reference's own bf16 rounding (oracle mirror mode) on the same inputs
    (~0.057 of the RMS here)."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    from coherent_inputs import coherent_inputs

    T = 16384
    x = coherent_inputs(T=T + 1)
    seq = ("q", "k", "v", "g", "delta", "beta")
    pre = {n: (t[:, :T] if n in seq else t) for n, t in x.items()}
    last = {n: (t[:, T:] if n in seq else t) for n, t in x.items()}
    with torch.no_grad():
        o, st = chunk_cyfa(**{n: t.to(DEV) for n, t in pre.items()}, output_final_state=True)
        od, _ = fused_recurrent_cyfa(**{n: t.to(DEV) for n, t in last.items()}, initial_state=st,
                                     output_final_state=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(od.float()).all()
    pre_d = {n: t.double() for n, t in pre.items()}
    ro, rst = O.chunk_cyfa(**pre_d, output_final_state=True)
    rm, _ = O.chunk_cyfa(**pre_d, mode="mirror")
    rod, _ = O.fused_recurrent_cyfa(**{n: t.double() for n, t in last.items()}, initial_state=rst,
                                    output_final_state=True)
    rms = ro.pow(2).mean().sqrt()
    own = (rm / rms - ro / rms).abs().max().item()
    assert_close(o.double().cpu() / rms, ro / rms, max_abs=max(2e-2, 1.5 * own), what="range guard o")
    for a, b, n in zip(st[:2], rst[:2], ("hk", "hv")):
        assert_close(a, b, max_abs=float("inf"), what=f"range guard {n}")
    drms = rod.pow(2).mean().sqrt()
    assert_close(od.double().cpu() / drms, rod / drms, what="range guard decode o")


def test_decode_refuses_host_tensors_before_launch():
    """A CPU initial state, or a precomputed table of the wrong dtype, raises
    ValueError before any launch (the kernel would otherwise read host memory)."""
    from cyclic_flow_attention.ops import fused_recurrent_cyfa

    x, init = _inputs(1, 1, 2, seed=3, state=True)
    xg, _ = _gpu(x, None)
    with pytest.raises(ValueError):
        fused_recurrent_cyfa(**xg, initial_state=init)
    with pytest.raises(ValueError):
        fused_recurrent_cyfa(**xg, table=torch.zeros(2, 127, 128, dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("B,H,K,V", [(1, 8, 256, 256), (3, 2, 256, 256), (2, 3, 128, 256), (1, 4, 256, 128),
                                     (5, 1, 128, 128), (15, 4, 256, 256)])
def test_decode_split_equals_one_workgroup_form(B, H, K, V):
    """Small batches (B H < 64) split each (b, h) across eight workgroups;
    the split form and the one-workgroup form give bit-identical outputs and
    states (raw and o are reduced in the same order in both), in place as
    well, and match the oracle."""
    from cyclic_flow_attention.ops import fused_recurrent_cyfa

    x, init = _inputs(B, 1, H, K, V, seed=B * 7 + H, state=True, clock_scale=1e4)
    xg, ig = _gpu(x, init)
    with torch.no_grad():
        o1, st1 = fused_recurrent_cyfa(**xg, initial_state=ig, output_final_state=True, split=False)
        o2, st2 = fused_recurrent_cyfa(**xg, initial_state=ig, output_final_state=True, split=True)
        buf = tuple(t.clone() for t in ig)
        o3, st3 = fused_recurrent_cyfa(**xg, initial_state=buf, output_final_state=True, inplace=True)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(o1, o3)
    for a, b, c in zip(st1, st2, st3):
        assert torch.equal(a, b) and torch.equal(a, c)
    ro, rst = O.fused_recurrent_cyfa(**_oracle(x, init)[0], initial_state=_oracle(x, init)[1], output_final_state=True)
    assert_close(o2, ro, what=f"split decode o B{B} H{H}")
    _check_states(st2, rst, "split decode")


# fp32 operands: fp32 arithmetic throughout (5e-7 mean-rel observed on
# MI355X); fp16: the same, with o returned in fp16, whose own rounding
# (2^-11 relative) gives about 1.8e-4 mean-rel
WIDE_BARS = {torch.float32: dict(max_abs=1e-4, mean_rel=1e-5), torch.float16: dict(max_abs=1e-3, mean_rel=5e-4)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_wide_operands_compute_in_fp32(dtype):
    """fp32 and fp16 q, k, v at the tuned shape (K = V = 256, 128 slots,
    chunk 64) are not rounded to bf16: like the reference, which takes its
    fused bf16 kernels only for bf16 inputs and otherwise computes in the
    input dtype (ops/chunk.py:209-223, 257-264, 285-331), they run in fp32.
    The chunk op, its final states and a decode step from them match the
    float64 oracle at fp32-level tolerance -- a bf16 rounding of q, k, v alone
    would give about 3e-3 mean-rel -- and o comes back in the input dtype."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    x, init = _inputs(2, 130, 2, seed=11, state=True)
    gen = torch.Generator().manual_seed(12)
    for name in ("q", "k", "v"):
        x[name] = torch.randn(x[name].shape, generator=gen).to(dtype)
    xg, ig = _gpu(x, init)
    xd, idd = _oracle(x, init)
    seq = ("q", "k", "v", "g", "delta", "beta")
    step = {k: (v[:, :1] if k in seq else v) for k, v in xg.items()}
    with torch.no_grad():
        o, st = chunk_cyfa(**xg, initial_state=ig, output_final_state=True)
        od, std = fused_recurrent_cyfa(**step, initial_state=st, output_final_state=True)
    torch.cuda.synchronize()
    assert o.dtype == dtype and od.dtype == dtype
    ro, rst = O.chunk_cyfa(**xd, initial_state=idd, output_final_state=True, mode="exact")
    stepd = {k: (v[:, :1] if k in seq else v) for k, v in xd.items()}
    rod, rstd = O.fused_recurrent_cyfa(**stepd, initial_state=rst, output_final_state=True, mode="exact")
    bar = WIDE_BARS[dtype]
    f32 = WIDE_BARS[torch.float32]
    assert_close(o, ro, what=f"{dtype} chunk o", **bar)
    assert_close(st[0], rst[0], what=f"{dtype} chunk hk", **f32)
    assert_close(st[1], rst[1], what=f"{dtype} chunk hv", **f32)
    torch.testing.assert_close(st[2].double().cpu(), rst[2], atol=1e-4, rtol=1e-6)
    assert_close(od, rod, what=f"{dtype} decode o", **bar)
    assert_close(std[0], rstd[0], what=f"{dtype} decode hk", **f32)
    assert_close(std[1], rstd[1], what=f"{dtype} decode hv", **f32)


@pytest.mark.parametrize("dtype,K,M", [(torch.bfloat16, 256, 128), (torch.float32, 256, 128),
                                       (torch.bfloat16, 64, 96)])
def test_forward_repeats_bit_for_bit_on_any_stream(dtype, K, M):
    """The chunk op and a decode step give identical bits when run twice, and
    when run on a side stream instead of the default one (every partial sum
    in the kernels is added in a fixed order; the launches go on the caller's
    current stream). Covers the tuned kernels (bf16, K = V = 256, 128 slots)
    and the general path (fp32 operands; another head size and slot count)."""
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    gen = torch.Generator().manual_seed(21)
    B, T, H = 2, 300, 2
    R = M - 1
    x = dict(q=torch.randn(B, T, H, K, generator=gen).to(dtype), k=torch.randn(B, T, H, K, generator=gen).to(dtype),
             v=torch.randn(B, T, H, K, generator=gen).to(dtype),
             g=torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=gen) + 3),
             delta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             readout=torch.eye(R).expand(H, R, R) + 0.05 * torch.randn(H, R, R, generator=gen),
             q_norm_weight=1 + 0.1 * torch.randn(K, generator=gen), k_norm_weight=1 + 0.1 * torch.randn(K, generator=gen))
    xg = {k: v.to(DEV) for k, v in x.items()}
    seq = ("q", "k", "v", "g", "delta", "beta")
    step = {k: (v[:, -1:] if k in seq else v) for k, v in xg.items()}

    def run():
        with torch.no_grad():
            o, st = chunk_cyfa(**xg, output_final_state=True)
            od, std = fused_recurrent_cyfa(**step, initial_state=st, output_final_state=True)
        return (o,) + tuple(st) + (od,) + tuple(std)

    first = run()
    second = run()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        third = run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for a, b, c in zip(first, second, third):
        assert torch.equal(a, b)
        assert torch.equal(a, c)
