"""Pins of the oracle's building blocks by closed forms and library routines.

What each test pins (oracle function -> independent check):
  basis            -> Phi Phi^T = I_127, column 1 = 0, and Phi^T x against numpy.fft
  readout_table    -> R = I gives Phi; random R against numpy matmul
  clock_phase      -> float64 2 pi p lam / 127 (mod 2 pi) up to lam = 1e5, both modes
  rotate           -> U(lam) U(-lam) = I, norm preservation, and against 2x2 rotation matrices
  write_vector     -> lam = 0 gives beta * Phi[0, :]; |w| = beta for every lam
  integer clock    -> Phi U(d) Phi^T equals the cyclic roll by d (np.roll)
  fractional clock -> Phi U(d) Phi^T equals the band-limited shift kernel of relative_time
  head_rmsnorm     -> torch.nn.functional.rms_norm
  slot_readout     -> R = I, lam = 0: softmax(Phi raw) by hand
"""

import math

import numpy as np
import pytest
import torch

from oracle import cyfa_oracle as O
from oracle.relative_time import shift_matrix

R = 127


def U_matrix(d):
    """Dense 128x128 U(d) built column by column with the oracle's rotate()."""
    eye = torch.eye(128, dtype=torch.float64)
    c, s = O.phase_cos_sin(torch.tensor([float(d)], dtype=torch.float64))
    return O.rotate(eye, c.expand(128, 64), s.expand(128, 64)).T


def test_basis_orthonormal_and_fft():
    phi = O.basis(128)
    assert phi.shape == (R, 128)
    assert torch.all(phi[:, 1] == 0)
    torch.testing.assert_close(phi @ phi.T, torch.eye(R, dtype=torch.float64), atol=1e-12, rtol=0)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(R)
    X = np.fft.fft(x)
    sp = np.where(np.arange(64) == 0, math.sqrt(1 / R), math.sqrt(2 / R))
    expect = np.stack([sp * X[:64].real, -sp * X[:64].imag], axis=-1).reshape(128)
    expect[1] = 0.0
    got = (phi.T @ torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, expect, atol=1e-12)


def test_basis_mirror_close_to_exact():
    # The reference builds Phi in fp32 from the unreduced phase r * p * 2 pi / R
    # (up to ~390 rad), so its entries carry ~|phase| * 2^-24 absolute error.
    torch.testing.assert_close(O.basis(128, "mirror").double(), O.basis(128), atol=1e-5, rtol=0)


def test_readout_table():
    torch.testing.assert_close(O.readout_table(torch.eye(R)[None].double()), O.basis(128)[None])
    rng = np.random.default_rng(1)
    Rm = rng.standard_normal((2, R, R))
    got = O.readout_table(torch.from_numpy(Rm)).numpy()
    np.testing.assert_allclose(got, Rm @ O.basis(128).numpy(), atol=1e-12)


@pytest.mark.parametrize("mode,tol", [("exact", 1e-9), ("mirror", 5e-5)])
def test_clock_phase_against_float64(mode, tol):
    rng = np.random.default_rng(2)
    lam32 = np.concatenate([
        rng.uniform(0, 3, 200), rng.uniform(0, 1e4, 300), rng.uniform(1e4, 1e5, 300),
        rng.uniform(-50, 0, 100), np.arange(0, 400, dtype=np.float64),
    ]).astype(np.float32)
    lam = torch.from_numpy(lam32)
    theta = O.clock_phase(lam if mode == "mirror" else lam.double(), mode).double().numpy()
    p = np.arange(64)
    ref = 2 * np.pi * p[None, :] * lam32.astype(np.float64)[:, None] / R
    np.testing.assert_allclose(np.cos(theta), np.cos(ref), atol=tol)
    np.testing.assert_allclose(np.sin(theta), np.sin(ref), atol=tol)
    coord = theta * R / (2 * np.pi)
    assert coord.max() <= R / 2 + 1e-3 and coord.min() > -R / 2 - 1e-3


def test_rotation_inverse_and_matrix():
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(5, 128, dtype=torch.float64, generator=gen)
    lam = torch.rand(5, dtype=torch.float64, generator=gen) * 300
    c, s = O.phase_cos_sin(lam)
    y = O.rotate(x, c, s)
    torch.testing.assert_close(O.rotate(y, c, s, negative=True), x, atol=1e-12, rtol=0)
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1), atol=1e-12, rtol=0)
    th = O.clock_phase(lam)
    for i in range(5):
        for p in (0, 1, 17, 63):
            rot = torch.tensor([[math.cos(th[i, p]), -math.sin(th[i, p])], [math.sin(th[i, p]), math.cos(th[i, p])]],
                               dtype=torch.float64)
            torch.testing.assert_close(y[i, 2 * p:2 * p + 2], rot @ x[i, 2 * p:2 * p + 2], atol=1e-12, rtol=0)


def test_write_vector_closed_form():
    beta = torch.tensor([0.3, 1.0], dtype=torch.float64)
    w0 = O.write_vector(torch.zeros(2, dtype=torch.float64), beta)
    phi = O.basis(128)
    torch.testing.assert_close(w0, beta[:, None] * phi[0][None, :], atol=1e-14, rtol=0)
    lam = torch.tensor([0.0, 0.37, 12.5, 999.9, 16384.25], dtype=torch.float64)
    w = O.write_vector(lam, torch.full_like(lam, 0.7))
    torch.testing.assert_close(w.norm(dim=-1), torch.full_like(lam, 0.7), atol=1e-12, rtol=0)
    c, s = O.phase_cos_sin(lam)
    b = phi[0].expand(5, 128)
    torch.testing.assert_close(w, 0.7 * O.rotate(b, c, s, negative=True), atol=1e-12, rtol=0)


@pytest.mark.parametrize("d", [0, 1, 2, 5, 63, 64, 126, 127, 300])
def test_integer_clock_is_cyclic_roll(d):
    phi = O.basis(128)
    P = phi @ U_matrix(d) @ phi.T
    expect = torch.from_numpy(np.roll(np.eye(R), d, axis=0))
    torch.testing.assert_close(P, expect, atol=1e-11, rtol=0)
    torch.testing.assert_close(shift_matrix(d), expect, atol=1e-11, rtol=0)


@pytest.mark.parametrize("d", [0.25, 0.5, 0.913, 3.7, 77.01])
def test_fractional_clock_matches_shift_kernel(d):
    phi = O.basis(128)
    torch.testing.assert_close(phi @ U_matrix(d) @ phi.T, shift_matrix(d), atol=1e-11, rtol=0)


def test_head_rmsnorm_matches_torch():
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(3, 7, 2, 256, dtype=torch.float64, generator=gen)
    w = torch.rand(256, dtype=torch.float64, generator=gen) + 0.5
    ref = torch.nn.functional.rms_norm(x, (256,), w, eps=1e-6)
    torch.testing.assert_close(O.head_rmsnorm(x, w, 1e-6), ref, atol=1e-12, rtol=0)
    # Mirror mode is the same normalisation followed by one bf16 rounding.
    xb = x.float().bfloat16().float()
    mirror = O.head_rmsnorm(xb, w.float(), 1e-6, "mirror")
    ref_b = torch.nn.functional.rms_norm(xb.double(), (256,), w, eps=1e-6)
    assert torch.equal(mirror, mirror.bfloat16().float())
    torch.testing.assert_close(mirror.double(), ref_b, atol=0, rtol=2**-8)


def test_slot_readout_identity_at_zero_clock():
    gen = torch.Generator().manual_seed(5)
    raw = torch.randn(1, 1, 4, 128, dtype=torch.float64, generator=gen)
    phi = O.basis(128)
    weights = O.slot_readout(raw, torch.zeros(1, 1, 4, dtype=torch.float64), phi[None])
    p = torch.softmax(raw @ phi.T, dim=-1)
    torch.testing.assert_close(weights, p @ phi, atol=1e-14, rtol=0)


def test_coherent_inputs_drive_the_readout_past_fp16():
    """The GPU range test's inputs (tests/coherent_inputs.py) really push the
    readout input z beyond the fp16 range: unscaled fp16 z would be infinite
    for most tokens and the softmax would return NaN, while the reference's
    own bf16 rounding of z and the table stays finite and close to exact."""
    from coherent_inputs import coherent_inputs, pass1_output

    x = coherent_inputs(T=16384)
    raw, z = pass1_output(x)
    over = (z.abs().amax(-1) > 65504).double().mean().item()
    assert over > 0.5, over
    table = O.readout_table(x["readout"].double())
    logits = torch.einsum("bhtm,hrm->bhtr", z.to(torch.float16).double(), table)
    assert torch.isnan(torch.softmax(logits, -1)).any()
    logits_bf16 = torch.einsum("bhtm,hrm->bhtr", z.to(torch.bfloat16).double(), table)
    assert torch.isfinite(torch.softmax(logits_bf16, -1)).all()


# The general-shape path runs the same oracle functions at other slot counts;
# these pin them there by the same mathematics.
GENERAL_M = [16, 64, 96, 256]


@pytest.mark.parametrize("M", GENERAL_M)
def test_basis_orthonormal_and_fft_any_slot_count(M):
    Rg = M - 1
    phi = O.basis(M)
    assert phi.shape == (Rg, M) and torch.all(phi[:, 1] == 0)
    torch.testing.assert_close(phi @ phi.T, torch.eye(Rg, dtype=torch.float64), atol=1e-12, rtol=0)
    x = np.random.default_rng(M).standard_normal(Rg)
    X = np.fft.fft(x)
    sp = np.where(np.arange(M // 2) == 0, math.sqrt(1 / Rg), math.sqrt(2 / Rg))
    expect = np.stack([sp * X[:M // 2].real, -sp * X[:M // 2].imag], axis=-1).reshape(M)
    expect[1] = 0.0
    np.testing.assert_allclose((phi.T @ torch.from_numpy(x)).numpy(), expect, atol=1e-12)


def _u_matrix(d, M):
    eye = torch.eye(M, dtype=torch.float64)
    c, s = O.phase_cos_sin(torch.tensor([float(d)], dtype=torch.float64), M=M)
    return O.rotate(eye, c.expand(M, M // 2), s.expand(M, M // 2)).T


@pytest.mark.parametrize("M", GENERAL_M)
@pytest.mark.parametrize("d", [1, 3, 200])
def test_integer_clock_is_cyclic_roll_any_slot_count(M, d):
    """U(d) for an integer clock moves slot r to slot r + d (mod R): the
    phase's integer range reduction at this R."""
    phi = O.basis(M)
    expect = torch.from_numpy(np.roll(np.eye(M - 1), d, axis=0))
    torch.testing.assert_close(phi @ _u_matrix(d, M) @ phi.T, expect, atol=1e-11, rtol=0)


@pytest.mark.parametrize("M", GENERAL_M)
def test_write_vector_and_readout_any_slot_count(M):
    phi = O.basis(M)
    beta = torch.tensor([0.3, 1.0], dtype=torch.float64)
    w0 = O.write_vector(torch.zeros(2, dtype=torch.float64), beta, M=M)
    torch.testing.assert_close(w0, beta[:, None] * phi[0][None, :], atol=1e-14, rtol=0)
    lam = torch.tensor([0.37, 12.5, 999.9], dtype=torch.float64)
    w = O.write_vector(lam, torch.full_like(lam, 0.7), M=M)
    c, s = O.phase_cos_sin(lam, M=M)
    torch.testing.assert_close(w, 0.7 * O.rotate(phi[0].expand(3, M), c, s, negative=True), atol=1e-12, rtol=0)
    # at a zero clock the readout is softmax(raw Phi^T) Phi
    raw = torch.randn(1, 1, 3, M, dtype=torch.float64, generator=torch.Generator().manual_seed(M))
    weights = O.slot_readout(raw, torch.zeros(1, 1, 3, dtype=torch.float64), phi[None])
    torch.testing.assert_close(weights, torch.softmax(raw @ phi.T, dim=-1) @ phi, atol=1e-14, rtol=0)
