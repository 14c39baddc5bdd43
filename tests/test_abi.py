"""The C-ABI library loads, exports every symbol include/cyfa_abi.h declares,
and its ctypes mirror has the C struct layout. No GPU compute is issued: only
host-side entry points (version, workspace size, argument validation that
fails before any HIP call) are called."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest
import torch

from cyclic_flow_attention import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cyfa_abi.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:const\s+)?\w+\s*\*?\s*(cyfa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _native.load_library()
    names = declared_functions()
    assert set(names) == set(_native.SIGNATURES), names
    for name in names:
        assert hasattr(lib, name), name
    assert lib.cyfa_abi_version() == _native.ABI_VERSION


def _c_layout(tmp_path, struct, fields):
    src = tmp_path / "layout.c"
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "cyfa_abi.h"', "int main(void) {",
             f'printf("%zu\\n", sizeof({struct}));']
    lines += [f'printf("%zu\\n", offsetof({struct}, {f}));' for f in fields]
    lines += ["return 0; }"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    return [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]


@pytest.mark.parametrize("cls,name", [(_native.CyfaChunkArgs, "CyfaChunkArgs"),
                                      (_native.CyfaDecodeArgs, "CyfaDecodeArgs"),
                                      (_native.CyfaOutNormArgs, "CyfaOutNormArgs"),
                                      (_native.CyfaSlaArgs, "CyfaSlaArgs"),
                                      (_native.CyfaDecodeLayerArgs, "CyfaDecodeLayerArgs"),
                                      (_native.CyfaNormArgs, "CyfaNormArgs"),
                                      (_native.CyfaConvArgs, "CyfaConvArgs"),
                                      (_native.CyfaLinearArgs, "CyfaLinearArgs"),
                                      (_native.CyfaRowNormArgs, "CyfaRowNormArgs"),
                                      (_native.CyfaChunkBwdArgs, "CyfaChunkBwdArgs")])
def test_struct_layout_matches_header(tmp_path, cls, name):
    fields = [f for f, _ in cls._fields_]
    got = [ctypes.sizeof(cls)] + [getattr(cls, f).offset for f in fields]
    assert got == _c_layout(tmp_path, name, fields)


def test_workspace_size_is_host_side():
    n = _native.chunk_workspace_bytes(8, 2048, 4, 256, 256)
    # clock [B*H*T] f32 + segment states + slot weights [B*H*T*128] bf16, at least
    assert n >= 8 * 4 * 2048 * (4 + 256)
    assert _native.chunk_workspace_bytes(1, 1, 1, 256, 256) > 0


def test_unsupported_shapes_fail_before_launch():
    lib = _native.load_library()
    args = _native.CyfaChunkArgs(B=1, T=64, H=1, K=256, V=256, M=64, C=64)
    assert lib.cyfa_chunk_fwd(ctypes.byref(args), None) == _native.CYFA_ERR_UNSUPPORTED
    assert b"num_slots" in lib.cyfa_last_error()
    args.M, args.C = 128, 32
    assert lib.cyfa_chunk_fwd(ctypes.byref(args), None) == _native.CYFA_ERR_UNSUPPORTED
    args.C = 64
    assert lib.cyfa_chunk_fwd(ctypes.byref(args), None) == _native.CYFA_ERR_VALUE  # null pointers
    dargs = _native.CyfaDecodeArgs(B=1, H=1, K=512, V=256, M=128)
    assert lib.cyfa_decode_step(ctypes.byref(dargs), None) == _native.CYFA_ERR_UNSUPPORTED
    assert lib.cyfa_readout_table(None, None, 1, 63, None) == _native.CYFA_ERR_UNSUPPORTED  # odd slot count
    assert lib.cyfa_readout_table(None, None, 1, 258, None) == _native.CYFA_ERR_UNSUPPORTED
    assert lib.cyfa_readout_table(None, None, 1, 64, None) == _native.CYFA_ERR_VALUE  # the general table's M


def test_general_path_checks_fail_before_launch():
    """cyfa_chunk_fwd_general / cyfa_decode_step_general refuse what the
    general kernels do not take, and a short workspace, before any launch."""
    lib = _native.load_library()
    bf, f32 = _native.CYFA_DTYPE_BF16, _native.CYFA_DTYPE_F32
    dummy = 256  # a nonzero pointer value; nothing is dereferenced before the checks fail
    args = _native.CyfaChunkArgs(B=1, T=100, H=2, K=128, V=64, M=64, C=32, scale=0.1)
    for name in ("q", "k", "v", "g", "delta", "beta", "table", "q_norm_weight", "k_norm_weight", "o"):
        setattr(args, name, dummy)
    need = lib.cyfa_chunk_general_workspace_bytes(1, 100, 2, 128, 64, 64, 32)
    Tp = 128  # 100 tokens padded to chunks of 32
    assert need >= 2 * 128 * (8 + 4 * (2 * 128 + 64 + 4 * 64))
    assert lib.cyfa_chunk_general_workspace_bytes(0, 100, 2, 128, 64, 64, 32) == 0
    assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), bf, None) == _native.CYFA_ERR_WORKSPACE
    args.workspace, args.workspace_bytes = 4096, need - 1
    assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), bf, None) == _native.CYFA_ERR_WORKSPACE
    assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), 7, None) == _native.CYFA_ERR_VALUE
    for field, bad in (("M", 63), ("M", 258), ("K", 2048), ("V", 0), ("C", 48)):
        old = getattr(args, field)
        setattr(args, field, bad)
        assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), f32, None) == _native.CYFA_ERR_UNSUPPORTED, field
        setattr(args, field, old)
    args.o = None
    assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), bf, None) == _native.CYFA_ERR_VALUE
    args.o, args.hk = dummy, dummy  # final states all or none
    assert lib.cyfa_chunk_fwd_general(ctypes.byref(args), bf, None) == _native.CYFA_ERR_VALUE
    assert Tp % args.C == 0
    dargs = _native.CyfaDecodeArgs(B=1, H=1, K=2048, V=64, M=64)
    assert lib.cyfa_decode_step_general(ctypes.byref(dargs), bf, None) == _native.CYFA_ERR_UNSUPPORTED
    dargs.K = 512
    assert lib.cyfa_decode_step_general(ctypes.byref(dargs), bf, None) == _native.CYFA_ERR_VALUE  # null pointers


def test_backward_checks_fail_before_launch():
    """cyfa_chunk_bwd refuses what its kernels do not take, missing outputs and
    a short workspace, before any launch."""
    lib = _native.load_library()
    bf = _native.CYFA_DTYPE_BF16
    dummy = 256  # a nonzero pointer value; nothing is dereferenced before the checks fail
    args = _native.CyfaChunkArgs(B=2, T=100, H=2, K=256, V=256, M=128, C=64, scale=0.0625)
    for name in ("q", "k", "v", "g", "delta", "beta", "table", "q_norm_weight", "k_norm_weight"):
        setattr(args, name, dummy)
    grads = _native.CyfaChunkBwdArgs()
    for name in ("dq", "dk", "dv", "dg", "ddelta", "dbeta", "dtable", "dq_norm_weight", "dk_norm_weight"):
        setattr(grads, name, dummy)
    need = lib.cyfa_chunk_bwd_workspace_bytes(2, 100, 2, 256, 256, 128)
    rows, chunks = 2 * 2 * 128, 2
    # at least the saved states of both passes and their cotangents
    assert need >= 4 * 4 * (2 * 2 * (chunks + 1) * 256 * 128) + 4 * rows * (2 * 256 + 256)
    assert lib.cyfa_chunk_bwd_workspace_bytes(0, 100, 2, 256, 256, 128) == 0
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_WORKSPACE
    grads.workspace, grads.workspace_bytes = 4096, need - 1
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_WORKSPACE
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), 7, ctypes.byref(grads), None) == _native.CYFA_ERR_VALUE
    for field, bad in (("M", 258), ("M", 63), ("K", 2048), ("V", 0)):
        old = getattr(args, field)
        setattr(args, field, bad)
        assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_UNSUPPORTED
        setattr(args, field, old)
    grads.dtable = None
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_VALUE
    grads.dtable, grads.dh0_k = dummy, dummy  # initial-state gradients all or none
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_VALUE
    grads.dh0_k = None
    args.scale = 0.0
    assert lib.cyfa_chunk_bwd(ctypes.byref(args), bf, ctypes.byref(grads), None) == _native.CYFA_ERR_VALUE


def test_python_backward_refusals():
    """What the backward does not cover is refused when the graph is built."""
    from cyclic_flow_attention.ops import chunk_cyfa

    q = torch.zeros(1, 2, 1, 256, dtype=torch.bfloat16, requires_grad=True)
    g = torch.zeros(1, 2, 1)
    w = torch.ones(256)
    with pytest.raises(NotImplementedError):  # 258 slots: beyond the backward's 256
        chunk_cyfa(q, q, q, g, g, g, torch.eye(257)[None], w, w)
    ro = torch.eye(127)[None]
    with pytest.raises(NotImplementedError):  # a precomputed table is inference-only
        chunk_cyfa(q, q, q, g, g, g, ro, w, w, table=torch.zeros(1, 127, 128))
    with pytest.raises(ValueError):  # CPU tensors: the HIP path has no CPU fallback, with or without grad
        chunk_cyfa(q, q, q, g, g, g, ro, w, w)


def test_python_ops_reject_like_the_reference():
    from cyclic_flow_attention.ops import chunk_cyfa, fused_recurrent_cyfa

    q = torch.zeros(1, 2, 1, 256, dtype=torch.bfloat16)
    g = torch.zeros(1, 2, 1)
    ro = torch.eye(127)[None]
    w = torch.ones(256)
    with pytest.raises(NotImplementedError):
        chunk_cyfa(q, q, q, g, g, g, ro, w, w, cu_seqlens=torch.tensor([0, 2]))
    with pytest.raises(NotImplementedError):
        chunk_cyfa(q, q, q, g, g, g, ro, w, w, checkpoint_level=1)
    with pytest.raises(NotImplementedError):
        fused_recurrent_cyfa(q, q, q, g, g, g, ro, w, w)  # T != 1
    q1 = q[:, :1].clone().requires_grad_(False)
    g1 = g[:, :1]
    with pytest.raises(ValueError):
        fused_recurrent_cyfa(q1, q1, q1, g1.clone().requires_grad_(True), g1, g1, ro, w, w)
    with pytest.raises(ValueError):
        chunk_cyfa(q, q, q, g, g, g, ro, w, w)  # CPU tensors: the HIP path has no CPU fallback


def test_layer_entry_points_validate_before_launch():
    lib = _native.load_library()
    n = _native.CyfaNormArgs(rows=4, D=384)
    assert lib.cyfa_rms_norm(ctypes.byref(n), None) == _native.CYFA_ERR_UNSUPPORTED
    n.D = 256
    assert lib.cyfa_rms_norm(ctypes.byref(n), None) == _native.CYFA_ERR_VALUE  # null pointers
    c = _native.CyfaConvArgs(B=1, T=4, D=64, W=5, split=64)
    assert lib.cyfa_short_conv(ctypes.byref(c), None) == _native.CYFA_ERR_UNSUPPORTED
    c.W, c.split = 4, 12
    assert lib.cyfa_short_conv(ctypes.byref(c), None) == _native.CYFA_ERR_UNSUPPORTED
    assert lib.cyfa_silu_mul(None, None, 1, 8, None) == _native.CYFA_ERR_VALUE
    assert lib.cyfa_argmax_rows(None, 8, 1, 8, None, None) == _native.CYFA_ERR_VALUE
    assert lib.cyfa_argmax_rows(0x10000, 100, 1, 100, 0x20000, None) == _native.CYFA_ERR_VALUE  # ldx % 8
    assert lib.cyfa_argmax_rows(0x10002, 104, 1, 100, 0x20000, None) == _native.CYFA_ERR_ALIGN
    assert lib.cyfa_gates(None, 12, None, None, None, None, None, 1, 4, None) == _native.CYFA_ERR_VALUE
    # the fused pre-norm: checked before anything is launched (the pointers are never dereferenced)
    a = _native.CyfaLinearArgs(M=4, N=64, K=4096, x=0x10000, ldx=4096, weight=0x20000, y=0x30000, ldy=64)
    nrm = _native.CyfaRowNormArgs(weight=0x40000, eps=1e-6)
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), ctypes.byref(nrm), None) == _native.CYFA_ERR_UNSUPPORTED
    a.K = a.ldx = 1024
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), None, None) == _native.CYFA_ERR_VALUE
    nrm.residual, nrm.ldr = 0x50000, 1024
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), ctypes.byref(nrm), None) == _native.CYFA_ERR_VALUE  # no sum_out
    nrm.sum_out, nrm.ldr = 0x60000, 1000
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), ctypes.byref(nrm), None) == _native.CYFA_ERR_VALUE  # ldr
    nrm.ldr, nrm.weight = 1024, 0x40004
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), ctypes.byref(nrm), None) == _native.CYFA_ERR_ALIGN


def test_scalar_la_validates_before_launch():
    from cyclic_flow_attention.ops.chunk import scalar_la

    lib = _native.load_library()
    a = _native.CyfaSlaArgs(B=1, T=64, H=1, K=256, V=256)
    assert lib.cyfa_scalar_la(ctypes.byref(a), None) == _native.CYFA_ERR_UNSUPPORTED
    a.V, a.T = 128, 100
    assert lib.cyfa_scalar_la(ctypes.byref(a), None) == _native.CYFA_ERR_VALUE  # T not a multiple of 64
    a.T = 128
    assert lib.cyfa_scalar_la(ctypes.byref(a), None) == _native.CYFA_ERR_VALUE  # null pointers
    assert _native.scalar_la_workspace_bytes(8, 4096, 4, 256, 128) > 0
    q = torch.zeros(1, 1, 64, 128, dtype=torch.bfloat16)
    g = torch.zeros(1, 1, 64)
    with pytest.raises(ValueError):
        scalar_la(q, q, torch.zeros(1, 1, 64, 256, dtype=torch.bfloat16), g, None)  # CPU tensors
    with pytest.raises(ValueError):
        scalar_la(q, q, torch.zeros(1, 1, 32, 256, dtype=torch.bfloat16), g, None)  # v shape
    with pytest.raises(NotImplementedError):
        scalar_la(q, q, torch.zeros(1, 1, 64, 256), g, None)  # fp32 v


def test_sequence_spans_beyond_32_bit_offsets_are_refused():
    """The kernels address one sequence's rows with 32-bit byte offsets, so
    calls whose per-sequence span reaches 2^32 bytes return
    CYFA_ERR_UNSUPPORTED before anything is launched (the pointers are never
    dereferenced)."""
    lib = _native.load_library()
    ptrs = dict(q=0x10000, k=0x20000, v=0x30000, g=0x40000, delta=0x50000, beta=0x60000, table=0x70000,
                q_norm_weight=0x80000, k_norm_weight=0x90000, o=0xa0000)
    # T * H * 512 = 2^32 exactly: one byte past the largest offset
    args = _native.CyfaChunkArgs(B=1, T=1 << 21, H=4, K=256, V=256, M=128, C=64, scale=0.0625, **ptrs)
    assert lib.cyfa_chunk_fwd(ctypes.byref(args), None) == _native.CYFA_ERR_UNSUPPORTED
    assert b"2^32" in lib.cyfa_last_error()
    args.T = (1 << 21) - 1  # below the limit: passes the span check, then fails on the missing workspace
    assert lib.cyfa_chunk_fwd(ctypes.byref(args), None) == _native.CYFA_ERR_WORKSPACE
    s = _native.CyfaSlaArgs(B=1, T=1 << 16, H=128, K=128, V=256, q=0x10000, k=0x20000, v=0x30000, g=0x40000,
                            o=0x50000, scale=1.0, v_bth=1)
    assert lib.cyfa_scalar_la(ctypes.byref(s), None) == _native.CYFA_ERR_UNSUPPORTED  # v rows span 2^32 bytes
    s.v_bth = 0
    assert lib.cyfa_scalar_la(ctypes.byref(s), None) == _native.CYFA_ERR_WORKSPACE
    s.output_bth, s.raw_output = 1, 1
    assert lib.cyfa_scalar_la(ctypes.byref(s), None) == _native.CYFA_ERR_UNSUPPORTED  # f32 o rows: 2^33 bytes


def test_decode_wrappers_check_every_tensor_before_launch():
    """Every tensor argument of the decode wrappers is checked for its device
    before any launch (CPU tensors raise ValueError), and a precomputed table
    must be float32 [H, M-1, M]."""
    from cyclic_flow_attention.ops import fused_recurrent_cyfa
    from cyclic_flow_attention.ops.utils import check_table

    q = torch.zeros(1, 1, 1, 256, dtype=torch.bfloat16)
    g = torch.zeros(1, 1, 1)
    ro = torch.eye(127)[None]
    w = torch.ones(256)
    state = (torch.zeros(1, 1, 256, 128), torch.zeros(1, 1, 128, 256), torch.zeros(1, 1))
    with pytest.raises(ValueError):
        fused_recurrent_cyfa(q, q, q, g, g, g, ro, w, w, initial_state=state)
    with pytest.raises(ValueError):
        check_table(torch.zeros(1, 127, 128, dtype=torch.bfloat16), 1, 128)
    with pytest.raises(ValueError):
        check_table(torch.zeros(2, 127, 128), 1, 128)
    check_table(torch.zeros(1, 127, 128), 1, 128)


def test_noalloc_entry_point_refuses_oversize_before_launch():
    """cyfa_chunk_fwd_noalloc checks its workspace against the scratch array
    before touching the device: B=64, T=2048, H=4 needs 132 MiB (> 80 MiB)."""
    lib = _native.load_library()
    ptrs = dict(q=0x10000, k=0x20000, v=0x30000, g=0x40000, delta=0x50000, beta=0x60000, table=0x70000,
                q_norm_weight=0x80000, k_norm_weight=0x90000, o=0xa0000)
    args = _native.CyfaChunkArgs(B=64, T=2048, H=4, K=256, V=256, M=128, C=64, scale=0.0625, **ptrs)
    assert _native.chunk_workspace_bytes(64, 2048, 4, 256, 256) > _native.NOALLOC_SCRATCH_BYTES
    assert lib.cyfa_chunk_fwd_noalloc(ctypes.byref(args), None, None) == _native.CYFA_ERR_UNSUPPORTED
    assert b"scratch" in lib.cyfa_last_error()
    assert _native.chunk_workspace_bytes(8, 2048, 4, 256, 256) <= _native.NOALLOC_SCRATCH_BYTES
    assert _native.chunk_workspace_bytes(1, 16384, 8, 256, 256) <= _native.NOALLOC_SCRATCH_BYTES


def test_decode_workspace_query():
    """The small-batch decode split needs B H x 8 slices x 128 floats of
    workspace below B H = 64 and none from there on (host-side query)."""
    lib = _native.load_library()
    assert lib.cyfa_decode_workspace_bytes(1, 8, 256, 256) == 8 * 8 * 128 * 4
    assert lib.cyfa_decode_workspace_bytes(15, 4, 256, 256) == 60 * 8 * 128 * 4
    assert lib.cyfa_decode_workspace_bytes(16, 4, 256, 256) == 0
    assert lib.cyfa_decode_workspace_bytes(2, 2, 128, 128) == 4 * 4 * 128 * 4
    assert lib.cyfa_decode_workspace_bytes(1, 1, 512, 256) == 0  # no kernel for K = 512


def test_decode_layer_prefetch_ranges_validated_before_launch():
    """cyfa_decode_layer_step checks its cache-prefetch ranges before any launch:
    a range with bytes needs a pointer, 16-byte alignment and fewer than 2^31
    bytes (the pointers are never dereferenced here)."""
    lib = _native.load_library()
    H = 8
    a = _native.CyfaDecodeArgs(B=1, H=H, K=256, V=256, M=128, table=0x10000, q_norm_weight=0x20000,
                               k_norm_weight=0x30000, scale=0.0625, o=0x40000, hk_out=0x50000, hv_out=0x60000,
                               clock_out=0x70000)
    ly = _native.CyfaDecodeLayerArgs(qkv=0x80000, qkv_row=3 * H * 256, conv_cache_out=0x90000,
                                     cache_row=3 * H * 256, cache_batch=9 * H * 256, conv_weight=0xa0000,
                                     abd=0xb0000, abd_row=3 * H, dt_bias=0xc0000, A_log=0xd0000, gate=0xe0000,
                                     gate_row=H * 256, norm_weight=0xf0000, norm_eps=1e-6, norm_prescale=127.0)
    ly.prefetch_bytes[1] = 4096  # bytes without a pointer
    assert lib.cyfa_decode_layer_step(ctypes.byref(a), ctypes.byref(ly), None) == _native.CYFA_ERR_VALUE
    assert b"prefetch range 1" in lib.cyfa_last_error()
    ly.prefetch[1] = 0x100008  # misaligned
    assert lib.cyfa_decode_layer_step(ctypes.byref(a), ctypes.byref(ly), None) == _native.CYFA_ERR_ALIGN
    ly.prefetch[1], ly.prefetch_bytes[1] = 0x100000, 1 << 31  # too large for the kernel's 32-bit offsets
    assert lib.cyfa_decode_layer_step(ctypes.byref(a), ctypes.byref(ly), None) == _native.CYFA_ERR_VALUE
    ly.prefetch_bytes[1], ly.prefetch_span[1] = 4096, 24  # a span must be a multiple of 16
    assert lib.cyfa_decode_layer_step(ctypes.byref(a), ctypes.byref(ly), None) == _native.CYFA_ERR_VALUE
    assert b"span" in lib.cyfa_last_error()


def test_linear_rows_prefetch_ranges_validated_before_launch():
    """cyfa_linear_rows checks its cache-prefetch ranges before any launch, as
    cyfa_decode_layer_step does (the pointers are never dereferenced here)."""
    lib = _native.load_library()
    a = _native.CyfaLinearArgs(M=64, N=1024, K=1024, x=0x10000, ldx=1024, weight=0x20000, y=0x30000, ldy=1024)
    a.prefetch_bytes[1] = 4096  # bytes without a pointer
    assert lib.cyfa_linear_rows(ctypes.byref(a), None) == _native.CYFA_ERR_VALUE
    assert b"prefetch range 1" in lib.cyfa_last_error()
    a.prefetch[1] = 0x100008  # misaligned
    assert lib.cyfa_linear_rows(ctypes.byref(a), None) == _native.CYFA_ERR_ALIGN
    a.prefetch[1], a.prefetch_bytes[1] = 0x100000, 1 << 31  # too large for the kernel's 32-bit offsets
    assert lib.cyfa_linear_rows(ctypes.byref(a), None) == _native.CYFA_ERR_VALUE
    a.prefetch_bytes[1], a.prefetch_span[1] = 4096, 24  # a span must be a multiple of 16
    n = _native.CyfaRowNormArgs(weight=0x40000, eps=1e-6)
    assert lib.cyfa_norm_linear_rows(ctypes.byref(a), ctypes.byref(n), None) == _native.CYFA_ERR_VALUE
    assert b"span" in lib.cyfa_last_error()


def test_linear_rows_span_query():
    """cyfa_linear_rows_span, the bytes of W each workgroup of a projection
    launch reads when the workgroups that read the bytes [c span, (c + 1)
    span) all run on XCD c mod 8: the one-row kernel's waves take RW rows
    each (four waves per workgroup, RW the most of 4, 2, 1 that keeps 256 or
    more workgroups), the tile kernel's N tile x the rows 16 CT x .. (with
    several row tiles the launcher pads the N tiles to a multiple of 8, so
    that every row tile of N tile x runs on the same XCD); 0 where one
    workgroup reads its rows in pieces (SwiGLU's interleaved gate and up rows
    in the one-row kernel) or the launchers refuse the shape."""
    span = _native.linear_rows_span
    assert span(1, 2048, 2048) == 4 * 2 * 2048 * 2     # o_proj of the 1.4B step: RW 2, 256 workgroups
    assert span(1, 2048, 5632) == 4 * 2 * 5632 * 2     # down
    assert span(1, 6424, 2048, norm=1) == 4 * 4 * 2048 * 2  # the input projection: RW 4, 402 workgroups
    assert span(1, 1024, 1024) == 4 * 1 * 1024 * 2     # RW 1: 256 workgroups of 4 rows
    assert span(1, 11264, 2048, swiglu=True, norm=1) == 0
    assert span(1, 2048, 2048, norm=2) != 4 * 2 * 2048 * 2  # the folded norm stays on the tile kernel
    g1 = span(1, 2048, 256)                             # K = 256: the tile kernel, one row tile
    assert g1 > 0 and g1 % (16 * 256 * 2) == 0
    assert span(64, 1024, 1024) == 16 * 1 * 1024 * 2    # 1 x 1 tiles: four row tiles read each W tile
    assert span(64, 3340, 1024, norm=1) == 16 * 2 * 1024 * 2  # 2 x 2 tiles, 105 N tiles padded to 112
    assert span(64, 5632, 1024, swiglu=True, norm=1) == 16 * 2 * 1024 * 2  # 4 x 2 tiles
    assert span(64, 32000, 1024) == 16 * 4 * 1024 * 2   # the lm_head's 4 x 4 tiles
    for bad in ((0, 64, 64), (65, 64, 64), (1, 64, 48), (1, 0, 64)):
        assert span(*bad) == 0
    assert span(1, 64, 4096, norm=1) == 0 and span(1, 48, 64, swiglu=True) == 0
    assert _native.load_library().cyfa_linear_rows_span(1, 2048, 2048, 0, 3) == 0
