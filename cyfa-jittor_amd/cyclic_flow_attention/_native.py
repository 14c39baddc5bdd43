"""ctypes binding of libcyfa_hip.so (C ABI declared in include/cyfa_abi.h).

PyTorch-ROCm tensors are the only device container: callers pass tensors,
this module passes their data pointers and the current HIP stream to the
library. There is no fallback: if the library is missing, or no GPU is
visible, every entry point raises.
"""

import ctypes
import os
from pathlib import Path

import torch
import torch.nn.functional as F

LIB_PATH = Path(os.environ.get("CYFA_LIB", Path(__file__).with_name("libcyfa_hip.so")))
ABI_VERSION = 11

CYFA_OK = 0
CYFA_ERR_VALUE = -1
CYFA_ERR_UNSUPPORTED = -2
CYFA_ERR_ALIGN = -3
CYFA_ERR_WORKSPACE = -4
CYFA_ERR_LAUNCH = -5

_c_int, _c_float, _c_void_p, _c_size_t = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# cyfa_decode_layer_step's cache-prefetch ranges, and the largest B H with
# which the kernel prefetches them (CYFA_PREFETCH_RANGES, CYFA_PREFETCH_MAX_BH)
PREFETCH_RANGES = 4
# cyfa_linear_rows' cache-prefetch ranges (CYFA_LINEAR_PREFETCH_RANGES)
LINEAR_PREFETCH_RANGES = 2
PREFETCH_MAX_BH = 64


class CyfaChunkArgs(ctypes.Structure):
    _fields_ = [
        ("B", _c_int), ("T", _c_int), ("H", _c_int), ("K", _c_int), ("V", _c_int), ("M", _c_int), ("C", _c_int),
        ("q", _c_void_p), ("k", _c_void_p), ("v", _c_void_p),
        ("g", _c_void_p), ("delta", _c_void_p), ("beta", _c_void_p),
        ("table", _c_void_p), ("q_norm_weight", _c_void_p), ("k_norm_weight", _c_void_p),
        ("q_norm_eps", _c_float), ("k_norm_eps", _c_float), ("scale", _c_float),
        ("h0_k", _c_void_p), ("h0_v", _c_void_p), ("clock0", _c_void_p),
        ("o", _c_void_p), ("hk", _c_void_p), ("hv", _c_void_p), ("clock", _c_void_p),
        ("workspace", _c_void_p), ("workspace_bytes", _c_size_t),
    ]


class CyfaChunkBwdArgs(ctypes.Structure):
    _fields_ = [
        ("d_o", _c_void_p), ("d_hk", _c_void_p), ("d_hv", _c_void_p), ("d_clock", _c_void_p),
        ("dq", _c_void_p), ("dk", _c_void_p), ("dv", _c_void_p),
        ("dg", _c_void_p), ("ddelta", _c_void_p), ("dbeta", _c_void_p),
        ("dtable", _c_void_p), ("dreadout", _c_void_p),
        ("dq_norm_weight", _c_void_p), ("dk_norm_weight", _c_void_p),
        ("dh0_k", _c_void_p), ("dh0_v", _c_void_p), ("dclock0", _c_void_p),
        ("workspace", _c_void_p), ("workspace_bytes", _c_size_t),
    ]


class CyfaOutNormArgs(ctypes.Structure):
    _fields_ = [("weight", _c_void_p), ("gate", _c_void_p), ("eps", _c_float), ("prescale", _c_float)]


class CyfaSlaArgs(ctypes.Structure):
    _fields_ = [
        ("B", _c_int), ("T", _c_int), ("H", _c_int), ("K", _c_int), ("V", _c_int),
        ("q", _c_void_p), ("k", _c_void_p), ("v", _c_void_p), ("g", _c_void_p), ("initial", _c_void_p),
        ("scale", _c_float), ("raw_output", _c_int), ("output_bth", _c_int), ("v_bth", _c_int),
        ("o", _c_void_p), ("final_state", _c_void_p),
        ("workspace", _c_void_p), ("workspace_bytes", _c_size_t),
    ]


class CyfaDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("B", _c_int), ("H", _c_int), ("K", _c_int), ("V", _c_int), ("M", _c_int),
        ("q", _c_void_p), ("k", _c_void_p), ("v", _c_void_p),
        ("g", _c_void_p), ("delta", _c_void_p), ("beta", _c_void_p),
        ("table", _c_void_p), ("q_norm_weight", _c_void_p), ("k_norm_weight", _c_void_p),
        ("q_norm_eps", _c_float), ("k_norm_eps", _c_float), ("scale", _c_float),
        ("hk_in", _c_void_p), ("hv_in", _c_void_p), ("clock_in", _c_void_p),
        ("o", _c_void_p), ("hk_out", _c_void_p), ("hv_out", _c_void_p), ("clock_out", _c_void_p),
        ("workspace", _c_void_p), ("workspace_bytes", _c_size_t),
    ]


class CyfaDecodeLayerArgs(ctypes.Structure):
    _fields_ = [
        ("qkv", _c_void_p), ("qkv_row", ctypes.c_longlong),
        ("conv_cache", _c_void_p), ("conv_cache_out", _c_void_p),
        ("cache_row", ctypes.c_longlong), ("cache_batch", ctypes.c_longlong),
        ("conv_weight", _c_void_p), ("abd", _c_void_p), ("abd_row", ctypes.c_longlong),
        ("dt_bias", _c_void_p), ("A_log", _c_void_p), ("gate", _c_void_p), ("gate_row", ctypes.c_longlong),
        ("norm_weight", _c_void_p), ("norm_eps", _c_float), ("norm_prescale", _c_float),
        ("g0", _c_void_p), ("g0_row", ctypes.c_longlong), ("g_weight", _c_void_p), ("g_bias", _c_void_p),
        ("prefetch", _c_void_p * PREFETCH_RANGES), ("prefetch_bytes", ctypes.c_ulonglong * PREFETCH_RANGES),
        ("prefetch_span", ctypes.c_ulonglong * PREFETCH_RANGES),
    ]


class CyfaNormArgs(ctypes.Structure):
    _fields_ = [
        ("rows", _c_int), ("D", _c_int),
        ("x", _c_void_p), ("residual", _c_void_p), ("sum_out", _c_void_p),
        ("weight", _c_void_p), ("gate", _c_void_p),
        ("eps", _c_float), ("prescale", _c_float),
        ("out", _c_void_p),
    ]


class CyfaLinearArgs(ctypes.Structure):
    _fields_ = [
        ("M", _c_int), ("N", _c_int), ("K", _c_int),
        ("x", _c_void_p), ("ldx", ctypes.c_longlong), ("weight", _c_void_p), ("bias", _c_void_p),
        ("y", _c_void_p), ("ldy", ctypes.c_longlong), ("swiglu", _c_int),
        ("residual", _c_void_p), ("ldr", ctypes.c_longlong),
        ("prefetch", _c_void_p * LINEAR_PREFETCH_RANGES),
        ("prefetch_bytes", ctypes.c_ulonglong * LINEAR_PREFETCH_RANGES),
        ("prefetch_span", ctypes.c_ulonglong * LINEAR_PREFETCH_RANGES),
    ]


class CyfaRowNormArgs(ctypes.Structure):
    _fields_ = [
        ("weight", _c_void_p), ("eps", ctypes.c_float), ("residual", _c_void_p), ("sum_out", _c_void_p),
        ("ldr", ctypes.c_longlong),
    ]


class CyfaConvArgs(ctypes.Structure):
    _fields_ = [
        ("B", _c_int), ("T", _c_int), ("D", _c_int), ("W", _c_int),
        ("x", _c_void_p), ("x_row", ctypes.c_longlong),
        ("cache", _c_void_p), ("cache_row", ctypes.c_longlong), ("cache_batch", ctypes.c_longlong),
        ("weight", _c_void_p), ("bias", _c_void_p),
        ("out", _c_void_p * 3), ("split", _c_int),
        ("cache_out", _c_void_p), ("cache_out_row", ctypes.c_longlong), ("cache_out_batch", ctypes.c_longlong),
    ]


class CyfaGatePathArgs(ctypes.Structure):
    _fields_ = [
        ("M", _c_int), ("K", _c_int), ("H", _c_int), ("Dv", _c_int),
        ("x", _c_void_p), ("ldx", ctypes.c_longlong), ("w1", _c_void_p), ("abd_bias", _c_void_p),
        ("w2", _c_void_p), ("b2", _c_void_p), ("dt_bias", _c_void_p), ("A_log", _c_void_p),
        ("gate", _c_void_p), ("ldg", ctypes.c_longlong), ("g", _c_void_p), ("beta", _c_void_p), ("delta", _c_void_p),
    ]


# Every symbol include/cyfa_abi.h declares, with its ctypes signature.
SIGNATURES = {
    "cyfa_chunk_fwd": (_c_int, [ctypes.POINTER(CyfaChunkArgs), _c_void_p]),
    "cyfa_chunk_fwd_normed": (_c_int, [ctypes.POINTER(CyfaChunkArgs), ctypes.POINTER(CyfaOutNormArgs), _c_void_p]),
    "cyfa_chunk_fwd_noalloc": (_c_int, [ctypes.POINTER(CyfaChunkArgs), ctypes.POINTER(CyfaOutNormArgs), _c_void_p]),
    "cyfa_chunk_workspace_bytes": (_c_size_t, [_c_int] * 7),
    "cyfa_scalar_la": (_c_int, [ctypes.POINTER(CyfaSlaArgs), _c_void_p]),
    "cyfa_scalar_la_workspace_bytes": (_c_size_t, [_c_int] * 5),
    "cyfa_decode_step": (_c_int, [ctypes.POINTER(CyfaDecodeArgs), _c_void_p]),
    "cyfa_decode_workspace_bytes": (_c_size_t, [_c_int] * 4),
    "cyfa_decode_layer_step": (_c_int, [ctypes.POINTER(CyfaDecodeArgs), ctypes.POINTER(CyfaDecodeLayerArgs), _c_void_p]),
    "cyfa_readout_table": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "cyfa_rms_norm": (_c_int, [ctypes.POINTER(CyfaNormArgs), _c_void_p]),
    "cyfa_short_conv": (_c_int, [ctypes.POINTER(CyfaConvArgs), _c_void_p]),
    "cyfa_linear_rows": (_c_int, [ctypes.POINTER(CyfaLinearArgs), _c_void_p]),
    "cyfa_linear_rows_span": (_c_size_t, [_c_int] * 5),
    "cyfa_norm_linear_rows": (_c_int, [ctypes.POINTER(CyfaLinearArgs), ctypes.POINTER(CyfaRowNormArgs), _c_void_p]),
    "cyfa_silu_mul": (_c_int, [_c_void_p, _c_void_p, _c_int, _c_int, _c_void_p]),
    "cyfa_argmax_rows": (_c_int, [_c_void_p, ctypes.c_longlong, _c_int, _c_int, _c_void_p, _c_void_p]),
    "cyfa_gates": (_c_int, [_c_void_p, ctypes.c_longlong, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                            _c_int, _c_int, _c_void_p]),
    "cyfa_gate_path": (_c_int, [ctypes.POINTER(CyfaGatePathArgs), _c_void_p]),
    "cyfa_chunk_general_workspace_bytes": (_c_size_t, [_c_int] * 7),
    "cyfa_chunk_fwd_general": (_c_int, [ctypes.POINTER(CyfaChunkArgs), _c_int, _c_void_p]),
    "cyfa_decode_step_general": (_c_int, [ctypes.POINTER(CyfaDecodeArgs), _c_int, _c_void_p]),
    "cyfa_chunk_bwd_workspace_bytes": (_c_size_t, [_c_int] * 6),
    "cyfa_chunk_bwd": (_c_int, [ctypes.POINTER(CyfaChunkArgs), _c_int, ctypes.POINTER(CyfaChunkBwdArgs), _c_void_p]),
    "cyfa_last_error": (ctypes.c_char_p, []),
    "cyfa_abi_version": (_c_int, []),
}

_lib = None


def load_library(path=None):
    """Load and type the shared library (no GPU needed). Raises if missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"CyFA HIP library not found at {p}; build it with `python cyfa-jittor_amd/build_native.py`"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.cyfa_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{p} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    if path is None:
        _lib = lib
    return lib


def _raise(code, what):
    msg = load_library().cyfa_last_error().decode(errors="replace") or what
    if code == CYFA_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if code in (CYFA_ERR_VALUE, CYFA_ERR_ALIGN, CYFA_ERR_WORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t):
    """Device pointer of a tensor, or None (NULL) for None."""
    return None if t is None else t.data_ptr()


def stream_handle(device):
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors):
    """All tensors must live on one HIP device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("CyFA HIP ops need tensors on a GPU device (got %s)" % t.device)
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("CyFA HIP ops need all tensors on one device")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def chunk_workspace_bytes(B, T, H, K, V, M=128, C=64):
    return int(load_library().cyfa_chunk_workspace_bytes(B, T, H, K, V, M, C))


class LaunchTimer:
    """Records HIP events around every library launch while active.

    Events are recorded on the stream the kernels are enqueued on (torch's
    current stream), so ``results()`` gives per-call device durations without
    a host sync per call."""

    def __init__(self):
        self.records = []

    def __enter__(self):
        _TIMERS.append(self)
        return self

    def __exit__(self, *exc):
        _TIMERS.remove(self)

    def results(self):
        """{entry point: [milliseconds per call]} (synchronises the device)."""
        torch.cuda.synchronize()
        out = {}
        for name, start, end in self.records:
            out.setdefault(name, []).append(start.elapsed_time(end))
        return out


_TIMERS = []


def _timed(name, fn):
    if not _TIMERS:
        return fn()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    rc = fn()
    end.record()
    for t in _TIMERS:
        t.records.append((name, start, end))
    return rc


def chunk_fwd(args: CyfaChunkArgs, device):
    lib = load_library()
    rc = _timed("cyfa_chunk_fwd", lambda: lib.cyfa_chunk_fwd(ctypes.byref(args), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_chunk_fwd failed")


def chunk_fwd_normed(args: CyfaChunkArgs, norm: CyfaOutNormArgs, device):
    lib = load_library()
    rc = _timed("cyfa_chunk_fwd_normed",
                lambda: lib.cyfa_chunk_fwd_normed(ctypes.byref(args), ctypes.byref(norm), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_chunk_fwd_normed failed")


NOALLOC_SCRATCH_BYTES = 80 << 20  # CYFA_NOALLOC_SCRATCH_BYTES


def chunk_fwd_noalloc(args: CyfaChunkArgs, norm, device):
    """cyfa_chunk_fwd_noalloc: the op with the library's per-device scratch
    array as its workspace (norm: CyfaOutNormArgs or None)."""
    lib = load_library()
    ref = None if norm is None else ctypes.byref(norm)
    rc = _timed("cyfa_chunk_fwd_noalloc", lambda: lib.cyfa_chunk_fwd_noalloc(ctypes.byref(args), ref,
                                                                              stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_chunk_fwd_noalloc failed")


def scalar_la_workspace_bytes(B, T, H, K, V):
    return int(load_library().cyfa_scalar_la_workspace_bytes(B, T, H, K, V))


def scalar_la(args: CyfaSlaArgs, device):
    lib = load_library()
    rc = _timed("cyfa_scalar_la", lambda: lib.cyfa_scalar_la(ctypes.byref(args), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_scalar_la failed")


def decode_workspace(B, H, K, V, device):
    """The split decode step's workspace for these dimensions, or None when
    the step runs one workgroup per (batch, head)."""
    n = int(load_library().cyfa_decode_workspace_bytes(B, H, K, V))
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def decode_step(args: CyfaDecodeArgs, device):
    lib = load_library()
    rc = _timed("cyfa_decode_step", lambda: lib.cyfa_decode_step(ctypes.byref(args), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_decode_step failed")


CYFA_DTYPE_BF16, CYFA_DTYPE_F32 = 0, 1


def general_dtype(x):
    """The general path's element type for q, k, v of this dtype: bf16 stays
    bf16; fp16 and fp32 run as fp32 (the caller converts fp16)."""
    return CYFA_DTYPE_BF16 if x.dtype == torch.bfloat16 else CYFA_DTYPE_F32


def chunk_general_workspace_bytes(B, T, H, K, V, M, C):
    return int(load_library().cyfa_chunk_general_workspace_bytes(B, T, H, K, V, M, C))


def chunk_fwd_general(args: CyfaChunkArgs, dtype, device):
    lib = load_library()
    rc = _timed("cyfa_chunk_fwd_general",
                lambda: lib.cyfa_chunk_fwd_general(ctypes.byref(args), dtype, stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_chunk_fwd_general failed")


def chunk_bwd_workspace_bytes(B, T, H, K, V, M):
    return int(load_library().cyfa_chunk_bwd_workspace_bytes(B, T, H, K, V, M))


def chunk_bwd(args: CyfaChunkArgs, dtype, grads: CyfaChunkBwdArgs, device):
    lib = load_library()
    rc = _timed("cyfa_chunk_bwd",
                lambda: lib.cyfa_chunk_bwd(ctypes.byref(args), dtype, ctypes.byref(grads), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_chunk_bwd failed")


def decode_step_general(args: CyfaDecodeArgs, dtype, device):
    lib = load_library()
    rc = _timed("cyfa_decode_step_general",
                lambda: lib.cyfa_decode_step_general(ctypes.byref(args), dtype, stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_decode_step_general failed")


def decode_layer_step(args: CyfaDecodeArgs, layer: CyfaDecodeLayerArgs, device):
    lib = load_library()
    rc = _timed("cyfa_decode_layer_step",
                lambda: lib.cyfa_decode_layer_step(ctypes.byref(args), ctypes.byref(layer), stream_handle(device)))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_decode_layer_step failed")


def readout_table(readout: torch.Tensor) -> torch.Tensor:
    """table = readout @ Phi on the GPU: readout f32 [H, R, R] -> [H, R, R+1]."""
    dev = require_device(readout)
    H, R = readout.shape[0], readout.shape[-1]
    src = readout.detach().to(torch.float32).contiguous()
    table = torch.empty(H, R, R + 1, dtype=torch.float32, device=dev)
    rc = load_library().cyfa_readout_table(ptr(src), ptr(table), H, R + 1, stream_handle(dev))
    if rc != CYFA_OK:
        _raise(rc, "cyfa_readout_table failed")
    return table


def _check(rc, what):
    if rc != CYFA_OK:
        _raise(rc, what + " failed")


def rms_norm(x, weight, eps, gate=None, residual=None, prescale=1.0):
    """Fused (residual add +) RMSNorm (+ sigmoid gate) over the last dim of bf16 x.

    Returns out, or (sum, out) when residual is given (sum = bf16(x + residual))."""
    dev = require_device(x, weight, gate, residual)
    D = x.shape[-1]
    x = x.contiguous()
    w = weight.detach().to(torch.float32).contiguous()
    out = torch.empty_like(x)
    total = None
    if residual is not None:
        residual = residual.contiguous()
        total = torch.empty_like(x)
    if gate is not None:
        gate = gate.contiguous()
    args = CyfaNormArgs(rows=x.numel() // D, D=D, x=ptr(x), residual=ptr(residual), sum_out=ptr(total),
                        weight=ptr(w), gate=ptr(gate), eps=float(eps), prescale=float(prescale), out=ptr(out))
    _check(load_library().cyfa_rms_norm(ctypes.byref(args), stream_handle(dev)), "cyfa_rms_norm")
    return out if residual is None else (total, out)


LINEAR_ROWS_MAX = 64


def _set_linear_prefetch(args, prefetch, dev, what):
    """Fill CyfaLinearArgs' prefetch ranges from (tensor, span) pairs (or bare
    tensors, span 0)."""
    if len(prefetch) > LINEAR_PREFETCH_RANGES:
        raise ValueError(f"{what}: at most {LINEAR_PREFETCH_RANGES} prefetch tensors")
    for i, item in enumerate(prefetch):
        t, span = item if isinstance(item, tuple) else (item, 0)
        if not t.is_contiguous() or t.device != dev:
            raise ValueError(f"{what}: prefetch tensors must be contiguous, on the call's device")
        args.prefetch[i] = t.data_ptr()
        args.prefetch_bytes[i] = t.numel() * t.element_size()
        args.prefetch_span[i] = int(span)


def linear(x, weight, bias=None, out_cols=None, residual=None, prefetch=()):
    """x W^T (+ bias), bf16, like F.linear; with ``residual``, the block's
    residual add residual + bf16(x W^T + bias). Calls with at most 64 rows
    (the one-token decode step) run on cyfa_linear_rows, which streams W once
    across the whole chip; larger calls go to the library GEMM. ``out_cols``
    (>= N) pads the output rows, so that column slices of the result start
    16-byte aligned. ``prefetch``: up to two contiguous device tensors, each
    bare or as (tensor, span) with span from linear_rows_span, that extra
    workgroups of the launch read into the caches for the projection after it
    (ignored where the library GEMM runs)."""
    K = weight.shape[-1]
    N = weight.shape[0]
    width = K
    if x.shape[-1] != width:
        raise ValueError(f"linear: x has {x.shape[-1]} columns, the weight needs {width}")
    rows = x.numel() // width if width else 0
    if (rows == 0 or rows > LINEAR_ROWS_MAX or K % 32 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16
            or (bias is not None and bias.dtype != torch.bfloat16) or not x.is_cuda
            or (residual is not None and residual.dtype != torch.bfloat16)
            or (torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad))):
        y = F.linear(x, weight, bias)
        return y if residual is None else residual + y
    require_device(x, weight, bias, residual)
    if residual is not None:
        residual = residual.reshape(rows, N)
        if residual.stride(-1) != 1:
            residual = residual.contiguous()
    x2 = x.reshape(rows, width)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w = weight.detach()
    if not w.is_contiguous():
        w = w.contiguous()
    ldy = max(N, out_cols or N)
    y = torch.empty(rows, ldy, dtype=torch.bfloat16, device=x.device)
    args = CyfaLinearArgs(M=rows, N=N, K=K, x=x2.data_ptr(), ldx=x2.stride(0), weight=w.data_ptr(),
                          bias=ptr(None if bias is None else bias.detach().contiguous()), y=y.data_ptr(), ldy=ldy,
                          residual=ptr(residual), ldr=0 if residual is None else residual.stride(0))
    _set_linear_prefetch(args, prefetch, x.device, "linear")
    _check(load_library().cyfa_linear_rows(ctypes.byref(args), stream_handle(x.device)), "cyfa_linear_rows")
    lead = tuple(x.shape[:-1])
    if not lead:
        return y.view(-1)[:N]
    strides = [ldy, 1]  # rows ldy apart, whatever the sizes of the leading dims
    for i in range(len(lead) - 2, -1, -1):
        strides.insert(0, strides[0] * lead[i + 1])
    return y.as_strided(lead + (N,), tuple(strides))


LINEAR_NORM_MAX_K = 2048


def fold_norm_weight(weight, norm_weight):
    """bf16(weight diag(norm_weight)): a projection's weight with the RMS norm
    weight in front of it multiplied in, for norm_linear(norm_weight=None)."""
    return (weight.detach().float() * norm_weight.detach().float()).to(weight.dtype)


def linear_rows_span(M, N, K, swiglu=False, norm=0):
    """Bytes of the weight each workgroup of a linear / norm_linear launch with
    M rows reads, when the workgroups that read the bytes [c span, (c + 1)
    span) all run on XCD c mod 8; 0 otherwise (cyfa_linear_rows_span; norm:
    0 none, 1 with the norm weight, 2 folded). For the prefetch spans of
    decode_layer_step, linear and norm_linear; no GPU needed."""
    return int(load_library().cyfa_linear_rows_span(int(M), int(N), int(K), int(bool(swiglu)), int(norm)))


def norm_linear(x, norm_weight, eps, weight, bias=None, residual=None, out_cols=None, swiglu=False, prefetch=()):
    """The block's pre-norm and its first projection in one cyfa_norm_linear_rows
    launch, for at most 64 bf16 rows of K <= 2048 columns:
    s = bf16(x + residual) (x itself without a residual), h = rms_norm(s), and
    y = linear(h, weight, bias) (linear_swiglu(h, weight) with ``swiglu``).
    Returns (s, y). Other shapes run rms_norm and the projection separately.
    h may differ from rms_norm's in the last bit: the sum of squares runs in
    another order.

    norm_weight None: ``weight`` already carries the norm weight
    (fold_norm_weight), and y = bf16(rsqrt(mean(s^2) + eps) (s weight^T) + bias)
    with the row scale on the fp32 product (the shapes above only).
    ``prefetch`` as in linear."""
    K = weight.shape[-1]
    N = weight.shape[0]
    if x.shape[-1] != K:
        raise ValueError(f"norm_linear: x has {x.shape[-1]} columns, the weight needs {K}")
    rows = x.numel() // K if K else 0
    if (rows == 0 or rows > LINEAR_ROWS_MAX or K % 32 or K > LINEAR_NORM_MAX_K or x.dtype != torch.bfloat16
            or weight.dtype != torch.bfloat16 or (bias is not None and bias.dtype != torch.bfloat16)
            or (residual is not None and residual.dtype != torch.bfloat16) or not x.is_cuda
            or (swiglu and (bias is not None or N % 32)) or torch.is_grad_enabled()):
        if norm_weight is None:
            raise ValueError("norm_linear: a folded norm weight needs at most 64 bf16 rows of K <= 2048 "
                             "on the GPU, without grad")
        if residual is None:
            s, h = x, rms_norm(x, norm_weight, eps)
        else:
            s, h = rms_norm(x, norm_weight, eps, residual=residual)
        return s, (linear_swiglu(h, weight) if swiglu else linear(h, weight, bias, out_cols))
    require_device(x, weight, bias, residual)
    x2 = x.reshape(rows, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w = weight.detach()
    if not w.is_contiguous():
        w = w.contiguous()
    nw = None if norm_weight is None else norm_weight.detach().to(torch.float32).contiguous()
    require_device(x, nw)
    s = x
    r2 = total = None
    if residual is not None:
        r2 = residual.reshape(rows, K).contiguous()
        if r2.data_ptr() % 16:
            r2 = r2.clone()
        total = torch.empty(rows, K, dtype=torch.bfloat16, device=x.device)
        s = total.view(x.shape)
    out_w = N // 2 if swiglu else N
    ldy = max(out_w, out_cols or out_w)
    y = torch.empty(rows, ldy, dtype=torch.bfloat16, device=x.device)
    args = CyfaLinearArgs(M=rows, N=N, K=K, x=x2.data_ptr(), ldx=x2.stride(0), weight=w.data_ptr(),
                          bias=ptr(None if bias is None else bias.detach().contiguous()), y=y.data_ptr(), ldy=ldy,
                          swiglu=1 if swiglu else 0)
    _set_linear_prefetch(args, prefetch, x.device, "norm_linear")
    nargs = CyfaRowNormArgs(weight=ptr(nw), eps=float(eps), residual=ptr(r2), sum_out=ptr(total), ldr=K)
    _check(load_library().cyfa_norm_linear_rows(ctypes.byref(args), ctypes.byref(nargs), stream_handle(x.device)),
           "cyfa_norm_linear_rows")
    lead = tuple(x.shape[:-1])
    if not lead:
        return s, y.view(-1)[:out_w]
    strides = [ldy, 1]  # rows ldy apart, whatever the sizes of the leading dims
    for i in range(len(lead) - 2, -1, -1):
        strides.insert(0, strides[0] * lead[i + 1])
    return s, y.as_strided(lead + (out_w,), tuple(strides))


def argmax_rows(x, out=None):
    """x.argmax(-1) for a bf16 CUDA tensor [..., n] (the first maximum, NaN
    largest, as torch.argmax), one cyfa_argmax_rows launch; int64 [...].
    ``out``: a contiguous int64 tensor of the result's size to write into (the
    graphed decode step's token buffer), returned reshaped."""
    require_device(x, out)
    if x.dtype != torch.bfloat16:
        raise ValueError("argmax_rows: bf16 input expected")
    n = x.shape[-1]
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    if out is None:
        out = torch.empty(x2.shape[0], dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or not out.is_contiguous() or out.numel() != x2.shape[0]:
        raise ValueError(f"argmax_rows: out must be a contiguous int64 tensor of {x2.shape[0]} elements")
    _check(load_library().cyfa_argmax_rows(x2.data_ptr(), x2.stride(0), x2.shape[0], n, out.data_ptr(),
                                           stream_handle(x.device)), "cyfa_argmax_rows")
    return out.view(x.shape[:-1])


def interleave_gate_up(gate_weight, up_weight):
    """[F, K] gate and up weights -> [2F, K] in groups of 32 rows (16 gate rows,
    then the matching 16 up rows), the layout linear_swiglu reads."""
    F_, K = gate_weight.shape
    if F_ % 16:
        raise ValueError("interleave_gate_up: the MLP width must be a multiple of 16")
    return torch.cat([gate_weight.reshape(F_ // 16, 16, K), up_weight.reshape(F_ // 16, 16, K)], 1).reshape(2 * F_, K)


def linear_swiglu(x, w_interleaved):
    """bf16(g sigmoid(g) u) of g = x W_gate^T, u = x W_up^T (each rounded to
    bf16), for at most 64 rows, in one cyfa_linear_rows launch; w_interleaved
    comes from interleave_gate_up."""
    K = w_interleaved.shape[-1]
    N = w_interleaved.shape[0]
    rows = x.numel() // K
    require_device(x, w_interleaved)
    if rows == 0 or rows > LINEAR_ROWS_MAX or K % 32 or N % 32 or x.shape[-1] != K:
        raise ValueError(f"linear_swiglu: {rows} rows of {x.shape[-1]} columns against a [{N}, {K}] weight")
    x2 = x.reshape(rows, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    y = torch.empty(rows, N // 2, dtype=torch.bfloat16, device=x.device)
    args = CyfaLinearArgs(M=rows, N=N, K=K, x=x2.data_ptr(), ldx=x2.stride(0), weight=w_interleaved.data_ptr(),
                          bias=None, y=y.data_ptr(), ldy=N // 2, swiglu=1)
    _check(load_library().cyfa_linear_rows(ctypes.byref(args), stream_handle(x.device)), "cyfa_linear_rows")
    return y.view(*x.shape[:-1], N // 2)


def short_conv(x, weight, bias=None, cache=None, split=None, cache_out=None):
    """Causal depthwise convolution over time of x [B, T, D] (rows may be strided).

    weight [D, W] bf16, cache an optional [B, W-1, D] view. The D channels are
    written to D // split contiguous [B, T, split] tensors (split defaults to D).
    ``cache_out`` [B, W-1, D] (channel stride 1) receives the last W-1 rows of
    cat(cache, x); it may be ``cache`` itself when T <= 32."""
    dev = require_device(x, weight, bias, cache)
    B, T, D = x.shape
    W = weight.shape[-1]
    split = D if split is None else split
    if x.stride(-1) != 1 or x.stride(0) != T * x.stride(1):
        x = x.contiguous()
    outs = [torch.empty(B, T, split, dtype=x.dtype, device=dev) for _ in range(D // split)]
    w = weight.reshape(D, W).contiguous()
    if cache is not None and cache.stride(-1) != 1:
        cache = cache.contiguous()
    args = CyfaConvArgs(B=B, T=T, D=D, W=W, x=ptr(x), x_row=x.stride(1),
                        cache=ptr(cache), cache_row=0 if cache is None else cache.stride(1),
                        cache_batch=0 if cache is None else cache.stride(0),
                        weight=ptr(w), bias=ptr(None if bias is None else bias.contiguous()), split=split,
                        cache_out=ptr(cache_out), cache_out_row=0 if cache_out is None else cache_out.stride(1),
                        cache_out_batch=0 if cache_out is None else cache_out.stride(0))
    for i, o in enumerate(outs):
        args.out[i] = o.data_ptr()
    _check(load_library().cyfa_short_conv(ctypes.byref(args), stream_handle(dev)), "cyfa_short_conv")
    return outs


def silu_mul(gu):
    """bf16(g * sigmoid(g) * u) for gu = [..., 2F] holding [g | u]."""
    dev = require_device(gu)
    gu = gu.contiguous()
    F2 = gu.shape[-1]
    out = torch.empty(*gu.shape[:-1], F2 // 2, dtype=gu.dtype, device=dev)
    _check(load_library().cyfa_silu_mul(ptr(gu), ptr(out), gu.numel() // F2, F2 // 2, stream_handle(dev)),
           "cyfa_silu_mul")
    return out


GATE_PATH_G0 = 256
GATE_PATH_MAX = 2048  # largest K and Dv cyfa_gate_path takes


def gate_path_ok(x, w1, w2, b2, H):
    """Whether gate_path takes these operands (else the separate projections)."""
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and w1.dtype == torch.bfloat16 and w2.dtype == torch.bfloat16
            and (b2 is None or b2.dtype == torch.bfloat16) and not torch.is_grad_enabled()
            and K % 64 == 0 and K <= GATE_PATH_MAX and 3 * H <= 32 and w1.shape == (GATE_PATH_G0 + 3 * H, K)
            and w2.shape[1] == GATE_PATH_G0 and w2.shape[0] % 256 == 0 and w2.shape[0] <= GATE_PATH_MAX)


def gate_path(x, w1, abd_bias, w2, b2, dt_bias, A_log, H):
    """The prefill gate path in one cyfa_gate_path launch: g0 = bf16(x W_g0^T),
    abd = bf16(x [W_a|W_b|W_d]^T + abd_bias), the gate activations of abd and
    gate = bf16(g0 W_g1^T + b2). w1 = [W_g0; W_a; W_b; W_d] [256 + 3H, K].
    Returns (gate [..., Dv] bf16, g, beta, delta [..., H] fp32)."""
    K = x.shape[-1]
    Dv = w2.shape[0]
    rows = x.numel() // K
    dev = require_device(x, w1, abd_bias, w2, b2, dt_bias, A_log)
    x2 = x.reshape(rows, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    w1c, w2c = w1.detach().contiguous(), w2.detach().contiguous()
    ab = abd_bias.detach().to(torch.bfloat16).contiguous()
    b2c = None if b2 is None else b2.detach().contiguous()
    db = dt_bias.detach().to(torch.float32).contiguous()
    al = A_log.detach().to(torch.float32).contiguous()
    gate = torch.empty(rows, Dv, dtype=torch.bfloat16, device=dev)
    g, beta, delta = (torch.empty(rows, H, dtype=torch.float32, device=dev) for _ in range(3))
    args = CyfaGatePathArgs(M=rows, K=K, H=H, Dv=Dv, x=x2.data_ptr(), ldx=x2.stride(0), w1=w1c.data_ptr(),
                            abd_bias=ab.data_ptr(), w2=w2c.data_ptr(), b2=ptr(b2c), dt_bias=db.data_ptr(),
                            A_log=al.data_ptr(), gate=gate.data_ptr(), ldg=Dv, g=g.data_ptr(), beta=beta.data_ptr(),
                            delta=delta.data_ptr())
    _check(load_library().cyfa_gate_path(ctypes.byref(args), stream_handle(dev)), "cyfa_gate_path")
    lead = tuple(x.shape[:-1])
    return gate.view(lead + (Dv,)), g.view(lead + (H,)), beta.view(lead + (H,)), delta.view(lead + (H,))


def gates(abd, dt_bias, A_log):
    """(g, beta, delta) fp32 [..., H] from the fused a|b|d projection [..., 3H]."""
    dev = require_device(abd, dt_bias, A_log)
    H = abd.shape[-1] // 3
    rows = abd.numel() // (3 * H)
    flat = abd.reshape(rows, 3 * H) if abd.dim() > 1 else abd.reshape(1, 3 * H)
    if flat.stride(-1) != 1:
        flat = flat.contiguous()
    shape = tuple(abd.shape[:-1]) + (H,)
    g, beta, delta = (torch.empty(shape, dtype=torch.float32, device=dev) for _ in range(3))
    db = dt_bias.detach().to(torch.float32).contiguous()
    al = A_log.detach().to(torch.float32).contiguous()
    _check(load_library().cyfa_gates(ptr(flat), flat.stride(0), ptr(db), ptr(al), ptr(g), ptr(beta), ptr(delta),
                                      rows, H, stream_handle(dev)), "cyfa_gates")
    return g, beta, delta
