"""Helpers shared by the CyFA op wrappers."""

import torch

from .. import _native


def check_forward_only(name, tensors):
    """The HIP path is forward/inference only; refuse to build an autograd graph."""
    if torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors):
        raise NotImplementedError(
            f"{name} runs the forward HIP kernels only; call it under torch.no_grad() "
            "(the backward pass is not implemented)"
        )


def readout_table(readout):
    """table = readout @ Phi, [H, M-1, M] fp32 (ops/chunk.py:82-103, 281)."""
    return _native.readout_table(readout)


def check_table(table, H, M):
    """A precomputed readout table must be contiguous float32 [H, M-1, M]."""
    if tuple(table.shape) != (H, M - 1, M) or table.dtype != torch.float32 or not table.is_contiguous():
        raise ValueError(
            f"table must be contiguous float32 [{H}, {M - 1}, {M}], got {tuple(table.shape)} {table.dtype}"
        )
