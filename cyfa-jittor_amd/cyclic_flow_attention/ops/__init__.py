"""CyFA operators on the MI355X HIP path (same entry points as the reference's
cyclic_flow_attention/ops/__init__.py:4-7)."""

from .chunk import chunk_cyfa
from .fused_recurrent import fused_recurrent_cyfa

__all__ = ["chunk_cyfa", "fused_recurrent_cyfa"]
