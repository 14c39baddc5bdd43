"""MI355X-native CyFA attention hot path behind the Chyxx/CyFA-Jittor interfaces.

The package mirrors the reference's public names (cyclic_flow_attention/__init__.py
of v0.1.2); the attention op runs as hand-written HIP kernels for gfx950 in
libcyfa_hip.so, loaded through ctypes by ``_native``.
"""

from .layers import CyclicFlowAttention
from .models.cyfa import (
    CyclicFlowAttentionConfig,
    CyclicFlowAttentionForCausalLM,
    CyclicFlowAttentionModel,
)

__version__ = "0.1.2"

__all__ = [
    "CyclicFlowAttention",
    "CyclicFlowAttentionConfig",
    "CyclicFlowAttentionForCausalLM",
    "CyclicFlowAttentionModel",
]
