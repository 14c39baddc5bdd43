from .configuration_cyfa import CyclicFlowAttentionConfig
from .modeling_cyfa import CyclicFlowAttentionForCausalLM, CyclicFlowAttentionModel

__all__ = ["CyclicFlowAttentionConfig", "CyclicFlowAttentionForCausalLM", "CyclicFlowAttentionModel"]
