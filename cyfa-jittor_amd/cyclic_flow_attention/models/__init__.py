from .cyfa import CyclicFlowAttentionConfig, CyclicFlowAttentionForCausalLM, CyclicFlowAttentionModel

__all__ = ["CyclicFlowAttentionConfig", "CyclicFlowAttentionForCausalLM", "CyclicFlowAttentionModel"]
