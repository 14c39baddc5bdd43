"""Configuration of the CyFA language models (models/cyfa/configuration_cyfa.py:9-35
of Chyxx/CyFA-Jittor v0.1.2; same fields and defaults)."""

from dataclasses import dataclass


@dataclass
class CyclicFlowAttentionConfig:
    hidden_size: int = 1024
    num_heads: int = 4
    head_dim: int = 256
    expand_k: float = 1.0
    expand_v: float = 1.0
    num_slots: int = 128
    num_hidden_layers: int = 24
    vocab_size: int = 32000
    hidden_ratio: float = 4.0
    intermediate_size: int | None = None
    use_short_conv: bool = True
    conv_size: int = 4
    conv_bias: bool = False
    norm_eps: float = 1e-6
    tie_word_embeddings: bool = False
    chunk_size: int = 64

    @classmethod
    def from_pretrained(cls, path):
        from ...utils import read_config

        return read_config(path)
