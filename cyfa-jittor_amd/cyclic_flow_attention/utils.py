"""Config reading and seeded initialisation (utils.py:92-129 of Chyxx/CyFA-Jittor v0.1.2)."""

import json
from pathlib import Path

import torch

from .models.cyfa import CyclicFlowAttentionConfig, CyclicFlowAttentionForCausalLM

CONFIG_DIR = Path(__file__).resolve().parent / "configs"


def read_config(path):
    """Read a config.json (or a directory holding one) into the dataclass.

    Unknown keys are ignored; checkpoint_level != 0 and non-SwiGLU models are
    rejected, as in the reference (utils.py:92-112)."""
    path = Path(path)
    if not path.exists() and (CONFIG_DIR / path.name).exists():
        path = CONFIG_DIR / path.name
    data = json.loads((path / "config.json" if path.is_dir() else path).read_text())
    if data.get("checkpoint_level", 0) != 0:
        raise ValueError("Only checkpoint_level=0 is supported")
    config = CyclicFlowAttentionConfig(
        **{k: v for k, v in data.items() if k in CyclicFlowAttentionConfig.__dataclass_fields__}
    )
    if config.hidden_size <= 0 or config.num_hidden_layers <= 0 or config.vocab_size <= 1:
        raise ValueError("Invalid model dimensions")
    if data.get("hidden_act", "swish") not in ("swish", "silu"):
        raise ValueError("Only the released SwiGLU model architecture is supported")
    return config


def initialize_model(config, std=0.02, seed=0):
    """Seeded random model (utils.py:122-129): every non-norm ``.weight`` ~ N(0, std),
    biases zero, dt_bias / A_log / readout at the layer defaults, then bf16
    except the fp32 parameters of ``to_bfloat16``. Built on the CPU with a
    torch.Generator so the same seed gives the same weights everywhere."""
    torch.manual_seed(seed)  # layer defaults (dt_bias, A_log, conv) draw from the global RNG
    model = CyclicFlowAttentionForCausalLM(config)
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith(".weight") and "norm" not in name:
                p.copy_(torch.randn(p.shape, generator=gen) * std)
            elif name.endswith(".bias"):
                p.zero_()
    return model.to_bfloat16()
