"""Config reading, seeded initialisation and the safetensors checkpoint
layout (utils.py:26-70, 92-177 of Chyxx/CyFA-Jittor v0.1.2)."""

import dataclasses
import json
import os
import struct
from pathlib import Path

import numpy as np
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


# safetensors dtype codes <-> torch dtypes (the codes the reference reads and
# writes, utils.py:16-23, 138)
_ST_DTYPES = {
    "BF16": torch.bfloat16,
    "F16": torch.float16,
    "F32": torch.float32,
    "I64": torch.int64,
    "I32": torch.int32,
    "U8": torch.uint8,
    "BOOL": torch.bool,
}
_ST_CODES = {torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32"}


def load_safetensors(path):
    """name -> CPU tensor for one .safetensors file (utils.py:26-47).

    The file is an 8-byte little-endian header length, a JSON header
    {name: {dtype, shape, data_offsets}} and the raw little-endian data.
    Tensors keep the stored dtype (BF16 stays bfloat16: the reference widens
    it to float32, which is exact)."""
    path = Path(path)
    with open(path, "rb") as f:
        (size,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(size))
    data = np.memmap(path, mode="r", dtype=np.uint8, offset=8 + size) if path.stat().st_size > 8 + size else None
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        code = meta["dtype"]
        if code not in _ST_DTYPES:
            raise ValueError(f"{path}: tensor {name} has unsupported dtype {code}")
        begin, end = meta["data_offsets"]
        dtype = _ST_DTYPES[code]
        shape = tuple(meta["shape"])
        nbytes = int(np.prod(shape, dtype=np.int64)) * torch.empty((), dtype=dtype).element_size()
        if end - begin != nbytes:
            raise ValueError(f"{path}: tensor {name} holds {end - begin} bytes, its shape needs {nbytes}")
        raw = bytearray(data[begin:end]) if nbytes else bytearray()
        out[name] = torch.frombuffer(raw, dtype=dtype).reshape(shape) if nbytes else torch.empty(shape, dtype=dtype)
    return out


def load_checkpoint(model, directory, strict=True):
    """Copy every *.safetensors file under ``directory`` into the model's
    parameters by name (utils.py:50-70), casting to each parameter's dtype.
    A shape mismatch raises ValueError((name, stored, expected)); with
    ``strict``, missing or unexpected names raise ValueError. Returns
    {"missing": [...], "unexpected": [...]}."""
    directory = Path(directory)
    files = sorted(directory.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError("No safetensors weights under " + str(directory))
    weights = {}
    for f in files:
        weights.update(load_safetensors(f))
    missing = []
    with torch.no_grad():
        for name, value in model.state_dict().items():
            if name not in weights:
                missing.append(name)
                continue
            stored = weights.pop(name)
            if tuple(stored.shape) != tuple(value.shape):
                raise ValueError((name, tuple(stored.shape), tuple(value.shape)))
            value.copy_(stored.to(value.dtype))
    result = {"missing": missing, "unexpected": list(weights)}
    if strict and (missing or weights):
        raise ValueError(result)
    return result


def save_safetensors(tensors, path):
    """Write name -> tensor as one .safetensors file in each tensor's storage
    dtype (BF16, F16 or F32), through a temporary file renamed into place
    (utils.py:132-160). The reference writes BF16 by truncating the float32
    value to its top 16 bits; a bfloat16 tensor's float32 value is exact, so
    that is its own bits, which are written here."""
    path = Path(path)
    header, offset, items = {}, 0, []
    for name, value in tensors.items():
        value = value.detach()
        if value.dtype not in _ST_CODES:
            raise ValueError(f"save_safetensors: {name} has dtype {value.dtype}")
        nbytes = value.numel() * value.element_size()
        header[name] = {"dtype": _ST_CODES[value.dtype], "shape": list(value.shape),
                        "data_offsets": [offset, offset + nbytes]}
        offset += nbytes
        items.append(value)
    encoded = json.dumps(header, separators=(",", ":")).encode()
    encoded += b" " * (-len(encoded) % 8)
    tmp = path.with_name(path.name + ".tmp")
    with tmp.open("wb") as f:
        f.write(struct.pack("<Q", len(encoded)))
        f.write(encoded)
        for value in items:
            flat = value.to("cpu").contiguous().reshape(-1)
            f.write(flat.view(torch.uint8).numpy().tobytes() if flat.numel() else b"")
    os.replace(tmp, path)


def save_model(model, directory, tokenizer=None):
    """config.json (the config fields plus model_type and architectures) and
    model.safetensors with the torch-checkpoint parameter names
    (utils.py:163-177). With a tokenizer, config.json also records its
    ``eos_id`` / ``bos_id`` as eos_token_id / bos_token_id and the
    tokenizer writes its own files into the directory (``tokenizer.save``)."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    config = dataclasses.asdict(model.config)
    config.update(model_type="cyclic_flow_attention", architectures=["CyclicFlowAttentionForCausalLM"])
    if tokenizer is not None:
        config.update(eos_token_id=tokenizer.eos_id, bos_token_id=tokenizer.bos_id)
    (directory / "config.json").write_text(json.dumps(config, indent=2) + "\n")
    save_safetensors(model.state_dict(), directory / "model.safetensors")
    if tokenizer is not None:
        tokenizer.save(directory)


def load_model(path):
    """(model, directory) for a local checkpoint directory: the config, a bf16
    model (fp32 norms, readout, A_log, dt_bias) and its weights, strictly
    (utils.py:115-119; no download: the path must exist)."""
    directory = Path(path).expanduser()
    if not directory.exists():
        raise FileNotFoundError(f"no checkpoint directory {directory}")
    model = CyclicFlowAttentionForCausalLM(read_config(directory)).to_bfloat16()
    load_checkpoint(model, directory)
    return model, directory
