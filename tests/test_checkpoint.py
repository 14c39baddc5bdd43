"""The safetensors checkpoint layout (utils.py:26-70, 115-177 of the
reference): round trips, the published file format (cross-checked with the
safetensors library), the reference's errors. Host-side, no GPU."""

import json
import struct

import pytest
import torch

from cyclic_flow_attention.utils import (initialize_model, load_checkpoint, load_model, load_safetensors, read_config,
                                         save_model, save_safetensors)

safetensors_torch = pytest.importorskip("safetensors.torch")


def _tiny():
    return initialize_model(read_config("tiny.json"), std=0.02, seed=5)


def test_model_round_trip_is_bit_exact(tmp_path):
    model = _tiny()
    save_model(model, tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["model_type"] == "cyclic_flow_attention" and cfg["hidden_size"] == 256
    loaded, directory = load_model(tmp_path)
    assert directory == tmp_path
    a, b = model.state_dict(), loaded.state_dict()
    assert a.keys() == b.keys()
    for name in a:
        assert a[name].dtype == b[name].dtype, name
        assert torch.equal(a[name].view(torch.uint8) if a[name].dtype == torch.bfloat16 else a[name],
                           b[name].view(torch.uint8) if b[name].dtype == torch.bfloat16 else b[name]), name
    # the fp32 parameters of the reference's bf16 policy stay fp32
    assert b["model.layers.0.attn.readout"].dtype == torch.float32
    assert b["model.layers.0.attn.q_proj.weight"].dtype == torch.bfloat16


def test_file_format_matches_the_safetensors_library(tmp_path):
    gen = torch.Generator().manual_seed(0)
    tensors = {
        "a.weight": torch.randn(7, 5, generator=gen).bfloat16(),
        "b.readout": torch.randn(3, 4, 2, generator=gen),
        "c.half": torch.randn(9, generator=gen).half(),
        "d.empty": torch.zeros(0, 4).bfloat16(),
    }
    ours = tmp_path / "ours.safetensors"
    save_safetensors(tensors, ours)
    (size,) = struct.unpack("<Q", ours.read_bytes()[:8])
    assert size % 8 == 0  # header padded with spaces to 8 bytes, as the reference writes it
    header = json.loads(ours.read_bytes()[8:8 + size])
    assert header["a.weight"]["dtype"] == "BF16" and header["b.readout"]["dtype"] == "F32"
    theirs = safetensors_torch.load_file(str(ours))
    for name, t in tensors.items():
        assert theirs[name].dtype == t.dtype and torch.equal(theirs[name].float(), t.float())
    lib = tmp_path / "lib.safetensors"
    safetensors_torch.save_file(tensors, str(lib))
    back = load_safetensors(lib)
    for name, t in tensors.items():
        assert back[name].dtype == t.dtype and torch.equal(back[name].float(), t.float())


def test_bf16_bits_are_written_as_the_reference_truncates_them(tmp_path):
    """The reference writes BF16 as the top 16 bits of the float32 value; for a
    bfloat16 tensor those are its own bits (signed zero, subnormals, inf, NaN)."""
    bits = torch.tensor([0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC1, 0x3F80, 0xC2F7], dtype=torch.int32)
    t = bits.to(torch.int16).view(torch.bfloat16)
    f = tmp_path / "bits.safetensors"
    save_safetensors({"t": t}, f)
    raw = f.read_bytes()
    (size,) = struct.unpack("<Q", raw[:8])
    stored = torch.frombuffer(bytearray(raw[8 + size:]), dtype=torch.int16).to(torch.int32) & 0xFFFF
    truncated = (t.float().view(torch.int32) >> 16) & 0xFFFF
    assert torch.equal(stored, truncated) and torch.equal(stored, bits)


def test_load_checkpoint_errors_like_the_reference(tmp_path):
    model = _tiny()
    with pytest.raises(FileNotFoundError):
        load_checkpoint(model, tmp_path)
    sd = {k: v for k, v in model.state_dict().items() if k != "lm_head.weight"}
    sd["extra.weight"] = torch.zeros(3)
    save_safetensors(sd, tmp_path / "model.safetensors")
    with pytest.raises(ValueError):
        load_checkpoint(model, tmp_path)  # strict: lm_head.weight missing, extra.weight unexpected
    result = load_checkpoint(model, tmp_path, strict=False)
    assert result == {"missing": ["lm_head.weight"], "unexpected": ["extra.weight"]}
    sd = dict(model.state_dict())
    sd["model.norm.weight"] = torch.ones(7)
    save_safetensors(sd, tmp_path / "model.safetensors")
    with pytest.raises(ValueError):
        load_checkpoint(model, tmp_path)  # shape mismatch
    with pytest.raises(FileNotFoundError):
        load_model(tmp_path / "absent")


def test_causal_lm_from_pretrained_and_save_pretrained(tmp_path):
    """The reference's model-class API (models/cyfa/modeling_cyfa.py:85-94):
    save_pretrained writes the checkpoint directory, from_pretrained loads it
    back bit for bit; a tokenizer adds its special-token ids to config.json
    and saves its own files."""
    from cyclic_flow_attention.models.cyfa import CyclicFlowAttentionForCausalLM

    class _Tok:
        eos_id, bos_id = 2, 1

        def save(self, directory):
            (directory / "tokenizer.model").write_bytes(b"tok")

    model = _tiny()
    model.save_pretrained(tmp_path / "a")
    loaded = CyclicFlowAttentionForCausalLM.from_pretrained(tmp_path / "a")
    assert isinstance(loaded, CyclicFlowAttentionForCausalLM)
    for name, value in model.state_dict().items():
        other = loaded.state_dict()[name]
        assert other.dtype == value.dtype and torch.equal(other.float(), value.float()), name
    model.save_pretrained(tmp_path / "b", tokenizer=_Tok())
    cfg = json.loads((tmp_path / "b" / "config.json").read_text())
    assert (cfg["eos_token_id"], cfg["bos_token_id"]) == (2, 1)
    assert (tmp_path / "b" / "tokenizer.model").read_bytes() == b"tok"
    with pytest.raises(FileNotFoundError):
        CyclicFlowAttentionForCausalLM.from_pretrained(tmp_path / "missing")
