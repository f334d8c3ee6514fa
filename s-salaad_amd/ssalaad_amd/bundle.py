"""Compressed-model bundles (format_version 1) and their loading onto the HIP modules.

A bundle is the dict `torch.save` writes at the end of the reference's
compression run (ssalaad/efficient/artifact.py:78-118, written by
ssalaad/inference/egar.py:529-570):

    {"format_version": 1,
     "layers": {module name: {"A", "B", "S", "block_p", "block_q", "nm_n", "nm_m"}
                              or {"W"}},
     "base_state_dict": every other model tensor,
     "model_config": the architecture fields,
     "meta": {"mode", "param_count", "p_tgt_million"} only}

`load_artifact` / `save_artifact` read and write that layout, with the
reference's checks and messages. `build_efficient_model` mirrors
ssalaad/efficient/model.py:11-60: it builds the Hugging Face model from the
config, loads the base weights and swaps every compressed linear for an
`LRSLinear` of this package (one fused HIP launch per call). It runs on a ROCm
GPU only; there is no CPU path.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import torch
from torch import nn

from .ls_linear import LRSLinear

# Architecture and tokenizer fields a bundle keeps (ssalaad/train/model.py:18-45).
MODEL_FIELDS = frozenset({
    "model_type", "architectures", "hidden_size", "intermediate_size", "hidden_act",
    "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim", "vocab_size",
    "max_sequence_length", "max_position_embeddings", "rms_norm_eps", "rope_theta",
    "rope_scaling", "rope_parameters", "initializer_range", "tie_word_embeddings",
    "attention_bias", "attention_dropout", "mlp_bias", "bos_token_id", "eos_token_id",
    "pad_token_id", "tokenizer_id", "use_cache",
})
ALLOWED_META = frozenset({"mode", "param_count", "p_tgt_million"})
FORMAT_VERSION = 1


def export_model_config(config: dict) -> dict:
    """Keep the architecture and tokenizer fields; drop a local tokenizer path
    (ssalaad/train/model.py:63-69)."""
    result = {k: v for k, v in config.items() if k in MODEL_FIELDS}
    tok = result.get("tokenizer_id", "")
    if tok and (Path(tok).is_absolute() or Path(tok).exists()):
        result.pop("tokenizer_id")
    return result


def _model_classes():
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    return {"llama": (LlamaConfig, LlamaForCausalLM), "qwen3": (Qwen3Config, Qwen3ForCausalLM)}


def build_model_from_config(config: dict, *, attn_implementation: str | None = None,
                            **overrides) -> nn.Module:
    """A Hugging Face causal LM from a bundle's config (ssalaad/train/model.py:78-94)."""
    config = dict(config)
    if "max_sequence_length" in config and "max_position_embeddings" not in config:
        config["max_position_embeddings"] = config.pop("max_sequence_length")
    if config.get("pad_token_id") == -1:
        config["pad_token_id"] = None
    config["use_cache"] = False
    if attn_implementation is not None:
        config["attn_implementation"] = attn_implementation
    config.update({k: v for k, v in overrides.items() if v is not None})
    model_type = config.get("model_type", "llama")
    classes = _model_classes()
    if model_type not in classes:
        raise ValueError(f"Unsupported model type: {model_type}")
    config_cls, model_cls = classes[model_type]
    return model_cls(config_cls(**config))


def save_artifact(path: str | Path, layers: dict[str, dict[str, Any]], meta: dict[str, Any], *,
                  model: nn.Module, model_config: dict) -> None:
    """Write a bundle: the compressed layers and every other model tensor
    (ssalaad/efficient/artifact.py:78-104)."""
    compressed = {name + ".weight" for name in layers}
    base_state = {k: t.detach().cpu().clone() for k, t in model.state_dict().items()
                  if k not in compressed}
    payload = {
        "format_version": FORMAT_VERSION,
        "layers": layers,
        "base_state_dict": base_state,
        "model_config": export_model_config(model_config),
        "meta": {k: v for k, v in meta.items() if k in ALLOWED_META},
    }
    dest = Path(path)
    dest.parent.mkdir(parents=True, exist_ok=True)
    torch.save(payload, dest)


def load_artifact(path: str | Path) -> dict[str, Any]:
    """Read a bundle with the tensor-only loader; legacy partial artifacts are
    rejected (ssalaad/efficient/artifact.py:107-118)."""
    payload = torch.load(path, map_location="cpu", weights_only=True)
    required = {"format_version", "layers", "base_state_dict", "model_config", "meta"}
    if not isinstance(payload, dict) or not required.issubset(payload):
        raise ValueError(
            "Expected a complete model bundle produced by the compression entry point."
        )
    if payload["format_version"] != FORMAT_VERSION:
        raise ValueError("Unsupported model bundle version.")
    return payload


def build_efficient_model(path, *, device="cuda", dtype=None):
    """Load a compressed model onto the GPU with HIP SLR linears
    (ssalaad/efficient/model.py:11-60). Returns (model, model_config, meta)."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(
            "the HIP SLR modules run on a ROCm GPU device; load the bundle with device='cuda'"
        )
    dtype = dtype or torch.bfloat16
    payload = load_artifact(path)
    model = build_model_from_config(payload["model_config"], attn_implementation="sdpa")
    layers = payload["layers"]
    missing, unexpected = model.load_state_dict(payload["base_state_dict"], strict=False)
    expected = {name + ".weight" for name in layers}
    if set(missing) != expected or unexpected:
        raise ValueError("The bundle does not contain exactly the required model weights.")
    model.to(dtype=dtype)
    for name, data in layers.items():
        old = model.get_submodule(name)
        if not isinstance(old, (nn.Linear, nn.Embedding)):
            raise TypeError(f"Unsupported compressed module: {name}")
        if "W" in data:
            weight = data["W"]
        elif isinstance(old, nn.Embedding):
            weight = data["A"].float() @ data["B"].float() + data["S"].to_dense().float()
        else:
            new = LRSLinear(
                data["A"].to(device=device, dtype=dtype),
                data["B"].to(device=device, dtype=dtype),
                data["S"].to(device=device, dtype=dtype),
                in_features=old.in_features,
                out_features=old.out_features,
                bias=old.bias.detach().to(device=device, dtype=dtype) if old.bias is not None else None,
                block_p=data.get("block_p"),
                block_q=data.get("block_q"),
                nm_n=data.get("nm_n"),
                nm_m=data.get("nm_m"),
            )
            parent_name, _, attr = name.rpartition(".")
            parent = model.get_submodule(parent_name) if parent_name else model
            setattr(parent, attr, new)
            continue
        if weight.shape != old.weight.shape:
            raise ValueError(f"Weight shape mismatch: {name}")
        with torch.no_grad():
            old.weight.copy_(weight.to(dtype=dtype))
    return model.to(device=device).eval(), payload["model_config"], payload["meta"]
