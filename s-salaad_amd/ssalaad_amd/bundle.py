"""Compressed-model bundles (format_version 1) and their loading onto the HIP modules.

A bundle is one `torch.save` file, the one the reference's compression run
writes (format: ssalaad/efficient/artifact.py:78-118; writer call:
ssalaad/inference/egar.py:529-570):

    {"format_version": 1,
     "layers": {module name: {"A", "B", "S", "block_p", "block_q", "nm_n", "nm_m"}
                              or {"W"}},
     "base_state_dict": every other model tensor,
     "model_config": the architecture fields,
     "meta": {"mode", "param_count", "p_tgt_million"} only}

What must stay identical for bundles to travel both ways is the format: the
payload keys, the version number, the config field list, the metadata
whitelist and the error texts. The code around it is this package's own:

  * `Bundle` holds a payload and is the one place it is checked, both when a
    file is read and before one is written;
  * `build_efficient_model` first turns every compressed layer into a
    `_Restore` step (an SLR module to install, or a dense weight to copy),
    checks the model's remaining weights against the bundle, and only then
    applies the steps. Every SLR projection becomes an `LRSLinear` of this
    package, run by the gfx950 kernels; there is no CPU path.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable

import torch
from torch import nn

from .ls_linear import LRSLinear

FORMAT_VERSION = 1
# The payload keys of a complete bundle.
PAYLOAD_KEYS = ("format_version", "layers", "base_state_dict", "model_config", "meta")
# Architecture and tokenizer fields a bundle's config keeps (the field list of
# ssalaad/train/model.py:18-45).
MODEL_FIELDS = frozenset({
    "model_type", "architectures", "hidden_size", "intermediate_size", "hidden_act",
    "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim", "vocab_size",
    "max_sequence_length", "max_position_embeddings", "rms_norm_eps", "rope_theta",
    "rope_scaling", "rope_parameters", "initializer_range", "tie_word_embeddings",
    "attention_bias", "attention_dropout", "mlp_bias", "bos_token_id", "eos_token_id",
    "pad_token_id", "tokenizer_id", "use_cache",
})
ALLOWED_META = frozenset({"mode", "param_count", "p_tgt_million"})

# Error texts shared with the reference, so callers that match them keep working.
_ERR_INCOMPLETE = "Expected a complete model bundle produced by the compression entry point."
_ERR_VERSION = "Unsupported model bundle version."
_ERR_WEIGHTS = "The bundle does not contain exactly the required model weights."


def _is_local_path(value: str) -> bool:
    p = Path(value)
    return p.is_absolute() or p.exists()


def export_model_config(config: dict) -> dict:
    """The config a bundle stores: architecture and tokenizer fields only, and
    no tokenizer that names a file on this machine (ssalaad/train/model.py:63-69)."""
    kept = {}
    for key in MODEL_FIELDS & config.keys():
        value = config[key]
        if key == "tokenizer_id" and value and _is_local_path(value):
            continue
        kept[key] = value
    return kept


def _model_classes() -> dict[str, tuple[type, type]]:
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen3Config, Qwen3ForCausalLM

    return {"llama": (LlamaConfig, LlamaForCausalLM), "qwen3": (Qwen3Config, Qwen3ForCausalLM)}


def _hf_config_kwargs(config: dict, attn_implementation: str | None, overrides: dict) -> dict:
    """Bundle config → keyword arguments of the Hugging Face config class.

    Normalisations (ssalaad/train/model.py:78-94): the older sequence-length
    name stands in for max_position_embeddings only when that field is absent,
    a pad id of −1 means "no pad token", and the model is built without a KV
    cache (the decode engine keeps its own)."""
    kw = {k: v for k, v in config.items() if k != "max_sequence_length"}
    if "max_sequence_length" in config:
        if "max_position_embeddings" in config:
            kw["max_sequence_length"] = config["max_sequence_length"]
        else:
            kw["max_position_embeddings"] = config["max_sequence_length"]
    if kw.get("pad_token_id") == -1:
        kw["pad_token_id"] = None
    kw["use_cache"] = False
    if attn_implementation is not None:
        kw["attn_implementation"] = attn_implementation
    kw.update((k, v) for k, v in overrides.items() if v is not None)
    return kw


def build_model_from_config(config: dict, *, attn_implementation: str | None = None,
                            **overrides) -> nn.Module:
    """The Hugging Face causal LM a bundle's config describes."""
    kw = _hf_config_kwargs(config, attn_implementation, overrides)
    kind = kw.get("model_type", "llama")
    classes = _model_classes().get(kind)
    if classes is None:
        raise ValueError(f"Unsupported model type: {kind}")
    config_cls, model_cls = classes
    return model_cls(config_cls(**kw))


@dataclass
class Bundle:
    """One bundle payload, checked on construction."""

    layers: dict[str, dict[str, Any]]
    base_state_dict: dict[str, torch.Tensor]
    model_config: dict
    meta: dict = field(default_factory=dict)
    format_version: int = FORMAT_VERSION

    def __post_init__(self) -> None:
        if self.format_version != FORMAT_VERSION:
            raise ValueError(_ERR_VERSION)

    @classmethod
    def from_payload(cls, payload: Any) -> "Bundle":
        if not isinstance(payload, dict) or any(k not in payload for k in PAYLOAD_KEYS):
            raise ValueError(_ERR_INCOMPLETE)
        return cls(**{k: payload[k] for k in PAYLOAD_KEYS})

    def payload(self) -> dict[str, Any]:
        return {k: getattr(self, k) for k in PAYLOAD_KEYS}


def save_artifact(path: str | Path, layers: dict[str, dict[str, Any]], meta: dict[str, Any], *,
                  model: nn.Module, model_config: dict) -> None:
    """Write a bundle: the compressed layers, every model tensor they do not
    replace, the exported config and the whitelisted metadata."""
    replaced = {f"{name}.weight" for name in layers}
    base = {k: t.detach().cpu().clone() for k, t in model.state_dict().items() if k not in replaced}
    b = Bundle(layers=layers, base_state_dict=base, model_config=export_model_config(model_config),
               meta={k: meta[k] for k in ALLOWED_META & meta.keys()})
    dest = Path(path)
    dest.parent.mkdir(parents=True, exist_ok=True)
    torch.save(b.payload(), dest)


def load_artifact(path: str | Path) -> dict[str, Any]:
    """Read a bundle with the tensor-only loader (nothing in the file runs);
    partial or other-version files are refused."""
    raw = torch.load(path, map_location="cpu", weights_only=True)
    return Bundle.from_payload(raw).payload()


# --------------------------------------------------------------------------
# Loading onto the GPU
# --------------------------------------------------------------------------
@dataclass
class _Restore:
    """What to do with one compressed layer of the model."""

    name: str
    apply: Callable[[nn.Module], None]


def _install(model: nn.Module, name: str, module: nn.Module) -> None:
    owner_name, _, attr = name.rpartition(".")
    owner = model.get_submodule(owner_name) if owner_name else model
    setattr(owner, attr, module)


def _restore_step(name: str, data: dict, target: nn.Module, device: torch.device,
                  dtype: torch.dtype) -> _Restore:
    """How one compressed layer comes back: a dense weight (stored `W`, or the
    factors and S of an embedding multiplied out), or an SLR linear module."""
    if not isinstance(target, (nn.Linear, nn.Embedding)):
        raise TypeError(f"Unsupported compressed module: {name}")
    if "W" not in data and isinstance(target, nn.Linear):
        on_dev = {k: data[k].to(device=device, dtype=dtype) for k in ("A", "B", "S")}
        bias = target.bias
        module = LRSLinear(
            on_dev["A"], on_dev["B"], on_dev["S"],
            in_features=target.in_features, out_features=target.out_features,
            bias=None if bias is None else bias.detach().to(device=device, dtype=dtype),
            block_p=data.get("block_p"), block_q=data.get("block_q"),
            nm_n=data.get("nm_n"), nm_m=data.get("nm_m"),
        )
        return _Restore(name, lambda model: _install(model, name, module))
    if "W" in data:
        weight = data["W"]
    else:  # a compressed embedding table runs dense
        weight = data["A"].float() @ data["B"].float() + data["S"].to_dense().float()
    if weight.shape != target.weight.shape:
        raise ValueError(f"Weight shape mismatch: {name}")

    def copy_weight(model: nn.Module) -> None:
        with torch.no_grad():
            model.get_submodule(name).weight.copy_(weight.to(dtype=dtype))

    return _Restore(name, copy_weight)


def build_efficient_model(path, *, device="cuda", dtype=None):
    """A compressed model on the GPU with HIP SLR linears; returns
    (model, model_config, meta), the result of ssalaad/efficient/model.py:11-60."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError(
            "the HIP SLR modules run on a ROCm GPU device; load the bundle with device='cuda'"
        )
    dtype = dtype or torch.bfloat16
    b = Bundle.from_payload(load_artifact(path))
    model = build_model_from_config(b.model_config, attn_implementation="sdpa")
    # The model's own tensors must be exactly the bundle's base tensors plus
    # one weight per compressed layer.
    own = set(model.state_dict())
    if set(b.base_state_dict) - own or own - set(b.base_state_dict) != {f"{n}.weight" for n in b.layers}:
        raise ValueError(_ERR_WEIGHTS)
    model.load_state_dict(b.base_state_dict, strict=False)
    model.to(dtype=dtype)
    steps = [_restore_step(name, data, model.get_submodule(name), device, dtype)
             for name, data in b.layers.items()]
    for step in steps:
        step.apply(model)
    return model.to(device=device).eval(), b.model_config, b.meta
