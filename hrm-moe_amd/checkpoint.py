"""MoE FFN weights from the reference's checkpoint formats (local files only).

The reference's Hugging Face release is one ``model.safetensors`` plus a
``config.json``.  Its keys differ from the native module tree only in their
prefixes (simple_inference_engine.py:139-145 maps release -> native;
conversion/convert_to_hf.py:17-30 maps native -> release and drops the rotary
buffers and ``model.zH_init``).  Under a layer's ``mlp.`` the MoE FFN's
parameter names are the same in both, and the same as this package's
``SparseMoESwiGLU`` (``gate.weight``, ``experts.gate_up_weight``,
``experts.down_weight``; models/layers.py:548, :272-283), so a layer's state
loads unchanged once the prefix is mapped.

Only safetensors and JSON are read (no pickled objects), and only from a local
directory: fetching the release from the hub is not part of this package.
"""
from __future__ import annotations

import json
import os
from typing import Optional

import torch

from .layers import SparseMoESwiGLU

# release prefix -> native prefix (simple_inference_engine.py:139-145)
_PREFIX_MAP = (
    ("model.H_module.layers.", "model.H_level.core.layers."),
    ("model.L_module.layers.", "model.L_level.core.layers."),
    ("model.z_L_init", "model.zL_init"),
)
_EMBED = ("model.embed_tokens.weight", "embed_tokens.embedding_weight")
# native keys the release leaves out (conversion/convert_to_hf.py:17-20)
_SKIP_PREFIXES = ("model.H_level.core.rotary_emb.", "model.L_level.core.rotary_emb.")
_DROP_KEYS = frozenset({"model.zH_init"})

MOE_PARAMS = ("gate.weight", "experts.gate_up_weight", "experts.down_weight")


def hf_to_native_key(key: str) -> str:
    """Release key -> native key (simple_inference_engine.py:139-145)."""
    for hf, native in _PREFIX_MAP:
        key = key.replace(hf, native)
    return _EMBED[1] if key == _EMBED[0] else key


def native_to_hf_key(key: str) -> Optional[str]:
    """Native key -> release key, or None for keys the release does not store (convert_to_hf.py:23-30)."""
    if key in _DROP_KEYS or key.startswith(_SKIP_PREFIXES):
        return None
    for hf, native in _PREFIX_MAP:
        key = key.replace(native, hf)
    return _EMBED[0] if key == _EMBED[1] else key


def moe_layer_prefixes(state: dict) -> list:
    """Prefixes ``p`` (ending in ``mlp.``) for which ``p + name`` exists for every MoE FFN parameter."""
    suffix = MOE_PARAMS[0]
    found = []
    for key in state:
        if key.endswith("mlp." + suffix):
            p = key[: -len(suffix)]
            if all(p + name in state for name in MOE_PARAMS):
                found.append(p)
    return sorted(found)


def moe_layer_config(state: dict, prefix: str, hf_config: Optional[dict] = None) -> dict:
    """Constructor arguments of the MoE layer under ``prefix``, from tensor shapes and the release config.

    Shapes give H, I and E (gate [E,H], gate_up [E,2I,H], down [E,H,I]); top-k
    and the renormalisation flag come from ``moe_top_k`` / ``moe_norm_topk_prob``
    with the reference's defaults (simple_inference_engine.py:174-181).
    """
    gate = state[prefix + "gate.weight"]
    gate_up = state[prefix + "experts.gate_up_weight"]
    down = state[prefix + "experts.down_weight"]
    e, h = gate.shape
    if gate_up.shape[0] != e or gate_up.shape[2] != h or gate_up.shape[1] % 2:
        raise ValueError(f"{prefix}experts.gate_up_weight has shape {tuple(gate_up.shape)} for gate {tuple(gate.shape)}")
    i = gate_up.shape[1] // 2
    if tuple(down.shape) != (e, h, i):
        raise ValueError(f"{prefix}experts.down_weight has shape {tuple(down.shape)}, expected {(e, h, i)}")
    cfg = hf_config or {}
    return dict(hidden_size=int(h), intermediate_size=int(i), num_experts=int(e),
                top_k=int(cfg.get("moe_top_k", 1)), norm_topk_prob=bool(cfg.get("moe_norm_topk_prob", True)))


def load_moe_layers(ckpt_dir: str, device="cuda", dtype: torch.dtype = torch.bfloat16,
                    implementation: str = "grouped_triton") -> dict:
    """Every MoE FFN layer of a local release directory, as ``{native prefix: SparseMoESwiGLU}``.

    Reads ``model.safetensors`` and, when present, ``config.json``; maps keys
    as the reference's loader does; builds each layer and loads its three
    tensors with ``strict=True``.
    """
    from safetensors.torch import load_file

    weights = os.path.join(ckpt_dir, "model.safetensors")
    if not os.path.exists(weights):
        raise FileNotFoundError(f"{weights} not found (only local release directories are read)")
    cfg_path = os.path.join(ckpt_dir, "config.json")
    hf_config = json.load(open(cfg_path)) if os.path.exists(cfg_path) else None
    state = {hf_to_native_key(k): v for k, v in load_file(weights, device="cpu").items()}
    layers = {}
    for prefix in moe_layer_prefixes(state):
        layer = SparseMoESwiGLU(**moe_layer_config(state, prefix, hf_config), implementation=implementation)
        layer.load_state_dict({name: state[prefix + name] for name in MOE_PARAMS}, strict=True)
        layers[prefix] = layer.to(device=device, dtype=dtype)
    return layers


def save_moe_layers(layers: dict, path: str) -> None:
    """Write ``{native prefix: module}`` MoE layers to a safetensors file under release keys."""
    from safetensors.torch import save_file

    out = {}
    for prefix, layer in layers.items():
        sd = layer.state_dict()
        for name in MOE_PARAMS:
            key = native_to_hf_key(prefix + name)
            if key is None:
                raise ValueError(f"{prefix + name} has no release key")
            out[key] = sd[name].detach().to("cpu").contiguous()
    save_file(out, path)
