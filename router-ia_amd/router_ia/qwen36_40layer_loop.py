"""Model constants and per-layer checkpoint access used by the attention cache.

Constants follow v2/src/router_ia/qwen36_40layer_loop.py:36-50 (Qwen3.6 hybrid
backbone: 3 Gated DeltaNet layers then 1 full-attention layer, repeated).
``attention_type`` probes the checkpoint the same way (:68-78) and caches the
answer per (root, layer).
"""

from __future__ import annotations

from pathlib import Path

import torch

from . import weights

HIDDEN = 2048
LINEAR_NUM_K_HEADS = 16
LINEAR_NUM_V_HEADS = 32
LINEAR_KEY_DIM = LINEAR_NUM_K_HEADS * 128
LINEAR_VALUE_DIM = LINEAR_NUM_V_HEADS * 128
FULL_NUM_HEADS = 16
FULL_NUM_KV_HEADS = 2
FULL_HEAD_DIM = 256
FULL_Q_DIM = FULL_NUM_HEADS * FULL_HEAD_DIM
FULL_KV_DIM = FULL_NUM_KV_HEADS * FULL_HEAD_DIM
FULL_Q_GATE_DIM = FULL_Q_DIM * 2
FULL_ROPE_DIM = int(FULL_HEAD_DIM * 0.25)
FULL_NUM_KV_GROUPS = FULL_NUM_HEADS // FULL_NUM_KV_HEADS
EPS = 1e-6
DEFAULT_LAYERS = 40

_ATTN_TYPE_CACHE: dict[tuple[Path, int], str] = {}


def layer_prefix(layer: int) -> str:
    return f"model.language_model.layers.{layer}."


def is_full_attention_layer(layer: int) -> bool:
    """Layer pattern of the family: every fourth layer (3, 7, ..., 39) is full attention."""
    return layer % 4 == 3


def load_layer_weight(root: Path, layer: int, suffix: str, device: str) -> torch.Tensor:
    return weights.load_tensor(root, layer_prefix(layer) + suffix, device=device)


def attention_type(root: Path, layer: int) -> str:
    key = (Path(root).resolve(), int(layer))
    cached = _ATTN_TYPE_CACHE.get(key)
    if cached is not None:
        return cached
    prefix = layer_prefix(layer)
    if weights.has_tensor(root, prefix + "linear_attn.in_proj_qkv.weight"):
        kind = "linear_attention"
    elif weights.has_tensor(root, prefix + "self_attn.q_proj.weight"):
        kind = "full_attention"
    else:
        raise KeyError(f"Could not identify attention type for layer {layer}")
    _ATTN_TYPE_CACHE[key] = kind
    return kind
