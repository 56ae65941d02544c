"""Minimal safetensors checkpoint access for the attention layers.

Weight loading is not part of the accelerated path; this module only gives
``step_attention`` the tensors it needs, with the reference's dtype contract:
projections are dense fp16 on a GPU and fp32 on the CPU, FP8 (e4m3) weights
are dequantised with their 128x128 block scales
(v2/src/router_ia/qwen36_cached_loop.py:526-560, v2/src/router_ia/qwen36_dequant.py:35-58).
Loaded tensors are cached per (root, name, device) for the life of the process.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors import safe_open


BLOCK = 128

_INDEX_CACHE: dict[Path, dict[str, Path]] = {}
_TENSOR_CACHE: dict[tuple[Path, str, str], torch.Tensor] = {}
_PROJ_CACHE: dict[tuple[Path, str, str], torch.Tensor] = {}


def _index(root: Path) -> dict[str, Path]:
    root = Path(root).resolve()
    idx = _INDEX_CACHE.get(root)
    if idx is not None:
        return idx
    idx = {}
    index_path = root / "model.safetensors.index.json"
    if index_path.is_file():
        payload = json.loads(index_path.read_text(encoding="utf-8"))
        for name, shard in payload.get("weight_map", {}).items():
            idx[name] = root / shard
    else:
        for shard in sorted(root.glob("*.safetensors")):
            with safe_open(str(shard), framework="pt", device="cpu") as handle:
                for name in handle.keys():
                    idx.setdefault(name, shard)
    _INDEX_CACHE[root] = idx
    return idx


def has_tensor(root: Path, name: str) -> bool:
    return name in _index(root)


def load_tensor(root: Path, name: str, device: str = "cpu") -> torch.Tensor:
    root = Path(root).resolve()
    key = (root, name, str(torch.device(device)))
    cached = _TENSOR_CACHE.get(key)
    if cached is not None:
        return cached
    shard = _index(root).get(name)
    if shard is None:
        raise KeyError(f"Tensor not found: {name}")
    with safe_open(str(shard), framework="pt", device="cpu") as handle:
        tensor = handle.get_tensor(name).to(device=device)
    _TENSOR_CACHE[key] = tensor
    return tensor


def dequantize_fp8_blockwise(weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    out_f, in_f = map(int, weight.shape)
    expanded = scale_inv.float().repeat_interleave(BLOCK, dim=0).repeat_interleave(BLOCK, dim=1)
    return weight.float() * expanded[:out_f, :in_f]


def cached_load_projection(root: Path, prefix: str, device: str) -> torch.Tensor:
    root = Path(root).resolve()
    key = (root, prefix, str(torch.device(device)))
    cached = _PROJ_CACHE.get(key)
    if cached is not None:
        return cached
    weight = load_tensor(root, prefix + ".weight", device="cpu")
    if weight.dtype == torch.float8_e4m3fn:
        scale = load_tensor(root, prefix + ".weight_scale_inv", device="cpu")
        out = dequantize_fp8_blockwise(weight, scale)
    else:
        out = weight.float()
    if torch.device(device).type == "cuda":  # a ROCm GPU
        out = out.to(device=device, dtype=torch.float16)
    _PROJ_CACHE[key] = out
    return out


def clear_caches() -> None:
    _INDEX_CACHE.clear()
    _TENSOR_CACHE.clear()
    _PROJ_CACHE.clear()
