"""A small synthetic safetensors checkpoint with the reference's tensor names.

Real Qwen3.6 attention shapes, random weights scaled so activations stay
O(1).  Only the attention tensors of the requested layers are written.
"""

from __future__ import annotations

from pathlib import Path

import torch
from safetensors.torch import save_file

HIDDEN = 2048


def _w(g, shape, scale, dtype=torch.bfloat16):
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def make_checkpoint(root: Path, kinds: dict[int, str], seed: int = 0) -> dict[int, dict[str, torch.Tensor]]:
    g = torch.Generator().manual_seed(seed)
    tensors: dict[str, torch.Tensor] = {}
    per_layer: dict[int, dict[str, torch.Tensor]] = {}
    s_in = HIDDEN ** -0.5
    for layer, kind in sorted(kinds.items()):
        w: dict[str, torch.Tensor] = {"input_layernorm.weight": _w(g, (HIDDEN,), 0.1)}
        if kind == "linear":
            w.update({
                "linear_attn.in_proj_qkv.weight": _w(g, (8192, HIDDEN), s_in),
                "linear_attn.in_proj_z.weight": _w(g, (4096, HIDDEN), s_in),
                "linear_attn.in_proj_a.weight": _w(g, (32, HIDDEN), s_in),
                "linear_attn.in_proj_b.weight": _w(g, (32, HIDDEN), s_in),
                "linear_attn.conv1d.weight": _w(g, (8192, 1, 4), 0.5),
                "linear_attn.A_log": torch.rand((32,), generator=g) * 4.0 - 4.0,
                "linear_attn.dt_bias": torch.randn((32,), generator=g) * 0.5,
                "linear_attn.norm.weight": _w(g, (128,), 1.0) + 1.0,
                "linear_attn.out_proj.weight": _w(g, (HIDDEN, 4096), 4096 ** -0.5),
            })
        else:
            w.update({
                "self_attn.q_proj.weight": _w(g, (8192, HIDDEN), s_in),
                "self_attn.k_proj.weight": _w(g, (512, HIDDEN), s_in),
                "self_attn.v_proj.weight": _w(g, (512, HIDDEN), s_in),
                "self_attn.q_norm.weight": _w(g, (256,), 0.1),
                "self_attn.k_norm.weight": _w(g, (256,), 0.1),
                "self_attn.o_proj.weight": _w(g, (HIDDEN, 4096), 4096 ** -0.5),
            })
        per_layer[layer] = w
        for name, t in w.items():
            tensors[f"model.language_model.layers.{layer}.{name}"] = t.contiguous()
    root.mkdir(parents=True, exist_ok=True)
    save_file(tensors, str(root / "model.safetensors"))
    return per_layer
