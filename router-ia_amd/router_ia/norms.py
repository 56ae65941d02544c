"""RMSNorm variants applied around the attention core (torch ops).

These sit outside the accelerated path; they keep the reference's dtype order
so that ``step_attention`` returns what the reference returns:
``rmsnorm`` (v2/src/router_ia/qwen36_op_probe.py:55-67, (1 + w) affine) and
``gated_rmsnorm`` (v2/src/router_ia/qwen36_gated_norm_probe.py:19-36).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

EPS = 1e-6


def rmsnorm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    input_dtype = x.dtype
    x32 = x.float()
    out = x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + EPS)
    out = out * (1.0 + weight.float())
    return out.to(dtype=input_dtype)


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    if x.shape != z.shape:
        raise ValueError(f"x/z shape mismatch: {tuple(x.shape)} vs {tuple(z.shape)}")
    input_dtype = x.dtype
    x32 = x.float()
    normalized = (x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + EPS)).to(input_dtype)
    weighted = weight.reshape(1, 1, -1) * normalized
    gate = F.silu(z.float())
    out = (weighted * gate).to(input_dtype)
    return out, weighted, gate
