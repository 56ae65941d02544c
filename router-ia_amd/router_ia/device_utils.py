"""Device parsing helpers (same contract as v2/src/router_ia/device_utils.py)."""

from __future__ import annotations

import argparse

import torch

DeviceLike = str | torch.device


def parse_device(value: str) -> torch.device:
    """Parse a PyTorch device string, keeping an optional device index."""
    try:
        return torch.device(value)
    except (RuntimeError, TypeError) as exc:
        raise argparse.ArgumentTypeError(f"invalid PyTorch device: {value!r}") from exc


def is_cuda(device: DeviceLike) -> bool:
    """True for any GPU device (ROCm devices use the ``cuda`` type in PyTorch)."""
    return torch.device(device).type == "cuda"


def is_cpu(device: DeviceLike) -> bool:
    return torch.device(device).type == "cpu"
