"""Comparison helpers shared by the parity tests."""

from __future__ import annotations

import torch

# Tolerances stated for the hot path: bf16-activation outputs and final
# states within rtol 2e-2 / atol 2e-3; the fp32 recurrent state within 1e-4
# relative (max-abs error over max-abs value).
ACT_RTOL = 2e-2
ACT_ATOL = 2e-3
STATE_REL = 1e-4


def assert_act_close(got: torch.Tensor, want: torch.Tensor, what: str = "") -> None:
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} != {tuple(want.shape)}"
    torch.testing.assert_close(got, want, rtol=ACT_RTOL, atol=ACT_ATOL, msg=lambda m: f"{what}: {m}")


def assert_residual_close(got: torch.Tensor, want: torch.Tensor, layers: int, what: str = "") -> None:
    """An fp32 residual stream after `layers` layers that each add an fp16-rounded projection.

    Two correct implementations may round each layer's fp16 projection output
    one unit in the last place apart (their fp32 accumulation orders differ),
    so besides the activation rtol the absolute bound is one fp16 ulp
    (2^-10 relative) of the stream's largest magnitude per layer.
    """
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, f"{what}: shape {tuple(got.shape)} != {tuple(want.shape)}"
    atol = max(ACT_ATOL, layers * 2.0 ** -10 * want.abs().max().item())
    torch.testing.assert_close(got, want, rtol=ACT_RTOL, atol=atol, msg=lambda m: f"{what} (atol {atol:.3g}): {m}")


def state_rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    scale = want.abs().max().item()
    return (got - want).abs().max().item() / max(scale, 1e-30)


def assert_state_close(got: torch.Tensor, want: torch.Tensor, what: str = "", rel: float = STATE_REL) -> None:
    err = state_rel_err(got, want)
    assert err <= rel, f"{what}: state relative error {err:.3e} > {rel:.1e}"


def ring_to_window(ring: torch.Tensor, steps: int) -> torch.Tensor:
    """Conv ring [4, C] after `steps` tokens -> the reference's shifting window [1, C, 4].

    The window holds the inputs of tokens steps-4 .. steps-1; token t sits in ring slot t mod 4.
    """
    slots = [(steps - 4 + m) % 4 for m in range(4)]
    return ring[slots].transpose(0, 1).unsqueeze(0)
