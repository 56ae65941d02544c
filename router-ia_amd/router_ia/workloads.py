"""Seeded synthetic inputs for the hybrid-attention workloads.

Shapes are the model family's (16 QK heads x 128, 32 V heads x 128, conv over
8192 channels; full attention 16 Q / 2 KV heads x 256).  The layer-step
workloads exclude the projections (each step gets its q/k/v, gate and decay
inputs directly); ``synthetic_layer`` gives whole layers, FP8 projections
included, for the batched forward loop.

Gating inputs are drawn so that the raw-gate formula of the reference
(qwen36_attention_cache.py:242-250) reproduces the requested distributions:
    b_raw ~ N(0,1)         -> beta = sigmoid(b_raw)
    a_raw ~ N(0,1), A_log ~ U(-4,0) per head, dt_bias = 0
                           -> g = -exp(A_log) * softplus(a_raw) = -softplus(N(0,1)) * exp(U(-4,0))
"""

from __future__ import annotations

import torch

NUM_K_HEADS = 16
NUM_V_HEADS = 32
HEAD_DIM = 128
CONV_DIM = (2 * NUM_K_HEADS + NUM_V_HEADS) * HEAD_DIM
FULL_Q_HEADS = 16
FULL_KV_HEADS = 2
FULL_HEAD_DIM = 256


def _gen(seed: int, device: torch.device | str) -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(seed)
    return g


def gdn_layer_params(seed: int, device="cpu") -> dict[str, torch.Tensor]:
    """Per-layer constants: conv weight ~N(0, 0.5) bf16 [8192,1,4], A_log ~U(-4,0), dt_bias = 0."""
    g = _gen(seed, device)
    conv_weight = (torch.randn((CONV_DIM, 1, 4), generator=g, device=device) * 0.5).to(torch.bfloat16)
    a_log = torch.rand((NUM_V_HEADS,), generator=g, device=device) * 4.0 - 4.0
    dt_bias = torch.zeros((NUM_V_HEADS,), device=device)
    return {"conv_weight": conv_weight, "A_log": a_log, "dt_bias": dt_bias}


def gdn_step_inputs(seed: int, steps: int, batch: int, device="cpu") -> dict[str, torch.Tensor]:
    """Per-token inputs: mixed q|k|v bf16 ~N(0,1) [steps,B,8192], a_raw, b_raw ~N(0,1) [steps,B,32]."""
    g = _gen(seed, device)
    mixed = torch.randn((steps, batch, CONV_DIM), generator=g, device=device).to(torch.bfloat16)
    a_raw = torch.randn((steps, batch, NUM_V_HEADS), generator=g, device=device)
    b_raw = torch.randn((steps, batch, NUM_V_HEADS), generator=g, device=device)
    return {"mixed": mixed, "a_raw": a_raw, "b_raw": b_raw}


def attn_step_inputs(seed: int, steps: int, batch: int, device="cpu") -> dict[str, torch.Tensor]:
    """Per-token inputs: q, gate bf16 [steps,B,16,256]; k, v bf16 [steps,B,2,256]; all ~N(0,1)."""
    g = _gen(seed, device)
    q = torch.randn((steps, batch, FULL_Q_HEADS, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    k = torch.randn((steps, batch, FULL_KV_HEADS, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((steps, batch, FULL_KV_HEADS, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    gate = torch.randn((steps, batch, FULL_Q_HEADS, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    return {"q": q, "k": k, "v": v, "gate": gate}


def prefilled_kv(seed: int, batch: int, tokens: int, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """Resident KV content bf16 ~N(0,1) [B, 2, T, 256] (keys already positioned)."""
    g = _gen(seed, device)
    k = torch.randn((batch, FULL_KV_HEADS, tokens, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((batch, FULL_KV_HEADS, tokens, FULL_HEAD_DIM), generator=g, device=device).to(torch.bfloat16)
    return k, v


def ragged_lengths(seed: int, batch: int, lo: int, hi: int) -> list[int]:
    """Context lengths uniform in [lo, hi] (inclusive), one per sequence."""
    g = torch.Generator()
    g.manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (batch,), generator=g)]


def norm_params(seed: int, device="cpu") -> dict[str, torch.Tensor]:
    """Norm weights around the attention arithmetic, fp32 as the kernels take them.

    q_norm / k_norm [256] and the layer input norm [2048] are (1 + w) RMSNorms
    (zero-centred w ~ N(0, 0.1)); the DeltaNet gated norm [128] multiplies by
    w directly (w ~ 1 + N(0, 0.1)).  Values are bf16-representable, like a
    checkpoint's bf16 weights widened to fp32.
    """
    g = _gen(seed, device)

    def bf(t):
        return t.to(torch.bfloat16).float()

    return {
        "q_norm": bf(torch.randn((FULL_HEAD_DIM,), generator=g, device=device) * 0.1),
        "k_norm": bf(torch.randn((FULL_HEAD_DIM,), generator=g, device=device) * 0.1),
        "gated_norm": bf(1.0 + torch.randn((HEAD_DIM,), generator=g, device=device) * 0.1),
        "input_norm": bf(torch.randn((2048,), generator=g, device=device) * 0.1),
    }


def gate_z_inputs(seed: int, steps: int, batch: int, device="cpu") -> torch.Tensor:
    """Gated-norm gates z bf16 ~N(0,1) [steps, B, 32, 128] (the in_proj_z output)."""
    g = _gen(seed, device)
    return torch.randn((steps, batch, NUM_V_HEADS, HEAD_DIM), generator=g, device=device).to(torch.bfloat16)


FP8_MAX = 448.0  # largest finite float8_e4m3fn


def fp8_block_weight(seed: int, n: int, k: int, std: float = 0.02,
                     device="cpu", on_device: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """A synthetic block-FP8 projection weight: float8_e4m3fn [n, k] and fp32 scale_inv [ceil(n/128), ceil(k/128)].

    Quantised the way block-FP8 checkpoints are: per 128x128 block,
    scale_inv = max|w| / 448 and w8 = e4m3(w / scale_inv).  Drawn on the CPU
    (the values of a seed do not depend on the device) unless on_device.
    """
    gen_dev = device if on_device else "cpu"
    g = _gen(seed, gen_dev)
    w = torch.randn((n, k), generator=g, device=gen_dev) * std
    nb, kb = (n + 127) // 128, (k + 127) // 128
    pad = torch.zeros((nb * 128, kb * 128), device=gen_dev)
    pad[:n, :k] = w
    amax = pad.reshape(nb, 128, kb, 128).abs().amax(dim=(1, 3))
    del pad
    scale_inv = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (w / scale_inv.repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]).clamp(-FP8_MAX, FP8_MAX)
    return q.to(torch.float8_e4m3fn).to(device), scale_inv.float().to(device)


# (N, K) of each FP8 projection of a layer, by checkpoint name (hidden 2048;
# qwen36_attention_cache.py:232-247, 268, 295-301, 318-320)
LINEAR_PROJECTIONS = {"in_proj_qkv": (CONV_DIM, 2048), "in_proj_z": (NUM_V_HEADS * HEAD_DIM, 2048),
                      "in_proj_a": (NUM_V_HEADS, 2048), "in_proj_b": (NUM_V_HEADS, 2048),
                      "out_proj": (2048, NUM_V_HEADS * HEAD_DIM)}
FULL_PROJECTIONS = {"q_proj": (2 * FULL_Q_HEADS * FULL_HEAD_DIM, 2048), "k_proj": (FULL_KV_HEADS * FULL_HEAD_DIM, 2048),
                    "v_proj": (FULL_KV_HEADS * FULL_HEAD_DIM, 2048), "o_proj": (2048, FULL_Q_HEADS * FULL_HEAD_DIM)}


def synthetic_layer(seed: int, model_layer: int, device="cpu", on_device: bool = False) -> dict[str, torch.Tensor]:
    """One layer's weights as a checkpoint holds them, keyed by the checkpoint's suffixes.

    Model layer 4i + 3 is full attention, the others Gated DeltaNet
    (qwen36_40layer_loop.py:68-78).  Projections are block-FP8 (``<name>.weight``
    e4m3 and ``<name>.weight_scale_inv``); norm weights are fp32 holding bf16
    values; the conv weight is bf16.
    """
    norms = norm_params(seed, device)
    out = {"input_layernorm.weight": norms["input_norm"]}
    if model_layer % 4 == 3:
        for j, (name, (n, k)) in enumerate(FULL_PROJECTIONS.items()):
            w8, s = fp8_block_weight(seed * 16 + j, n, k, 0.02, device=device, on_device=on_device)
            out[f"self_attn.{name}.weight"], out[f"self_attn.{name}.weight_scale_inv"] = w8, s
        out["self_attn.q_norm.weight"] = norms["q_norm"]
        out["self_attn.k_norm.weight"] = norms["k_norm"]
    else:
        for j, (name, (n, k)) in enumerate(LINEAR_PROJECTIONS.items()):
            w8, s = fp8_block_weight(seed * 16 + j, n, k, 0.02, device=device, on_device=on_device)
            out[f"linear_attn.{name}.weight"], out[f"linear_attn.{name}.weight_scale_inv"] = w8, s
        p = gdn_layer_params(seed, device)
        out["linear_attn.conv1d.weight"] = p["conv_weight"]
        out["linear_attn.A_log"] = p["A_log"]
        out["linear_attn.dt_bias"] = p["dt_bias"]
        out["linear_attn.norm.weight"] = norms["gated_norm"]
    return out
