"""CPU restatement of router-ia's stateful hybrid-attention arithmetic.

TEST INFRASTRUCTURE ONLY.  This module is the parity oracle: only tests/,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker / the timed CPU baseline.  Nothing in the
``router_ia`` package imports it.

Every function restates one piece of v2/src/router_ia/qwen36_attention_cache.py
with the same torch ops, op order and dtypes as the reference's CPU path
(fp32 compute, conv in the bf16 conv-weight dtype, fp32 KV), so that rounding
matches the reference on the same inputs.  The reference works on one
sequence (batch 1); ``*_batched`` helpers loop over sequences.

Pinning (tests/test_oracle_*.py): each function is checked against an
independent float64 brute force (oracle/fp64.py), closed forms and
invariants, torch library routines (conv1d, scaled_dot_product_attention),
the transformers 5.15.0 functions the reference itself defers to, and the
committed fixtures under tests/golden/.  The layer composites
(linear_layer_step, full_layer_step) are checked against transformers'
Qwen3.5-MoE GatedDeltaNet and attention modules driven as cached one-token
decodes, and their GPU-path casts against the reference's dtype order
(tests/test_oracle_composites.py).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

ROPE_THETA = 10_000_000.0          # qwen36_attention_cache.py:17
FULL_HEAD_DIM = 256                # qwen36_40layer_loop.py:44
ROPE_DIM = int(FULL_HEAD_DIM * 0.25)  # qwen36_attention_cache.py:18
CONV_KERNEL = 4                    # :19
CONV_STATE = CONV_KERNEL           # :23
NUM_K_HEADS = 16                   # qwen36_40layer_loop.py:37-38
NUM_V_HEADS = 32
HEAD_DIM = 128
KEY_DIM = NUM_K_HEADS * HEAD_DIM
VALUE_DIM = NUM_V_HEADS * HEAD_DIM
CONV_DIM = KEY_DIM * 2 + VALUE_DIM  # :24
FULL_NUM_HEADS = 16                # qwen36_40layer_loop.py:41-47
FULL_NUM_KV_HEADS = 2
FULL_NUM_KV_GROUPS = FULL_NUM_HEADS // FULL_NUM_KV_HEADS
EPS = 1e-6


# ----------------------------------------------------------------------------- RoPE
def rope(position: int, dtype: torch.dtype = torch.float32, rope_dim: int = ROPE_DIM,
         theta: float = ROPE_THETA) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:137-146 (_rope)."""
    if rope_dim <= 0 or rope_dim % 2:
        raise ValueError(f"Invalid rotary dimension: {rope_dim}")
    inv_freq = 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim))
    angles = float(position) * inv_freq
    emb = torch.cat((angles, angles), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def inv_freq(rope_dim: int = ROPE_DIM, theta: float = ROPE_THETA) -> torch.Tensor:
    """The inv_freq vector inside rope() (qwen36_attention_cache.py:140-143)."""
    return 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """qwen36_attention_cache.py:149-151."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(q: torch.Tensor, k: torch.Tensor, position: int,
               rope_dim: int = ROPE_DIM) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:154-162 (_apply_rope); q, k [..., head_dim]."""
    cos, sin = rope(position, q.dtype, rope_dim)
    q_rot, q_pass = q[..., :rope_dim], q[..., rope_dim:]
    k_rot, k_pass = k[..., :rope_dim], k[..., rope_dim:]
    q_rot = q_rot * cos + rotate_half(q_rot) * sin
    k_rot = k_rot * cos + rotate_half(k_rot) * sin
    return torch.cat((q_rot, q_pass), dim=-1), torch.cat((k_rot, k_pass), dim=-1)


def l2norm(x: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """qwen36_attention_cache.py:169-173 (_l2norm)."""
    x = x.float()
    inv_norm = torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)
    return x * inv_norm


# ----------------------------------------------------------------------------- conv
def causal_conv1d_step(conv_state: torch.Tensor | None, mixed_qkv: torch.Tensor,
                       conv_weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:176-221 (_causal_conv1d_step) for one sequence.

    mixed_qkv [1, C]; conv_weight [C, 1, 4]; conv_state [1, C, 4] in the conv
    dtype or None (zero-initialised).  Returns (out [1, C] in mixed_qkv's dtype,
    new conv state).
    """
    channels = int(mixed_qkv.shape[-1])
    conv_dtype = conv_weight.dtype
    mixed = mixed_qkv.to(dtype=conv_dtype).reshape(1, channels, 1)
    if conv_state is None or tuple(conv_state.shape) != (1, channels, CONV_STATE):
        conv_state = torch.zeros((1, channels, CONV_STATE), dtype=conv_dtype)
    history = torch.cat((conv_state, mixed), dim=-1)
    new_state = history[:, :, -CONV_STATE:].clone()
    out = F.conv1d(history, conv_weight, bias=None, stride=1, padding=0, dilation=1, groups=channels)
    out = F.silu(out[:, :, -1:])
    return out[:, :, 0].to(dtype=mixed_qkv.dtype), new_state


# ----------------------------------------------------------------------------- DeltaNet
def gating(a_raw: torch.Tensor, b_raw: torch.Tensor, a_log: torch.Tensor,
           dt_bias: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:244-249: beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias)."""
    beta = torch.sigmoid(b_raw.float())
    g = -torch.exp(a_log.float()) * F.softplus(a_raw.float() + dt_bias.float())
    return beta, g


def split_qkv(mixed: torch.Tensor, num_k_heads: int = NUM_K_HEADS,
              num_v_heads: int = NUM_V_HEADS) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:237-240: split, then QK head h//2 serves V heads h."""
    kd = num_k_heads * HEAD_DIM
    q, k, v = torch.split(mixed, [kd, kd, num_v_heads * HEAD_DIM], dim=-1)
    rep = num_v_heads // num_k_heads
    q = q.reshape(1, num_k_heads, HEAD_DIM).repeat_interleave(rep, dim=1)
    k = k.reshape(1, num_k_heads, HEAD_DIM).repeat_interleave(rep, dim=1)
    v = v.reshape(1, num_v_heads, HEAD_DIM)
    return q, k, v


def gated_delta_step(linear_state: torch.Tensor | None, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     beta: torch.Tensor, g: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:250-266 for one sequence.

    q, k, v [1, Hv, 128] (post-conv, GQA-expanded); beta, g [1, Hv].
    Returns (attn [1, Hv, 128] fp32, new state [1, Hv, 128, 128] fp32).
    """
    num_v_heads = int(v.shape[1])
    decay = torch.exp(g)
    q = l2norm(q)
    q = q * (128 ** -0.5)
    k = l2norm(k)
    shape = (1, num_v_heads, 128, 128)
    if linear_state is None or tuple(linear_state.shape) != shape:
        linear_state = torch.zeros(shape, dtype=torch.float32)
    linear_state = linear_state * decay.unsqueeze(-1).unsqueeze(-1)
    retrieved = (linear_state * k.unsqueeze(-1)).sum(dim=-2)
    delta = (v.float() - retrieved) * beta.unsqueeze(-1)
    linear_state = linear_state + k.unsqueeze(-1) * delta.unsqueeze(-2)
    attn = (linear_state * q.unsqueeze(-1)).sum(dim=-2)
    return attn, linear_state


def linear_decode_step(conv_state: torch.Tensor | None, linear_state: torch.Tensor | None,
                       mixed_qkv: torch.Tensor, conv_weight: torch.Tensor, beta: torch.Tensor, g: torch.Tensor,
                       num_k_heads: int = NUM_K_HEADS, num_v_heads: int = NUM_V_HEADS):
    """qwen36_attention_cache.py:235-266: conv step, split, recurrence and read-out.

    mixed_qkv [1, conv_dim] (any dtype; the reference CPU path hands fp32).
    Returns (attn [1, Hv, 128], conv_state, linear_state).
    """
    mixed, conv_state = causal_conv1d_step(conv_state, mixed_qkv, conv_weight)
    q, k, v = split_qkv(mixed, num_k_heads, num_v_heads)
    attn, linear_state = gated_delta_step(linear_state, q, k, v, beta, g)
    return attn, conv_state, linear_state


# ----------------------------------------------------------------------------- full attention
def full_kv_bytes(keys: list[torch.Tensor], values: list[torch.Tensor]) -> int:
    """qwen36_attention_cache.py:327-331."""
    return sum(int(t.numel() * t.element_size()) for t in [*keys, *values])


def append_full_kv(full_k: torch.Tensor | None, full_v: torch.Tensor | None, k_token: torch.Tensor,
                   v_token: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen36_attention_cache.py:365-370: contiguous append along the sequence dim."""
    if full_k is None or full_v is None:
        return k_token.detach(), v_token.detach()
    return torch.cat((full_k, k_token.detach()), dim=2), torch.cat((full_v, v_token.detach()), dim=2)


def full_decode_step(full_k: torch.Tensor | None, full_v: torch.Tensor | None, q: torch.Tensor,
                     k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor, position: int,
                     num_kv_groups: int = FULL_NUM_KV_GROUPS):
    """qwen36_attention_cache.py:304-317 for one sequence, after the projections and norms.

    q, gate [1, Hq, 256]; k, v [1, Hkv, 256].  RoPE at `position`, append
    (fp32 KV like the reference CPU path), GQA expansion, softmax attention
    over every resident token, then attn * sigmoid(gate).
    Returns (out [1, Hq, 256] fp32, full_k, full_v).
    """
    q = q.float().unsqueeze(2)
    k = k.float().unsqueeze(2)
    q, k_token = apply_rope(q, k, position)
    v_token = v.float().unsqueeze(2)
    full_k, full_v = append_full_kv(full_k, full_v, k_token, v_token)
    k_expanded = full_k.repeat_interleave(num_kv_groups, dim=1).float()
    v_expanded = full_v.repeat_interleave(num_kv_groups, dim=1).float()
    q_now = q.squeeze(2)
    scores = torch.einsum("bhd,bhld->bhl", q_now, k_expanded) * (FULL_HEAD_DIM ** -0.5)
    attn_weights = torch.softmax(scores, dim=-1)
    attn = torch.einsum("bhl,bhld->bhd", attn_weights, v_expanded)
    attn = attn * torch.sigmoid(gate.float())
    return attn, full_k, full_v


def attention_over_cache(q_rot: torch.Tensor, full_k: torch.Tensor, full_v: torch.Tensor,
                         gate: torch.Tensor, num_kv_groups: int = FULL_NUM_KV_GROUPS) -> torch.Tensor:
    """The attention half of full_decode_step (:309-317) over an existing cache.

    q_rot [1, Hq, 256] (already rotated); full_k/full_v [1, Hkv, T, 256].
    """
    k_expanded = full_k.repeat_interleave(num_kv_groups, dim=1).float()
    v_expanded = full_v.repeat_interleave(num_kv_groups, dim=1).float()
    scores = torch.einsum("bhd,bhld->bhl", q_rot.float(), k_expanded) * (FULL_HEAD_DIM ** -0.5)
    attn_weights = torch.softmax(scores, dim=-1)
    attn = torch.einsum("bhl,bhld->bhd", attn_weights, v_expanded)
    return attn * torch.sigmoid(gate.float())


def attention_over_cache_grouped(q_rot: torch.Tensor, full_k: torch.Tensor, full_v: torch.Tensor,
                                 gate: torch.Tensor, num_kv_groups: int = FULL_NUM_KV_GROUPS) -> torch.Tensor:
    """attention_over_cache with the GQA mapping as a grouped product instead of the 8x expansion.

    Query head h reads KV head h // num_kv_groups (qwen36_attention_cache.py:309-310,
    ``repeat_interleave`` along the head dim), so the expanded einsum equals a
    product of each KV head's K/V with its group of query rows; the scores,
    softmax, P V and gate follow :312-317 in fp32.  Used where the expanded
    copy of a long cache would be too large (every row of a 128-sequence
    batch).  q_rot [1, Hq, 256]; full_k/full_v [1, Hkv, T, 256].
    """
    hq = q_rot.shape[1]
    hkv = full_k.shape[1]
    assert hq == hkv * num_kv_groups
    q = q_rot.float().reshape(hkv, num_kv_groups, FULL_HEAD_DIM)
    k = full_k[0].float()
    v = full_v[0].float()
    scores = torch.bmm(q, k.transpose(1, 2).contiguous()) * (FULL_HEAD_DIM ** -0.5)  # [Hkv, G, T]
    attn_weights = torch.softmax(scores, dim=-1)
    attn = torch.bmm(attn_weights, v).reshape(1, hq, FULL_HEAD_DIM)
    return attn * torch.sigmoid(gate.float())


def full_decode_step_grouped(full_k: torch.Tensor | None, full_v: torch.Tensor | None, q: torch.Tensor,
                             k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor, position: int):
    """full_decode_step (:304-317) with attention_over_cache_grouped for the attention half."""
    q = q.float().unsqueeze(2)
    k = k.float().unsqueeze(2)
    q, k_token = apply_rope(q, k, position)
    full_k, full_v = append_full_kv(full_k, full_v, k_token, v.float().unsqueeze(2))
    return attention_over_cache_grouped(q.squeeze(2), full_k, full_v, gate), full_k, full_v


# ----------------------------------------------------------------------------- batched drivers
class SequenceState:
    """Per-sequence attention state of the oracle (the reference AttentionState's tensors)."""

    def __init__(self):
        self.conv: dict[int, torch.Tensor] = {}
        self.linear: dict[int, torch.Tensor] = {}
        self.keys: dict[int, torch.Tensor] = {}
        self.values: dict[int, torch.Tensor] = {}
        self.tokens_seen = 0


def linear_step_batched(states: list[SequenceState], layer: int, mixed_qkv: torch.Tensor,
                        conv_weight: torch.Tensor, beta: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """linear_decode_step for each sequence row; mixed_qkv [B, conv_dim], beta/g [B, Hv]."""
    outs = []
    for b, st in enumerate(states):
        attn, st.conv[layer], st.linear[layer] = linear_decode_step(
            st.conv.get(layer), st.linear.get(layer), mixed_qkv[b:b + 1], conv_weight, beta[b:b + 1], g[b:b + 1])
        outs.append(attn)
    return torch.cat(outs, dim=0)


def full_step_batched(states: list[SequenceState], layer: int, q: torch.Tensor, k: torch.Tensor,
                      v: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """full_decode_step for each row at its own tokens_seen; q/gate [B, Hq, 256], k/v [B, Hkv, 256]."""
    outs = []
    for b, st in enumerate(states):
        out, st.keys[layer], st.values[layer] = full_decode_step(
            st.keys.get(layer), st.values.get(layer), q[b:b + 1], k[b:b + 1], v[b:b + 1], gate[b:b + 1],
            st.tokens_seen)
        outs.append(out)
    return torch.cat(outs, dim=0)


# ----------------------------------------------------------------------------- layer composites
def rmsnorm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """v2/src/router_ia/qwen36_op_probe.py:55-67: fp32 RMSNorm with (1 + w), cast back to x's dtype."""
    x32 = x.float()
    out = x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + EPS)
    return (out * (1.0 + weight.float())).to(x.dtype)


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """v2/src/router_ia/qwen36_gated_norm_probe.py:19-36 (first output)."""
    x32 = x.float()
    normalized = (x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + EPS)).to(x.dtype)
    weighted = weight.reshape(1, 1, -1) * normalized
    return (weighted * F.silu(z.float())).to(x.dtype)


def layer_compute_dtype(kind: str, gpu_dtypes: bool) -> torch.dtype:
    """The dtype the normed input h is cast to before a layer's projections.

    qwen36_attention_cache.py:229-230 (DeltaNet: bf16 on the GPU path) and
    :293-294 (attention: fp16 on the GPU path); fp32 on the CPU path.
    """
    if not gpu_dtypes:
        return torch.float32
    return torch.bfloat16 if kind == "linear" else torch.float16


def linear_layer_step(w: dict[str, torch.Tensor], st: SequenceState, layer: int, x0: torch.Tensor,
                      gpu_dtypes: bool = False) -> torch.Tensor:
    """qwen36_attention_cache.py:224-282 for one token of one sequence (projections included).

    w holds the layer's tensors under their checkpoint suffixes.  With
    gpu_dtypes the reference's CUDA-path casts are applied (bf16 h, fp16
    projections, :229-233); otherwise its CPU path (fp32).
    """
    proj = (lambda t: t.to(torch.float16)) if gpu_dtypes else (lambda t: t.float())
    h = rmsnorm(x0, w["input_layernorm.weight"])
    h_c = h.to(layer_compute_dtype("linear", gpu_dtypes))
    qkv_w = proj(w["linear_attn.in_proj_qkv.weight"])
    mixed = F.linear(h_c.to(qkv_w.dtype), qkv_w).reshape(1, CONV_DIM)
    mixed, st.conv[layer] = causal_conv1d_step(st.conv.get(layer), mixed, w["linear_attn.conv1d.weight"])
    q, k, v = split_qkv(mixed)
    a_w, b_w = proj(w["linear_attn.in_proj_a.weight"]), proj(w["linear_attn.in_proj_b.weight"])
    a_raw = F.linear(h_c.to(a_w.dtype), a_w).reshape(1, NUM_V_HEADS).float()
    b_raw = F.linear(h_c.to(b_w.dtype), b_w).reshape(1, NUM_V_HEADS).float()
    beta, g = gating(a_raw, b_raw, w["linear_attn.A_log"].reshape(1, -1), w["linear_attn.dt_bias"].reshape(1, -1))
    attn, st.linear[layer] = gated_delta_step(st.linear.get(layer), q, k, v, beta, g)
    z_w = proj(w["linear_attn.in_proj_z.weight"])
    z = F.linear(h_c.to(z_w.dtype), z_w).reshape(1, NUM_V_HEADS, 128)
    gated = gated_rmsnorm(attn, z, w["linear_attn.norm.weight"])
    out_w = proj(w["linear_attn.out_proj.weight"])
    g_c = gated.reshape(1, VALUE_DIM).to(out_w.dtype if gpu_dtypes else torch.float32)
    return x0.reshape(1, -1).float() + F.linear(g_c, out_w).float()


def full_layer_step(w: dict[str, torch.Tensor], st: SequenceState, layer: int, x0: torch.Tensor,
                    gpu_dtypes: bool = False) -> torch.Tensor:
    """qwen36_attention_cache.py:285-324 for one token of one sequence at position st.tokens_seen."""
    proj = (lambda t: t.to(torch.float16)) if gpu_dtypes else (lambda t: t.float())
    h = rmsnorm(x0, w["input_layernorm.weight"])
    h_c = h.to(layer_compute_dtype("full", gpu_dtypes))
    q_w, k_w, v_w = (proj(w[f"self_attn.{n}_proj.weight"]) for n in ("q", "k", "v"))
    q_gate = F.linear(h_c.to(q_w.dtype), q_w).reshape(1, FULL_NUM_HEADS, FULL_HEAD_DIM * 2)
    q, gate = torch.chunk(q_gate, 2, dim=-1)
    k = F.linear(h_c.to(k_w.dtype), k_w).reshape(1, FULL_NUM_KV_HEADS, FULL_HEAD_DIM)
    v = F.linear(h_c.to(v_w.dtype), v_w).reshape(1, FULL_NUM_KV_HEADS, FULL_HEAD_DIM)
    q = rmsnorm(q, w["self_attn.q_norm.weight"]).float()
    k = rmsnorm(k, w["self_attn.k_norm.weight"]).float()
    attn, st.keys[layer], st.values[layer] = full_decode_step(st.keys.get(layer), st.values.get(layer), q, k,
                                                              v.float(), gate, st.tokens_seen)
    o_w = proj(w["self_attn.o_proj.weight"])
    a_c = attn.reshape(1, -1).to(o_w.dtype if gpu_dtypes else torch.float32)
    return x0.reshape(1, -1).float() + F.linear(a_c, o_w).float()


# ----------------------------------------------------------------------------- FP8 projections
FP8_BLOCK = 128  # qwen36_dequant.py:13


def dequantize_fp8_blockwise(weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """v2/src/router_ia/qwen36_dequant.py:35-58: fp32 weight times its 128x128 block's scale.

    (The reference reshapes when both dims divide by 128 and expands the
    scale grid otherwise; both give weight.float() * scale elementwise.)
    """
    out_f, in_f = weight.shape
    expanded = scale_inv.float().repeat_interleave(FP8_BLOCK, dim=0).repeat_interleave(FP8_BLOCK, dim=1)
    return weight.float() * expanded[:out_f, :in_f]


def projection_fp8(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """A projection as the reference's GPU path computes it.

    The FP8 weight is dequantised once and cast to fp16
    (qwen36_cached_loop.py:537-542); F.linear then multiplies the fp16
    activation by it (qwen36_attention_cache.py:232-247) with fp32
    accumulation, returning fp16.
    """
    w16 = dequantize_fp8_blockwise(weight, scale_inv).to(torch.float16)
    return F.linear(x.to(torch.float16).float(), w16.float()).to(torch.float16)
