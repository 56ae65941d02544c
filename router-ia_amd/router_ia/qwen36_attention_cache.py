"""Persistent attention state for Qwen3.6 decoding, on gfx950 HIP kernels.

Drop-in for v2/src/router_ia/qwen36_attention_cache.py: the same module-level
names, signatures, errors and snapshot keys, with the per-token arithmetic
moved into the HIP library (include/ria_hybrid_attn.h):

  reference (file:line)                      here
  ----------------------------------------   ----------------------------------
  AttentionState + registry  :27-134         same dataclass / functions
  _rope / _apply_rope        :137-162        ria_rope_table / ria_rope_apply
  _l2norm                    :169-173        ria_l2norm
  _causal_conv1d_step        :176-221        ria_conv1d_step (4-slot conv ring)
  _linear_stateful           :224-282        ria_rmsnorm (input norm) +
                                             ria_gdn_decode (conv + gating +
                                             l2norm + recurrence + read-out +
                                             gated RMSNorm)
  _full_stateful             :285-324        ria_rmsnorm (input norm) +
                                             ria_kv_append (k_norm, RoPE k) +
                                             ria_attn_decode (q_norm, RoPE q,
                                             gate)
  _append_full_kv            :334-373        limits on the host, then
                                             ria_kv_append into 16-bit pages
  step_attention / stats     :376-404        same

Differences a caller can observe, all inside the stated tolerances:
  * GPU KV is stored in 16-bit 16-token pages (fp16 on the step_attention
    path, whose projections are fp16 like the reference's GPU path; bf16 for
    bf16 tokens); ``full_keys[layer]`` / ``full_values[layer]`` hold
    ``PagedKVView`` objects with the reference's shape [1, Hkv, T, 256] and
    byte accounting of what is really stored.  ``.materialize()`` gathers
    the contiguous tensor.
  * The conv state is a 4-slot ring (token n in slot n mod 4) exposed with
    the reference's shape [1, conv_dim, 4]; ``conv_state_window`` returns the
    reference's shifting-window order.
  * Tensors on the CPU raise: the arithmetic exists only as HIP kernels.
    ``_append_full_kv`` on CPU tensors keeps the reference's contiguous
    storage, because the reference's limit semantics are tested with CPU
    tensors and that path only stores.

Projections and weight loading are outside the accelerated path and use
torch (``weights``), keeping the reference's dtype order (fp16 projections on
the GPU).  The norms run in the HIP library: the layer-input RMSNorm as its
own launch, q_norm / k_norm and the DeltaNet gated RMSNorm fused into the
attention launches.  ``rmsnorm`` / ``gated_rmsnorm`` remain module
attributes (the torch forms, usable on any device) as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch
import torch.nn.functional as F

from . import _native as nat
from . import kernels as K
from . import qwen36_40layer_loop as base
from . import weights as cached
from .batched_state import rope_inv_freq
from .device_utils import is_cuda
from .norms import gated_rmsnorm, rmsnorm

ROPE_THETA = 10_000_000.0
ROPE_DIM = int(base.FULL_HEAD_DIM * 0.25)
LINEAR_CONV_KERNEL = 4
# The conv keeps four positions per channel (the current token stays in the
# state after each update); only the last three are read by the next step.
LINEAR_CONV_STATE = LINEAR_CONV_KERNEL
LINEAR_CONV_DIM = base.LINEAR_KEY_DIM * 2 + base.LINEAR_VALUE_DIM

_PAGE = K.PAGE_TOKENS


class PagedKVView:
    """One layer's keys or values in the paged 16-bit cache, seen as [1, Hkv, T, 256]."""

    def __init__(self, store: "_LayerKV", which: str):
        self._store = store
        self._which = which

    @property
    def shape(self) -> torch.Size:
        return torch.Size((1, self._store.num_kv_heads, self._store.length, K.ATTN_HEAD_DIM))

    @property
    def dtype(self) -> torch.dtype:
        return self._store.dtype

    @property
    def device(self) -> torch.device:
        return self._store.device

    def numel(self) -> int:
        return self._store.num_kv_heads * self._store.length * K.ATTN_HEAD_DIM

    def element_size(self) -> int:
        return 2

    def materialize(self) -> torch.Tensor:
        k, v = self._store.gather()
        return k if self._which == "k" else v

    def __repr__(self) -> str:
        return f"PagedKVView({self._which}, shape={tuple(self.shape)}, dtype={self.dtype}, device={self.device})"


class _LayerKV:
    """Paged KV of one full-attention layer of one sequence (identity page table, grown by doubling).

    Elements are fp16 when the activations come from fp16 projections (the
    GPU path) and bf16 for bf16 activations, so appended values stay exact.
    """

    def __init__(self, num_kv_heads: int, device: torch.device, dtype: torch.dtype, pages: int = 16):
        self.num_kv_heads = num_kv_heads
        self.device = device
        self.dtype = dtype
        self.length = 0
        self._alloc(pages)

    def _alloc(self, pages: int) -> None:
        k = torch.zeros((pages, self.num_kv_heads, *K.K_TILE_SHAPE), dtype=self.dtype, device=self.device)
        v = torch.zeros((pages, self.num_kv_heads, K.ATTN_HEAD_DIM, _PAGE), dtype=self.dtype, device=self.device)
        if hasattr(self, "k"):
            used = (self.length + _PAGE - 1) // _PAGE
            k[:used].copy_(self.k[:used])
            v[:used].copy_(self.v[:used])
        self.k, self.v = k, v
        self.page_table = torch.arange(pages, dtype=torch.int32, device=self.device).reshape(1, pages)

    def reserve(self, tokens: int) -> None:
        pages = int(self.k.shape[0])
        need = (tokens + _PAGE - 1) // _PAGE
        if need > pages:
            while pages < need:
                pages *= 2
            self._alloc(pages)

    def gather(self) -> tuple[torch.Tensor, torch.Tensor]:
        return K.kv_gather(self.k, self.v, self.page_table, batch=1, start=0, count=self.length)


@dataclass
class AttentionState:
    full_keys: dict[int, Any] = field(default_factory=dict)
    full_values: dict[int, Any] = field(default_factory=dict)
    linear_states: dict[int, torch.Tensor] = field(default_factory=dict)
    linear_conv_states: dict[int, torch.Tensor] = field(default_factory=dict)
    # Zero disables a limit.  There is no sliding window: limits fail before a
    # token is added instead of changing the attention semantics.
    max_context_tokens: int = 0
    max_full_kv_bytes: int = 0
    tokens_seen: int = 0
    device: str | None = None
    # Per-layer conv step counters (ring slot of the next input) and GPU KV stores.
    conv_steps: dict[int, int] = field(default_factory=dict, repr=False)
    kv_stores: dict[int, _LayerKV] = field(default_factory=dict, repr=False)

    def reset(self) -> None:
        self.full_keys.clear()
        self.full_values.clear()
        self.linear_states.clear()
        self.linear_conv_states.clear()
        self.conv_steps.clear()
        self.kv_stores.clear()
        self.tokens_seen = 0

    def bind(self, device: str) -> None:
        if self.device != device:
            self.reset()
            self.device = device

    def configure(self, *, max_context_tokens: int = 0, max_full_kv_bytes: int = 0) -> None:
        if max_context_tokens < 0:
            raise ValueError("max_context_tokens must be non-negative")
        if max_full_kv_bytes < 0:
            raise ValueError("max_full_kv_bytes must be non-negative")
        self.max_context_tokens = int(max_context_tokens)
        self.max_full_kv_bytes = int(max_full_kv_bytes)

    def snapshot(self) -> dict[str, int | float]:
        # KV layout is (batch, kv_heads, sequence, head_dim): length at dim -2.
        full_lengths = [int(value.shape[-2]) for value in self.full_keys.values()]
        full_tokens_resident = max(full_lengths, default=0)
        full_token_entries = sum(full_lengths)
        linear_bytes = sum(int(v.numel() * v.element_size()) for v in self.linear_states.values())
        conv_bytes = sum(int(v.numel() * v.element_size()) for v in self.linear_conv_states.values())
        full_bytes = _full_kv_bytes(self)
        return {
            "tokens_seen": int(self.tokens_seen),
            "absolute_position": int(self.tokens_seen),
            "kv_start_position": max(int(self.tokens_seen) - full_tokens_resident, 0),
            "full_layers_cached": len(self.full_keys),
            "full_tokens": full_tokens_resident,
            "full_tokens_resident": full_tokens_resident,
            "full_token_entries": full_token_entries,
            "full_bytes": full_bytes,
            "max_context_tokens": int(self.max_context_tokens),
            "max_full_kv_bytes": int(self.max_full_kv_bytes),
            "linear_layers_cached": len(self.linear_states),
            "linear_bytes": linear_bytes,
            "linear_conv_layers_cached": len(self.linear_conv_states),
            "linear_conv_bytes": conv_bytes,
            "bytes": full_bytes + linear_bytes + conv_bytes,
        }


_STATES: dict[Path, AttentionState] = {}
_ACTIVE_STATES: dict[Path, AttentionState] = {}


def state_for(root: Path, device: str) -> AttentionState:
    key = Path(root).resolve()
    state = _STATES.get(key)
    if state is None:
        state = AttentionState()
        _STATES[key] = state
    state.bind(device)
    return state


def reset(root: Path) -> AttentionState:
    key = Path(root).resolve()
    state = _STATES.get(key)
    if state is None:
        state = AttentionState()
        _STATES[key] = state
    state.reset()
    return state


def activate(root: Path, state: AttentionState) -> None:
    _ACTIVE_STATES[Path(root).resolve()] = state


def deactivate(root: Path) -> None:
    _ACTIVE_STATES.pop(Path(root).resolve(), None)


def active(root: Path, device: str) -> AttentionState:
    key = Path(root).resolve()
    state = _ACTIVE_STATES.get(key)
    if state is None:
        state = state_for(key, device)
        _ACTIVE_STATES[key] = state
    state.bind(device)
    return state


# ------------------------------------------------------------------ helpers on the GPU
_INV_FREQ: dict[torch.device, torch.Tensor] = {}


def _inv_freq(device: torch.device) -> torch.Tensor:
    dev = torch.device(device)
    t = _INV_FREQ.get(dev)
    if t is None:
        t = rope_inv_freq(ROPE_THETA, ROPE_DIM).to(dev)
        _INV_FREQ[dev] = t
    return t


def _require_gpu_tensor(name: str, t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name}: the attention arithmetic runs only on a ROCm GPU; got a tensor on {t.device}")


def _rope(position: int, device: torch.device, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    if ROPE_DIM <= 0 or ROPE_DIM % 2:
        raise ValueError(f"Invalid rotary dimension: {ROPE_DIM}")
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("_rope: the attention arithmetic runs only on a ROCm GPU")
    cos, sin = K.rope_table(int(position), _inv_freq(dev))
    return cos.to(dtype), sin.to(dtype)


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def _apply_rope(q: torch.Tensor, k: torch.Tensor, position: int) -> tuple[torch.Tensor, torch.Tensor]:
    _require_gpu_tensor("_apply_rope", q)
    _require_gpu_tensor("_apply_rope", k)
    if q.dtype != torch.float32 or k.dtype != torch.float32:
        raise TypeError("_apply_rope expects fp32 q and k (the reference rotates in the query dtype, fp32)")
    inv = _inv_freq(q.device)
    return K.rope_apply(q, int(position), inv), K.rope_apply(k, int(position), inv)


def _projection(root: Path, prefix: str, device: str) -> torch.Tensor:
    return cached.cached_load_projection(root, prefix, device)


def _l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    _require_gpu_tensor("_l2norm", x)
    return K.l2norm(x, eps)


def _conv_ring(state: AttentionState, layer: int, device: torch.device) -> torch.Tensor:
    """The layer's conv ring [1, 4, conv_dim] (created zeroed, like the reference's zero state)."""
    view = state.linear_conv_states.get(int(layer))
    expected = (1, LINEAR_CONV_DIM, LINEAR_CONV_STATE)
    if view is None or view.device != device or tuple(view.shape) != expected or view.dtype != torch.bfloat16:
        ring = torch.zeros((1, LINEAR_CONV_STATE, LINEAR_CONV_DIM), dtype=torch.bfloat16, device=device)
        state.linear_conv_states[int(layer)] = ring.permute(0, 2, 1)
        state.conv_steps[int(layer)] = 0
        return ring
    return view.permute(0, 2, 1)


def conv_state_window(state: AttentionState, layer: int) -> torch.Tensor:
    """The layer's conv state in the reference's order: the last four inputs, oldest first."""
    view = state.linear_conv_states[int(layer)]
    n = state.conv_steps.get(int(layer), 0)
    slots = [(n - 4 + m) % 4 for m in range(4)]
    return view[:, :, slots]


def _causal_conv1d_step(
    state: AttentionState,
    layer: int,
    mixed_qkv: torch.Tensor,
    conv_weight: torch.Tensor,
) -> torch.Tensor:
    """One-token causal depthwise conv (kernel 4) + SiLU with the rolling conv state."""
    if mixed_qkv.ndim != 2 or mixed_qkv.shape != (1, LINEAR_CONV_DIM):
        raise ValueError(f"Unexpected mixed_qkv shape: {tuple(mixed_qkv.shape)}")
    if conv_weight.ndim != 3:
        raise ValueError(f"Unexpected conv weight shape: {tuple(conv_weight.shape)}")
    if (
        conv_weight.shape[0] != LINEAR_CONV_DIM
        or conv_weight.shape[1] != 1
        or conv_weight.shape[2] != LINEAR_CONV_KERNEL
    ):
        raise ValueError(f"Unexpected conv weight shape: {tuple(conv_weight.shape)}")
    _require_gpu_tensor("_causal_conv1d_step", mixed_qkv)
    if conv_weight.dtype != torch.bfloat16:
        raise TypeError("_causal_conv1d_step: the HIP conv computes in bf16 and needs a bf16 conv weight")
    ring = _conv_ring(state, layer, mixed_qkv.device)
    out = torch.empty_like(mixed_qkv)
    K.conv1d_step(mixed_qkv.contiguous(), conv_weight.contiguous(), ring, out,
                  conv_pos=state.conv_steps[int(layer)])
    state.conv_steps[int(layer)] += 1
    return out


_ORIGINAL_CONV_STEP = _causal_conv1d_step


def _linear_state(state: AttentionState, layer: int, device: torch.device) -> torch.Tensor:
    expected = (1, base.LINEAR_NUM_V_HEADS, 128, 128)
    s = state.linear_states.get(int(layer))
    if s is None or s.device != device or tuple(s.shape) != expected or s.dtype != torch.float32 \
            or not s.is_contiguous():
        s = torch.zeros(expected, device=device, dtype=torch.float32)
        state.linear_states[int(layer)] = s
    return s


def _input_norm(x0: torch.Tensor, weight: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """rmsnorm(x0, input_layernorm) (:227, :291) cast to the layer's compute dtype, in one launch."""
    x = x0.reshape(1, base.HIDDEN).contiguous()
    out = torch.empty((1, base.HIDDEN), device=x.device, dtype=out_dtype)
    return K.rmsnorm(x, weight.float().contiguous(), out=out)


def _linear_stateful(root: Path, layer: int, x0: torch.Tensor, device: str) -> torch.Tensor:
    state = active(root, device)
    prefix = base.layer_prefix(layer)
    if not is_cuda(device):
        raise RuntimeError("_linear_stateful: the attention arithmetic runs only on a ROCm GPU device")
    input_norm = base.load_layer_weight(root, layer, "input_layernorm.weight", device)
    # rmsnorm(x0) in fp32, then .to(bf16) (:227-229), in one launch
    h_compute = _input_norm(x0, input_norm, torch.bfloat16)

    qkv_w = _projection(root, prefix + "linear_attn.in_proj_qkv", device)
    mixed = F.linear(h_compute.to(dtype=qkv_w.dtype), qkv_w).reshape(1, LINEAR_CONV_DIM)
    conv_w = base.load_layer_weight(root, layer, "linear_attn.conv1d.weight", device)

    a_w = _projection(root, prefix + "linear_attn.in_proj_a", device)
    b_w = _projection(root, prefix + "linear_attn.in_proj_b", device)
    a_log = base.load_layer_weight(root, layer, "linear_attn.A_log", device).float().reshape(base.LINEAR_NUM_V_HEADS)
    dt_bias = base.load_layer_weight(root, layer, "linear_attn.dt_bias", device).float().reshape(
        base.LINEAR_NUM_V_HEADS)
    a_raw = F.linear(h_compute.to(dtype=a_w.dtype), a_w).reshape(1, base.LINEAR_NUM_V_HEADS).float()
    b_raw = F.linear(h_compute.to(dtype=b_w.dtype), b_w).reshape(1, base.LINEAR_NUM_V_HEADS).float()

    z_w = _projection(root, prefix + "linear_attn.in_proj_z", device)
    z = F.linear(h_compute.to(dtype=z_w.dtype), z_w).reshape(1, base.LINEAR_NUM_V_HEADS, 128)
    norm_w = base.load_layer_weight(root, layer, "linear_attn.norm.weight", device).float().contiguous()
    out_w = _projection(root, prefix + "linear_attn.out_proj", device)

    dev = x0.device
    linear_state = _linear_state(state, layer, dev)
    # the read-out leaves the kernel through the gated RMSNorm (:268-271), cast
    # to the out_proj dtype as the reference casts `gated` (:273-275)
    gated = torch.empty((1, base.LINEAR_NUM_V_HEADS, 128), device=dev, dtype=out_w.dtype)
    conv_step = globals()["_causal_conv1d_step"]
    if conv_step is _ORIGINAL_CONV_STEP:
        if conv_w.dtype != torch.bfloat16:
            raise TypeError("_linear_stateful: the HIP conv computes in bf16 and needs a bf16 conv weight")
        ring = _conv_ring(state, layer, dev)
        K.gdn_decode(mixed, linear_state, a_raw.contiguous(), b_raw.contiguous(), gated,
                     num_k_heads=base.LINEAR_NUM_K_HEADS, num_v_heads=base.LINEAR_NUM_V_HEADS, fuse_conv=True,
                     conv_weight=conv_w.contiguous(), conv_ring=ring, conv_pos=state.conv_steps[int(layer)],
                     gate_mode=nat.RIA_GATE_RAW, A_log=a_log.contiguous(), dt_bias=dt_bias.contiguous(),
                     z=z, norm_weight=norm_w)
        state.conv_steps[int(layer)] += 1
    else:
        # A replaced conv step (probes swap this module attribute): run it, then
        # the recurrence on its output.
        mixed = conv_step(state, layer, mixed, conv_w)
        K.gdn_decode(mixed.contiguous(), linear_state, a_raw.contiguous(), b_raw.contiguous(), gated,
                     num_k_heads=base.LINEAR_NUM_K_HEADS, num_v_heads=base.LINEAR_NUM_V_HEADS, fuse_conv=False,
                     gate_mode=nat.RIA_GATE_RAW, A_log=a_log.contiguous(), dt_bias=dt_bias.contiguous(),
                     z=z, norm_weight=norm_w)

    gated_compute = gated.reshape(1, base.LINEAR_VALUE_DIM)
    attn_projected = F.linear(gated_compute, out_w).float()
    return x0.reshape(1, base.HIDDEN).float() + attn_projected


def _full_store(state: AttentionState, layer: int, device: torch.device, dtype: torch.dtype) -> _LayerKV:
    store = state.kv_stores.get(int(layer))
    if store is None or store.device != device:
        store = _LayerKV(base.FULL_NUM_KV_HEADS, device, dtype)
        state.kv_stores[int(layer)] = store
        state.full_keys[int(layer)] = PagedKVView(store, "k")
        state.full_values[int(layer)] = PagedKVView(store, "v")
    return store


def _check_full_kv_limits(state: AttentionState, layer: int, append_bytes: int) -> None:
    """The reference's hard limits, checked before anything is stored (:341-363)."""
    full_k = state.full_keys.get(int(layer))
    resident_tokens = int(full_k.shape[-2]) if full_k is not None else 0
    if state.max_context_tokens and resident_tokens >= state.max_context_tokens:
        raise RuntimeError(
            "Full-attention KV context limit reached "
            f"at absolute position {state.tokens_seen}: "
            f"max_context_tokens={state.max_context_tokens}. "
            "This checkpoint runtime has no verified sliding-window policy; "
            "start a new context or raise --max-context-tokens."
        )
    projected_bytes = _full_kv_bytes(state) + append_bytes
    if state.max_full_kv_bytes and projected_bytes > state.max_full_kv_bytes:
        raise RuntimeError(
            "Full-attention KV byte budget reached "
            f"at absolute position {state.tokens_seen}: "
            f"projected={projected_bytes} bytes exceeds "
            f"max_full_kv_bytes={state.max_full_kv_bytes}. "
            "This checkpoint runtime has no verified sliding-window policy; "
            "start a new context or raise --max-full-kv-bytes."
        )


def _paged_append(state: AttentionState, layer: int, k_token: torch.Tensor, v_token: torch.Tensor,
                  position: int | None, kv_dtype: torch.dtype,
                  k_norm_weight: torch.Tensor | None = None) -> _LayerKV:
    """Append [1, Hkv, 1, 256] k/v into the layer's pages (k_norm, then RoPE on k, when position is given)."""
    store = _full_store(state, layer, k_token.device, kv_dtype)
    store.reserve(store.length + 1)
    k2 = k_token.reshape(1, base.FULL_NUM_KV_HEADS, K.ATTN_HEAD_DIM).contiguous()
    v2 = v_token.reshape(1, base.FULL_NUM_KV_HEADS, K.ATTN_HEAD_DIM).contiguous()
    if position is None:
        inv = torch.empty(0, device=k_token.device)  # rope_dim 0: k is already rotated
    else:
        inv = _inv_freq(k_token.device)
    K.kv_append(k2, v2, store.k, store.v, store.page_table, positions=int(position or 0), slots=store.length,
                inv_freq=inv, k_norm_weight=k_norm_weight)
    store.length += 1
    return store


def _full_stateful(root: Path, layer: int, x0: torch.Tensor, device: str) -> torch.Tensor:
    state = active(root, device)
    prefix = base.layer_prefix(layer)
    if not is_cuda(device):
        raise RuntimeError("_full_stateful: the attention arithmetic runs only on a ROCm GPU device")
    # RoPE uses the absolute position even if a cache policy changes how many
    # earlier entries stay resident.
    position = int(state.tokens_seen)
    input_norm = base.load_layer_weight(root, layer, "input_layernorm.weight", device)
    compute_dtype = torch.float16
    h_compute = _input_norm(x0, input_norm, compute_dtype)
    q_w = _projection(root, prefix + "self_attn.q_proj", device)
    k_w = _projection(root, prefix + "self_attn.k_proj", device)
    v_w = _projection(root, prefix + "self_attn.v_proj", device)
    q_gate = F.linear(h_compute.to(dtype=q_w.dtype), q_w).reshape(1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM * 2)
    q, gate = torch.chunk(q_gate, 2, dim=-1)
    k = F.linear(h_compute.to(dtype=k_w.dtype), k_w).reshape(1, base.FULL_NUM_KV_HEADS, base.FULL_HEAD_DIM)
    v = F.linear(h_compute.to(dtype=v_w.dtype), v_w).reshape(1, base.FULL_NUM_KV_HEADS, base.FULL_HEAD_DIM)
    # q_norm / k_norm (:302-305) run inside the append and attention launches:
    # RMSNorm in fp32, cast back to the projection dtype, then RoPE
    q_norm_w = base.load_layer_weight(root, layer, "self_attn.q_norm.weight", device).float().contiguous()
    k_norm_w = base.load_layer_weight(root, layer, "self_attn.k_norm.weight", device).float().contiguous()
    q = q.contiguous()
    k = k.contiguous()
    v = v.float().contiguous()

    _check_full_kv_limits(state, layer, append_bytes=2 * base.FULL_NUM_KV_HEADS * base.FULL_HEAD_DIM * 2)
    store = _paged_append(state, layer, k, v, position, torch.float16, k_norm_weight=k_norm_w)
    attn = _attend(store, q, gate.contiguous(), position, q_norm_weight=q_norm_w)
    if attn.shape != (1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM):
        raise RuntimeError(f"Unexpected full-attention output shape: {tuple(attn.shape)}")
    attn_flat = attn.reshape(1, base.FULL_Q_DIM).to(dtype=compute_dtype)
    out_w = _projection(root, prefix + "self_attn.o_proj", device)
    attn_projected = F.linear(attn_flat.to(dtype=out_w.dtype), out_w).float()
    return x0.reshape(1, base.HIDDEN).float() + attn_projected


def _attend(store: _LayerKV, q: torch.Tensor, gate: torch.Tensor, position: int,
            q_norm_weight: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(RoPE(q_norm(q)) K^T / 16) V * sigmoid(gate) over the store's resident tokens (fp32 out)."""
    dev = q.device
    ctx = store.length
    pages_cap = int(store.page_table.shape[1]) * _PAGE
    split = K.attn_decode_split_tokens(base.FULL_NUM_KV_HEADS, [ctx])
    ws = torch.empty(K.attn_decode_workspace_bytes(1, base.FULL_NUM_HEADS, base.FULL_NUM_KV_HEADS, max(ctx, 1),
                                                   split), dtype=torch.uint8, device=dev)
    out = torch.empty((1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM), dtype=torch.float32, device=dev)
    K.attn_decode(q, gate, store.k, store.v, store.page_table, out, positions=int(position), ctx_lens=ctx,
                  max_ctx=min(ctx, pages_cap), inv_freq=_inv_freq(dev), scale=base.FULL_HEAD_DIM ** -0.5,
                  workspace=ws, split_tokens=split, q_norm_weight=q_norm_weight)
    return out


def _full_kv_bytes(state: AttentionState) -> int:
    return sum(
        int(tensor.numel() * tensor.element_size())
        for tensor in [*state.full_keys.values(), *state.full_values.values()]
    )


def _append_full_kv(
    state: AttentionState,
    layer: int,
    k_token: torch.Tensor,
    v_token: torch.Tensor,
) -> tuple[Any, Any]:
    """Append one (already rotated) full-attention token after enforcing the hard limits."""
    if k_token.device.type == "cuda":
        # Budgets count what the cache stores: 16-bit elements on the GPU.
        _check_full_kv_limits(state, layer, append_bytes=2 * (k_token.numel() + v_token.numel()))
        kv_dtype = torch.bfloat16 if k_token.dtype == torch.bfloat16 else torch.float16
        _paged_append(state, layer, k_token, v_token, None, kv_dtype)
        return state.full_keys[int(layer)], state.full_values[int(layer)]
    append_bytes = int(k_token.numel() * k_token.element_size()) + int(v_token.numel() * v_token.element_size())
    _check_full_kv_limits(state, layer, append_bytes)
    full_k = state.full_keys.get(int(layer))
    full_v = state.full_values.get(int(layer))
    if full_k is None or full_v is None or isinstance(full_k, PagedKVView) or full_k.device != k_token.device:
        full_k = k_token.detach()
        full_v = v_token.detach()
    else:
        full_k = torch.cat((full_k, k_token.detach()), dim=2)
        full_v = torch.cat((full_v, v_token.detach()), dim=2)
    state.full_keys[int(layer)] = full_k
    state.full_values[int(layer)] = full_v
    return full_k, full_v


def step_attention(root: Path, layer: int, x0: torch.Tensor, device: str) -> torch.Tensor:
    if base.attention_type(root, layer) == "linear_attention":
        return _linear_stateful(root, layer, x0, device)
    return _full_stateful(root, layer, x0, device)


def stats(root: Path) -> dict[str, int | float]:
    state = _STATES.get(Path(root).resolve())
    return (
        state.snapshot()
        if state is not None
        else {
            "tokens_seen": 0,
            "absolute_position": 0,
            "kv_start_position": 0,
            "full_layers_cached": 0,
            "full_tokens": 0,
            "full_tokens_resident": 0,
            "full_token_entries": 0,
            "full_bytes": 0,
            "max_context_tokens": 0,
            "max_full_kv_bytes": 0,
            "linear_layers_cached": 0,
            "linear_bytes": 0,
            "linear_conv_layers_cached": 0,
            "linear_conv_bytes": 0,
            "bytes": 0,
        }
    )
