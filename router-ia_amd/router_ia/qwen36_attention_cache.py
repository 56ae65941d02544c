"""Persistent attention state for Qwen3.6 decoding, on gfx950 HIP kernels.

Drop-in for v2/src/router_ia/qwen36_attention_cache.py: the same module-level
names, signatures, errors, snapshot keys and state dicts, with the per-token
arithmetic moved into the HIP library (include/ria_hybrid_attn.h):

  reference (file:line)                      here
  ----------------------------------------   ----------------------------------
  AttentionState + registry  :27-134         same dataclass / functions
  _rope / _apply_rope        :137-162        ria_rope_table / ria_rope_apply
  _l2norm                    :169-173        ria_l2norm
  _causal_conv1d_step        :176-221        ria_conv1d_window_step
  _linear_stateful           :224-282        ria_rmsnorm (input norm) +
                                             ria_gdn_decode_ex (conv + gating +
                                             l2norm + recurrence + read-out +
                                             gated RMSNorm)
  _full_stateful             :285-324        ria_rmsnorm (input norm) +
                                             ria_kv_append (k_norm, RoPE k) +
                                             ria_attn_decode (q_norm, RoPE q,
                                             gate)
  _append_full_kv            :334-373        limits on the host, then
                                             ria_kv_append into 16-bit pages
  step_attention / stats     :376-404        same
  rmsnorm / gated_rmsnorm    qwen36_op_probe.py:55-67,
                             qwen36_gated_norm_probe.py:19-36
                                             ria_rmsnorm / ria_gated_rmsnorm

The state dicts hold what the reference holds:
  * ``linear_states[layer]``: a new fp32 [1, 32, 128, 128] tensor per step
    (the kernel reads the dict's tensor and writes the next one).
  * ``linear_conv_states[layer]``: the conv-weight-dtype (bf16) window
    [1, conv_dim, 4] of the last four inputs, oldest first, a new tensor per
    step.
  * ``full_keys[layer]`` / ``full_values[layer]``: [1, Hkv, T, 256] tensors in
    the dtype of the appended tokens (fp32 on the step path), read out of
    the layer's 16-bit KV pages when used (``PagedKVTensor``).  Their
    ``numel() * element_size()`` is what the reference's tensors would
    occupy, so the byte budget and ``snapshot()`` count exactly as in the
    reference; ``paged_kv_bytes()`` gives the bytes the pages really use.
A tensor a caller stores into one of the dicts is what the next step reads.

Module attributes the reference's probes replace are looked up at call time:
``rmsnorm``, ``gated_rmsnorm``, ``_l2norm``, ``_apply_rope``,
``_causal_conv1d_step``, ``_append_full_kv`` and ``_projection``, and the
``torch.einsum`` / ``torch.softmax`` of the module's ``torch``.  While all of
them are the originals, a layer runs its fused launches; once one is
replaced, that layer runs the reference's sequence of calls through the
module attributes, with the HIP kernels for what remains (with einsum or
softmax replaced, the attention itself is the reference's torch sequence
over the cache, so the replacements see its operands).

The kernels attend over 16-bit pages (fp16 for the fp32 and fp16 tokens of
the step path, bf16 for bf16 tokens): attention outputs differ from the
reference's fp32 cache within the stated tolerances, while the dicts read
fp32 keys and values back exactly as appended.  Tensors on the CPU raise: the
arithmetic exists only as HIP kernels.  ``_append_full_kv`` on CPU tensors
keeps the reference's contiguous storage, because the reference's limit
semantics are tested with CPU tensors and that path only stores.

Projections and weight loading are outside the accelerated path and use
torch (``weights``), keeping the reference's dtype order (fp16 projections on
the GPU).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch
import torch.nn.functional as F
from torch.utils._pytree import tree_map

from . import _native as nat
from . import kernels as K
from . import qwen36_40layer_loop as base
from . import weights as cached
from .batched_state import rope_inv_freq

ROPE_THETA = 10_000_000.0
ROPE_DIM = int(base.FULL_HEAD_DIM * 0.25)
LINEAR_CONV_KERNEL = 4
# The conv keeps four positions per channel (the current token stays in the
# state after each update); only the last three are read by the next step.
LINEAR_CONV_STATE = LINEAR_CONV_KERNEL
LINEAR_CONV_DIM = base.LINEAR_KEY_DIM * 2 + base.LINEAR_VALUE_DIM

_PAGE = K.PAGE_TOKENS
NORM_EPS = 1e-6


def _on_gpu(device: str | torch.device) -> bool:
    """True for a ROCm GPU device (PyTorch names it ``cuda``)."""
    return torch.device(device).type == "cuda"


class PagedKVTensor(torch.Tensor):
    """Keys or values [1, Hkv, T, 256] of one layer, read out of its KV pages when used.

    Shape, dtype, device and ``requires_grad`` (False: the cache is detached,
    :365-372) are known without touching the pages; any other use (``detach``,
    ``float``, indexing, arithmetic, comparisons) reads the first T tokens in
    logical order (fp32 tokens from the copies kept as appended, others out
    of the pages with ria_kv_gather) in the tensor's dtype.
    Pages only grow, so a tensor taken before later appends keeps reading
    the T tokens it was created with.
    """

    @staticmethod
    def __new__(cls, store: "_LayerKV", which: str, length: int):
        shape = (1, store.num_kv_heads, int(length), K.ATTN_HEAD_DIM)
        t = torch.Tensor._make_wrapper_subclass(cls, shape, dtype=store.dtype, device=store.device,
                                                requires_grad=False)
        t._store = store
        t._which = which
        t._length = int(length)
        return t

    def __init__(self, store: "_LayerKV", which: str, length: int):
        super().__init__()

    __torch_function__ = torch._C._disabled_torch_function_impl

    def materialize(self) -> torch.Tensor:
        """The contiguous [1, Hkv, T, 256] tensor, in this tensor's dtype."""
        k, v = self._store.gather(self._length)
        return (k if self._which == "k" else v).to(self.dtype)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        def unwrap(x):
            return x.materialize() if isinstance(x, PagedKVTensor) else x

        return func(*tree_map(unwrap, args), **tree_map(unwrap, kwargs or {}))

    def __repr__(self) -> str:
        return f"PagedKVTensor({self.materialize()!r})"


class _LayerKV:
    """Paged KV of one full-attention layer of one sequence (identity page table, grown by doubling).

    ``dtype`` is the dtype of the appended tokens, in which the dict tensors
    report and materialise; the pages hold bf16 for bf16 tokens and fp16
    otherwise (fp16 keeps the fp16 projection outputs of the GPU path exact).
    fp32 tokens (the step path's, as the reference appends them, :306-307)
    are also kept as they were appended, token-major [T, Hkv, 256] in
    ``k32`` / ``v32``, so the dicts read back exactly what the reference
    stores; the kernels attend over the pages.
    """

    def __init__(self, num_kv_heads: int, device: torch.device, dtype: torch.dtype, pages: int = 16):
        self.num_kv_heads = num_kv_heads
        self.device = torch.device(device)
        self.dtype = dtype
        self.page_dtype = torch.bfloat16 if dtype == torch.bfloat16 else torch.float16
        self.exact = dtype == torch.float32
        self.length = 0
        self.views: tuple[PagedKVTensor, PagedKVTensor] | None = None
        self.k32 = self.v32 = None
        self._alloc(pages)

    def _alloc(self, pages: int) -> None:
        k = torch.zeros((pages, self.num_kv_heads, *K.K_TILE_SHAPE), dtype=self.page_dtype, device=self.device)
        v = torch.zeros((pages, self.num_kv_heads, K.ATTN_HEAD_DIM, _PAGE), dtype=self.page_dtype,
                        device=self.device)
        if hasattr(self, "k"):
            used = (self.length + _PAGE - 1) // _PAGE
            k[:used].copy_(self.k[:used])
            v[:used].copy_(self.v[:used])
        self.k, self.v = k, v
        if self.exact:
            shape = (pages * _PAGE, self.num_kv_heads, K.ATTN_HEAD_DIM)
            k32 = torch.empty(shape, dtype=torch.float32, device=self.device)
            v32 = torch.empty(shape, dtype=torch.float32, device=self.device)
            if self.k32 is not None:
                k32[:self.length].copy_(self.k32[:self.length])
                v32[:self.length].copy_(self.v32[:self.length])
            self.k32, self.v32 = k32, v32
        self.page_table = torch.arange(pages, dtype=torch.int32, device=self.device).reshape(1, pages)

    def reserve(self, tokens: int) -> None:
        pages = int(self.k.shape[0])
        need = (tokens + _PAGE - 1) // _PAGE
        if need > pages:
            while pages < need:
                pages *= 2
            self._alloc(pages)

    def gather(self, count: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Tokens 0 .. count - 1 as [1, Hkv, count, 256]: the fp32 tokens as appended, else out of the pages."""
        if self.exact:
            count = int(count)
            return (self.k32[:count].transpose(0, 1).unsqueeze(0).contiguous(),
                    self.v32[:count].transpose(0, 1).unsqueeze(0).contiguous())
        return K.kv_gather(self.k, self.v, self.page_table, batch=1, start=0, count=int(count))

    def publish(self) -> tuple[PagedKVTensor, PagedKVTensor]:
        """The dict tensors of the current length (kept to recognise them on the next step)."""
        self.views = (PagedKVTensor(self, "k", self.length), PagedKVTensor(self, "v", self.length))
        return self.views

    def import_tokens(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Store [1, Hkv, T, 256] keys (already rotated) and values as tokens 0..T-1."""
        count = int(k.shape[-2])
        self.reserve(count + 1)
        if count:
            k_rows = k.reshape(self.num_kv_heads, count, K.ATTN_HEAD_DIM).transpose(0, 1).contiguous()
            v_rows = v.reshape(self.num_kv_heads, count, K.ATTN_HEAD_DIM).transpose(0, 1).contiguous()
            K.kv_append_seq(k_rows, v_rows.to(k_rows.dtype), self.k, self.v, self.page_table[0], start=0,
                            inv_freq=None)
            if self.exact:
                self.k32[:count].copy_(k_rows)
                self.v32[:count].copy_(v_rows)
        self.length = count


@dataclass
class AttentionState:
    full_keys: dict[int, torch.Tensor] = field(default_factory=dict)
    full_values: dict[int, torch.Tensor] = field(default_factory=dict)
    linear_states: dict[int, torch.Tensor] = field(default_factory=dict)
    linear_conv_states: dict[int, torch.Tensor] = field(default_factory=dict)
    # Zero disables a limit.  There is no sliding window: limits fail before a
    # token is added instead of changing the attention semantics.
    max_context_tokens: int = 0
    max_full_kv_bytes: int = 0
    tokens_seen: int = 0
    device: str | None = None
    # The KV pages behind full_keys / full_values, per layer.
    kv_stores: dict[int, _LayerKV] = field(default_factory=dict, repr=False)

    def reset(self) -> None:
        self.full_keys.clear()
        self.full_values.clear()
        self.linear_states.clear()
        self.linear_conv_states.clear()
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

    def paged_kv_bytes(self) -> int:
        """Bytes the resident keys and values occupy in their 16-bit pages (2 bytes per element; the
        fp32 copies kept for the dicts are what ``full_bytes`` counts)."""
        return sum(2 * 2 * s.num_kv_heads * s.length * K.ATTN_HEAD_DIM for s in self.kv_stores.values())


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


def _f32_weight(w: torch.Tensor) -> torch.Tensor:
    """A norm weight as the kernels take it: contiguous, 16-byte aligned fp32."""
    if w.dtype == torch.float32 and w.is_contiguous() and w.data_ptr() % 16 == 0:
        return w
    return w.float().contiguous().clone()


def rmsnorm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Qwen RMSNorm over the last dim: fp32 normalisation, (1 + w) affine, cast back to x's dtype (ria_rmsnorm).

    The reference's ``rmsnorm`` (qwen36_op_probe.py:55-67), used for the layer
    input (:227, :291) and the q / k norms (:304-305).
    """
    _require_gpu_tensor("rmsnorm", x)
    dim = int(x.shape[-1])
    rows = x.reshape(-1, dim)
    if rows.shape[0] > 1 and rows.stride(0) != dim or dim > 1 and rows.stride(1) != 1:
        rows = rows.contiguous()
    return K.rmsnorm(rows, _f32_weight(weight), eps=NORM_EPS).reshape(x.shape)


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor,
                  weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Qwen gated RMSNorm (qwen36_gated_norm_probe.py:19-36): returns (out, weighted, gate).

    ``out`` = (w * RMSNorm(x).to(x.dtype) * SiLU(z)).to(x.dtype) comes from
    ria_gated_rmsnorm; ``weighted`` and ``gate``, the intermediates the
    reference also returns, are formed with torch ops on x's device.
    """
    if x.shape != z.shape:
        raise ValueError(f"x/z shape mismatch: {tuple(x.shape)} vs {tuple(z.shape)}")
    if x.ndim != 3 or x.shape[1:] != (base.LINEAR_NUM_V_HEADS, 128):
        raise ValueError(f"Expected (batch, {base.LINEAR_NUM_V_HEADS}, 128), got {tuple(x.shape)}")
    if weight.numel() != 128:
        raise ValueError(f"Expected norm weight with 128 values, got {weight.numel()}")
    _require_gpu_tensor("gated_rmsnorm", x)
    out = K.gated_rmsnorm(x.contiguous(), z.contiguous(), _f32_weight(weight), eps=NORM_EPS)
    x32 = x.float()
    normalized = (x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + NORM_EPS)).to(x.dtype)
    weighted = weight.reshape(1, 1, 128) * normalized
    gate = F.silu(z.float())
    return out, weighted, gate


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


def _conv_window(state: AttentionState, layer: int, device: torch.device) -> torch.Tensor:
    """The layer's conv window [1, conv_dim, 4] as the kernels read it (zeros when missing, :202-205)."""
    window = state.linear_conv_states.get(int(layer))
    expected = (1, LINEAR_CONV_DIM, LINEAR_CONV_STATE)
    if window is None or window.device != device or tuple(window.shape) != expected:
        return torch.zeros(expected, dtype=torch.bfloat16, device=device)
    if window.dtype != torch.bfloat16 or not window.is_contiguous() or window.data_ptr() % 8:
        window = window.to(torch.bfloat16).contiguous().clone()
    return window


def _causal_conv1d_step(
    state: AttentionState,
    layer: int,
    mixed_qkv: torch.Tensor,
    conv_weight: torch.Tensor,
) -> torch.Tensor:
    """One-token causal depthwise conv (kernel 4) + SiLU; the layer's window moves on by one input."""
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
    window_in = _conv_window(state, layer, mixed_qkv.device)
    window_out = torch.empty_like(window_in)
    out = torch.empty_like(mixed_qkv, memory_format=torch.contiguous_format)
    K.conv1d_window_step(mixed_qkv.contiguous(), conv_weight.contiguous(), window_in, window_out, out)
    state.linear_conv_states[int(layer)] = window_out
    return out


def _linear_state(state: AttentionState, layer: int, device: torch.device) -> torch.Tensor:
    """The layer's recurrent state as the kernel reads it (zeros when missing, :256-259)."""
    expected = (1, base.LINEAR_NUM_V_HEADS, 128, 128)
    s = state.linear_states.get(int(layer))
    if s is None or s.device != device or tuple(s.shape) != expected:
        return torch.zeros(expected, device=device, dtype=torch.float32)
    if s.dtype != torch.float32 or not s.is_contiguous() or s.data_ptr() % 16:
        s = s.float().contiguous().clone()
    return s


def _input_norm(x0: torch.Tensor, weight: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """rmsnorm(x0, input_layernorm).to(out_dtype) (:227-230, :291-294).

    With the module's own ``rmsnorm`` this is one launch that writes the
    compute dtype directly; a replaced ``rmsnorm`` is called as the reference
    calls it.
    """
    norm = globals()["rmsnorm"]
    if norm is not _HIP_RMSNORM:
        return norm(x0, weight).to(dtype=out_dtype)
    x = x0.reshape(1, base.HIDDEN).contiguous()
    out = torch.empty((1, base.HIDDEN), device=x.device, dtype=out_dtype)
    return K.rmsnorm(x, _f32_weight(weight), out=out, eps=NORM_EPS)


def _linear_stateful(root: Path, layer: int, x0: torch.Tensor, device: str) -> torch.Tensor:
    state = active(root, device)
    prefix = base.layer_prefix(layer)
    if not _on_gpu(device):
        raise RuntimeError("_linear_stateful: the attention arithmetic runs only on a ROCm GPU device")
    input_norm = base.load_layer_weight(root, layer, "input_layernorm.weight", device)
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
    norm_w = base.load_layer_weight(root, layer, "linear_attn.norm.weight", device)
    out_w = _projection(root, prefix + "linear_attn.out_proj", device)

    dev = x0.device
    s_in = _linear_state(state, layer, dev)
    s_out = torch.empty_like(s_in)  # the reference stores a new state tensor every step (:261-265)
    conv_step = globals()["_causal_conv1d_step"]
    l2norm = globals()["_l2norm"]
    fused_norm = globals()["gated_rmsnorm"] is _HIP_GATED_RMSNORM
    # the read-out leaves the kernel through the gated RMSNorm (:268-271), cast
    # to the out_proj dtype as the reference casts `gated` (:273-275); with a
    # replaced gated_rmsnorm the kernel returns the fp32 read-out instead
    attn = torch.empty((1, base.LINEAR_NUM_V_HEADS, 128), device=dev,
                       dtype=out_w.dtype if fused_norm else torch.float32)
    common = dict(num_k_heads=base.LINEAR_NUM_K_HEADS, num_v_heads=base.LINEAR_NUM_V_HEADS,
                  gate_mode=nat.RIA_GATE_RAW, A_log=a_log.contiguous(), dt_bias=dt_bias.contiguous(),
                  z=z if fused_norm else None, norm_weight=_f32_weight(norm_w) if fused_norm else None)
    if conv_step is _HIP_CONV_STEP and l2norm is _HIP_L2NORM:
        if conv_w.dtype != torch.bfloat16:
            raise TypeError("_linear_stateful: the HIP conv computes in bf16 and needs a bf16 conv weight")
        window_in = _conv_window(state, layer, dev)
        window_out = torch.empty_like(window_in)
        K.gdn_decode_ex(mixed, s_in, s_out, a_raw.contiguous(), b_raw.contiguous(), attn,
                        conv_layout=nat.RIA_CONV_WINDOW, conv_weight=conv_w.contiguous(), conv_window_in=window_in,
                        conv_window_out=window_out, **common)
        state.linear_conv_states[int(layer)] = window_out
    else:
        # A replaced seam: the reference's calls in its order (:236-254), each
        # through the module attribute, then the recurrence on their results.
        mixed = conv_step(state, layer, mixed, conv_w)
        if l2norm is _HIP_L2NORM:
            K.gdn_decode_ex(mixed.contiguous(), s_in, s_out, a_raw.contiguous(), b_raw.contiguous(), attn,
                            **common)
        else:
            q, k, v = torch.split(mixed, [base.LINEAR_KEY_DIM, base.LINEAR_KEY_DIM, base.LINEAR_VALUE_DIM], dim=-1)
            q = q.reshape(1, base.LINEAR_NUM_K_HEADS, 128).repeat_interleave(2, dim=1)
            k = k.reshape(1, base.LINEAR_NUM_K_HEADS, 128).repeat_interleave(2, dim=1)
            q = l2norm(q)
            q = q * (128 ** -0.5)
            k = l2norm(k)
            qkv = torch.cat((q.reshape(1, -1).float(), k.reshape(1, -1).float(), v.reshape(1, -1).float()), dim=-1)
            K.gdn_decode_ex(qkv, s_in, s_out, a_raw.contiguous(), b_raw.contiguous(), attn,
                            qk_mode=nat.RIA_QK_NORMALIZED, **common)
    state.linear_states[int(layer)] = s_out

    if fused_norm:
        gated_compute = attn.reshape(1, base.LINEAR_VALUE_DIM)
    else:
        gated, _, _ = globals()["gated_rmsnorm"](attn, z, norm_w)
        gated_compute = gated.reshape(1, base.LINEAR_VALUE_DIM).to(dtype=out_w.dtype)
    attn_projected = F.linear(gated_compute, out_w).float()
    return x0.reshape(1, base.HIDDEN).float() + attn_projected


def _full_store(state: AttentionState, layer: int, device: torch.device, dtype: torch.dtype) -> _LayerKV:
    """The pages behind full_keys[layer] / full_values[layer].

    The dict tensors are the state: if they are not the ones the pages last
    published (a caller stored other tensors, or removed them), the pages are
    rebuilt from what the dicts hold.
    """
    key = int(layer)
    store = state.kv_stores.get(key)
    full_k, full_v = state.full_keys.get(key), state.full_values.get(key)
    if store is not None and store.device == device and store.views is not None \
            and full_k is store.views[0] and full_v is store.views[1]:
        return store
    if (full_k is None) != (full_v is None):
        raise RuntimeError(f"full_keys and full_values disagree for layer {key}")
    if full_k is not None and full_k.device == device:
        if full_k.shape != full_v.shape or full_k.dim() != 4 or full_k.shape[0] != 1 \
                or full_k.shape[1] != base.FULL_NUM_KV_HEADS or full_k.shape[-1] != K.ATTN_HEAD_DIM:
            raise RuntimeError(f"full-attention cache of layer {key} has shape {tuple(full_k.shape)}, "
                               f"expected [1, {base.FULL_NUM_KV_HEADS}, T, {K.ATTN_HEAD_DIM}]")
        store = _LayerKV(base.FULL_NUM_KV_HEADS, device, full_k.dtype)
        store.import_tokens(full_k.detach(), full_v.detach())
    else:
        store = _LayerKV(base.FULL_NUM_KV_HEADS, device, dtype)
    state.kv_stores[key] = store
    state.full_keys[key], state.full_values[key] = store.publish()
    if store.length == 0:
        # an empty cache is no entry at all in the reference (:365-367)
        del state.full_keys[key], state.full_values[key]
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
                  position: int | None, dtype: torch.dtype,
                  k_norm_weight: torch.Tensor | None = None) -> _LayerKV:
    """Append [1, Hkv, 1, 256] k/v into the layer's pages (k_norm, then RoPE on k, when position is given)."""
    store = _full_store(state, layer, k_token.device, dtype)
    store.reserve(store.length + 1)
    k2 = k_token.reshape(1, base.FULL_NUM_KV_HEADS, K.ATTN_HEAD_DIM).contiguous()
    v2 = v_token.reshape(1, base.FULL_NUM_KV_HEADS, K.ATTN_HEAD_DIM).contiguous()
    inv = None if position is None else _inv_freq(k_token.device)  # no RoPE: k is already rotated
    slot = store.length
    if store.exact and position is not None:
        # the kernel returns k after k_norm and RoPE in fp32, the token the reference stores
        K.kv_append(k2, v2, store.k, store.v, store.page_table, positions=int(position), slots=slot, inv_freq=inv,
                    k_norm_weight=k_norm_weight, k_rot_out=store.k32[slot:slot + 1])
    else:
        K.kv_append(k2, v2, store.k, store.v, store.page_table, positions=int(position or 0), slots=slot,
                    inv_freq=inv, k_norm_weight=k_norm_weight)
        if store.exact:
            store.k32[slot].copy_(k2[0])
    if store.exact:
        store.v32[slot].copy_(v2[0])
    store.length += 1
    state.full_keys[int(layer)], state.full_values[int(layer)] = store.publish()
    return store


def _full_stateful(root: Path, layer: int, x0: torch.Tensor, device: str) -> torch.Tensor:
    state = active(root, device)
    prefix = base.layer_prefix(layer)
    if not _on_gpu(device):
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
    q_norm_w = base.load_layer_weight(root, layer, "self_attn.q_norm.weight", device)
    k_norm_w = base.load_layer_weight(root, layer, "self_attn.k_norm.weight", device)
    gate = gate.contiguous()
    norm = globals()["rmsnorm"]
    rope = globals()["_apply_rope"]
    append = globals()["_append_full_kv"]

    if norm is _HIP_RMSNORM and rope is _HIP_APPLY_ROPE and append is _HIP_APPEND_FULL_KV \
            and not _attention_ops_replaced():
        # q_norm / k_norm (:302-305) and RoPE run inside the append and
        # attention launches: RMSNorm in fp32, cast back to the projection
        # dtype, then RoPE.  The tokens the reference appends are fp32 (:306-307).
        token_bytes = base.FULL_NUM_KV_HEADS * base.FULL_HEAD_DIM * 4
        _check_full_kv_limits(state, layer, append_bytes=2 * token_bytes)
        store = _paged_append(state, layer, k.contiguous(), v.float().contiguous(), position, torch.float32,
                              k_norm_weight=_f32_weight(k_norm_w))
        attn = _attend(store, q.contiguous(), gate, position, q_norm_weight=_f32_weight(q_norm_w))
    else:
        # A replaced seam: the reference's sequence (:304-308) through the
        # module attributes, then attention over the cache they produced.
        q = norm(q, q_norm_w).float().unsqueeze(2)
        k = norm(k, k_norm_w).float().unsqueeze(2)
        q, k_token = rope(q, k, position)
        v_token = v.float().unsqueeze(2)
        full_k, full_v = append(state, layer, k_token, v_token)
        if _attention_ops_replaced():
            attn = _attend_torch(full_k, full_v, q, gate)
        else:
            attn = _attend_tensors(state, layer, full_k, full_v, q.squeeze(2).contiguous(), gate)
    if attn.shape != (1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM):
        raise RuntimeError(f"Unexpected full-attention output shape: {tuple(attn.shape)}")
    attn_flat = attn.reshape(1, base.FULL_Q_DIM).to(dtype=compute_dtype)
    out_w = _projection(root, prefix + "self_attn.o_proj", device)
    attn_projected = F.linear(attn_flat.to(dtype=out_w.dtype), out_w).float()
    return x0.reshape(1, base.HIDDEN).float() + attn_projected


def _attention_ops_replaced() -> bool:
    """True while a caller has replaced ``torch.einsum`` or ``torch.softmax`` (the module's ``torch``).

    The reference's probes capture the score, softmax and P V intermediates
    by replacing them (qwen36_full_attention_residual_probe.py:104-153); a
    layer then attends through them, as the reference does.
    """
    return torch.einsum is not _TORCH_EINSUM or torch.softmax is not _TORCH_SOFTMAX


def _attend_torch(full_k: torch.Tensor, full_v: torch.Tensor, q: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """The reference's attention sequence (:309-317) over the cache tensors, through ``torch.einsum`` /
    ``torch.softmax`` as they are at call time.  Runs only while one of them is replaced."""
    k_expanded = full_k.repeat_interleave(base.FULL_NUM_KV_GROUPS, dim=1).float()
    v_expanded = full_v.repeat_interleave(base.FULL_NUM_KV_GROUPS, dim=1).float()
    q_now = q.squeeze(2)
    scores = torch.einsum("bhd,bhld->bhl", q_now, k_expanded) * (base.FULL_HEAD_DIM ** -0.5)
    attn_weights = torch.softmax(scores, dim=-1)
    attn = torch.einsum("bhl,bhld->bhd", attn_weights, v_expanded)
    if attn.shape != (1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM):
        raise RuntimeError(f"Unexpected full-attention output shape: {tuple(attn.shape)}")
    return attn * torch.sigmoid(gate.float())


def _attend(store: _LayerKV, q: torch.Tensor, gate: torch.Tensor, position: int | None,
            q_norm_weight: torch.Tensor | None = None) -> torch.Tensor:
    """softmax(q K^T / 16) V * sigmoid(gate) over the store's resident tokens (fp32 out).

    With a position, q is q_norm'd (when a weight is given) and rotated in the
    launch; without one, q arrives rotated.
    """
    dev = q.device
    ctx = store.length
    pages_cap = int(store.page_table.shape[1]) * _PAGE
    split = K.attn_decode_split_tokens(base.FULL_NUM_KV_HEADS, [ctx])
    ws = torch.empty(K.attn_decode_workspace_bytes(1, base.FULL_NUM_HEADS, base.FULL_NUM_KV_HEADS, max(ctx, 1),
                                                   split), dtype=torch.uint8, device=dev)
    out = torch.empty((1, base.FULL_NUM_HEADS, base.FULL_HEAD_DIM), dtype=torch.float32, device=dev)
    K.attn_decode(q, gate, store.k, store.v, store.page_table, out, positions=int(position or 0), ctx_lens=ctx,
                  max_ctx=min(ctx, pages_cap), inv_freq=None if position is None else _inv_freq(dev),
                  scale=base.FULL_HEAD_DIM ** -0.5, workspace=ws, split_tokens=split, q_norm_weight=q_norm_weight)
    return out


def _attend_tensors(state: AttentionState, layer: int, full_k: torch.Tensor, full_v: torch.Tensor,
                    q_rot: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Attention of the rotated q [1, Hq, 256] over the cache tensors an _append_full_kv returned (:309-317)."""
    store = state.kv_stores.get(int(layer))
    if not (store is not None and store.views is not None and full_k is store.views[0] and full_v is store.views[1]):
        if full_k.device != q_rot.device:
            raise RuntimeError(f"full-attention cache of layer {layer} is on {full_k.device}, q on {q_rot.device}")
        store = _LayerKV(base.FULL_NUM_KV_HEADS, q_rot.device, full_k.dtype)
        store.import_tokens(full_k.detach(), full_v.detach())
    return _attend(store, q_rot, gate, None)


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
) -> tuple[torch.Tensor, torch.Tensor]:
    """Append one (already rotated) full-attention token after enforcing the hard limits."""
    append_bytes = int(k_token.numel() * k_token.element_size()) + int(v_token.numel() * v_token.element_size())
    _check_full_kv_limits(state, layer, append_bytes)
    if k_token.device.type == "cuda":
        _paged_append(state, layer, k_token, v_token, None, k_token.dtype)
        return state.full_keys[int(layer)], state.full_values[int(layer)]
    full_k = state.full_keys.get(int(layer))
    full_v = state.full_values.get(int(layer))
    if full_k is None or full_v is None or full_k.device != k_token.device:
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


# The module's own forms of the replaceable seams: a layer runs fused while
# the module attributes are these objects.
_HIP_RMSNORM = rmsnorm
_HIP_GATED_RMSNORM = gated_rmsnorm
_HIP_L2NORM = _l2norm
_HIP_APPLY_ROPE = _apply_rope
_HIP_CONV_STEP = _causal_conv1d_step
_HIP_APPEND_FULL_KV = _append_full_kv
_TORCH_EINSUM = torch.einsum
_TORCH_SOFTMAX = torch.softmax
