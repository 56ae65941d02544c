"""Typed torch-tensor wrappers over the C ABI (include/ria_hybrid_attn.h).

Each wrapper checks shapes, dtypes, devices and strides on the host, then
launches on the current HIP stream of the tensors' device.  Tensors must live
on a ROCm GPU: there is no CPU implementation behind these calls.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat

GDN_HEAD_DIM = 128
CONV_TAPS = 4
CONV_RING = 4
ATTN_HEAD_DIM = 256
PAGE_TOKENS = 16

_DTYPE_CODE = {torch.bfloat16: nat.RIA_DT_BF16, torch.float16: nat.RIA_DT_F16, torch.float32: nat.RIA_DT_F32}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported activation dtype {t.dtype}; expected bf16, fp16 or fp32") from None


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_gpu(name: str, t: torch.Tensor | None, device: torch.device | None = None) -> None:
    if t is None:
        return
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{name} is on {t.device}; the hybrid-attention kernels run only on a ROCm GPU (no CPU path)"
        )
    if device is not None and t.device != device:
        raise RuntimeError(f"{name} is on {t.device}, expected {device}")


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _rows_i32(name: str, t: torch.Tensor | int | None, batch: int, device: torch.device) -> tuple[torch.Tensor | None, int]:
    """Per-row int32 tensor or scalar -> (tensor or None, scalar)."""
    if t is None:
        return None, 0
    if isinstance(t, int):
        return None, int(t)
    _require_gpu(name, t, device)
    if t.dtype != torch.int32 or t.dim() != 1 or t.shape[0] < batch or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 vector of length >= {batch}")
    return t, 0


def _row_stride(name: str, t: torch.Tensor, batch: int, row_elems: int) -> int:
    """Row stride (elements) of a [batch, ...] tensor whose rows are contiguous."""
    flat = t.reshape(t.shape[0], -1) if t.dim() > 2 else t
    if flat.dim() != 2 or flat.shape[0] != batch or flat.shape[1] != row_elems:
        raise ValueError(f"{name} must have {batch} rows of {row_elems} elements, got {tuple(t.shape)}")
    if flat.shape[1] > 1 and flat.stride(1) != 1:
        raise ValueError(f"{name} rows must be contiguous")
    if t.dim() > 2 and not t[0].is_contiguous():
        raise ValueError(f"{name} rows must be contiguous")
    return int(flat.stride(0)) if batch > 1 else row_elems


def conv_dim(num_k_heads: int, num_v_heads: int) -> int:
    return (2 * num_k_heads + num_v_heads) * GDN_HEAD_DIM


def _norm_weight(name: str, w: torch.Tensor | None, n: int, dev: torch.device) -> ctypes.c_void_p | None:
    """A norm weight as the ABI takes it: contiguous fp32 [n] on the device (16-byte aligned)."""
    if w is None:
        return None
    _require_gpu(name, w, dev)
    if w.dtype != torch.float32 or w.numel() != n or not w.is_contiguous() or w.data_ptr() % 16:
        raise ValueError(f"{name} must be a contiguous, 16-byte aligned fp32 tensor of {n} values "
                         f"(convert the checkpoint weight with .float() once)")
    return _ptr(w)


def gdn_decode(
    mixed_qkv: torch.Tensor,
    state: torch.Tensor,
    gate_a: torch.Tensor,
    gate_b: torch.Tensor,
    out: torch.Tensor,
    *,
    num_k_heads: int,
    num_v_heads: int,
    fuse_conv: bool = True,
    conv_weight: torch.Tensor | None = None,
    conv_ring: torch.Tensor | None = None,
    conv_pos: torch.Tensor | int = 0,
    seq_slot: torch.Tensor | None = None,
    gate_mode: int = nat.RIA_GATE_PRECOMPUTED,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    z: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused conv + gated delta-rule decode step (ria_gdn_decode).

    With ``z`` ([batch, Hv, 128] or [batch, >= Hv*128] rows) and the fp32
    ``norm_weight`` [128], ``out`` receives the gated RMSNorm of the read-out
    (qwen36_attention_cache.py:268-271) instead of the read-out itself.
    """
    batch = int(mixed_qkv.shape[0])
    dev = mixed_qkv.device
    cdim = conv_dim(num_k_heads, num_v_heads)
    for name, t in (("mixed_qkv", mixed_qkv), ("state", state), ("gate_a", gate_a), ("gate_b", gate_b),
                    ("out", out), ("conv_weight", conv_weight), ("conv_ring", conv_ring), ("seq_slot", seq_slot),
                    ("A_log", A_log), ("dt_bias", dt_bias)):
        _require_gpu(name, t, dev)
    x_stride = _row_stride("mixed_qkv", mixed_qkv, batch, cdim)
    if state.dtype != torch.float32 or state.dim() != 4 or tuple(state.shape[1:]) != (num_v_heads, 128, 128) \
            or not state.is_contiguous():
        raise ValueError(f"state must be contiguous fp32 [pool, {num_v_heads}, 128, 128], got {tuple(state.shape)}")
    if seq_slot is None and state.shape[0] < batch:
        raise ValueError("state pool smaller than batch")
    if gate_a.dtype != torch.float32 or gate_b.dtype != torch.float32:
        raise ValueError("gate_a / gate_b must be fp32")
    g_stride = _row_stride("gate_a", gate_a, batch, num_v_heads)
    if _row_stride("gate_b", gate_b, batch, num_v_heads) != g_stride:
        raise ValueError("gate_a and gate_b must share a row stride")
    if tuple(out.shape) != (batch, num_v_heads, GDN_HEAD_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {num_v_heads}, 128]")
    if fuse_conv:
        if conv_weight is None or conv_ring is None:
            raise ValueError("fuse_conv needs conv_weight and conv_ring")
        _check_conv_tensors(conv_weight, conv_ring, cdim, batch if seq_slot is None else 0)
    if gate_mode == nat.RIA_GATE_RAW:
        for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
            if t is None or t.dtype != torch.float32 or t.numel() != num_v_heads or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous fp32 tensor of {num_v_heads} values")
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    pos_t, pos_s = _rows_i32("conv_pos", conv_pos, batch, dev)
    z_stride = 0
    if (z is None) != (norm_weight is None):
        raise ValueError("the gated norm needs both z and norm_weight")
    if z is not None:
        _require_gpu("z", z, dev)
        z_stride = _row_stride("z", z, batch, num_v_heads * GDN_HEAD_DIM) if z.dim() == 3 else int(z.stride(0))
        if z.dim() == 2 and (z.shape[0] != batch or z.shape[1] < num_v_heads * GDN_HEAD_DIM or z.stride(1) != 1):
            raise ValueError(f"z must have {batch} rows of >= {num_v_heads * GDN_HEAD_DIM} contiguous elements")
    w_ptr = _norm_weight("norm_weight", norm_weight, GDN_HEAD_DIM, dev)
    lib = nat.load()
    rc = lib.ria_gdn_decode(
        batch, num_k_heads, num_v_heads, _ptr(mixed_qkv), dtype_code(mixed_qkv), x_stride, int(bool(fuse_conv)),
        _ptr(conv_weight) if fuse_conv else None, _ptr(conv_ring) if fuse_conv else None, _ptr(pos_t), pos_s,
        _ptr(state), _ptr(seq_slot), _ptr(gate_a), _ptr(gate_b), g_stride, int(gate_mode),
        _ptr(A_log) if gate_mode == nat.RIA_GATE_RAW else None,
        _ptr(dt_bias) if gate_mode == nat.RIA_GATE_RAW else None,
        _ptr(out), dtype_code(out), _ptr(z), dtype_code(z) if z is not None else 0, z_stride, w_ptr, _stream(dev))
    nat.check(rc, "ria_gdn_decode")
    return out


def gdn_decode_ex(
    x: torch.Tensor,
    state_in: torch.Tensor,
    state_out: torch.Tensor,
    gate_a: torch.Tensor,
    gate_b: torch.Tensor,
    out: torch.Tensor,
    *,
    num_k_heads: int,
    num_v_heads: int,
    conv_layout: int = nat.RIA_CONV_NONE,
    conv_weight: torch.Tensor | None = None,
    conv_ring: torch.Tensor | None = None,
    conv_pos: torch.Tensor | int = 0,
    conv_window_in: torch.Tensor | None = None,
    conv_window_out: torch.Tensor | None = None,
    seq_slot: torch.Tensor | None = None,
    gate_mode: int = nat.RIA_GATE_PRECOMPUTED,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    qk_mode: int = nat.RIA_QK_RAW,
    z: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """DeltaNet decode step with a separate output state and the conv state in ring or window layout.

    ``state_out`` may be ``state_in`` (in place) or a disjoint tensor of the
    same shape.  ``conv_layout``: RIA_CONV_NONE (x already convolved),
    RIA_CONV_RING (``conv_ring`` / ``conv_pos``) or RIA_CONV_WINDOW (the
    reference's window [pool, conv_dim, 4] in ``conv_window_in``, the shifted
    one written to ``conv_window_out``).  ``qk_mode`` RIA_QK_NORMALIZED takes x
    as [B, Hv*128 q | Hv*128 k | Hv*128 v] with q, k normalised by the caller
    (ria_gdn_decode_ex).
    """
    batch = int(x.shape[0])
    dev = x.device
    cdim = conv_dim(num_k_heads, num_v_heads)
    for name, t in (("x", x), ("state_in", state_in), ("state_out", state_out), ("gate_a", gate_a),
                    ("gate_b", gate_b), ("out", out), ("conv_weight", conv_weight), ("conv_ring", conv_ring),
                    ("conv_window_in", conv_window_in), ("conv_window_out", conv_window_out),
                    ("seq_slot", seq_slot), ("A_log", A_log), ("dt_bias", dt_bias)):
        _require_gpu(name, t, dev)
    width = 3 * num_v_heads * GDN_HEAD_DIM if qk_mode == nat.RIA_QK_NORMALIZED else cdim
    x_stride = _row_stride("x", x, batch, width)
    for name, st in (("state_in", state_in), ("state_out", state_out)):
        if st.dtype != torch.float32 or st.dim() != 4 or tuple(st.shape[1:]) != (num_v_heads, 128, 128) \
                or not st.is_contiguous():
            raise ValueError(f"{name} must be contiguous fp32 [pool, {num_v_heads}, 128, 128], got {tuple(st.shape)}")
        if seq_slot is None and st.shape[0] < batch:
            raise ValueError(f"{name} pool smaller than batch")
    if state_out.data_ptr() != state_in.data_ptr() and state_out.shape[0] != state_in.shape[0]:
        raise ValueError("state_out must be state_in or a tensor of its shape")
    if gate_a.dtype != torch.float32 or gate_b.dtype != torch.float32:
        raise ValueError("gate_a / gate_b must be fp32")
    g_stride = _row_stride("gate_a", gate_a, batch, num_v_heads)
    if _row_stride("gate_b", gate_b, batch, num_v_heads) != g_stride:
        raise ValueError("gate_a and gate_b must share a row stride")
    if tuple(out.shape) != (batch, num_v_heads, GDN_HEAD_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {num_v_heads}, 128]")
    if conv_layout == nat.RIA_CONV_RING:
        if conv_weight is None or conv_ring is None:
            raise ValueError("RIA_CONV_RING needs conv_weight and conv_ring")
        _check_conv_tensors(conv_weight, conv_ring, cdim, batch if seq_slot is None else 0)
    elif conv_layout == nat.RIA_CONV_WINDOW:
        if conv_weight is None or conv_window_in is None or conv_window_out is None:
            raise ValueError("RIA_CONV_WINDOW needs conv_weight, conv_window_in and conv_window_out")
        _check_conv_window(conv_weight, conv_window_in, conv_window_out, cdim, batch if seq_slot is None else 0)
        if seq_slot is not None and {conv_window_in.shape[0], conv_window_out.shape[0]} != {state_in.shape[0]}:
            raise ValueError("with seq_slot the conv window pools must have the state pool's rows")
    elif conv_layout != nat.RIA_CONV_NONE:
        raise ValueError(f"unknown conv_layout {conv_layout}")
    if gate_mode == nat.RIA_GATE_RAW:
        for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
            if t is None or t.dtype != torch.float32 or t.numel() != num_v_heads or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous fp32 tensor of {num_v_heads} values")
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    pos_t, pos_s = _rows_i32("conv_pos", conv_pos, batch, dev)
    z_stride = 0
    if (z is None) != (norm_weight is None):
        raise ValueError("the gated norm needs both z and norm_weight")
    if z is not None:
        _require_gpu("z", z, dev)
        z_stride = _row_stride("z", z, batch, num_v_heads * GDN_HEAD_DIM)
    w_ptr = _norm_weight("norm_weight", norm_weight, GDN_HEAD_DIM, dev)

    def addr(t):
        return None if t is None else t.data_ptr()

    d = nat.GdnDecodeDesc(
        batch=batch, num_k_heads=num_k_heads, num_v_heads=num_v_heads, x=addr(x), x_dtype=dtype_code(x),
        x_row_stride=x_stride, conv_layout=int(conv_layout),
        conv_weight=addr(conv_weight) if conv_layout != nat.RIA_CONV_NONE else None,
        conv_ring=addr(conv_ring) if conv_layout == nat.RIA_CONV_RING else None, conv_pos=addr(pos_t),
        conv_pos_scalar=pos_s,
        conv_window_in=addr(conv_window_in) if conv_layout == nat.RIA_CONV_WINDOW else None,
        conv_window_out=addr(conv_window_out) if conv_layout == nat.RIA_CONV_WINDOW else None,
        state_in=addr(state_in), state_out=addr(state_out), seq_slot=addr(seq_slot), gate_a=addr(gate_a),
        gate_b=addr(gate_b), gate_row_stride=g_stride, gate_mode=int(gate_mode),
        A_log=addr(A_log) if gate_mode == nat.RIA_GATE_RAW else None,
        dt_bias=addr(dt_bias) if gate_mode == nat.RIA_GATE_RAW else None, qk_mode=int(qk_mode), out=addr(out),
        out_dtype=dtype_code(out), z=addr(z), z_dtype=dtype_code(z) if z is not None else 0, z_row_stride=z_stride,
        norm_weight=w_ptr.value if w_ptr is not None else None, pool_rows=int(state_in.shape[0]))
    rc = nat.load().ria_gdn_decode_ex(ctypes.byref(d), _stream(dev))
    nat.check(rc, "ria_gdn_decode_ex")
    return out


def _check_conv_window(conv_weight: torch.Tensor, window_in: torch.Tensor, window_out: torch.Tensor, channels: int,
                       min_pool: int) -> None:
    if conv_weight.dtype != torch.bfloat16 or conv_weight.numel() != channels * CONV_TAPS \
            or not conv_weight.is_contiguous():
        raise ValueError(f"conv_weight must be contiguous bf16 [{channels}, 1, 4]")
    for name, w in (("conv_window_in", window_in), ("conv_window_out", window_out)):
        if w.dtype != torch.bfloat16 or w.dim() != 3 or tuple(w.shape[1:]) != (channels, CONV_TAPS) \
                or not w.is_contiguous():
            raise ValueError(f"{name} must be contiguous bf16 [pool, {channels}, 4], got {tuple(w.shape)}")
        if w.shape[0] < min_pool:
            raise ValueError(f"{name} pool smaller than batch")


def conv1d_window_step(x: torch.Tensor, conv_weight: torch.Tensor, window_in: torch.Tensor,
                       window_out: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Depthwise causal conv step + SiLU on the reference's window [B, C, 4] (ria_conv1d_window_step)."""
    batch, channels = int(x.shape[0]), int(x.shape[-1])
    dev = x.device
    for name, t in (("x", x), ("conv_weight", conv_weight), ("window_in", window_in), ("window_out", window_out),
                    ("out", out)):
        _require_gpu(name, t, dev)
    stride = _row_stride("x", x, batch, channels)
    _check_conv_window(conv_weight, window_in, window_out, channels, batch)
    if tuple(out.shape) != (batch, channels) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {channels}]")
    rc = nat.load().ria_conv1d_window_step(batch, channels, _ptr(x), dtype_code(x), stride, _ptr(conv_weight),
                                           _ptr(window_in), _ptr(window_out), _ptr(out), dtype_code(out),
                                           _stream(dev))
    nat.check(rc, "ria_conv1d_window_step")
    return out


def _check_conv_tensors(conv_weight: torch.Tensor, conv_ring: torch.Tensor, channels: int, min_pool: int) -> None:
    if conv_weight.dtype != torch.bfloat16 or conv_weight.numel() != channels * CONV_TAPS \
            or not conv_weight.is_contiguous():
        raise ValueError(f"conv_weight must be contiguous bf16 [{channels}, 1, 4]")
    if conv_ring.dtype != torch.bfloat16 or conv_ring.dim() != 3 or tuple(conv_ring.shape[1:]) != (CONV_RING, channels) \
            or not conv_ring.is_contiguous():
        raise ValueError(f"conv_ring must be contiguous bf16 [pool, 4, {channels}], got {tuple(conv_ring.shape)}")
    if conv_ring.shape[0] < min_pool:
        raise ValueError("conv ring pool smaller than batch")


def conv1d_step(
    x: torch.Tensor,
    conv_weight: torch.Tensor,
    conv_ring: torch.Tensor,
    out: torch.Tensor,
    *,
    conv_pos: torch.Tensor | int,
    seq_slot: torch.Tensor | None = None,
) -> torch.Tensor:
    """Depthwise causal conv step + SiLU with the conv ring (ria_conv1d_step)."""
    batch, channels = int(x.shape[0]), int(x.shape[-1])
    dev = x.device
    for name, t in (("x", x), ("conv_weight", conv_weight), ("conv_ring", conv_ring), ("out", out),
                    ("seq_slot", seq_slot)):
        _require_gpu(name, t, dev)
    stride = _row_stride("x", x, batch, channels)
    _check_conv_tensors(conv_weight, conv_ring, channels, batch if seq_slot is None else 0)
    if tuple(out.shape) != (batch, channels) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {channels}]")
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    pos_t, pos_s = _rows_i32("conv_pos", conv_pos, batch, dev)
    rc = nat.load().ria_conv1d_step(batch, channels, _ptr(x), dtype_code(x), stride, _ptr(conv_weight),
                                    _ptr(conv_ring), _ptr(seq_slot), _ptr(pos_t), pos_s, _ptr(out), dtype_code(out),
                                    _stream(dev))
    nat.check(rc, "ria_conv1d_step")
    return out


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(sum(x^2, -1) + eps) in fp32 (ria_l2norm)."""
    _require_gpu("x", x)
    xc = x.contiguous()
    out = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    dim = int(x.shape[-1])
    rows = xc.numel() // dim if dim else 0
    rc = nat.load().ria_l2norm(rows, dim, _ptr(xc), dtype_code(xc), float(eps), _ptr(out), _stream(x.device))
    nat.check(rc, "ria_l2norm")
    return out


def _token_rows(name: str, t: torch.Tensor, dim: int) -> tuple[int, int, int]:
    """[T, D] or [T, H, D] with contiguous heads inside each token -> (T, H, token stride)."""
    if t.dim() == 2:
        tokens, heads = int(t.shape[0]), 1
        inner = t.shape[1] == 1 or t.stride(1) == 1
    elif t.dim() == 3:
        tokens, heads = int(t.shape[0]), int(t.shape[1])
        inner = (t.shape[2] == 1 or t.stride(2) == 1) and (heads == 1 or t.stride(1) == dim)
    else:
        raise ValueError(f"{name} must be [tokens, dim] or [tokens, heads, dim], got {tuple(t.shape)}")
    if int(t.shape[-1]) != dim or not inner:
        raise ValueError(f"{name} needs rows of {dim} contiguous elements, got shape {tuple(t.shape)} "
                         f"strides {t.stride()}")
    return tokens, heads, (int(t.stride(0)) if tokens > 1 else heads * dim)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor | None = None,
            eps: float = 1e-6) -> torch.Tensor:
    """(1 + w) RMSNorm over the last dim in fp32, cast back to x's dtype (ria_rmsnorm).

    x is [tokens, dim] or [tokens, heads, dim]; ``out`` (same shape) may have
    another dtype, into which the x-dtype result is converted.
    """
    _require_gpu("x", x)
    dim = int(x.shape[-1])
    tokens, heads, xs = _token_rows("x", x, dim)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    _require_gpu("out", out, x.device)
    if tuple(out.shape) != tuple(x.shape):
        raise ValueError(f"out shape {tuple(out.shape)} != x shape {tuple(x.shape)}")
    _, _, os_ = _token_rows("out", out, dim)
    rc = nat.load().ria_rmsnorm(tokens, heads, dim, _ptr(x), dtype_code(x), xs,
                                _norm_weight("weight", weight, dim, x.device), float(eps), _ptr(out),
                                dtype_code(out), os_, _stream(x.device))
    nat.check(rc, "ria_rmsnorm")
    return out


def gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, *, out: torch.Tensor | None = None,
                  eps: float = 1e-6) -> torch.Tensor:
    """weight * RMSNorm(x) * SiLU(z) per row, in x's dtype (ria_gated_rmsnorm)."""
    _require_gpu("x", x)
    _require_gpu("z", z, x.device)
    if tuple(z.shape) != tuple(x.shape):
        raise ValueError(f"x/z shape mismatch: {tuple(x.shape)} vs {tuple(z.shape)}")
    dim = int(x.shape[-1])
    tokens, heads, xs = _token_rows("x", x, dim)
    _, _, zs = _token_rows("z", z, dim)
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
    _require_gpu("out", out, x.device)
    if tuple(out.shape) != tuple(x.shape):
        raise ValueError(f"out shape {tuple(out.shape)} != x shape {tuple(x.shape)}")
    _, _, os_ = _token_rows("out", out, dim)
    rc = nat.load().ria_gated_rmsnorm(tokens, heads, dim, _ptr(x), dtype_code(x), xs, _ptr(z), dtype_code(z), zs,
                                      _norm_weight("weight", weight, dim, x.device), float(eps), _ptr(out),
                                      dtype_code(out), os_, _stream(x.device))
    nat.check(rc, "ria_gated_rmsnorm")
    return out


def rope_table(position: int, inv_freq: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) of position * inv_freq over both halves, fp32 (ria_rope_table)."""
    _require_gpu("inv_freq", inv_freq)
    rope_dim = 2 * int(inv_freq.numel())
    cos = torch.empty(rope_dim, device=inv_freq.device, dtype=torch.float32)
    sin = torch.empty_like(cos)
    rc = nat.load().ria_rope_table(int(position), _ptr(inv_freq), rope_dim, _ptr(cos), _ptr(sin),
                                   _stream(inv_freq.device))
    nat.check(rc, "ria_rope_table")
    return cos, sin


def rope_apply(x: torch.Tensor, position: int, inv_freq: torch.Tensor) -> torch.Tensor:
    """Partial half-split rotary embedding of fp32 rows (ria_rope_apply)."""
    _require_gpu("x", x)
    _require_gpu("inv_freq", inv_freq, x.device)
    if x.dtype != torch.float32:
        raise ValueError("rope_apply expects fp32 input")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    head_dim = int(x.shape[-1])
    rows = xc.numel() // head_dim
    rc = nat.load().ria_rope_apply(rows, head_dim, 2 * int(inv_freq.numel()), _ptr(xc), _ptr(out), _ptr(inv_freq),
                                   int(position), _stream(x.device))
    nat.check(rc, "ria_rope_apply")
    return out


K_TILE_SHAPE = (8, 4, PAGE_TOKENS, 8)  # (dim % 64) // 8, dim // 64, token, dim % 8


def k_tile_index(token: torch.Tensor | int, dim: torch.Tensor | int):
    """Index of key element (token, dim) inside a K page tile of shape K_TILE_SHAPE."""
    return (dim % 64) // 8, dim // 64, token, dim % 8


KV_DTYPES = (torch.bfloat16, torch.float16)


def _check_kv_cache(k_cache: torch.Tensor, v_cache: torch.Tensor, num_kv_heads: int) -> int:
    if k_cache.dtype not in KV_DTYPES or v_cache.dtype != k_cache.dtype:
        raise ValueError("KV caches must both be bf16 or both fp16")
    if k_cache.dim() != 6 or tuple(k_cache.shape[1:]) != (num_kv_heads, *K_TILE_SHAPE):
        raise ValueError(f"k_cache must be [pages, {num_kv_heads}, 8, 4, 16, 8], got {tuple(k_cache.shape)}")
    if v_cache.dim() != 4 or tuple(v_cache.shape[1:]) != (num_kv_heads, ATTN_HEAD_DIM, PAGE_TOKENS):
        raise ValueError(f"v_cache must be [pages, {num_kv_heads}, 256, 16], got {tuple(v_cache.shape)}")
    if k_cache.shape[0] != v_cache.shape[0] or not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise ValueError("k_cache / v_cache must be contiguous with equal page counts")
    return int(k_cache.shape[0])


def _check_page_table(page_table: torch.Tensor, dev: torch.device) -> int:
    _require_gpu("page_table", page_table, dev)
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.stride(1) != 1:
        raise ValueError("page_table must be int32 [pool, max_pages] with contiguous rows")
    return int(page_table.stride(0))


def kv_append(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    *,
    positions: torch.Tensor | int,
    slots: torch.Tensor | int,
    inv_freq: torch.Tensor,
    seq_slot: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    k_rot_out: torch.Tensor | None = None,
) -> None:
    """RoPE k and append k, v of one token per sequence into the paged cache (ria_kv_append).

    With the fp32 ``k_norm_weight`` [256], k is RMSNorm'd ((1 + w), cast back
    to k's dtype) before RoPE (qwen36_attention_cache.py:303-305).  With
    ``k_rot_out`` (contiguous fp32 [batch, Hkv, 256]) the normed, rotated k
    is also written there in fp32, before its rounding to the page dtype
    (ria_kv_append_out).
    """
    batch = int(k.shape[0])
    num_kv_heads = int(k.shape[1]) if k.dim() == 3 else int(k.numel() // max(batch, 1) // ATTN_HEAD_DIM)
    dev = k.device
    for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache), ("inv_freq", inv_freq),
                    ("seq_slot", seq_slot)):
        _require_gpu(name, t, dev)
    ks = _row_stride("k", k, batch, num_kv_heads * ATTN_HEAD_DIM)
    vs = _row_stride("v", v, batch, num_kv_heads * ATTN_HEAD_DIM)
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    pts = _check_page_table(page_table, dev)
    if seq_slot is None and page_table.shape[0] < batch:
        raise ValueError("page table has fewer rows than batch")
    pos_t, pos_s = _rows_i32("positions", positions, batch, dev)
    slot_t, slot_s = _rows_i32("slots", slots, batch, dev)
    if slot_t is None and slot_s >= page_table.shape[1] * PAGE_TOKENS:
        raise ValueError(f"slot {slot_s} beyond the page table's {page_table.shape[1] * PAGE_TOKENS} tokens")
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    args = (batch, num_kv_heads, _ptr(k), dtype_code(k), ks, _ptr(v), dtype_code(v), vs, _ptr(k_cache),
            _ptr(v_cache), dtype_code(k_cache), pages, _ptr(page_table), pts, _ptr(seq_slot), _ptr(pos_t), pos_s,
            _ptr(slot_t), slot_s, _ptr(inv_freq), 0 if inv_freq is None else 2 * int(inv_freq.numel()),
            _norm_weight("k_norm_weight", k_norm_weight, ATTN_HEAD_DIM, dev))
    if k_rot_out is None:
        rc = nat.load().ria_kv_append(*args, _stream(dev))
        nat.check(rc, "ria_kv_append")
        return
    _require_gpu("k_rot_out", k_rot_out, dev)
    if k_rot_out.dtype != torch.float32 or tuple(k_rot_out.shape) != (batch, num_kv_heads, ATTN_HEAD_DIM) \
            or not k_rot_out.is_contiguous():
        raise ValueError(f"k_rot_out must be contiguous fp32 [{batch}, {num_kv_heads}, {ATTN_HEAD_DIM}]")
    rc = nat.load().ria_kv_append_out(*args, _ptr(k_rot_out), _stream(dev))
    nat.check(rc, "ria_kv_append_out")


def attn_decode_split_tokens(num_kv_heads: int, ctx_lens: list[int]) -> int:
    """Split size the decode kernel's heuristic picks for these context lengths."""
    arr = (ctypes.c_int32 * len(ctx_lens))(*[int(x) for x in ctx_lens])
    return int(nat.load().ria_attn_decode_split_tokens(num_kv_heads, ctypes.cast(arr, ctypes.c_void_p), len(ctx_lens)))


def attn_decode_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, max_ctx: int,
                                split_tokens: int = 0) -> int:
    return int(nat.load().ria_attn_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, max_ctx, split_tokens))


def attn_decode(
    q: torch.Tensor,
    gate: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    out: torch.Tensor,
    *,
    positions: torch.Tensor | int,
    ctx_lens: torch.Tensor | int,
    max_ctx: int,
    inv_freq: torch.Tensor | None,
    scale: float,
    workspace: torch.Tensor,
    seq_slot: torch.Tensor | None = None,
    split_tokens: int = 0,
    phase: int = nat.RIA_ATTN_BOTH,
    q_norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """Split-K paged GQA decode with RoPE on q and a sigmoid gate (ria_attn_decode_phase).

    phase selects the split-K launch, the combine launch or both (the default).
    With the fp32 ``q_norm_weight`` [256], q is RMSNorm'd ((1 + w), cast back
    to q's dtype) before RoPE (qwen36_attention_cache.py:302-304).
    """
    batch = int(q.shape[0])
    num_q_heads = int(q.shape[1])
    num_kv_heads = int(k_cache.shape[1])
    dev = q.device
    for name, t in (("q", q), ("gate", gate), ("k_cache", k_cache), ("v_cache", v_cache), ("out", out),
                    ("inv_freq", inv_freq), ("workspace", workspace), ("seq_slot", seq_slot)):
        _require_gpu(name, t, dev)
    qs = _row_stride("q", q, batch, num_q_heads * ATTN_HEAD_DIM)
    gs = _row_stride("gate", gate, batch, num_q_heads * ATTN_HEAD_DIM)
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    pts = _check_page_table(page_table, dev)
    if max_ctx > page_table.shape[1] * PAGE_TOKENS:
        raise ValueError(f"max_ctx {max_ctx} exceeds the page table capacity {page_table.shape[1] * PAGE_TOKENS}")
    if seq_slot is None and page_table.shape[0] < batch:
        raise ValueError("page table has fewer rows than batch")
    if tuple(out.shape) != (batch, num_q_heads, ATTN_HEAD_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {num_q_heads}, 256]")
    if not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    pos_t, pos_s = _rows_i32("positions", positions, batch, dev)
    ctx_t, ctx_s = _rows_i32("ctx_lens", ctx_lens, batch, dev)
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    rope_dim = 0 if inv_freq is None else 2 * int(inv_freq.numel())
    ws_bytes = workspace.numel() * workspace.element_size()
    rc = nat.load().ria_attn_decode_phase(batch, num_q_heads, num_kv_heads, _ptr(q), dtype_code(q), qs, _ptr(gate),
                                          dtype_code(gate), gs, _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache),
                                          pages, _ptr(page_table), pts, _ptr(seq_slot), _ptr(pos_t), pos_s, _ptr(ctx_t), ctx_s, int(max_ctx),
                                          _ptr(inv_freq), rope_dim,
                                          _norm_weight("q_norm_weight", q_norm_weight, ATTN_HEAD_DIM, dev),
                                          float(scale), int(split_tokens), _ptr(workspace),
                                          ws_bytes, _ptr(out), dtype_code(out), int(phase), _stream(dev))
    nat.check(rc, "ria_attn_decode")
    return out


def kv_gather(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    *,
    batch: int,
    start: int,
    count: int,
    seq_slot: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Logical-order copy of tokens [start, start+count) out of the paged cache (ria_kv_gather)."""
    num_kv_heads = int(k_cache.shape[1])
    dev = k_cache.device
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    pts = _check_page_table(page_table, dev)
    if start < 0 or count < 0 or start + count > page_table.shape[1] * PAGE_TOKENS:
        raise ValueError("gather range outside the page table")
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    k_out = torch.empty((batch, num_kv_heads, count, ATTN_HEAD_DIM), device=dev, dtype=k_cache.dtype)
    v_out = torch.empty_like(k_out)
    rc = nat.load().ria_kv_gather(batch, num_kv_heads, _ptr(k_cache), _ptr(v_cache), pages, _ptr(page_table), pts,
                                  _ptr(seq_slot), int(start), int(count), _ptr(k_out), _ptr(v_out), _stream(dev))
    nat.check(rc, "ria_kv_gather")
    return k_out, v_out


FP8_BLOCK = 128


def _fp8_weight(name: str, w: torch.Tensor, scale_inv: torch.Tensor, dev: torch.device) -> tuple[int, int]:
    _require_gpu(name, w, dev)
    _require_gpu(name + " scale_inv", scale_inv, dev)
    if w.dtype not in (torch.float8_e4m3fn, torch.uint8) or w.dim() != 2 or not w.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float8_e4m3fn (or its uint8 bytes) [N, K] tensor")
    n, k = int(w.shape[0]), int(w.shape[1])
    grid = ((n + FP8_BLOCK - 1) // FP8_BLOCK, (k + FP8_BLOCK - 1) // FP8_BLOCK)
    if scale_inv.dtype != torch.float32 or tuple(scale_inv.shape) != grid or not scale_inv.is_contiguous():
        raise ValueError(f"{name} scale_inv must be contiguous fp32 {grid}, got {tuple(scale_inv.shape)}")
    return n, k


def dequant_fp8(weight: torch.Tensor, scale_inv: torch.Tensor, out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """float(w) * s per 128x128 block, rounded once to out_dtype (ria_dequant_fp8)."""
    dev = weight.device
    n, k = _fp8_weight("weight", weight, scale_inv, dev)
    out = torch.empty((n, k), dtype=out_dtype, device=dev)
    rc = nat.load().ria_dequant_fp8(n, k, _ptr(weight), _ptr(scale_inv), _ptr(out), dtype_code(out), _stream(dev))
    nat.check(rc, "ria_dequant_fp8")
    return out


def linear_fp8(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor, *, out: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """fp16(x) @ fp16(w * s)^T with fp32 accumulation, rounded to fp16 (ria_linear_fp8).

    x [M, K] (rows may be strided); weight [N, K] float8_e4m3fn; scale_inv the
    fp32 per-128x128-block scales; returns / fills y [M, N].
    """
    dev = x.device
    _require_gpu("x", x, dev)
    n, k = _fp8_weight("weight", weight, scale_inv, dev)
    if x.dim() != 2 or x.shape[1] != k or (x.shape[1] > 1 and x.stride(1) != 1):
        raise ValueError(f"x must be [M, {k}] with contiguous rows, got {tuple(x.shape)}")
    m = int(x.shape[0])
    xs = int(x.stride(0)) if m > 1 else k
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=dev)
    _require_gpu("out", out, dev)
    if out.dim() != 2 or tuple(out.shape) != (m, n) or (n > 1 and out.stride(1) != 1):
        raise ValueError(f"out must be [{m}, {n}] with contiguous rows")
    ys = int(out.stride(0)) if m > 1 else n
    rc = nat.load().ria_linear_fp8(m, n, k, _ptr(x), dtype_code(x), xs, _ptr(weight), _ptr(scale_inv), _ptr(out),
                                   dtype_code(out), ys, _stream(dev))
    nat.check(rc, "ria_linear_fp8")
    return out


def linear_fp8_group(x: torch.Tensor, projections: list[tuple[torch.Tensor, torch.Tensor]], *,
                     out: list[torch.Tensor] | None = None,
                     out_dtype: torch.dtype | list[torch.dtype] = torch.float16,
                     accumulate: list[bool] | None = None, norm_weight: torch.Tensor | None = None,
                     norm_dtype: torch.dtype = torch.bfloat16, eps: float = 1e-6) -> list[torch.Tensor]:
    """Up to 4 FP8 projections of the same x in one launch (ria_linear_fp8_group).

    projections: (weight [N_j, K] float8_e4m3fn, scale_inv) pairs; returns /
    fills y_j [M, N_j] (each in its own dtype), each equal to linear_fp8(x, w_j, s_j).
    With accumulate[j], the fp32 out[j] receives out[j] + y_j (a residual add).
    With the fp32 ``norm_weight`` [K], x is the fp32 residual stream and the
    projections read its (1 + w) RMSNorm rounded to norm_dtype
    (ria_linear_fp8_group_normed; up to 4 rows).
    """
    dev = x.device
    _require_gpu("x", x, dev)
    if not 1 <= len(projections) <= nat.LINEAR_GROUP_MAX:
        raise ValueError(f"1 to {nat.LINEAR_GROUP_MAX} projections per call, got {len(projections)}")
    shapes = [_fp8_weight(f"weight {j}", w, s, dev) for j, (w, s) in enumerate(projections)]
    k = shapes[0][1]
    if any(kk != k for _, kk in shapes):
        raise ValueError(f"all projections must share K, got {[kk for _, kk in shapes]}")
    if x.dim() != 2 or x.shape[1] != k or (x.shape[1] > 1 and x.stride(1) != 1):
        raise ValueError(f"x must be [M, {k}] with contiguous rows, got {tuple(x.shape)}")
    m = int(x.shape[0])
    xs = int(x.stride(0)) if m > 1 else k
    if out is None:
        dts = out_dtype if isinstance(out_dtype, (list, tuple)) else [out_dtype] * len(shapes)
        out = [torch.empty((m, n), dtype=dt, device=dev) for (n, _), dt in zip(shapes, dts)]
    if len(out) != len(projections):
        raise ValueError("out must hold one tensor per projection")
    arr = (nat.Fp8Proj * len(projections))()
    for j, ((w, s), (n, _), y) in enumerate(zip(projections, shapes, out)):
        _require_gpu(f"out {j}", y, dev)
        if y.dim() != 2 or tuple(y.shape) != (m, n) or (n > 1 and y.stride(1) != 1):
            raise ValueError(f"out {j} must be [{m}, {n}] with contiguous rows")
        add = bool(accumulate[j]) if accumulate is not None else False
        if add and y.dtype != torch.float32:
            raise ValueError(f"out {j}: accumulating needs fp32")
        arr[j] = nat.Fp8Proj(_ptr(w), _ptr(s), _ptr(y), int(y.stride(0)) if m > 1 else n, n, dtype_code(y), int(add))
    if norm_weight is None:
        rc = nat.load().ria_linear_fp8_group(m, k, _ptr(x), dtype_code(x), xs, len(projections),
                                             ctypes.addressof(arr), _stream(dev))
        nat.check(rc, "ria_linear_fp8_group")
        return out
    if x.dtype != torch.float32:
        raise ValueError("the fused input norm reads fp32 x")
    if norm_dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("norm_dtype must be bf16 or fp16")
    rc = nat.load().ria_linear_fp8_group_normed(m, k, _ptr(x), xs, _norm_weight("norm_weight", norm_weight, k, dev),
                                                float(eps), nat.RIA_DT_BF16 if norm_dtype == torch.bfloat16
                                                else nat.RIA_DT_F16, len(projections), ctypes.addressof(arr),
                                                _stream(dev))
    nat.check(rc, "ria_linear_fp8_group_normed")
    return out


def seq_state_bytes(num_linear_layers: int, num_v_heads: int, conv_dim: int, num_full_layers: int,
                    num_kv_heads: int, tokens: int) -> int:
    """Payload bytes of one sequence's snapshot (ria_seq_state_bytes)."""
    return int(nat.load().ria_seq_state_bytes(num_linear_layers, num_v_heads, conv_dim, num_full_layers,
                                               num_kv_heads, tokens))


def _seq_state_args(states, rings, k_all, v_all, page_table, payload):
    for name, t in (("linear_states", states), ("conv_rings", rings), ("k_cache", k_all), ("v_cache", v_all),
                    ("page_table", page_table), ("payload", payload)):
        _require_gpu(name, t, payload.device)
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if states.dtype != torch.float32 or states.dim() != 5 or tuple(states.shape[3:]) != (GDN_HEAD_DIM, GDN_HEAD_DIM):
        raise ValueError("linear_states must be fp32 [L_lin, rows, Hv, 128, 128]")
    if rings.dtype != torch.bfloat16 or rings.dim() != 4 or tuple(rings.shape[:2]) != tuple(states.shape[:2]) \
            or rings.shape[2] != CONV_RING:
        raise ValueError("conv_rings must be bf16 [L_lin, rows, 4, conv_dim] matching linear_states")
    if k_all.dim() != 7 or v_all.dim() != 5 or k_all.shape[:3] != v_all.shape[:3] or k_all.dtype != v_all.dtype \
            or k_all.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("k/v caches must be 16-bit [L_full, pages, Hkv, tile] of one dtype")
    if page_table.dtype != torch.int32 or page_table.dim() != 2:
        raise ValueError("page_table must be int32 [rows, pages per row]")
    if payload.dtype != torch.uint8 or payload.dim() != 1:
        raise ValueError("payload must be a 1-D uint8 tensor")
    return (int(states.shape[1]), int(states.shape[0]), int(states.shape[2]), int(rings.shape[3]),
            int(k_all.shape[0]), int(k_all.shape[2]), int(k_all.shape[1]))


def seq_state_save(states: torch.Tensor, rings: torch.Tensor, k_all: torch.Tensor, v_all: torch.Tensor,
                   page_table: torch.Tensor, *, row: int, tokens: int, payload: torch.Tensor) -> torch.Tensor:
    """Copy row `row` (tokens seen `tokens`) of the pools into `payload` (ria_seq_state_save)."""
    rows, n_lin, hv, cdim, n_full, hkv, pages = _seq_state_args(states, rings, k_all, v_all, page_table, payload)
    rc = nat.load().ria_seq_state_save(int(row), rows, n_lin, hv, _ptr(states), _ptr(rings), cdim, n_full, hkv, pages,
                                       _ptr(k_all), _ptr(v_all), _ptr(page_table), int(page_table.shape[1]),
                                       int(tokens), _ptr(payload), payload.numel(), _stream(payload.device))
    nat.check(rc, "ria_seq_state_save")
    return payload


def seq_state_restore(states: torch.Tensor, rings: torch.Tensor, k_all: torch.Tensor, v_all: torch.Tensor,
                      page_table: torch.Tensor, *, row: int, tokens: int, payload: torch.Tensor) -> None:
    """Copy a snapshot payload into row `row` of the pools, whose pages must be allocated (ria_seq_state_restore)."""
    rows, n_lin, hv, cdim, n_full, hkv, pages = _seq_state_args(states, rings, k_all, v_all, page_table, payload)
    rc = nat.load().ria_seq_state_restore(int(row), rows, n_lin, hv, _ptr(states), _ptr(rings), cdim, n_full, hkv,
                                          pages, _ptr(k_all), _ptr(v_all), _ptr(page_table),
                                          int(page_table.shape[1]), int(tokens), _ptr(payload), payload.numel(),
                                          _stream(payload.device))
    nat.check(rc, "ria_seq_state_restore")


def gdn_prefill_workspace_bytes(num_k_heads: int, num_v_heads: int, segment_tokens: int) -> int:
    return int(nat.load().ria_gdn_prefill_workspace_bytes(num_k_heads, num_v_heads, segment_tokens))


def gdn_prefill(
    mixed_qkv: torch.Tensor,
    state: torch.Tensor,
    gate_a: torch.Tensor,
    gate_b: torch.Tensor,
    out: torch.Tensor,
    *,
    num_k_heads: int,
    num_v_heads: int,
    conv_weight: torch.Tensor,
    conv_ring: torch.Tensor,
    conv_pos: int,
    workspace: torch.Tensor,
    gate_mode: int = nat.RIA_GATE_PRECOMPUTED,
    A_log: torch.Tensor | None = None,
    dt_bias: torch.Tensor | None = None,
    z: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """Chunked Gated DeltaNet prefill of one sequence (ria_gdn_prefill).

    mixed_qkv [L, conv_dim]; state [Hv, 128, 128] fp32 (updated in place);
    conv_ring [4, conv_dim] bf16 (updated); gate_a/b [L, Hv]; out [L, Hv, 128].
    With ``z`` [L, Hv, 128] (or rows of >= Hv*128) and the fp32 ``norm_weight``
    [128], out receives the gated RMSNorm of the read-out.
    """
    length = int(mixed_qkv.shape[0])
    dev = mixed_qkv.device
    cdim = conv_dim(num_k_heads, num_v_heads)
    for name, t in (("mixed_qkv", mixed_qkv), ("state", state), ("gate_a", gate_a), ("gate_b", gate_b),
                    ("out", out), ("conv_weight", conv_weight), ("conv_ring", conv_ring), ("workspace", workspace),
                    ("A_log", A_log), ("dt_bias", dt_bias)):
        _require_gpu(name, t, dev)
    xs = _row_stride("mixed_qkv", mixed_qkv, length, cdim)
    if state.dtype != torch.float32 or tuple(state.shape) != (num_v_heads, 128, 128) or not state.is_contiguous():
        raise ValueError(f"state must be contiguous fp32 [{num_v_heads}, 128, 128]")
    _check_conv_tensors(conv_weight, conv_ring.reshape(1, CONV_RING, cdim), cdim, 1)
    if gate_a.dtype != torch.float32 or gate_b.dtype != torch.float32:
        raise ValueError("gate_a / gate_b must be fp32")
    gs = _row_stride("gate_a", gate_a, length, num_v_heads)
    if _row_stride("gate_b", gate_b, length, num_v_heads) != gs:
        raise ValueError("gate_a and gate_b must share a row stride")
    if tuple(out.shape) != (length, num_v_heads, GDN_HEAD_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{length}, {num_v_heads}, 128]")
    if gate_mode == nat.RIA_GATE_RAW:
        for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
            if t is None or t.dtype != torch.float32 or t.numel() != num_v_heads or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous fp32 tensor of {num_v_heads} values")
    if not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    if (z is None) != (norm_weight is None):
        raise ValueError("the gated norm needs both z and norm_weight")
    z_stride = 0
    if z is not None:
        _require_gpu("z", z, dev)
        if z.dim() == 3:
            z_stride = _row_stride("z", z, length, num_v_heads * GDN_HEAD_DIM)
        elif z.dim() == 2 and z.shape[0] == length and z.shape[1] >= num_v_heads * GDN_HEAD_DIM and z.stride(1) == 1:
            z_stride = int(z.stride(0))
        else:
            raise ValueError(f"z must have {length} rows of >= {num_v_heads * GDN_HEAD_DIM} contiguous elements")
    raw = gate_mode == nat.RIA_GATE_RAW
    rc = nat.load().ria_gdn_prefill(length, num_k_heads, num_v_heads, _ptr(mixed_qkv), dtype_code(mixed_qkv), xs,
                                    _ptr(conv_weight), _ptr(conv_ring), int(conv_pos), _ptr(state), _ptr(gate_a),
                                    _ptr(gate_b), gs, int(gate_mode), _ptr(A_log) if raw else None,
                                    _ptr(dt_bias) if raw else None, _ptr(out), dtype_code(out), _ptr(z),
                                    dtype_code(z) if z is not None else 0, z_stride,
                                    _norm_weight("norm_weight", norm_weight, GDN_HEAD_DIM, dev), _ptr(workspace),
                                    workspace.numel() * workspace.element_size(), _stream(dev))
    nat.check(rc, "ria_gdn_prefill")
    return out


def _page_row(page_table: torch.Tensor, dev: torch.device) -> int:
    """Check a single sequence's page-table row (1-D int32); returns its capacity in pages."""
    _require_gpu("page_table", page_table, dev)
    if page_table.dtype != torch.int32 or page_table.dim() != 1 or not page_table.is_contiguous():
        raise ValueError("page_table must be one contiguous int32 row")
    return int(page_table.numel())



def attn_decode_append(
    q: torch.Tensor,
    gate: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    out: torch.Tensor,
    *,
    positions: torch.Tensor | int,
    ctx_lens: torch.Tensor | int,
    max_ctx: int,
    inv_freq: torch.Tensor | None,
    scale: float,
    workspace: torch.Tensor,
    seq_slot: torch.Tensor | None = None,
    split_tokens: int = 0,
    phase: int = nat.RIA_ATTN_BOTH,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """kv_append + attn_decode without a launch of its own (ria_attn_decode_append).

    Row b's new token (k, v [batch, Hkv, 256] in q's dtype) goes into slot
    ``ctx_lens[b] - 1`` at RoPE position ``positions[b]``: the split-K launch
    stops before it, the combine launch computes it with kv_append's
    arithmetic (the pages hold the same bits), writes it into the page and
    folds it into the row's softmax.  Both phases take the same arguments.
    ``workspace`` (the split-K partials) is required; callers that cannot
    allocate use attn_decode_append_noalloc.
    """
    if workspace is None:
        raise ValueError("attn_decode_append: workspace is required (attn_decode_append_noalloc needs none)")
    return _attn_decode_append(q, gate, k, v, k_cache, v_cache, page_table, out, positions=positions,
                               ctx_lens=ctx_lens, max_ctx=max_ctx, inv_freq=inv_freq, scale=scale,
                               workspace=workspace, seq_slot=seq_slot, split_tokens=split_tokens, phase=phase,
                               q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight)


def attn_decode_append_noalloc(
    q: torch.Tensor,
    gate: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    out: torch.Tensor,
    *,
    positions: torch.Tensor | int,
    ctx_lens: torch.Tensor | int,
    max_ctx: int,
    inv_freq: torch.Tensor | None,
    scale: float,
    seq_slot: torch.Tensor | None = None,
    split_tokens: int = 0,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
) -> torch.Tensor:
    """attn_decode_append with no workspace (ria_attn_decode_append_noalloc).

    The split-K partials go into the library's own 16 MiB device array, one
    per GPU: nothing is allocated, both phases run in the one call, sizes
    whose partials exceed the array raise, and calls that overlap on one GPU
    (concurrent streams) race.
    """
    return _attn_decode_append(q, gate, k, v, k_cache, v_cache, page_table, out, positions=positions,
                               ctx_lens=ctx_lens, max_ctx=max_ctx, inv_freq=inv_freq, scale=scale, workspace=None,
                               seq_slot=seq_slot, split_tokens=split_tokens, phase=nat.RIA_ATTN_BOTH,
                               q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight)


def _attn_decode_append(q, gate, k, v, k_cache, v_cache, page_table, out, *, positions, ctx_lens, max_ctx, inv_freq,
                        scale, workspace, seq_slot, split_tokens, phase, q_norm_weight, k_norm_weight):
    batch = int(q.shape[0])
    num_q_heads = int(q.shape[1])
    num_kv_heads = int(k_cache.shape[1])
    dev = q.device
    for name, t in (("q", q), ("gate", gate), ("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("out", out), ("inv_freq", inv_freq), ("workspace", workspace), ("seq_slot", seq_slot)):
        _require_gpu(name, t, dev)  # (a None workspace is the no-alloc path's)
    if k.dtype != q.dtype or v.dtype != q.dtype or gate.dtype != q.dtype:
        raise ValueError("attn_decode_append: q, gate, k and v must share one dtype")
    qs = _row_stride("q", q, batch, num_q_heads * ATTN_HEAD_DIM)
    gs = _row_stride("gate", gate, batch, num_q_heads * ATTN_HEAD_DIM)
    ks = _row_stride("k", k, batch, num_kv_heads * ATTN_HEAD_DIM)
    vs = _row_stride("v", v, batch, num_kv_heads * ATTN_HEAD_DIM)
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    pts = _check_page_table(page_table, dev)
    if max_ctx > page_table.shape[1] * PAGE_TOKENS:
        raise ValueError(f"max_ctx {max_ctx} exceeds the page table capacity {page_table.shape[1] * PAGE_TOKENS}")
    if seq_slot is None and page_table.shape[0] < batch:
        raise ValueError("page table has fewer rows than batch")
    if tuple(out.shape) != (batch, num_q_heads, ATTN_HEAD_DIM) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous [{batch}, {num_q_heads}, 256]")
    if workspace is not None and not workspace.is_contiguous():
        raise ValueError("workspace must be contiguous")
    pos_t, pos_s = _rows_i32("positions", positions, batch, dev)
    ctx_t, ctx_s = _rows_i32("ctx_lens", ctx_lens, batch, dev)
    if seq_slot is not None:
        _rows_i32("seq_slot", seq_slot, batch, dev)
    rope_dim = 0 if inv_freq is None else 2 * int(inv_freq.numel())
    head = (batch, num_q_heads, num_kv_heads, _ptr(q), dtype_code(q), qs, _ptr(gate), dtype_code(gate), gs,
            _ptr(k), ks, _ptr(v), vs, _norm_weight("k_norm_weight", k_norm_weight, ATTN_HEAD_DIM, dev),
            _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache), pages, _ptr(page_table), pts, _ptr(seq_slot),
            _ptr(pos_t), pos_s, _ptr(ctx_t), ctx_s, int(max_ctx), _ptr(inv_freq), rope_dim,
            _norm_weight("q_norm_weight", q_norm_weight, ATTN_HEAD_DIM, dev), float(scale), int(split_tokens))
    tail = (_ptr(out), dtype_code(out), int(phase), _stream(dev))
    lib = nat.load()
    if workspace is None:
        rc = lib.ria_attn_decode_append_noalloc(*head, *tail)
        nat.check(rc, "ria_attn_decode_append_noalloc")
    else:
        ws_bytes = workspace.numel() * workspace.element_size()
        rc = lib.ria_attn_decode_append(*head, _ptr(workspace), ws_bytes, *tail)
        nat.check(rc, "ria_attn_decode_append")
    return out

def kv_append_seq(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    *,
    start: int,
    inv_freq: torch.Tensor | None,
    k_norm_weight: torch.Tensor | None = None,
) -> None:
    """Append a prompt's k (RoPE at start + i) and v at slots start + i of one sequence (ria_kv_append_seq).

    k, v [L, Hkv, 256]; page_table is the sequence's page-table row; with the
    fp32 ``k_norm_weight`` [256] k is RMSNorm'd before RoPE.
    """
    length = int(k.shape[0])
    num_kv_heads = int(k_cache.shape[1])
    dev = k.device
    for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache), ("inv_freq", inv_freq)):
        _require_gpu(name, t, dev)
    ks = _row_stride("k", k, length, num_kv_heads * ATTN_HEAD_DIM)
    vs = _row_stride("v", v, length, num_kv_heads * ATTN_HEAD_DIM)
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    cap = _page_row(page_table, dev)
    if start < 0 or start + length > cap * PAGE_TOKENS:
        raise ValueError(f"{start} + {length} tokens exceed the row's {cap} pages")
    rope_dim = 0 if inv_freq is None else 2 * int(inv_freq.numel())
    rc = nat.load().ria_kv_append_seq(length, num_kv_heads, _ptr(k), dtype_code(k), ks, _ptr(v), dtype_code(v), vs,
                                      _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache), pages, _ptr(page_table),
                                      cap, int(start), _ptr(inv_freq), rope_dim,
                                      _norm_weight("k_norm_weight", k_norm_weight, ATTN_HEAD_DIM, dev), _stream(dev))
    nat.check(rc, "ria_kv_append_seq")


def attn_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gate: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_table: torch.Tensor,
    out: torch.Tensor | None = None,
    *,
    start: int,
    inv_freq: torch.Tensor | None,
    scale: float,
    phase: int = nat.RIA_PREFILL_BOTH,
    q_norm_weight: torch.Tensor | None = None,
    k_norm_weight: torch.Tensor | None = None,
    stage: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal GQA prefill of one sequence's prompt over its paged cache (ria_attn_prefill_phase).

    q, gate [L, Hq, 256]; k, v [L, Hkv, 256], all of one dtype; the prompt's
    k/v are appended at slots start .. start + L - 1 first.  Returns out
    [L, Hq, 256] in that dtype.  phase selects the append launch, the
    attention launch or both (the default).  With the fp32 q_norm / k_norm
    weights [256], q and k are RMSNorm'd before RoPE.  With a ``stage`` (a
    uint8 device tensor of at least prefill_stage_bytes(L, Hkv); both phases
    take the same one) a prompt that starts the sequence (start 0) is
    attended over fp16 copies of its own keys and values
    (ria_attn_prefill_staged).
    """
    length = int(q.shape[0])
    num_q_heads = int(q.shape[1])
    num_kv_heads = int(k_cache.shape[1])
    dev = q.device
    for name, t in (("q", q), ("k", k), ("v", v), ("gate", gate), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("inv_freq", inv_freq)):
        _require_gpu(name, t, dev)
    if len({q.dtype, k.dtype, v.dtype, gate.dtype}) != 1:
        raise ValueError("q, k, v and gate must share a dtype")
    qs = _row_stride("q", q, length, num_q_heads * ATTN_HEAD_DIM)
    gs = _row_stride("gate", gate, length, num_q_heads * ATTN_HEAD_DIM)
    ks = _row_stride("k", k, length, num_kv_heads * ATTN_HEAD_DIM)
    vs = _row_stride("v", v, length, num_kv_heads * ATTN_HEAD_DIM)
    pages = _check_kv_cache(k_cache, v_cache, num_kv_heads)
    cap = _page_row(page_table, dev)
    if start < 0 or start + length > cap * PAGE_TOKENS:
        raise ValueError(f"{start} + {length} tokens exceed the row's {cap} pages")
    if out is None:
        out = torch.empty((length, num_q_heads, ATTN_HEAD_DIM), device=dev, dtype=q.dtype)
    _require_gpu("out", out, dev)
    if tuple(out.shape) != (length, num_q_heads, ATTN_HEAD_DIM) or not out.is_contiguous() or out.dtype != q.dtype:
        raise ValueError(f"out must be contiguous [{length}, {num_q_heads}, 256] of q's dtype")
    rope_dim = 0 if inv_freq is None else 2 * int(inv_freq.numel())
    head = (length, num_q_heads, num_kv_heads, _ptr(q), qs, _ptr(k), ks, _ptr(v), vs, _ptr(gate), gs, dtype_code(q),
            _ptr(k_cache), _ptr(v_cache), dtype_code(k_cache), pages, _ptr(page_table), cap, int(start),
            _ptr(inv_freq), rope_dim, _norm_weight("q_norm_weight", q_norm_weight, ATTN_HEAD_DIM, dev),
            _norm_weight("k_norm_weight", k_norm_weight, ATTN_HEAD_DIM, dev), float(scale))
    if stage is None:
        rc = nat.load().ria_attn_prefill_phase(*head, _ptr(out), int(phase), _stream(dev))
    else:
        _require_gpu("stage", stage, dev)
        if not stage.is_contiguous():
            raise ValueError("stage must be contiguous")
        rc = nat.load().ria_attn_prefill_staged(*head, _ptr(stage), stage.numel() * stage.element_size(), _ptr(out),
                                                int(phase), _stream(dev))
    nat.check(rc, "ria_attn_prefill")
    return out


def prefill_stage_bytes(length: int, num_kv_heads: int) -> int:
    """Bytes of the fp16 stage attn_prefill takes for a prompt of `length` tokens (ria_attn_prefill_stage_bytes)."""
    return int(nat.load().ria_attn_prefill_stage_bytes(int(length), int(num_kv_heads)))
