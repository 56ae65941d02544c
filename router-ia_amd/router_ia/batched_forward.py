"""Batched token forward through the attention side of the 40-layer stack.

The reference runs one sequence's token through the model at a time:
``run_forward_token`` (v2/src/router_ia/qwen36_chat_batch.py:181-207) loops
over the 40 layers calling ``step_attention`` (the layer's input RMSNorm,
projections, Gated DeltaNet or gated full attention, output projection and
residual add; qwen36_attention_cache.py:224-324) and then the layer's MoE
block, and bumps ``tokens_seen`` after the last layer.  ``BatchedForward``
runs that loop for B sequences at once on a ``BatchedAttentionState``: every
step of every layer is one launch over the batch, and the projections read
the checkpoint's FP8 block-scaled weights as stored.  The MoE block (and the
embedding, final norm and lm_head around the loop) stay the caller's: pass a
callable ``mlp(model_layer, x) -> x`` to run between layers, as the
reference does.

Per layer (B rows, hidden 2048, the reference's CUDA dtypes):

    DeltaNet (model layer 4i, 4i+1, 4i+2)        full attention (model layer 4i+3)
    h = bf16(rmsnorm(x))           ria_rmsnorm     h = fp16(rmsnorm(x))
                                   (inside the projection launch up to 4 rows)
    qkv, z (fp16), a, b (fp32)     one grouped     q, gate, k, v (fp16)  one grouped
                                   FP8 launch                            FP8 launch
    conv, gates, delta rule,       ria_gdn_decode  k_norm + RoPE + append, q_norm +
    read-out, gated RMSNorm (fp16)                 RoPE + attention + gate (fp16)
    x += out_proj(.) in the projection launch      x += o_proj(.) likewise

q_proj's rows interleave each head's query and gate (:295-299); they are split
once, when the weights are prepared, into two projections whose outputs are
the contiguous q and gate the attention launch reads.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch

from . import _native as nat
from . import kernels as K
from .batched_state import BatchedAttentionState

HIDDEN = 2048
FUSED_NORM_ROWS = 4  # up to this many rows the input RMSNorm runs inside the projection launch
FP8_KERNEL_ROWS = 16  # up to this many rows the projections read the FP8 weights (one-pass kernel)


@dataclass
class Fp8Projection:
    """A checkpoint projection: float8_e4m3fn weight [N, K] and fp32 weight_scale_inv [ceil(N/128), K/128]."""
    weight: torch.Tensor
    scale_inv: torch.Tensor

    def pair(self) -> tuple[torch.Tensor, torch.Tensor]:
        return self.weight, self.scale_inv


@dataclass
class LinearLayerWeights:
    """One Gated DeltaNet layer (qwen36_attention_cache.py:224-282); norm weights fp32."""
    input_norm: torch.Tensor      # [2048], (1 + w) RMSNorm
    in_proj_qkv: Fp8Projection    # [8192, 2048]
    in_proj_z: Fp8Projection      # [4096, 2048]
    in_proj_a: Fp8Projection      # [32, 2048]
    in_proj_b: Fp8Projection      # [32, 2048]
    out_proj: Fp8Projection       # [2048, 4096]
    conv_weight: torch.Tensor     # bf16 [8192, 1, 4]
    A_log: torch.Tensor           # [32]
    dt_bias: torch.Tensor         # [32]
    norm_weight: torch.Tensor     # [128], gated RMSNorm


@dataclass
class FullLayerWeights:
    """One gated full-attention layer (qwen36_attention_cache.py:285-324); norm weights fp32."""
    input_norm: torch.Tensor      # [2048]
    query: Fp8Projection          # the query rows of q_proj [16 * 256, 2048]
    gate: Fp8Projection           # the gate rows of q_proj [16 * 256, 2048]
    k_proj: Fp8Projection         # [512, 2048]
    v_proj: Fp8Projection         # [512, 2048]
    o_proj: Fp8Projection         # [2048, 4096]
    q_norm: torch.Tensor          # [256]
    k_norm: torch.Tensor          # [256]

    @classmethod
    def from_checkpoint(cls, input_norm: torch.Tensor, q_proj: Fp8Projection, k_proj: Fp8Projection,
                        v_proj: Fp8Projection, o_proj: Fp8Projection, q_norm: torch.Tensor, k_norm: torch.Tensor,
                        num_heads: int = 16, head_dim: int = 256) -> "FullLayerWeights":
        query, gate = split_query_gate(q_proj, num_heads, head_dim)
        return cls(input_norm, query, gate, k_proj, v_proj, o_proj, q_norm, k_norm)


def split_query_gate(q_proj: Fp8Projection, num_heads: int = 16,
                     head_dim: int = 256) -> tuple[Fp8Projection, Fp8Projection]:
    """q_proj's rows per head are [query (head_dim) | gate (head_dim)] (:295-299): split them into two projections.

    head_dim is a multiple of the 128-row scale block, so each half keeps whole
    scale rows and the dequantised values are unchanged.
    """
    if head_dim % K.FP8_BLOCK:
        raise ValueError(f"head_dim {head_dim} must be a multiple of {K.FP8_BLOCK}")
    w, s = q_proj.weight, q_proj.scale_inv
    if tuple(w.shape[:1]) != (2 * num_heads * head_dim,):
        raise ValueError(f"q_proj must have {2 * num_heads * head_dim} rows, got {tuple(w.shape)}")
    kdim = int(w.shape[1])
    wb = w.view(torch.uint8).reshape(num_heads, 2, head_dim, kdim)
    sb = s.reshape(num_heads, 2, head_dim // K.FP8_BLOCK, -1)

    def half(i: int) -> Fp8Projection:
        return Fp8Projection(wb[:, i].reshape(num_heads * head_dim, kdim).contiguous().view(w.dtype),
                             sb[:, i].reshape(num_heads * head_dim // K.FP8_BLOCK, -1).contiguous())

    return half(0), half(1)


def layer_weights(ckpt: dict[str, torch.Tensor], model_layer: int,
                  device: torch.device | str | None = None) -> LinearLayerWeights | FullLayerWeights:
    """A layer's weights from its checkpoint tensors (keys: the checkpoint's suffixes after the layer prefix).

    Norm weights are widened to fp32 once here; FP8 projections stay as stored.
    """
    def t(key, dtype=None):
        x = ckpt[key]
        x = x.to(device) if device is not None else x
        return x.to(dtype).contiguous() if dtype is not None else x.contiguous()

    def proj(prefix):
        return Fp8Projection(t(prefix + ".weight"), t(prefix + ".weight_scale_inv", torch.float32))

    if model_layer % 4 == 3:
        return FullLayerWeights.from_checkpoint(
            t("input_layernorm.weight", torch.float32), proj("self_attn.q_proj"), proj("self_attn.k_proj"),
            proj("self_attn.v_proj"), proj("self_attn.o_proj"), t("self_attn.q_norm.weight", torch.float32),
            t("self_attn.k_norm.weight", torch.float32))
    return LinearLayerWeights(
        t("input_layernorm.weight", torch.float32), proj("linear_attn.in_proj_qkv"), proj("linear_attn.in_proj_z"),
        proj("linear_attn.in_proj_a"), proj("linear_attn.in_proj_b"), proj("linear_attn.out_proj"),
        t("linear_attn.conv1d.weight", torch.bfloat16), t("linear_attn.A_log", torch.float32),
        t("linear_attn.dt_bias", torch.float32), t("linear_attn.norm.weight", torch.float32))


class BatchedForward:
    """The attention side of every layer for one token of each of B sequences (see the module docstring)."""

    def __init__(self, state: BatchedAttentionState, layers: list[LinearLayerWeights | FullLayerWeights],
                 projections: str = "fp8"):
        """projections: "fp8" (the default) reads the FP8 weights at every batch size; "fp16" runs
        batches of more than 16 rows on the library fp16 GEMM over weights dequantised once
        (ria_dequant_fp8: the reference's fp16 weights, bit for bit; 2.6 GB for the 40 layers)."""
        n_lin = sum(isinstance(w, LinearLayerWeights) for w in layers)
        n_full = sum(isinstance(w, FullLayerWeights) for w in layers)
        if n_lin + n_full != len(layers):
            raise TypeError("layers must be LinearLayerWeights or FullLayerWeights")
        if (n_lin, n_full) != (state.num_linear_layers, state.num_full_layers):
            raise ValueError(f"{n_lin} DeltaNet + {n_full} attention layers given, the state holds "
                             f"{state.num_linear_layers} + {state.num_full_layers}")
        self.state = state
        self.layers = layers
        self.index = []  # model layer -> index among its kind
        counts = [0, 0]
        for w in layers:
            kind = int(isinstance(w, FullLayerWeights))
            self.index.append(counts[kind])
            counts[kind] += 1
        b, dev = state.max_seqs, state.device
        hv, hq, hkv = state.num_v_heads, state.num_q_heads, state.num_kv_heads

        def buf(*shape, dtype=torch.float16):
            return torch.empty(shape, dtype=dtype, device=dev)

        self.h_bf16 = buf(b, HIDDEN, dtype=torch.bfloat16)   # DeltaNet layers: bf16(h) (:229)
        self.h_f16 = buf(b, HIDDEN)                          # attention layers: fp16(h) (:292-293)
        self.mixed = buf(b, state.conv_dim)
        self.z = buf(b, hv * 128)
        self.gate_a = buf(b, hv, dtype=torch.float32)        # a_raw, b_raw .float() (:245-246)
        self.gate_b = buf(b, hv, dtype=torch.float32)
        self.gated = buf(b, hv, 128)
        self.q = buf(b, hq, 256)
        self.gate = buf(b, hq, 256)
        self.k = buf(b, hkv, 256)
        self.v = buf(b, hkv, 256)
        self.attn = buf(b, hq, 256)
        self._stepped = False
        if projections not in ("fp8", "fp16"):
            raise ValueError(f"projections must be 'fp8' or 'fp16', got {projections!r}")
        # The FP8 kernels outrun the library's fp16 GEMM on the dequantised weights at every batch
        # size measured (all 40 layers' projections at 128 rows: 1.14 against 1.29 ms per step), and
        # need no fp16 copy of the weights; "fp16" keeps the library path for comparison.
        self.gemm16 = projections == "fp16" and b > FP8_KERNEL_ROWS
        self.w16: list[tuple[torch.Tensor, torch.Tensor]] = []
        if self.gemm16:
            self.gate_ab = buf(b, 2 * hv, dtype=torch.float32)  # a | b of one row side by side
            for w in layers:
                if isinstance(w, LinearLayerWeights):
                    parts, wo = [w.in_proj_qkv, w.in_proj_z, w.in_proj_a, w.in_proj_b], w.out_proj
                else:
                    parts, wo = [w.query, w.gate, w.k_proj, w.v_proj], w.o_proj
                w_in = torch.cat([K.dequant_fp8(p.weight, p.scale_inv) for p in parts], 0)
                self.w16.append((w_in, K.dequant_fp8(wo.weight, wo.scale_inv)))

    def layer(self, model_layer: int, x: torch.Tensor) -> torch.Tensor:
        """x [B, 2048] fp32 += this layer's attention output (in place); returns x."""
        w = self.layers[model_layer]
        i = self.index[model_layer]
        st = self.state
        b = st.max_seqs
        fused = b <= FUSED_NORM_ROWS  # the input norm inside the projection launch
        if self.gemm16:
            return self._layer_gemm16(w, i, model_layer, x)
        if isinstance(w, LinearLayerWeights):
            projs = [w.in_proj_qkv.pair(), w.in_proj_z.pair(), w.in_proj_a.pair(), w.in_proj_b.pair()]
            outs = [self.mixed, self.z, self.gate_a, self.gate_b]
            if fused:
                K.linear_fp8_group(x, projs, out=outs, norm_weight=w.input_norm, norm_dtype=torch.bfloat16)
            else:
                # bf16(h); the projection kernels take it as F.linear's fp16 x (exact in
                # fp16's range), converting it as it goes into their operand staging
                K.rmsnorm(x, w.input_norm, out=self.h_bf16)
                K.linear_fp8_group(self.h_bf16, projs, out=outs)
            st.linear_step(i, self.mixed, w.conv_weight, self.gate_a, self.gate_b, gate_mode=nat.RIA_GATE_RAW,
                           A_log=w.A_log, dt_bias=w.dt_bias, out=self.gated, z=self.z, norm_weight=w.norm_weight)
            K.linear_fp8_group(self.gated.view(b, -1), [w.out_proj.pair()], out=[x], accumulate=[True])
        else:
            projs = [w.query.pair(), w.gate.pair(), w.k_proj.pair(), w.v_proj.pair()]
            outs = [self.q.view(b, -1), self.gate.view(b, -1), self.k.view(b, -1), self.v.view(b, -1)]
            if fused:
                K.linear_fp8_group(x, projs, out=outs, norm_weight=w.input_norm, norm_dtype=torch.float16)
            else:
                K.rmsnorm(x, w.input_norm, out=self.h_f16)
                K.linear_fp8_group(self.h_f16, projs, out=outs)
            st.full_step(i, self.q, self.k, self.v, self.gate, out=self.attn, q_norm_weight=w.q_norm,
                         k_norm_weight=w.k_norm)
            K.linear_fp8_group(self.attn.view(b, -1), [w.o_proj.pair()], out=[x], accumulate=[True])
        return x

    def _layer_gemm16(self, w, i: int, model_layer: int, x: torch.Tensor) -> torch.Tensor:
        """``layer`` with the projections as fp16 GEMMs: F.linear(fp16(h), W16), the reference's
        CUDA projection (qwen36_attention_cache.py:232-247, 268, 295-301, 318-320), one GEMM per
        layer's input projections (their weights stacked) and one for the output projection."""
        st = self.state
        b = st.max_seqs
        w_in, w_out = self.w16[model_layer]
        if isinstance(w, LinearLayerWeights):
            K.rmsnorm(x, w.input_norm, out=self.h_bf16)
            h = self.h_f16.copy_(self.h_bf16)  # bf16(h) -> fp16, as F.linear on fp16 weights takes it
            y = torch.nn.functional.linear(h, w_in)  # [B, qkv | z | a | b] fp16
            nq, nz = self.mixed.shape[1], self.z.shape[1]
            hv = st.num_v_heads
            ab = self.gate_ab.copy_(y[:, nq + nz:nq + nz + 2 * hv])  # a, b .float() (:245-246), one launch
            st.linear_step(i, y[:, :nq], w.conv_weight, ab[:, :hv], ab[:, hv:], gate_mode=nat.RIA_GATE_RAW,
                           A_log=w.A_log, dt_bias=w.dt_bias, out=self.gated, z=y[:, nq:nq + nz],
                           norm_weight=w.norm_weight)
            x.add_(torch.nn.functional.linear(self.gated.view(b, -1), w_out))
        else:
            K.rmsnorm(x, w.input_norm, out=self.h_f16)
            y = torch.nn.functional.linear(self.h_f16, w_in)  # [B, query | gate | k | v] fp16
            hq, hkv = st.num_q_heads, st.num_kv_heads
            nq, nk = hq * 256, hkv * 256
            q = y[:, :nq].view(b, hq, 256)
            gate = y[:, nq:2 * nq].view(b, hq, 256)
            k = y[:, 2 * nq:2 * nq + nk].view(b, hkv, 256)
            v = y[:, 2 * nq + nk:2 * nq + 2 * nk].view(b, hkv, 256)
            st.full_step(i, q, k, v, gate, out=self.attn, q_norm_weight=w.q_norm, k_norm_weight=w.k_norm)
            x.add_(torch.nn.functional.linear(self.attn.view(b, -1), w_out))
        return x

    def capture(self, steps: int,
                mlp: Callable[[int, torch.Tensor], torch.Tensor] | None = None) -> "ForwardGraph":
        """Record one ``step`` as a HIP graph that can be replayed for the next `steps` tokens.

        KV pages for `steps` more tokens of every row are reserved first, so a
        replay does no host work beyond the launch.  Every launch of a step reads
        positions and context lengths from device memory (the balanced split-K
        attention schedules itself from them on the device), so one recording
        serves every position.  Run one eager ``step`` before the first capture,
        so that every kernel has been loaded.
        """
        st = self.state
        if not self._stepped:
            raise RuntimeError("run one eager step() before capture(), so every kernel is loaded")
        if st.split_tokens != 0:
            raise RuntimeError("capture needs the balanced attention schedule (split_tokens=0): a fixed split "
                               "sizes its grid from the host-side context length")
        st.reserve(steps)
        return ForwardGraph(self, steps, mlp)

    def step(self, x: torch.Tensor,
             mlp: Callable[[int, torch.Tensor], torch.Tensor] | None = None) -> torch.Tensor:
        """One token per sequence through all layers (qwen36_chat_batch.py:181-187), then advance the positions.

        x [B, 2048] fp32 is the residual stream entering layer 0 (updated in
        place); ``mlp(model_layer, x)`` runs after each layer's attention, where
        the reference runs the layer's MoE block.
        """
        if x.dtype != torch.float32 or tuple(x.shape) != (self.state.max_seqs, HIDDEN) or not x.is_contiguous():
            raise ValueError(f"x must be contiguous fp32 [{self.state.max_seqs}, {HIDDEN}]")
        for m in range(len(self.layers)):
            self.layer(m, x)
            if mlp is not None:
                x = mlp(m, x)
        self.state.advance()
        self._stepped = True
        return x


class ForwardGraph:
    """A recorded ``BatchedForward.step``: write the inputs into ``x``, call ``replay()``, read ``out``.

    ``x`` is the buffer the recording reads its input from and ``out`` the one
    it leaves the step's result in.  They are the same tensor when the mlp
    updates the residual stream in place; an mlp that returns a new tensor
    makes ``out`` a buffer of the graph's own pool.  Both stay referenced here
    for the life of the graph, so neither is ever handed back to the allocator
    while a replay can still write it.
    """

    def __init__(self, fwd: BatchedForward, steps: int, mlp: Callable[[int, torch.Tensor], torch.Tensor] | None):
        st = fwd.state
        self.fwd = fwd
        self.remaining = int(steps)
        self.x = torch.zeros((st.max_seqs, HIDDEN), dtype=torch.float32, device=st.device)
        host_seen, headroom = list(st._host_seen), st._min_headroom
        self.graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device=st.device)
        stream.wait_stream(torch.cuda.current_stream(st.device))
        with torch.cuda.stream(stream):
            with torch.cuda.graph(self.graph, stream=stream):
                out = fwd.step(self.x, mlp)
        torch.cuda.current_stream(st.device).wait_stream(stream)
        self.out = out
        # recording ran the host side of advance(); nothing ran on the device yet
        st._host_seen, st._min_headroom = host_seen, headroom

    def replay(self) -> torch.Tensor:
        """One token per sequence (input in ``x``); returns ``out``. Positions advance as with step()."""
        if self.remaining <= 0:
            raise RuntimeError("the graph's reserved steps are used up: capture again")
        st = self.fwd.state
        if max(st._host_seen) + 1 >= st.max_context:
            raise RuntimeError(f"context reaches max_context={st.max_context}")
        self.graph.replay()
        st._host_seen = [n + 1 for n in st._host_seen]
        st._min_headroom -= 1
        self.remaining -= 1
        return self.out
