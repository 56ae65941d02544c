"""Batched attention state: B sequences decoding the 40-layer hybrid stack together.

The reference keeps one ``AttentionState`` per sequence with per-layer dicts
of tensors (v2/src/router_ia/qwen36_attention_cache.py:27-92) and advances it
one sequence at a time.  Here all sequences live in fixed HBM pools so every
layer is one kernel launch over the whole batch:

    DeltaNet state   f32  [L_lin, B, Hv, 128, 128]   (2 MiB per sequence-layer)
    conv ring        bf16 [L_lin, B, 4, conv_dim]     (slot = token index mod 4)
    K / V pages      bf16 per full layer (see paged_kv)
    tokens_seen      i32  [B] absolute position of the next token (RoPE
                     position, conv ring index and KV slot of that token)
    ctx_lens         i32  [B] tokens_seen + 1, the attention's context
                     (tokens_seen and ctx_lens are the two rows of one
                     tensor: update them in place, never rebind them)

Per token the caller runs ``linear_step`` / ``full_step`` for each layer and
then ``advance()``, the batched equivalent of the reference caller bumping
``tokens_seen`` after all 40 layers (v2/src/router_ia/qwen36_chat_batch.py:204-206).
A prompt enters one row at a time through ``begin_prefill`` /
``linear_prefill`` / ``full_prefill`` / ``end_prefill`` (chunked DeltaNet and
causal attention prefill), equal to decoding it token by token.

``save_row`` / ``restore_row`` move one row's whole state (DeltaNet states,
conv ring, KV pages) to and from a ``SequenceSnapshot``, e.g. to preempt a
sequence and resume it later in any row.

The norms on either side of the attention arithmetic run inside the same
launches when their fp32 weights are passed: the gated RMSNorm of the
DeltaNet read-out (``z``, ``norm_weight``; :268-271) and the q_norm / k_norm
RMSNorms before RoPE (``q_norm_weight``, ``k_norm_weight``; :302-305).
"""

from __future__ import annotations

import torch

from . import _native as nat
from . import kernels as K
from .paged_kv import PagedKVCache
from .snapshot import SequenceSnapshot


def rope_inv_freq(theta: float, rope_dim: int) -> torch.Tensor:
    """inv_freq exactly as the reference computes it in fp32 (qwen36_attention_cache.py:140-143)."""
    if rope_dim <= 0 or rope_dim % 2:
        raise ValueError(f"Invalid rotary dimension: {rope_dim}")
    return 1.0 / (theta ** (torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim))


class BatchedAttentionState:
    def __init__(
        self,
        max_seqs: int,
        max_context: int,
        *,
        num_linear_layers: int = 30,
        num_full_layers: int = 10,
        num_k_heads: int = 16,
        num_v_heads: int = 32,
        num_q_heads: int = 16,
        num_kv_heads: int = 2,
        rope_theta: float = 10_000_000.0,
        rope_dim: int = 64,
        num_pages: int | None = None,
        device: str | torch.device = "cuda",
        page_shuffle_seed: int | None = None,
        split_tokens: int = 0,
        kv_dtype: torch.dtype = torch.bfloat16,
        prefill_segment_tokens: int = 4096,
        fused_append: bool = True,
    ):
        self.device = torch.device(device)
        # decode steps append each row's k, v inside the attention's combine launch (ria_attn_decode_append)
        self.fused_append = bool(fused_append)
        if self.device.type != "cuda":
            raise RuntimeError("BatchedAttentionState needs a ROCm GPU device; there is no CPU implementation")
        nat.load()
        self.max_seqs = int(max_seqs)
        self.max_context = int(max_context)
        self.num_linear_layers = num_linear_layers
        self.num_full_layers = num_full_layers
        self.num_k_heads = num_k_heads
        self.num_v_heads = num_v_heads
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.conv_dim = K.conv_dim(num_k_heads, num_v_heads)
        self.split_tokens = split_tokens
        dev = self.device
        self.linear_states = torch.zeros((num_linear_layers, max_seqs, num_v_heads, 128, 128),
                                         dtype=torch.float32, device=dev)
        self.conv_rings = torch.zeros((num_linear_layers, max_seqs, K.CONV_RING, self.conv_dim),
                                      dtype=torch.bfloat16, device=dev)
        max_pages_per_seq = (max_context + K.PAGE_TOKENS - 1) // K.PAGE_TOKENS
        if num_pages is None:
            num_pages = max_seqs * max_pages_per_seq
        self.kv = PagedKVCache(num_full_layers, num_pages, max_seqs, max_pages_per_seq,
                               num_kv_heads=num_kv_heads, device=dev, shuffle_seed=page_shuffle_seed,
                               dtype=kv_dtype)
        # positions and context lengths are the two rows of one tensor, so a
        # decode step advances both with one launch
        self._pos_ctx = torch.stack([torch.zeros(max_seqs, dtype=torch.int32, device=dev),
                                     torch.ones(max_seqs, dtype=torch.int32, device=dev)])
        self.tokens_seen = self._pos_ctx[0]
        self.ctx_lens = self._pos_ctx[1]
        self._host_seen = [0] * max_seqs
        self._min_headroom = 0  # min over rows of (KV capacity - tokens seen)
        self.inv_freq = rope_inv_freq(rope_theta, rope_dim).to(dev)
        self.scale = 256 ** -0.5
        self._size_workspace()
        # DeltaNet prefill runs prompts in segments of this many tokens; its
        # workspace (about 75 KB per token) is allocated on the first prefill
        self.prefill_segment_tokens = max(64, int(prefill_segment_tokens))
        self.prefill_workspace: torch.Tensor | None = None
        self.prefill_stage: torch.Tensor | None = None  # fp16 keys of a prompt from slot 0 (attention prefill)

    def _size_workspace(self) -> None:
        ws = K.attn_decode_workspace_bytes(self.max_seqs, self.num_q_heads, self.num_kv_heads, self.max_context,
                                           self.split_tokens)
        self.workspace = torch.empty(max(ws, 4), dtype=torch.uint8, device=self.device)

    # ---------------------------------------------------------------- bookkeeping
    def set_positions(self, lengths: list[int]) -> None:
        """Declare that row b already holds lengths[b] tokens of state and KV."""
        if len(lengths) != self.max_seqs:
            raise ValueError("one length per sequence row is required")
        if max(lengths) >= self.max_context:
            raise ValueError("a context length reaches max_context")
        self._host_seen = [int(x) for x in lengths]
        self._ensure([n + 1 for n in self._host_seen])
        self.tokens_seen.copy_(torch.tensor(self._host_seen, dtype=torch.int32))
        self.ctx_lens.copy_(self.tokens_seen + 1)

    def reserve(self, extra_tokens: int) -> None:
        """Allocate KV pages so every row can take `extra_tokens` more tokens without host work."""
        self._ensure([min(n + extra_tokens, self.max_context) for n in self._host_seen])

    def _ensure(self, n_tokens: list[int]) -> None:
        self.kv.ensure_many(n_tokens)
        self._min_headroom = min(self.kv.alloc.capacity_tokens(r) - self._host_seen[r] for r in range(self.max_seqs))

    def reset_row(self, row: int) -> None:
        self.linear_states[:, row].zero_()
        self.conv_rings[:, row].zero_()
        self.kv.release(row)
        self._min_headroom = 0
        self._host_seen[row] = 0
        self.tokens_seen[row] = 0
        self.ctx_lens[row] = 1

    def advance(self) -> None:
        self._host_seen = [n + 1 for n in self._host_seen]
        self._min_headroom -= 1
        self._pos_ctx.add_(1)  # tokens_seen and ctx_lens

    @property
    def max_seen(self) -> int:
        return max(self._host_seen)

    # ---------------------------------------------------------------- layer steps
    def linear_step(
        self,
        layer: int,
        mixed_qkv: torch.Tensor,
        conv_weight: torch.Tensor,
        gate_a: torch.Tensor,
        gate_b: torch.Tensor,
        *,
        gate_mode: int = nat.RIA_GATE_PRECOMPUTED,
        A_log: torch.Tensor | None = None,
        dt_bias: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
        out_dtype: torch.dtype = torch.bfloat16,
        z: torch.Tensor | None = None,
        norm_weight: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """One Gated DeltaNet token for every row (conv + recurrence + read-out [+ gated RMSNorm])."""
        if out is None:
            out = torch.empty((self.max_seqs, self.num_v_heads, 128), dtype=out_dtype, device=self.device)
        return K.gdn_decode(
            mixed_qkv, self.linear_states[layer], gate_a, gate_b, out,
            num_k_heads=self.num_k_heads, num_v_heads=self.num_v_heads, fuse_conv=True,
            conv_weight=conv_weight, conv_ring=self.conv_rings[layer], conv_pos=self.tokens_seen,
            gate_mode=gate_mode, A_log=A_log, dt_bias=dt_bias, z=z, norm_weight=norm_weight)

    def full_step(
        self,
        layer: int,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        gate: torch.Tensor,
        *,
        out: torch.Tensor | None = None,
        out_dtype: torch.dtype = torch.bfloat16,
        q_norm_weight: torch.Tensor | None = None,
        k_norm_weight: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Append this token's k, v (RoPE on k) and attend over each row's whole context."""
        max_ctx = self.max_seen + 1
        if max_ctx > self.max_context:
            raise RuntimeError(f"context {max_ctx} exceeds max_context={self.max_context}")
        if self._min_headroom < 1:
            self._ensure([n + 1 for n in self._host_seen])
        k_cache, v_cache = self.kv.layer(layer)
        if out is None:
            out = torch.empty((self.max_seqs, self.num_q_heads, 256), dtype=out_dtype, device=self.device)
        if self.fused_append and k.dtype == q.dtype and v.dtype == q.dtype and gate.dtype == q.dtype:
            # no append launch: the attention's combine launch writes each row's token (slot tokens_seen = ctx - 1)
            return K.attn_decode_append(q, gate, k, v, k_cache, v_cache, self.kv.page_table, out,
                                        positions=self.tokens_seen, ctx_lens=self.ctx_lens, max_ctx=max_ctx,
                                        inv_freq=self.inv_freq, scale=self.scale, workspace=self.workspace,
                                        split_tokens=self.split_tokens, q_norm_weight=q_norm_weight,
                                        k_norm_weight=k_norm_weight)
        K.kv_append(k, v, k_cache, v_cache, self.kv.page_table, positions=self.tokens_seen,
                    slots=self.tokens_seen, inv_freq=self.inv_freq, k_norm_weight=k_norm_weight)
        return K.attn_decode(q, gate, k_cache, v_cache, self.kv.page_table, out, positions=self.tokens_seen,
                             ctx_lens=self.ctx_lens, max_ctx=max_ctx, inv_freq=self.inv_freq, scale=self.scale,
                             workspace=self.workspace, split_tokens=self.split_tokens, q_norm_weight=q_norm_weight)

    # ---------------------------------------------------------------- prompt prefill (one row)
    # A prompt enters one sequence row at a time: begin_prefill(row, L), then
    # linear_prefill / full_prefill for every layer, then end_prefill(row, L).
    # The result equals L decode steps of that row (the reference prefills
    # token by token, qwen36_chat_batch.py:255-258).
    def begin_prefill(self, row: int, length: int) -> None:
        """Reserve KV pages for `length` more tokens of `row` (plus the next decode token)."""
        target = self._host_seen[row] + length + 1
        if target > self.max_context:
            raise RuntimeError(f"prompt of {length} tokens exceeds max_context={self.max_context}")
        self._ensure([target if r == row else n + 1 for r, n in enumerate(self._host_seen)])

    def _prefill_workspace(self, length: int) -> torch.Tensor:
        seg = min(length, self.prefill_segment_tokens)
        need = K.gdn_prefill_workspace_bytes(self.num_k_heads, self.num_v_heads, max(seg, 64))
        if self.prefill_workspace is None or self.prefill_workspace.numel() < need:
            self.prefill_workspace = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self.prefill_workspace

    def linear_prefill(
        self,
        layer: int,
        row: int,
        mixed_qkv: torch.Tensor,
        conv_weight: torch.Tensor,
        gate_a: torch.Tensor,
        gate_b: torch.Tensor,
        *,
        gate_mode: int = nat.RIA_GATE_PRECOMPUTED,
        A_log: torch.Tensor | None = None,
        dt_bias: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
        out_dtype: torch.dtype = torch.bfloat16,
        z: torch.Tensor | None = None,
        norm_weight: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """A prompt's Gated DeltaNet tokens for one row (chunked prefill); mixed_qkv [L, conv_dim]."""
        length = int(mixed_qkv.shape[0])
        if out is None:
            out = torch.empty((length, self.num_v_heads, 128), dtype=out_dtype, device=self.device)
        return K.gdn_prefill(
            mixed_qkv, self.linear_states[layer, row], gate_a, gate_b, out,
            num_k_heads=self.num_k_heads, num_v_heads=self.num_v_heads, conv_weight=conv_weight,
            conv_ring=self.conv_rings[layer, row], conv_pos=self._host_seen[row],
            workspace=self._prefill_workspace(length), gate_mode=gate_mode, A_log=A_log, dt_bias=dt_bias, z=z,
            norm_weight=norm_weight)

    def full_prefill(
        self,
        layer: int,
        row: int,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        gate: torch.Tensor,
        *,
        out: torch.Tensor | None = None,
        q_norm_weight: torch.Tensor | None = None,
        k_norm_weight: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Append a prompt's k, v (RoPE on k) to one row and run its causal attention; q, gate [L, Hq, 256]."""
        k_cache, v_cache = self.kv.layer(layer)
        start = self._host_seen[row]
        # a prompt that starts the row attends over fp16 copies of its own keys (the stage)
        stage = self._prefill_stage(int(q.shape[0])) if start == 0 else None
        return K.attn_prefill(q, k, v, gate, k_cache, v_cache, self.kv.page_table[row], out,
                              start=start, inv_freq=self.inv_freq, scale=self.scale,
                              q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight, stage=stage)

    def _prefill_stage(self, length: int) -> torch.Tensor:
        need = K.prefill_stage_bytes(length, self.num_kv_heads)
        if self.prefill_stage is None or self.prefill_stage.numel() < need:
            self.prefill_stage = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self.prefill_stage

    def end_prefill(self, row: int, length: int) -> None:
        """The row's position moves past the prompt (after every layer has run it)."""
        self._host_seen[row] += length
        self.tokens_seen[row] += length
        self.ctx_lens[row] += length
        self._min_headroom = min(self.kv.alloc.capacity_tokens(r) - self._host_seen[r] for r in range(self.max_seqs))

    # ---------------------------------------------------------------- snapshots
    def save_row(self, row: int, out: torch.Tensor | None = None) -> SequenceSnapshot:
        """Copy row `row`'s DeltaNet states, conv rings and KV pages into a snapshot (ria_seq_state_save)."""
        tokens = self._host_seen[row]
        n = SequenceSnapshot.nbytes(self.num_linear_layers, self.num_v_heads, self.conv_dim, self.num_full_layers,
                                    self.num_kv_heads, tokens)
        if out is None:
            out = torch.empty(n, dtype=torch.uint8, device=self.device)
        elif out.numel() < n:
            raise ValueError(f"snapshot buffer holds {out.numel()} bytes, {n} needed")
        K.seq_state_save(self.linear_states, self.conv_rings, self.kv.k, self.kv.v, self.kv.page_table, row=row,
                         tokens=tokens, payload=out)
        return SequenceSnapshot(out[:n], tokens, self.num_linear_layers, self.num_full_layers, self.num_v_heads,
                                self.num_kv_heads, self.conv_dim, self.kv.dtype)

    def restore_row(self, row: int, snap: SequenceSnapshot) -> None:
        """Make row `row` continue the snapshot's sequence: new pages, then ria_seq_state_restore."""
        shape = (snap.num_linear_layers, snap.num_full_layers, snap.num_v_heads, snap.num_kv_heads, snap.conv_dim,
                 snap.kv_dtype)
        mine = (self.num_linear_layers, self.num_full_layers, self.num_v_heads, self.num_kv_heads, self.conv_dim,
                self.kv.dtype)
        if shape != mine:
            raise ValueError(f"snapshot shapes {shape} do not match this state's {mine}")
        if snap.tokens + 1 > self.max_context:
            raise RuntimeError(f"snapshot of {snap.tokens} tokens exceeds max_context={self.max_context}")
        # room first: releasing the row's pages and then failing to find new
        # ones would leave the row with neither its old state nor the new one
        need = (snap.tokens + 1 + K.PAGE_TOKENS - 1) // K.PAGE_TOKENS
        if need > self.kv.alloc.max_pages_per_seq:
            raise RuntimeError(f"snapshot of {snap.tokens} tokens needs {need} pages, the page table holds "
                               f"{self.kv.alloc.max_pages_per_seq}")
        if need > self.kv.alloc.free_pages + len(self.kv.alloc.tables[row]):
            raise RuntimeError(f"KV page pool exhausted: the snapshot needs {need} pages, "
                               f"{self.kv.alloc.free_pages + len(self.kv.alloc.tables[row])} available to row {row}")
        self.kv.release(row)
        self.kv.ensure(row, snap.tokens + 1)
        K.seq_state_restore(self.linear_states, self.conv_rings, self.kv.k, self.kv.v, self.kv.page_table, row=row,
                            tokens=snap.tokens, payload=snap.payload)
        self._host_seen[row] = snap.tokens
        self.tokens_seen[row] = snap.tokens
        self.ctx_lens[row] = snap.tokens + 1
        self._min_headroom = min(self.kv.alloc.capacity_tokens(r) - self._host_seen[r] for r in range(self.max_seqs))

    # ---------------------------------------------------------------- inspection
    def gather_kv(self, layer: int, start: int, count: int) -> tuple[torch.Tensor, torch.Tensor]:
        k_cache, v_cache = self.kv.layer(layer)
        return K.kv_gather(k_cache, v_cache, self.kv.page_table, batch=self.max_seqs, start=start, count=count)

    def resident_bytes(self) -> dict[str, int]:
        return {
            "linear_bytes": self.linear_states.numel() * 4,
            "linear_conv_bytes": self.conv_rings.numel() * 2,
            "full_bytes_allocated": self.kv.k.numel() * 2 + self.kv.v.numel() * 2,
        }
