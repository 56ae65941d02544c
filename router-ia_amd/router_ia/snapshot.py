"""Sequence snapshots: the attention state of one sequence as one device payload.

The reference keeps a sequence's state as per-layer tensors of its
``AttentionState`` (v2/src/router_ia/qwen36_attention_cache.py:27-92):
``linear_states[layer]`` [1, Hv, 128, 128] fp32, ``linear_conv_states[layer]``
[1, conv_dim, 4] (the last four conv inputs, oldest first, :207-209),
``full_keys`` / ``full_values[layer]`` [1, Hkv, T, 256] and ``tokens_seen``.
It has no way to save or reload them.  A ``SequenceSnapshot`` holds the same
information for one row of the batched pools as one contiguous device
payload, written and read by ``ria_seq_state_save`` / ``ria_seq_state_restore``:

    DeltaNet states  f32  [L_lin, Hv, 128, 128]
    conv rings       bf16 [L_lin, 4, conv_dim]         token t in slot t mod 4
    K tiles          kv   [L_full, pages, Hkv, 8, 4, 16, 8]   the cache's tile order
    V tiles          kv   [L_full, pages, Hkv, 256, 16]

each section on a 256-byte boundary, pages = ceil(T / 16), slots past T zero.
``to_reference`` / ``from_reference`` convert to and from the reference's
per-layer tensors, keyed by model layer (layer 4i+3 is full attention,
qwen36_40layer_loop.py:68-78), so a state can move between the two.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels as K

PAGE = K.PAGE_TOKENS
K_TILE = (8, 4, PAGE, 8)  # K tile axes: [dim % 64 / 8, dim / 64, token, dim % 8]


def _align256(x: int) -> int:
    return (x + 255) // 256 * 256


def linear_model_layers(num_linear_layers: int) -> list[int]:
    """Model layer of each DeltaNet layer index: 0, 1, 2, 4, 5, 6, 8, ... (layer 4i+3 is full attention)."""
    return [i + i // 3 for i in range(num_linear_layers)]


def full_model_layers(num_full_layers: int) -> list[int]:
    """Model layer of each full-attention layer index: 3, 7, 11, ..."""
    return [4 * i + 3 for i in range(num_full_layers)]


@dataclass
class SequenceSnapshot:
    payload: torch.Tensor  # uint8, on the device
    tokens: int            # tokens seen: position of the next token
    num_linear_layers: int
    num_full_layers: int
    num_v_heads: int
    num_kv_heads: int
    conv_dim: int
    kv_dtype: torch.dtype

    # ------------------------------------------------------------- layout
    @property
    def pages(self) -> int:
        return (self.tokens + PAGE - 1) // PAGE

    def _offsets(self) -> tuple[int, int, int, int, int]:
        lin = self.num_linear_layers * self.num_v_heads * 128 * 128 * 4
        conv = self.num_linear_layers * 4 * self.conv_dim * 2
        kv = self.num_full_layers * self.pages * self.num_kv_heads * PAGE * K.ATTN_HEAD_DIM * 2
        off_conv = _align256(lin)
        off_k = _align256(off_conv + conv)
        off_v = _align256(off_k + kv)
        return 0, off_conv, off_k, off_v, _align256(off_v + kv)

    @staticmethod
    def nbytes(num_linear_layers: int, num_v_heads: int, conv_dim: int, num_full_layers: int, num_kv_heads: int,
               tokens: int) -> int:
        return K.seq_state_bytes(num_linear_layers, num_v_heads, conv_dim, num_full_layers, num_kv_heads, tokens)

    def _section(self, start: int, nbytes: int, dtype: torch.dtype, shape: tuple[int, ...]) -> torch.Tensor:
        return self.payload[start:start + nbytes].view(dtype).reshape(shape)

    def linear_states(self) -> torch.Tensor:
        """[L_lin, Hv, 128, 128] fp32 view of the payload."""
        n = self.num_linear_layers * self.num_v_heads * 128 * 128 * 4
        return self._section(0, n, torch.float32, (self.num_linear_layers, self.num_v_heads, 128, 128))

    def conv_rings(self) -> torch.Tensor:
        """[L_lin, 4, conv_dim] bf16 view: token t's conv input in slot t mod 4."""
        off = self._offsets()[1]
        n = self.num_linear_layers * 4 * self.conv_dim * 2
        return self._section(off, n, torch.bfloat16, (self.num_linear_layers, 4, self.conv_dim))

    def _tiles(self, which: str) -> torch.Tensor:
        _, _, off_k, off_v, _ = self._offsets()
        n = self.num_full_layers * self.pages * self.num_kv_heads * PAGE * K.ATTN_HEAD_DIM * 2
        shape = (self.num_full_layers, self.pages, self.num_kv_heads)
        if which == "k":
            return self._section(off_k, n, self.kv_dtype, shape + K_TILE)
        return self._section(off_v, n, self.kv_dtype, shape + (K.ATTN_HEAD_DIM, PAGE))

    def keys(self) -> torch.Tensor:
        """[L_full, Hkv, T, 256] keys in token order (RoPE applied, as stored)."""
        t = self._tiles("k")  # [L, P, H, kk, g, tok, j]; dim = 64 g + 8 kk + j
        lf, p, h = t.shape[:3]
        out = t.permute(0, 2, 1, 5, 4, 3, 6).reshape(lf, h, p * PAGE, K.ATTN_HEAD_DIM)
        return out[:, :, :self.tokens]

    def values(self) -> torch.Tensor:
        """[L_full, Hkv, T, 256] values in token order."""
        t = self._tiles("v")  # [L, P, H, dim, tok]
        lf, p, h = t.shape[:3]
        return t.permute(0, 2, 1, 4, 3).reshape(lf, h, p * PAGE, K.ATTN_HEAD_DIM)[:, :, :self.tokens]

    # ------------------------------------------------------------- reference layout
    def to_reference(self) -> dict:
        """The reference's per-layer tensors (AttentionState fields), keyed by model layer."""
        states = self.linear_states()
        rings = self.conv_rings()
        slots = [(self.tokens - 4 + m) % 4 for m in range(4)]  # oldest .. newest input
        keys, values = self.keys(), self.values()
        return {
            "linear_states": {m: states[i].unsqueeze(0).clone()
                              for i, m in enumerate(linear_model_layers(self.num_linear_layers))},
            "linear_conv_states": {m: rings[i, slots].transpose(0, 1).unsqueeze(0).contiguous()
                                   for i, m in enumerate(linear_model_layers(self.num_linear_layers))},
            "full_keys": {m: keys[i].unsqueeze(0).contiguous()
                          for i, m in enumerate(full_model_layers(self.num_full_layers))},
            "full_values": {m: values[i].unsqueeze(0).contiguous()
                            for i, m in enumerate(full_model_layers(self.num_full_layers))},
            "tokens_seen": self.tokens,
        }

    @classmethod
    def from_reference(cls, state: dict, *, num_linear_layers: int, num_full_layers: int, num_v_heads: int = 32,
                       num_kv_heads: int = 2, conv_dim: int = 8192, kv_dtype: torch.dtype = torch.bfloat16,
                       device: torch.device | str = "cuda") -> "SequenceSnapshot":
        """Build a snapshot from the reference's per-layer tensors (missing layers start from zeros).

        Conv windows are taken as bf16 (the conv weight's dtype), KV in kv_dtype.
        """
        dev = torch.device(device)
        tokens = int(state["tokens_seen"])
        n = K.seq_state_bytes(num_linear_layers, num_v_heads, conv_dim, num_full_layers, num_kv_heads, tokens)
        snap = cls(torch.zeros(n, dtype=torch.uint8, device=dev), tokens, num_linear_layers, num_full_layers,
                   num_v_heads, num_kv_heads, conv_dim, kv_dtype)
        states, rings = snap.linear_states(), snap.conv_rings()
        slots = [(tokens - 4 + m) % 4 for m in range(4)]
        for i, m in enumerate(linear_model_layers(num_linear_layers)):
            if m in state.get("linear_states", {}):
                states[i] = state["linear_states"][m].reshape(num_v_heads, 128, 128).to(dev, torch.float32)
            if m in state.get("linear_conv_states", {}):
                win = state["linear_conv_states"][m].reshape(conv_dim, 4).to(dev, torch.bfloat16)
                rings[i, slots] = win.transpose(0, 1)
        p = snap.pages
        kt, vt = snap._tiles("k"), snap._tiles("v")
        for i, m in enumerate(full_model_layers(num_full_layers)):
            for name, tiles in (("full_keys", kt), ("full_values", vt)):
                if m not in state.get(name, {}):
                    continue
                x = state[name][m].reshape(num_kv_heads, -1, K.ATTN_HEAD_DIM)
                if x.shape[1] != tokens:
                    raise ValueError(f"{name}[{m}] holds {x.shape[1]} tokens, tokens_seen is {tokens}")
                full = torch.zeros((num_kv_heads, p * PAGE, K.ATTN_HEAD_DIM), device=dev, dtype=kv_dtype)
                full[:, :tokens] = x.to(dev, kv_dtype)
                if name == "full_keys":  # [H, P, tok, g, kk, j] -> [P, H, kk, g, tok, j]
                    tiles[i] = full.reshape(num_kv_heads, p, PAGE, 4, 8, 8).permute(1, 0, 4, 3, 2, 5)
                else:                    # [H, P, tok, dim] -> [P, H, dim, tok]
                    tiles[i] = full.reshape(num_kv_heads, p, PAGE, K.ATTN_HEAD_DIM).permute(1, 0, 3, 2)
        return snap

