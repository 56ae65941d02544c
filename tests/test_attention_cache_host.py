"""Host logic of the drop-in attention cache (no GPU needed).

The first two tests restate the reference's own unit tests
(v2/tests/test_qwen36_attention_cache.py:15-52) against this package's
``router_ia.qwen36_attention_cache``: same inputs, same assertions.
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch

from router_ia import qwen36_attention_cache as ac
from router_ia.qwen36_attention_cache import AttentionState, _append_full_kv

SNAPSHOT_KEYS = [
    "tokens_seen", "absolute_position", "kv_start_position", "full_layers_cached", "full_tokens",
    "full_tokens_resident", "full_token_entries", "full_bytes", "max_context_tokens", "max_full_kv_bytes",
    "linear_layers_cached", "linear_bytes", "linear_conv_layers_cached", "linear_conv_bytes", "bytes",
]


def _token() -> tuple[torch.Tensor, torch.Tensor]:
    # (batch, kv_heads, sequence, head_dim), matching the cache layout.
    return torch.zeros((1, 1, 1, 2)), torch.zeros((1, 1, 1, 2))


def test_full_kv_growth_stops_before_exceeding_context_limit() -> None:
    state = AttentionState(max_context_tokens=3)
    for absolute_position in range(3):
        state.tokens_seen = absolute_position
        key, value = _token()
        _append_full_kv(state, 0, key, value)
        assert state.full_keys[0].shape[-2] <= 3
        assert state.full_values[0].shape[-2] <= 3
    state.tokens_seen = 3
    key, value = _token()
    with pytest.raises(RuntimeError, match=r"max_context_tokens=3"):
        _append_full_kv(state, 0, key, value)
    stats = state.snapshot()
    assert state.full_keys[0].shape[-2] == 3
    assert stats["absolute_position"] == 3
    assert stats["full_tokens_resident"] == 3
    assert stats["kv_start_position"] == 0


def test_full_kv_growth_stops_before_exceeding_byte_budget() -> None:
    key, value = _token()
    token_bytes = key.numel() * key.element_size() + value.numel() * value.element_size()
    state = AttentionState(max_full_kv_bytes=token_bytes * 2)
    for absolute_position in range(2):
        state.tokens_seen = absolute_position
        _append_full_kv(state, 0, key, value)
        assert state.snapshot()["full_bytes"] <= token_bytes * 2
    state.tokens_seen = 2
    with pytest.raises(RuntimeError, match=r"max_full_kv_bytes"):
        _append_full_kv(state, 0, key, value)
    assert state.full_keys[0].shape[-2] == 2
    assert state.snapshot()["full_bytes"] == token_bytes * 2


def test_append_keeps_tokens_in_order() -> None:
    state = AttentionState()
    for t in range(5):
        k = torch.full((1, 2, 1, 4), float(t))
        _append_full_kv(state, 3, k, -k)
    assert torch.equal(state.full_keys[3][0, 0, :, 0], torch.arange(5, dtype=torch.float32))
    assert torch.equal(state.full_values[3], -state.full_keys[3])
    snap = state.snapshot()
    assert snap["full_token_entries"] == 5 and snap["full_layers_cached"] == 1


def test_configure_rejects_negative_limits() -> None:
    state = AttentionState()
    with pytest.raises(ValueError):
        state.configure(max_context_tokens=-1)
    with pytest.raises(ValueError):
        state.configure(max_full_kv_bytes=-1)
    state.configure(max_context_tokens=7, max_full_kv_bytes=9)
    assert (state.max_context_tokens, state.max_full_kv_bytes) == (7, 9)


def test_snapshot_and_stats_keys_match_reference() -> None:
    assert list(AttentionState().snapshot()) == SNAPSHOT_KEYS
    assert list(ac.stats(Path("/nonexistent/root/for/stats"))) == SNAPSHOT_KEYS
    assert all(v == 0 for v in ac.stats(Path("/nonexistent/root/for/stats")).values())


def test_registry_semantics(tmp_path: Path) -> None:
    s1 = ac.state_for(tmp_path, "cpu")
    assert ac.state_for(tmp_path / ".", "cpu") is s1  # keyed by resolved path
    s1.tokens_seen = 5
    s1.linear_states[0] = torch.zeros(1)
    ac.state_for(tmp_path, "cpu")
    assert s1.tokens_seen == 5  # same device: kept
    ac.state_for(tmp_path, "meta")
    assert s1.tokens_seen == 0 and not s1.linear_states  # device change resets
    other = AttentionState()
    ac.activate(tmp_path, other)
    assert ac.active(tmp_path, "meta") is other
    ac.deactivate(tmp_path)
    assert ac.active(tmp_path, "meta") is s1
    assert ac.reset(tmp_path) is s1
    ac.deactivate(tmp_path)


def test_constants_match_reference() -> None:
    assert ac.ROPE_THETA == 10_000_000.0
    assert ac.ROPE_DIM == 64
    assert ac.LINEAR_CONV_KERNEL == ac.LINEAR_CONV_STATE == 4
    assert ac.LINEAR_CONV_DIM == 8192


def test_gpu_only_functions_refuse_cpu_tensors() -> None:
    x = torch.zeros((1, 32, 128))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac._l2norm(x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac._apply_rope(torch.zeros(1, 16, 1, 256), torch.zeros(1, 2, 1, 256), 3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac._rope(3, torch.device("cpu"), torch.float32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac._causal_conv1d_step(AttentionState(), 0, torch.zeros(1, 8192), torch.zeros(8192, 1, 4))


def test_conv_step_shape_errors_match_reference() -> None:
    state = AttentionState()
    with pytest.raises(ValueError, match="Unexpected mixed_qkv shape"):
        ac._causal_conv1d_step(state, 0, torch.zeros(2, 8192), torch.zeros(8192, 1, 4))
    with pytest.raises(ValueError, match="Unexpected conv weight shape"):
        ac._causal_conv1d_step(state, 0, torch.zeros(1, 8192), torch.zeros(8192, 4))
    with pytest.raises(ValueError, match="Unexpected conv weight shape"):
        ac._causal_conv1d_step(state, 0, torch.zeros(1, 8192), torch.zeros(8192, 1, 3))


def test_step_attention_refuses_cpu_device(tmp_path: Path) -> None:
    from safetensors.torch import save_file

    save_file({"model.language_model.layers.0.linear_attn.in_proj_qkv.weight": torch.zeros(2, 2),
               "model.language_model.layers.0.input_layernorm.weight": torch.zeros(2048)},
              str(tmp_path / "model.safetensors"))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac.step_attention(tmp_path, 0, torch.zeros(1, 2048), "cpu")


class _HostPages:
    """A stand-in for a layer's KV pages on the CPU: gather(count) returns the first `count` tokens."""

    num_kv_heads = 2
    device = torch.device("cpu")

    def __init__(self, dtype: torch.dtype, tokens: int):
        g = torch.Generator().manual_seed(tokens)
        self.dtype = dtype
        self.k = torch.randn((1, 2, tokens, 256), generator=g).to(torch.float16)
        self.v = torch.randn((1, 2, tokens, 256), generator=g).to(torch.float16)
        self.gathered = 0

    def gather(self, count: int):
        self.gathered += 1
        return self.k[:, :, :count], self.v[:, :, :count]


def test_paged_kv_tensor_behaves_as_the_reference_cache_tensor() -> None:
    pages = _HostPages(torch.float32, 40)
    k = ac.PagedKVTensor(pages, "k", 33)
    v = ac.PagedKVTensor(pages, "v", 33)
    # metadata without touching the pages
    assert isinstance(k, torch.Tensor) and k.shape == (1, 2, 33, 256) and k.shape[-2] == 33
    assert k.dtype == torch.float32 and not k.requires_grad and not v.requires_grad
    assert k.numel() * k.element_size() == 2 * 33 * 256 * 4  # the bytes the reference's fp32 tensor holds
    assert pages.gathered == 0
    # every use reads the first 33 tokens, converted to the tensor's dtype
    want_k, want_v = pages.k[:, :, :33].float(), pages.v[:, :, :33].float()
    assert torch.equal(k.detach().float(), want_k)
    assert torch.equal(v.detach().clone(), want_v)
    assert torch.equal(k + 1, want_k + 1)
    assert torch.equal(k[:, :, 5:7], want_k[:, :, 5:7])
    assert torch.equal(torch.cat((k, want_k[:, :, :1]), dim=2)[:, :, 33], want_k[:, :, 0])
    assert torch.equal(k.repeat_interleave(8, dim=1).float(), want_k.repeat_interleave(8, dim=1))
    torch.testing.assert_close(k, want_k)
    assert type(k.detach()) is torch.Tensor  # what a caller keeps is a plain tensor
    # a tensor taken earlier keeps its own length
    assert ac.PagedKVTensor(pages, "k", 7).shape[-2] == 7


def test_snapshot_and_limits_count_the_reference_bytes_for_paged_tensors() -> None:
    pages = _HostPages(torch.float32, 40)
    state = AttentionState()
    state.full_keys[3] = ac.PagedKVTensor(pages, "k", 10)
    state.full_values[3] = ac.PagedKVTensor(pages, "v", 10)
    state.tokens_seen = 10
    snap = state.snapshot()
    assert snap["full_tokens_resident"] == 10 and snap["full_layers_cached"] == 1
    assert snap["full_bytes"] == 2 * 2 * 10 * 256 * 4
    assert pages.gathered == 0  # snapshot() reads shapes only
    state.configure(max_full_kv_bytes=2 * 2 * 10 * 256 * 4 + 1)
    with pytest.raises(RuntimeError, match="max_full_kv_bytes"):
        ac._check_full_kv_limits(state, 3, append_bytes=2 * 2 * 256 * 4)
    state.configure(max_context_tokens=10)
    with pytest.raises(RuntimeError, match="max_context_tokens=10"):
        ac._check_full_kv_limits(state, 3, append_bytes=0)


def test_replaceable_seams_are_module_attributes() -> None:
    # the probes of the reference swap these module attributes; the layers look them up at call time
    for name in ("rmsnorm", "gated_rmsnorm", "_l2norm", "_apply_rope", "_causal_conv1d_step", "_append_full_kv",
                 "_projection", "step_attention"):
        assert callable(getattr(ac, name))
    assert ac._HIP_RMSNORM is ac.rmsnorm and ac._HIP_CONV_STEP is ac._causal_conv1d_step
    assert ac._HIP_APPEND_FULL_KV is ac._append_full_kv and ac._HIP_APPLY_ROPE is ac._apply_rope
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ac.rmsnorm(torch.zeros(1, 8), torch.zeros(8))
    with pytest.raises(ValueError, match="x/z shape mismatch"):
        ac.gated_rmsnorm(torch.zeros(1, 32, 128), torch.zeros(1, 32, 64), torch.zeros(128))
