"""Host logic of the drop-in attention cache (no GPU needed).

The limit tests check the semantics the reference's unit tests pin
(v2/tests/test_qwen36_attention_cache.py): a KV limit raises before the cache
is mutated, with the messages its callers match, and the byte budget counts
the stored tensors' own dtype.
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


def _kv(fill: float, heads: int = 2, dim: int = 8, dtype: torch.dtype = torch.float32):
    """One decode token's k and v, [batch=1, kv heads, 1 token, head dim]."""
    k = torch.full((1, heads, 1, dim), fill, dtype=dtype)
    return k, k + 0.5


def _fill(state: AttentionState, layer: int, count: int) -> None:
    """Append `count` tokens at positions 0 .. count - 1 (the caller advances tokens_seen)."""
    for pos in range(count):
        state.tokens_seen = pos
        _append_full_kv(state, layer, *_kv(float(pos)))


@pytest.mark.parametrize("limit", [1, 5])
def test_context_limit_refuses_the_next_token_and_leaves_the_cache_as_it_was(limit: int) -> None:
    # qwen36_attention_cache.py:341-352: the check runs before any tensor is touched
    state = AttentionState(max_context_tokens=limit)
    _fill(state, 2, limit)
    keys_before = state.full_keys[2].clone()
    values_before = state.full_values[2].clone()
    state.tokens_seen = limit
    with pytest.raises(RuntimeError, match=rf"max_context_tokens={limit}\b"):
        _append_full_kv(state, 2, *_kv(99.0))
    assert torch.equal(state.full_keys[2], keys_before)
    assert torch.equal(state.full_values[2], values_before)
    snap = state.snapshot()
    assert (snap["absolute_position"], snap["full_tokens_resident"], snap["kv_start_position"]) == (limit, limit, 0)
    assert snap["full_token_entries"] == limit


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_byte_budget_counts_the_stored_dtype_and_refuses_before_mutation(dtype: torch.dtype) -> None:
    # qwen36_attention_cache.py:327-339, 353-364: bytes are those of the tensors
    # as given (element_size of their dtype), both k and v of every layer
    k, v = _kv(1.0, heads=2, dim=8, dtype=dtype)
    per_token = 2 * k.numel() * k.element_size()
    budget = 3 * per_token + per_token // 2  # room for three tokens, not four
    state = AttentionState(max_full_kv_bytes=budget)
    for pos in range(3):
        state.tokens_seen = pos
        _append_full_kv(state, 0, k, v)
    assert state.snapshot()["full_bytes"] == 3 * per_token
    state.tokens_seen = 3
    with pytest.raises(RuntimeError, match=r"max_full_kv_bytes"):
        _append_full_kv(state, 0, k, v)
    assert state.full_keys[0].shape[-2] == 3 and state.full_values[0].shape[-2] == 3
    assert state.snapshot()["full_bytes"] == 3 * per_token
    # a second layer's tokens count against the same budget
    state.tokens_seen = 0
    with pytest.raises(RuntimeError, match=r"max_full_kv_bytes"):
        _append_full_kv(state, 7, k, v)
    assert 7 not in state.full_keys


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
