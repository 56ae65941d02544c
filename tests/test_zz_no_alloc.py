"""GPU: ria_attn_decode_append_noalloc equals ria_attn_decode_append, with no workspace and no allocation.

The no-allocation entry point keeps the split-K partials in the library's own
device array instead of a caller workspace; the kernels are the same, so its
outputs and the tokens it appends into the pages must equal those of
ria_attn_decode_append bit for bit.  Two calls in a row, the second with a
smaller batch and shorter contexts, both through the C ABI.  Sizes whose
partials exceed the array are refused before any launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import announce
from router_ia import _native as nat
from router_ia import kernels as K
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState

pytestmark = pytest.mark.gpu


def _case(dev, batch, lo, hi, seed):
    lengths = W.ragged_lengths(seed, batch, lo, hi)
    st = BatchedAttentionState(batch, max(lengths) + 8, num_linear_layers=0, num_full_layers=1, device=dev,
                               page_shuffle_seed=seed)
    st.set_positions(lengths)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    st.kv.k.normal_(0.0, 1.0, generator=gen)
    st.kv.v.normal_(0.0, 1.0, generator=gen)
    q = torch.randn((batch, 16, 256), generator=gen, device=dev).to(torch.bfloat16)
    gate = torch.randn((batch, 16, 256), generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn((batch, 2, 256), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((batch, 2, 256), generator=gen, device=dev).to(torch.bfloat16)
    qn = 0.1 * torch.randn((256,), generator=gen, device=dev)
    kn = 0.1 * torch.randn((256,), generator=gen, device=dev)
    return st, lengths, (q, gate, k, v), (qn, kn)


def _call(st, inputs, norms, out, workspace):
    q, gate, k, v = inputs
    qn, kn = norms
    kc, vc = st.kv.layer(0)
    common = dict(positions=st.tokens_seen, ctx_lens=st.ctx_lens, max_ctx=st.max_seen + 1, inv_freq=st.inv_freq,
                  scale=st.scale, q_norm_weight=qn, k_norm_weight=kn)
    if workspace is None:
        return K.attn_decode_append_noalloc(q, gate, k, v, kc, vc, st.kv.page_table, out, **common)
    return K.attn_decode_append(q, gate, k, v, kc, vc, st.kv.page_table, out, workspace=workspace, **common)


@pytest.mark.parametrize("batch,lo,hi,seed", [(96, 200, 6000, 61), (5, 1, 900, 62)], ids=["B96", "B5-smaller"])
def test_noalloc_equals_the_workspace_entry_point(gpu, batch, lo, hi, seed):
    announce(f"no-alloc decode append: B={batch}, contexts U[{lo}, {hi}], vs ria_attn_decode_append")
    st, lengths, inputs, norms = _case(gpu, batch, lo, hi, seed)
    k0, v0 = st.kv.k.clone(), st.kv.v.clone()
    want = torch.empty((batch, 16, 256), device=gpu, dtype=torch.float32)
    _call(st, inputs, norms, want, st.workspace)
    k_want, v_want = st.kv.k.clone(), st.kv.v.clone()
    st.kv.k.copy_(k0)
    st.kv.v.copy_(v0)
    got = torch.full((batch, 16, 256), float("nan"), device=gpu, dtype=torch.float32)
    _call(st, inputs, norms, got, None)  # ria_attn_decode_append_noalloc
    torch.cuda.synchronize()
    assert torch.equal(got, want), "outputs differ from ria_attn_decode_append"
    assert torch.equal(st.kv.k, k_want) and torch.equal(st.kv.v, v_want), "appended pages differ"
    assert not torch.equal(st.kv.v, v0)  # the new tokens were written


def _noalloc_raw(lib, batch, max_ctx, split_tokens, phase):
    # every pointer null: the checks under test come first, and a regression
    # that skipped them would meet the null-pointer refusal, never a launch
    return lib.ria_attn_decode_append_noalloc(batch, 16, 2, None, 0, 4096, None, 0, 4096, None, 512, None, 512, None,
                                              None, None, 0, 1, None, 2048, None, None, 0, None, 1, max_ctx, None, 0,
                                              None, 0.0625, split_tokens, None, 0, phase, None)


def test_noalloc_refuses_sizes_beyond_its_array(gpu):
    announce("no-alloc decode append: sizes beyond the 16 MiB array are refused before any launch")
    lib = nat.load()
    # 4096 rows x 2 KV heads at long fixed splits: far more partials than 16 MiB
    need = lib.ria_attn_decode_workspace_bytes(4096, 16, 2, 32768, 64)
    assert need > 16 << 20
    assert _noalloc_raw(lib, 4096, 32768, 64, nat.RIA_ATTN_BOTH) == 3 and b"scratch" in lib.ria_last_error()


@pytest.mark.parametrize("phase", ["RIA_ATTN_SPLITK", "RIA_ATTN_COMBINE"])
def test_noalloc_refuses_a_single_phase(gpu, phase):
    announce(f"no-alloc decode append: {phase} alone is refused (partials do not outlive a call)")
    lib = nat.load()
    assert _noalloc_raw(lib, 4, 4096, 0, getattr(nat, phase)) == 1 and b"RIA_ATTN_BOTH" in lib.ria_last_error()
