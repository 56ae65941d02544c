"""Committed fixtures (tests/golden/*.safetensors, written by make_golden.py).

The oracle is checked against them on the CPU, and the HIP kernels are
checked against the same fixtures on the GPU.
"""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import load_file

from conftest import GOLDEN, announce
from helpers import assert_act_close, assert_state_close
from oracle import chunked as C
from oracle import qwen36_cpu as O


def _fx(name: str) -> dict[str, torch.Tensor]:
    return load_file(str(GOLDEN / f"{name}.safetensors"))


# ----------------------------------------------------------------------------- oracle (CPU)
def test_oracle_recurrent_rule_matches_fixture():
    f = _fx("delta_recurrent_L64_H4")
    o, s = C.recurrent_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], f["state0"])
    torch.testing.assert_close(o, f["out"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s, f["state"], rtol=1e-5, atol=1e-6)


def test_oracle_chunk_rule_matches_fixture():
    f = _fx("delta_chunk_L130_H4")
    o, s = C.chunk_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], f["state0"])
    torch.testing.assert_close(o, f["out"], rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(s, f["state"], rtol=2e-4, atol=2e-5)


def test_oracle_conv_matches_fixture():
    f = _fx("conv_update_C512_T5")
    state = f["state0"]
    for t in range(5):
        out, state = O.causal_conv1d_step(state, f["x"][t:t + 1], f["weight"].reshape(512, 1, 4))
        assert torch.equal(out[0], f["out"][t])
    assert torch.equal(state, f["state"])


def test_oracle_rope_matches_fixture():
    f = _fx("rope_tables")
    for i, pos in enumerate(f["positions"].tolist()):
        cos, sin = O.rope(pos)
        torch.testing.assert_close(cos, f["cos"][i], rtol=0, atol=1e-6)
        torch.testing.assert_close(sin, f["sin"][i], rtol=0, atol=1e-6)


def test_oracle_decode_attention_matches_fixture():
    f = _fx("decode_attention_T33")
    out = O.attention_over_cache(f["q_rot"][None], f["k"][None], f["v"][None], f["gate"][None])
    torch.testing.assert_close(out[0], f["out"], rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------------------- kernels (GPU)
@pytest.mark.gpu
def test_gdn_kernel_matches_recurrent_fixture(gpu):
    announce("golden: gdn_decode (unfused) vs transformers recurrent rule, 4 heads, 64 tokens")
    from router_ia import kernels as K

    f = _fx("delta_recurrent_L64_H4")
    state = f["state0"][None].clone().to(gpu)
    outs = []
    for t in range(64):
        mixed = torch.cat([f["q"][t].reshape(-1), f["k"][t].reshape(-1), f["v"][t].reshape(-1)])[None].to(gpu)
        out = torch.empty((1, 4, 128), device=gpu)
        K.gdn_decode(mixed, state, f["g"][t][None].to(gpu), f["beta"][t][None].to(gpu), out, num_k_heads=4,
                     num_v_heads=4, fuse_conv=False)
        outs.append(out[0].cpu())
    assert_act_close(torch.stack(outs), f["out"], "outputs")
    assert_state_close(state[0].cpu(), f["state"], "final state")


@pytest.mark.gpu
def test_conv_kernel_matches_fixture(gpu):
    announce("golden: conv1d_step vs transformers causal_conv1d_update")
    from helpers import ring_to_window
    from router_ia import kernels as K

    f = _fx("conv_update_C512_T5")
    ring = f["state0"][0].transpose(0, 1).contiguous()[None].to(gpu)  # window slots == ring slots at step 4
    w = f["weight"].reshape(512, 1, 4).contiguous().to(gpu)
    for t in range(5):
        out = torch.empty((1, 512), dtype=torch.bfloat16, device=gpu)
        K.conv1d_step(f["x"][t:t + 1].to(gpu), w, ring, out, conv_pos=4 + t)
        torch.testing.assert_close(out[0].cpu().float(), f["out"][t].float(), rtol=8e-3, atol=1e-6)
    assert torch.equal(ring_to_window(ring[0].cpu(), 9), f["state"])


@pytest.mark.gpu
def test_rope_kernel_matches_fixture(gpu):
    announce("golden: rope_table vs transformers rotary embedding")
    from router_ia import kernels as K
    from router_ia.batched_state import rope_inv_freq

    f = _fx("rope_tables")
    inv = rope_inv_freq(1e7, 64).to(gpu)
    for i, pos in enumerate(f["positions"].tolist()):
        cos, sin = K.rope_table(pos, inv)
        torch.testing.assert_close(cos.cpu(), f["cos"][i], rtol=0, atol=2e-6)
        torch.testing.assert_close(sin.cpu(), f["sin"][i], rtol=0, atol=2e-6)


@pytest.mark.gpu
def test_attention_kernel_matches_fixture(gpu):
    announce("golden: attn_decode vs float64 attention, T=33")
    from router_ia import kernels as K
    from router_ia.paged_kv import PagedKVCache

    f = _fx("decode_attention_T33")
    cache = PagedKVCache(1, 4, 1, 4, num_kv_heads=2, device=gpu, shuffle_seed=2)
    cache.ensure(0, 33)
    cache.write_tokens(0, 0, 0, f["k"].transpose(0, 1), f["v"].transpose(0, 1))
    ws = torch.empty(K.attn_decode_workspace_bytes(1, 16, 2, 33, 64), dtype=torch.uint8, device=gpu)
    out = torch.empty((1, 16, 256), device=gpu)
    K.attn_decode(f["q_rot"][None].to(gpu), f["gate"][None].to(gpu), cache.k[0], cache.v[0], cache.page_table, out,
                  positions=0, ctx_lens=33, max_ctx=33, inv_freq=None, scale=1 / 16, workspace=ws, split_tokens=64)
    # bf16 K/V and bf16 probabilities: the stated activation tolerance
    assert_act_close(out[0], f["out"], "attention output")
