"""Cross-check the oracle against transformers 5.15.0, the library the reference defers to.

The reference's HF-compatible path calls transformers' Qwen3.5-MoE helpers
(v2/src/router_ia/qwen36_linear_attention_hf.py:81-100); its fidelity probes
compare against the same module (src/router_ia/qwen36_layer_fidelity_probe.py).
Skipped where transformers is not importable.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import chunked as C
from oracle import qwen36_cpu as O

hf = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")


def _seq(seed, length, heads=4, dk=128):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((length, heads, dk), generator=g)
    k = torch.randn((length, heads, dk), generator=g)
    v = torch.randn((length, heads, dk), generator=g)
    gl = -F.softplus(torch.randn((length, heads), generator=g)) * torch.exp(torch.rand((length, heads), generator=g) * 4 - 4)
    beta = torch.sigmoid(torch.randn((length, heads), generator=g))
    return q, k, v, gl, beta


def test_recurrent_rule_matches_transformers():
    q, k, v, g, beta = _seq(1, 20)
    s0 = torch.randn((1, 4, 128, 128), generator=torch.Generator().manual_seed(2)) * 0.02
    o_hf, s_hf = hf.torch_recurrent_gated_delta_rule(q[None], k[None], v[None], g[None], beta[None],
                                                    initial_state=s0, output_final_state=True,
                                                    use_qk_l2norm_in_kernel=True)
    o, s = C.recurrent_gated_delta_rule(q, k, v, g, beta, s0[0])
    torch.testing.assert_close(o, o_hf[0], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s, s_hf[0], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("length", [64, 130])
def test_chunk_rule_matches_transformers(length):
    q, k, v, g, beta = _seq(3, length)
    o_hf, s_hf = hf.torch_chunk_gated_delta_rule(q[None], k[None], v[None], g[None], beta[None],
                                                initial_state=None, output_final_state=True,
                                                use_qk_l2norm_in_kernel=True)
    o, s = C.chunk_gated_delta_rule(q, k, v, g, beta)
    torch.testing.assert_close(o, o_hf[0], rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(s, s_hf[0], rtol=2e-4, atol=2e-5)


def test_conv_step_matches_transformers_update():
    g = torch.Generator().manual_seed(4)
    w = (torch.randn((8192, 4), generator=g) * 0.5).to(torch.bfloat16)
    state = torch.randn((1, 8192, 4), generator=g).to(torch.bfloat16)
    x = torch.randn((1, 8192), generator=g).to(torch.bfloat16)
    hf_state = state.clone()
    out_hf = hf.causal_conv1d_update(x.reshape(1, 8192, 1), hf_state, w, activation="silu")
    out, new_state = O.causal_conv1d_step(state, x, w.reshape(8192, 1, 4))
    assert torch.equal(out, out_hf[:, :, 0])
    assert torch.equal(new_state, hf_state)


def test_rope_matches_transformers():
    g = torch.Generator().manual_seed(5)
    q = torch.randn((1, 16, 1, 256), generator=g)
    k = torch.randn((1, 2, 1, 256), generator=g)
    for pos in (0, 17, 4096, 32767):
        cos, sin = O.rope(pos)
        q_hf, k_hf = hf.apply_rotary_pos_emb(q, k, cos.view(1, 1, 64), sin.view(1, 1, 64))
        qr, kr = O.apply_rope(q, k, pos)
        assert torch.equal(qr, q_hf) and torch.equal(kr, k_hf)


def test_l2norm_and_repeat_kv_match_transformers():
    x = torch.randn((3, 7, 128), generator=torch.Generator().manual_seed(6))
    assert torch.equal(O.l2norm(x), hf.l2norm(x, dim=-1, eps=1e-6))
    kv = torch.randn((1, 2, 5, 256), generator=torch.Generator().manual_seed(7))
    assert torch.equal(kv.repeat_interleave(8, dim=1), hf.repeat_kv(kv, 8))


def test_rmsnorms_match_transformers():
    g = torch.Generator().manual_seed(8)
    norm = hf.Qwen3_5MoeRMSNorm(256, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(256, generator=g) * 0.1)
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        x = (torch.randn((1, 16, 256), generator=g) * 4).to(dt)
        with torch.no_grad():
            assert torch.equal(O.rmsnorm(x, norm.weight), norm(x))
    gated = hf.Qwen3_5MoeRMSNormGated(128, eps=1e-6)
    with torch.no_grad():
        gated.weight.copy_(torch.randn(128, generator=g))
    x = torch.randn((1, 32, 128), generator=g) * 0.2
    z = torch.randn((1, 32, 128), generator=g)
    with torch.no_grad():
        assert torch.equal(O.gated_rmsnorm(x, z, gated.weight), gated(x, gate=z))


def test_fp8_dequant_matches_transformers():
    from transformers.integrations.finegrained_fp8 import Fp8Dequantize

    g = torch.Generator().manual_seed(9)
    w8 = (torch.randn((256, 384), generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    s = torch.rand((2, 3), generator=g) + 0.01
    hf_w = Fp8Dequantize(None)._dequantize_one(w8, s, output_dtype=torch.float32)
    assert torch.equal(O.dequantize_fp8_blockwise(w8, s), hf_w)
    hf16 = Fp8Dequantize(None)._dequantize_one(w8, s, output_dtype=torch.float16)
    assert torch.equal(O.dequantize_fp8_blockwise(w8, s).to(torch.float16), hf16)
