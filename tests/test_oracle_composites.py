"""Pin the oracle's layer composites (linear_layer_step, full_layer_step).

The composites restate qwen36_attention_cache.py:224-324: input RMSNorm,
projections, conv, gating, l2norm, recurrence, gated norm and out_proj for a
DeltaNet layer; projections, q/k norms, RoPE, KV append, gated attention and
o_proj for an attention layer.  They are pinned three ways:

* on the CPU path (fp32) against transformers 5.15.0's own Qwen3.5-MoE modules
  (``Qwen3_5MoeGatedDeltaNet``, ``Qwen3_5MoeAttention``, the decoder layer's
  ``Qwen3_5MoeRMSNorm``), driven as one-token cached decodes with a
  ``DynamicCache``, the way the reference's fidelity probe compares a layer
  with transformers (src/router_ia/qwen36_layer_fidelity_probe.py:58-64,
  134-164): every output, the recurrent and conv states, and the KV cache;
* the GPU path's casts (:229-233, :293-294): DeltaNet projections see h
  rounded to bf16 and then fp16, attention projections h rounded to fp16,
  all weights in fp16;
* a planted mistake (the DeltaNet bf16 cast dropped, in the oracle) is
  caught by that check.
"""

from __future__ import annotations

import pytest
import torch

from oracle import qwen36_cpu as O

hf = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
cache_utils = pytest.importorskip("transformers.cache_utils")
hf_config = pytest.importorskip("transformers.models.qwen3_5_moe.configuration_qwen3_5_moe")

HIDDEN = 2048


def _config():
    cfg = hf_config.Qwen3_5MoeTextConfig(
        num_hidden_layers=4, num_experts=4, num_experts_per_tok=2,
        rope_parameters={"rope_type": "default", "rope_theta": O.ROPE_THETA, "partial_rotary_factor": 0.25})
    cfg._attn_implementation = "eager"
    assert cfg.layer_types == ["linear_attention"] * 3 + ["full_attention"]
    return cfg


def _weights(kind: str, seed: int) -> dict[str, torch.Tensor]:
    """fp32 weights under the checkpoint's suffixes, at O(1) activation scale."""
    g = torch.Generator().manual_seed(seed)

    def w(*shape, scale):
        return torch.randn(shape, generator=g) * scale

    out = {"input_layernorm.weight": w(HIDDEN, scale=0.1)}
    if kind == "linear":
        out.update({
            "linear_attn.in_proj_qkv.weight": w(O.CONV_DIM, HIDDEN, scale=HIDDEN ** -0.5),
            "linear_attn.in_proj_z.weight": w(O.VALUE_DIM, HIDDEN, scale=HIDDEN ** -0.5),
            "linear_attn.in_proj_a.weight": w(O.NUM_V_HEADS, HIDDEN, scale=HIDDEN ** -0.5),
            "linear_attn.in_proj_b.weight": w(O.NUM_V_HEADS, HIDDEN, scale=HIDDEN ** -0.5),
            # fp32 conv weight: the conv then runs in fp32 in the oracle (it computes in the conv
            # weight's dtype, :200-221) and in the fp32 transformers module alike
            "linear_attn.conv1d.weight": w(O.CONV_DIM, 1, 4, scale=0.5),
            "linear_attn.A_log": torch.rand((O.NUM_V_HEADS,), generator=g) * 4.0 - 4.0,
            "linear_attn.dt_bias": w(O.NUM_V_HEADS, scale=0.5),
            "linear_attn.norm.weight": 1.0 + w(128, scale=0.1),
            "linear_attn.out_proj.weight": w(HIDDEN, O.VALUE_DIM, scale=O.VALUE_DIM ** -0.5),
        })
    else:
        out.update({
            "self_attn.q_proj.weight": w(2 * O.FULL_NUM_HEADS * O.FULL_HEAD_DIM, HIDDEN, scale=HIDDEN ** -0.5),
            "self_attn.k_proj.weight": w(O.FULL_NUM_KV_HEADS * O.FULL_HEAD_DIM, HIDDEN, scale=HIDDEN ** -0.5),
            "self_attn.v_proj.weight": w(O.FULL_NUM_KV_HEADS * O.FULL_HEAD_DIM, HIDDEN, scale=HIDDEN ** -0.5),
            "self_attn.q_norm.weight": w(O.FULL_HEAD_DIM, scale=0.1),
            "self_attn.k_norm.weight": w(O.FULL_HEAD_DIM, scale=0.1),
            "self_attn.o_proj.weight": w(HIDDEN, O.FULL_NUM_HEADS * O.FULL_HEAD_DIM, scale=2048 ** -0.5),
        })
    return out


def _load(module: torch.nn.Module, weights: dict[str, torch.Tensor], prefix: str) -> None:
    params = dict(module.named_parameters())
    with torch.no_grad():
        for name, p in params.items():
            p.copy_(weights[prefix + name])
    assert {prefix + n for n in params} <= set(weights)


def _input_norm(cfg, weights):
    norm = hf.Qwen3_5MoeRMSNorm(HIDDEN, eps=cfg.rms_norm_eps)
    with torch.no_grad():
        norm.weight.copy_(weights["input_layernorm.weight"])
    return norm


def test_linear_layer_step_matches_transformers_gated_deltanet():
    cfg = _config()
    weights = _weights("linear", 31)
    layer = hf.Qwen3_5MoeGatedDeltaNet(cfg, 0).eval()
    _load(layer, weights, "linear_attn.")
    norm = _input_norm(cfg, weights)
    cache = cache_utils.DynamicCache(config=cfg)
    st = O.SequenceState()
    xs = torch.randn((6, HIDDEN), generator=torch.Generator().manual_seed(32))
    with torch.no_grad():
        for t in range(6):
            x = xs[t:t + 1]
            want = x + layer(norm(x)[None], cache_params=cache)[0]  # residual + token mixer (decoder layer)
            got = O.linear_layer_step(weights, st, 0, x)
            torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5, msg=lambda m: f"token {t}: {m}")
            lc = cache.layers[0]
            torch.testing.assert_close(st.linear[0], lc.recurrent_states[0], rtol=1e-4, atol=1e-6)
            torch.testing.assert_close(st.conv[0], lc.conv_states[0], rtol=0, atol=0)  # the inputs, as stored


@pytest.mark.parametrize("resident", [0, 37])
def test_full_layer_step_matches_transformers_attention(resident):
    cfg = _config()
    weights = _weights("full", 33)
    attn = hf.Qwen3_5MoeAttention(cfg, 3).eval()
    _load(attn, weights, "self_attn.")
    norm = _input_norm(cfg, weights)
    rotary = hf.Qwen3_5MoeTextRotaryEmbedding(cfg)
    cache = cache_utils.DynamicCache(config=cfg)
    st = O.SequenceState()
    g = torch.Generator().manual_seed(34)
    if resident:
        # a cache already holding `resident` rotated keys and values
        k0 = torch.randn((1, O.FULL_NUM_KV_HEADS, resident, O.FULL_HEAD_DIM), generator=g)
        v0 = torch.randn((1, O.FULL_NUM_KV_HEADS, resident, O.FULL_HEAD_DIM), generator=g)
        cache.update(k0.clone(), v0.clone(), 3)
        st.keys[3], st.values[3] = k0.clone(), v0.clone()
        st.tokens_seen = resident
    xs = torch.randn((4, HIDDEN), generator=g)
    with torch.no_grad():
        for t in range(4):
            x = xs[t:t + 1]
            pos = resident + t
            h = norm(x)[None]
            cos, sin = rotary(h, torch.tensor([[pos]]))
            out, _ = attn(h, position_embeddings=(cos, sin), attention_mask=None, past_key_values=cache)
            want = x + out[0]
            got = O.full_layer_step(weights, st, 3, x)
            st.tokens_seen += 1
            torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5, msg=lambda m: f"token {t}: {m}")
            hk, hv = cache.layers[3].keys, cache.layers[3].values
            torch.testing.assert_close(st.keys[3], hk, rtol=1e-5, atol=1e-6)
            torch.testing.assert_close(st.values[3], hv, rtol=0, atol=0)


def _projection_inputs(monkeypatch, kind: str):
    """Run one GPU-dtype step of a composite and return the inputs and weights its F.linear calls saw."""
    seen = []
    linear = O.F.linear

    def capture(x, w, b=None):
        seen.append((x.detach().clone(), w.dtype))
        return linear(x, w, b)

    weights = _weights(kind, 35)
    if kind == "linear":
        weights["linear_attn.conv1d.weight"] = weights["linear_attn.conv1d.weight"].to(torch.bfloat16)
    x = torch.randn((1, HIDDEN), generator=torch.Generator().manual_seed(36)) * 3.0
    with monkeypatch.context() as m:
        m.setattr(O.F, "linear", capture)
        (O.linear_layer_step if kind == "linear" else O.full_layer_step)(weights, O.SequenceState(), 0, x,
                                                                         gpu_dtypes=True)
    return seen


def _bf16_exact(t: torch.Tensor) -> bool:
    return bool(torch.equal(t.float(), t.to(torch.bfloat16).float()))


def _check_gpu_cast_chain(monkeypatch) -> None:
    lin = _projection_inputs(monkeypatch, "linear")
    full = _projection_inputs(monkeypatch, "full")
    # DeltaNet: in_proj_qkv, in_proj_a, in_proj_b, in_proj_z see h.to(bf16) cast to the fp16 weights
    for x, wdt in lin[:4]:
        assert wdt == torch.float16 and x.dtype == torch.float16
        assert _bf16_exact(x), "DeltaNet projections must see h rounded to bf16 first (:229-233)"
    # attention: q/k/v see h.to(fp16) directly, which bf16 cannot hold in general
    for x, wdt in full[:3]:
        assert wdt == torch.float16 and x.dtype == torch.float16
    assert not _bf16_exact(full[0][0]), "attention projections see h rounded to fp16 only (:293-294)"


def test_gpu_cast_chain_of_the_composites(monkeypatch):
    _check_gpu_cast_chain(monkeypatch)


def test_a_dropped_bf16_cast_is_caught(monkeypatch):
    # the mistake planted in the oracle: DeltaNet projections fed fp16 h instead of bf16 h
    real = O.layer_compute_dtype
    monkeypatch.setattr(O, "layer_compute_dtype",
                        lambda kind, gpu: torch.float16 if gpu else real(kind, gpu))
    with pytest.raises(AssertionError, match="bf16"):
        _check_gpu_cast_chain(monkeypatch)
