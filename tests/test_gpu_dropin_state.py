"""GPU: the drop-in's AttentionState holds what the reference's holds, and every seam is honoured.

The reference keeps per-layer tensors in AttentionState's dicts
(v2/src/router_ia/qwen36_attention_cache.py:27-32) and its callers read them
as tensors: a cache probe compares ``full_keys[layer]`` with its own keys,
checks ``shape[-2]`` and ``requires_grad``; a fidelity probe reads
``linear_conv_states[layer].detach().float()`` and compares it with the
window its own conv keeps (:202-209).  The tests make those reads after a
token count that is not a multiple of 4, check that each step stores new
tensors (what a caller held is not changed by the next step), that a tensor a
caller stores into a dict is what the next step reads, and that a replaced
module attribute (rmsnorm, gated_rmsnorm, _l2norm, _apply_rope,
_append_full_kv) is called and gives the reference's result.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_residual_close, assert_state_close
from oracle import qwen36_cpu as O
from synthetic_checkpoint import make_checkpoint

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt_state")
    weights = make_checkpoint(root, {0: "linear", 1: "full"}, seed=11)
    return root, weights


def _begin(ac, root):
    st = ac.state_for(root, DEV)
    ac.reset(root)
    ac.activate(root, st)
    return st


def _token(ac, root, st, ref, weights, x, proj_out=None):
    """One token through both layers on the GPU and in the oracle; returns (got0, got1, want0, want1).

    With a list ``proj_out``, the DeltaNet layer's F.linear outputs (in_proj_qkv, a, b, z, out_proj) are
    appended to it as they leave the GPU projections.
    """
    if proj_out is None:
        got0 = ac.step_attention(root, 0, x.to(DEV), DEV).cpu()
    else:
        linear = ac.F.linear
        outs = []

        def capture(inp, weight, bias=None):
            y = linear(inp, weight, bias)
            outs.append(y.detach().clone())
            return y

        ac.F.linear = capture
        try:
            got0 = ac.step_attention(root, 0, x.to(DEV), DEV).cpu()
        finally:
            ac.F.linear = linear
        proj_out.append(outs)
    got1 = ac.step_attention(root, 1, x.to(DEV), DEV).cpu()
    want0 = O.linear_layer_step(weights[0], ref, 0, x, gpu_dtypes=True)
    want1 = O.full_layer_step(weights[1], ref, 1, x, gpu_dtypes=True)
    st.tokens_seen += 1
    ref.tokens_seen += 1
    return got0, got1, want0, want1


def test_state_dicts_read_as_the_reference_tensors(gpu, ckpt):
    announce("drop-in state: full_keys/values as [1,2,T,256] tensors, conv window oldest-first, 7 tokens")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    st = _begin(ac, root)
    ref = O.SequenceState()
    xs = torch.randn((7, 2048), generator=torch.Generator().manual_seed(21))
    w0 = weights[0]
    # the DeltaNet recurrence continued on the GPU's own projection outputs: the state path alone
    proj_conv, proj_state = None, None
    try:
        for t in range(7):
            held = None
            if t:
                held = {name: (d[layer], d[layer].detach().clone()) for name, d, layer in (
                    ("state", st.linear_states, 0), ("conv", st.linear_conv_states, 0), ("keys", st.full_keys, 1),
                    ("values", st.full_values, 1))}
            proj = []
            got0, got1, want0, want1 = _token(ac, root, st, ref, weights, xs[t:t + 1], proj_out=proj)
            qkv, a_raw, b_raw = proj[0][0].cpu(), proj[0][1].float().cpu(), proj[0][2].float().cpu()
            beta, g = O.gating(a_raw, b_raw, w0["linear_attn.A_log"].reshape(1, -1),
                               w0["linear_attn.dt_bias"].reshape(1, -1))
            _, proj_conv, proj_state = O.linear_decode_step(proj_conv, proj_state, qkv.reshape(1, 8192),
                                                            w0["linear_attn.conv1d.weight"], beta, g)
            # the stated bounds on the state path: conv window bit for bit, fp32 state within 1e-4
            assert torch.equal(st.linear_conv_states[0].cpu(), proj_conv), f"conv window, token {t}"
            assert_state_close(st.linear_states[0].cpu(), proj_state, f"state on the GPU projections, token {t}")
            # residual streams through fp16 projections that the CPU may round one unit apart
            assert_residual_close(got0, want0, 1, f"DeltaNet layer, token {t}")
            assert_residual_close(got1, want1, 1, f"full layer, token {t}")
            # the reads a cache probe makes
            got_k, got_v = st.full_keys[1], st.full_values[1]
            assert isinstance(got_k, torch.Tensor) and got_k.shape == (1, 2, t + 1, 256)
            assert int(got_k.shape[-2]) == t + 1 and not got_k.requires_grad and not got_v.requires_grad
            assert got_k.dtype == ref.keys[1].dtype == torch.float32
            # keys and values as stored: the fp32 tokens rounded once to fp16
            torch.testing.assert_close(got_k.cpu(), ref.keys[1].to(torch.float16).float(), rtol=2e-2, atol=2e-3)
            torch.testing.assert_close(got_v.detach().float().cpu(), ref.values[1].to(torch.float16).float(),
                                       rtol=2e-2, atol=2e-3)
            # the reads a DeltaNet fidelity probe makes
            conv = st.linear_conv_states[0].detach().float()
            assert conv.shape == (1, 8192, 4)
            torch.testing.assert_close(conv.cpu(), ref.conv[0].float(), rtol=1.6e-2, atol=1e-3)
            # end to end, through CPU projections that may round an fp16 output differently
            assert_state_close(st.linear_states[0].detach().float().cpu(), ref.linear[0], f"state, token {t}",
                               rel=1e-2)
            # each step stored new tensors: what was held across it is unchanged
            if held:
                for name, (tensor, copy) in held.items():
                    assert torch.equal(tensor.detach().cpu(), copy.cpu()), f"{name} changed after token {t}"
                assert held["keys"][0].shape[-2] == t
    finally:
        ac.deactivate(root)
    assert st.snapshot()["linear_conv_layers_cached"] == 1


def test_tensors_a_caller_stores_are_what_the_next_step_reads(gpu, ckpt):
    announce("drop-in state: caller-stored linear state, conv window and truncated KV are read by the next step")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    st = _begin(ac, root)
    ref = O.SequenceState()
    xs = torch.randn((5, 2048), generator=torch.Generator().manual_seed(22))
    try:
        for t in range(3):
            _token(ac, root, st, ref, weights, xs[t:t + 1])
        g = torch.Generator().manual_seed(23)
        new_state = torch.randn((1, 32, 128, 128), generator=g) * 0.02
        new_conv = torch.randn((1, 8192, 4), generator=g).to(torch.bfloat16)
        keep = 2  # the first two tokens of the KV (as a cache-trimming caller might keep)
        k_keep = ref.keys[1][:, :, :keep].to(torch.float16).float()
        v_keep = ref.values[1][:, :, :keep].to(torch.float16).float()
        st.linear_states[0] = new_state.to(DEV)
        st.linear_conv_states[0] = new_conv.to(DEV)
        st.full_keys[1] = k_keep.to(DEV)
        st.full_values[1] = v_keep.to(DEV)
        ref.linear[0], ref.conv[0] = new_state.clone(), new_conv.clone()
        ref.keys[1], ref.values[1] = k_keep.clone(), v_keep.clone()
        for t in range(3, 5):
            got0, got1, want0, want1 = _token(ac, root, st, ref, weights, xs[t:t + 1])
            assert_residual_close(got0, want0, 1, f"DeltaNet layer after the caller's state, token {t}")
            assert_residual_close(got1, want1, 1, f"full layer after the caller's cache, token {t}")
        assert st.full_keys[1].shape[-2] == keep + 2
        assert_state_close(st.linear_states[0].cpu(), ref.linear[0], "state after the caller's state", rel=1e-3)
    finally:
        ac.deactivate(root)


def _run(ac, root, xs):
    st = _begin(ac, root)
    outs = []
    try:
        for t in range(xs.shape[0]):
            x = xs[t:t + 1].to(DEV)
            outs.append((ac.step_attention(root, 0, x, DEV).cpu(), ac.step_attention(root, 1, x, DEV).cpu()))
            st.tokens_seen += 1
    finally:
        ac.deactivate(root)
    return outs, st


@pytest.mark.parametrize("seams", [("rmsnorm",), ("_apply_rope",), ("rmsnorm", "_apply_rope"), ("_l2norm",),
                                   ("gated_rmsnorm",), ("_append_full_kv",), ("_causal_conv1d_step", "_l2norm")])
def test_replaced_seams_are_called_and_give_the_reference_result(gpu, ckpt, monkeypatch, seams):
    announce(f"drop-in seams: replaced {seams}, 5 tokens")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    xs = torch.randn((5, 2048), generator=torch.Generator().manual_seed(24))
    fused, fused_st = _run(ac, root, xs)
    fused_keys = fused_st.full_keys[1].detach().cpu()
    calls: dict[str, int] = {}
    for name in seams:
        original = getattr(ac, name)

        def wrapped(*args, _name=name, _orig=original, **kwargs):
            calls[_name] = calls.get(_name, 0) + 1
            return _orig(*args, **kwargs)

        monkeypatch.setattr(ac, name, wrapped)
    unfused, st = _run(ac, root, xs)
    per_token = {"rmsnorm": 4, "_apply_rope": 1, "_l2norm": 2, "gated_rmsnorm": 1, "_append_full_kv": 1,
                 "_causal_conv1d_step": 1}  # rmsnorm: DeltaNet input, attention input, q_norm, k_norm
    assert calls == {name: 5 * per_token[name] for name in seams}
    ref = O.SequenceState()
    for t in range(5):
        want0 = O.linear_layer_step(weights[0], ref, 0, xs[t:t + 1], gpu_dtypes=True)
        want1 = O.full_layer_step(weights[1], ref, 1, xs[t:t + 1], gpu_dtypes=True)
        ref.tokens_seen += 1
        assert_residual_close(unfused[t][0], want0, 1, f"DeltaNet layer with {seams} replaced, token {t}")
        assert_residual_close(unfused[t][1], want1, 1, f"full layer with {seams} replaced, token {t}")
        # and close to the fused launches: the same arithmetic up to summation order, which can move an
        # fp16 projection output by one unit in the last place
        for j in (0, 1):
            ulp = 2.0 ** -10 * fused[t][j].abs().max().item()
            torch.testing.assert_close(unfused[t][j], fused[t][j], rtol=1e-3, atol=ulp)
    torch.testing.assert_close(st.full_keys[1].detach().cpu(), fused_keys, rtol=1e-3, atol=1e-3)
    assert_state_close(st.linear_states[0].cpu(), ref.linear[0], f"state with {seams} replaced", rel=1e-3)
