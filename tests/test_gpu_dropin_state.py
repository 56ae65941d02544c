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
_append_full_kv) is called and gives the reference's result.  The cached keys
and values read back the fp32 tokens the reference appends (its KV probe's
max-abs 1e-3), and a replaced torch.einsum / torch.softmax sees the score, softmax
and P V intermediates the reference's residual probe captures.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_residual_close, assert_state_close
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
            # keys and values read back as the fp32 tokens (through CPU projections that may round an fp16
            # projection output one unit apart; the exact check on the GPU's own projections is below)
            torch.testing.assert_close(got_k.cpu(), ref.keys[1], rtol=2e-2, atol=2e-3)
            torch.testing.assert_close(got_v.detach().float().cpu(), ref.values[1], rtol=2e-2, atol=2e-3)
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


def _assert_within_fp16_unit(got, want, what):
    """|got - want| <= one fp16 unit of the normed value (2^-10 relative) + 1e-5 for the fp32 rotation."""
    bound = 2.0 ** -10 * want.abs() + 1e-5
    excess = ((got - want).abs() - bound).max().item()
    assert excess <= 0, f"{what}: beyond one fp16 unit by {excess:.3e}"


def _capture_linear(ac, outs):
    linear = ac.F.linear

    def capture(inp, weight, bias=None):
        y = linear(inp, weight, bias)
        outs.append(y.detach().clone())
        return y

    return linear, capture


def test_cached_kv_reads_back_the_fp32_tokens_the_reference_stores(gpu, ckpt):
    # the reference appends k after k_norm and RoPE in fp32 and v.float() (qwen36_attention_cache.py:304-307,
    # 365-372); its KV probe compares them at max-abs 1e-3 (src/router_ia/qwen36_kv_cache_probe.py:16, 147-157)
    announce("drop-in KV: full_keys / full_values read back the appended fp32 tokens, 9 tokens")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    w1 = weights[1]
    st = _begin(ac, root)
    xs = torch.randn((9, 2048), generator=torch.Generator().manual_seed(25))
    keys, values = [], []
    try:
        for t in range(9):
            outs = []
            linear, capture = _capture_linear(ac, outs)
            ac.F.linear = capture
            try:
                ac.step_attention(root, 1, xs[t:t + 1].to(DEV), DEV)
            finally:
                ac.F.linear = linear
            # the oracle's token from this step's GPU projections (q_gate, k, v, o_proj in call order)
            k = O.rmsnorm(outs[1].cpu().reshape(1, 2, 256), w1["self_attn.k_norm.weight"]).float()
            _, k_rot = O.apply_rope(k.unsqueeze(2), k.unsqueeze(2), t)
            keys.append(k_rot)
            values.append(outs[2].cpu().reshape(1, 2, 1, 256).float())
            st.tokens_seen += 1
            got_k, got_v = st.full_keys[1], st.full_values[1]
            want_k, want_v = torch.cat(keys, dim=2), torch.cat(values, dim=2)
            assert got_k.dtype == got_v.dtype == torch.float32 and got_k.shape == want_k.shape
            assert torch.equal(got_v.cpu(), want_v), f"values, token {t}"
            # k: the kernel's k_norm (rounded to the projection's fp16, where two summation orders can
            # land one unit apart) and fp32 RoPE against the oracle's
            _assert_within_fp16_unit(got_k.cpu(), want_k, f"keys, token {t}")
            assert (got_k.cpu() - want_k).abs().max().item() <= 1e-3  # the KV probe's bound
    finally:
        ac.deactivate(root)


def test_replaced_einsum_and_softmax_see_the_attention_intermediates(gpu, ckpt, monkeypatch):
    # the reference's residual probe replaces cache.torch.einsum / cache.torch.softmax (and F.linear,
    # rmsnorm, _apply_rope) and reports "attention intermediates MISSING" unless the score einsum, the
    # softmax and the P V einsum are seen (src/router_ia/qwen36_full_attention_residual_probe.py:104-153,
    # 207-230)
    announce("drop-in seams: replaced torch.einsum / torch.softmax capture the attention intermediates, 4 tokens")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    w1 = weights[1]
    xs = torch.randn((4, 2048), generator=torch.Generator().manual_seed(26))
    fused, _ = _run(ac, root, xs)
    einsums, softmaxes = [], []
    orig_einsum, orig_softmax = ac.torch.einsum, ac.torch.softmax

    def einsum(equation, *operands, **kwargs):
        out = orig_einsum(equation, *operands, **kwargs)
        einsums.append((equation, [op.detach().clone() for op in operands], out.detach().clone()))
        return out

    def softmax(inp, dim=None, *args, **kwargs):
        out = orig_softmax(inp, dim=dim, *args, **kwargs)
        softmaxes.append((inp.detach().clone(), out.detach().clone()))
        return out

    monkeypatch.setattr(ac.torch, "einsum", einsum)
    monkeypatch.setattr(ac.torch, "softmax", softmax)
    st = _begin(ac, root)
    keys, values = [], []
    try:
        for t in range(4):
            einsums.clear()
            softmaxes.clear()
            outs = []
            linear, capture = _capture_linear(ac, outs)
            ac.F.linear = capture
            try:
                got = ac.step_attention(root, 1, xs[t:t + 1].to(DEV), DEV).cpu()
            finally:
                ac.F.linear = linear
            st.tokens_seen += 1
            # the oracle's operands from this step's GPU projections
            q_gate = outs[0].cpu().reshape(1, 16, 512)
            q, gate = torch.chunk(q_gate, 2, dim=-1)
            q = O.rmsnorm(q, w1["self_attn.q_norm.weight"]).float()
            k = O.rmsnorm(outs[1].cpu().reshape(1, 2, 256), w1["self_attn.k_norm.weight"]).float()
            q_rot, k_rot = O.apply_rope(q.unsqueeze(2), k.unsqueeze(2), t)
            keys.append(k_rot)
            values.append(outs[2].cpu().reshape(1, 2, 1, 256).float())
            k_exp = torch.cat(keys, dim=2).repeat_interleave(8, dim=1)
            v_exp = torch.cat(values, dim=2).repeat_interleave(8, dim=1)
            eqs = [e[0] for e in einsums]
            assert eqs == ["bhd,bhld->bhl", "bhl,bhld->bhd"] and len(softmaxes) == 1, (eqs, len(softmaxes))
            (_, (sq, sk), raw), (_, (pw, pv), attn) = einsums
            sm_in, sm_out = softmaxes[0]
            _assert_within_fp16_unit(sq.cpu(), q_rot.squeeze(2), f"score q operand, token {t}")
            _assert_within_fp16_unit(sk.cpu(), k_exp, f"score k operand, token {t}")
            assert torch.equal(pv.cpu(), v_exp)
            torch.testing.assert_close(sm_in.cpu(), raw.cpu() * 256 ** -0.5, rtol=1e-6, atol=1e-6)
            assert torch.equal(pw, sm_out)
            want_attn = O.attention_over_cache(q_rot.squeeze(2), torch.cat(keys, 2), torch.cat(values, 2),
                                               torch.zeros_like(gate)) * 2.0  # sigmoid(0) = 1/2
            assert_act_close(attn.cpu(), want_attn, f"P V einsum, token {t}")
            # the layer's result equals the fused launches' up to one fp16 unit of the output projection
            ulp = 2.0 ** -10 * fused[t][1].abs().max().item()
            torch.testing.assert_close(got, fused[t][1], rtol=1e-3, atol=ulp)
    finally:
        ac.deactivate(root)
