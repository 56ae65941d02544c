"""GPU parity of the drop-in module ``router_ia.qwen36_attention_cache``.

``step_attention`` runs a DeltaNet layer and a full-attention layer of a
synthetic checkpoint token by token, the way the reference's token loop
drives it (v2/src/router_ia/qwen36_chat_batch.py:181-207: every layer, then
tokens_seen += 1), and is compared with the oracle's restatement of the
reference composites on the CPU with the reference's CUDA-path dtypes.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close
from oracle import qwen36_cpu as O
from synthetic_checkpoint import make_checkpoint

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt")
    weights = make_checkpoint(root, {0: "linear", 1: "full"}, seed=3)
    return root, weights


def _run_dropin(ac, root, xs, device="cuda:0"):
    st = ac.state_for(root, device)
    ac.reset(root)
    ac.activate(root, st)
    outs = []
    for t in range(xs.shape[0]):
        x = xs[t:t + 1].to(device)
        outs.append((ac.step_attention(root, 0, x, device).cpu(), ac.step_attention(root, 1, x, device).cpu()))
        st.tokens_seen += 1
    ac.deactivate(root)
    return outs, st


def test_step_attention_matches_reference_composites(gpu, ckpt):
    announce("drop-in: step_attention, DeltaNet + full layer, 6 tokens")
    from router_ia import qwen36_attention_cache as ac

    root, weights = ckpt
    xs = torch.randn((6, 2048), generator=torch.Generator().manual_seed(4))
    outs, st = _run_dropin(ac, root, xs)
    ref = O.SequenceState()
    for t in range(6):
        want0 = O.linear_layer_step(weights[0], ref, 0, xs[t:t + 1], gpu_dtypes=True)
        want1 = O.full_layer_step(weights[1], ref, 1, xs[t:t + 1], gpu_dtypes=True)
        ref.tokens_seen += 1
        assert_act_close(outs[t][0], want0, f"DeltaNet layer, token {t}")
        assert_act_close(outs[t][1], want1, f"full layer, token {t}")
    assert_state_close(st.linear_states[0].cpu(), ref.linear[0], "DeltaNet state", rel=1e-3)
    # conv state: the bf16 projection outputs of the last four tokens (GPU and CPU fp16 GEMVs may
    # round a few elements differently, hence a bf16-ulp tolerance rather than equality)
    # the dict holds the reference's window [1, 8192, 4], oldest input first (6 tokens: not a multiple of 4)
    conv = st.linear_conv_states[0]
    assert conv.shape == (1, 8192, 4) and conv.dtype == torch.bfloat16
    torch.testing.assert_close(conv.cpu().float(), ref.conv[0].float(), rtol=1.6e-2, atol=1e-3)
    snap = st.snapshot()
    assert snap["full_tokens_resident"] == 6 and snap["tokens_seen"] == 6
    assert snap["full_bytes"] == 6 * 2 * 2 * 256 * 4  # the reference's fp32 K and V, 2 heads x 256
    assert snap["linear_bytes"] == 32 * 128 * 128 * 4 and snap["linear_conv_bytes"] == 8192 * 4 * 2
    k_mat = st.full_keys[1].detach().cpu().float()
    torch.testing.assert_close(k_mat, ref.keys[1].to(torch.float16).float(), rtol=2e-2, atol=2e-3)


def test_replaced_conv_step_is_called_and_gives_the_same_result(gpu, ckpt, monkeypatch):
    announce("drop-in: monkeypatched _causal_conv1d_step seam")
    from router_ia import qwen36_attention_cache as ac

    root, _ = ckpt
    xs = torch.randn((3, 2048), generator=torch.Generator().manual_seed(5))
    fused, _ = _run_dropin(ac, root, xs)
    calls = []
    original = ac._causal_conv1d_step

    def wrapped(state, layer, mixed, w):
        calls.append(layer)
        return original(state, layer, mixed, w)

    monkeypatch.setattr(ac, "_causal_conv1d_step", wrapped)
    unfused, _ = _run_dropin(ac, root, xs)
    assert calls == [0, 0, 0]
    for (a0, _), (b0, _) in zip(fused, unfused):
        # fused conv returns bf16 values cast through the fp16 input dtype, like the standalone step
        torch.testing.assert_close(b0, a0, rtol=1e-5, atol=1e-5)


def test_module_helpers_match_oracle(gpu):
    announce("drop-in: _rope, _apply_rope, _l2norm, _causal_conv1d_step")
    from router_ia import qwen36_attention_cache as ac

    for pos in (0, 17, 4096, 32767):
        cos, sin = ac._rope(pos, torch.device("cuda:0"), torch.float32)
        c, s = O.rope(pos)
        torch.testing.assert_close(cos.cpu(), c, rtol=0, atol=2e-6)
        torch.testing.assert_close(sin.cpu(), s, rtol=0, atol=2e-6)
    g = torch.Generator().manual_seed(6)
    q, k = torch.randn((1, 16, 1, 256), generator=g), torch.randn((1, 2, 1, 256), generator=g)
    qr, kr = ac._apply_rope(q.cuda(), k.cuda(), 4351)
    wq, wk = O.apply_rope(q, k, 4351)
    torch.testing.assert_close(qr.cpu(), wq, rtol=1e-5, atol=2e-6)
    torch.testing.assert_close(kr.cpu(), wk, rtol=1e-5, atol=2e-6)
    x = torch.randn((1, 32, 128), generator=g)
    torch.testing.assert_close(ac._l2norm(x.cuda()).cpu(), O.l2norm(x), rtol=1e-6, atol=1e-7)
    st = ac.AttentionState()
    w = (torch.randn((8192, 1, 4), generator=g) * 0.5).to(torch.bfloat16)
    state = None
    for t in range(5):
        m = torch.randn((1, 8192), generator=g)
        out = ac._causal_conv1d_step(st, 0, m.cuda(), w.cuda())
        want, state = O.causal_conv1d_step(state, m, w)
        torch.testing.assert_close(out.cpu(), want, rtol=8e-3, atol=1e-6)
    assert torch.equal(st.linear_conv_states[0].cpu(), state)  # the reference's window, bit for bit


def test_append_full_kv_limits_on_gpu_count_the_reference_bytes(gpu):
    announce("drop-in: _append_full_kv limits with GPU tensors")
    from router_ia import qwen36_attention_cache as ac

    g = torch.Generator().manual_seed(7)
    tok = lambda: (torch.randn((1, 2, 1, 256), generator=g).cuda(), torch.randn((1, 2, 1, 256), generator=g).cuda())
    st = ac.AttentionState(max_context_tokens=3)
    keys = []
    for p in range(3):
        st.tokens_seen = p
        k, v = tok()
        keys.append(k)
        fk, fv = ac._append_full_kv(st, 5, k, v)
        assert fk.shape[-2] == p + 1
    with pytest.raises(RuntimeError, match="max_context_tokens=3"):
        ac._append_full_kv(st, 5, *tok())
    assert st.full_keys[5].shape[-2] == 3
    mat = st.full_keys[5].detach().cpu()
    assert mat.dtype == torch.float32  # the dtype of the tokens, read back as appended (the pages are fp16)
    assert torch.equal(mat, torch.cat(keys, dim=2).cpu())
    assert st.paged_kv_bytes() == 3 * 2 * 2 * 256 * 2
    token_bytes = 2 * 2 * 256 * 4  # fp32 k and v tokens, counted as the reference counts them
    st2 = ac.AttentionState(max_full_kv_bytes=2 * token_bytes)
    ac._append_full_kv(st2, 0, *tok())
    ac._append_full_kv(st2, 0, *tok())
    with pytest.raises(RuntimeError, match="max_full_kv_bytes"):
        ac._append_full_kv(st2, 0, *tok())
    assert st2.snapshot()["full_bytes"] == 2 * token_bytes
