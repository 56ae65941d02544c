"""GPU parity: the RMSNorms around the attention arithmetic, standalone and fused.

The reference normalises on either side of the hot path: the (1 + w) RMSNorm
of the layer input and of q / k before RoPE (qwen36_op_probe.py:55-67, used at
qwen36_attention_cache.py:227,302-305) and the gated RMSNorm of the DeltaNet
read-out (qwen36_gated_norm_probe.py:19-36, used at :268-271).  Checked
against the oracle's restatements (pinned by fp64 and by transformers'
Qwen3.5 norm modules in the oracle tests): the standalone kernels directly,
and every fused form both against the same computation run unfused (the norm
as its own launch) and against the oracle composite.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close
from oracle import chunked as OC
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import kernels as K
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState, rope_inv_freq
from router_ia.paged_kv import PagedKVCache

pytestmark = pytest.mark.gpu

HK, HV = W.NUM_K_HEADS, W.NUM_V_HEADS
# One unit in the last place of each output dtype, as a relative tolerance
# for two roundings of nearly equal fp32 values.
ULP_RTOL = {torch.bfloat16: 8e-3, torch.float16: 1e-3, torch.float32: 2e-6}


def _ulp_close(got, want, dtype, what):
    torch.testing.assert_close(got.detach().cpu().float(), want.detach().cpu().float(), rtol=ULP_RTOL[dtype],
                               atol=1e-6, msg=lambda m: f"{what}: {m}")


# ----------------------------------------------------------------------------- standalone kernels
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rmsnorm_matches_oracle(gpu, dtype):
    announce(f"rmsnorm: input norm [5, 2048] and q heads [7, 16, 256] in wider rows, {dtype}")
    w = W.norm_params(61)
    g = torch.Generator().manual_seed(62)
    x = (torch.randn((5, 2048), generator=g) * 3).to(dtype)
    got = K.rmsnorm(x.to(gpu), w["input_norm"].to(gpu))
    assert got.dtype == dtype
    _ulp_close(got, O.rmsnorm(x, w["input_norm"]), dtype, "input norm")
    # q heads inside rows of a wider projection output (token stride 4160)
    wide = (torch.randn((7, 16 * 256 + 64), generator=g) * 2).to(dtype)
    q = wide[:, :4096].unflatten(1, (16, 256))
    got = K.rmsnorm(q.to(gpu), w["q_norm"].to(gpu))
    _ulp_close(got, O.rmsnorm(q, w["q_norm"]), dtype, "q heads")
    # fp32 math, result cast to x's dtype, then stored as the out dtype
    out = torch.empty((7, 16, 256), dtype=torch.float32, device=gpu)
    K.rmsnorm(q.to(gpu), w["q_norm"].to(gpu), out=out)
    assert torch.equal(out.cpu(), got.cpu().float())
    # rows one element off 4-element alignment take the scalar form
    odd = wide.to(gpu)[:, 1:2049]
    _ulp_close(K.rmsnorm(odd, w["input_norm"].to(gpu)), O.rmsnorm(wide[:, 1:2049], w["input_norm"]), dtype,
               "unaligned rows")
    # 96-element rows: 16 lanes per row, some lanes take two 4-element chunks
    x96 = (torch.randn((9, 3, 96), generator=g) * 2).to(dtype)
    w96 = torch.randn(96, generator=g).to(torch.bfloat16).float() * 0.1
    _ulp_close(K.rmsnorm(x96.to(gpu), w96.to(gpu)), O.rmsnorm(x96, w96), dtype, "96-element rows")


@pytest.mark.parametrize("z_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gated_rmsnorm_matches_oracle(gpu, z_dtype):
    announce(f"gated_rmsnorm: [6, 32, 128] fp32 read-out, z {z_dtype}")
    w = W.norm_params(63)["gated_norm"]
    g = torch.Generator().manual_seed(64)
    x = torch.randn((6, HV, 128), generator=g) * 0.3
    z = torch.randn((6, HV, 128), generator=g).to(z_dtype)
    want = O.gated_rmsnorm(x, z, w)
    got = K.gated_rmsnorm(x.to(gpu), z.to(gpu), w.to(gpu))
    _ulp_close(got, want, torch.float32, "fp32 out")
    out = torch.empty((6, HV, 128), dtype=torch.bfloat16, device=gpu)
    K.gated_rmsnorm(x.to(gpu), z.to(gpu), w.to(gpu), out=out)
    assert torch.equal(out.cpu(), got.cpu().to(torch.bfloat16))


# ----------------------------------------------------------------------------- DeltaNet decode epilogue
def _gdn_steps(dev, params, inputs, zs, w, steps, batch, state0, ring0, *, fused, out_dtype):
    state, ring = state0.clone().to(dev), ring0.clone().to(dev)
    pos = torch.full((batch,), 9, dtype=torch.int32, device=dev)
    outs = []
    for t in range(steps):
        out = torch.empty((batch, HV, 128), dtype=out_dtype, device=dev)
        K.gdn_decode(inputs["mixed"][t].to(dev), state, inputs["a_raw"][t].to(dev), inputs["b_raw"][t].to(dev), out,
                     num_k_heads=HK, num_v_heads=HV, conv_weight=params["conv_weight"].to(dev), conv_ring=ring,
                     conv_pos=pos, gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(dev),
                     dt_bias=params["dt_bias"].to(dev), z=zs[t].to(dev) if fused else None,
                     norm_weight=w.to(dev) if fused else None)
        pos += 1
        outs.append(out)
    torch.cuda.synchronize()
    return torch.stack(outs).cpu(), state.cpu()


@pytest.mark.parametrize("batch", [1, 3, 40])
def test_gdn_decode_fused_gated_norm(gpu, batch):
    announce(f"gdn_decode + gated norm: B={batch}, 3 steps, random state")
    steps = 3
    params = W.gdn_layer_params(65)
    inputs = W.gdn_step_inputs(66, steps, batch)
    zs = W.gate_z_inputs(67, steps, batch)
    w = W.norm_params(68)["gated_norm"]
    g = torch.Generator().manual_seed(69)
    state0 = torch.randn((batch, HV, 128, 128), generator=g) * 0.02
    ring0 = torch.randn((batch, 4, W.CONV_DIM), generator=g).to(torch.bfloat16)
    plain, s_plain = _gdn_steps(gpu, params, inputs, zs, w, steps, batch, state0, ring0, fused=False,
                                out_dtype=torch.float32)
    fused, s_fused = _gdn_steps(gpu, params, inputs, zs, w, steps, batch, state0, ring0, fused=True,
                                out_dtype=torch.float32)
    fused16, _ = _gdn_steps(gpu, params, inputs, zs, w, steps, batch, state0, ring0, fused=True,
                            out_dtype=torch.bfloat16)
    # the norm leaves the state alone; the unfused launch splits heads into
    # column blocks (32 or 64 columns; the fused one needs whole heads), which
    # sums the read-out in another order, so the states agree to the state
    # tolerance rather than bit for bit
    assert_state_close(s_fused, s_plain, "state, fused vs unfused")
    for t in range(steps):
        sep = K.gated_rmsnorm(plain[t].to(gpu), zs[t].to(gpu), w.to(gpu)).cpu()
        _ulp_close(fused[t], sep, torch.float32, f"step {t}: fused vs separate norm launch")
    assert torch.equal(fused16, fused.to(torch.bfloat16))
    # the oracle composite: recurrence, then the gated norm of the fp32 read-out
    window = ring0[:, [(9 - 4 + m) % 4 for m in range(4)]].transpose(1, 2)
    for b in range(batch):
        conv, st = window[b:b + 1], state0[b:b + 1]
        for t in range(steps):
            beta, gl = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
            attn, conv, st = O.linear_decode_step(conv, st, inputs["mixed"][t][b:b + 1], params["conv_weight"],
                                                  beta[b:b + 1], gl[b:b + 1])
            want = O.gated_rmsnorm(attn, zs[t][b:b + 1], w)
            assert_act_close(fused[t, b:b + 1], want, f"row {b} step {t}")


# ----------------------------------------------------------------------------- q / k norms before RoPE
def test_kv_append_fused_k_norm(gpu):
    announce("kv_append + k_norm: B=3 fp16 rows at positions 5, 17, 4096")
    batch, positions = 3, [5, 17, 4096]
    wk = W.norm_params(70)["k_norm"]
    g = torch.Generator().manual_seed(71)
    k = (torch.randn((batch, 2, 256), generator=g) * 3).to(torch.float16)
    v = torch.randn((batch, 2, 256), generator=g).to(torch.float16)
    inv = rope_inv_freq(10_000_000.0, 64).to(gpu)
    pos = torch.tensor(positions, dtype=torch.int32, device=gpu)
    slots = torch.tensor([0, 1, 2], dtype=torch.int32, device=gpu)

    def run(fused):
        kv = PagedKVCache(1, 8, batch, 2, num_kv_heads=2, device=gpu, shuffle_seed=7, dtype=torch.float16)
        for r in range(batch):
            kv.ensure(r, 16)
        kin = k.to(gpu) if fused else K.rmsnorm(k.to(gpu), wk.to(gpu))
        K.kv_append(kin, v.to(gpu), kv.k[0], kv.v[0], kv.page_table, positions=pos, slots=slots, inv_freq=inv,
                    k_norm_weight=wk.to(gpu) if fused else None)
        kg, vg = K.kv_gather(kv.k[0], kv.v[0], kv.page_table, batch=batch, start=0, count=3)
        return kg.cpu(), vg.cpu()

    kf, vf = run(True)
    ku, vu = run(False)
    assert torch.equal(vf, vu)
    _ulp_close(kf, ku, torch.float16, "fused vs separate k_norm")
    for b in range(batch):
        kn = O.rmsnorm(k[b:b + 1], wk).float().unsqueeze(2)
        _, kr = O.apply_rope(kn, kn, positions[b])
        assert_act_close(kf[b, :, b], kr[0, :, 0].to(torch.float16), f"row {b}")


@pytest.mark.parametrize("split_tokens", [0, 64])
def test_attn_decode_fused_q_and_k_norms(gpu, split_tokens):
    announce(f"full_step + q/k norms: ragged B=3, split_tokens={split_tokens}")
    lengths, steps = [5, 300, 1000], 3
    batch = len(lengths)
    wn = W.norm_params(72)
    kpre, vpre = W.prefilled_kv(73, batch, max(lengths))
    x = W.attn_step_inputs(74, steps, batch)
    st = BatchedAttentionState(batch, max(lengths) + steps + 32, num_linear_layers=0, num_full_layers=1,
                               device=gpu, page_shuffle_seed=4, split_tokens=split_tokens)
    st.set_positions(lengths)
    for b, n in enumerate(lengths):
        st.kv.write_tokens(0, b, 0, kpre[b, :, :n].permute(1, 0, 2), vpre[b, :, :n].permute(1, 0, 2))
    states = []
    for b, n in enumerate(lengths):
        s = O.SequenceState()
        s.keys[0], s.values[0], s.tokens_seen = kpre[b:b + 1, :, :n].float(), vpre[b:b + 1, :, :n].float(), n
        states.append(s)
    wq, wk = wn["q_norm"].to(gpu), wn["k_norm"].to(gpu)
    for t in range(steps):
        out = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu), x["gate"][t].to(gpu),
                           out_dtype=torch.float32, q_norm_weight=wq, k_norm_weight=wk)
        st.advance()
        for b, s in enumerate(states):
            qn = O.rmsnorm(x["q"][t][b:b + 1], wn["q_norm"]).float()
            kn = O.rmsnorm(x["k"][t][b:b + 1], wn["k_norm"]).float()
            want, s.keys[0], s.values[0] = O.full_decode_step(s.keys[0], s.values[0], qn, kn, x["v"][t][b:b + 1],
                                                              x["gate"][t][b:b + 1], s.tokens_seen)
            s.tokens_seen += 1
            assert_act_close(out[b:b + 1].cpu(), want, f"step {t} row {b}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attn_prefill_fused_q_and_k_norms(gpu, dtype):
    announce(f"attn_prefill + q/k norms: 100 + 77 tokens (continued prompt), {dtype}")
    n0, n1 = 100, 77
    wn = W.norm_params(75)
    g = torch.Generator().manual_seed(76)
    q = (torch.randn((n0 + n1, 16, 256), generator=g) * 2).to(dtype)
    k = (torch.randn((n0 + n1, 2, 256), generator=g) * 2).to(dtype)
    v = torch.randn((n0 + n1, 2, 256), generator=g).to(dtype)
    gate = torch.randn((n0 + n1, 16, 256), generator=g).to(dtype)
    pages = (n0 + n1 + 15) // 16 + 2
    kv = PagedKVCache(1, pages, 1, pages, num_kv_heads=2, device=gpu, shuffle_seed=8, dtype=dtype)
    kv.ensure(0, n0 + n1)
    inv = rope_inv_freq(10_000_000.0, 64).to(gpu)
    wq, wk = wn["q_norm"].to(gpu), wn["k_norm"].to(gpu)
    outs = []
    for s0, s1 in ((0, n0), (n0, n0 + n1)):
        outs.append(K.attn_prefill(q[s0:s1].to(gpu), k[s0:s1].to(gpu), v[s0:s1].to(gpu), gate[s0:s1].to(gpu),
                                   kv.k[0], kv.v[0], kv.page_table[0], start=s0, inv_freq=inv, scale=256 ** -0.5,
                                   q_norm_weight=wq, k_norm_weight=wk).cpu())
    got = torch.cat(outs)
    want, kr = OC.causal_attention_prefill(O.rmsnorm(q, wn["q_norm"]), O.rmsnorm(k, wn["k_norm"]), v, gate,
                                           torch.arange(n0 + n1))
    assert_act_close(got, want, "prefill outputs")
    kg, _ = K.kv_gather(kv.k[0], kv.v[0], kv.page_table, batch=1, start=0, count=n0 + n1)
    _ulp_close(kg[0].cpu(), kr.transpose(0, 1).to(dtype), dtype, "rotated normalised keys in the pages")


# ----------------------------------------------------------------------------- DeltaNet prefill
@pytest.mark.parametrize("seg_tokens", [None, 64])
def test_gdn_prefill_fused_gated_norm(gpu, seg_tokens):
    announce(f"gdn_prefill + gated norm: 130 tokens, segment {seg_tokens or 'whole'}")
    length = 130
    params = W.gdn_layer_params(77)
    inputs = W.gdn_step_inputs(78, length, 1)
    z = W.gate_z_inputs(79, length, 1)[:, 0]
    w = W.norm_params(80)["gated_norm"]
    g = torch.Generator().manual_seed(81)
    state0 = torch.randn((HV, 128, 128), generator=g) * 0.02
    ring0 = torch.randn((4, W.CONV_DIM), generator=g).to(torch.bfloat16)

    def run(fused, out_dtype):
        state, ring = state0.clone().to(gpu), ring0.clone().to(gpu)
        ws = torch.empty(K.gdn_prefill_workspace_bytes(HK, HV, seg_tokens or length), dtype=torch.uint8,
                         device=gpu)
        out = torch.empty((length, HV, 128), dtype=out_dtype, device=gpu)
        K.gdn_prefill(inputs["mixed"][:, 0].to(gpu), state, inputs["a_raw"][:, 0].to(gpu),
                      inputs["b_raw"][:, 0].to(gpu), out, num_k_heads=HK, num_v_heads=HV,
                      conv_weight=params["conv_weight"].to(gpu), conv_ring=ring, conv_pos=3, workspace=ws,
                      gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(gpu), dt_bias=params["dt_bias"].to(gpu),
                      z=z.to(gpu) if fused else None, norm_weight=w.to(gpu) if fused else None)
        torch.cuda.synchronize()
        return out.cpu(), state.cpu(), ring.cpu()

    plain, s_plain, r_plain = run(False, torch.float32)
    fused, s_fused, r_fused = run(True, torch.float32)
    fused16, _, _ = run(True, torch.bfloat16)
    assert torch.equal(s_fused, s_plain) and torch.equal(r_fused, r_plain)
    # the fused form is the scan's fp32 read-out followed by the same norm kernel
    sep = K.gated_rmsnorm(plain.to(gpu), z.to(gpu), w.to(gpu)).cpu()
    assert torch.equal(fused, sep)
    assert torch.equal(fused16, fused.to(torch.bfloat16))
    window = ring0[[(3 - 4 + m) % 4 for m in range(4)]].transpose(0, 1).unsqueeze(0)
    conv, st = window, state0[None]
    for t in range(length):
        beta, gl = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
        attn, conv, st = O.linear_decode_step(conv, st, inputs["mixed"][t], params["conv_weight"], beta, gl)
        assert_act_close(fused[t:t + 1], O.gated_rmsnorm(attn, z[t:t + 1], w), f"token {t}")
