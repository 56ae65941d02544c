"""GPU parity: fused Gated DeltaNet decode (ria_gdn_decode) against the oracle.

Covers the single-layer batch-1 workload (64 tokens, seed 0), the 4096-token
fp32 state drift bound, batch sizes that select each column blocking, input
dtypes, both gate modes and the unfused (post-conv input) form.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close, ring_to_window, state_rel_err
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import kernels as K
from router_ia import workloads as W

pytestmark = pytest.mark.gpu

HK, HV = W.NUM_K_HEADS, W.NUM_V_HEADS


def _run_gpu(dev, params, inputs, steps, batch, *, x_dtype=torch.bfloat16, gate_mode=nat.RIA_GATE_RAW,
             state0=None, ring0=None, pos0=0, out_dtype=torch.float32):
    state = torch.zeros((batch, HV, 128, 128), device=dev) if state0 is None else state0.clone().to(dev)
    ring = torch.zeros((batch, 4, W.CONV_DIM), dtype=torch.bfloat16, device=dev) if ring0 is None \
        else ring0.clone().to(dev)
    cw = params["conv_weight"].to(dev)
    a_log = params["A_log"].to(dev)
    dt_bias = params["dt_bias"].to(dev)
    outs = []
    pos = torch.full((batch,), pos0, dtype=torch.int32, device=dev)
    for t in range(steps):
        x = inputs["mixed"][t].to(device=dev, dtype=x_dtype)
        if gate_mode == nat.RIA_GATE_RAW:
            ga, gb = inputs["a_raw"][t].to(dev), inputs["b_raw"][t].to(dev)
        else:
            beta, g = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
            ga, gb = g.to(dev), beta.to(dev)
        out = torch.empty((batch, HV, 128), dtype=out_dtype, device=dev)
        K.gdn_decode(x, state, ga, gb, out, num_k_heads=HK, num_v_heads=HV, conv_weight=cw, conv_ring=ring,
                     conv_pos=pos, gate_mode=gate_mode, A_log=a_log, dt_bias=dt_bias)
        pos += 1
        outs.append(out)
    torch.cuda.synchronize()
    return torch.stack(outs).cpu(), state.cpu(), ring.cpu()


def _run_oracle(params, inputs, steps, batch, *, x_dtype=torch.bfloat16, states=None, convs=None):
    states = [None] * batch if states is None else list(states)
    convs = [None] * batch if convs is None else list(convs)
    outs = []
    for t in range(steps):
        beta, g = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
        row_out = []
        for b in range(batch):
            x = inputs["mixed"][t][b:b + 1].to(x_dtype)
            attn, convs[b], states[b] = O.linear_decode_step(convs[b], states[b], x, params["conv_weight"],
                                                             beta[b:b + 1], g[b:b + 1])
            row_out.append(attn)
        outs.append(torch.cat(row_out))
    return torch.stack(outs), states, convs


def test_gdn_decode_single_layer_batch1_64_tokens(gpu):
    announce("gdn_decode: 1 layer, B=1, 64 tokens, seed 0")
    params = W.gdn_layer_params(0)
    inputs = W.gdn_step_inputs(0, 64, 1)
    got, state, ring = _run_gpu(gpu, params, inputs, 64, 1)
    want, states, convs = _run_oracle(params, inputs, 64, 1)
    assert_act_close(got, want, "outputs")
    assert_state_close(state[0:1], states[0], "final state")
    # conv state holds raw bf16 inputs: exact
    assert torch.equal(ring_to_window(ring[0], 64), convs[0])


@pytest.mark.parametrize("batch", [3, 8, 33])
def test_gdn_decode_batched_column_blocking(gpu, batch):
    announce(f"gdn_decode: B={batch}, 12 tokens, seed 5")
    params = W.gdn_layer_params(5)
    inputs = W.gdn_step_inputs(6, 12, batch)
    gen = torch.Generator().manual_seed(7)
    state0 = torch.randn((batch, HV, 128, 128), generator=gen) * 0.02
    ring0 = torch.randn((batch, 4, W.CONV_DIM), generator=gen).to(torch.bfloat16)
    pos0 = 9  # ring slots of tokens 6, 7, 8 hold the history
    got, state, ring = _run_gpu(gpu, params, inputs, 12, batch, state0=state0, ring0=ring0, pos0=pos0)
    convs0 = [ring_to_window(ring0[b], pos0) for b in range(batch)]
    want, states, convs = _run_oracle(params, inputs, 12, batch, states=[state0[b:b + 1] for b in range(batch)],
                                      convs=convs0)
    assert_act_close(got, want, "outputs")
    for b in range(batch):
        assert_state_close(state[b:b + 1], states[b], f"state row {b}")
        assert torch.equal(ring_to_window(ring[b], pos0 + 12), convs[b])


@pytest.mark.parametrize("x_dtype", [torch.float16, torch.float32])
def test_gdn_decode_input_dtypes(gpu, x_dtype):
    announce(f"gdn_decode: input dtype {x_dtype}")
    params = W.gdn_layer_params(11)
    inputs = W.gdn_step_inputs(12, 8, 2)
    inputs["mixed"] = inputs["mixed"].float() * 3.0  # values that are not bf16-exact
    got, state, _ = _run_gpu(gpu, params, inputs, 8, 2, x_dtype=x_dtype)
    want, states, _ = _run_oracle(params, inputs, 8, 2, x_dtype=x_dtype)
    assert_act_close(got, want, "outputs")
    for b in range(2):
        assert_state_close(state[b:b + 1], states[b], f"state row {b}")


def test_gdn_decode_precomputed_gate_and_bf16_out(gpu):
    announce("gdn_decode: precomputed beta/g, bf16 output")
    params = W.gdn_layer_params(13)
    inputs = W.gdn_step_inputs(14, 6, 4)
    got, _, _ = _run_gpu(gpu, params, inputs, 6, 4, gate_mode=nat.RIA_GATE_PRECOMPUTED, out_dtype=torch.bfloat16)
    want, _, _ = _run_oracle(params, inputs, 6, 4)
    assert got.dtype == torch.bfloat16
    assert_act_close(got, want, "outputs")


def test_gdn_decode_unfused_post_conv_input(gpu):
    announce("gdn_decode: fuse_conv=0")
    params = W.gdn_layer_params(15)
    inputs = W.gdn_step_inputs(16, 5, 2)
    dev = gpu
    state = torch.zeros((2, HV, 128, 128), device=dev)
    states = [None, None]
    convs = [None, None]
    for t in range(5):
        beta, g = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
        mixed_post = []
        want = []
        for b in range(2):
            m, convs[b] = O.causal_conv1d_step(convs[b], inputs["mixed"][t][b:b + 1].float(), params["conv_weight"])
            q, k, v = O.split_qkv(m)
            attn, states[b] = O.gated_delta_step(states[b], q, k, v, beta[b:b + 1], g[b:b + 1])
            mixed_post.append(m)
            want.append(attn)
        out = torch.empty((2, HV, 128), device=dev)
        K.gdn_decode(torch.cat(mixed_post).to(dev), state, g.to(dev), beta.to(dev), out, num_k_heads=HK,
                     num_v_heads=HV, fuse_conv=False)
        assert_act_close(out, torch.cat(want), f"outputs step {t}")
    for b in range(2):
        assert_state_close(state[b:b + 1], states[b], f"state row {b}")


def test_gdn_decode_state_drift_4096_tokens(gpu):
    announce("gdn_decode: 4096-token fp32 state drift, B=1, seed 0")
    params = W.gdn_layer_params(0)
    inputs = W.gdn_step_inputs(100, 4096, 1)
    got, state, _ = _run_gpu(gpu, params, inputs, 4096, 1)
    want, states, _ = _run_oracle(params, inputs, 4096, 1)
    err = state_rel_err(state[0:1], states[0])
    print(f"4096-token state relative error: {err:.3e}")
    assert_state_close(state[0:1], states[0], "state after 4096 tokens")
    assert_act_close(got[-64:], want[-64:], "last 64 outputs")


def test_conv1d_step_standalone(gpu):
    announce("conv1d_step: standalone, B=3")
    params = W.gdn_layer_params(17)
    inputs = W.gdn_step_inputs(18, 6, 3)
    dev = gpu
    ring = torch.zeros((3, 4, W.CONV_DIM), dtype=torch.bfloat16, device=dev)
    cw = params["conv_weight"].to(dev)
    convs = [None] * 3
    for t in range(6):
        x = inputs["mixed"][t].float()
        out = torch.empty((3, W.CONV_DIM), device=dev)
        K.conv1d_step(x.to(dev), cw, ring, out, conv_pos=t)
        for b in range(3):
            want, convs[b] = O.causal_conv1d_step(convs[b], x[b:b + 1], params["conv_weight"])
            # Same bf16 conv result; allow one bf16 ulp for a different fp32 accumulation order.
            torch.testing.assert_close(out[b:b + 1].cpu(), want, rtol=8e-3, atol=1e-6)
    for b in range(3):
        assert torch.equal(ring_to_window(ring[b].cpu(), 6), convs[b])


def _bf16_rne(bits32: np.ndarray) -> np.ndarray:
    return ((bits32 + 0x7FFF + ((bits32 >> 16) & 1)) >> 16).astype(np.uint32)


def test_conv1d_step_silu_every_bf16_input(gpu):
    """The SiLU after the conv over all 65536 bf16 values.

    Conv weights (0, 0, 0, 1) and a zero history make the conv output the
    input itself (-0 becomes +0 in the sum), so row r, channel c takes the
    bf16 value with bits r * 8192 + c.  The bar is the fp32 SiLU torch computes
    (x / (1 + exp(-x)), exp overflowing past x = -88.7) rounded to bf16: the
    float64 SiLU, rounded to fp32 and then to bf16, wherever that fp32 value
    is not itself a bf16 rounding midpoint (258 inputs, where either
    neighbour is accepted), and torch's CPU bf16 F.silu (the oracle's conv
    activation) on the same inputs.  The hardware exp2 and reciprocal alone,
    without the accurate form near midpoints, fail it at x = 5.9375.
    """
    announce("conv1d_step: SiLU over all 65536 bf16 inputs")
    dev = gpu
    rows, ch = 8, W.CONV_DIM
    bits = torch.arange(rows * ch, dtype=torch.int32)
    x = bits.to(torch.int16).view(torch.bfloat16).reshape(rows, ch)
    cw = torch.zeros((ch, 1, 4), dtype=torch.bfloat16)
    cw[:, 0, 3] = 1.0
    ring = torch.zeros((rows, 4, ch), dtype=torch.bfloat16, device=dev)
    out = torch.empty((rows, ch), dtype=torch.bfloat16, device=dev)
    K.conv1d_step(x.to(dev), cw.to(dev), ring, out, conv_pos=0)
    got = out.cpu().reshape(-1).view(torch.int16).numpy().astype(np.uint32) & 0xFFFF

    with np.errstate(over="ignore", invalid="ignore"):
        v = x.reshape(-1).float().numpy().astype(np.float64) + 0.0
        e = np.exp(-v)
        e[-v > np.log(np.finfo(np.float32).max)] = np.inf
        y32 = (v / (1.0 + e)).astype(np.float32)
    b32 = y32.view(np.uint32).astype(np.int64)
    nan = np.isnan(y32)
    near = ((b32 & 0xFFFF) == 0x8000) & ~nan
    want = _bf16_rne(b32.astype(np.uint32)) & 0xFFFF
    got_nan = (got & 0x7F80) == 0x7F80
    got_nan &= (got & 0x7F) != 0
    assert np.array_equal(got_nan, nan), "NaN results differ"
    ok = ~nan & ~near
    bad = np.nonzero(got[ok] != want[ok])[0]
    assert bad.size == 0, f"{bad.size} inputs differ from the rounded fp32 SiLU, first bits " \
                          f"{hex(int(bits.numpy()[ok][bad[0]]))}"
    # on a midpoint: one bf16 step at most from the float64 rounding
    diff = np.abs(got[near].astype(np.int64) - want[near].astype(np.int64))
    assert diff.max(initial=0) <= 1
    torch_bits = torch.nn.functional.silu(x.reshape(-1) + 0.0).view(torch.int16).numpy().astype(np.uint32) & 0xFFFF
    off = np.nonzero((torch_bits != got) & ~nan & ~near)[0]
    assert off.size == 0, f"{off.size} inputs differ from torch's bf16 SiLU away from midpoints"
    print(f"{int(near.sum())} inputs on a midpoint; {int((torch_bits[near] != got[near]).sum())} of them "
          f"differ from torch's CPU bf16 SiLU")
