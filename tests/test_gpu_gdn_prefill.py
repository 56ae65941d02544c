"""GPU parity: chunked Gated DeltaNet prefill (ria_gdn_prefill) against the
reference's token-by-token recurrence, restated in the oracle.

Covers a ragged last chunk with a non-zero starting state and conv history,
precomputed gates, segmenting (a workspace of one chunk gives the same bits as one pass),
bf16 / fp16 outputs (the fp32 read-out rounded once, no row written past the
prompt),
prefill followed by decode, and the single-layer 16384-token prefill
(zero state, seed 3) checked on every output and the final state.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close, ring_to_window, state_rel_err
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import kernels as K
from router_ia import workloads as W

pytestmark = pytest.mark.gpu


def _oracle_tokens(params, inputs, length, state=None, conv=None):
    outs = []
    for t in range(length):
        beta, g = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
        attn, conv, state = O.linear_decode_step(conv, state, inputs["mixed"][t], params["conv_weight"], beta, g)
        outs.append(attn[0])
    return torch.stack(outs), state, conv


def _gpu_prefill(dev, params, inputs, length, state0, ring0, pos0, ws_tokens=None, out_dtype=torch.float32,
                 precomputed=False):
    state = state0.clone().to(dev)
    ring = ring0.clone().to(dev)
    seg = ws_tokens or length
    ws = torch.empty(K.gdn_prefill_workspace_bytes(16, 32, seg), dtype=torch.uint8, device=dev)
    out = torch.empty((length, 32, 128), dtype=out_dtype, device=dev)
    if precomputed:
        # g and beta from the oracle's gating (the reference's sigmoid / softplus prologue)
        gates = [O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
                 for t in range(length)]
        ga = torch.cat([g for _, g in gates]).float().contiguous()
        gb = torch.cat([b for b, _ in gates]).float().contiguous()
        gate_kw = dict(gate_mode=nat.RIA_GATE_PRECOMPUTED)
    else:
        ga, gb = inputs["a_raw"][:length, 0], inputs["b_raw"][:length, 0]
        gate_kw = dict(gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(dev), dt_bias=params["dt_bias"].to(dev))
    K.gdn_prefill(inputs["mixed"][:length, 0].to(dev), state, ga.to(dev), gb.to(dev), out, num_k_heads=16,
                  num_v_heads=32, conv_weight=params["conv_weight"].to(dev), conv_ring=ring, conv_pos=pos0,
                  workspace=ws, **gate_kw)
    torch.cuda.synchronize()
    return out.cpu(), state.cpu(), ring.cpu()


def _init(seed):
    g = torch.Generator().manual_seed(seed)
    state0 = torch.randn((32, 128, 128), generator=g) * 0.02
    ring0 = torch.randn((4, W.CONV_DIM), generator=g).to(torch.bfloat16)
    return state0, ring0


def test_prefill_ragged_chunks_with_history(gpu):
    announce("gdn_prefill: 130 tokens (3 chunks), random state and conv history")
    params = W.gdn_layer_params(31)
    inputs = W.gdn_step_inputs(32, 130, 1)
    state0, ring0 = _init(33)
    pos0 = 7
    got, state, ring = _gpu_prefill(gpu, params, inputs, 130, state0, ring0, pos0)
    want, s_want, c_want = _oracle_tokens(params, inputs, 130, state0[None], ring_to_window(ring0, pos0))
    assert_act_close(got, want, "prefill outputs")
    assert_state_close(state[None], s_want, "final state")
    assert torch.equal(ring_to_window(ring, pos0 + 130), c_want)


def test_prefill_precomputed_gates(gpu):
    """g and beta passed in (RIA_GATE_PRECOMPUTED) instead of derived from the
    raw projections, over segments of two chunks: the gate pass reads them as
    given and the cumulative decay restarts in every chunk."""
    announce("gdn_prefill: precomputed g / beta, 200 tokens, 128-token segments, random state and history")
    params = W.gdn_layer_params(37)
    inputs = W.gdn_step_inputs(38, 200, 1)
    state0, ring0 = _init(39)
    pos0 = 2
    got, state, ring = _gpu_prefill(gpu, params, inputs, 200, state0, ring0, pos0, ws_tokens=128, precomputed=True)
    want, s_want, c_want = _oracle_tokens(params, inputs, 200, state0[None], ring_to_window(ring0, pos0))
    assert_act_close(got, want, "prefill outputs")
    assert_state_close(state[None], s_want, "final state")
    assert torch.equal(ring_to_window(ring, pos0 + 200), c_want)
    raw, s_raw, _ = _gpu_prefill(gpu, params, inputs, 200, state0, ring0, pos0, ws_tokens=128)
    assert_act_close(got, raw, "precomputed against raw gates")
    assert_state_close(state[None], s_raw[None], "precomputed against raw gates, state")


def test_prefill_segmenting_is_bit_identical(gpu):
    announce("gdn_prefill: one-chunk workspace vs whole-sequence workspace, 200 tokens")
    params = W.gdn_layer_params(34)
    inputs = W.gdn_step_inputs(35, 200, 1)
    state0, ring0 = _init(36)
    a, sa, ra = _gpu_prefill(gpu, params, inputs, 200, state0, ring0, 0)
    b, sb, rb = _gpu_prefill(gpu, params, inputs, 200, state0, ring0, 0, ws_tokens=64)
    assert torch.equal(a, b) and torch.equal(sa, sb) and torch.equal(ra, rb)


@pytest.mark.parametrize("length,ws_tokens", [(130, None), (777, 192)])
def test_prefill_16bit_outputs_round_the_fp32_read_out(gpu, length, ws_tokens):
    """bf16 and fp16 outputs are the fp32 read-out rounded once, bit for bit,
    and nothing is written past the prompt's last row: the scan stores each
    chunk's rows through a buffer range that ends at the last token, so the
    last chunk's rows past it are dropped by the hardware (checked on a
    ragged last chunk, in one pass and in segments of three chunks)."""
    announce(f"gdn_prefill: {length} tokens, bf16 / fp16 outputs against the fp32 read-out, guard rows untouched")
    params = W.gdn_layer_params(61)
    inputs = W.gdn_step_inputs(62, length, 1)
    state0, ring0 = _init(63)
    ref, s_ref, _ = _gpu_prefill(gpu, params, inputs, length, state0, ring0, 5, ws_tokens=ws_tokens)
    for dt in (torch.bfloat16, torch.float16):
        guard = 64  # rows after the prompt in the same allocation
        big = torch.full((length + guard, 32, 128), 7.0, dtype=dt, device=gpu)
        state = state0.clone().to(gpu)
        ring = ring0.clone().to(gpu)
        ws = torch.empty(K.gdn_prefill_workspace_bytes(16, 32, ws_tokens or length), dtype=torch.uint8, device=gpu)
        K.gdn_prefill(inputs["mixed"][:length, 0].to(gpu), state, inputs["a_raw"][:length, 0].to(gpu),
                      inputs["b_raw"][:length, 0].to(gpu), big[:length], num_k_heads=16, num_v_heads=32,
                      conv_weight=params["conv_weight"].to(gpu), conv_ring=ring, conv_pos=5, workspace=ws,
                      gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(gpu), dt_bias=params["dt_bias"].to(gpu))
        torch.cuda.synchronize()
        got = big.cpu()
        assert torch.equal(got[:length], ref.to(dt)), f"{dt} outputs"
        assert torch.equal(got[length:], torch.full((guard, 32, 128), 7.0, dtype=dt)), f"{dt} rows past the prompt"
        assert torch.equal(state.cpu(), s_ref), f"state with {dt} outputs"


@pytest.mark.parametrize("length", [1, 3, 64])
def test_prefill_short_prompts_then_decode(gpu, length):
    announce(f"gdn_prefill: {length} tokens then 3 decode steps")
    params = W.gdn_layer_params(37)
    inputs = W.gdn_step_inputs(38, length + 3, 1)
    state0 = torch.zeros((32, 128, 128))
    ring0 = torch.zeros((4, W.CONV_DIM), dtype=torch.bfloat16)
    got, state, ring = _gpu_prefill(gpu, params, inputs, length, state0, ring0, 0)
    want, s_want, c_want = _oracle_tokens(params, inputs, length + 3)
    assert_act_close(got, want[:length], "prefill outputs")
    dev = gpu
    st, rg = state[None].to(dev), ring[None].to(dev)
    for t in range(length, length + 3):
        out = torch.empty((1, 32, 128), device=dev)
        K.gdn_decode(inputs["mixed"][t].to(dev), st, inputs["a_raw"][t].to(dev), inputs["b_raw"][t].to(dev), out,
                     num_k_heads=16, num_v_heads=32, conv_weight=params["conv_weight"].to(dev), conv_ring=rg,
                     conv_pos=t, gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(dev),
                     dt_bias=params["dt_bias"].to(dev))
        assert_act_close(out[0].cpu(), want[t], f"decode after prefill, token {t}")
    assert_state_close(st.cpu(), s_want, "state after prefill + decode")


def test_prefill_16384_tokens_single_layer(gpu):
    announce("gdn_prefill: 1 layer, batch 1, 16384 tokens, zero state, seed 3")
    length = 16384
    params = W.gdn_layer_params(3)
    inputs = W.gdn_step_inputs(3, length, 1)
    zero_s = torch.zeros((32, 128, 128))
    zero_r = torch.zeros((4, W.CONV_DIM), dtype=torch.bfloat16)
    got, state, _ = _gpu_prefill(gpu, params, inputs, length, zero_s, zero_r, 0)
    want, s_want, _ = _oracle_tokens(params, inputs, length)
    print(f"16384-token prefill: max |out err| {(got - want).abs().max().item():.3e}, "
          f"state rel err {state_rel_err(state[None], s_want):.3e}", flush=True)
    assert_act_close(got, want, "all 16384 outputs")
    # the fp32 state after 16384 tokens, within the stated 1e-4 relative bound
    assert_state_close(state[None], s_want, "final state after 16384 tokens")


def test_prefill_conv_load_paths_agree(gpu):
    """bf16 rows at an even stride load a thread's two channels as one 32-bit
    word, all of a tile's tokens at once; an odd row stride takes the
    per-channel batched loads.  Same arithmetic: the same bits."""
    announce("gdn_prefill: paired 32-bit conv loads vs per-channel loads (odd row stride), 200 tokens")
    params = W.gdn_layer_params(51)
    inputs = W.gdn_step_inputs(52, 200, 1)
    state0, ring0 = _init(53)
    length = 200
    mixed = inputs["mixed"][:length, 0]
    wide = torch.zeros((length, W.CONV_DIM + 1), dtype=mixed.dtype)
    wide[:, :W.CONV_DIM] = mixed
    res = []
    for x in (mixed.to(gpu), wide.to(gpu)[:, :W.CONV_DIM]):  # row stride 8192, then 8193
        state = state0.clone().to(gpu)
        ring = ring0.clone().to(gpu)
        ws = torch.empty(K.gdn_prefill_workspace_bytes(16, 32, length), dtype=torch.uint8, device=gpu)
        out = torch.empty((length, 32, 128), dtype=torch.float32, device=gpu)
        K.gdn_prefill(x, state, inputs["a_raw"][:length, 0].to(gpu), inputs["b_raw"][:length, 0].to(gpu), out,
                      num_k_heads=16, num_v_heads=32, conv_weight=params["conv_weight"].to(gpu), conv_ring=ring,
                      conv_pos=5, workspace=ws, gate_mode=nat.RIA_GATE_RAW, A_log=params["A_log"].to(gpu),
                      dt_bias=params["dt_bias"].to(gpu))
        torch.cuda.synchronize()
        res.append((out.cpu(), state.cpu(), ring.cpu()))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    assert torch.equal(res[0][2], res[1][2])
    want, s_want, _ = _oracle_tokens(params, inputs, length, state0[None], ring_to_window(ring0, 5))
    assert_act_close(res[0][0], want, "outputs vs oracle")
    assert_state_close(res[0][1][None], s_want, "final state vs oracle")
