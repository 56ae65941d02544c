"""GPU parity of the whole 40-layer decode stack through BatchedAttentionState.

Layers 4i..4i+2 are DeltaNet, 4i+3 full attention; every sequence starts from
resident state (DeltaNet state ~N(0, 0.02), conv ring ~N(0, 1), KV ~N(0, 1))
at its own ragged context length, over a shuffled page table.  All 40 layer
outputs of every step are compared with the oracle.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close, ring_to_window
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lengths,steps", [([9, 130, 517], 3), ([4095, 2], 2)])
def test_forty_layer_stack_matches_oracle(gpu, lengths, steps):
    announce(f"stack: 40 layers, contexts {lengths}, {steps} steps")
    batch = len(lengths)
    g = torch.Generator().manual_seed(sum(lengths))
    st = BatchedAttentionState(batch, max(lengths) + steps + 40, device=gpu, page_shuffle_seed=9)
    st.set_positions(lengths)
    oracle = [O.SequenceState() for _ in lengths]
    for b, n in enumerate(lengths):
        oracle[b].tokens_seen = n
    for li in range(30):
        s0 = torch.randn((batch, 32, 128, 128), generator=g) * 0.02
        ring = torch.randn((batch, 4, W.CONV_DIM), generator=g).to(torch.bfloat16)
        st.linear_states[li].copy_(s0)
        st.conv_rings[li].copy_(ring)
        for b, n in enumerate(lengths):
            oracle[b].linear[li] = s0[b:b + 1].clone()
            oracle[b].conv[li] = ring_to_window(ring[b], n)
    for fi in range(10):
        for b, n in enumerate(lengths):
            k = torch.randn((n, 2, 256), generator=g).to(torch.bfloat16)
            v = torch.randn((n, 2, 256), generator=g).to(torch.bfloat16)
            st.kv.write_tokens(fi, b, 0, k, v)
            oracle[b].keys[fi] = k.float().permute(1, 0, 2).unsqueeze(0)
            oracle[b].values[fi] = v.float().permute(1, 0, 2).unsqueeze(0)
    params = [W.gdn_layer_params(200 + li) for li in range(30)]
    params_dev = [{k: v.to(gpu) for k, v in p.items()} for p in params]
    for s in range(steps):
        gin = W.gdn_step_inputs(300 + s, 30, batch)  # one "step" per layer
        ain = W.attn_step_inputs(400 + s, 10, batch)
        for layer in range(40):
            if layer % 4 == 3:
                fi = layer // 4
                out = st.full_step(fi, ain["q"][fi].to(gpu), ain["k"][fi].to(gpu), ain["v"][fi].to(gpu),
                                   ain["gate"][fi].to(gpu), out_dtype=torch.float32)
                want = O.full_step_batched(oracle, fi, ain["q"][fi], ain["k"][fi], ain["v"][fi], ain["gate"][fi])
            else:
                li = layer - layer // 4
                p = params_dev[li]
                out = st.linear_step(li, gin["mixed"][li].to(gpu), p["conv_weight"], gin["a_raw"][li].to(gpu),
                                     gin["b_raw"][li].to(gpu), gate_mode=nat.RIA_GATE_RAW, A_log=p["A_log"],
                                     dt_bias=p["dt_bias"], out_dtype=torch.float32)
                beta, gg = O.gating(gin["a_raw"][li], gin["b_raw"][li], params[li]["A_log"], params[li]["dt_bias"])
                want = O.linear_step_batched(oracle, li, gin["mixed"][li], params[li]["conv_weight"], beta, gg)
            assert_act_close(out, want, f"step {s} layer {layer}")
        st.advance()
        for o in oracle:
            o.tokens_seen += 1
    for li in (0, 17, 29):
        for b in range(batch):
            assert_state_close(st.linear_states[li][b:b + 1].cpu(), oracle[b].linear[li], f"state layer {li} row {b}")
