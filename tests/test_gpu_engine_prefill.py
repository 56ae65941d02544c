"""GPU parity: prompt prefill through the batched engine, then decode.

Two rows of a BatchedAttentionState (one DeltaNet and one attention layer)
take prompts of different lengths with the prefill kernels, then decode three
tokens together; every output is compared with the oracle running the same
sequences token by token, as the reference does
(qwen36_chat_batch.py:255-258 -> qwen36_attention_cache.py:176-317).
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState

pytestmark = pytest.mark.gpu


def test_engine_prefill_then_decode(gpu):
    announce("engine: rows prefilled with 100 and 37 tokens, then 3 decode steps")
    prompts = [100, 37]
    steps = 3
    total = max(prompts) + steps
    params = W.gdn_layer_params(61)
    lin = W.gdn_step_inputs(62, total, 2)    # [T, 2, ...]
    att = W.attn_step_inputs(63, total, 2)
    st = BatchedAttentionState(2, 256, num_linear_layers=1, num_full_layers=1, device=gpu, page_shuffle_seed=5,
                               prefill_segment_tokens=64)
    st.set_positions([0, 0])
    dev = gpu
    cw, alog, dtb = params["conv_weight"].to(dev), params["A_log"].to(dev), params["dt_bias"].to(dev)
    got_lin = [[] for _ in prompts]
    got_att = [[] for _ in prompts]
    for row, n in enumerate(prompts):
        st.begin_prefill(row, n)
        o_lin = st.linear_prefill(0, row, lin["mixed"][:n, row].to(dev), cw, lin["a_raw"][:n, row].to(dev),
                                  lin["b_raw"][:n, row].to(dev), gate_mode=nat.RIA_GATE_RAW, A_log=alog,
                                  dt_bias=dtb, out_dtype=torch.float32)
        o_att = st.full_prefill(0, row, att["q"][:n, row].to(dev), att["k"][:n, row].to(dev),
                                att["v"][:n, row].to(dev), att["gate"][:n, row].to(dev))
        st.end_prefill(row, n)
        got_lin[row] += list(o_lin.cpu())
        got_att[row] += list(o_att.float().cpu())
    # decode: row r feeds its own next inputs (token prompts[r] + i)
    st.reserve(steps)
    for i in range(steps):
        idx = [n + i for n in prompts]
        mixed = torch.stack([lin["mixed"][t, r] for r, t in enumerate(idx)]).to(dev)
        a = torch.stack([lin["a_raw"][t, r] for r, t in enumerate(idx)]).to(dev)
        b = torch.stack([lin["b_raw"][t, r] for r, t in enumerate(idx)]).to(dev)
        o_lin = st.linear_step(0, mixed, cw, a, b, gate_mode=nat.RIA_GATE_RAW, A_log=alog, dt_bias=dtb,
                               out_dtype=torch.float32)
        qkvg = {name: torch.stack([att[name][t, r] for r, t in enumerate(idx)]).to(dev)
                for name in ("q", "k", "v", "gate")}
        o_att = st.full_step(0, qkvg["q"], qkvg["k"], qkvg["v"], qkvg["gate"], out_dtype=torch.float32)
        st.advance()
        for r in range(2):
            got_lin[r].append(o_lin[r].cpu())
            got_att[r].append(o_att[r].cpu())
    for r, n in enumerate(prompts):
        s = O.SequenceState()
        for t in range(n + steps):
            beta, g = O.gating(lin["a_raw"][t, r:r + 1], lin["b_raw"][t, r:r + 1], params["A_log"], params["dt_bias"])
            want, s.conv[0], s.linear[0] = O.linear_decode_step(s.conv.get(0), s.linear.get(0),
                                                                 lin["mixed"][t, r:r + 1], params["conv_weight"],
                                                                 beta, g)
            assert_act_close(got_lin[r][t], want[0], f"row {r} DeltaNet token {t}")
            want, s.keys[0], s.values[0] = O.full_decode_step(s.keys.get(0), s.values.get(0), att["q"][t, r:r + 1],
                                                              att["k"][t, r:r + 1], att["v"][t, r:r + 1],
                                                              att["gate"][t, r:r + 1], t)
            assert_act_close(got_att[r][t], want[0], f"row {r} attention token {t}")
        assert_state_close(st.linear_states[0, r].cpu()[None], s.linear[0], f"row {r} final state")
