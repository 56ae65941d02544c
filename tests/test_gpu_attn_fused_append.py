"""GPU parity: the KV append fused into the decode attention launches (ria_attn_decode_append).

The fused path (the split-K launch over the resident tokens, the combine
launch computing, storing and folding in the new token) must leave the paged
cache bit-identical to ria_kv_append followed by ria_attn_decode (same
k_norm, RoPE and rounding), attend over the appended token and match the
oracle.  Cases: the balanced partition (padded and not),
fixed splits whose last split holds one token, q/k norms, fp16 activations
with fp16 pages, and ragged rows whose new token opens a page.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close
from oracle import qwen36_cpu as O
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState


def _state(dev, batch, max_context, *, fused, split_tokens=0, kv_dtype=torch.bfloat16):
    return BatchedAttentionState(batch, max_context, num_linear_layers=0, num_full_layers=1, device=dev,
                                 page_shuffle_seed=5, split_tokens=split_tokens, kv_dtype=kv_dtype,
                                 fused_append=fused)


def _load(st, lengths, kpre, vpre):
    st.set_positions(lengths)
    for b, n in enumerate(lengths):
        st.kv.write_tokens(0, b, 0, kpre[b, :, :n].permute(1, 0, 2), vpre[b, :, :n].permute(1, 0, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("lengths,split_tokens,norms,act", [
    ([4095], 0, False, torch.bfloat16),                 # B=1: padded balanced partition
    ([1, 15, 16, 17, 300, 1000], 0, True, torch.bfloat16),  # tiny and page-aligned rows, q/k norms
    ([1, 15, 16, 17, 300, 1000], 64, False, torch.bfloat16),  # fixed splits: a last split of one token
    ([31, 32, 33, 5000], 0, True, torch.float16),       # fp16 activations, fp16 pages
])
def test_fused_append_matches_separate_append(gpu, lengths, split_tokens, norms, act):
    announce(f"attn_decode_append: lengths {lengths}, split_tokens {split_tokens}, norms {norms}, {act}")
    batch, steps = len(lengths), 3
    kvd = torch.float16 if act == torch.float16 else torch.bfloat16
    kpre, vpre = W.prefilled_kv(41, batch, max(lengths))
    kpre, vpre = kpre.to(kvd), vpre.to(kvd)
    x = W.attn_step_inputs(42, steps, batch)
    x = {k: t.to(act) for k, t in x.items()}
    g = torch.Generator().manual_seed(43)
    qnw = (0.1 * torch.randn(256, generator=g)).to(gpu) if norms else None
    knw = (0.1 * torch.randn(256, generator=g)).to(gpu) if norms else None
    sts = {}
    for fused in (True, False):
        st = _state(gpu, batch, max(lengths) + steps + 32, fused=fused, split_tokens=split_tokens, kv_dtype=kvd)
        _load(st, lengths, kpre, vpre)
        sts[fused] = st
    states = []
    for b, n in enumerate(lengths):
        s = O.SequenceState()
        s.keys[0], s.values[0], s.tokens_seen = kpre[b:b + 1, :, :n].float(), vpre[b:b + 1, :, :n].float(), n
        states.append(s)
    for t in range(steps):
        outs = {}
        for fused, st in sts.items():
            outs[fused] = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu),
                                       x["gate"][t].to(gpu), out_dtype=torch.float32, q_norm_weight=qnw,
                                       k_norm_weight=knw)
            st.advance()
        # the cache: bit for bit what the separate append writes
        for b, n in enumerate(lengths):
            kf, vf = sts[True].gather_kv(0, 0, n + t + 1)
            ku, vu = sts[False].gather_kv(0, 0, n + t + 1)
            assert torch.equal(kf[b], ku[b]) and torch.equal(vf[b], vu[b]), (t, b)
        # the output: the new token's score and weight are exact fp32 in the combine (hi/lo MFMA
        # operands in the split-K launch), so the two agree to far below the activation tolerance
        torch.testing.assert_close(outs[True].cpu(), outs[False].cpu(), rtol=1e-4, atol=1e-5)
        if not norms:
            want = O.full_step_batched(states, 0, x["q"][t].float(), x["k"][t].float(), x["v"][t].float(),
                                       x["gate"][t].float())
            for s in states:
                s.tokens_seen += 1
            assert_act_close(outs[True], want, f"step {t}")
