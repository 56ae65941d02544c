"""Pin the sequence forms in oracle/chunked.py.

The chunked (WY) rule must equal the token-by-token recurrence (a closed-form
identity of the algebra), the sequence conv must equal repeated one-token
steps, and the causal prefill must equal repeated decode steps.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import chunked as C
from oracle import qwen36_cpu as O


def _inputs(seed, length, heads=4, dk=32, dv=32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((length, heads, dk), generator=g)
    k = torch.randn((length, heads, dk), generator=g)
    v = torch.randn((length, heads, dv), generator=g)
    gl = -F.softplus(torch.randn((length, heads), generator=g)) * torch.exp(torch.rand((length, heads), generator=g) * 4 - 4)
    beta = torch.sigmoid(torch.randn((length, heads), generator=g))
    return q, k, v, gl, beta


@pytest.mark.parametrize("length", [1, 63, 64, 65, 130])
def test_chunked_equals_recurrent(length):
    q, k, v, g, beta = _inputs(length, length)
    o1, s1 = C.recurrent_gated_delta_rule(q, k, v, g, beta)
    o2, s2 = C.chunk_gated_delta_rule(q, k, v, g, beta)
    torch.testing.assert_close(o2, o1, rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(s2, s1, rtol=2e-4, atol=2e-5)


def test_chunked_equals_recurrent_with_initial_state_full_head_dim():
    q, k, v, g, beta = _inputs(7, 100, heads=2, dk=128, dv=128)
    s0 = torch.randn((2, 128, 128), generator=torch.Generator().manual_seed(8)) * 0.02
    o1, s1 = C.recurrent_gated_delta_rule(q, k, v, g, beta, s0)
    o2, s2 = C.chunk_gated_delta_rule(q, k, v, g, beta, s0)
    torch.testing.assert_close(o2, o1, rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(s2, s1, rtol=2e-4, atol=2e-5)


def test_chunk_size_does_not_matter():
    q, k, v, g, beta = _inputs(9, 96)
    a, sa = C.chunk_gated_delta_rule(q, k, v, g, beta, chunk=16)
    b, sb = C.chunk_gated_delta_rule(q, k, v, g, beta, chunk=64)
    torch.testing.assert_close(a, b, rtol=2e-4, atol=2e-5)
    torch.testing.assert_close(sa, sb, rtol=2e-4, atol=2e-5)


def test_recurrent_matches_decode_step_of_the_attention_cache():
    # The batch-1 decode step of the cache (after GQA expansion) is one token of the rule.
    q, k, v, g, beta = _inputs(10, 5, heads=2, dk=128, dv=128)
    o_seq, s_seq = C.recurrent_gated_delta_rule(q, k, v, g, beta)
    s = None
    for t in range(5):
        o, s = O.gated_delta_step(s, q[t:t + 1], k[t:t + 1], v[t:t + 1], beta[t:t + 1], g[t:t + 1])
        torch.testing.assert_close(o[0], o_seq[t], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s[0], s_seq, rtol=1e-5, atol=1e-6)


def test_sequence_conv_equals_repeated_steps():
    g = torch.Generator().manual_seed(11)
    w = (torch.randn((64, 1, 4), generator=g) * 0.5).to(torch.bfloat16)
    x = torch.randn((9, 64), generator=g).to(torch.bfloat16)
    init = torch.randn((1, 64, 4), generator=g).to(torch.bfloat16)
    out, win = C.causal_conv1d_sequence(x, w, init)
    state = init
    for t in range(9):
        o, state = O.causal_conv1d_step(state, x[t:t + 1], w)
        assert torch.equal(out[t:t + 1], o)
    assert torch.equal(win, state)


def test_causal_prefill_equals_repeated_decode():
    g = torch.Generator().manual_seed(12)
    length = 11
    q = torch.randn((length, 16, 256), generator=g)
    k = torch.randn((length, 2, 256), generator=g)
    v = torch.randn((length, 2, 256), generator=g)
    gate = torch.randn((length, 16, 256), generator=g)
    out, kr = C.causal_attention_prefill(q, k, v, gate, list(range(100, 100 + length)))
    fk = fv = None
    for t in range(length):
        o, fk, fv = O.full_decode_step(fk, fv, q[t:t + 1], k[t:t + 1], v[t:t + 1], gate[t:t + 1], 100 + t)
        torch.testing.assert_close(out[t], o[0], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(kr.transpose(0, 1), fk[0])
