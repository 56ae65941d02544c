"""Sequence (prefill) forms of the gated delta rule and of causal attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference prefills token by token through the recurrent rule
(v2/src/router_ia/qwen36_chat_batch.py:255-258 -> qwen36_attention_cache.py:256-266);
its HF-compatible path instead hands the first token of a sequence to
transformers' ``torch_chunk_gated_delta_rule`` (chunk 64,
v2/src/router_ia/qwen36_linear_attention_hf.py:91-100) and later tokens to
``gated_delta_recurrent`` (:108-137).  transformers (5.15.0 in this image)
is a third-party dependency absent from the reference tree; its chunk rule is
the WY-representation algorithm of the gated delta rule (Yang et al.,
"Gated Delta Networks", 2024).  Both forms are restated here from the
mathematics, batch 1, heads in the middle: x[L, H, d].

Per head, with k, q l2-normalised, q scaled by dk^-0.5 and chunks of C
tokens (cumulative log-decay G within the chunk, D[i,j] = exp(G_i - G_j) for
j <= i):
    L   = strict_lower((beta k) k^T o D)            intra-chunk interactions
    T   = (I + L)^-1                               forward substitution
    U   = T (beta v),  W = T (beta exp(G) k)        WY factors
    v'  = U - W S                                  corrected values
    o   = (exp(G) q) S + (q k^T o D, j <= i) v'
    S  <- exp(G_C) S + (exp(G_C - G) k)^T v'
"""

from __future__ import annotations

import torch

from .qwen36_cpu import l2norm


def _prep(q, k, v, g, beta):
    dk = q.shape[-1]
    q = l2norm(q.float()) * (dk ** -0.5)
    k = l2norm(k.float())
    return q, k, v.float(), g.float(), beta.float()


def recurrent_gated_delta_rule(q, k, v, g, beta, state=None):
    """Token-by-token rule.  q, k [L, H, dk]; v [L, H, dv]; g, beta [L, H].

    Returns (o [L, H, dv] fp32, final state [H, dk, dv] fp32).  Same step as
    qwen36_attention_cache.py:261-266 applied to every token in order.
    """
    q, k, v, g, beta = _prep(q, k, v, g, beta)
    length, heads, dk = q.shape
    dv = v.shape[-1]
    s = torch.zeros((heads, dk, dv)) if state is None else state.float().clone()
    out = torch.zeros((length, heads, dv))
    for t in range(length):
        s = s * torch.exp(g[t])[:, None, None]
        retrieved = (s * k[t][:, :, None]).sum(dim=1)
        delta = (v[t] - retrieved) * beta[t][:, None]
        s = s + k[t][:, :, None] * delta[:, None, :]
        out[t] = (s * q[t][:, :, None]).sum(dim=1)
    return out, s


def chunk_gated_delta_rule(q, k, v, g, beta, state=None, chunk: int = 64):
    """WY chunk form of the same rule; same contract as recurrent_gated_delta_rule."""
    q, k, v, g, beta = _prep(q, k, v, g, beta)
    length, heads, dk = q.shape
    dv = v.shape[-1]
    pad = (-length) % chunk
    if pad:
        # padded tokens: k = v = beta = g = 0 leave the state untouched
        q, k, v = (torch.cat([x, x.new_zeros((pad, heads, x.shape[-1]))]) for x in (q, k, v))
        g, beta = (torch.cat([x, x.new_zeros((pad, heads))]) for x in (g, beta))
    n_chunks = (length + pad) // chunk
    s = torch.zeros((heads, dk, dv)) if state is None else state.float().clone()
    out = torch.zeros((n_chunks * chunk, heads, dv))
    lower = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool))
    strict = torch.tril(torch.ones(chunk, chunk, dtype=torch.bool), diagonal=-1)
    eye = torch.eye(chunk)
    for c in range(n_chunks):
        sl = slice(c * chunk, (c + 1) * chunk)
        qc, kc, vc = (x[sl].transpose(0, 1) for x in (q, k, v))  # [H, C, d]
        gc, bc = g[sl].transpose(0, 1), beta[sl].transpose(0, 1)  # [H, C]
        G = torch.cumsum(gc, dim=-1)
        D = torch.exp((G[:, :, None] - G[:, None, :]).masked_fill(~lower, 0.0)) * lower
        kb = kc * bc[..., None]
        Lm = (kb @ kc.transpose(1, 2)) * D * strict
        T = torch.linalg.solve_triangular(eye + Lm, eye.expand(heads, chunk, chunk), upper=False,
                                          unitriangular=True)
        U = T @ (vc * bc[..., None])
        W = T @ (kb * torch.exp(G)[..., None])
        v_new = U - W @ s
        qk = (qc @ kc.transpose(1, 2)) * D
        o = (qc * torch.exp(G)[..., None]) @ s + qk @ v_new
        out[sl] = o.transpose(0, 1)
        g_last = G[:, -1]
        s = s * torch.exp(g_last)[:, None, None] + (kc * torch.exp(g_last[:, None] - G)[..., None]).transpose(1, 2) @ v_new
    return out[:length], s


def causal_conv1d_sequence(x, conv_weight, conv_state=None):
    """Causal depthwise conv + SiLU over a sequence, in the conv-weight dtype.

    x [L, C]; conv_weight [C, 1, 4]; conv_state [1, C, 4] (the reference's
    window, newest last) or None.  Equal to calling the one-token step
    (qwen36_attention_cache.py:176-221) L times.  Returns (out [L, C] in x's
    dtype, final window [1, C, 4]).
    """
    length, channels = x.shape
    dt = conv_weight.dtype
    if conv_state is None:
        conv_state = torch.zeros((1, channels, 4), dtype=dt)
    hist = torch.cat([conv_state.to(dt)[0, :, 1:], x.to(dt).transpose(0, 1)], dim=1)  # [C, 3 + L]
    out = torch.nn.functional.conv1d(hist.unsqueeze(0), conv_weight, groups=channels)[0]  # [C, L]
    out = torch.nn.functional.silu(out).transpose(0, 1).to(x.dtype)
    window = torch.cat([conv_state.to(dt)[0], x.to(dt).transpose(0, 1)], dim=1)[:, -4:].unsqueeze(0)
    return out, window


def causal_attention_prefill(q, k, v, gate, positions, num_kv_groups: int = 8, scale: float = 256 ** -0.5):
    """Gated causal GQA attention over a whole sequence, with partial RoPE.

    q, gate [L, Hq, 256]; k, v [L, Hkv, 256]; positions [L] ints.  Token t
    attends to tokens 0..t, exactly what L decode steps of
    qwen36_attention_cache.py:306-317 compute.  Returns (out [L, Hq, 256] fp32,
    rotated keys [L, Hkv, 256] fp32).
    """
    from .qwen36_cpu import apply_rope

    length = q.shape[0]
    qr = torch.empty(q.shape)
    kr = torch.empty(k.shape)
    for t in range(length):
        a, b = apply_rope(q[t:t + 1].float(), k[t:t + 1].float(), int(positions[t]))
        qr[t], kr[t] = a[0], b[0]
    kx = kr.repeat_interleave(num_kv_groups, dim=1).transpose(0, 1)  # [Hq, L, d]
    vx = v.float().repeat_interleave(num_kv_groups, dim=1).transpose(0, 1)
    scores = (qr.transpose(0, 1) @ kx.transpose(1, 2)) * scale  # [Hq, L, L]
    mask = torch.triu(torch.ones(length, length, dtype=torch.bool), diagonal=1)
    probs = torch.softmax(scores.masked_fill(mask, float("-inf")), dim=-1)
    out = (probs @ vx).transpose(0, 1) * torch.sigmoid(gate.float())
    return out, kr
