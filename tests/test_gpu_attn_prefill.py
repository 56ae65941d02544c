"""GPU parity: causal GQA attention prefill over the paged KV cache.

The reference prefills by running one decode step per prompt token
(qwen36_chat_batch.py:255-258 -> qwen36_attention_cache.py:306-317), so the
oracle is `oracle.chunked.causal_attention_prefill` (pinned against that
token-by-token recurrence in test_oracle_chunked.py).  Covered here: ragged
prompt lengths over shuffled pages, a prompt continued after resident
context, fp16 activations with fp16 pages, GQA groups below 8, the pages the
prefill writes (bit-exact against the decode append), prefill == decode
steps, and a 16384-token prompt checked row-by-row on sampled tokens.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close
from oracle import chunked as OC
from oracle import qwen36_cpu as O
from router_ia import kernels as K
from router_ia.batched_state import rope_inv_freq
from router_ia.paged_kv import PagedKVCache

SCALE = 256 ** -0.5


def _inputs(seed, length, hq=16, hkv=2, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((length, hq, 256), generator=g).to(dtype)
    k = torch.randn((length, hkv, 256), generator=g).to(dtype)
    v = torch.randn((length, hkv, 256), generator=g).to(dtype)
    gate = torch.randn((length, hq, 256), generator=g).to(dtype)
    return q, k, v, gate


def _cache(dev, tokens, hkv=2, dtype=torch.bfloat16, shuffle_seed=5):
    pages = (tokens + 15) // 16 + 3
    kv = PagedKVCache(1, pages, 1, pages, num_kv_heads=hkv, device=dev, shuffle_seed=shuffle_seed, dtype=dtype)
    kv.ensure(0, tokens)
    return kv


def _run(dev, kv, q, k, v, gate, start, staged=False, phase=None):
    inv = rope_inv_freq(10_000_000.0, 64).to(dev)
    length, hkv = int(q.shape[0]), int(k.shape[1])
    stage = torch.empty(K.prefill_stage_bytes(length, hkv), dtype=torch.uint8, device=dev) if staged else None
    qd, kd, vd, gd = q.to(dev), k.to(dev), v.to(dev), gate.to(dev)
    if phase is None:
        return K.attn_prefill(qd, kd, vd, gd, kv.k[0], kv.v[0], kv.page_table[0], start=start, inv_freq=inv,
                              scale=SCALE, stage=stage)
    from router_ia import _native as nat
    out = K.attn_prefill(qd, kd, vd, gd, kv.k[0], kv.v[0], kv.page_table[0], start=start, inv_freq=inv,
                         scale=SCALE, stage=stage, phase=nat.RIA_PREFILL_APPEND)
    return K.attn_prefill(qd, kd, vd, gd, kv.k[0], kv.v[0], kv.page_table[0], out, start=start, inv_freq=inv,
                          scale=SCALE, stage=stage, phase=nat.RIA_PREFILL_ATTEND)


@pytest.mark.gpu
@pytest.mark.parametrize("length", [1, 15, 16, 17, 300, 1000])
def test_attn_prefill_matches_oracle(gpu, length):
    announce(f"attn_prefill: L={length}, bf16, shuffled pages")
    q, k, v, gate = _inputs(100 + length, length)
    kv = _cache(gpu, length)
    out = _run(gpu, kv, q, k, v, gate, 0)
    want, kr = OC.causal_attention_prefill(q, k, v, gate, torch.arange(length))
    assert_act_close(out, want, f"L={length}")
    # the pages hold v exactly and the rotated keys rounded once to bf16
    kg, vg = K.kv_gather(kv.k[0], kv.v[0], kv.page_table, batch=1, start=0, count=length)
    assert torch.equal(vg[0].cpu(), v.transpose(0, 1))
    torch.testing.assert_close(kg[0].cpu().float(), kr.transpose(0, 1).to(torch.bfloat16).float(),
                               rtol=8e-3, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("length,hq,hkv,phases", [(1, 16, 2, False), (17, 16, 2, True), (300, 16, 2, False),
                                                   (1000, 16, 2, True), (130, 6, 2, False)])
def test_attn_prefill_staged_fp16_keys(gpu, length, hq, hkv, phases):
    # a prompt from slot 0 with an fp16 stage: the pages get exactly what the unstaged append writes, the
    # attention reads the prompt's fp16 keys (single fp16 MFMA operands) and matches the oracle
    announce(f"attn_prefill staged: L={length}, Hq={hq}, Hkv={hkv}, {'two phases' if phases else 'one call'}")
    q, k, v, gate = _inputs(200 + length, length, hq, hkv)
    kv_s, kv_u = _cache(gpu, length, hkv=hkv), _cache(gpu, length, hkv=hkv)
    out_s = _run(gpu, kv_s, q, k, v, gate, 0, staged=True, phase=phases or None)
    out_u = _run(gpu, kv_u, q, k, v, gate, 0)
    assert torch.equal(kv_s.k, kv_u.k) and torch.equal(kv_s.v, kv_u.v), "pages differ from the unstaged append"
    want, _ = OC.causal_attention_prefill(q, k, v, gate, torch.arange(length), num_kv_groups=hq // hkv)
    assert_act_close(out_s, want, f"staged L={length}")


@pytest.mark.gpu
def test_attn_prefill_continues_after_resident_context(gpu):
    """Prompt of 157 tokens on top of 100 prefilled ones == one 257-token prompt."""
    announce("attn_prefill: 100 + 157 tokens in two calls")
    n0, n1 = 100, 157
    q, k, v, gate = _inputs(7, n0 + n1)
    kv = _cache(gpu, n0 + n1)
    out0 = _run(gpu, kv, q[:n0], k[:n0], v[:n0], gate[:n0], 0, staged=True)
    # (a stage is ignored past slot 0: the resident keys are only in the pages)
    out1 = _run(gpu, kv, q[n0:], k[n0:], v[n0:], gate[n0:], n0, staged=True)
    want, _ = OC.causal_attention_prefill(q, k, v, gate, torch.arange(n0 + n1))
    assert_act_close(torch.cat([out0.cpu(), out1.cpu()]), want, "two-call prefill")


@pytest.mark.gpu
def test_attn_prefill_fp16_pages(gpu):
    announce("attn_prefill: L=333, fp16 activations and fp16 pages")
    length = 333
    q, k, v, gate = _inputs(9, length, dtype=torch.float16)
    kv = _cache(gpu, length, dtype=torch.float16)
    out = _run(gpu, kv, q, k, v, gate, 0)
    assert out.dtype == torch.float16
    want, _ = OC.causal_attention_prefill(q, k, v, gate, torch.arange(length))
    assert_act_close(out, want, "fp16")


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv", [(8, 2), (6, 2), (4, 4), (1, 1)])
def test_attn_prefill_gqa_groups(gpu, hq, hkv):
    announce(f"attn_prefill: Hq={hq}, Hkv={hkv}, L=130")
    length = 130
    q, k, v, gate = _inputs(11 + hq, length, hq, hkv)
    kv = _cache(gpu, length, hkv=hkv)
    out = _run(gpu, kv, q, k, v, gate, 0)
    want, _ = OC.causal_attention_prefill(q, k, v, gate, torch.arange(length), num_kv_groups=hq // hkv)
    assert_act_close(out, want, f"Hq={hq} Hkv={hkv}")


@pytest.mark.gpu
def test_attn_prefill_equals_decode_steps(gpu):
    """The prefill writes the same pages as per-token appends, and its outputs match per-token decode."""
    announce("attn_prefill vs decode steps: L=200")
    length = 200
    q, k, v, gate = _inputs(13, length)
    inv = rope_inv_freq(10_000_000.0, 64).to(gpu)
    kv_a = _cache(gpu, length, shuffle_seed=1)
    out_p = _run(gpu, kv_a, q, k, v, gate, 0)
    kv_b = _cache(gpu, length, shuffle_seed=2)
    ws = torch.empty(K.attn_decode_workspace_bytes(1, 16, 2, length, 64) // 4 + 64, dtype=torch.float32,
                     device=gpu)
    outs = []
    for t in range(length):
        K.kv_append(k[t:t + 1].to(gpu), v[t:t + 1].to(gpu), kv_b.k[0], kv_b.v[0], kv_b.page_table, positions=t,
                    slots=t, inv_freq=inv)
        o = torch.empty((1, 16, 256), dtype=torch.float32, device=gpu)
        K.attn_decode(q[t:t + 1].to(gpu), gate[t:t + 1].to(gpu), kv_b.k[0], kv_b.v[0], kv_b.page_table, o,
                      positions=t, ctx_lens=t + 1, max_ctx=length, inv_freq=inv, scale=SCALE, workspace=ws,
                      split_tokens=64)
        outs.append(o.cpu())
    dec = torch.cat(outs)
    assert_act_close(out_p, dec, "prefill vs decode")
    ka, va = K.kv_gather(kv_a.k[0], kv_a.v[0], kv_a.page_table, batch=1, start=0, count=length)
    kb, vb = K.kv_gather(kv_b.k[0], kv_b.v[0], kv_b.page_table, batch=1, start=0, count=length)
    assert torch.equal(ka, kb) and torch.equal(va, vb)


def _row_reference(qr, kr, v, gate, t, group=8):
    """fp64 attention of query token t over keys 0..t (all heads)."""
    kx = kr[: t + 1].double().repeat_interleave(group, dim=1)  # [t+1, Hq, d]
    vx = v[: t + 1].double().repeat_interleave(group, dim=1)
    s = torch.einsum("hd,thd->ht", qr[t].double(), kx) * SCALE
    p = torch.softmax(s, dim=-1)
    return torch.einsum("ht,thd->hd", p, vx) * torch.sigmoid(gate[t].double())


@pytest.mark.gpu
@pytest.mark.parametrize("staged", [False, True], ids=["pages", "stage"])
def test_attn_prefill_16384_sampled_rows(gpu, staged):
    """Full-size prompt: 16384 tokens, 48 sampled query rows against fp64 attention."""
    announce(f"attn_prefill: L=16384, sampled rows vs fp64, keys from the {'stage' if staged else 'pages'}")
    length = 16384
    q, k, v, gate = _inputs(17, length)
    kv = _cache(gpu, length)
    out = _run(gpu, kv, q, k, v, gate, 0, staged=staged).cpu()
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(3)
    rows = sorted(set([0, 1, 15, 16, 4095, 8191, length - 1] + torch.randint(0, length, (41,), generator=g).tolist()))
    qr = torch.empty(len(rows), 16, 256)
    kr = torch.empty(length, 2, 256)
    for t in range(length):  # each key rotated at its own position
        _, kt = O.apply_rope(k[t:t + 1].float(), k[t:t + 1].float(), t)
        kr[t] = kt[0]
    for i, t in enumerate(rows):
        qt, _ = O.apply_rope(q[t:t + 1].float(), q[t:t + 1].float(), t)
        qr[i] = qt[0]
    for i, t in enumerate(rows):
        qfull = torch.zeros(t + 1, 16, 256)
        qfull[t] = qr[i]
        want = _row_reference(qfull, kr, v.float(), gate.float(), t)
        assert_act_close(out[t], want.float(), f"row {t}")


@pytest.mark.gpu
@pytest.mark.parametrize("staged,bound", [(False, 0.7), (True, 0.35)], ids=["pages", "stage"])
def test_attn_prefill_keeps_its_tolerance_margin(gpu, staged, bound):
    """The worst error against the oracle stays well inside the activation
    tolerance across seeds and lengths (bf16 pages: q and P run as bf16 hi + lo
    pairs, a single bf16 P reached the tolerance itself on short prompts; fp16
    stage: single fp16 q and P over keys rounded once to fp16)."""
    announce(f"attn_prefill: error / tolerance over 9 prompts, keys from the {'stage' if staged else 'pages'}")
    from helpers import ACT_ATOL, ACT_RTOL
    worst = 0.0
    for length in (17, 300, 1000):
        for seed in (7, 42, 100 + length):
            q, k, v, gate = _inputs(seed, length)
            kv = _cache(gpu, length)
            out = _run(gpu, kv, q, k, v, gate, 0, staged=staged).float().cpu()
            want, _ = OC.causal_attention_prefill(q, k, v, gate, torch.arange(length))
            ratio = ((out - want.float()).abs() / (ACT_ATOL + ACT_RTOL * want.float().abs())).max().item()
            worst = max(worst, ratio)
    print(f"worst error / tolerance: {worst:.3f}", flush=True)
    assert worst <= bound, f"worst error is {worst:.3f} of the tolerance"
