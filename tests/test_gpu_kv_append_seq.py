"""GPU parity: a prompt's append (ria_kv_append_seq, one workgroup per page)
writes the same page bits as one ria_kv_append per token.

Both follow the reference's per-token cache update (qwen36_attention_cache.py:
303-305 k_norm, :154-162 RoPE, :365-372 the appended k and v): the prompt
kernel must reproduce the one-token kernel's sums of squares, rotation and
rounding exactly, write whole pages with wide stores, and leave the tokens of
its first and last pages that lie outside the prompt untouched.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from router_ia import kernels as K

HKV, POOL, ROW_PAGES = 2, 40, 24


@pytest.mark.gpu
@pytest.mark.parametrize(
    "start,length,kv_dtype,norm",
    [
        (0, 64, torch.bfloat16, False),    # whole pages only
        (5, 40, torch.bfloat16, True),     # partial first and last pages, k_norm
        (13, 3, torch.float16, True),      # inside one page
        (16, 17, torch.bfloat16, False),   # one token on the last page
        (7, 300, torch.float16, False),    # many pages, fp16 cache
        (0, 1, torch.bfloat16, True),      # a single token
    ],
)
def test_prompt_append_matches_token_appends(gpu, start, length, kv_dtype, norm):
    announce(f"kv_append_seq vs kv_append: start {start}, length {length}, {kv_dtype}, k_norm {norm}")
    g = torch.Generator().manual_seed(1000 + start + length)
    k = torch.randn((length, HKV, 256), generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn((length, HKV, 256), generator=g).to(torch.bfloat16).to(gpu)
    perm = torch.randperm(POOL, generator=g)[:ROW_PAGES].to(torch.int32).to(gpu)
    # caches start full of other tokens, so untouched slots are checked as well
    k_a = torch.randn((POOL, HKV, 8, 4, 16, 8), generator=g).to(kv_dtype).to(gpu)
    v_a = torch.randn((POOL, HKV, 256, 16), generator=g).to(kv_dtype).to(gpu)
    k_b, v_b = k_a.clone(), v_a.clone()
    inv_freq = (1.0 / (1e7 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(gpu)
    knw = (0.1 * torch.randn((256,), generator=g)).to(gpu) if norm else None

    K.kv_append_seq(k, v, k_a, v_a, perm, start=start, inv_freq=inv_freq, k_norm_weight=knw)
    table = perm.view(1, -1)
    for i in range(length):
        K.kv_append(k[i:i + 1], v[i:i + 1], k_b, v_b, table, positions=start + i, slots=start + i,
                    inv_freq=inv_freq, k_norm_weight=knw)
    torch.cuda.synchronize()
    assert torch.equal(k_a.view(torch.int16), k_b.view(torch.int16))
    assert torch.equal(v_a.view(torch.int16), v_b.view(torch.int16))
