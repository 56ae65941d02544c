"""Host-side pieces of the batched forward loop (no GPU).

q_proj's rows hold each head's query then its gate (qwen36_attention_cache.py:
295-299: reshape to [1, 16, 512], chunk in two); ``split_query_gate`` must
give two FP8 projections whose dequantised rows are exactly those halves.
"""

from __future__ import annotations

import pytest
import torch

from oracle import qwen36_cpu as O
from router_ia import batched_forward as BF
from router_ia import workloads as W


def test_split_query_gate_keeps_the_dequantised_rows():
    w8, s = W.fp8_block_weight(7, 2 * 16 * 256, 256)
    query, gate = BF.split_query_gate(BF.Fp8Projection(w8, s))
    assert query.weight.dtype == torch.float8_e4m3fn and query.weight.shape == (4096, 256)
    assert query.scale_inv.shape == (32, 2) and gate.scale_inv.shape == (32, 2)
    full = O.dequantize_fp8_blockwise(w8, s).reshape(16, 512, 256)
    want_q, want_g = torch.chunk(full, 2, dim=1)  # per head: first 256 rows query, last 256 gate
    assert torch.equal(O.dequantize_fp8_blockwise(query.weight, query.scale_inv), want_q.reshape(4096, 256))
    assert torch.equal(O.dequantize_fp8_blockwise(gate.weight, gate.scale_inv), want_g.reshape(4096, 256))


def test_split_query_gate_rejects_bad_shapes():
    w8, s = W.fp8_block_weight(8, 2 * 4 * 64, 128)
    with pytest.raises(ValueError, match="multiple of 128"):
        BF.split_query_gate(BF.Fp8Projection(w8, s), num_heads=4, head_dim=64)
    w8, s = W.fp8_block_weight(9, 1024, 128)
    with pytest.raises(ValueError, match="rows"):
        BF.split_query_gate(BF.Fp8Projection(w8, s))


def test_layer_weights_from_checkpoint_names():
    lin = BF.layer_weights(W.synthetic_layer(1, 0), 0)
    full = BF.layer_weights(W.synthetic_layer(2, 3), 3)
    assert isinstance(lin, BF.LinearLayerWeights) and isinstance(full, BF.FullLayerWeights)
    assert lin.in_proj_qkv.weight.shape == (8192, 2048) and lin.out_proj.weight.shape == (2048, 4096)
    assert lin.conv_weight.dtype == torch.bfloat16 and lin.norm_weight.dtype == torch.float32
    assert full.query.weight.shape == (4096, 2048) and full.k_proj.weight.shape == (512, 2048)
    assert full.q_norm.dtype == torch.float32 and full.o_proj.scale_inv.shape == (16, 32)
