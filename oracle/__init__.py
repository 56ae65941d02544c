"""Parity oracle for the hybrid-attention hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the router_ia package.  The modules
restate the reference's algorithm on the CPU:

  qwen36_cpu  torch-CPU restatement of v2/src/router_ia/qwen36_attention_cache.py
              (same ops, order and dtypes as the reference CPU path)
  fp64        independent float64 brute force used to pin qwen36_cpu
  chunked     chunked (WY, chunk 64) gated delta rule and causal attention
              prefill, restated from transformers 5.15.0's
              torch_chunk_gated_delta_rule, which the reference calls at
              v2/src/router_ia/qwen36_linear_attention_hf.py:91-100
"""
