"""GPU parity of the 40-layer decode stack at the full sizes of the two stack workloads.

* 32 sequences, every one at context 8192 (seed 2);
* 128 sequences at contexts uniform in [1024, 32768] (seed 4), 16-token pages
  with a shuffled page table (about 147k pages per layer, 45 GB of KV).

Both run the benchmark's own decode path for 2 steps: per full-attention
layer one ``ria_attn_decode_append`` (balanced stream-K split over every
row's resident pages; the combine launch appends each row's new token into
its page and folds it in), per DeltaNet layer one ``ria_gdn_decode`` (fused
conv, raw gates), bf16 outputs.  Resident state and per-step inputs are
seeded draws made on the device, as the benchmark makes them.

Checked, following the reference's per-sequence semantics
(v2/src/router_ia/qwen36_attention_cache.py:256-266, 306-317):
  * every row at step 0: the first DeltaNet layer's output and new state, and
    the first attention layer's output (over the row's resident tokens read
    out of the pages, the oracle's grouped GQA product);
  * four sampled rows (the shortest, the longest and two others), exported
    with ``save_row(r).to_reference()`` before the first step and continued
    by the oracle: every layer's output of every step within the activation
    tolerance, and the final DeltaNet state of every layer within 1e-4
    relative;
  * every row: outputs finite; each appended token at
    page_table[row][t // 16] * 16 + t % 16 of every full layer, bit for bit
    (v, and the 192 dims of k that RoPE leaves unrotated), its rotated dims
    within the activation tolerance; pages in no row's table unchanged.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close, assert_state_close
from oracle import qwen36_cpu as O
from router_ia import _native as nat
from router_ia import kernels as K
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState
from router_ia.snapshot import full_model_layers, linear_model_layers

pytestmark = pytest.mark.gpu

LAYERS = 40
STEPS = 2
CASES = {
    "batch32-ctx8192": dict(batch=32, lo=8192, hi=8192, seed=2),
    "ragged128": dict(batch=128, lo=1024, hi=32768, seed=4),
}


def _sampled_rows(lengths: list[int]) -> list[int]:
    order = sorted(range(len(lengths)), key=lambda r: (lengths[r], r))
    rows = [order[0], order[-1], order[len(order) // 3], order[(2 * len(order)) // 3]]
    return sorted(set(rows))


@pytest.mark.timeout(480)
@pytest.mark.parametrize("case", sorted(CASES))
def test_stack_at_full_size_matches_oracle(gpu, case):
    cfg = CASES[case]
    batch = cfg["batch"]
    lengths = W.ragged_lengths(cfg["seed"], batch, cfg["lo"], cfg["hi"])
    rows = _sampled_rows(lengths)
    announce(f"full-size stack {case}: B={batch}, mean context {sum(lengths) / batch:.0f}, max {max(lengths)}, "
             f"sampled rows {rows} at {[lengths[r] for r in rows]}")
    num_pages = sum((n + STEPS + 15) // 16 for n in lengths) + batch
    st = BatchedAttentionState(batch, max(lengths) + STEPS + 16, num_pages=num_pages, device=gpu,
                               page_shuffle_seed=cfg["seed"])
    assert st.split_tokens == 0  # the balanced partition the benchmark runs
    st.set_positions(lengths)
    st.reserve(STEPS)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(cfg["seed"])
    for li in range(st.num_linear_layers):
        st.linear_states[li].normal_(0.0, 0.02, generator=gen)
        st.conv_rings[li].normal_(0.0, 1.0, generator=gen)
    for fi in range(st.num_full_layers):
        st.kv.k[fi].normal_(0.0, 1.0, generator=gen)
        st.kv.v[fi].normal_(0.0, 1.0, generator=gen)
    conv_w = [(torch.randn((W.CONV_DIM, 1, 4), generator=gen, device=gpu) * 0.5).to(torch.bfloat16)
              for _ in range(st.num_linear_layers)]
    a_log = [torch.rand((W.NUM_V_HEADS,), generator=gen, device=gpu) * 4.0 - 4.0
             for _ in range(st.num_linear_layers)]
    dt_bias = [torch.zeros((W.NUM_V_HEADS,), device=gpu) for _ in range(st.num_linear_layers)]
    torch.cuda.synchronize()

    # the sampled rows' state in the reference's layout, continued by the oracle
    lin_layers, full_layers = linear_model_layers(30), full_model_layers(10)
    oracle = {}
    for r in rows:
        ref = st.save_row(r).to_reference()
        s = O.SequenceState()
        s.tokens_seen = ref["tokens_seen"]
        for li, m in enumerate(lin_layers):
            s.linear[li] = ref["linear_states"][m].cpu()
            s.conv[li] = ref["linear_conv_states"][m].cpu()
        for fi, m in enumerate(full_layers):
            s.keys[fi] = ref["full_keys"][m].float().cpu()
            s.values[fi] = ref["full_values"][m].float().cpu()
        del ref
        oracle[r] = s
    assert all(oracle[r].tokens_seen == lengths[r] for r in rows)
    announce(f"{case}: oracle state exported for rows {rows}")

    # pages in no row's table: their contents must not change
    used = {p for table in st.kv.alloc.tables for p in table}
    free = torch.tensor(sorted(set(range(num_pages)) - used), dtype=torch.long, device=gpu)
    assert free.numel() > 0
    free_k, free_v = st.kv.k[:, free].clone(), st.kv.v[:, free].clone()

    # every row at step 0: the first DeltaNet layer's state before the step
    lin0_before = st.linear_states[0].cpu()
    ring0_before = st.conv_rings[0].cpu()
    first = {}  # step 0's inputs and outputs of model layers 0 and 3, every row

    gdn_out = torch.empty((batch, W.NUM_V_HEADS, 128), device=gpu, dtype=torch.bfloat16)
    attn_out = torch.empty((batch, W.FULL_Q_HEADS, W.FULL_HEAD_DIM), device=gpu, dtype=torch.bfloat16)
    appended = []  # (step, layer index, positions, k, v) of every appended token
    rsel = torch.tensor(rows, dtype=torch.long)
    for s in range(STEPS):
        mixed = torch.randn((st.num_linear_layers, batch, W.CONV_DIM), generator=gen, device=gpu,
                            dtype=torch.bfloat16)
        gate_ab = torch.randn((st.num_linear_layers, 2, batch, W.NUM_V_HEADS), generator=gen, device=gpu)
        qg = torch.randn((st.num_full_layers, 2, batch, W.FULL_Q_HEADS, W.FULL_HEAD_DIM), generator=gen,
                         device=gpu, dtype=torch.bfloat16)
        kv_in = torch.randn((st.num_full_layers, 2, batch, W.FULL_KV_HEADS, W.FULL_HEAD_DIM), generator=gen,
                            device=gpu, dtype=torch.bfloat16)
        positions = list(st._host_seen)
        max_ctx = st.max_seen + 1
        for layer in range(LAYERS):
            if layer % 4 == 3:
                fi = layer // 4
                kc, vc = st.kv.layer(fi)
                K.attn_decode_append(qg[fi, 0], qg[fi, 1], kv_in[fi, 0], kv_in[fi, 1], kc, vc, st.kv.page_table,
                                     attn_out, positions=st.tokens_seen, ctx_lens=st.ctx_lens, max_ctx=max_ctx,
                                     inv_freq=st.inv_freq, scale=st.scale, workspace=st.workspace)
                out = attn_out
                want = O.full_step_batched([oracle[r] for r in rows], fi, qg[fi, 0][rsel].cpu(),
                                           kv_in[fi, 0][rsel].cpu(), kv_in[fi, 1][rsel].cpu(),
                                           qg[fi, 1][rsel].cpu())
                appended.append((s, fi, positions, kv_in[fi, 0].clone(), kv_in[fi, 1].clone()))
                if s == 0 and fi == 0:
                    first["attn"] = (attn_out.float().cpu(), qg[0, 0].cpu(), qg[0, 1].cpu(), kv_in[0, 0].cpu(),
                                     kv_in[0, 1].cpu())
            else:
                li = layer - layer // 4
                K.gdn_decode(mixed[li], st.linear_states[li], gate_ab[li, 0], gate_ab[li, 1], gdn_out,
                             num_k_heads=st.num_k_heads, num_v_heads=st.num_v_heads, conv_weight=conv_w[li],
                             conv_ring=st.conv_rings[li], conv_pos=st.tokens_seen, gate_mode=nat.RIA_GATE_RAW,
                             A_log=a_log[li], dt_bias=dt_bias[li])
                out = gdn_out
                if s == 0 and li == 0:
                    first["gdn"] = (gdn_out.float().cpu(), st.linear_states[0].cpu(), mixed[0].cpu(),
                                    gate_ab[0, 0].cpu(), gate_ab[0, 1].cpu())
                beta, g = O.gating(gate_ab[li, 0][rsel].cpu(), gate_ab[li, 1][rsel].cpu(), a_log[li].cpu(),
                                   dt_bias[li].cpu())
                want = O.linear_step_batched([oracle[r] for r in rows], li, mixed[li][rsel].cpu(),
                                             conv_w[li].cpu(), beta, g)
            assert bool(torch.isfinite(out.float()).all()), f"non-finite output, step {s} layer {layer}"
            assert_act_close(out[rsel], want, f"{case} step {s} layer {layer} rows {rows}")
        st.advance()
        for r in rows:
            oracle[r].tokens_seen += 1
        announce(f"{case}: step {s} matches the oracle on rows {rows} through all {LAYERS} layers")

    torch.cuda.synchronize()
    for li in range(st.num_linear_layers):
        for r in rows:
            assert_state_close(st.linear_states[li, r].cpu().unsqueeze(0), oracle[r].linear[li],
                               f"{case} final state layer {li} row {r}")

    # every row's appended tokens, at their slots of every full layer, through the host page tables
    tables = [list(t) for t in st.kv.alloc.tables]
    for s, fi, positions, k_in, v_in in appended:
        tok = torch.tensor(positions, dtype=torch.long)
        phys = torch.tensor([tables[b][int(t) // 16] for b, t in enumerate(tok)], dtype=torch.long, device=gpu)
        off = (tok % 16).to(gpu)
        v_got = st.kv.v[fi][phys, :, :, off]                   # [B, Hkv, 256]
        assert torch.equal(v_got, v_in), f"{case}: v slot mapping, step {s} layer {fi}"
        dims = torch.arange(256, device=gpu)
        kk, gg, jj = (dims % 64) // 8, dims // 64, dims % 8
        k_got = st.kv.k[fi][phys[:, None, None], torch.arange(2, device=gpu)[None, :, None], kk, gg,
                            off[:, None, None], jj]          # [B, Hkv, 256] in dim order
        assert torch.equal(k_got[:, :, 64:], k_in[:, :, 64:]), f"{case}: k slot mapping, step {s} layer {fi}"
        for b in rows:
            _, k_rot = O.apply_rope(k_in[b:b + 1].float().cpu(), k_in[b:b + 1].float().cpu(), positions[b])
            assert_act_close(k_got[b].cpu(), k_rot[0], f"{case}: rotated k, row {b} step {s} layer {fi}")
    assert torch.equal(st.kv.k[:, free], free_k) and torch.equal(st.kv.v[:, free], free_v), \
        f"{case}: a page in no row's table changed"

    # every row, step 0, model layer 0 (DeltaNet) and layer 3 (full attention) against the oracle
    out0, lin0_after, mixed0, a0, b0 = first["gdn"]
    beta, g = O.gating(a0, b0, a_log[0].cpu(), dt_bias[0].cpu())
    for r in range(batch):
        t = lengths[r]
        # the ring holds token n's conv input in slot n mod 4; the reference's window is oldest first
        window = ring0_before[r, [(t - 4 + m) % 4 for m in range(4)]].t().unsqueeze(0)
        want, _, s_new = O.linear_decode_step(window, lin0_before[r:r + 1], mixed0[r:r + 1], conv_w[0].cpu(),
                                              beta[r:r + 1], g[r:r + 1])
        assert_act_close(out0[r:r + 1], want, f"{case}: step 0 layer 0 row {r}")
        assert_state_close(lin0_after[r:r + 1], s_new, f"{case}: step 0 layer 0 state row {r}")
    announce(f"{case}: step 0, DeltaNet layer 0 matches the oracle on all {batch} rows")
    out3, q3, gate3, k3, v3 = first["attn"]
    for r in range(batch):
        t = lengths[r]
        # the row's resident tokens [0, t) in logical order, read out of the pages through the host table
        phys = torch.tensor(tables[r][:(t + 15) // 16], dtype=torch.long, device=gpu)
        k_rows = st.kv.k[0][phys].permute(1, 0, 4, 3, 2, 5).reshape(2, -1, 256)[:, :t]  # [Hkv, T, 256]
        v_rows = st.kv.v[0][phys].permute(1, 0, 3, 2).reshape(2, -1, 256)[:, :t]
        want, _, _ = O.full_decode_step_grouped(k_rows.float().cpu().unsqueeze(0), v_rows.float().cpu().unsqueeze(0),
                                                q3[r:r + 1], k3[r:r + 1], v3[r:r + 1], gate3[r:r + 1], t)
        assert_act_close(out3[r:r + 1], want, f"{case}: step 0 layer 3 row {r} (context {t})")
    announce(f"{case}: step 0, attention layer 3 matches the oracle on all {batch} rows")
