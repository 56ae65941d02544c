"""GPU parity: paged KV append with RoPE and split-K gated decode attention.

Covers the single-layer batch-1 workload (4096 prefilled tokens + 256 decode
steps, seed 1), ragged batches over a shuffled page table, forced split
sizes, the bit-exact slot mapping of the paged cache, and the gather used to
materialise the reference's contiguous KV view.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close
from oracle import qwen36_cpu as O
from router_ia import kernels as K
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState


def _attn_state(dev, batch, max_context, *, shuffle_seed=None, split_tokens=0):
    return BatchedAttentionState(batch, max_context, num_linear_layers=0, num_full_layers=1, device=dev,
                                 page_shuffle_seed=shuffle_seed, split_tokens=split_tokens)


def _prefill(st, lengths, kpre, vpre):
    """Load resident context: row b holds kpre[b, :, :lengths[b]] (already positioned keys)."""
    st.set_positions(lengths)
    for b, n in enumerate(lengths):
        st.kv.write_tokens(0, b, 0, kpre[b, :, :n].permute(1, 0, 2), vpre[b, :, :n].permute(1, 0, 2))


@pytest.mark.gpu
def test_attn_decode_single_layer_batch1_4096_plus_256(gpu):
    announce("attn_decode: 1 layer, B=1, 4096 prefilled + 256 steps, seed 1")
    steps, t0 = 256, 4096
    kpre, vpre = W.prefilled_kv(1, 1, t0)
    x = W.attn_step_inputs(1, steps, 1)
    st = _attn_state(gpu, 1, t0 + steps + 16)
    _prefill(st, [t0], kpre, vpre)
    got = []
    for t in range(steps):
        out = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu), x["gate"][t].to(gpu),
                           out_dtype=torch.float32)
        st.advance()
        got.append(out.cpu())
    fk, fv = kpre.float(), vpre.float()
    for t in range(steps):
        want, fk, fv = O.full_decode_step(fk, fv, x["q"][t], x["k"][t], x["v"][t], x["gate"][t], t0 + t)
        assert_act_close(got[t], want, f"step {t}")
    # the appended keys are RoPE-rotated at their own positions, stored in bf16
    k_g, v_g = st.gather_kv(0, t0, steps)
    assert torch.equal(v_g.cpu(), fv[:, :, t0:].to(torch.bfloat16))
    torch.testing.assert_close(k_g.cpu().float(), fk[:, :, t0:].to(torch.bfloat16).float(), rtol=8e-3, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("split_tokens", [0, 64, 192])
def test_attn_decode_ragged_shuffled_pages(gpu, split_tokens):
    announce(f"attn_decode: ragged B=6, shuffled pages, split_tokens={split_tokens}")
    lengths = [1, 15, 16, 17, 300, 1000]
    steps = 5
    batch = len(lengths)
    kpre, vpre = W.prefilled_kv(21, batch, max(lengths))
    x = W.attn_step_inputs(22, steps, batch)
    st = _attn_state(gpu, batch, max(lengths) + steps + 32, shuffle_seed=3, split_tokens=split_tokens)
    _prefill(st, lengths, kpre, vpre)
    states = []
    for b, n in enumerate(lengths):
        s = O.SequenceState()
        s.keys[0], s.values[0], s.tokens_seen = kpre[b:b + 1, :, :n].float(), vpre[b:b + 1, :, :n].float(), n
        states.append(s)
    for t in range(steps):
        out = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu), x["gate"][t].to(gpu),
                           out_dtype=torch.float32)
        want = O.full_step_batched(states, 0, x["q"][t], x["k"][t], x["v"][t], x["gate"][t])
        st.advance()
        for s in states:
            s.tokens_seen += 1
        assert_act_close(out, want, f"step {t}")


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", [[1], [40], [5000, 17, 2049], [3000, 3001, 16, 1, 777], [0, 9, 4096]])
def test_attn_decode_padded_partition_few_units(gpu, lengths):
    """Few (sequence, KV head) units against a large grid: every unit's page range is
    padded to whole chunks (units x 32 <= workgroups), so no workgroup straddles two
    units; tiny, page-aligned and ragged contexts in one launch."""
    announce(f"attn_decode: padded balanced partition, lengths {lengths}")
    batch, steps = len(lengths), 3
    kpre, vpre = W.prefilled_kv(27, batch, max(lengths))
    x = W.attn_step_inputs(28, steps, batch)
    st = _attn_state(gpu, batch, max(lengths) + steps + 32, shuffle_seed=11)
    assert st.split_tokens == 0  # the balanced partition
    _prefill(st, lengths, kpre, vpre)
    states = []
    for b, n in enumerate(lengths):
        s = O.SequenceState()
        s.keys[0], s.values[0], s.tokens_seen = kpre[b:b + 1, :, :n].float(), vpre[b:b + 1, :, :n].float(), n
        states.append(s)
    for t in range(steps):
        out = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu), x["gate"][t].to(gpu),
                           out_dtype=torch.float32)
        want = O.full_step_batched(states, 0, x["q"][t], x["k"][t], x["v"][t], x["gate"][t])
        st.advance()
        for s in states:
            s.tokens_seen += 1
        assert_act_close(out, want, f"step {t}")


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [24, 48], ids=["wave_partition", "block_partition"])
def test_attn_decode_balanced_partition_many_units(gpu, batch):
    """Balanced (stream-K) decode: 24 or 48 ragged rows, ~4.8k / ~9.6k pages over
    the grid, so workgroups cross unit boundaries and units span several
    workgroups.  48 units take the one-wave partition (up to 64 units), 96
    the block-wide scan."""
    announce(f"attn_decode: balanced partition, B={batch}, contexts U[200, 3000], shuffled pages")
    steps = 2
    lengths = W.ragged_lengths(24, batch, 200, 3000)
    kpre, vpre = W.prefilled_kv(25, batch, max(lengths))
    x = W.attn_step_inputs(26, steps, batch)
    st = _attn_state(gpu, batch, max(lengths) + steps + 32, shuffle_seed=7)
    assert st.split_tokens == 0  # the balanced partition
    _prefill(st, lengths, kpre, vpre)
    states = []
    for b, n in enumerate(lengths):
        s = O.SequenceState()
        s.keys[0], s.values[0], s.tokens_seen = kpre[b:b + 1, :, :n].float(), vpre[b:b + 1, :, :n].float(), n
        states.append(s)
    for t in range(steps):
        out = st.full_step(0, x["q"][t].to(gpu), x["k"][t].to(gpu), x["v"][t].to(gpu), x["gate"][t].to(gpu),
                           out_dtype=torch.float32)
        want = O.full_step_batched(states, 0, x["q"][t], x["k"][t], x["v"][t], x["gate"][t])
        st.advance()
        for s in states:
            s.tokens_seen += 1
        assert_act_close(out, want, f"step {t}")


@pytest.mark.gpu
def test_kv_append_slot_mapping_bit_exact(gpu):
    """Every appended token lands at page_table[row][t // 16] * 16 + t % 16 of its layer pool."""
    announce("kv_append: slot mapping, B=4, shuffled pages")
    batch, steps = 4, 40
    lengths = [0, 5, 16, 31]
    st = _attn_state(gpu, batch, 128, shuffle_seed=11)
    st.set_positions(lengths)
    st.reserve(steps)
    x = W.attn_step_inputs(23, steps, batch)
    for t in range(steps):
        K.kv_append(x["k"][t].to(gpu), x["v"][t].to(gpu), st.kv.k[0], st.kv.v[0], st.kv.page_table,
                    positions=st.tokens_seen, slots=st.tokens_seen, inv_freq=st.inv_freq)
        st.advance()
    torch.cuda.synchronize()
    vc = st.kv.v[0].cpu()
    for b, n0 in enumerate(lengths):
        for t in range(steps):
            tok = n0 + t
            slot = st.kv.alloc.slot_of(b, tok)
            page, off = divmod(slot, 16)
            assert page == st.kv.alloc.tables[b][tok // 16]
            assert torch.equal(vc[page, :, :, off], x["v"][t][b]), (b, tok)
            _, k_rot = O.apply_rope(x["k"][t][b:b + 1].float(), x["k"][t][b:b + 1].float(), tok)
            k_row = torch.stack([st.kv.key_row(0, page, h, off).cpu() for h in range(2)])
            torch.testing.assert_close(k_row.float(), k_rot[0].to(torch.bfloat16).float(), rtol=8e-3, atol=1e-5)
