"""GPU parity: sequence snapshots (ria_seq_state_save / ria_seq_state_restore).

A row's DeltaNet states, conv ring and KV pages saved into a payload and
restored into another row of another pool (other page order, other batch
size) must decode on bit for bit like the original row.  The payload's
reference-layout view (``to_reference``) must be the state the reference's
AttentionState would hold (qwen36_attention_cache.py:27-92): checked by
continuing the decode with the oracle from it.  A state built from the
reference's tensors (``from_reference``) must decode as the oracle does from
the same tensors.
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
from router_ia.snapshot import SequenceSnapshot

pytestmark = pytest.mark.gpu

N_LIN, N_FULL = 3, 1  # model layers 0, 1, 2 (DeltaNet) and 3 (full attention)


def _engine(dev, rows, shuffle, lengths, seed):
    st = BatchedAttentionState(rows, 1100, num_linear_layers=N_LIN, num_full_layers=N_FULL, device=dev,
                               page_shuffle_seed=shuffle, split_tokens=64)
    st.set_positions(lengths)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    st.linear_states.normal_(0.0, 0.02, generator=g)
    st.conv_rings.normal_(0.0, 1.0, generator=g)
    st.kv.k.normal_(0.0, 1.0, generator=g)  # every slot, also past each row's tokens
    st.kv.v.normal_(0.0, 1.0, generator=g)
    return st


def _params(seed):
    return [W.gdn_layer_params(seed + i) for i in range(N_LIN)]


def _step(st, params, gdn_x, attn_x, rows_map=None):
    """One decode step through the 4 layers; returns the per-layer outputs (fp32)."""
    dev = st.device
    outs = []
    for li in range(N_LIN):
        p = params[li]
        outs.append(st.linear_step(li, gdn_x["mixed"][li].to(dev), p["conv_weight"].to(dev),
                                   gdn_x["a_raw"][li].to(dev), gdn_x["b_raw"][li].to(dev),
                                   gate_mode=nat.RIA_GATE_RAW, A_log=p["A_log"].to(dev),
                                   dt_bias=p["dt_bias"].to(dev), out_dtype=torch.float32).cpu())
    outs.append(st.full_step(0, attn_x["q"][0].to(dev), attn_x["k"][0].to(dev), attn_x["v"][0].to(dev),
                             attn_x["gate"][0].to(dev), out_dtype=torch.float32).cpu())
    st.advance()
    return outs


def _inputs(seed, rows):
    gdn = W.gdn_step_inputs(seed, N_LIN, rows)          # indexed by layer instead of step
    attn = W.attn_step_inputs(seed + 1, 1, rows)
    return gdn, attn


def _row_inputs(gdn, attn, src_row, rows, dst_row):
    """Inputs for a `rows`-row engine whose row dst_row gets row src_row of the given inputs."""
    def pick(t):
        out = torch.zeros((t.shape[0], rows, *t.shape[2:]), dtype=t.dtype)
        out[:, dst_row] = t[:, src_row]
        return out
    return {k: pick(v) for k, v in gdn.items()}, {k: pick(v) for k, v in attn.items()}


def test_snapshot_restores_into_another_pool_bit_exact(gpu):
    announce("snapshot: rows [37, 200, 515] -> save row 1 -> restore into row 0 of a 2-row pool; 3 steps")
    params = _params(90)
    a = _engine(gpu, 3, 1, [37, 200, 515], 91)
    for s in range(2):
        _step(a, params, *_inputs(92 + s, 3))
    snap = a.save_row(1)
    assert snap.tokens == 202
    b = _engine(gpu, 2, 7, [5, 60], 93)
    b.restore_row(0, snap)
    for s in range(3):
        gdn, attn = _inputs(100 + s, 3)
        oa = _step(a, params, gdn, attn)
        ob = _step(b, params, *_row_inputs(gdn, attn, 1, 2, 0))
        for layer, (x, y) in enumerate(zip(oa, ob)):
            assert torch.equal(x[1], y[0]), f"step {s} layer {layer}"
    torch.cuda.synchronize()
    assert torch.equal(a.linear_states[:, 1].cpu(), b.linear_states[:, 0].cpu())
    assert torch.equal(a.conv_rings[:, 1].cpu(), b.conv_rings[:, 0].cpu())
    ka, va = a.gather_kv(0, 0, 205)
    kb, vb = b.gather_kv(0, 0, 205)
    assert torch.equal(ka[1].cpu(), kb[0].cpu()) and torch.equal(va[1].cpu(), vb[0].cpu())


def test_snapshot_bytes_are_deterministic_with_zero_tail(gpu):
    announce("snapshot: save twice, tail slots of the last page are zero although the cache holds noise")
    a = _engine(gpu, 2, 3, [37, 100], 94)
    s1 = a.save_row(0)
    s2 = a.save_row(0)
    torch.cuda.synchronize()
    assert torch.equal(s1.payload.cpu(), s2.payload.cpu())
    kt, vt = s1._tiles("k"), s1._tiles("v")
    assert not kt[:, -1, :, :, :, 37 % 16:, :].any() and not vt[:, -1, :, :, 37 % 16:].any()
    assert kt[:, -1, :, :, :, : 37 % 16, :].any()
    # the sections agree with the pools they were copied from
    assert torch.equal(s1.linear_states().cpu(), a.linear_states[:, 0].cpu())
    assert torch.equal(s1.conv_rings().cpu(), a.conv_rings[:, 0].cpu())
    k, v = a.gather_kv(0, 0, 37)
    assert torch.equal(s1.keys()[0].cpu(), k[0].cpu()) and torch.equal(s1.values()[0].cpu(), v[0].cpu())


def _oracle_steps(ref, params, steps_inputs, row):
    """Continue the reference state `ref` (one sequence) with the oracle; per-step layer outputs."""
    conv = {m: ref["linear_conv_states"][m].cpu() for m in (0, 1, 2)}
    lin = {m: ref["linear_states"][m].cpu() for m in (0, 1, 2)}
    fk = ref["full_keys"][3].cpu().float()
    fv = ref["full_values"][3].cpu().float()
    pos = ref["tokens_seen"]
    outs = []
    for gdn, attn in steps_inputs:
        step = []
        for li, m in enumerate((0, 1, 2)):
            p = params[li]
            beta, g = O.gating(gdn["a_raw"][li][row:row + 1], gdn["b_raw"][li][row:row + 1], p["A_log"],
                               p["dt_bias"])
            o, conv[m], lin[m] = O.linear_decode_step(conv[m], lin[m], gdn["mixed"][li][row:row + 1],
                                                      p["conv_weight"], beta, g)
            step.append(o)
        o, fk, fv = O.full_decode_step(fk, fv, attn["q"][0][row:row + 1], attn["k"][0][row:row + 1],
                                       attn["v"][0][row:row + 1], attn["gate"][0][row:row + 1], pos)
        step.append(o)
        pos += 1
        outs.append(step)
    return outs, lin


def test_reference_layout_export_continues_like_the_oracle(gpu):
    announce("snapshot.to_reference: oracle continues row 2 (515 tokens) for 2 steps")
    params = _params(95)
    a = _engine(gpu, 3, 2, [37, 200, 515], 96)
    snap = a.save_row(2)
    ref = snap.to_reference()
    assert torch.equal(ref["linear_states"][1].cpu(), a.linear_states[1, 2:3].cpu())
    inputs = [_inputs(97 + s, 3) for s in range(2)]
    got = [_step(a, params, *x) for x in inputs]
    want, lin = _oracle_steps(ref, params, inputs, 2)
    for s in range(2):
        for layer in range(4):
            assert_act_close(got[s][layer][2:3], want[s][layer], f"step {s} layer {layer}")
    for li, m in enumerate((0, 1, 2)):
        assert_state_close(a.linear_states[li, 2:3].cpu(), lin[m], f"state layer {m}")


def test_reference_layout_import_decodes_like_the_oracle(gpu):
    announce("SequenceSnapshot.from_reference: 45-token reference state restored into row 1, 2 steps")
    g = torch.Generator().manual_seed(98)
    tokens = 45
    ref = {
        "linear_states": {m: torch.randn((1, 32, 128, 128), generator=g) * 0.02 for m in (0, 1, 2)},
        "linear_conv_states": {m: torch.randn((1, 8192, 4), generator=g).to(torch.bfloat16) for m in (0, 1, 2)},
        "full_keys": {3: torch.randn((1, 2, tokens, 256), generator=g).to(torch.bfloat16)},
        "full_values": {3: torch.randn((1, 2, tokens, 256), generator=g).to(torch.bfloat16)},
        "tokens_seen": tokens,
    }
    snap = SequenceSnapshot.from_reference(ref, num_linear_layers=N_LIN, num_full_layers=N_FULL, device=gpu)
    params = _params(99)
    a = _engine(gpu, 2, 4, [10, 300], 100)
    a.restore_row(1, snap)
    inputs = [_inputs(101 + s, 2) for s in range(2)]
    got = [_step(a, params, *x) for x in inputs]
    want, _ = _oracle_steps(ref, params, inputs, 1)
    for s in range(2):
        for layer in range(4):
            assert_act_close(got[s][layer][1:2], want[s][layer], f"step {s} layer {layer}")
