"""GPU parity: the batched token forward loop (router_ia.batched_forward).

B sequences at different positions go through a 4-layer stack (model layers
0-2 Gated DeltaNet, 3 full attention) with FP8 projections, one token each per
step.  Each row must follow the oracle's restatement of the reference's
per-sequence composites (qwen36_attention_cache.py:224-324 with the CUDA-path
dtypes and the fp16 dequantised weights), started from the same state: the
engine's rows exported with ``SequenceSnapshot.to_reference()``.  The MoE
callable runs between layers where the reference runs its MoE block.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_residual_close, assert_state_close
from oracle import qwen36_cpu as O
from router_ia import batched_forward as BF
from router_ia import workloads as W
from router_ia.batched_state import BatchedAttentionState

pytestmark = pytest.mark.gpu

LAYERS = 4  # model layers 0, 1, 2 (DeltaNet) and 3 (full attention)
LENGTHS = [37, 200, 515]
# 20 rows: more than the 16 of the one-pass projection kernel, so the
# projections take the K-split FP8 kernels on the fp16 copy of the normed input
# (or, with projections="fp16", the library fp16 GEMM over the dequantised
# weights)
LENGTHS_20 = LENGTHS + [1, 2, 15, 16, 17, 31, 64, 99, 128, 250, 300, 333, 401, 480, 512, 550, 600]


def _setup(dev, split_tokens=64, lengths=LENGTHS, projections="fp8"):
    ckpts = [W.synthetic_layer(700 + m, m) for m in range(LAYERS)]
    st = BatchedAttentionState(len(lengths), 1100, num_linear_layers=3, num_full_layers=1, device=dev,
                               page_shuffle_seed=5, split_tokens=split_tokens)
    st.set_positions(lengths)
    g = torch.Generator(device=dev)
    g.manual_seed(71)
    st.linear_states.normal_(0.0, 0.02, generator=g)
    st.conv_rings.normal_(0.0, 1.0, generator=g)
    st.kv.k.normal_(0.0, 1.0, generator=g)
    st.kv.v.normal_(0.0, 1.0, generator=g)
    fwd = BF.BatchedForward(st, [BF.layer_weights(ck, m, dev) for m, ck in enumerate(ckpts)],
                            projections=projections)
    return ckpts, st, fwd


def _oracle_weights(ck):
    """The reference's fp16 weights: each FP8 projection dequantised (then cast to fp16 by the oracle)."""
    out = {}
    for key, t in ck.items():
        if key.endswith(".weight_scale_inv"):
            continue
        scale = ck.get(key + "_scale_inv")
        out[key] = O.dequantize_fp8_blockwise(t, scale) if scale is not None else t
    return out


def _oracle_states(st):
    states = []
    for row in range(st.max_seqs):
        ref = st.save_row(row).to_reference()
        s = O.SequenceState()
        s.conv = {m: t.cpu() for m, t in ref["linear_conv_states"].items()}
        s.linear = {m: t.cpu() for m, t in ref["linear_states"].items()}
        s.keys = {m: t.cpu().float() for m, t in ref["full_keys"].items()}
        s.values = {m: t.cpu().float() for m, t in ref["full_values"].items()}
        s.tokens_seen = ref["tokens_seen"]
        states.append(s)
    return states


def _oracle_layer(w, s, m, x):
    step = O.full_layer_step if m % 4 == 3 else O.linear_layer_step
    return step(w, s, m, x, gpu_dtypes=True)


@pytest.mark.parametrize("lengths,projections", [(LENGTHS, "fp8"), (LENGTHS_20, "fp16"), (LENGTHS_20, "fp8")],
                         ids=["3rows", "20rows-gemm16", "20rows-fp8"])
def test_batched_forward_matches_the_reference_composites(gpu, lengths, projections):
    announce(f"batched forward: {LAYERS} layers, rows at {lengths}, 2 steps, projections {projections}")
    ckpts, st, fwd = _setup(gpu, lengths=lengths, projections=projections)
    ws = [_oracle_weights(ck) for ck in ckpts]
    ref = _oracle_states(st)
    for step in range(2):
        x0 = torch.randn((len(lengths), 2048), generator=torch.Generator().manual_seed(80 + step))
        x = x0.to(gpu).contiguous()
        want = [x0[row:row + 1] for row in range(len(lengths))]
        for m in range(LAYERS):  # layer by layer, so a mismatch names its layer
            fwd.layer(m, x)
            got = x.cpu()
            for row, s in enumerate(ref):
                want[row] = _oracle_layer(ws[m], s, m, want[row])
                assert_residual_close(got[row:row + 1], want[row], m + 1, f"step {step} layer {m} row {row}")
        st.advance()
        for s in ref:
            s.tokens_seen += 1
    # The states take k, v and the gates from fp16 projections whose two
    # implementations may round an element one fp16 ulp apart (different fp32
    # accumulation orders), so even layer 0, which sees the same input on both
    # sides, is held to 5e-3 (an ulp of a unit-size v moves the state by about
    # 1e-3 of its largest entry); later layers take the previous layer's output,
    # equal to the activation tolerance, and are held to that.
    for i, m in enumerate((0, 1, 2)):
        for row, s in enumerate(ref):
            assert_state_close(st.linear_states[i, row].cpu(), s.linear[m][0], f"state layer {m} row {row}",
                               rel=5e-3 if m == 0 else 2e-2)


def test_capture_refuses_a_fixed_split(gpu):
    _, st, fwd = _setup(gpu)
    fwd.step(torch.zeros((len(LENGTHS), 2048), device=gpu))
    with pytest.raises(RuntimeError, match="balanced"):
        fwd.capture(2)


def test_step_runs_every_layer_and_the_mlp_between(gpu):
    announce("batched forward: step() == layer() loop + advance, mlp called per layer")
    _, st, fwd = _setup(gpu)
    x0 = torch.randn((len(LENGTHS), 2048), generator=torch.Generator().manual_seed(90)).to(gpu)
    snaps = [st.save_row(r) for r in range(len(LENGTHS))]
    calls = []

    def mlp(m, x):
        calls.append(m)
        return x.mul_(0.5)

    got = fwd.step(x0.clone(), mlp=mlp)
    assert calls == list(range(LAYERS))
    assert st.max_seen == max(LENGTHS) + 1
    # the same by hand from the same state
    for r, snap in enumerate(snaps):
        st.restore_row(r, snap)
    x = x0.clone()
    for m in range(LAYERS):
        fwd.layer(m, x)
        x.mul_(0.5)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), x.cpu())


@pytest.mark.parametrize("lengths", [LENGTHS, LENGTHS_20], ids=["3rows", "20rows"])
def test_graph_replays_equal_eager_steps(gpu, lengths):
    announce(f"batched forward: captured step replayed 3 times == 3 eager steps (bit for bit), {len(lengths)} rows")
    _, st, fwd = _setup(gpu, split_tokens=0, lengths=lengths)  # the balanced attention schedule, which a graph can replay
    xs = torch.randn((4, len(lengths), 2048), generator=torch.Generator().manual_seed(91)).to(gpu)
    fwd.step(xs[0].clone())  # one eager step loads every kernel
    snaps = [st.save_row(r) for r in range(len(lengths))]
    graph = fwd.capture(3)
    replayed = []
    for s in range(1, 4):
        graph.x.copy_(xs[s])
        replayed.append(graph.replay().clone())
        torch.cuda.synchronize()  # eager work and a sync between replays
        assert st.max_seen == max(lengths) + 1 + s
    with pytest.raises(RuntimeError, match="used up"):
        graph.replay()
    for r, snap in enumerate(snaps):
        st.restore_row(r, snap)
    for s in range(1, 4):
        got = fwd.step(xs[s].clone())
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), replayed[s - 1].cpu()), f"replay {s}"


def test_graph_replay_with_an_mlp_that_returns_a_new_tensor(gpu):
    announce("batched forward: captured step with a non-in-place mlp (x * 0.5) == eager steps, bit for bit")
    _, st, fwd = _setup(gpu, split_tokens=0)

    def mlp(m, x):
        return x * 0.5  # a new tensor every layer: the step's output is not its input buffer

    xs = torch.randn((4, len(LENGTHS), 2048), generator=torch.Generator().manual_seed(92)).to(gpu)
    fwd.step(xs[0].clone(), mlp=mlp)
    snaps = [st.save_row(r) for r in range(len(LENGTHS))]
    graph = fwd.capture(3, mlp=mlp)
    assert graph.out.data_ptr() != graph.x.data_ptr()
    replayed = []
    for s in range(1, 4):
        graph.x.copy_(xs[s])
        junk = torch.randn_like(xs[s])  # allocations between replays must not land on the graph's buffers
        replayed.append(graph.replay().clone())
        torch.cuda.synchronize()
        del junk
    for r, snap in enumerate(snaps):
        st.restore_row(r, snap)
    for s in range(1, 4):
        got = fwd.step(xs[s].clone(), mlp=mlp)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), replayed[s - 1].cpu()), f"replay {s}"
