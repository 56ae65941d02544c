#!/usr/bin/env python3
"""Decode throughput of the 40-layer hybrid attention stack on one MI355X.

Workload (default ``ragged128``): 128 concurrent sequences, context lengths
uniform in [1024, 32768] (seed 4), 30 Gated DeltaNet layers + 10 GQA
full-attention layers (layer 4i+3 is full attention), 16-token KV pages with a
shuffled page table.  Every sequence starts with resident state: DeltaNet
states ~N(0, 0.02) fp32, conv rings ~N(0, 1) bf16, KV ~N(0, 1) bf16.  Each
decode step gives every layer fresh synthetic inputs (projections excluded):
DeltaNet q|k|v + gate logits, attention q, k, v and gate logits, all
pre-generated in HBM before timing.

One step = one token for every sequence through all 40 layers (append, conv,
recurrence, attention, gate) followed by the position advance.  Output: one
JSON line with tok/s, the roofline of the dominant kernel (split-K attention)
from HIP events around each of its launches, the step-level HBM fraction, and
the reference CPU path (the oracle's torch-CPU restatement) timed on a
bounded sample of the same workload on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "router-ia_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

METRIC = "attn-stack decode tok/s (40 layers, B=1..128); state+KV HBM GB/s % of peak"
HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, AMD specification
LAYERS = 40
NUM_V_HEADS = 32
NUM_Q_HEADS = 16
NUM_KV_HEADS = 2
HEAD_DIM_ATTN = 256
CONV_DIM = 8192

# Algorithmic bytes (state + KV + activations), per (sequence, layer, token).
GDN_BYTES_PER_SEQ = 2 * 2_097_152 + 49_152 + 16_384 + 16_384 + 256 + 8_192  # 4,284,672
GDN_BYTES_PER_LAYER = 65_536  # conv weight, shared by the batch
GDN_NORM_BYTES_PER_SEQ = NUM_V_HEADS * 128 * 2  # the gated norm's z gate, bf16: 8,192
ATTN_KV_BYTES_PER_TOKEN = 2 * NUM_KV_HEADS * HEAD_DIM_ATTN * 2  # 2048 B of K+V per context token
ATTN_APPEND_BYTES = 2_048
ATTN_ACT_BYTES = 3 * NUM_Q_HEADS * HEAD_DIM_ATTN * 2  # q, gate, out in bf16: 24,576
SPLITK_Q_BYTES = NUM_Q_HEADS * HEAD_DIM_ATTN * 2  # the split-K launch reads q

MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, AMD specification
PREFILL_METRIC = "prefill tok/s (1 Gated DeltaNet + 1 full-attention layer, one 16384-token prompt); MFMA TFLOP/s % of peak"
GDN_CHUNK_FLOP = 11_710_000  # chunked WY form, per (V head, 64-token chunk): KK^T, QK^T, T, U, W, scan
PREFILL_LEN = 16384


def attn_prefill_flop(length: int) -> int:
    """Causal GQA attention FLOPs: QK^T and PV over keys 0..t for every query t, 16 heads x 256 dims."""
    return NUM_Q_HEADS * length * (length + 1) // 2 * HEAD_DIM_ATTN * 4


WORKLOADS = {
    "prefill16k": dict(batch=1, lo=PREFILL_LEN, hi=PREFILL_LEN, seed=3, prefill=True,
                       desc="prefill of one 16384-token prompt through 1 Gated DeltaNet layer (chunk 64) and "
                            "1 GQA full-attention layer (causal, fills 16-token KV pages, shuffled page table)"),
    "prefill16k-norms": dict(batch=1, lo=PREFILL_LEN, hi=PREFILL_LEN, seed=3, prefill=True, norms=True,
                             desc="prefill16k with q_norm/k_norm fused into the append and attention launches and "
                                  "the gated RMSNorm applied to the DeltaNet read-out"),
    "ragged128": dict(batch=128, lo=1024, hi=32768, seed=4,
                      desc="40-layer stack, B=128, context U[1024,32768] (seed 4), 16-token pages, shuffled page table"),
    "ragged128-norms": dict(batch=128, lo=1024, hi=32768, seed=4, norms=True,
                            desc="40-layer stack as ragged128, with q_norm/k_norm fused into the append and attention "
                                 "launches and the gated RMSNorm fused into the DeltaNet read-out"),
    "snapshot128": dict(batch=128, lo=1024, hi=32768, seed=4, snapshot=True,
                        desc="save + restore of every sequence of the ragged128 stack (40 layers, B=128, "
                             "context U[1024,32768]): DeltaNet states, conv rings and KV pages to one payload "
                             "per sequence and back"),
    "proj128": dict(batch=128, seed=5, proj=True,
                    desc="every projection of the 40-layer stack for one decode step of B=128 tokens, FP8 "
                         "block-scaled weights (DeltaNet in_proj_qkv/z/a/b + out_proj, attention q/k/v/o_proj), "
                         "fp16 outputs"),
    "forward128": dict(batch=128, lo=1024, hi=32768, seed=4, forward=True,
                       desc="attention side of the 40-layer stack for one decode step of B=128 sequences (context "
                            "U[1024,32768], seed 4): input RMSNorm, FP8 block-scaled projections, conv + DeltaNet + "
                            "gated RMSNorm / q,k norms + RoPE + paged GQA attention + gate, output projection and "
                            "residual add per layer (router_ia.batched_forward; the MoE block is the caller's)"),
    "forward1": dict(batch=1, lo=16384, hi=16384, seed=4, forward=True, graph=True,
                     desc="the forward128 loop for one sequence at context 16384 (the reference's batch-1 decode), "
                          "each step replayed as one captured HIP graph"),
    "forward1-eager": dict(batch=1, lo=16384, hi=16384, seed=4, forward=True,
                           desc="forward1 with every launch issued from Python (no graph)"),
    "proj1": dict(batch=1, seed=5, proj=True,
                  desc="every projection of the 40-layer stack for one decode step of B=1 token, FP8 block-scaled "
                       "weights, fp16 outputs"),
    "batch32": dict(batch=32, lo=8192, hi=8192, seed=2, graph=True,
                    desc="40-layer stack, B=32, context 8192 (seed 2), 16-token pages, shuffled page table; each "
                         "step replayed as one captured HIP graph"),
    "batch8": dict(batch=8, lo=8192, hi=8192, seed=2, graph=True,
                   desc="40-layer stack, B=8, context 8192 (seed 2), 16-token pages, shuffled page table; each "
                        "step replayed as one captured HIP graph"),
    "batch64": dict(batch=64, lo=8192, hi=8192, seed=2, graph=True,
                    desc="40-layer stack, B=64, context 8192 (seed 2), 16-token pages, shuffled page table; each "
                         "step replayed as one captured HIP graph"),
    "batch128": dict(batch=128, lo=8192, hi=8192, seed=2, graph=True,
                     desc="40-layer stack, B=128, context 8192 (seed 2), 16-token pages, shuffled page table; each "
                          "step replayed as one captured HIP graph"),
    "batch1": dict(batch=1, lo=8192, hi=8192, seed=2, graph=True,
                   desc="40-layer stack, B=1, context 8192 (seed 2), 16-token pages, shuffled page table; each "
                        "step (fresh inputs copied in, 40 layers, advance) replayed as one captured HIP graph"),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hipEventDisableSystemFence (hip_runtime_api.h)


class KernelTimer:
    """Per-launch kernel timing with HIP events recorded on the launch stream.

    The events are created with hipEventDisableSystemFence: a default event
    record ends with a system-scope fence (cache write-back and invalidation)
    that the next launch pays for, which adds tens of microseconds to a
    timed 0.7 ms attention launch on MI355X; these events time the launch
    without perturbing it.  They come from the HIP runtime the process
    already uses (torch's), through ctypes.
    """

    def __init__(self, pairs: int):
        import ctypes

        self._ct = ctypes
        self._hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
        self._hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self._hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self._hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self._hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self._events = []
        for _ in range(2 * pairs):
            ev = ctypes.c_void_p()
            rc = self._hip.hipEventCreateWithFlags(ctypes.byref(ev), HIP_EVENT_DISABLE_SYSTEM_FENCE)
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            self._events.append(ev)
        self._next = 0
        self.pairs: list[tuple[ctypes.c_void_p, ctypes.c_void_p]] = []

    def start(self) -> None:
        self._record()

    def stop(self) -> None:
        self._record()
        self.pairs.append((self._events[self._next - 2], self._events[self._next - 1]))

    def _record(self) -> None:
        if self._next >= len(self._events):
            raise RuntimeError("KernelTimer: more launches timed than events created")
        stream = torch.cuda.current_stream().cuda_stream
        rc = self._hip.hipEventRecord(self._events[self._next], self._ct.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")
        self._next += 1

    def elapsed_ms(self) -> list[float]:
        """Duration of every timed launch (call after the stream has synchronised)."""
        out = []
        for e0, e1 in self.pairs:
            ms = self._ct.c_float()
            rc = self._hip.hipEventElapsedTime(self._ct.byref(ms), e0, e1)
            if rc != 0:
                raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
            out.append(ms.value)
        return out

    def close(self) -> None:
        for ev in self._events:
            self._hip.hipEventDestroy(ev)
        self._events = []


def is_full(layer: int) -> bool:
    return layer % 4 == 3


STACK_KINDS = ["full" if is_full(layer) else "linear" for layer in range(LAYERS)]


def step_bytes(ctx: list[int], norms: bool = False, kinds: list[str] | None = None) -> int:
    """Algorithmic bytes of one decode step; ctx[b] = context incl. the new token."""
    kinds = STACK_KINDS if kinds is None else kinds
    n_lin = sum(1 for k in kinds if k == "linear")
    n_full = len(kinds) - n_lin
    b = len(ctx)
    per_seq = GDN_BYTES_PER_SEQ + (GDN_NORM_BYTES_PER_SEQ if norms else 0)
    lin = n_lin * (b * per_seq + GDN_BYTES_PER_LAYER)
    full = n_full * sum(ATTN_KV_BYTES_PER_TOKEN * t + ATTN_APPEND_BYTES + ATTN_ACT_BYTES for t in ctx)
    return lin + full


TRAFFIC_PROFILE = ROOT / "profiles" / "decode_stack_ragged128_hbm_traffic.md"


def profiled_traffic(kernel: str) -> dict | None:
    """HBM bytes per launch of `kernel` from the committed FETCH_SIZE/WRITE_SIZE profile."""
    if not TRAFFIC_PROFILE.is_file():
        return None
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 6 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
            return {"bytes": int(parts[3]), "algorithmic": int(parts[5]), "source": TRAFFIC_PROFILE.name}
    return None


def run_gpu(args, wl) -> dict:
    from router_ia import _native as nat
    from router_ia import kernels as K
    from router_ia import workloads as W
    from router_ia.batched_state import BatchedAttentionState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batch = wl["batch"]
    lengths = W.ragged_lengths(wl["seed"], batch, wl["lo"], wl["hi"])
    total_new = args.warmup + args.steps
    max_context = max(lengths) + total_new + 16
    num_pages = sum((n + total_new + 15) // 16 for n in lengths) + batch
    log(f"[bench] {wl['desc']}: B={batch}, mean context {sum(lengths) / batch:.0f}, max {max(lengths)}, "
        f"{num_pages} pages/layer")
    st = BatchedAttentionState(batch, max_context, num_pages=num_pages, device=dev, page_shuffle_seed=wl["seed"])
    st.set_positions(lengths)
    st.reserve(total_new)

    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    # Resident state.
    for li in range(st.num_linear_layers):
        st.linear_states[li].normal_(0.0, 0.02, generator=gen)
        st.conv_rings[li].normal_(0.0, 1.0, generator=gen)
    for fi in range(st.num_full_layers):
        st.kv.k[fi].normal_(0.0, 1.0, generator=gen)
        st.kv.v[fi].normal_(0.0, 1.0, generator=gen)
    # Per-layer constants.
    conv_w = [(torch.randn((CONV_DIM, 1, 4), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
              for _ in range(st.num_linear_layers)]
    a_log = [torch.rand((NUM_V_HEADS,), generator=gen, device=dev) * 4.0 - 4.0 for _ in range(st.num_linear_layers)]
    dt_bias = [torch.zeros((NUM_V_HEADS,), device=dev) for _ in range(st.num_linear_layers)]
    # Per-step inputs for every layer, resident before timing.
    n_lin, n_full = st.num_linear_layers, st.num_full_layers
    mixed = torch.randn((total_new, n_lin, batch, CONV_DIM), generator=gen, device=dev, dtype=torch.bfloat16)
    gate_ab = torch.randn((total_new, n_lin, 2, batch, NUM_V_HEADS), generator=gen, device=dev)
    qg = torch.randn((total_new, n_full, 2, batch, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev,
                     dtype=torch.bfloat16)
    kv_in = torch.randn((total_new, n_full, 2, batch, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev,
                        dtype=torch.bfloat16)
    norms = bool(wl.get("norms"))
    if norms:
        # gated-norm gates z per (step, layer) and fp32 norm weights per layer
        z_in = torch.randn((total_new, n_lin, batch, NUM_V_HEADS, 128), generator=gen, device=dev,
                           dtype=torch.bfloat16)
        gnw = [1.0 + 0.1 * torch.randn((128,), generator=gen, device=dev) for _ in range(n_lin)]
        qnw = [0.1 * torch.randn((HEAD_DIM_ATTN,), generator=gen, device=dev) for _ in range(n_full)]
        knw = [0.1 * torch.randn((HEAD_DIM_ATTN,), generator=gen, device=dev) for _ in range(n_full)]
    gdn_out = torch.empty((batch, NUM_V_HEADS, 128), device=dev, dtype=torch.bfloat16)
    attn_out = torch.empty((batch, NUM_Q_HEADS, HEAD_DIM_ATTN), device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    log(f"[bench] resident: {torch.cuda.memory_allocated(dev) / 2**30:.1f} GiB allocated")

    n_full_layers = sum(1 for layer in range(LAYERS) if is_full(layer))
    attn_timer = KernelTimer(n_full_layers * args.steps)
    gdn_timer = KernelTimer((LAYERS - n_full_layers) * args.steps)
    attn_bytes: list[int] = []

    def one_step(s: int, timed: bool) -> None:
        max_ctx = st.max_seen + 1
        ctx_bytes = None
        for layer in range(LAYERS):
            if is_full(layer):
                fi = layer // 4
                kc, vc = st.kv.layer(fi)
                kw = dict(positions=st.tokens_seen, ctx_lens=st.ctx_lens, max_ctx=max_ctx, inv_freq=st.inv_freq,
                          scale=st.scale, workspace=st.workspace, q_norm_weight=qnw[fi] if norms else None)
                if timed:
                    attn_timer.start()
                # split-K over each row's resident tokens; the combine launch appends the new token
                # (k_norm, RoPE, into the page) and folds it into the row's softmax
                app = dict(k_norm_weight=knw[fi] if norms else None)
                K.attn_decode_append(qg[s, fi, 0], qg[s, fi, 1], kv_in[s, fi, 0], kv_in[s, fi, 1], kc, vc,
                                     st.kv.page_table, attn_out, phase=nat.RIA_ATTN_SPLITK, **app, **kw)
                if timed:
                    attn_timer.stop()
                    if ctx_bytes is None:
                        ctx_bytes = sum(ATTN_KV_BYTES_PER_TOKEN * n + SPLITK_Q_BYTES for n in st._host_seen)
                    attn_bytes.append(ctx_bytes)
                K.attn_decode_append(qg[s, fi, 0], qg[s, fi, 1], kv_in[s, fi, 0], kv_in[s, fi, 1], kc, vc,
                                     st.kv.page_table, attn_out, phase=nat.RIA_ATTN_COMBINE, **app, **kw)
            else:
                li = layer - layer // 4
                if timed:
                    gdn_timer.start()
                K.gdn_decode(mixed[s, li], st.linear_states[li], gate_ab[s, li, 0], gate_ab[s, li, 1], gdn_out,
                             num_k_heads=st.num_k_heads, num_v_heads=st.num_v_heads, conv_weight=conv_w[li],
                             conv_ring=st.conv_rings[li], conv_pos=st.tokens_seen, gate_mode=nat.RIA_GATE_RAW,
                             A_log=a_log[li], dt_bias=dt_bias[li], z=z_in[s, li] if norms else None,
                             norm_weight=gnw[li] if norms else None)
                if timed:
                    gdn_timer.stop()
        st.advance()

    for s in range(args.warmup):
        one_step(s, False)
    torch.cuda.synchronize()
    ctx_at_start = [n + 1 for n in st._host_seen]
    algo_bytes = sum(step_bytes([c + i for c in ctx_at_start], norms) for i in range(args.steps))
    log(f"[bench] warmup {args.warmup} steps done; timing {args.steps} steps")
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record()
    for s in range(args.warmup, args.warmup + args.steps):
        one_step(s, True)
        if (s - args.warmup) % 64 == 63:
            log(f"[bench] step {s - args.warmup + 1}/{args.steps} issued")
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    elapsed_s = t_start.elapsed_time(t_end) / 1e3
    attn_ms = attn_timer.elapsed_ms()
    gdn_ms = gdn_timer.elapsed_ms()
    attn_timer.close()
    gdn_timer.close()
    attn_avg_s = sum(attn_ms) / len(attn_ms) / 1e3
    attn_bytes_avg = sum(attn_bytes) / len(attn_bytes)
    gdn_avg_s = sum(gdn_ms) / len(gdn_ms) / 1e3
    gdn_bytes = batch * (GDN_BYTES_PER_SEQ + (GDN_NORM_BYTES_PER_SEQ if norms else 0)) + GDN_BYTES_PER_LAYER
    achieved = attn_bytes_avg / attn_avg_s / 1e9
    step_gbps = algo_bytes / elapsed_s / 1e9
    return {
        "batch": batch,
        "lengths": lengths,
        "elapsed_s": elapsed_s,
        "wall_s": wall,
        "tok_s": batch * args.steps / elapsed_s,
        "ms_per_step": elapsed_s / args.steps * 1e3,
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_splitk_kernel (ria_attn_decode_append split-K phase, over the resident tokens)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "traffic_note": None,
            "algorithmic_bytes_per_launch": round(attn_bytes_avg),
            "avg_launch_us": round(attn_avg_s * 1e6, 2),
            "launches": len(attn_ms),
            "timing": "HIP events around each launch on its stream, created with hipEventDisableSystemFence",
        },
        "kernels": {
            "gdn_decode_kernel": {
                "avg_launch_us": round(gdn_avg_s * 1e6, 2),
                "algorithmic_bytes_per_launch": gdn_bytes,
                "achieved_GBps": round(gdn_bytes / gdn_avg_s / 1e9, 1),
                "frac": round(gdn_bytes / gdn_avg_s / 1e9 / HBM_PEAK_GBPS, 4),
                "launches": len(gdn_ms),
            },
            "attn_splitk_kernel_share_of_step": round(sum(attn_ms) / 1e3 / elapsed_s, 4),
            "gdn_decode_kernel_share_of_step": round(sum(gdn_ms) / 1e3 / elapsed_s, 4),
        },
        "step_hbm": {
            "algorithmic_bytes_per_step": round(algo_bytes / args.steps),
            "achieved_GBps": round(step_gbps, 1),
            "frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        },
    }


def run_cpu_baseline(wl, lengths: list[int], n_seqs: int, n_steps: int) -> dict:
    """The reference CPU path (oracle restatement: fp32, torch.cat KV) on a sample of the workload."""
    from oracle import qwen36_cpu as O

    torch.set_num_threads(os.cpu_count() or 1)
    sample = lengths[:n_seqs]
    gen = torch.Generator().manual_seed(wl["seed"])
    states = []
    for n in sample:
        s = O.SequenceState()
        s.tokens_seen = n
        for li in range(30):
            s.linear[li] = torch.randn((1, 32, 128, 128), generator=gen) * 0.02
            s.conv[li] = torch.randn((1, CONV_DIM, 4), generator=gen).to(torch.bfloat16)
        for fi in range(10):
            s.keys[fi] = torch.randn((1, NUM_KV_HEADS, n, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16).float()
            s.values[fi] = torch.randn((1, NUM_KV_HEADS, n, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16).float()
        states.append(s)
    conv_w = [(torch.randn((CONV_DIM, 1, 4), generator=gen) * 0.5).to(torch.bfloat16) for _ in range(30)]
    a_log = [torch.rand((32,), generator=gen) * 4.0 - 4.0 for _ in range(30)]
    b = len(sample)
    inputs = []
    for _ in range(n_steps):
        per_layer = []
        for layer in range(LAYERS):
            if is_full(layer):
                per_layer.append(tuple(torch.randn(shape, generator=gen).to(torch.bfloat16) for shape in (
                    (b, 16, 256), (b, 2, 256), (b, 2, 256), (b, 16, 256))))
            else:
                per_layer.append((torch.randn((b, CONV_DIM), generator=gen).to(torch.bfloat16),
                                  torch.randn((b, 32), generator=gen), torch.randn((b, 32), generator=gen)))
        inputs.append(per_layer)
    zero_bias = torch.zeros(32)
    t0 = time.perf_counter()
    for step in range(n_steps):
        for layer in range(LAYERS):
            x = inputs[step][layer]
            if is_full(layer):
                O.full_step_batched(states, layer // 4, x[0], x[1], x[2], x[3])
            else:
                li = layer - layer // 4
                beta, g = O.gating(x[1], x[2], a_log[li], zero_bias)
                O.linear_step_batched(states, li, x[0], conv_w[li], beta, g)
        for s in states:
            s.tokens_seen += 1
    dt = time.perf_counter() - t0
    return {
        "value": round(b * n_steps / dt, 4),
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{b} sequences (rows 0..{b - 1} of the seeded lengths: {sample}), all 40 layers, "
                   f"{n_steps} decode steps, torch-CPU restatement of the reference (fp32 state and KV, "
                   f"torch.cat KV append); {dt:.1f} s"),
    }


# Projection launches of one layer, each a list of the (N, K) projections that
# read the same x: DeltaNet in_proj_qkv, in_proj_z, in_proj_a, in_proj_b on the
# normed hidden state, then out_proj (qwen36_attention_cache.py:232-247,
# 268-276); attention q (with gate), k, v, then o (:295-301, 318-320); hidden
# 2048 (qwen36_40layer_loop.py:36-50).
GDN_PROJ = [[(8192, 2048), (4096, 2048), (32, 2048), (32, 2048)], [(2048, 4096)]]
ATTN_PROJ = [[(8192, 2048), (512, 2048), (512, 2048)], [(2048, 4096)]]


def run_proj_gpu(args, wl) -> dict:
    """All projections of one decode step (40 layers) with FP8 weights, `steps` times."""
    from router_ia import kernels as K
    from router_ia import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    b = wl["batch"]
    launches = [grp for layer in range(LAYERS) for grp in (ATTN_PROJ if is_full(layer) else GDN_PROJ)]
    shapes = [s for grp in launches for s in grp]
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])

    def weight(n, k):  # distinct weights per layer, so nothing stays in L2 between steps
        w8 = (torch.randn((n, k), generator=gen, device=dev) * 8.0).clamp(-448, 448).to(torch.float8_e4m3fn)
        s = torch.rand(((n + 127) // 128, (k + 127) // 128), generator=gen, device=dev) * 1e-3 + 1e-4
        return w8, s

    weights = [[weight(n, k) for n, k in grp] for grp in launches]
    xs = {k: torch.randn((b, k), generator=gen, device=dev).to(torch.float16) for k in (2048, 4096)}
    ys = [[torch.empty((b, n), device=dev, dtype=torch.float16) for n, _ in grp] for grp in launches]
    wbytes = sum(n * k for n, k in shapes)
    io_bytes = sum(2 * b * n for n, _ in shapes) + sum(2 * b * grp[0][1] for grp in launches)
    flop = sum(2 * b * n * k for n, k in shapes)
    log(f"[bench] {wl['desc']}: {len(shapes)} projections in {len(launches)} launches, "
        f"{wbytes / 1e9:.3f} GB of FP8 weights per step")

    def one_step():
        for grp, w, y in zip(launches, weights, ys):
            K.linear_fp8_group(xs[grp[0][1]], w, out=y)

    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    # The step is 80 short launches; replaying it as one captured HIP graph
    # keeps the host's per-call work out of the GPU timeline.
    graph = torch.cuda.CUDAGraph()
    capture = torch.cuda.Stream()
    capture.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(capture):
        with torch.cuda.graph(graph, stream=capture):
            one_step()
    torch.cuda.current_stream().wait_stream(capture)
    graph.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    elapsed = t0.elapsed_time(t1) / 1e3
    step_s = elapsed / args.steps
    achieved = (wbytes + io_bytes) / step_s / 1e9
    return {"batch": b, "elapsed_s": elapsed, "ms_per_step": step_s * 1e3, "tok_s": b / step_s,
            "weight_bytes": wbytes, "flop": flop, "achieved_GBps": achieved,
            "TFLOPs": flop / step_s / 1e12}


def run_forward_gpu(args, wl) -> dict:
    """BatchedForward.step over the 40-layer stack with synthetic FP8 weights, `steps` times."""
    from router_ia import batched_forward as BF
    from router_ia import workloads as W
    from router_ia.batched_state import BatchedAttentionState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batch = wl["batch"]
    lengths = W.ragged_lengths(wl["seed"], batch, wl["lo"], wl["hi"])
    total_new = max(args.warmup, 1) + args.steps
    max_context = max(lengths) + total_new + 16
    num_pages = sum((n + total_new + 15) // 16 for n in lengths) + batch
    st = BatchedAttentionState(batch, max_context, num_pages=num_pages, device=dev, page_shuffle_seed=wl["seed"])
    st.set_positions(lengths)
    st.reserve(total_new)
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    for li in range(st.num_linear_layers):
        st.linear_states[li].normal_(0.0, 0.02, generator=gen)
        st.conv_rings[li].normal_(0.0, 1.0, generator=gen)
    for fi in range(st.num_full_layers):
        st.kv.k[fi].normal_(0.0, 1.0, generator=gen)
        st.kv.v[fi].normal_(0.0, 1.0, generator=gen)
    layers = [BF.layer_weights(W.synthetic_layer(100 * wl["seed"] + m, m, device=dev, on_device=True), m)
              for m in range(LAYERS)]
    fwd = BF.BatchedForward(st, layers)
    xs = torch.randn((total_new, batch, BF.HIDDEN), generator=gen, device=dev)
    wbytes = sum(p.weight.numel() + 4 * p.scale_inv.numel() for w in layers for p in vars(w).values()
                 if isinstance(p, BF.Fp8Projection))
    torch.cuda.synchronize()
    log(f"[bench] {wl['desc']}: B={batch}, mean context {sum(lengths) / batch:.0f}, "
        f"{wbytes / 1e9:.3f} GB of FP8 weights, {torch.cuda.memory_allocated(dev) / 2**30:.1f} GiB allocated")
    warm = max(args.warmup, 1)  # at least one eager step: it loads every kernel before a capture
    for s in range(warm):
        fwd.step(xs[s])
    graph = fwd.capture(args.steps) if wl.get("graph") else None
    torch.cuda.synchronize()
    ctx = [n + 1 for n in st._host_seen]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for s in range(warm, total_new):
        if graph is None:
            fwd.step(xs[s])
        else:
            graph.x.copy_(xs[s])
            graph.replay()
    t1.record()
    torch.cuda.synchronize()
    elapsed = t0.elapsed_time(t1) / 1e3
    step_s = elapsed / args.steps
    # bytes of one step: the state path (states, conv rings, KV, norm inputs), the
    # projection weights, and the residual stream in and out of every layer
    nbytes = step_bytes(ctx, norms=True) + wbytes + LAYERS * batch * BF.HIDDEN * 4 * 2
    return {"batch": batch, "elapsed_s": elapsed, "ms_per_step": step_s * 1e3, "tok_s": batch / step_s,
            "weight_bytes": wbytes, "step_bytes": nbytes, "achieved_GBps": nbytes / step_s / 1e9,
            "mean_ctx": sum(lengths) / batch}


def run_stack_graph(args, wl) -> dict:
    """The 40-layer state stack (projections excluded) with each decode step replayed as one HIP graph."""
    from router_ia import _native as nat
    from router_ia import workloads as W
    from router_ia.batched_state import BatchedAttentionState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batch = wl["batch"]
    kinds = wl.get("kinds", STACK_KINDS)
    lengths = W.ragged_lengths(wl["seed"], batch, wl["lo"], wl["hi"])
    warm = max(args.warmup, 1)
    total_new = warm + args.steps
    max_context = max(lengths) + total_new + 16
    num_pages = sum((n + total_new + 15) // 16 for n in lengths) + batch
    st = BatchedAttentionState(batch, max_context, num_pages=num_pages, device=dev, page_shuffle_seed=wl["seed"],
                               num_linear_layers=kinds.count("linear"), num_full_layers=kinds.count("full"))
    st.set_positions(lengths)
    st.reserve(total_new)
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    for li in range(st.num_linear_layers):
        st.linear_states[li].normal_(0.0, 0.02, generator=gen)
        st.conv_rings[li].normal_(0.0, 1.0, generator=gen)
    for fi in range(st.num_full_layers):
        st.kv.k[fi].normal_(0.0, 1.0, generator=gen)
        st.kv.v[fi].normal_(0.0, 1.0, generator=gen)
    n_lin, n_full = st.num_linear_layers, st.num_full_layers
    conv_w = [(torch.randn((CONV_DIM, 1, 4), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
              for _ in range(n_lin)]
    a_log = [torch.rand((NUM_V_HEADS,), generator=gen, device=dev) * 4.0 - 4.0 for _ in range(n_lin)]
    dt_bias = [torch.zeros((NUM_V_HEADS,), device=dev) for _ in range(n_lin)]
    # fresh per-step inputs (pool) and the fixed buffers the graph reads
    pool = {
        "mixed": torch.randn((total_new, n_lin, batch, CONV_DIM), generator=gen, device=dev, dtype=torch.bfloat16),
        "gate_ab": torch.randn((total_new, n_lin, 2, batch, NUM_V_HEADS), generator=gen, device=dev),
        "qg": torch.randn((total_new, n_full, 2, batch, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev,
                          dtype=torch.bfloat16),
        "kv": torch.randn((total_new, n_full, 2, batch, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev,
                          dtype=torch.bfloat16),
    }
    # each step's inputs packed into one byte row, so feeding a step is one copy
    # into the staging row the graph reads (every size is a multiple of 16 bytes)
    names = [k for k in pool if pool[k].numel()]  # a one-kind stack has no inputs of the other kind
    nbytes = [pool[k][0].numel() * pool[k].element_size() for k in names]
    packed = torch.cat([pool[k].reshape(total_new, -1).view(torch.uint8) for k in names], dim=1)
    staging = torch.empty((packed.shape[1],), dtype=torch.uint8, device=dev)
    inp, off = {}, 0
    for k, n in zip(names, nbytes):
        inp[k] = staging[off:off + n].view(pool[k].dtype).view(pool[k].shape[1:])
        off += n
    del pool
    gdn_out = torch.empty((batch, NUM_V_HEADS, 128), device=dev, dtype=torch.bfloat16)
    attn_out = torch.empty((batch, NUM_Q_HEADS, HEAD_DIM_ATTN), device=dev, dtype=torch.bfloat16)

    def step():
        fi = li = 0
        for kind in kinds:
            if kind == "full":
                st.full_step(fi, inp["qg"][fi, 0], inp["kv"][fi, 0], inp["kv"][fi, 1], inp["qg"][fi, 1], out=attn_out)
                fi += 1
            else:
                st.linear_step(li, inp["mixed"][li], conv_w[li], inp["gate_ab"][li, 0], inp["gate_ab"][li, 1],
                               gate_mode=nat.RIA_GATE_RAW, A_log=a_log[li], dt_bias=dt_bias[li], out=gdn_out)
                li += 1
        st.advance()

    def feed(s):
        staging.copy_(packed[s])

    for s in range(warm):
        feed(s)
        step()
    torch.cuda.synchronize()
    # record one step; recording runs the host side of advance(), which the replays redo
    host_seen, headroom = list(st._host_seen), st._min_headroom
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            step()
    torch.cuda.current_stream().wait_stream(cs)
    st._host_seen, st._min_headroom = host_seen, headroom
    torch.cuda.synchronize()
    ctx = [n + 1 for n in st._host_seen]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for s in range(warm, total_new):
        feed(s)
        graph.replay()
    t1.record()
    torch.cuda.synchronize()
    elapsed = t0.elapsed_time(t1) / 1e3
    step_s = elapsed / args.steps
    nbytes = step_bytes(ctx, kinds=kinds)
    return {"batch": batch, "ms_per_step": step_s * 1e3, "tok_s": batch / step_s, "step_bytes": nbytes,
            "achieved_GBps": nbytes / step_s / 1e9, "mean_ctx": sum(lengths) / batch}


def stack_graph_main(args, wl) -> int:
    gpu = run_stack_graph(args, wl)
    result = {
        "metric": "attn-stack decode tok/s (40 layers, B=1..128); state+KV HBM GB/s % of peak",
        "value": round(gpu["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 state, bf16 KV and activations",
        "data": "synthetic (seeded random state, KV and per-layer inputs; projections excluded)",
        "config": {"workload": wl["desc"], "batch": gpu["batch"], "mean_context": round(gpu["mean_ctx"]),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "whole step (all launches, one graph)",
                     "achieved": round(gpu["achieved_GBps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gpu["achieved_GBps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_step": gpu["step_bytes"]},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def forward_main(args, wl) -> int:
    gpu = run_forward_gpu(args, wl)
    result = {
        "metric": "decode tok/s through the attention side of the 40-layer stack (norms, FP8 projections, state "
                  "path, output projections, residual)",
        "value": round(gpu["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 state and residual, bf16 KV, fp8 e4m3 weights with fp16 MFMA",
        "data": "synthetic (seeded random state, KV, FP8 weights and residual-stream inputs)",
        "config": {"workload": wl["desc"], "batch": gpu["batch"], "mean_context": round(gpu["mean_ctx"]),
                   "fp8_weight_GB": round(gpu["weight_bytes"] / 1e9, 3), "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "whole step (all launches)", "achieved": round(gpu["achieved_GBps"], 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gpu["achieved_GBps"] / HBM_PEAK_GBPS, 4),
                     "traffic": None, "bytes_per_step": gpu["step_bytes"]},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def proj_main(args, wl) -> int:
    gpu = run_proj_gpu(args, wl)
    result = {
        "metric": "projection pass tok/s (all 40 layers' FP8 projections for one decode step); weight GB/s % of HBM peak",
        "value": round(gpu["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 e4m3 weights (128x128 block scales), fp16 activations and MFMA, fp32 accumulation",
        "data": "synthetic (random FP8 weights and scales, random activations)",
        "config": {"workload": wl["desc"], "batch": gpu["batch"], "fp8_weight_GB": round(gpu["weight_bytes"] / 1e9, 3),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm",
                     "kernel": ("gemv_fp8_kernel" if gpu["batch"] <= 16 else "linear_fp8_ks_kernel")
                     + " (ria_linear_fp8_group), all launches of the step",
                     "achieved": round(gpu["achieved_GBps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gpu["achieved_GBps"] / HBM_PEAK_GBPS, 4), "traffic": None,
                     "mfma_TFLOPs": round(gpu["TFLOPs"], 1),
                     "mfma_frac": round(gpu["TFLOPs"] / MFMA_PEAK_TFLOPS, 4)},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_snapshot_gpu(args, wl) -> dict:
    """Save every row of the ragged stack into a payload and restore it, `steps` times."""
    from router_ia import kernels as K
    from router_ia import workloads as W
    from router_ia.batched_state import BatchedAttentionState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batch = wl["batch"]
    lengths = W.ragged_lengths(wl["seed"], batch, wl["lo"], wl["hi"])
    num_pages = sum((n + 16) // 16 for n in lengths) + batch
    st = BatchedAttentionState(batch, max(lengths) + 16, num_pages=num_pages, device=dev,
                               page_shuffle_seed=wl["seed"])
    st.set_positions(lengths)
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    st.linear_states.normal_(0.0, 0.02, generator=gen)
    st.conv_rings.normal_(0.0, 1.0, generator=gen)
    st.kv.k.normal_(0.0, 1.0, generator=gen)
    st.kv.v.normal_(0.0, 1.0, generator=gen)
    sizes = [K.seq_state_bytes(st.num_linear_layers, st.num_v_heads, st.conv_dim, st.num_full_layers,
                               st.num_kv_heads, n) for n in lengths]
    payload = torch.empty(max(sizes), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    log(f"[bench] {wl['desc']}: payload {sum(sizes) / 2**30:.1f} GiB over {batch} sequences")
    pools = (st.linear_states, st.conv_rings, st.kv.k, st.kv.v, st.kv.page_table)

    def one_pass(ev):
        for r, n in enumerate(lengths):
            e0 = torch.cuda.Event(enable_timing=True) if ev is not None else None
            if e0 is not None:
                e0.record()
            K.seq_state_save(*pools, row=r, tokens=n, payload=payload)
            K.seq_state_restore(*pools, row=r, tokens=n, payload=payload)
            if e0 is not None:
                e1 = torch.cuda.Event(enable_timing=True)
                e1.record()
                ev.append((e0, e1, 4 * sizes[r]))

    for _ in range(args.warmup):
        one_pass(None)
    torch.cuda.synchronize()
    ev: list = []
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        one_pass(ev)
    t1.record()
    torch.cuda.synchronize()
    elapsed = t0.elapsed_time(t1) / 1e3
    moved = 4 * sum(sizes) * args.steps  # save reads + writes the payload's bytes, restore the same again
    per_row_s = sum(a.elapsed_time(b) for a, b, _ in ev) / 1e3
    achieved = sum(nb for _, _, nb in ev) / per_row_s / 1e9
    return {
        "batch": batch, "lengths": lengths, "elapsed_s": elapsed,
        "seq_per_s": batch * args.steps / elapsed,
        "ms_per_step": elapsed / args.steps * 1e3,
        "payload_bytes": sum(sizes),
        "roofline": {"bound": "hbm", "kernel": "ria_seq_state_save + ria_seq_state_restore (dense + tile copies)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_pass": moved // args.steps},
        "step_GBps": round(moved / elapsed / 1e9, 1),
    }


def snapshot_main(args, wl) -> int:
    gpu = run_snapshot_gpu(args, wl)
    result = {
        "metric": "sequence snapshot save+restore GB/s (40 layers, B=128 ragged 1k-32k); % of HBM peak",
        "value": gpu["step_GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bytes (fp32 state, bf16 conv ring and KV)",
        "data": "synthetic (seeded random state and KV)",
        "config": {"workload": wl["desc"], "batch": gpu["batch"], "payload_GiB": round(gpu["payload_bytes"] / 2**30, 2),
                   "sequences_per_s": round(gpu["seq_per_s"], 1), "parallelism": "single GPU"},
        "roofline": gpu["roofline"],
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def run_prefill_gpu(args, wl) -> dict:
    """One 16384-token prompt through one DeltaNet layer and one attention layer, `steps` times."""
    from router_ia import _native as nat
    from router_ia import kernels as K
    from router_ia.batched_state import rope_inv_freq
    from router_ia.paged_kv import PagedKVCache

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = PREFILL_LEN
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    mixed = torch.randn((L, CONV_DIM), generator=gen, device=dev).to(torch.bfloat16)
    a_raw = torch.randn((L, NUM_V_HEADS), generator=gen, device=dev)
    b_raw = torch.randn((L, NUM_V_HEADS), generator=gen, device=dev)
    conv_w = (torch.randn((CONV_DIM, 1, 4), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    a_log = torch.rand((NUM_V_HEADS,), generator=gen, device=dev) * 4.0 - 4.0
    dt_bias = torch.zeros((NUM_V_HEADS,), device=dev)
    state = torch.zeros((NUM_V_HEADS, 128, 128), device=dev)
    ring = torch.zeros((4, CONV_DIM), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(K.gdn_prefill_workspace_bytes(16, NUM_V_HEADS, L), dtype=torch.uint8, device=dev)
    gdn_out = torch.empty((L, NUM_V_HEADS, 128), device=dev, dtype=torch.bfloat16)
    q = torch.randn((L, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev).to(torch.bfloat16)
    gate = torch.randn((L, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev).to(torch.bfloat16)
    k = torch.randn((L, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((L, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev).to(torch.bfloat16)
    pages = L // 16 + 2
    kv = PagedKVCache(1, pages, 1, pages, num_kv_heads=NUM_KV_HEADS, device=dev, shuffle_seed=wl["seed"])
    kv.ensure(0, L)
    inv_freq = rope_inv_freq(1e7, 64).to(dev)
    attn_out = torch.empty((L, NUM_Q_HEADS, HEAD_DIM_ATTN), device=dev, dtype=torch.bfloat16)
    norms = bool(wl.get("norms"))
    z = torch.randn((L, NUM_V_HEADS, 128), generator=gen, device=dev).to(torch.bfloat16) if norms else None
    gnw = 1.0 + 0.1 * torch.randn((128,), generator=gen, device=dev) if norms else None
    qnw = 0.1 * torch.randn((HEAD_DIM_ATTN,), generator=gen, device=dev) if norms else None
    knw = 0.1 * torch.randn((HEAD_DIM_ATTN,), generator=gen, device=dev) if norms else None
    log(f"[bench] {wl['desc']}")

    def gdn():
        K.gdn_prefill(mixed, state, a_raw, b_raw, gdn_out, num_k_heads=16, num_v_heads=NUM_V_HEADS,
                      conv_weight=conv_w, conv_ring=ring, conv_pos=0, workspace=ws, gate_mode=nat.RIA_GATE_RAW,
                      A_log=a_log, dt_bias=dt_bias, z=z, norm_weight=gnw)

    stage = torch.empty(K.prefill_stage_bytes(L, NUM_KV_HEADS), dtype=torch.uint8, device=dev)

    def attn(phase):
        # the prompt starts the sequence: its attention reads fp16 copies of its keys (the stage)
        K.attn_prefill(q, k, v, gate, kv.k[0], kv.v[0], kv.page_table[0], attn_out, start=0, inv_freq=inv_freq,
                       scale=HEAD_DIM_ATTN ** -0.5, phase=phase, q_norm_weight=qnw, k_norm_weight=knw, stage=stage)

    for _ in range(args.warmup):
        gdn()
        attn(nat.RIA_PREFILL_BOTH)
    torch.cuda.synchronize()
    ev = {name: [] for name in ("gdn", "append", "attend")}
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t_start.record()
    for _ in range(args.steps):
        for name, fn in (("gdn", gdn), ("append", lambda: attn(nat.RIA_PREFILL_APPEND)),
                         ("attend", lambda: attn(nat.RIA_PREFILL_ATTEND))):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            ev[name].append((e0, e1))
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    elapsed_s = t_start.elapsed_time(t_end) / 1e3
    avg = {name: sum(a.elapsed_time(b) for a, b in pairs) / len(pairs) / 1e3 for name, pairs in ev.items()}
    attn_flop = attn_prefill_flop(L)
    gdn_flop = GDN_CHUNK_FLOP * NUM_V_HEADS * (L // 64)
    achieved = attn_flop / avg["attend"] / 1e12
    return {
        "batch": 1,
        "lengths": [L],
        "elapsed_s": elapsed_s,
        "wall_s": wall,
        "tok_s": L * args.steps / elapsed_s,
        "ms_per_step": elapsed_s / args.steps * 1e3,
        "roofline": {
            "bound": "mfma",
            "kernel": "attn_prefill_kernel (ria_attn_prefill_phase, attention launch)",
            "achieved": round(achieved, 1),
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_flop_per_launch": attn_flop,
            "avg_launch_us": round(avg["attend"] * 1e6, 1),
            "launches": len(ev["attend"]),
            "mfma_work_note": ("the prompt's keys and values are read from fp16 copies (the stage), so q and the "
                               "probabilities are single fp16 operands: the MFMA pipe executes the algorithmic "
                               "FLOPs once"),
        },
        "kernels": {
            "gdn_prefill (conv + chunk prep + chunk scan)": {
                "avg_call_us": round(avg["gdn"] * 1e6, 1),
                "algorithmic_flop": gdn_flop,
                "achieved_TFLOPs": round(gdn_flop / avg["gdn"] / 1e12, 1),
                "frac": round(gdn_flop / avg["gdn"] / 1e12 / MFMA_PEAK_TFLOPS, 4),
            },
            "kv_append_kernel (prompt k/v into pages)": {"avg_call_us": round(avg["append"] * 1e6, 1)},
        },
    }


def run_prefill_cpu(wl, n_gdn: int, n_attn: int) -> dict:
    """The reference's token-by-token prefill (oracle restatement) timed per token on this host.

    Per token the reference runs one DeltaNet decode step (position independent)
    and one attention decode step over every earlier token; over a 16384-token
    prompt the mean attention context is 8192, so the attention step is timed
    at positions 8192.. with an 8192-token fp32 cache.
    """
    from oracle import qwen36_cpu as O

    torch.set_num_threads(os.cpu_count() or 1)
    gen = torch.Generator().manual_seed(wl["seed"])
    conv_w = (torch.randn((CONV_DIM, 1, 4), generator=gen) * 0.5).to(torch.bfloat16)
    a_log = torch.rand((NUM_V_HEADS,), generator=gen) * 4.0 - 4.0
    zero_bias = torch.zeros(NUM_V_HEADS)
    xs = torch.randn((n_gdn, 1, CONV_DIM), generator=gen).to(torch.bfloat16)
    ab = torch.randn((n_gdn, 2, 1, NUM_V_HEADS), generator=gen)
    conv_state = lin_state = None
    t0 = time.perf_counter()
    for i in range(n_gdn):
        beta, g = O.gating(ab[i, 0], ab[i, 1], a_log, zero_bias)
        _, conv_state, lin_state = O.linear_decode_step(conv_state, lin_state, xs[i], conv_w, beta, g)
    t_gdn = (time.perf_counter() - t0) / n_gdn
    ctx = PREFILL_LEN // 2
    fk = torch.randn((1, NUM_KV_HEADS, ctx, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16).float()
    fv = torch.randn((1, NUM_KV_HEADS, ctx, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16).float()
    qa = torch.randn((n_attn, 2, 1, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16)
    kva = torch.randn((n_attn, 2, 1, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16)
    t0 = time.perf_counter()
    for i in range(n_attn):
        _, fk, fv = O.full_decode_step(fk, fv, qa[i, 0], kva[i, 0], kva[i, 1], qa[i, 1], ctx + i)
    t_attn = (time.perf_counter() - t0) / n_attn
    return {
        "value": round(1.0 / (t_gdn + t_attn), 3),
        "unit": "tok/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"token-by-token prefill as the reference runs it (torch-CPU restatement, fp32): {n_gdn} DeltaNet "
                   f"decode steps ({t_gdn * 1e3:.2f} ms/token) + {n_attn} attention decode steps at positions "
                   f"{ctx}..{ctx + n_attn - 1}, the prompt's mean context ({t_attn * 1e3:.2f} ms/token)"),
    }


def run_prefill_cpu_full(wl) -> dict:
    """The whole 16384-token prompt through the reference's token-by-token CPU path (oracle restatement):
    every DeltaNet step and every attention step from an empty cache, as the reference prefills.  Takes
    minutes (the attention's torch.cat cache grows to the prompt's length), so it is an option of its own."""
    from oracle import qwen36_cpu as O

    torch.set_num_threads(os.cpu_count() or 1)
    n = PREFILL_LEN
    gen = torch.Generator().manual_seed(wl["seed"])
    conv_w = (torch.randn((CONV_DIM, 1, 4), generator=gen) * 0.5).to(torch.bfloat16)
    a_log = torch.rand((NUM_V_HEADS,), generator=gen) * 4.0 - 4.0
    zero_bias = torch.zeros(NUM_V_HEADS)
    conv_state = lin_state = None
    t0 = time.perf_counter()
    for i in range(n):
        x = torch.randn((1, CONV_DIM), generator=gen).to(torch.bfloat16)
        ab = torch.randn((2, 1, NUM_V_HEADS), generator=gen)
        beta, g = O.gating(ab[0], ab[1], a_log, zero_bias)
        _, conv_state, lin_state = O.linear_decode_step(conv_state, lin_state, x, conv_w, beta, g)
        if (i + 1) % 4096 == 0:
            log(f"[bench] CPU DeltaNet prefill: {i + 1} / {n} tokens, {time.perf_counter() - t0:.1f} s")
    t_gdn = time.perf_counter() - t0
    fk = fv = torch.zeros((1, NUM_KV_HEADS, 0, HEAD_DIM_ATTN))
    t0 = time.perf_counter()
    for i in range(n):
        q = torch.randn((2, 1, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16)
        kv = torch.randn((2, 1, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen).to(torch.bfloat16)
        _, fk, fv = O.full_decode_step(fk, fv, q[0], kv[0], kv[1], q[1], i)
        if (i + 1) % 1024 == 0:
            log(f"[bench] CPU attention prefill: {i + 1} / {n} tokens, {time.perf_counter() - t0:.1f} s")
    t_attn = time.perf_counter() - t0
    return {
        "metric": "prefill tok/s of one 16384-token prompt, 1 DeltaNet + 1 attention layer, reference CPU path",
        "value": round(n / (t_gdn + t_attn), 3), "unit": "tok/s", "cores": torch.get_num_threads(),
        "kind": "port", "deltanet_s": round(t_gdn, 2), "attention_s": round(t_attn, 2),
        "sample": "the whole prompt, token by token, as the reference prefills it (torch-CPU restatement, fp32, "
                  "torch.cat KV cache from empty)",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="ragged128")
    ap.add_argument("--cpu-seqs", type=int, default=8)
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batches", action="store_true",
                    help="skip the B=1/8/32 sub-record of the default workload")
    ap.add_argument("--cpu-prefill-full", action="store_true",
                    help="only time the whole 16384-token prompt on the reference's CPU path (minutes; no GPU)")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="only run a plain device copy of this many bytes three times (counter calibration)")
    args = ap.parse_args()
    if args.cpu_prefill_full:
        print(json.dumps(run_prefill_cpu_full(WORKLOADS["prefill16k"])), flush=True)
        return 0
    if args.copy_bytes:
        src = torch.ones(args.copy_bytes // 4, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copied {src.numel() * 4} bytes x3", file=sys.stderr)
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (sequences shard across GPUs "
              "with no communication; see the sharding design). Run with --gpus 1.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    wl = WORKLOADS[args.workload]
    if wl.get("prefill"):
        return prefill_main(args, wl)
    if wl.get("snapshot"):
        return snapshot_main(args, wl)
    if wl.get("proj"):
        return proj_main(args, wl)
    if wl.get("forward"):
        return forward_main(args, wl)
    if wl.get("graph"):
        return stack_graph_main(args, wl)
    gpu = run_gpu(args, wl)
    prof = profiled_traffic("attn_splitk_kernel") if args.workload == "ragged128" else None
    if prof:
        gpu["roofline"]["traffic"] = prof["bytes"]
        gpu["roofline"]["traffic_note"] = (
            f"FETCH_SIZE*2.0 + WRITE_SIZE per launch from {prof['source']} (rocprofv3 --pmc, same workload); "
            f"algorithmic bytes of those launches {prof['algorithmic']}")
    batches = None if args.no_batches else run_batches()
    layer_configs = prefill = None
    if not args.no_batches:
        layer_configs = run_layer_configs(cpu=not args.no_cpu_baseline)
        prefill = run_prefill_sub(cpu=not args.no_cpu_baseline)
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU reference path on a sample")
        cpu = run_cpu_baseline(wl, gpu["lengths"], args.cpu_seqs, args.cpu_steps)
    result = {
        "metric": METRIC,
        "value": round(gpu["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 state + bf16 KV/activations (fp32 accumulate)",
        "data": "synthetic (seeded random state, KV and per-layer inputs; projections excluded)",
        "config": {
            "workload": wl["desc"],
            "batch": gpu["batch"],
            "layers": "30 Gated DeltaNet + 10 GQA full attention",
            "mean_context": round(sum(gpu["lengths"]) / len(gpu["lengths"])),
            "decode_steps": args.steps,
            "parallelism": "single GPU",
        },
        "roofline": gpu["roofline"],
        "step_hbm": gpu["step_hbm"],
        "kernels": gpu["kernels"],
        "batches": batches,
        "layer_configs": layer_configs,
        "prefill16k": prefill,
        "device": device_record(),
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def device_record() -> dict:
    """hipGetDeviceProperties of the measured GPU, with the peaks the fractions are quoted against."""
    from router_ia import _native as nat

    rec = nat.device_record(torch.cuda.current_device())
    rec["hbm_peak_GBps_used"] = HBM_PEAK_GBPS
    rec["mfma_bf16_dense_peak_TFLOPs_used"] = MFMA_PEAK_TFLOPS
    return rec


PREFILL_SUB_STEPS, PREFILL_SUB_WARMUP = 5, 2


def run_prefill_sub(cpu: bool) -> dict:
    """The 16384-token prompt (one DeltaNet layer, chunked; one attention layer, causal) as a sub-record:
    per-call times and MFMA fractions, with the reference's token-by-token CPU path on a sample."""
    wl = WORKLOADS["prefill16k"]
    r = run_prefill_gpu(argparse.Namespace(steps=PREFILL_SUB_STEPS, warmup=PREFILL_SUB_WARMUP), wl)
    gdn = r["kernels"]["gdn_prefill (conv + chunk prep + chunk scan)"]
    out = {
        "prompt_tokens": PREFILL_LEN, "steps": PREFILL_SUB_STEPS,
        "tok_s": round(r["tok_s"], 1), "ms_per_prompt": round(r["ms_per_step"], 4),
        "deltanet_ms": round(gdn["avg_call_us"] / 1e3, 4), "deltanet_TFLOPs": gdn["achieved_TFLOPs"],
        "deltanet_mfma_frac": gdn["frac"],
        "attention_ms": round(r["roofline"]["avg_launch_us"] / 1e3, 4),
        "attention_TFLOPs": r["roofline"]["achieved"], "attention_mfma_frac": r["roofline"]["frac"],
        "kv_append_us": r["kernels"]["kv_append_kernel (prompt k/v into pages)"]["avg_call_us"],
        "peak_TFLOPs": MFMA_PEAK_TFLOPS,
        "timing": "HIP events around each call",
    }
    torch.cuda.empty_cache()
    if cpu:
        out["cpu_baseline"] = run_prefill_cpu(wl, 96, 96)
    log(f"[bench] prefill16k: DeltaNet {out['deltanet_ms']} ms ({out['deltanet_mfma_frac']:.3f} of MFMA peak), "
        f"attention {out['attention_ms']} ms ({out['attention_mfma_frac']:.3f})")
    return out


BATCH_STEPS, BATCH_WARMUP = 48, 4

# The two single-layer batch-1 decode configurations, each run in full (every
# step of the configuration, one graph replay per token).
LAYER_CONFIGS = {
    "gdn_layer_b1_64": dict(batch=1, lo=0, hi=0, seed=0, kinds=["linear"], steps=64,
                            desc="single Gated DeltaNet layer, recurrent decode of 64 tokens, batch 1, zero state "
                                 "(fused conv, raw gates, bf16 inputs)"),
    "attn_layer_b1_4096_256": dict(batch=1, lo=4096, hi=4096, seed=1, kinds=["full"], steps=256,
                                   desc="single full-attention layer decode, batch 1, 256 tokens appended to a "
                                        "prefilled 4096-token bf16 KV cache (partial RoPE, sigmoid gate)"),
}


def run_layer_config_gpu(wl) -> dict:
    """Every token of a single-layer batch-1 configuration captured as one HIP graph (the launches of all
    tokens back to back, as a decode loop issues them), replayed from the starting position."""
    from router_ia import _native as nat
    from router_ia.batched_state import BatchedAttentionState

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kinds, steps, ctx0 = wl["kinds"], wl["steps"], wl["lo"]
    linear = kinds == ["linear"]
    st = BatchedAttentionState(1, ctx0 + steps + 16, num_pages=(ctx0 + steps + 15) // 16 + 1, device=dev,
                               page_shuffle_seed=wl["seed"], num_linear_layers=int(linear),
                               num_full_layers=int(not linear))
    st.set_positions([ctx0])
    st.reserve(steps)
    gen = torch.Generator(device=dev)
    gen.manual_seed(wl["seed"])
    if linear:
        conv_w = (torch.randn((CONV_DIM, 1, 4), generator=gen, device=dev) * 0.5).to(torch.bfloat16)
        a_log = torch.rand((NUM_V_HEADS,), generator=gen, device=dev) * 4.0 - 4.0
        dt_bias = torch.zeros((NUM_V_HEADS,), device=dev)
        mixed = torch.randn((steps, 1, CONV_DIM), generator=gen, device=dev, dtype=torch.bfloat16)
        gate_ab = torch.randn((steps, 2, 1, NUM_V_HEADS), generator=gen, device=dev)
        out = torch.empty((1, NUM_V_HEADS, 128), device=dev, dtype=torch.bfloat16)
    else:
        st.kv.k[0].normal_(0.0, 1.0, generator=gen)
        st.kv.v[0].normal_(0.0, 1.0, generator=gen)
        qg = torch.randn((steps, 2, 1, NUM_Q_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev, dtype=torch.bfloat16)
        kv = torch.randn((steps, 2, 1, NUM_KV_HEADS, HEAD_DIM_ATTN), generator=gen, device=dev, dtype=torch.bfloat16)
        out = torch.empty((1, NUM_Q_HEADS, HEAD_DIM_ATTN), device=dev, dtype=torch.bfloat16)

    def tokens():
        for t in range(steps):
            if linear:
                st.linear_step(0, mixed[t], conv_w, gate_ab[t, 0], gate_ab[t, 1], gate_mode=nat.RIA_GATE_RAW,
                               A_log=a_log, dt_bias=dt_bias, out=out)
            else:
                st.full_step(0, qg[t, 0], kv[t, 0], kv[t, 1], qg[t, 1], out=out)
            st.advance()

    pos0 = st._pos_ctx.clone()
    host = (list(st._host_seen), st._min_headroom)

    def rewind():
        st._pos_ctx.copy_(pos0)
        st._host_seen, st._min_headroom = list(host[0]), host[1]

    tokens()  # eager once
    torch.cuda.synchronize()
    rewind()
    graph = torch.cuda.CUDAGraph()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        with torch.cuda.graph(graph, stream=cs):
            tokens()
    torch.cuda.current_stream().wait_stream(cs)
    rewind()
    graph.replay()
    rewind()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    graph.replay()
    t1.record()
    torch.cuda.synchronize()
    per_token = t0.elapsed_time(t1) / 1e3 / steps
    nbytes = sum(step_bytes([ctx0 + t + 1], kinds=kinds) for t in range(steps)) / steps
    return {"us_per_token": per_token * 1e6, "tok_s": 1.0 / per_token, "achieved_GBps": nbytes / per_token / 1e9}


def run_layer_configs(cpu: bool) -> dict:
    """The single-layer batch-1 configurations: GPU (all tokens in one graph) and, with `cpu`, the reference's
    CPU path (the oracle's torch-CPU restatement) over the same number of tokens on this host."""
    out = {"timing": "HIP events around one replay of the graph of every token; CPU wall time of the oracle"}
    for name, wl in LAYER_CONFIGS.items():
        r = run_layer_config_gpu(wl)
        rec = {"desc": wl["desc"], "tokens": wl["steps"], "gpu_us_per_token": round(r["us_per_token"], 2),
               "gpu_tok_s": round(r["tok_s"], 1), "achieved_GBps": round(r["achieved_GBps"], 1),
               "frac": round(r["achieved_GBps"] / HBM_PEAK_GBPS, 4)}
        torch.cuda.empty_cache()
        if cpu:
            cpu_s = time_layer_config_cpu(wl)
            rec["cpu_tok_s"] = round(wl["steps"] / cpu_s, 2)
            rec["cpu_cores"] = torch.get_num_threads()
            rec["cpu_s"] = round(cpu_s, 3)
        log(f"[bench] {name}: {rec['gpu_us_per_token']} us per token on the GPU"
            + (f", CPU {rec['cpu_tok_s']} tok/s" if cpu else ""))
        out[name] = rec
    return out


def time_layer_config_cpu(wl) -> float:
    """Wall seconds of the oracle over every token of a single-layer configuration (its own seeded inputs)."""
    from oracle import qwen36_cpu as O
    from router_ia import workloads as W

    torch.set_num_threads(os.cpu_count() or 1)
    steps = wl["steps"]
    if wl["kinds"] == ["linear"]:
        params = W.gdn_layer_params(wl["seed"])
        inputs = W.gdn_step_inputs(wl["seed"], steps, 1)
        conv_s = lin_s = None
        t0 = time.perf_counter()
        for t in range(steps):
            beta, g = O.gating(inputs["a_raw"][t], inputs["b_raw"][t], params["A_log"], params["dt_bias"])
            _, conv_s, lin_s = O.linear_decode_step(conv_s, lin_s, inputs["mixed"][t], params["conv_weight"], beta, g)
        return time.perf_counter() - t0
    kpre, vpre = W.prefilled_kv(wl["seed"], 1, wl["lo"])
    x = W.attn_step_inputs(wl["seed"], steps, 1)
    fk, fv = kpre.float(), vpre.float()
    t0 = time.perf_counter()
    for t in range(steps):
        _, fk, fv = O.full_decode_step(fk, fv, x["q"][t], x["k"][t], x["v"][t], x["gate"][t], wl["lo"] + t)
    return time.perf_counter() - t0


def run_batches() -> dict:
    """The metric's small-batch end: the 40-layer stack at B=1, 8 and 32, every row at context 8192 (seed 2).

    Each decode step (fresh inputs copied in, 40 layers, position advance) is
    replayed as one captured HIP graph, as a serving loop would issue it; the
    fraction is the step's algorithmic bytes (state, conv history, KV and
    activations) over its time, against 8 TB/s.
    """
    out = {"context": 8192, "steps": BATCH_STEPS, "warmup": BATCH_WARMUP,
           "timing": "HIP events around the replayed step graphs"}
    for name in ("batch1", "batch8", "batch32"):
        sub = argparse.Namespace(steps=BATCH_STEPS, warmup=BATCH_WARMUP)
        r = run_stack_graph(sub, WORKLOADS[name])
        out[f"B{r['batch']}"] = {"ms_per_step": round(r["ms_per_step"], 4), "tok_s": round(r["tok_s"], 1),
                                 "achieved_GBps": round(r["achieved_GBps"], 1),
                                 "frac": round(r["achieved_GBps"] / HBM_PEAK_GBPS, 4)}
        log(f"[bench] {name}: {r['ms_per_step']:.4f} ms per step, {r['achieved_GBps'] / HBM_PEAK_GBPS:.3f} of HBM peak")
        torch.cuda.empty_cache()
    return out


def prefill_main(args, wl) -> int:
    gpu = run_prefill_gpu(args, wl)
    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU reference path (token-by-token prefill) on a sample")
        cpu = run_prefill_cpu(wl, 96, 96)
    result = {
        "metric": PREFILL_METRIC,
        "value": round(gpu["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16 activations and KV pages, fp32 state and accumulate (DeltaNet: MFMA bf16 hi+lo operands; "
                  "attention: fp16 copies of the prompt's keys and values, fp16 operands)"),
        "data": "synthetic (seeded random prompt inputs; projections excluded)",
        "config": {
            "workload": wl["desc"],
            "prompt_tokens": PREFILL_LEN,
            "layers": "1 Gated DeltaNet (chunk 64) + 1 GQA full attention (16 Q / 2 KV heads x 256)",
            "parallelism": "single GPU",
        },
        "roofline": gpu["roofline"],
        "kernels": gpu["kernels"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
