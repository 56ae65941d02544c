"""Pin the CPU oracle (oracle/qwen36_cpu.py) before trusting it.

Each oracle function is checked against something it does not share code
with: the float64 brute force in oracle/fp64.py, closed forms, invariants
the mathematics fixes, and torch library routines (conv1d,
scaled_dot_product_attention).  The checks are chosen so that a plausible
slip (dead conv slot read, wrong rotate-half sign, missing decay, read-out
from the pre-update state, wrong GQA head mapping, gate applied per head
instead of per (head, dim)) fails at least one of them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp64
from oracle import qwen36_cpu as O


def _gen(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("position", [0, 1, 17, 63])
def test_rope_tables_match_closed_form_small_positions(position):
    cos, sin = O.rope(position)
    c64, s64 = fp64.rope_tables(position)
    np.testing.assert_allclose(cos.numpy(), c64, atol=2e-6)
    np.testing.assert_allclose(sin.numpy(), s64, atol=2e-6)


@pytest.mark.parametrize("position", [4096, 4351, 32767])
def test_rope_tables_at_large_positions_use_fp32_angles(position):
    # The reference forms the angle in fp32 (float(position) * inv_freq), so at
    # large positions it differs from the exact angle; cos/sin of that fp32
    # angle must still be correct to ~1 ulp.
    cos, sin = O.rope(position)
    ang = (np.float32(position) * O.inv_freq().numpy()).astype(np.float64)
    ang = np.concatenate([ang, ang])
    np.testing.assert_allclose(cos.numpy(), np.cos(ang), atol=1e-6)
    np.testing.assert_allclose(sin.numpy(), np.sin(ang), atol=1e-6)


def test_inv_freq_closed_form():
    inv = O.inv_freq().double().numpy()
    want = np.array([1e7 ** (-(2.0 * i) / 64) for i in range(32)])
    np.testing.assert_allclose(inv, want, rtol=1e-6)
    assert inv[0] == 1.0


def test_apply_rope_matches_fp64_rotation_and_invariants():
    g = _gen(0)
    q = torch.randn((1, 16, 1, 256), generator=g)
    k = torch.randn((1, 2, 1, 256), generator=g)
    for pos in (0, 5, 300):
        qr, kr = O.apply_rope(q, k, pos)
        # fp32 angles drift from the exact ones by ~pos * 6e-8 rad; |x| < 5 here
        tol = 1e-5 + 5 * 1.2e-7 * pos
        np.testing.assert_allclose(qr.numpy(), fp64.apply_rope(q.numpy(), pos), atol=tol)
        np.testing.assert_allclose(kr.numpy(), fp64.apply_rope(k.numpy(), pos), atol=tol)
        assert torch.equal(qr[..., 64:], q[..., 64:])  # pass-through dims untouched
        # each rotary pair keeps its norm
        pair_in = q[..., :32] ** 2 + q[..., 32:64] ** 2
        pair_out = qr[..., :32] ** 2 + qr[..., 32:64] ** 2
        torch.testing.assert_close(pair_out, pair_in, rtol=1e-5, atol=1e-6)
    qr0, _ = O.apply_rope(q, k, 0)
    assert torch.equal(qr0, q)


def test_apply_rope_composes_over_positions():
    # RoPE(p1) then RoPE(p2) == RoPE(p1 + p2) for the same head: a rotation group.
    g = _gen(1)
    x = torch.randn((1, 1, 1, 256), generator=g, dtype=torch.float64)
    a = torch.from_numpy(fp64.apply_rope(fp64.apply_rope(x.numpy(), 7), 9))
    b = torch.from_numpy(fp64.apply_rope(x.numpy(), 16))
    torch.testing.assert_close(a, b)
    r16, _ = O.apply_rope(x.float(), x.float(), 16)
    torch.testing.assert_close(r16.double(), b, rtol=1e-5, atol=1e-5)


def test_l2norm_matches_fp64_and_unit_norm():
    x = torch.randn((3, 32, 128), generator=_gen(2)) * 5
    y = O.l2norm(x)
    np.testing.assert_allclose(y.numpy(), fp64.l2norm(x.numpy()), rtol=2e-6, atol=1e-7)
    torch.testing.assert_close(y.norm(dim=-1), torch.ones(3, 32), rtol=1e-5, atol=1e-5)
    # eps matters only near zero
    z = O.l2norm(torch.zeros(1, 4))
    assert torch.equal(z, torch.zeros(1, 4))


def test_rmsnorm_matches_fp64_and_invariants():
    g = _gen(21)
    x = torch.randn((3, 16, 256), generator=g) * 3
    w = torch.randn(256, generator=g) * 0.1
    y = O.rmsnorm(x, w)
    np.testing.assert_allclose(y.numpy(), fp64.rmsnorm(x.numpy(), w.numpy()), rtol=2e-6, atol=2e-6)
    # the affine factor is (1 + w): w = 0 leaves rows of unit RMS (not zeros)
    u = O.rmsnorm(x, torch.zeros(256))
    torch.testing.assert_close(u.pow(2).mean(-1), torch.ones(3, 16), rtol=1e-5, atol=1e-5)
    # positive rescaling of a row cancels (eps aside)
    torch.testing.assert_close(O.rmsnorm(x * 7.5, w), y, rtol=1e-5, atol=1e-5)
    # the result is cast back to the input dtype after the fp32 math
    xh = x.to(torch.float16)
    yh = O.rmsnorm(xh, w.to(torch.bfloat16))
    assert yh.dtype == torch.float16
    ref = fp64.rmsnorm(xh.float().numpy(), w.to(torch.bfloat16).float().numpy())
    # within one fp16 ulp of the fp64 value rounded to fp16 (double rounding)
    torch.testing.assert_close(yh, torch.from_numpy(ref).to(torch.float16), rtol=1e-3, atol=0)


def test_gated_rmsnorm_matches_fp64_and_invariants():
    g = _gen(22)
    x = torch.randn((2, 32, 128), generator=g) * 0.3
    z = torch.randn((2, 32, 128), generator=g) * 2
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    y = O.gated_rmsnorm(x, z, w)
    assert y.dtype == torch.float32
    np.testing.assert_allclose(y.numpy(), fp64.gated_rmsnorm(x.numpy(), z.numpy(), w.float().numpy()),
                               rtol=3e-6, atol=2e-6)
    # the weight multiplies as w (no 1 +): w = 0 gives zeros; the gate is SiLU(z) per element
    assert torch.equal(O.gated_rmsnorm(x, z, torch.zeros(128)), torch.zeros_like(x))
    assert torch.equal(O.gated_rmsnorm(x, torch.zeros_like(z), w), torch.zeros_like(x))
    big = torch.full_like(z, 30.0)
    n = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    torch.testing.assert_close(O.gated_rmsnorm(x, big, w), w.float() * n * 30.0, rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------------------- conv
def _conv_case(seed, channels=64):
    g = _gen(seed)
    w = (torch.randn((channels, 1, 4), generator=g) * 0.5).to(torch.bfloat16)
    xs = torch.randn((6, 1, channels), generator=g).to(torch.bfloat16)
    return w, xs


def test_conv_step_matches_fp64_brute_force_and_shift():
    w, xs = _conv_case(3)
    state = None
    hist = [torch.zeros(64)] * 3
    for t in range(6):
        out, state = O.causal_conv1d_step(state, xs[t], w)
        want = fp64.conv_step(torch.stack(hist, 1).double().numpy(), xs[t][0].double().numpy(),
                              w[:, 0].double().numpy())
        # the reference rounds the conv to bf16, then SiLU to bf16
        np.testing.assert_allclose(out[0].float().numpy(), want, rtol=1.6e-2, atol=1e-2)
        hist = hist[1:] + [xs[t][0].float()]
        # new state = the last four inputs, oldest first
        assert torch.equal(state[0, :, 3], xs[t][0])
        if t >= 1:
            assert torch.equal(state[0, :, 2], xs[t - 1][0])


def test_conv_step_never_reads_slot_zero():
    w, xs = _conv_case(4)
    g = _gen(5)
    base_state = torch.randn((1, 64, 4), generator=g).to(torch.bfloat16)
    other = base_state.clone()
    other[:, :, 0] = 1000.0
    a, _ = O.causal_conv1d_step(base_state, xs[0], w)
    b, _ = O.causal_conv1d_step(other, xs[0], w)
    assert torch.equal(a, b)
    changed = base_state.clone()
    changed[:, :, 1] += 1.0
    c, _ = O.causal_conv1d_step(changed, xs[0], w)
    assert not torch.equal(a, c)


def test_conv_step_equals_library_conv_over_history():
    w, xs = _conv_case(6)
    state = torch.randn((1, 64, 4), generator=_gen(7)).to(torch.bfloat16)
    out, _ = O.causal_conv1d_step(state, xs[0], w)
    hist = torch.cat([state[:, :, 1:], xs[0].reshape(1, 64, 1)], dim=-1).float()
    lib = F.silu(F.conv1d(hist, w.float(), groups=64)[:, :, -1])
    torch.testing.assert_close(out.float(), lib, rtol=1.6e-2, atol=1e-2)


# ----------------------------------------------------------------------------- delta rule
def _delta_case(seed, hv=2):
    g = _gen(seed)
    q = torch.randn((1, hv, 128), generator=g)
    k = torch.randn((1, hv, 128), generator=g)
    v = torch.randn((1, hv, 128), generator=g)
    beta = torch.sigmoid(torch.randn((1, hv), generator=g))
    gl = -F.softplus(torch.randn((1, hv), generator=g)) * torch.exp(torch.rand((1, hv), generator=g) * 4 - 4)
    s0 = torch.randn((1, hv, 128, 128), generator=g) * 0.02
    return q, k, v, beta, gl, s0


def test_delta_step_matches_fp64_brute_force():
    q, k, v, beta, g, s0 = _delta_case(8)
    attn, s1 = O.gated_delta_step(s0, q, k, v, beta, g)
    for h in range(2):
        qn = fp64.l2norm(q[0, h].double().numpy()) * 128 ** -0.5
        kn = fp64.l2norm(k[0, h].double().numpy())
        o, sn = fp64.delta_step(s0[0, h].double().numpy(), qn, kn, v[0, h].double().numpy(),
                                float(beta[0, h]), float(g[0, h]))
        np.testing.assert_allclose(attn[0, h].numpy(), o, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(s1[0, h].numpy(), sn, rtol=1e-5, atol=1e-6)


def test_delta_step_invariants():
    q, k, v, beta, g, s0 = _delta_case(9)
    # beta = 0: only the decay acts, and the read-out is from the decayed state
    attn, s1 = O.gated_delta_step(s0, q, k, v, torch.zeros_like(beta), g)
    decay = torch.exp(g)[..., None, None]
    torch.testing.assert_close(s1, s0 * decay)
    qn = O.l2norm(q) * 128 ** -0.5
    torch.testing.assert_close(attn, (s1 * qn.unsqueeze(-1)).sum(-2))
    # decay 1, beta 1: the update makes the state map k exactly onto v (S^T k = v)
    attn, s1 = O.gated_delta_step(s0, q, k, v, torch.ones_like(beta), torch.zeros_like(g))
    kn = O.l2norm(k)
    torch.testing.assert_close((s1 * kn.unsqueeze(-1)).sum(-2), v, rtol=1e-4, atol=1e-4)
    # zero state: o = beta (q . k) v, read from the updated state
    attn, _ = O.gated_delta_step(None, q, k, v, beta, g)
    want = beta[..., None] * (qn * kn).sum(-1, keepdim=True) * v
    torch.testing.assert_close(attn, want, rtol=1e-5, atol=1e-6)


def test_gating_closed_form():
    a = torch.tensor([[-30.0, 0.0, 3.0, 25.0]])
    b = torch.tensor([[-2.0, 0.0, 1.0, 4.0]])
    a_log = torch.tensor([0.5, -1.0, -4.0, 0.0])
    dt = torch.tensor([0.1, 0.0, -0.2, 0.0])
    beta, g = O.gating(a, b, a_log, dt)
    x = (a + dt).double()
    sp = torch.where(x > 20, x, torch.log1p(torch.exp(x)))
    torch.testing.assert_close(g.double(), -torch.exp(a_log.double()) * sp, rtol=1e-6, atol=1e-9)
    torch.testing.assert_close(beta.double(), 1 / (1 + torch.exp(-b.double())))


def test_split_qkv_shares_each_qk_head_with_two_v_heads():
    mixed = torch.arange(8192, dtype=torch.float32).reshape(1, 8192)
    q, k, v = O.split_qkv(mixed)
    assert torch.equal(q[0, 5], mixed[0, 2 * 128:3 * 128])  # V head 5 -> QK head 2
    assert torch.equal(k[0, 31], mixed[0, 2048 + 15 * 128:2048 + 16 * 128])
    assert torch.equal(v[0, 31], mixed[0, 4096 + 31 * 128:])


# ----------------------------------------------------------------------------- full attention
def test_full_decode_matches_sdpa_and_fp64():
    g = _gen(10)
    t0 = 37
    fk = torch.randn((1, 2, t0, 256), generator=g)
    fv = torch.randn((1, 2, t0, 256), generator=g)
    q = torch.randn((1, 16, 256), generator=g)
    k = torch.randn((1, 2, 256), generator=g)
    v = torch.randn((1, 2, 256), generator=g)
    gate = torch.randn((1, 16, 256), generator=g)
    out, fk2, fv2 = O.full_decode_step(fk, fv, q, k, v, gate, t0)
    assert fk2.shape == (1, 2, t0 + 1, 256)
    qr = torch.from_numpy(fp64.apply_rope(q.double().numpy(), t0))
    kr = torch.from_numpy(fp64.apply_rope(k.double().numpy(), t0))
    K_all = torch.cat([fk.double(), kr.unsqueeze(2)], 2)
    V_all = torch.cat([fv.double(), v.double().unsqueeze(2)], 2)
    sdpa = F.scaled_dot_product_attention(qr.unsqueeze(2), K_all.repeat_interleave(8, 1), V_all.repeat_interleave(8, 1))
    want = sdpa[:, :, 0] * torch.sigmoid(gate.double())
    torch.testing.assert_close(out.double(), want, rtol=1e-4, atol=1e-5)
    for h in (0, 7, 8, 15):  # heads 0-7 read KV head 0, heads 8-15 KV head 1
        o = fp64.attention(qr[0, h].numpy(), K_all[0, h // 8].numpy(), V_all[0, h // 8].numpy(), 1 / 16)
        np.testing.assert_allclose(out[0, h].double().numpy(), o * fp64.sigmoid(gate[0, h].numpy()), rtol=1e-4,
                                   atol=1e-5)


@pytest.mark.parametrize("t0", [0, 16, 1000])
def test_grouped_attention_equals_the_expanded_form_and_fp64(t0):
    # the grouped GQA product (no 8x expanded copy) against the expanded
    # einsum of full_decode_step and the fp64 brute force per head
    g = _gen(12 + t0)
    fk = torch.randn((1, 2, t0, 256), generator=g) if t0 else None
    fv = torch.randn((1, 2, t0, 256), generator=g) if t0 else None
    q, gate = torch.randn((1, 16, 256), generator=g), torch.randn((1, 16, 256), generator=g)
    k, v = torch.randn((1, 2, 256), generator=g), torch.randn((1, 2, 256), generator=g)
    want, fk_w, fv_w = O.full_decode_step(fk, fv, q, k, v, gate, t0)
    got, fk_g, fv_g = O.full_decode_step_grouped(fk, fv, q, k, v, gate, t0)
    assert torch.equal(fk_w, fk_g) and torch.equal(fv_w, fv_g)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
    qr = fp64.apply_rope(q.double().numpy(), t0)
    for h in (0, 5, 8, 15):  # query head h reads KV head h // 8
        o = fp64.attention(qr[0, h], fk_w[0, h // 8].double().numpy(), fv_w[0, h // 8].double().numpy(), 1 / 16)
        np.testing.assert_allclose(got[0, h].double().numpy(), o * fp64.sigmoid(gate[0, h].numpy()), rtol=1e-4,
                                   atol=1e-5)


def test_full_decode_gate_is_per_head_and_dim():
    g = _gen(11)
    fk = torch.randn((1, 2, 5, 256), generator=g)
    fv = torch.randn((1, 2, 5, 256), generator=g)
    q, gate = torch.randn((1, 16, 256), generator=g), torch.zeros((1, 16, 256))
    k, v = torch.randn((1, 2, 256), generator=g), torch.randn((1, 2, 256), generator=g)
    base_out, _, _ = O.full_decode_step(fk, fv, q, k, v, gate, 5)
    gate2 = gate.clone()
    gate2[0, 3, 17] = 3.0
    out2, _, _ = O.full_decode_step(fk, fv, q, k, v, gate2, 5)
    diff = (out2 - base_out).abs() > 0
    assert diff[0, 3, 17] and diff.sum() == 1


# ----------------------------------------------------------------------------- FP8 projections
def test_e4m3fn_decoding_known_values_and_library_conversion():
    known = {0x00: 0.0, 0x38: 1.0, 0xB8: -1.0, 0x7E: 448.0, 0x01: 2.0 ** -9, 0x08: 2.0 ** -6, 0x3C: 1.5,
             0x30: 0.5, 0x77: 240.0}
    for b, v in known.items():
        assert fp64.e4m3fn_value(b) == v, hex(b)
    assert np.isnan(fp64.e4m3fn_value(0x7F)) and np.isnan(fp64.e4m3fn_value(0xFF))
    # torch's float8_e4m3fn conversion (the reference's weight.float()) agrees on all 256 bytes
    allb = torch.arange(256, dtype=torch.uint8)
    lib = allb.view(torch.float8_e4m3fn).float().double().numpy()
    mine = np.array([fp64.e4m3fn_value(b) for b in range(256)])
    np.testing.assert_array_equal(lib, mine)


def _fp8_weight(seed, n, k):
    g = _gen(seed)
    w = (torch.randn((n, k), generator=g) * 0.05).float()
    grid = (-(-n // 128), -(-k // 128))
    s = torch.rand(grid, generator=g) * 1e-3 + 1e-4
    q = (w / s.repeat_interleave(128, 0).repeat_interleave(128, 1)[:n, :k]).clamp(-448, 448)
    return q.to(torch.float8_e4m3fn), s


def test_dequantize_fp8_matches_fp64_including_ragged_blocks():
    w8, s = _fp8_weight(31, 130, 200)
    got = O.dequantize_fp8_blockwise(w8, s)
    want = fp64.dequant_fp8(w8.view(torch.uint8).numpy(), s.double().numpy())
    # one fp32 rounding of an exact product
    np.testing.assert_allclose(got.double().numpy(), want, rtol=2 ** -24, atol=0)
    # the scale of block (1, 1) reaches row 128 / col 128 and not before
    assert torch.equal(got[128:, 128:], w8[128:, 128:].float() * s[1, 1])
    assert torch.equal(got[:128, :128], w8[:128, :128].float() * s[0, 0])


def test_projection_fp8_rounds_like_an_fp16_linear():
    w8, s = _fp8_weight(32, 64, 256)
    x = torch.randn((5, 256), generator=_gen(33))
    y = O.projection_fp8(x, w8, s)
    assert y.dtype == torch.float16
    w16 = (w8.float().double() * torch.from_numpy(np.kron(s.double().numpy(), np.ones((128, 128))))[:64, :256])
    ref = x.to(torch.float16).double() @ w16.to(torch.float16).double().T
    torch.testing.assert_close(y.double(), ref.to(torch.float16).double(), rtol=1e-3, atol=1e-4)
