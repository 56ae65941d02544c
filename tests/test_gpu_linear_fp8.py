"""GPU parity: projections with FP8 block-scaled weights (ria_dequant_fp8, ria_linear_fp8[_group]).

The reference dequantises its float8_e4m3fn checkpoint weights once to fp16
(qwen36_dequant.py:35-58, qwen36_cached_loop.py:537-542) and runs fp16
F.linear.  The oracle (oracle.qwen36_cpu.projection_fp8, pinned against
fp64, torch's e4m3fn decoding and transformers' Fp8Dequantize) restates
that; the kernels must give the same dequantised weights bit for bit and
the same fp16 projection up to the order of the fp32 accumulation.
"""

from __future__ import annotations

import pytest
import torch

from conftest import announce
from helpers import assert_act_close
from oracle import qwen36_cpu as O
from router_ia import kernels as K
from router_ia import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_dequant_all_byte_values_bit_exact(gpu, out_dtype):
    announce(f"dequant_fp8: all 256 e4m3 bytes x 4 scale blocks -> {out_dtype}")
    w8 = torch.arange(256, dtype=torch.uint8).repeat(130, 1)  # [130, 256]: every byte in every block
    w8[:, :128] = w8[:, :128].roll(7, dims=1)
    s = torch.tensor([[1.0, 0.5], [3.0e-3, 117.25]])
    got = K.dequant_fp8(w8.to(gpu), s.to(gpu), out_dtype).cpu()
    want = O.dequantize_fp8_blockwise(w8.view(torch.float8_e4m3fn), s).to(out_dtype)
    torch.testing.assert_close(got, want, rtol=0, atol=0, equal_nan=True)


CASES = [  # (m, n, k, x dtype): decode batches, one and two 128-row blocks, 16- and 32-wide tiles
    (1, 8192, 2048, torch.bfloat16),   # up to 16 rows and K a multiple of 512: the one-pass decode kernel
    (7, 4096, 2048, torch.float16),
    (16, 2048, 4096, torch.float32),
    (9, 256, 512, torch.bfloat16),     # one wave of K
    (17, 512, 2048, torch.float16),    # one row past the decode kernel: the K-split kernel (fp16 x)
    (32, 2048, 4096, torch.float32),
    (128, 2048, 4096, torch.float16),  # 64-row workgroups: two per 16 features
    (70, 2048, 4096, torch.bfloat16),  # .. the second one with 6 rows
    (128, 512, 2048, torch.bfloat16),
    (128, 8192, 2048, torch.float16),
    (200, 32, 2048, torch.float16),
    (5, 1024, 1408, torch.bfloat16),   # 11 chunks: one ring group and a 3-chunk tail
    (3, 512, 384, torch.float16),      # 3 chunks: the tail alone
    (1, 64, 128, torch.bfloat16),      # one chunk
]


@pytest.mark.parametrize("m,n,k,xdt", CASES)
def test_linear_fp8_matches_oracle(gpu, m, n, k, xdt):
    announce(f"linear_fp8: M={m} N={n} K={k} x {xdt}")
    w8, s = W.fp8_block_weight(200 + m, n, k)
    g = torch.Generator().manual_seed(300 + m)
    # x rows inside a wider buffer (a strided view, as a fused projection output would be)
    wide = torch.randn((m, k + 64), generator=g).to(xdt)
    x = wide[:, :k]
    got = K.linear_fp8(x.to(gpu), w8.to(gpu), s.to(gpu)).cpu()
    want = O.projection_fp8(x, w8, s)
    assert got.dtype == torch.float16
    assert_act_close(got, want, f"M={m} N={n} K={k}")
    # Against the exact product of the same fp16 operands, the kernel is as
    # accurate as the oracle's fp32-accumulated F.linear: both err by the fp16
    # rounding of the result plus an fp32 summation error that depends on the
    # order (about 1e-4 here, where the K terms sum to ~26 in magnitude).
    w16 = O.dequantize_fp8_blockwise(w8, s).to(torch.float16)
    exact = x.to(torch.float16).double() @ w16.double().T
    e_got = (got.double() - exact).abs().max().item()
    e_ref = (want.double() - exact).abs().max().item()
    assert e_got <= 1.5 * e_ref + 1e-6, (e_got, e_ref)


KSPLIT_F16 = [  # fp16 x past 16 rows (the forward loop's projections): the K-split kernel's
    (96, 12288, 2048),   # tile shapes, with whole and partial row blocks and column tiles
    (128, 8192, 2048),
    (100, 20480, 2048),
    (64, 8192, 512),
    (128, 2048, 4096),   # the output projections' shape
    (128, 8192, 4096),   # K = 4096 with a wide N: 64-row x 64-feature tiles
    (70, 2048, 4096),
    (17, 512, 512),
    (33, 96, 128),       # one chunk of K, a partial last column tile
]


@pytest.mark.parametrize("m,n,k", KSPLIT_F16)
def test_ksplit_kernel_fp16_x_matches_oracle(gpu, m, n, k):
    announce(f"linear_fp8 K-split: M={m} N={n} K={k} x fp16")
    w8, s = W.fp8_block_weight(250 + m, n, k)
    g = torch.Generator().manual_seed(350 + m)
    wide = torch.randn((m, k + 64), generator=g).to(torch.float16)
    x = wide[:, :k]
    got = K.linear_fp8(x.to(gpu), w8.to(gpu), s.to(gpu)).cpu()
    want = O.projection_fp8(x, w8, s)
    assert_act_close(got, want, f"M={m} N={n} K={k}")
    w16 = O.dequantize_fp8_blockwise(w8, s).to(torch.float16)
    exact = x.double() @ w16.double().T
    e_got = (got.double() - exact).abs().max().item()
    e_ref = (want.double() - exact).abs().max().item()
    assert e_got <= 1.5 * e_ref + 1e-6, (e_got, e_ref)


@pytest.mark.parametrize("m", [9, 100])
def test_linear_fp8_output_dtypes_round_through_fp16(gpu, m):
    announce(f"linear_fp8: M={m} fp32 and bf16 outputs carry the fp16 result")
    w8, s = W.fp8_block_weight(400, 512, 2048)
    x = torch.randn((m, 2048), generator=torch.Generator().manual_seed(401)).to(torch.bfloat16).to(gpu)
    w8, s = w8.to(gpu), s.to(gpu)
    y16 = K.linear_fp8(x, w8, s)
    y32 = K.linear_fp8(x, w8, s, out_dtype=torch.float32)
    yb = K.linear_fp8(x, w8, s, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(y32.cpu(), y16.cpu().float())
    assert torch.equal(yb.cpu(), y16.cpu().to(torch.bfloat16))


GROUPS = [  # (m, [n_j], k): a DeltaNet layer's input projections, attention q/k/v, 16-wide tiles
    (1, [8192, 4096, 32, 32], 2048),
    (128, [8192, 4096, 32, 32], 2048),
    (37, [8192, 512, 512], 2048),
    (130, [48, 256], 1408),
    (40, [8192, 48], 2048),   # 64-wide tiles: the 48-wide projection fills part of one
]


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,ns,k", GROUPS)
def test_linear_fp8_group_equals_separate_calls(gpu, m, ns, k, xdt):
    announce(f"linear_fp8_group: M={m} N={ns} K={k} x {xdt}")
    proj = [W.fp8_block_weight(500 + j, n, k) for j, n in enumerate(ns)]
    x = torch.randn((m, k), generator=torch.Generator().manual_seed(510 + m)).to(xdt).to(gpu)
    proj_d = [(w.to(gpu), s.to(gpu)) for w, s in proj]
    dts = [torch.bfloat16, torch.float32, torch.float16, torch.float32][:len(ns)]  # each projection its own dtype
    ys = K.linear_fp8_group(x, proj_d, out_dtype=dts)
    for j, (w, s) in enumerate(proj_d):
        sep = K.linear_fp8(x, w, s, out_dtype=dts[j])
        torch.cuda.synchronize()
        assert ys[j].dtype == dts[j] and torch.equal(ys[j].cpu(), sep.cpu()), f"projection {j}"
    # and each against the oracle
    for j, (w, s) in enumerate(proj):
        want = O.projection_fp8(x.cpu(), w, s).to(dts[j])
        assert_act_close(ys[j].cpu(), want, f"projection {j}")


@pytest.mark.parametrize("m,n,k", [(100, 8192, 2048), (128, 2048, 4096), (37, 96, 128)])
def test_bf16_x_equals_its_fp16_conversion(gpu, m, n, k):
    """F.linear takes h.to(float16): bf16 x past 16 rows is converted inside the
    K-split kernel, which must give the bits of the same call on x.to(float16)
    (values spanning fp16's normal range, small ones included)."""
    announce(f"linear_fp8 bf16 x: M={m} N={n} K={k}")
    w8, s = W.fp8_block_weight(700 + m, n, k)
    g = torch.Generator().manual_seed(710 + m)
    x = torch.randn((m, k), generator=g) * torch.exp2(torch.randint(-12, 8, (m, k), generator=g).float())
    xb = x.to(torch.bfloat16).to(gpu)
    wd, sd = w8.to(gpu), s.to(gpu)
    got = K.linear_fp8(xb, wd, sd)
    ref = K.linear_fp8(xb.to(torch.float16), wd, sd)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), ref.cpu())


@pytest.mark.parametrize("m", [3, 100, 128])  # one-pass kernel; past 16 rows with partial and with whole row blocks
def test_linear_fp8_group_accumulates_into_fp32(gpu, m):
    announce(f"linear_fp8_group: M={m} y += fp16 result (residual add)")
    w8, s = W.fp8_block_weight(600, 2048, 4096)
    g = torch.Generator().manual_seed(601)
    x = torch.randn((m, 4096), generator=g).to(torch.float16).to(gpu)
    base = torch.randn((m, 2048), generator=g).to(gpu)
    y = base.clone()
    K.linear_fp8_group(x, [(w8.to(gpu), s.to(gpu))], out=[y], accumulate=[True])
    sep = K.linear_fp8(x, w8.to(gpu), s.to(gpu), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), base.cpu() + sep.cpu())


@pytest.mark.parametrize("m,k,hdt", [(1, 2048, torch.bfloat16), (3, 2048, torch.float16), (4, 4096, torch.bfloat16)])
def test_linear_fp8_group_with_fused_input_norm(gpu, m, k, hdt):
    announce(f"linear_fp8_group_normed: M={m} K={k} h {hdt}")
    ns = [8192, 4096, 32, 32] if k == 2048 else [2048]
    proj = [W.fp8_block_weight(700 + j, n, k) for j, n in enumerate(ns)]
    g = torch.Generator().manual_seed(710 + m)
    x = (torch.randn((m, k), generator=g) * 3.0).to(gpu)
    wn = (torch.randn((k,), generator=g) * 0.1).to(torch.bfloat16).float().to(gpu)
    proj_d = [(w.to(gpu), s.to(gpu)) for w, s in proj]
    fused = K.linear_fp8_group(x, proj_d, norm_weight=wn, norm_dtype=hdt)
    h = K.rmsnorm(x, wn, out=torch.empty((m, k), dtype=hdt, device=gpu))
    separate = K.linear_fp8_group(h, proj_d)
    for j, (w, s) in enumerate(proj):
        # both against the oracle's rmsnorm -> dtype -> fp16 projection
        want = O.projection_fp8(O.rmsnorm(x.cpu(), wn.cpu()).to(hdt), w, s)
        assert_act_close(fused[j].cpu(), want, f"fused projection {j}")
        assert_act_close(separate[j].cpu(), want, f"separate projection {j}")


def test_linear_fp8_group_normed_host_checks(gpu):
    w8, s = W.fp8_block_weight(720, 64, 2048)
    x = torch.randn((5, 2048)).to(gpu)
    wn = torch.zeros((2048,), device=gpu)
    with pytest.raises(RuntimeError, match="up to 4 rows"):
        K.linear_fp8_group(x, [(w8.to(gpu), s.to(gpu))], norm_weight=wn)
