"""The C-ABI library loads on the host and exports every declared entry point.

No compute call is made here: only entry points that validate arguments on
the host and return before touching a GPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from router_ia import _native as nat

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def _declared() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ria_\w+)\s*\(", text, flags=re.M))
    return names


def test_header_declares_entry_points() -> None:
    names = _declared()
    assert {"ria_gdn_decode", "ria_attn_decode", "ria_kv_append", "ria_last_error", "ria_abi_version"} <= names


def test_library_exports_every_declared_symbol() -> None:
    lib = ctypes.CDLL(str(nat.library_path()))
    missing = [n for n in sorted(_declared()) if not hasattr(lib, n)]
    assert not missing, f"declared in include/ but not exported: {missing}"


def test_binding_covers_every_declared_symbol() -> None:
    assert _declared() == set(nat.SIGNATURES), set(nat.SIGNATURES) ^ _declared()


def test_abi_version_and_host_side_validation() -> None:
    lib = nat.load()
    assert lib.ria_abi_version() == nat.ABI_VERSION
    rc = lib.ria_gdn_decode(-1, 16, 32, None, 0, 0, 1, None, None, None, 0, None, None, None, None, 0, 0,
                            None, None, None, 0, None, 0, 0, None, None)
    assert rc == 1 and b"batch" in lib.ria_last_error()
    rc = lib.ria_attn_decode(1, 16, 2, None, 0, 4096, None, 0, 4096, None, None, 0, 1, None, 1, None, None, 0,
                             None, 1, 1, None, 64, None, 0.0625, 0, None, 0, None, 0, None)
    assert rc == 1 and b"null" in lib.ria_last_error()
    assert lib.ria_attn_decode_workspace_bytes(0, 16, 2, 10, 0) == 0
    assert lib.ria_attn_decode_workspace_bytes(1, 16, 2, 64, 64) > 0


@pytest.mark.parametrize("ctx,expect", [([4097], 64), ([8193] * 32, 512), ([32768] * 128, 3072)])
def test_split_heuristic(ctx, expect) -> None:
    from router_ia import kernels as K

    assert K.attn_decode_split_tokens(2, ctx) == expect


def test_prefill_attention_host_validation() -> None:
    lib = nat.load()
    # 16 query heads per KV head is beyond the kernel's group limit
    rc = lib.ria_attn_prefill(16, 32, 2, None, 8192, None, 512, None, 512, None, 8192, 0, None, None, 0, 4, None,
                              4, 0, None, 64, None, None, 0.0625, None, None)
    assert rc == 1 and b"at most 8" in lib.ria_last_error()
    # the prompt must fit in the row's pages: 60 + 10 tokens > 4 pages of 16
    fake = ctypes.c_void_p(256)
    rc = lib.ria_attn_prefill(10, 16, 2, fake, 4096, fake, 512, fake, 512, fake, 4096, 0, fake, fake, 0, 4, fake,
                              4, 60, fake, 64, None, None, 0.0625, fake, None)
    assert rc == 1 and b"exceed" in lib.ria_last_error()
    rc = lib.ria_kv_append_seq(10, 2, fake, 0, 512, fake, 0, 512, fake, fake, 0, 4, fake, 4, 60, fake, 64, None,
                               None)
    assert rc == 1 and b"exceed" in lib.ria_last_error()
    # zero-length prompts are a no-op
    assert lib.ria_attn_prefill(0, 16, 2, fake, 4096, fake, 512, fake, 512, fake, 4096, 0, fake, fake, 0, 4, fake,
                                4, 0, fake, 64, None, None, 0.0625, fake, None) == 0
    # the prefill kernel reads the q_norm weight in 16-byte vectors
    rc = lib.ria_attn_prefill(10, 16, 2, fake, 4096, fake, 512, fake, 512, fake, 4096, 0, fake, fake, 0, 4, fake,
                              4, 0, fake, 64, ctypes.c_void_p(260), None, 0.0625, fake, None)
    assert rc == 1 and b"q_norm_weight" in lib.ria_last_error()


def test_norm_entry_points_host_validation() -> None:
    lib = nat.load()
    fake = ctypes.c_void_p(256)
    # zero tokens: nothing to do, even with null pointers
    assert lib.ria_rmsnorm(0, 16, 256, None, 0, 4096, None, 1e-6, None, 0, 4096, None) == 0
    assert lib.ria_gated_rmsnorm(0, 32, 128, None, 2, 4096, None, 0, 4096, None, 1e-6, None, 0, 4096, None) == 0
    rc = lib.ria_rmsnorm(1, 16, 256, fake, 7, 4096, fake, 1e-6, fake, 0, 4096, None)
    assert rc == 1 and b"dtype" in lib.ria_last_error()
    rc = lib.ria_rmsnorm(2, 16, 256, fake, 0, 2048, fake, 1e-6, fake, 0, 4096, None)
    assert rc == 1 and b"stride" in lib.ria_last_error()
    rc = lib.ria_gated_rmsnorm(1, 32, 128, fake, 2, 4096, None, 0, 4096, fake, 1e-6, fake, 0, 4096, None)
    assert rc == 1 and b"null" in lib.ria_last_error()
    # a gated DeltaNet read-out needs the norm weight with its gate
    rc = lib.ria_gdn_decode(1, 16, 32, fake, 0, 8192, 0, None, None, None, 0, fake, None, fake, fake, 32, 0,
                            None, None, fake, 0, fake, 0, 4096, None, None)
    assert rc == 1 and b"norm_weight" in lib.ria_last_error()
    rc = lib.ria_gdn_prefill(64, 16, 32, fake, 0, 8192, fake, fake, 0, fake, fake, fake, 32, 0, None, None, fake, 0,
                             fake, 0, 4096, None, fake, 1 << 30, None)
    assert rc == 1 and b"norm_weight" in lib.ria_last_error()


def test_fp8_projection_host_validation() -> None:
    lib = nat.load()
    fake = ctypes.c_void_p(256)
    rc = lib.ria_dequant_fp8(4, 40, fake, fake, fake, 1, None)
    assert rc == 1 and b"multiple of 16" in lib.ria_last_error()
    rc = lib.ria_linear_fp8(1, 40, 2048, fake, 1, 2048, fake, fake, fake, 1, 40, None)
    assert rc == 1 and b"multiple of 16" in lib.ria_last_error()
    rc = lib.ria_linear_fp8(1, 32, 200, fake, 1, 256, fake, fake, fake, 1, 32, None)
    assert rc == 1 and b"multiple of 128" in lib.ria_last_error()
    rc = lib.ria_linear_fp8(1, 32, 128 * 257, fake, 1, 128 * 257, fake, fake, fake, 1, 32, None)
    assert rc == 1 and b"32768" in lib.ria_last_error()
    rc = lib.ria_linear_fp8(1, 32, 2048, ctypes.c_void_p(8), 1, 2048, fake, fake, fake, 1, 32, None)
    assert rc == 1 and b"aligned" in lib.ria_last_error()
    # zero rows: nothing to launch, even with null pointers
    assert lib.ria_linear_fp8(0, 32, 2048, None, 1, 2048, None, None, None, 1, 32, None) == 0

    def group(*ns, m=1, stride=None):
        arr = (nat.Fp8Proj * max(1, len(ns)))()
        for j, n in enumerate(ns):
            arr[j] = nat.Fp8Proj(256, 256, 256, n if stride is None else stride, n, 1, 0)
        return lib.ria_linear_fp8_group(m, 2048, fake, 1, 2048, len(ns), ctypes.addressof(arr), None)

    assert group(m=0) == 1 and b"1 to 4" in lib.ria_last_error()
    assert group(32, 32, 32, 32, 32) == 1 and b"1 to 4" in lib.ria_last_error()
    assert group(8192, 4096, 40) == 1 and b"projection 2" in lib.ria_last_error()
    assert group(512, 512, stride=256) == 1 and b"stride" in lib.ria_last_error()
    assert group(8192, 4096, 32, 32, m=0) == 0
    rc = lib.ria_linear_fp8_group(1, 2048, fake, 1, 2048, 2, None, None)
    assert rc == 1 and b"null" in lib.ria_last_error()
    arr = (nat.Fp8Proj * 1)()
    arr[0] = nat.Fp8Proj(256, 256, 256, 64, 64, 9, 0)
    rc = lib.ria_linear_fp8_group(1, 2048, fake, 1, 2048, 1, ctypes.addressof(arr), None)
    assert rc == 1 and b"dtype" in lib.ria_last_error()
    arr[0] = nat.Fp8Proj(256, 256, 256, 64, 64, 1, 1)  # accumulating into fp16
    rc = lib.ria_linear_fp8_group(1, 2048, fake, 1, 2048, 1, ctypes.addressof(arr), None)
    assert rc == 1 and b"y_add" in lib.ria_last_error()


def _c_layout(struct: str, fields: list[str], tmp_path: Path) -> list[int]:
    """sizeof and field offsets of a header struct, from a host program compiled with gcc."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    inc = HEADERS[0].parent
    body = "".join(f'  printf("%zu\\n", offsetof({struct}, {f}));\n' for f in fields)
    src = tmp_path / "layout.c"
    src.write_text(f'#include <stddef.h>\n#include <stdio.h>\n#include "ria_hybrid_attn.h"\n'
                   f'int main(void) {{\n  printf("%zu\\n", sizeof({struct}));\n{body}  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{inc}", str(src), "-o", str(exe)], check=True)
    return [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]


@pytest.mark.parametrize("cls,struct", [(nat.GdnDecodeDesc, "ria_gdn_decode_desc"), (nat.Fp8Proj, "ria_fp8_proj"),
                                        (nat.DeviceRecord, "ria_device_record")])
def test_ctypes_structs_match_the_header(cls, struct, tmp_path) -> None:
    names = [name for name, _ in cls._fields_]
    want = _c_layout(struct, names, tmp_path)
    got = [ctypes.sizeof(cls)] + [getattr(cls, n).offset for n in names]
    assert got == want, dict(zip(["sizeof"] + names, zip(got, want)))


def test_gdn_decode_ex_and_window_conv_host_validation() -> None:
    lib = nat.load()
    fake = ctypes.c_void_p(256)

    def desc(**kw):
        d = nat.GdnDecodeDesc(batch=1, num_k_heads=16, num_v_heads=32, x=256, x_dtype=0, x_row_stride=8192,
                              conv_layout=nat.RIA_CONV_WINDOW, conv_weight=256, conv_window_in=1 << 20,
                              conv_window_out=1 << 21, state_in=1 << 24, state_out=1 << 26, gate_a=256, gate_b=256,
                              gate_row_stride=32, gate_mode=0, qk_mode=0, out=256, out_dtype=2)
        for k, v in kw.items():
            setattr(d, k, v)
        return lib.ria_gdn_decode_ex(ctypes.byref(d), None)

    assert lib.ria_gdn_decode_ex(None, None) == 1 and b"null" in lib.ria_last_error()
    assert desc(conv_layout=7) == 1 and b"conv_layout" in lib.ria_last_error()
    assert desc(qk_mode=nat.RIA_QK_NORMALIZED) == 1 and b"RIA_CONV_NONE" in lib.ria_last_error()
    assert desc(conv_window_out=(1 << 20) + 8) == 1 and b"overlap" in lib.ria_last_error()
    assert desc(conv_window_out=None) == 1 and b"conv_window_out" in lib.ria_last_error()
    assert desc(state_out=(1 << 24) + 4096) == 1 and b"overlaps" in lib.ria_last_error()
    assert desc(conv_layout=nat.RIA_CONV_NONE, qk_mode=nat.RIA_QK_NORMALIZED,
                x_row_stride=8192) == 1 and b"x_row_stride" in lib.ria_last_error()
    assert desc(conv_layout=nat.RIA_CONV_RING) == 1 and b"conv_ring" in lib.ria_last_error()
    assert desc(batch=0) == 0  # nothing to launch
    # with seq_slot the pools' extent comes from pool_rows: required, and partial overlaps are refused
    slots = dict(seq_slot=256)
    assert desc(**slots) == 1 and b"pool_rows" in lib.ria_last_error()
    state_bytes = 32 * 128 * 128 * 4
    assert desc(pool_rows=8, state_out=(1 << 24) + 3 * state_bytes, **slots) == 1 \
        and b"overlaps" in lib.ria_last_error()
    window_bytes = 8192 * 4 * 2
    assert desc(pool_rows=8, conv_window_out=(1 << 20) + window_bytes, **slots) == 1 \
        and b"conv_window_out" in lib.ria_last_error()
    rc = lib.ria_conv1d_window_step(1, 8192, fake, 0, 8192, fake, ctypes.c_void_p(260), fake, fake, 2, None)
    assert rc == 1 and b"aligned" in lib.ria_last_error()
    rc = lib.ria_conv1d_window_step(1, 8192, fake, 0, 4096, fake, fake, fake, fake, 2, None)
    assert rc == 1 and b"x_row_stride" in lib.ria_last_error()
