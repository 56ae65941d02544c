"""ctypes binding of the gfx950 hybrid-attention library (include/ria_hybrid_attn.h).

The library is located the way the reference locates its native memory pool
(src/router_ia/qwen36_native_memory.py:29-45): an explicit path in the
``RIA_HIP_LIB`` environment variable wins, otherwise the in-tree build
``router_ia/_lib/libria_hip.so`` is used.  There is no fallback: if the
library cannot be loaded every compute entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_ENV = "RIA_HIP_LIB"
DEFAULT_LIB = Path(__file__).resolve().parent / "_lib" / "libria_hip.so"
ABI_VERSION = 5

RIA_DT_BF16 = 0
RIA_DT_F16 = 1
RIA_DT_F32 = 2
RIA_GATE_PRECOMPUTED = 0
RIA_GATE_RAW = 1
RIA_ATTN_SPLITK = 1
RIA_ATTN_COMBINE = 2
RIA_ATTN_BOTH = 3
RIA_PREFILL_APPEND = 1
RIA_PREFILL_ATTEND = 2
RIA_PREFILL_BOTH = 3
RIA_CONV_NONE = 0
RIA_CONV_RING = 1
RIA_CONV_WINDOW = 2
RIA_QK_RAW = 0
RIA_QK_NORMALIZED = 1

_c_int = ctypes.c_int
_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/ria_hybrid_attn.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ria_abi_version": (_c_int, []),
    "ria_device_info": (_c_int, [_c_int, _vp]),
    "ria_last_error": (ctypes.c_char_p, []),
    "ria_gdn_decode": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _c_int, _vp, _vp, _vp, _c_i32, _vp, _vp,
         _vp, _vp, _c_i64, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_i64, _vp, _vp],
    ),
    "ria_conv1d_step": (
        _c_int,
        [_c_int, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _vp, _vp, _c_i32, _vp, _c_int, _vp],
    ),
    "ria_conv1d_window_step": (
        _c_int,
        [_c_int, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _vp, _vp, _c_int, _vp],
    ),
    "ria_gdn_decode_ex": (_c_int, [_vp, _vp]),
    "ria_l2norm": (_c_int, [_c_i64, _c_int, _vp, _c_int, _c_f32, _vp, _vp]),
    "ria_rmsnorm": (_c_int, [_c_i64, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_f32, _vp, _c_int, _c_i64, _vp]),
    "ria_gated_rmsnorm": (
        _c_int,
        [_c_i64, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _c_f32, _vp, _c_int, _c_i64, _vp],
    ),
    "ria_rope_table": (_c_int, [_c_i32, _vp, _c_int, _vp, _vp, _vp]),
    "ria_rope_apply": (_c_int, [_c_i64, _c_int, _c_int, _vp, _vp, _vp, _c_i32, _vp]),
    "ria_kv_append": (
        _c_int,
        [_c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_int, _c_int, _vp, _c_i64,
         _vp, _vp, _c_i32, _vp, _c_i32, _vp, _c_int, _vp, _vp],
    ),
    "ria_kv_append_out": (
        _c_int,
        [_c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_int, _c_int, _vp, _c_i64,
         _vp, _vp, _c_i32, _vp, _c_i32, _vp, _c_int, _vp, _vp, _vp],
    ),
    "ria_attn_decode_split_tokens": (_c_int, [_c_int, _vp, _c_int]),
    "ria_attn_decode_workspace_bytes": (_c_i64, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ria_attn_decode": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_int, _c_int, _vp,
         _c_i64, _vp, _vp, _c_i32, _vp, _c_i32, _c_int, _vp, _c_int, _vp, _c_f32, _c_int, _vp, _c_i64,
         _vp, _c_int, _vp],
    ),
    "ria_attn_decode_phase": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_int, _c_int, _vp,
         _c_i64, _vp, _vp, _c_i32, _vp, _c_i32, _c_int, _vp, _c_int, _vp, _c_f32, _c_int, _vp, _c_i64,
         _vp, _c_int, _c_int, _vp],
    ),
    "ria_attn_decode_append": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp,
         _vp, _vp, _c_int, _c_int, _vp, _c_i64, _vp, _vp, _c_i32, _vp, _c_i32, _c_int, _vp, _c_int, _vp,
         _c_f32, _c_int, _vp, _c_i64, _vp, _c_int, _c_int, _vp],
    ),
    "ria_attn_decode_append_noalloc": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp,
         _vp, _vp, _c_int, _c_int, _vp, _c_i64, _vp, _vp, _c_i32, _vp, _c_i32, _c_int, _vp, _c_int, _vp,
         _c_f32, _c_int, _vp, _c_int, _c_int, _vp],
    ),
    "ria_gdn_prefill_workspace_bytes": (_c_i64, [_c_int, _c_int, _c_int]),
    "ria_gdn_prefill": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _c_i32, _vp, _vp, _vp, _c_i64, _c_int,
         _vp, _vp, _vp, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _c_i64, _vp],
    ),
    "ria_dequant_fp8": (_c_int, [_c_i64, _c_int, _vp, _vp, _vp, _c_int, _vp]),
    "ria_linear_fp8": (_c_int, [_c_int, _c_int, _c_int, _vp, _c_int, _c_i64, _vp, _vp, _vp, _c_int, _c_i64, _vp]),
    "ria_linear_fp8_group": (_c_int, [_c_int, _c_int, _vp, _c_int, _c_i64, _c_int, _vp, _vp]),
    "ria_linear_fp8_group_normed": (_c_int, [_c_int, _c_int, _vp, _c_i64, _vp, _c_f32, _c_int, _c_int, _vp, _vp]),
    "ria_seq_state_bytes": (_c_i64, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ria_seq_state_save": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_i64, _c_int,
         _vp, _c_i64, _vp],
    ),
    "ria_seq_state_restore": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_i64, _c_int,
         _vp, _c_i64, _vp],
    ),
    "ria_kv_gather": (
        _c_int,
        [_c_int, _c_int, _vp, _vp, _c_int, _vp, _c_i64, _vp, _c_i32, _c_i32, _vp, _vp, _vp],
    ),
    "ria_kv_append_seq": (
        _c_int,
        [_c_int, _c_int, _vp, _c_int, _c_i64, _vp, _c_int, _c_i64, _vp, _vp, _c_int, _c_int, _vp, _c_i64,
         _c_i32, _vp, _c_int, _vp, _vp],
    ),
    "ria_attn_prefill": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _vp, _vp,
         _c_int, _c_int, _vp, _c_i64, _c_i32, _vp, _c_int, _vp, _vp, _c_f32, _vp, _vp],
    ),
    "ria_attn_prefill_phase": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _vp, _vp,
         _c_int, _c_int, _vp, _c_i64, _c_i32, _vp, _c_int, _vp, _vp, _c_f32, _vp, _c_int, _vp],
    ),
    "ria_attn_prefill_stage_bytes": (_c_i64, [_c_int, _c_int]),
    "ria_attn_prefill_staged": (
        _c_int,
        [_c_int, _c_int, _c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _vp, _vp,
         _c_int, _c_int, _vp, _c_i64, _c_i32, _vp, _c_int, _vp, _vp, _c_f32, _vp, _c_i64, _vp, _c_int, _vp],
    ),
}



class GdnDecodeDesc(ctypes.Structure):
    """struct ria_gdn_decode_desc: one ria_gdn_decode_ex call."""
    _fields_ = [("batch", _c_int), ("num_k_heads", _c_int), ("num_v_heads", _c_int), ("x", _vp),
                ("x_dtype", _c_int), ("x_row_stride", _c_i64), ("conv_layout", _c_int), ("conv_weight", _vp),
                ("conv_ring", _vp), ("conv_pos", _vp), ("conv_pos_scalar", _c_i32), ("conv_window_in", _vp),
                ("conv_window_out", _vp), ("state_in", _vp), ("state_out", _vp), ("seq_slot", _vp),
                ("gate_a", _vp), ("gate_b", _vp), ("gate_row_stride", _c_i64), ("gate_mode", _c_int),
                ("A_log", _vp), ("dt_bias", _vp), ("qk_mode", _c_int), ("out", _vp), ("out_dtype", _c_int),
                ("z", _vp), ("z_dtype", _c_int), ("z_row_stride", _c_i64), ("norm_weight", _vp),
                ("pool_rows", _c_i64)]


class DeviceRecord(ctypes.Structure):
    """struct ria_device_record: the device a measurement ran on."""
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 256), ("compute_units", _c_int),
                ("clock_khz", _c_int), ("memory_clock_khz", _c_int), ("memory_bus_bits", _c_int),
                ("memory_bytes", _c_i64), ("l2_bytes", _c_int), ("lds_bytes_per_cu", _c_int),
                ("wavefront_size", _c_int)]


def device_record(device: int = 0) -> dict:
    """hipGetDeviceProperties of `device` as a dict (ria_device_info)."""
    rec = DeviceRecord()
    check(load().ria_device_info(int(device), ctypes.byref(rec)), "ria_device_info")
    out = {name: getattr(rec, name) for name, _ in DeviceRecord._fields_}
    out["name"], out["arch"] = rec.name.decode(errors="replace"), rec.arch.decode(errors="replace")
    return out


class Fp8Proj(ctypes.Structure):
    """struct ria_fp8_proj: one projection of a ria_linear_fp8_group call."""
    _fields_ = [("weight", _vp), ("scale_inv", _vp), ("y", _vp), ("y_row_stride", _c_i64), ("n", _c_int),
                ("y_dtype", _c_int), ("y_add", _c_int)]


LINEAR_GROUP_MAX = 4  # projections per ria_linear_fp8_group call

_LIB: ctypes.CDLL | None = None


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed a call."""


def library_path() -> Path:
    override = os.environ.get(LIB_ENV)
    return Path(override) if override else DEFAULT_LIB


def load() -> ctypes.CDLL:
    """Load (once) and type the HIP library; raise if it is absent or stale."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.is_file():
        raise NativeLibraryError(
            f"HIP library not found at {path}; build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            f"or `make -C router-ia_amd/csrc`, or point {LIB_ENV} at a built libria_hip.so"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.ria_abi_version()
    if version != ABI_VERSION:
        raise NativeLibraryError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().ria_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{what} failed (status {rc}): {msg}")
