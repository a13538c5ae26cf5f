"""ctypes binding of libtilemix_hip.so (the C ABI declared in include/tilemix_hip.h).

The library is loaded lazily, after ``torch`` so that it binds to the HIP
runtime torch already loaded (both carry the SONAME libamdhip64.so.7).  There
is no fallback: if the library is missing or does not match this module's view
of the ABI, every GPU entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtilemix_hip.so"
ABI_VERSION = 3

ROUTING_MIXED = 0
ROUTING_FP16 = 1
ROUTING_INT8 = 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float


class QuantParams(ctypes.Structure):
    """Mirror of ``tilemix_quant_params``."""

    _fields_ = [
        ("input", _vp),
        ("output", _vp),
        ("scale", _vp),
        ("scale_half", _vp),
        ("cu_seqlens", _vp),
        ("cu_seqlens_scale", _vp),
        ("stride_in_token", _i64),
        ("stride_in_head", _i64),
        ("stride_out_token", _i64),
        ("stride_out_head", _i64),
        ("scale_rows_capacity", _i64),
        ("sm_scale", _f32),
        ("heads", _i32),
        ("head_dim", _i32),
        ("blk_tokens", _i32),
        ("batch", _i32),
        ("max_seqlen", _i32),
    ]


class AttnParams(ctypes.Structure):
    """Mirror of ``tilemix_attn_params``."""

    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("bias", _vp), ("out", _vp),
        ("precision_bitmask", _vp),
        ("q8", _vp), ("k8", _vp), ("v8", _vp),
        ("sq", _vp), ("sk", _vp), ("sv", _vp),
        ("cu_seqlens_q", _vp), ("cu_seqlens_k", _vp),
        ("cu_q_scale", _vp), ("cu_k_scale", _vp), ("cu_v_scale", _vp),
        ("stride_q_token", _i64), ("stride_q_head", _i64),
        ("stride_k_token", _i64), ("stride_k_head", _i64),
        ("stride_v_token", _i64), ("stride_v_head", _i64),
        ("stride_o_token", _i64), ("stride_o_head", _i64),
        ("stride_q8_token", _i64), ("stride_q8_head", _i64),
        ("stride_k8_token", _i64), ("stride_k8_head", _i64),
        ("stride_v8_token", _i64), ("stride_v8_head", _i64),
        ("stride_bias_head", _i64), ("stride_bias_m", _i64), ("stride_bias_n", _i64),
        ("sm_scale", _f32),
        ("heads_q", _i32), ("heads_k", _i32), ("head_dim", _i32), ("batch", _i32),
        ("max_seqlen_q", _i32), ("max_seqlen_k", _i32),
        ("block_m", _i32), ("block_n", _i32), ("block_n_mask", _i32),
        ("blkq", _i32), ("blkk", _i32),
        ("causal", _i32),
        ("routing_mode", _i32),
        ("int8_use_fp16_v", _i32),
        ("q_quant_in_kernel", _i32),
    ]


class RmsNormParams(ctypes.Structure):
    """Mirror of ``tilemix_rmsnorm_params``."""

    _fields_ = [
        ("x", _vp), ("weight", _vp), ("out", _vp),
        ("rows", _i64), ("stride_x", _i64), ("stride_out", _i64),
        ("cols", _i32), ("eps", _f32),
    ]


class RotaryParams(ctypes.Structure):
    """Mirror of ``tilemix_rotary_params``."""

    _fields_ = [
        ("q", _vp), ("k", _vp), ("cos", _vp), ("sin", _vp), ("q_out", _vp), ("k_out", _vp),
        ("stride_q_batch", _i64), ("stride_q_head", _i64), ("stride_q_token", _i64),
        ("stride_k_batch", _i64), ("stride_k_head", _i64), ("stride_k_token", _i64),
        ("stride_cos_batch", _i64), ("stride_cos_token", _i64),
        ("stride_sin_batch", _i64), ("stride_sin_token", _i64),
        ("batch", _i32), ("tokens", _i32), ("heads_q", _i32), ("heads_k", _i32), ("head_dim", _i32),
    ]


EXPORTED_SYMBOLS = (
    "tilemix_quant_per_block_int8",
    "tilemix_attn_fwd",
    "tilemix_attn_fwd_debug",
    "tilemix_rms_norm_f16",
    "tilemix_rotary_f16",
    "tilemix_silu_mul_f16",
    "tilemix_abi_version",
    "tilemix_params_size",
    "tilemix_last_error",
)

_lib = None
_lock = threading.Lock()


class TileMixLibraryError(RuntimeError):
    """The native library is missing, stale or failed a call."""


def load_library(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load (once) and validate libtilemix_hip.so; raise if absent or mismatched."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib_path = Path(path) if path is not None else LIB_PATH
        if not lib_path.exists():
            raise TileMixLibraryError(
                f"{lib_path} is missing: build it with `python -m tilemix_amd.csrc.build` "
                "(or __graft_entry__.build()); there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(lib_path), mode=ctypes.RTLD_LOCAL)
        lib.tilemix_quant_per_block_int8.argtypes = [ctypes.POINTER(QuantParams), _vp]
        lib.tilemix_quant_per_block_int8.restype = ctypes.c_int
        lib.tilemix_attn_fwd.argtypes = [ctypes.POINTER(AttnParams), _vp]
        lib.tilemix_attn_fwd.restype = ctypes.c_int
        lib.tilemix_attn_fwd_debug.argtypes = [ctypes.POINTER(AttnParams), _vp, _vp, _i64, _i64, _vp]
        lib.tilemix_attn_fwd_debug.restype = ctypes.c_int
        lib.tilemix_rms_norm_f16.argtypes = [ctypes.POINTER(RmsNormParams), _vp]
        lib.tilemix_rms_norm_f16.restype = ctypes.c_int
        lib.tilemix_rotary_f16.argtypes = [ctypes.POINTER(RotaryParams), _vp]
        lib.tilemix_rotary_f16.restype = ctypes.c_int
        lib.tilemix_silu_mul_f16.argtypes = [_vp, _vp, _vp, _i64, _vp]
        lib.tilemix_silu_mul_f16.restype = ctypes.c_int
        lib.tilemix_abi_version.argtypes = []
        lib.tilemix_abi_version.restype = ctypes.c_int
        lib.tilemix_params_size.argtypes = [ctypes.c_int]
        lib.tilemix_params_size.restype = ctypes.c_int64
        lib.tilemix_last_error.argtypes = []
        lib.tilemix_last_error.restype = ctypes.c_char_p
        if lib.tilemix_abi_version() != ABI_VERSION:
            raise TileMixLibraryError(
                f"{lib_path}: ABI version {lib.tilemix_abi_version()} != {ABI_VERSION}; rebuild it"
            )
        for which, struct in ((0, QuantParams), (1, AttnParams), (2, RmsNormParams), (3, RotaryParams)):
            if lib.tilemix_params_size(which) != ctypes.sizeof(struct):
                raise TileMixLibraryError(
                    f"{lib_path}: {struct.__name__} size {lib.tilemix_params_size(which)} != "
                    f"{ctypes.sizeof(struct)} (header and binding disagree); rebuild it"
                )
        if path is None:
            _lib = lib
        return lib


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def current_stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check(status: int, lib: ctypes.CDLL) -> None:
    if status != 0:
        msg = lib.tilemix_last_error().decode(errors="replace")
        raise TileMixLibraryError(f"libtilemix_hip: {msg} (status {status})")


def quant_per_block_int8(params: QuantParams, device: torch.device) -> None:
    lib = load_library()
    with torch.cuda.device(device):
        _check(lib.tilemix_quant_per_block_int8(ctypes.byref(params), current_stream(device)), lib)


def attn_fwd(params: AttnParams, device: torch.device) -> None:
    lib = load_library()
    with torch.cuda.device(device):
        _check(lib.tilemix_attn_fwd(ctypes.byref(params), current_stream(device)), lib)


def attn_fwd_debug(params: AttnParams, qk_i32: torch.Tensor | None, qk_f16: torch.Tensor | None,
                   device: torch.device) -> None:
    lib = load_library()
    ref = qk_i32 if qk_i32 is not None else qk_f16
    with torch.cuda.device(device):
        _check(
            lib.tilemix_attn_fwd_debug(
                ctypes.byref(params), ptr(qk_i32), ptr(qk_f16), ref.stride(0), ref.stride(1),
                current_stream(device),
            ),
            lib,
        )


def rms_norm_f16(params: RmsNormParams, device: torch.device) -> None:
    lib = load_library()
    with torch.cuda.device(device):
        _check(lib.tilemix_rms_norm_f16(ctypes.byref(params), current_stream(device)), lib)


def rotary_f16(params: RotaryParams, device: torch.device) -> None:
    lib = load_library()
    with torch.cuda.device(device):
        _check(lib.tilemix_rotary_f16(ctypes.byref(params), current_stream(device)), lib)


def silu_mul_f16(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor) -> None:
    lib = load_library()
    device = gate.device
    with torch.cuda.device(device):
        _check(lib.tilemix_silu_mul_f16(ptr(gate), ptr(up), ptr(out), gate.numel(), current_stream(device)), lib)
