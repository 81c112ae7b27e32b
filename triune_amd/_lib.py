"""ctypes binding of libtriune_hip.so (the C ABI declared in include/triune_hip.h).

The loader follows the reference's native-library convention (one shared library beside the
Python package, found by a fixed file name and bound with ctypes argtypes at load time:
triune/ops/_c_bridge.py:48-149), but there is no silent fallback: if the library is missing or
a call fails, a TriuneHipError is raised.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtriune_hip.so"
ABI_VERSION = 3

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
FLAG_TAIL_UNCLAMPED = 0x1
FLAG_SEG_SHIFT = 8
FLAG_BWD_ACC_QKG = 0x2
FLAG_BWD_ACC_V = 0x4
BETA_NONE, BETA_HEAD, BETA_KEY, BETA_VALUE = 0, 1, 2, 3

_DT = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float16: DT_F16}

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

_LIB = None


class TriuneHipError(RuntimeError):
    """Raised when libtriune_hip.so is missing or one of its entry points returns an error."""


def _bind(lib):
    sig = {
        "triune_hip_abi_version": ([], _i),
        "triune_hip_error_string": ([_i], ctypes.c_char_p),
        "triune_hip_set_output_kernel_events": ([_vp, _vp], _i),
        "triune_hip_gla_decode_step": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _vp, _vp, _i64, _vp, _i, _i64, _i64, _i, _i, _vp],
            _i,
        ),
        "triune_hip_last_error": ([], _i),
        "launch_gla_decode_step": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp], None),
        "triune_gla_recurrent_step_f32": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i], None),
        "triune_hip_gla_prefill_workspace_size": ([_i64, _i64, _i64, _i, _i, _i], _sz),
        "triune_hip_gla_prefill": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i, _i, _vp, _sz, _vp],
            _i,
        ),
        "triune_hip_gla_prefill_prep": (
            [_vp, _vp, _vp, _vp, _i, _i64p, _vp, _vp, _i64, _i, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _vp, _sz,
             _vp],
            _i,
        ),
        "triune_hip_gla_prefill_onepass_supported": ([_i64, _i64, _i64, _i, _i, _i, _i, _i], _i),
        "triune_hip_gla_prefill_onepass_workspace_size": ([_i64, _i64, _i64, _i], _sz),
        "triune_hip_gla_prefill_onepass_ctrl_size": ([_i64, _i64, _i64, _i], _sz),
        "triune_hip_gla_prefill_onepass": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _vp, _i64, _i, _i, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i,
             _vp, _sz, _vp, _sz, _vp],
            _i,
        ),
        "triune_hip_gla_prefill_noalloc_max_bytes": ([], _sz),
        "triune_hip_gla_prefill_noalloc": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i, _i, _vp],
            _i,
        ),
        "triune_hip_gla_prefill_varlen_workspace_size": ([_i64, _i64, _i64, _i, _i, _i], _sz),
        "triune_hip_gla_prefill_varlen": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _i64, _i64, _vp, _vp, _i, _vp, _i64, _i, _i, _i, _vp, _sz, _vp],
            _i,
        ),
        "triune_hip_recurrent_scan_fwd": ([_vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _i64, _i64, _i64, _i, _i, _vp], _i),
        "triune_hip_gla_prefill_varlen_pool": (
            [_vp, _vp, _vp, _vp, _i, _i, _i64p, _vp, _i64, _i64, _vp, _vp, _i64, _vp, _i, _i64, _i, _i, _i, _vp, _sz,
             _vp],
            _i,
        ),
        "triune_hip_gla_prefill_bwd_workspace_size": ([_i64, _i64, _i64, _i, _i, _i], ctypes.c_size_t),
        "triune_hip_gla_prefill_bwd": (
            [_vp, _vp, _vp, _vp, _i, _i, _vp, _i64p, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp,
             _i64, _i64, _i64, _i, _i, _i, _vp, ctypes.c_size_t, _vp],
            _i,
        ),
        "triune_hip_recurrent_scan_bwd": (
            [_vp, _i, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _i, _i64, _i64, _i64, _i, _i, _vp],
            _i,
        ),
        "triune_hip_gdn_prefill": (
            [_vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i, _vp],
            _i,
        ),
        "triune_hip_gla_qkvg_prep": ([_vp, _vp, _i, _i64p, _vp, _vp, _i, _i64, _i, _i64, _i64, _i64, _i, _vp], _i),
        "triune_hip_gla_fused_decode_step": (
            [_vp, _i, _i64p, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _i, _i64p, _i64, _i64, _i, _vp],
            _i,
        ),
        "triune_hip_gla_fused_decode_step_slots": (
            [_vp, _i, _i64p, _vp, _vp, _i, _i, _vp, _i, _vp, _i64, _vp, _i, _i64p, _i64, _i64, _i, _vp],
            _i,
        ),
        "triune_hip_gdn_prefill_chunked_workspace_size": ([_i64, _i64, _i64, _i, _i], _sz),
        "triune_hip_gdn_prefill_chunked": (
            [_vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i, _vp, _sz,
             _vp],
            _i,
        ),
        "triune_hip_gdn_bwd_workspace_size": ([_i64, _i64, _i64, _i, _i, _i], _sz),
        "triune_hip_gdn_bwd": (
            [_vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
             _i64, _i64, _i, _i, _vp, _sz, _vp],
            _i,
        ),
        "triune_hip_gdn_prefill_scalar_decay_workspace_size": ([_i64, _i64, _i64, _i, _i], _sz),
        "triune_hip_gdn_prefill_scalar_decay": (
            [_vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i64p, _vp, _vp, _i, _vp, _i64, _i64, _i64, _i, _i, _vp, _sz,
             _vp],
            _i,
        ),
    }
    for name, (argtypes, restype) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


EXPORTS = (
    "triune_hip_abi_version",
    "triune_hip_error_string",
    "triune_hip_set_output_kernel_events",
    "triune_hip_gla_decode_step",
    "triune_hip_last_error",
    "launch_gla_decode_step",
    "triune_gla_recurrent_step_f32",
    "triune_hip_gla_prefill_workspace_size",
    "triune_hip_gla_prefill",
    "triune_hip_gla_prefill_prep",
    "triune_hip_gla_prefill_onepass_supported",
    "triune_hip_gla_prefill_onepass_workspace_size",
    "triune_hip_gla_prefill_onepass_ctrl_size",
    "triune_hip_gla_prefill_onepass",
    "triune_hip_gla_prefill_noalloc_max_bytes",
    "triune_hip_gla_prefill_noalloc",
    "triune_hip_gla_prefill_varlen_workspace_size",
    "triune_hip_gla_prefill_varlen",
    "triune_hip_recurrent_scan_fwd",
    "triune_hip_gla_prefill_varlen_pool",
    "triune_hip_gla_prefill_bwd_workspace_size",
    "triune_hip_gla_prefill_bwd",
    "triune_hip_recurrent_scan_bwd",
    "triune_hip_gdn_prefill",
    "triune_hip_gdn_prefill_chunked_workspace_size",
    "triune_hip_gdn_prefill_chunked",
    "triune_hip_gdn_prefill_scalar_decay_workspace_size",
    "triune_hip_gdn_prefill_scalar_decay",
    "triune_hip_gdn_bwd_workspace_size",
    "triune_hip_gdn_bwd",
    "triune_hip_gla_qkvg_prep",
    "triune_hip_gla_fused_decode_step",
    "triune_hip_gla_fused_decode_step_slots",
)


def lib():
    """The loaded library (raises TriuneHipError if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.is_file():
            raise TriuneHipError(
                f"{LIB_PATH} is missing: build it with `python -m triune_amd.build` (hipcc, gfx950)"
            )
        _LIB = _bind(ctypes.CDLL(str(LIB_PATH)))
        if _LIB.triune_hip_abi_version() != ABI_VERSION:
            raise TriuneHipError("libtriune_hip.so ABI version mismatch")
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().triune_hip_error_string(rc).decode()
        raise TriuneHipError(f"{what} failed: {msg} (code {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def strides(*pairs) -> ctypes.Array:
    flat = [int(s) for p in pairs for s in p]
    return (ctypes.c_int64 * len(flat))(*flat)


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_CTRL: dict = {}


def onepass_ctrl(device: torch.device, nbytes: int) -> torch.Tensor:
    """The control block of triune_hip_gla_prefill_onepass for calls on the current stream of
    `device`: zero when first made, left ready for the next call by every call, one per (device,
    stream) so that calls on different streams never share one.  Grown (as a new zeroed block)
    when a call needs more flags than the block holds."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    blk = _CTRL.get(key)
    if blk is None or blk.numel() < nbytes:
        blk = torch.zeros(max(int(nbytes), 4096), device=device, dtype=torch.uint8)
        _CTRL[key] = blk
    return blk
