"""ctypes binding of libnsmoe.so (the C ABI declared in include/nsmoe.h).

The library is loaded lazily on first use.  A missing or unloadable library is an
error, never a silent fallback: `lib()` raises NativeLibraryError and every HIP op in
moe_kernel.py goes through it.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnsmoe.so"

BF16, F16, F32 = 0, 1, 2
ROUTE_PROBS, ROUTE_NORMALIZE, ROUTE_LOGITS16 = 1, 2, 4
BLOCK_PACK, BLOCK_SAVE_ACT, BLOCK_NORM = 8, 16, 32
ABI_VERSION = 8

# Every symbol include/nsmoe.h declares, with (restype, argtypes).
_vp, _i32, _i64, _sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t


class ExpertsArgs(ctypes.Structure):
    """Mirror of `nsmoe_experts_args`."""

    _fields_ = [
        ("dtype", _i32), ("activation", _i32), ("n_tokens", _i64),
        ("d_model", _i32), ("d_hidden", _i32), ("n_experts", _i32), ("n_shared", _i32),
        ("top_k", _i32), ("reserved0", _i32), ("l_cap", _i64),
        ("x", _vp), ("w_in", _vp), ("w_out", _vp), ("b_in", _vp), ("b_out", _vp),
        ("w_sh_in", _vp), ("w_sh_out", _vp), ("b_sh_in", _vp), ("b_sh_out", _vp),
        ("topk_w", _vp), ("sorted_ids", _vp), ("pad_offsets", _vp), ("counts", _vp),
        ("w_in_packed", _vp), ("w_out_packed", _vp),
    ]


class ExpertsGrads(ctypes.Structure):
    """Mirror of `nsmoe_experts_grads`."""

    _fields_ = [(n, _vp) for n in (
        "dx", "dw_in", "dw_out", "dw_sh_in", "dw_sh_out", "dtopk_w",
        "db_in", "db_out", "db_sh_in", "db_sh_out")]


class AttnArgs(ctypes.Structure):
    """Mirror of `nsmoe_attn_args`."""

    _fields_ = [
        ("dtype", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("batch", _i64), ("seq_len", _i64), ("ld", _i32), ("window", _i32),
        ("eps", ctypes.c_float), ("reserved", _i32),
        ("qkv", _vp), ("q_gamma", _vp), ("k_gamma", _vp), ("cos", _vp), ("sin", _vp),
        ("out", _vp),
    ]


class BlockNorm(ctypes.Structure):
    """Mirror of `nsmoe_block_norm`."""

    _fields_ = [("weight", _vp), ("grad_weight", _vp), ("eps", ctypes.c_float),
                ("reserved", _i32)]


SIGNATURES = {
    "nsmoe_last_error": (ctypes.c_char_p, []),
    "nsmoe_launch_count": (ctypes.c_uint64, []),
    "nsmoe_abi_version": (_i32, []),
    "nsmoe_timing_enable": (ctypes.c_int, [_i32]),
    "nsmoe_timing_read": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(_i64)]),
    "nsmoe_set_option": (ctypes.c_int, [ctypes.c_char_p, _i64]),
    "nsmoe_get_option": (_i64, [ctypes.c_char_p]),
    "nsmoe_route_fwd": (ctypes.c_int, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "nsmoe_route_bwd": (ctypes.c_int, [_vp, _vp, _vp, _i32, _vp, _vp, _vp, ctypes.c_float, _i64,
                                       _i32, _i32, _i32, _vp, _vp]),
    "nsmoe_balance_loss_workspace_size": (_sz, [_i64, _i32]),
    "nsmoe_balance_loss": (ctypes.c_int, [_vp, _vp, _i64, _i32, ctypes.c_float, _vp, _vp, _sz,
                                          _vp]),
    "nsmoe_align_m": (_i64, []),
    "nsmoe_dispatch_l_cap": (_i64, [_i64, _i32]),
    "nsmoe_dispatch_workspace_size": (_sz, [_i64, _i32]),
    "nsmoe_dispatch": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "nsmoe_dispatch_noalloc": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                              _vp]),
    "nsmoe_pack_sizes": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), ctypes.POINTER(_sz),
                                        ctypes.POINTER(_sz)]),
    "nsmoe_pack_weights": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), _vp, _vp, _vp]),
    "nsmoe_experts_fwd_workspace_size": (_sz, [ctypes.POINTER(ExpertsArgs)]),
    "nsmoe_experts_fwd": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), _vp, _vp, _vp, _sz, _vp]),
    "nsmoe_experts_bwd_workspace_size": (_sz, [ctypes.POINTER(ExpertsArgs)]),
    "nsmoe_experts_bwd": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), _vp, _vp,
                                         ctypes.POINTER(ExpertsGrads), _vp, _sz, _vp]),
    "nsmoe_block_saved_layout": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), _i32,
                                                ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "nsmoe_block_fwd_workspace_size": (_sz, [ctypes.POINTER(ExpertsArgs), _i32]),
    "nsmoe_block_fwd": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), ctypes.POINTER(BlockNorm),
                                       _vp, _vp, _vp, _i32, ctypes.c_float, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _sz, _vp]),
    "nsmoe_block_bwd_workspace_size": (_sz, [ctypes.POINTER(ExpertsArgs), _i32, _i32]),
    "nsmoe_block_bwd": (ctypes.c_int, [ctypes.POINTER(ExpertsArgs), ctypes.POINTER(BlockNorm),
                                       _vp, _i32, ctypes.c_float, _vp, _vp, _vp, _vp, _vp,
                                       ctypes.POINTER(ExpertsGrads), _vp, _vp, _vp, _vp, _sz,
                                       _vp]),
    "nsmoe_rms_norm": (ctypes.c_int, [_i32, _vp, _vp, ctypes.c_float, _i64, _i32, _vp, _vp,
                                      _vp]),
    "nsmoe_attn_prefill": (ctypes.c_int, [ctypes.POINTER(AttnArgs), _vp]),
    "nsmoe_cross_entropy_rows": (ctypes.c_int, [_i32, _vp, _i64, _i64, _i32, _vp, _i64, _vp,
                                                _vp, _vp, _vp]),
}

# Parts of the block's `saved` buffer (NSMOE_SAVED_* in nsmoe.h).
SAVED_TOPK_W, SAVED_PROBS, SAVED_INV, SAVED_ACT, SAVED_XN, SAVED_RSTD = 0, 1, 6, 7, 8, 9
BLOCK_NSAVED = 10


class NativeLibraryError(RuntimeError):
    """libnsmoe.so is missing, fails to load, or a call into it failed."""


_LIB: "ctypes.CDLL | None" = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises NativeLibraryError if it cannot be loaded."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise NativeLibraryError(
            f"{LIB_PATH} not found: build it with `python -m nanospeaker_amd.build` "
            "(hipcc, gfx950).  The MoE kernel path has no fallback.")
    try:
        handle = ctypes.CDLL(str(LIB_PATH))
    except OSError as e:  # pragma: no cover - depends on the machine
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = res, args
    if handle.nsmoe_abi_version() != ABI_VERSION:
        raise NativeLibraryError("libnsmoe.so ABI version mismatch; rebuild it")
    _LIB = handle
    return handle


def available() -> bool:
    try:
        lib()
        return True
    except NativeLibraryError:
        return False


def check(rc: int, what: str) -> None:
    """Raises with the library's error string when a call returned non-zero."""
    if rc != 0:
        msg = lib().nsmoe_last_error().decode(errors="replace")
        raise NativeLibraryError(f"{what} failed ({rc}): {msg}")


def launch_count() -> int:
    return int(lib().nsmoe_launch_count())


def timing_enable(capacity: int) -> None:
    """Start recording HIP event pairs around the library's kernels (0 stops)."""
    check(lib().nsmoe_timing_enable(capacity), "nsmoe_timing_enable")


def set_option(name: str, value: int) -> None:
    """A process-wide tuning option of the library (nsmoe_set_option; 0 = its default)."""
    check(lib().nsmoe_set_option(name.encode(), int(value)), f"nsmoe_set_option({name})")


def get_option(name: str) -> int:
    v = int(lib().nsmoe_get_option(name.encode()))
    if v < 0:
        raise NativeLibraryError(f"unknown option {name!r}")
    return v


def timing_read(kernel: str) -> "tuple[float, int]":
    """(summed milliseconds, launches) recorded for `kernel` since timing_enable."""
    ms, n = ctypes.c_double(), ctypes.c_int64()
    check(lib().nsmoe_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)),
          "nsmoe_timing_read")
    return ms.value, n.value
