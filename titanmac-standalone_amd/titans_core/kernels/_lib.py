"""Loader and ctypes signatures of libtmac.so (the C ABI declared in include/tmac.h).

The library is hand-written HIP for gfx950. It is loaded lazily on first use;
a missing or mismatched library raises ImportError at that point, and there is
no fallback implementation: every hot-path op either runs the HIP kernel or
raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path

import torch  # the HIP runtime torch loads (libamdhip64.so.7) also serves libtmac.so

ABI_VERSION = 8

F32, BF16, F16 = 0, 1, 2
EPI_NONE, EPI_GELU = 0, 1
PATTERN_BAND, PATTERN_BLOCKWIN = 0, 1
MEM_CLIP_MEMORY, MEM_CLIP_KERNEL = 0, 1
MEM_MAX_TENSORS = 16

_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_PKG_ROOT = Path(__file__).resolve().parents[2]  # titanmac-standalone_amd/
DEFAULT_LIB_PATH = _PKG_ROOT / "lib" / "libtmac.so"

_lock = threading.Lock()
_lib = None

_i, _i64, _u64, _vp, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes (every function returns int except tmac_status_string and
# tmac_wattn_mask_workspace, set below)
SIGNATURES = {
    "tmac_abi_version": [],
    "tmac_bell_sample_col_idx": [_u64, _i, _i, _i, _vp],
    "tmac_bell_validate": [_vp, _i, _i, _i],
    "tmac_bell_transpose": [_vp, _i, _i, _i, _vp, _vp, _vp, _vp],
    "tmac_bell_group_schedule": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i, ctypes.POINTER(_i),
                                 ctypes.POINTER(_i)],
    "tmac_bell_group_tile_order": [_vp, _i, _i, _vp, _i, ctypes.POINTER(_i)],
    "tmac_bell_fwd_grouped": [_vp, _i64, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _vp, _vp, _i64, _i, _i,
                              _i, _i, _i, _i, _vp],
    "tmac_bell_fwd_grouped_gelu_aux": [_vp, _i64, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _vp, _vp, _i64,
                                       _vp, _i64, _i, _i, _i, _i, _i, _vp],
    "tmac_bell_fwd": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i, _i, _i, _i, _i, _i, _vp],
    "tmac_bell_fwd_gelu_aux": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i, _i, _i,
                               _i, _i, _vp],
    "tmac_bell_gelu_bwd_workspace": [_i, _i, ctypes.POINTER(_sz)],
    "tmac_bell_gelu_bwd": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _sz, _i, _i, _i, _vp],
    "tmac_bell_bias_grad": [_vp, _i64, _vp, _vp, _sz, _i, _i, _i, _vp],
    "tmac_bell_dx": [_vp, _i64, _vp, _vp, _vp, _i64, _i, _i, _i, _i, _i, _vp],
    "tmac_bell_sddmm_workspace": [_i, _i, _i, _i, ctypes.POINTER(_sz)],
    "tmac_bell_sddmm": [_vp, _i64, _vp, _i64, _vp, _vp, _i, _vp, _sz, _i, _i, _i, _i, _i, _vp],
    "tmac_wattn_tile_kinds": [_i, _i, _i, _i, _i, _i, _i, _i, _vp],
    "tmac_wattn_schedule": [_i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, ctypes.POINTER(_i)],
    "tmac_wattn_launch_order": [_vp, _i, _vp, ctypes.POINTER(_i)],
    "tmac_wattn_mask_spans": [_i, _i, _i, _i, _i, _i, _vp, _vp],
    "tmac_wattn_fwd": [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                       _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp, _i,
                       _i, _vp],
    "tmac_wattn_schedule_kv": [_i, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _i, ctypes.POINTER(_i)],
    "tmac_wattn_bwd": [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                       _vp, _i64p, _vp, _i64p, _vp, _i64p,
                       _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp, _i,
                       _vp, _vp, _vp, _i, _i, _vp],
    "tmac_wattn_bwd_noalloc": [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                               _vp, _i64p, _vp, _i64p, _vp, _i64p,
                               _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp,
                               _i, _vp, _vp, _vp, _i, _i, _vp],
    "tmac_wattn_fwd_ex": [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp,
                          _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp, _i,
                          _i, _vp, _vp],
    "tmac_wattn_bwd_ex": [_vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _i64p, _vp, _vp,
                          _vp, _i64p, _vp, _i64p, _vp, _i64p,
                          _i, _i, _i, _i, _i, _i, _i, _i, _i, ctypes.c_float, _vp, _vp, _vp, _i,
                          _vp, _vp, _vp, _i, _i, _vp, _vp],
    "tmac_wattn_mask_lists": [_vp, _i, _vp],
    "tmac_wattn_mask_grad_reduce": [_vp, _i, _i, _i, _i, _i, _vp, _vp],
    "tmac_dwconv_causal": [_vp, _i64, _vp, _vp, _i64, _i, _i, _i, _i, _i, _vp],
    "tmac_dwconv_causal_bwd_workspace": [_i, _i, _i, _i, ctypes.POINTER(_sz)],
    "tmac_dwconv_causal_bwd": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _sz, _i, _i, _i, _i,
                               _i, _vp],
    "tmac_rmsnorm_fwd": [_vp, _i64, _vp, _vp, _i64, _vp, _i, _i, ctypes.c_float, _i, _vp],
    "tmac_rmsnorm_bwd_workspace": [_i, _i, ctypes.POINTER(_sz)],
    "tmac_rmsnorm_bwd": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _sz, _i, _i, _i, _vp],
    "tmac_mem_update_workspace": [_i64p, _i, ctypes.POINTER(_sz)],
    "tmac_mem_update": [_vp, _vp, _vp, _vp, _i64p, _i, _vp, _vp, _vp, ctypes.c_float,
                        ctypes.c_float, _i, _vp, _vp, _sz, _i, _vp],
    "tmac_silu_bwd": [_vp, _vp, _vp, _i64, _i, _vp],
    "tmac_mse_grad": [_vp, _vp, _vp, _i64, ctypes.c_float, _i, _vp],
}


def lib_path() -> Path:
    return Path(os.environ.get("TMAC_LIB", DEFAULT_LIB_PATH))


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not path.exists():
                raise ImportError(
                    f"libtmac.so not found at {path}; build it with "
                    f"`python titanmac-standalone_amd/build.py` (hipcc, gfx950)")
            L = ctypes.CDLL(str(path))
            for name, args in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = _i
            L.tmac_wattn_mask_workspace.argtypes = [_i, _i, _i]
            L.tmac_wattn_mask_workspace.restype = _sz
            L.tmac_status_string.argtypes = [_i]
            L.tmac_status_string.restype = ctypes.c_char_p
            got = L.tmac_abi_version()
            if got != ABI_VERSION:
                raise ImportError(f"libtmac.so ABI {got} != expected {ABI_VERSION}; rebuild it")
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    """Raise for a non-zero return code: ValueError for argument errors (the
    reference's convention for invalid configurations and masks), RuntimeError
    for HIP launch errors."""
    if rc == 0:
        return
    msg = lib().tmac_status_string(rc).decode()
    if rc < 0:
        raise ValueError(f"{what}: {msg} (tmac status {rc})")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def stream_ptr(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on `device` (the same
    handle as torch.cuda.current_stream(device).cuda_stream, without building
    a Stream object on every launch)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def ptr(t: torch.Tensor | None) -> int:
    """Device address of t (0 for None), for a c_void_p argument."""
    return 0 if t is None else t.data_ptr()


_NO_GUARD = contextlib.nullcontext()


def device_guard(device: torch.device):
    """torch.cuda.device(device), or nothing when it is already the current device."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(device)


_PLAIN = (torch.Tensor, torch.nn.Parameter)


def direct_call(*tensors: torch.Tensor | None) -> bool:
    """Whether an op may run its implementation directly instead of through the
    torch.library dispatcher: eager mode (no torch.compile tracing), plain
    tensors (no fake or wrapper subclasses) and no autograd graph to record.
    The dispatcher adds several µs of host time per call, more than many of
    these kernels take on the GPU."""
    if torch.compiler.is_compiling():
        return False
    grad = torch.is_grad_enabled()
    for t in tensors:
        if t is None:
            continue
        if type(t) not in _PLAIN or (grad and t.requires_grad):
            return False
    return True


def require_device(*tensors: torch.Tensor, what: str) -> torch.device:
    """All tensors on the same ROCm device; returns it. No CPU path exists."""
    dev = tensors[0].device
    if dev.type != "cuda":
        raise RuntimeError(
            f"{what}: the TitanMAC hot path runs only on the GPU (HIP kernels for gfx950); "
            f"got a tensor on {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} and {t.device})")
    return dev
