"""ctypes binding of the gfx950 kernel library (``include/trainscale_amd.h``).

The library is loaded lazily on first use. There is no fallback: if the
shared object is missing or a GPU tensor is not on a ROCm device, the call
raises. Build the library with ``python -m trainscale_amd.build``.
"""
from __future__ import annotations

import contextlib
import ctypes
import re
import threading
from pathlib import Path

import torch

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "lib" / "libtrainscale_amd.so"
HEADER_PATH = PKG_DIR.parent / "include" / "trainscale_amd.h"

TS_F32, TS_BF16, TS_F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: TS_F32, torch.bfloat16: TS_BF16, torch.float16: TS_F16}

STATUS_NAMES = {
    0: "TS_OK",
    -1: "TS_ERR_INVALID_ARGUMENT",
    -2: "TS_ERR_UNSUPPORTED_DTYPE",
    -3: "TS_ERR_SHAPE",
    -4: "TS_ERR_WORKSPACE",
    -5: "TS_ERR_LAUNCH",
    -6: "TS_ERR_DEVICE",
}


class KernelLibraryError(RuntimeError):
    """The native library is missing or cannot be loaded."""


class KernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, what: str, code: int, message: str):
        super().__init__(f"{what} failed with {STATUS_NAMES.get(code, code)}: {message}")
        self.code = code


P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# argtypes of every exported entry point, in header order
SIGNATURES = {
    "ts_last_error": ([], ctypes.c_char_p),
    "ts_version": ([], ctypes.c_char_p),
    "ts_rmsnorm_fwd": ([P, I64, I32, P, I32, P, I64, P, I64, I64, F32, I32, P], I32),
    "ts_add_rmsnorm_fwd": ([P, I64, P, I64, I32, P, I32, P, I64, P, I64, P, I64, I64, F32, I32, P],
                           I32),
    "ts_rmsnorm_bwd_workspace_size": ([I64, I64], SZ),
    "ts_rmsnorm_bwd": ([P, I64, P, I64, I32, P, I32, P, P, I64, P, P, SZ, I64, I64, P], I32),
    "ts_rmsnorm_bwd_noalloc_max_bytes": ([], SZ),
    "ts_rmsnorm_bwd_noalloc": ([P, I64, P, I64, I32, P, I32, P, P, I64, P, I64, I64, P], I32),
    "ts_rope_apply": (
        [P, P, I64, I64, I64, I64, I64, I64, I64,   # q
         P, P, I64, I64, I64, I64, I64, I64, I64,   # k
         I32, I64, I64, I64,                        # dtype, B, S, D
         P, P, I32, I64, I64,                       # tables
         P, F32, F32,                               # inv_freq (host), pos_div, angle_scale
         P, I64, I64, I64,                          # position_ids, strides, offset
         I32, I32, P],                              # interleaved, backward, stream
        I32),
    "ts_ce_fwd": ([P, I64, I32, P, I64, I64, I64, F32, F32, F32, P, P, P], I32),
    "ts_ce_bwd": ([P, I64, I32, P, P, P, I64, F32, P, I64, I32, I64, I64, I64, F32, F32, F32, P],
                  I32),
    "ts_ce_fwd_bwd": ([P, I64, I32, P, I64, I64, I64, F32, F32, F32, P, I64, F32, P, P, P, I64,
                       I32, P], I32),
    "ts_ce_vocab_shard_stats": ([P, I64, I32, P, I64, I64, I64, P, P], I32),
    "ts_ce_vocab_merge": ([P, I64, I64, I64, I64, F32, P, P, P], I32),
    "ts_ce_vocab_shard_bwd": ([P, I64, I32, P, P, P, F32, I64, I64, I64, F32, P, I64, I32, P],
                              I32),
    "ts_flce_vocab_workspace_size": ([I64, I64], SZ),
    "ts_flce_vocab_fwd": ([P, I64, P, I64, P, I64, I64, I64, I64, P, P, SZ, P], I32),
    "ts_flce_vocab_bwd": ([P, I64, P, I64, P, I64, I64, I64, I64, P, I64, I64, I32, P, P, P, P,
                           P, P, SZ, P], I32),
    "ts_flce_workspace_size": ([I64, I64, I64, I64, I32], SZ),
    "ts_flce_fwd_bwd": ([P, I64, P, I64, P, I64, I64, I64, I64, I32, P, P, P, P, P, I64, I32, P,
                         SZ, P], I32),
    "ts_flce_forward_workspace_size": ([I64, I64], SZ),
    "ts_flce_forward": ([P, I64, P, I64, P, I64, I64, I64, I64, I32, F32, F32, F32, P, P, P, P,
                         SZ, P], I32),
    "ts_flce_backward_workspace_size": ([I64, I64, I64, I64], SZ),
    "ts_flce_backward": ([P, I64, P, I64, P, I64, I64, I64, I64, I32, F32, F32, F32, P, P, I64,
                          P, P, I64, P, SZ, P], I32),
    "ts_flce_forward_keep": ([P, I64, P, I64, P, I64, I64, I64, I64, I32, F32, F32, F32, P, P, P,
                              P, P, SZ, P], I32),
    "ts_flce_backward_kept_workspace_size": ([I64], SZ),
    "ts_flce_backward_kept": ([P, I64, P, I64, P, I64, I64, I64, I64, I32, F32, F32, F32, P, P,
                               I64, P, P, P, P, SZ, P], I32),
    "ts_scale_inplace": ([P, I64, I32, P, P], I32),
    "ts_swiglu_fwd": ([P, P, P, I64, I32, P], I32),
    "ts_swiglu_bwd": ([P, P, P, P, P, I64, I32, P], I32),
    "ts_rescale_inplace": ([P, I64, I32, P, P, P, P], I32),
    "ts_stream_copy": ([P, P, I64, P], I32),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def header_symbols() -> list[str]:
    """Names of the functions declared in include/trainscale_amd.h."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(ts_[a-z0-9_]+)\s*\(",
                      text, flags=re.M)


def load() -> ctypes.CDLL:
    """Loads the library (once) and declares the ctypes signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelLibraryError(
                f"{LIB_PATH} is missing: build it with `python -m trainscale_amd.build`")
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise KernelLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def last_error() -> str:
    return load().ts_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != 0:
        raise KernelError(what, status, last_error())


# torch's current-stream query without building a Stream object (the form torch's
# own kernel launchers use); the public API where a build lacks it
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    """The HIP stream torch is currently using on `device`."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def on_device(device: torch.device):
    """A context under which `device` is the current device, for a launch on its stream
    (a no-op context when it already is, the common case)."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def require_gpu(what: str, *tensors: torch.Tensor | None) -> torch.device:
    """Raises unless every given tensor lives on the same ROCm GPU."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"{what}: the MI355X kernel layer needs GPU tensors (got a tensor on {t.device}); "
                "there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors are on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{what}: no tensor given")
    if torch.version.hip is None:
        raise RuntimeError(f"{what}: this torch build is not ROCm")
    return dev


def dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype} (float32/bfloat16/float16)") from None
