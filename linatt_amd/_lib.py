"""ctypes binding of ``liblinatt_hip.so`` (declared in ``include/linatt_hip.h``).

The library is required: importing an op module without it raises
``ImportError`` naming the build command.  There is no CPU or PyTorch
fallback on the product path.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.environ.get(
    "LINATT_LIB",
    os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "liblinatt_hip.so"),
)

ABI_VERSION = 3

LINATT_FLOAT32, LINATT_BFLOAT16, LINATT_FLOAT16 = 0, 1, 2
LINATT_KATA_CONCAT, LINATT_KATA_SUM = 0, 1
LINATT_KATA_PACKED_STATE = 4  # OR-ed into a linatt_kata_gen_* variant
STATUS = {0: "LINATT_OK", -1: "LINATT_EINVAL", -2: "LINATT_EUNSUPPORTED", -3: "LINATT_ELAUNCH"}

_DTYPES = {torch.float32: LINATT_FLOAT32, torch.bfloat16: LINATT_BFLOAT16, torch.float16: LINATT_FLOAT16}

_lock = threading.Lock()
_lib = None

_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/linatt_hip.h
SIGNATURES = {
    "linatt_abi_version": (_i, []),
    "linatt_last_error": (ctypes.c_char_p, []),
    "linatt_kata_supported": (_i, [_i, _i, _i, _i, _i, _i]),
    "linatt_kata_fwd": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _i, _i, _vp]),
    "linatt_kata_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "linatt_kata_bwd": (_i, [_vp] * 10 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_kata_bwd_dq": (_i, [_vp] * 10 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_kata_bwd_decay": (_i, [_vp] * 12 + [_i] * 7 + [_f, _i, _vp]),
    "linatt_kata_bwd_dkdv": (_i, [_vp] * 10 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_kata_bwd_noalloc": (_i, [_vp] * 9 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_noalloc_scratch_bytes": (_sz, []),
    "linatt_kata_fwd_onorm": (_i, [_vp] * 7 + [_f, _vp, _vp] + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_kata_bwd_onorm_workspace_bytes": (_sz, [_i] * 5),
    "linatt_kata_fwd_num": (_i, [_vp] * 5 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_kata_bwd_onorm": (_i, [_vp] * 15 + [_i] * 7 + [_f, _i, _i, _vp]),
    "linatt_delta_supported": (_i, [_i, _i, _i]),
    "linatt_delta_ctx_bytes": (_sz, [_i] * 6),
    "linatt_delta_bwd_workspace_bytes": (_sz, [_i] * 6),
    "linatt_delta_fwd": (_i, [_vp] * 9 + [_i] * 5 + [_f, _i, _vp]),
    "linatt_delta_bwd": (_i, [_vp] * 16 + [_i] * 5 + [_f, _i, _vp]),
    "linatt_delta_fwd_stages": (_i, [_vp] * 9 + [_i] * 5 + [_f, _i, _i, _vp]),
    "linatt_delta_bwd_stages": (_i, [_vp] * 16 + [_i] * 5 + [_f, _i, _i, _vp]),
    "linatt_l2norm_fwd": (_i, [_vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "linatt_l2norm_bwd": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "linatt_kata_state_supported": (_i, [_i, _i, _i, _i]),
    "linatt_kata_gen_state_rows": (_i, [_i, _i, _i]),
    "linatt_kata_gen_decode": (_i, [_vp] * 7 + [_i] * 6 + [_f, _f, _i, _vp]),
    "linatt_kata_gen_decode_workspace_bytes": (_sz, [_i] * 5),
    "linatt_kata_decode_workspace_bytes": (_sz, [_i] * 5),
    "linatt_kata_decode_step_split": (_i, [_vp] * 7 + [_sz] + [_i] * 6 + [_f, _f, _i, _vp]),
    "linatt_kata_gen_decode_split": (_i, [_vp] * 8 + [_sz] + [_i] * 6 + [_f, _f, _i, _vp]),
    "linatt_kata_gen_readout": (_i, [_vp] * 6 + [_i] * 7 + [_f, _f, _i, _vp]),
    "linatt_kata_gen_update": (_i, [_vp] * 5 + [_i] * 8 + [_f, _i, _vp]),
    "linatt_kata_prefill_workspace_bytes": (_sz, [_i] * 8),
    "linatt_kata_prefill": (_i, [_vp] * 8 + [_i] * 6 + [_f, _f, _i, _i, _i, _vp]),
    "linatt_kata_prefill_state": (_i, [_vp] * 10 + [_i] * 6 + [_f, _f, _i, _i, _i, _vp]),
    "linatt_kata_decode_step": (_i, [_vp] * 6 + [_i] * 5 + [_f, _f, _i, _vp]),
    "linatt_kata_prefill_state_packed": (_i, [_vp] * 10 + [_i] * 6 + [_f, _f, _i, _i, _i, _vp]),
    "linatt_kata_decode_step_packed": (_i, [_vp] * 6 + [_i] * 5 + [_f, _f, _i, _vp]),
    "linatt_short_conv_fwd": (_i, [_vp] * 6 + [_i] * 6 + [_vp]),
    "linatt_short_conv_bwd_workspace_bytes": (_sz, [_i] * 4),
    "linatt_short_conv_bwd": (_i, [_vp] * 9 + [_i] * 6 + [_vp]),
    "linatt_rope": (_i, [_vp] * 2 + [_i] * 5 + [_f] + [_i] * 4 + [_vp]),
    "linatt_qk_prologue_fwd": (_i, [_vp] * 7 + [_i] * 7 + [_f, _i, _i, _f, _i, _i, _i, _vp]),
    "linatt_qk_prologue_bwd_workspace_bytes": (_sz, [_i] * 5),
    "linatt_qk_prologue_bwd": (_i, [_vp] * 11 + [_i] * 7 + [_f, _i, _i, _f, _i, _i, _i, _vp]),
    "linatt_linear_scan_fwd": (_i, [_vp] * 5 + [_i] * 5 + [_f] * 2 + [_i] + [_vp]),
    "linatt_rmsnorm_fwd": (_i, [_vp] * 4 + [_i, _i, _f, _i, _vp]),
    "linatt_rmsnorm_bwd_workspace_bytes": (_sz, [_i, _i]),
    "linatt_rmsnorm_bwd": (_i, [_vp] * 7 + [_i] * 3 + [_vp]),
    "linatt_dkata_supported": (_i, [_i, _i, _i, _i]),
    "linatt_dkata_workspace_bytes": (_sz, [_i] * 6),
    "linatt_dkata_fwd": (_i, [_vp] * 8 + [_i] * 6 + [_f, _i, _f, _i, _vp]),
    "linatt_dkata_fwd_train": (_i, [_vp] * 8 + [_i] * 6 + [_f, _i, _f, _i, _vp]),
    "linatt_dkata_bwd_workspace_bytes": (_sz, [_i] * 6),
    "linatt_dkata_bwd": (_i, [_vp] * 14 + [_i] * 6 + [_f, _i, _f, _i, _vp]),
}


class LinattError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} -> {STATUS.get(status, status)}: {msg}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise ImportError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"linatt_amd: HIP library not found at {LIB_PATH}; "
                "build it with `python -m linatt_amd.build` (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.linatt_abi_version() != ABI_VERSION:
            raise ImportError(f"linatt_amd: ABI {lib.linatt_abi_version()} != {ABI_VERSION}")
        _lib = lib
    return _lib


def check(fn: str, status: int) -> None:
    if status != 0:
        raise LinattError(fn, status, load().linatt_last_error().decode())


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"linatt_amd: unsupported dtype {dt}") from None


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """Current HIP stream of the tensor's device, as a void pointer."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_scratch_by_stream: dict = {}


def stream_scratch(device: torch.device, nbytes: int):
    """A uint8 device buffer of at least ``nbytes``, kept per (device, current
    stream) and reused by the next call on that stream, which runs after this
    one's kernels (stream order).  Under graph capture a fresh buffer from the
    graph's pool is returned and not kept.  ``None`` for ``nbytes == 0``."""
    if not nbytes:
        return None
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes, device=device, dtype=torch.uint8)
    stream = torch.cuda.current_stream(device)
    key = (stream.device_index, stream.cuda_stream)
    buf = _scratch_by_stream.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, device=device, dtype=torch.uint8)
        _scratch_by_stream[key] = buf
    return buf


def split_decode_pays(rows: int) -> bool:
    """Whether a decode step should split each (b, h)'s rows over several
    workgroups (when the library offers a split at all): under graph capture
    the step is bound by its kernels, and a split fills the chip; called
    eagerly the host's launches bound a short step, and the split's second
    launch pays only for states of 1024 or more rows."""
    return rows >= 1024 or torch.cuda.is_current_stream_capturing()


def require_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "linatt_amd runs only on a ROCm GPU device; got a tensor on "
                f"{t.device} (there is no CPU path)")
