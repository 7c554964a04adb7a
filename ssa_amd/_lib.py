"""ctypes binding of libssa_hip.so (the C ABI declared in include/ssa_hip.h).

Loading is lazy and loud: any entry point raises if the library is missing or was built for a
different ABI, and a non-zero status from the library becomes an exception carrying
ssa_last_error(). There is no fallback path.
"""
from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libssa_hip.so"
ABI_VERSION = 7

SSA_OK, SSA_ERR_INVALID, SSA_ERR_UNSUPPORTED, SSA_ERR_HIP, SSA_ERR_WORKSPACE = 0, -1, -2, -3, -4
F32, F16, BF16 = 0, 1, 2
STATS_POP, STATS_UNBIASED, STATS_QMEAN = 0, 1, 2
ROUTE_BUDGET, ROUTE_FLAT, ROUTE_QUERY, ROUTE_STARTED = 0, 1, 2, 3
ATTN_VT_READY = 1
ATTN_ROTATE = 2
ATTN_EXACT = 4
ATTN_PREPARED = 8
MASKED_MASKS_READY = 1
DECODE_STATIC_SCRATCH_BYTES = 16 << 20  # SSA_DECODE_STATIC_SCRATCH_BYTES

_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_f = ctypes.c_float
_c_p = ctypes.c_void_p
_c_sz = ctypes.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "ssa_abi_version": (_c_int, []),
    "ssa_last_error": (ctypes.c_char_p, []),
    "ssa_device_supported": (_c_int, [_c_int]),
    "ssa_block_summary": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_p]),
    "ssa_route_width": (_c_i64, [_c_int, _c_i64, _c_i64, _c_i64, _c_f, _c_i64, _c_i64, _c_i64]),
    "ssa_route_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "ssa_route_workspace_size_split": (_c_sz, [_c_i64] * 7),
    "ssa_route": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_p] + [_c_i64] * 6 +
                  [_c_int, _c_i64, _c_f, _c_i64, _c_f, _c_f, _c_i64, _c_i64, _c_p, _c_p, _c_i64,
                   _c_p, _c_sz, _c_p]),
    "ssa_route_pooled": (_c_int, [_c_p, _c_int, _c_p, _c_p, _c_p] + [_c_i64] * 7 +
                         [_c_int, _c_i64, _c_f, _c_i64, _c_f, _c_f, _c_i64, _c_i64, _c_p, _c_p,
                          _c_i64, _c_p, _c_sz, _c_p]),
    "ssa_project_rows": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p]),
    "ssa_expand_selection": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "ssa_ivf_index_size": (_c_sz, [_c_i64] * 4),
    "ssa_ivf_build": (_c_int, [_c_p] + [_c_i64] * 5 + [_c_p, _c_sz, _c_p]),
    "ssa_ivf_route": (_c_int, [_c_p, _c_p] + [_c_i64] * 9 + [_c_p, _c_p, _c_i64, _c_p]),
    "ssa_tree_size": (_c_sz, [_c_i64] * 5),
    "ssa_tree_build": (_c_int, [_c_p, _c_int] + [_c_i64] * 5 + [_c_p, _c_i64, _c_i64, _c_p, _c_sz,
                                                                _c_p]),
    "ssa_tree_descend": (_c_int, [_c_p, _c_p, _c_p] + [_c_i64] * 8 + [_c_f, _c_p, _c_p]),
    "ssa_tree_pack": (_c_int, [_c_p] + [_c_i64] * 4 + [_c_p, _c_p, _c_i64, _c_p]),
    "ssa_ccc_index_size": (_c_sz, [_c_i64] * 3),
    "ssa_ccc_stage": (_c_int, [_c_p, _c_int] + [_c_i64] * 4 + [_c_p] + [_c_i64] * 3 +
                      [_c_p] * 4 + [_c_sz, _c_p]),
    "ssa_ccc_kmeans": (_c_int, [_c_p] + [_c_i64] * 4 + [_c_int, _c_p, _c_p, _c_sz, _c_p]),
    "ssa_ccc_assign": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_sz, _c_p]),
    "ssa_ccc_index_build": (_c_int, [_c_p] + [_c_i64] * 3 + [_c_p, _c_p, _c_i64, _c_sz, _c_p]),
    "ssa_ccc_index_add": (_c_int, [_c_p] + [_c_i64] * 4 + [_c_p, _c_i64, _c_sz, _c_p]),
    "ssa_ccc_route": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p,
                               _c_i64, _c_i64, _c_p, _c_p] + [_c_i64] * 9 +
                      [_c_int, _c_f, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "ssa_masked_attn_workspace_size": (_c_sz, [_c_i64] * 6),
    "ssa_masked_attn_fwd": (_c_int, [_c_p] * 5 + [_c_int] + [_c_i64] * 6 +
                            [_c_p] * 3 + [_c_i64, _c_f, _c_p, _c_sz, _c_p]),
    "ssa_masked_attn_bwd": (_c_int, [_c_p] * 9 + [_c_int, _c_int, _c_int] + [_c_i64] * 6 +
                            [_c_p] * 3 + [_c_i64, _c_f, _c_p, _c_sz, _c_p]),
    "ssa_sparse_attn_workspace_size": (_c_sz, [_c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "ssa_sparse_attn_prepare": (_c_int, [_c_p, _c_p, _c_int] + [_c_i64] * 5 + [_c_p, _c_p, _c_sz,
                                                                            _c_p]),
    "ssa_transpose_v": (_c_int, [_c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_i64, _c_i64, _c_p, _c_sz, _c_p]),
    "ssa_sparse_attn_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_i64, _c_i64, _c_i64,
                                     _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_f, _c_p,
                                     _c_int, _c_p, _c_sz, _c_p]),
    "ssa_decode_attend_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "ssa_decode_attend": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_f,
                                   _c_p, _c_sz, _c_p]),
    "ssa_decode_step_workspace_size": (_c_sz, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "ssa_decode_step": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int, _c_i64,
                                 _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_f,
                                 _c_i64, _c_f, _c_f, _c_p, _c_p, _c_i64, _c_p, _c_sz, _c_p]),
    "ssa_decode_step_static": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int,
                                        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                        _c_p, _c_i64, _c_f, _c_i64, _c_f, _c_f, _c_p, _c_p, _c_i64,
                                        _c_p]),
}

_lock = threading.Lock()
_lib = None


class SSAError(RuntimeError):
    """A libssa_hip.so call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed (status {status}): {message}")
        self.status = status


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use; raises if absent or ABI-mismatched)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m ssa_amd.build` "
                    "(ssa_amd has no CPU or PyTorch fallback)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            ver = handle.ssa_abi_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH} has ABI {ver}, expected {ABI_VERSION}: rebuild it")
            _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def call(name: str, *args) -> int:
    """Calls a status-returning entry point and raises SSAError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != SSA_OK:
        msg = lib().ssa_last_error()
        raise SSAError(name, rc, msg.decode() if msg else "")
    return rc


@functools.lru_cache(maxsize=4096)
def query(name: str, *args):
    """Calls a size/width query (no status). The queries are pure functions of their arguments,
    so results are cached (a ctypes call per training step costs more than the kernels of a
    small one)."""
    return getattr(lib(), name)(*args)


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DTYPES[t]
    except KeyError:
        raise TypeError(f"ssa_amd supports float32/float16/bfloat16 tensors, got {t}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of t's device as a raw handle."""
    return torch.cuda.current_stream(t.device).cuda_stream


def i64_array(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(values))(*[int(v) for v in values])
    return arr


def require_device(*tensors: torch.Tensor) -> None:
    """The kernels run on ROCm device tensors only; CPU tensors are an error, never a fallback."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("ssa_amd kernels take ROCm device tensors (got a CPU tensor); "
                               "there is no CPU fallback")
