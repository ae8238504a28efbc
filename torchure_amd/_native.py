"""Loader and thin ctypes binding of the gfx950 C-ABI library ``libtorchure_amd.so``.

The library is the only compute path of this package: there is no CPU or
PyTorch fallback. If it is missing or fails to load, every entry point raises.

torch is imported before the library is opened so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch has already
loaded (both carry that SONAME); the library then shares torch's device
context and can be handed torch's stream handles.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np
import torch  # noqa: F401  (must be loaded before the HIP library, see above)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtorchure_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "torchure_amd.h")

ABI_VERSION = 3

TM_OK = 0
TM_GRAD_BF16 = 0
TM_GRAD_F32 = 1
TM_FLAG_CLIP = 2
TM_MAX_GROUPS = 16
TM_CHUNK_ALIGN = 2048
TM_NORM_PARTIALS = 2048
TM_NOALLOC_MAX_TENSORS = 16384

# tm_tensor_t (include/torchure_amd.h), 64 bytes.
TENSOR_DTYPE = np.dtype(
    [
        ("master", "<u8"),
        ("exp_avg", "<u8"),
        ("exp_avg_sq", "<u8"),
        ("grad", "<u8"),
        ("param_bf16", "<u8"),
        ("step", "<u8"),
        ("numel", "<i8"),
        ("group", "<i4"),
        ("flags", "<u4"),
    ]
)
assert TENSOR_DTYPE.itemsize == 64

# tm_accum_t, 32 bytes.
ACCUM_DTYPE = np.dtype([("acc", "<u8"), ("micro", "<u8"), ("numel", "<i8"), ("flags", "<i8")])
TM_ACCUM_ASSIGN = 1
assert ACCUM_DTYPE.itemsize == 32

# tm_chunk_t, 8 bytes.
CHUNK_DTYPE = np.dtype([("tensor", "<u4"), ("chunk", "<u4")])


class TmHyper(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("eps", ctypes.c_double),
    ]


# Every symbol include/torchure_amd.h declares, with its ctypes signature.
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_SIGNATURES = {
    "tm_abi_version": (ctypes.c_int, []),
    "tm_last_error": (ctypes.c_char_p, []),
    "tm_workspace_bytes": (ctypes.c_size_t, [_i64]),
    "tm_count_chunks": (_i64, [_vp, _i64, _i64]),
    "tm_fill_chunks": (_i64, [_vp, _i64, _i64, _vp, _i64]),
    "tm_grad_norm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _i64, ctypes.c_float, ctypes.c_int, _vp, _vp, _vp, _vp],
    ),
    "tm_grad_scale": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "tm_adamw_step": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _i64, ctypes.POINTER(TmHyper), ctypes.c_int32, _vp, _vp, _vp],
    ),
    "tm_adamw_step_noalloc": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _i64, ctypes.POINTER(TmHyper), ctypes.c_int32, _vp, _vp],
    ),
    "tm_accum_norm_workspace_bytes": (ctypes.c_size_t, [_i64, _i64]),
    "tm_grad_accumulate_list": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, ctypes.c_int, _vp, ctypes.c_size_t, _vp, _vp]),
    "tm_clip_coef": (ctypes.c_int, [_vp, ctypes.c_float, _vp, _vp]),
    "tm_grad_accumulate_bf16": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "tm_stream_copy": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "tm_cast_bf16": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "tm_cast_bf16_list": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _vp]),
    "tm_ce_rows_bf16": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "tm_ce_rows_loss_bf16": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "tm_ce_rows_f32": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "tm_ce_rows_loss_f32": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _vp, _vp]),
    "tm_ce_loss": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "tm_ce_scale_grads": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    "tm_ce_grad_w": (ctypes.c_int, [_vp, _vp, _i64, ctypes.c_int, _vp, _vp, _vp]),
    "tm_ce_grad_w2": (ctypes.c_int, [_vp, _vp, _vp, _i64, ctypes.c_int, _vp, _vp, _vp]),
    "tm_ce_grad_w_fold": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _i64, ctypes.c_int, _vp, _vp, _vp]),
    "tm_ce_widen_scale": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _vp]),
    "tm_ce_grad_h_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64]),
    "tm_ce_grad_h_bf16": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, ctypes.c_size_t, _vp]),
    "tm_ce_logits_bf16": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "tm_ce_grad_w_bf16": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp]),
}

EXPORTED = tuple(_SIGNATURES)

_LIB: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def lib() -> ctypes.CDLL:
    """The loaded library; raises RuntimeError if it is not built or not loadable."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"torchure_amd: native library {LIB_PATH} is not built; run "
            "`python -c 'import __graft_entry__ as g; g.build()'` from the repo root"
        )
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    got = handle.tm_abi_version()
    if got != ABI_VERSION:
        raise RuntimeError(f"torchure_amd: library ABI {got}, expected {ABI_VERSION}")
    _LIB = handle
    return handle


_HOST = None


def host():
    """The host-side list primitives (``_tm_host``, CPU-only C++); raises if not built."""
    global _HOST
    if _HOST is None:
        try:
            from torchure_amd import _tm_host
        except ImportError as e:
            raise RuntimeError(
                "torchure_amd: host extension _tm_host is not built; run "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repo root") from e
        _HOST = _tm_host
    return _HOST


def check(rc: int, what: str) -> None:
    if rc != TM_OK:
        msg = lib().tm_last_error().decode(errors="replace")
        raise NativeError(f"{what} failed ({rc}): {msg}")


def workspace_bytes(n_tensors: int) -> int:
    return int(lib().tm_workspace_bytes(n_tensors))


def fill_chunks(numels: np.ndarray, chunk_elems: int) -> np.ndarray:
    """Chunk table (CHUNK_DTYPE records) for the given tensor sizes."""
    numels = np.ascontiguousarray(numels, dtype=np.int64)
    n = int(lib().tm_count_chunks(numels.ctypes.data, len(numels), chunk_elems))
    if n < 0:
        check(n, "tm_count_chunks")
    out = np.zeros(max(n, 1), dtype=CHUNK_DTYPE)
    k = int(lib().tm_fill_chunks(numels.ctypes.data, len(numels), chunk_elems, out.ctypes.data, n))
    if k < 0:
        check(k, "tm_fill_chunks")
    return out[:k]


def hyper_array(groups: list[tuple[float, float, float, float, float]]):
    """ctypes array of tm_hyper_t from (lr, beta1, beta2, weight_decay, eps) tuples."""
    arr = (TmHyper * max(len(groups), 1))()
    for i, (lr, b1, b2, wd, eps) in enumerate(groups):
        arr[i] = TmHyper(float(lr), float(b1), float(b2), float(wd), float(eps))
    return arr


def stream_handle(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)
