"""Host side of the multi-tensor launcher: tensor tables and chunk tables.

A launch covers a whole list of tensors. The host describes the list with one
64-byte ``tm_tensor_t`` record per tensor (raw device pointers, size, group,
flags) and splits it into fixed-size chunks with a ``tm_chunk_t`` table; both
go to device memory and one kernel launch walks them (one workgroup per chunk).
This replaces torch's MultiTensorApply batching of at most 36 tensors / 320
blocks per launch (torch/include/ATen/native/hip/MultiTensorApply.cuh:16-23)
with a single launch over the full list.

The chunk table depends only on the tensor sizes, so it is cached; the tensor
table carries grad pointers, which change whenever autograd allocates fresh
grads, so it is rebuilt per call (a few KB over PCIe, stream-ordered).
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from torchure_amd import _native

# Elements per chunk (one workgroup). A multiple of TM_CHUNK_ALIGN.
DEFAULT_CHUNK_ELEMS = 16384


def upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """Stream-ordered host->device copy of a small record array via pinned memory.

    torch's pinned-host allocator keeps the staging block alive until the copy
    has run, so the returned device tensor is safe to use on the current stream.
    """
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    staging = torch.empty(raw.size, dtype=torch.uint8, pin_memory=True)
    staging.numpy()[:] = raw
    return staging.to(device, non_blocking=True)


class ChunkTableCache:
    """Device chunk tables keyed by (sizes, chunk_elems, device)."""

    def __init__(self, capacity: int = 8):
        self._cap = capacity
        self._d: OrderedDict = OrderedDict()

    def get(self, numels: tuple[int, ...], chunk_elems: int, device: torch.device):
        key = (numels, chunk_elems, str(device))
        hit = self._d.get(key)
        if hit is not None:
            self._d.move_to_end(key)
            return hit
        table = _native.fill_chunks(np.asarray(numels, dtype=np.int64), chunk_elems)
        dev = upload(table, device) if len(table) else torch.empty(8, dtype=torch.uint8, device=device)
        val = (dev, len(table))
        self._d[key] = val
        if len(self._d) > self._cap:
            self._d.popitem(last=False)
        return val


CHUNKS = ChunkTableCache()


def check_chunk_elems(chunk_elems: int) -> int:
    chunk_elems = int(chunk_elems)
    if chunk_elems <= 0 or chunk_elems % _native.TM_CHUNK_ALIGN:
        raise ValueError(
            f"chunk_elems must be a positive multiple of {_native.TM_CHUNK_ALIGN}, got {chunk_elems}"
        )
    return chunk_elems


def grad_flags(g: torch.Tensor, who: str) -> int:
    if g.dtype == torch.bfloat16:
        return _native.TM_GRAD_BF16
    if g.dtype == torch.float32:
        return _native.TM_GRAD_F32
    raise RuntimeError(f"{who}: gradient dtype {g.dtype} is not supported (bfloat16 or float32)")


def require_device_tensor(t: torch.Tensor, who: str, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{who}: {what} must be on a ROCm GPU device, got {t.device} "
            "(torchure_amd has no CPU path)"
        )
    if not t.is_contiguous():
        raise RuntimeError(f"{who}: {what} must be contiguous")


def grad_table(grads: list[torch.Tensor], who: str) -> np.ndarray:
    """tm_tensor_t rows for a grad-only call (norm / scale)."""
    ptrs, numels, flags = [], [], []
    for g in grads:
        require_device_tensor(g, who, "grad")
        ptrs.append(g.data_ptr())
        numels.append(g.numel())
        flags.append(grad_flags(g, who))
    rows = np.zeros(len(grads), dtype=_native.TENSOR_DTYPE)
    rows["grad"] = np.asarray(ptrs, dtype=np.uint64)
    rows["numel"] = np.asarray(numels, dtype=np.int64)
    rows["flags"] = np.asarray(flags, dtype=np.uint32)
    return rows
