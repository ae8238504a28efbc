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

import threading
from collections import OrderedDict

import numpy as np
import torch

from torchure_amd import _native

# Elements per chunk (one workgroup). A multiple of TM_CHUNK_ALIGN.
DEFAULT_CHUNK_ELEMS = 16384


def upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """One-off stream-ordered host->device copy of a small record array via pinned memory.

    torch's pinned-host allocator keeps the staging block alive until the copy
    has run, so the returned device tensor is safe to use on the current stream.
    """
    raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    staging = torch.empty(raw.size, dtype=torch.uint8, pin_memory=True)
    staging.numpy()[:] = raw
    return staging.to(device, non_blocking=True)


class TableUploader:
    """Per-step upload of a record table (tensor or accumulation list).

    If the table's bytes equal the previous upload on the same device and stream,
    the previous device copy is returned (steady-state training usually gets the
    same grad addresses back from the caching allocator, so nothing moves).
    Otherwise the bytes are staged through one of ``slots`` pinned buffers, each
    reused only after the copy that last read it has completed, and copied
    asynchronously on the current stream. No per-step pinned allocation, and the
    host blocks only if it runs more than ``slots`` uploads ahead of the device.
    Calls from several host threads are serialised, so two uploads never share a slot.
    """

    def __init__(self, slots: int = 4):
        self._slots: list = [None] * slots  # (pinned uint8 tensor, event or None)
        self._next = 0
        self._last = None  # (bytes, device tensor, stream handle)
        self._lock = threading.Lock()

    def __call__(self, arr: np.ndarray, device: torch.device) -> torch.Tensor:
        with self._lock:
            return self._upload(arr, device)

    def _upload(self, arr: np.ndarray, device: torch.device) -> torch.Tensor:
        raw = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        stream = torch.cuda.current_stream(device)
        last = self._last
        if (last is not None and last[1].device == device and last[2] == stream.cuda_stream
                and last[0].size == raw.size and np.array_equal(last[0], raw)):
            return last[1]
        i = self._next
        self._next = (i + 1) % len(self._slots)
        slot = self._slots[i]
        if slot is not None and slot[1] is not None:
            slot[1].synchronize()
        if slot is None or slot[0].numel() < raw.size:
            buf = torch.empty(max(raw.size, 4096) * 2, dtype=torch.uint8, pin_memory=True)
        else:
            buf = slot[0]
        buf.numpy()[: raw.size] = raw
        dev = torch.empty(max(raw.size, 8), dtype=torch.uint8, device=device)
        dev[: raw.size].copy_(buf[: raw.size], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        self._slots[i] = (buf, ev)
        self._last = (raw.copy(), dev, stream.cuda_stream)
        return dev


def make_ready(table: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Makes a cached device table safe to read on the device's current stream.

    A cached table was uploaded asynchronously on the stream current at the time
    (``_tm_home``), and its upload is marked by ``_tm_ready``, an event recorded there
    after the copy. On any other stream, the current stream first waits for that
    event, so a launch there never reads a table whose copy has not run yet, and
    record_stream keeps the caching allocator from reusing its block before that
    stream's work has run, should the table be evicted and freed."""
    cur = torch.cuda.current_stream(device)
    home = getattr(table, "_tm_home", None)
    if home is not None and cur != home:
        cur.wait_event(table._tm_ready)
        table.record_stream(cur)
    return table


class ChunkTableCache:
    """Device chunk tables keyed by (sizes, chunk_elems, device)."""

    def __init__(self, capacity: int = 8):
        self._cap = capacity
        self._d: OrderedDict = OrderedDict()

    def get(self, numels, chunk_elems: int, device: torch.device):
        """``(table, n_chunks)`` for these sizes (any int sequence), ready for a launch
        on the device's current stream (``make_ready``: a hit from a stream other than
        the one that uploaded the table waits for its upload)."""
        numels = np.ascontiguousarray(numels, dtype=np.int64)
        key = (numels.tobytes(), chunk_elems, str(device))
        hit = self._d.get(key)
        if hit is not None:
            self._d.move_to_end(key)
            make_ready(hit[0], device)
            return hit
        table = _native.fill_chunks(numels, chunk_elems)
        dev = upload(table, device) if len(table) else torch.empty(8, dtype=torch.uint8, device=device)
        home = torch.cuda.current_stream(device)
        ready = torch.cuda.Event()
        ready.record(home)
        dev._tm_home = home
        dev._tm_ready = ready
        val = (dev, len(table))
        self._d[key] = val
        if len(self._d) > self._cap:
            self._d.popitem(last=False)
        return val


CHUNKS = ChunkTableCache()


def follow_home_stream(home, device: torch.device, tensors) -> None:
    """Before a launch that was planned on stream ``home`` runs on the device's current stream:
    if the two differ, the current stream waits for ``home`` (the tables were uploaded there,
    asynchronously) and each tensor is marked as used on the current stream, so the caching
    allocator does not hand its block to other work before this stream is done with it."""
    cur = torch.cuda.current_stream(device)
    if cur == home:
        return
    cur.wait_stream(home)
    for t in tensors:
        if t is not None:
            t.record_stream(cur)


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
    if not grads:
        return np.zeros(0, _native.TENSOR_DTYPE)
    ptr, numel, code = _native.host().grad_fields(grads)
    if not (code != 255).all():
        return _grad_table_checked(grads, who)  # raises with the reason
    rows = np.zeros(len(grads), dtype=_native.TENSOR_DTYPE)
    rows["grad"] = ptr
    rows["numel"] = numel
    rows["flags"] = code  # 0 = TM_GRAD_BF16, 1 = TM_GRAD_F32
    return rows


def _grad_table_checked(grads: list[torch.Tensor], who: str) -> np.ndarray:
    bf16, f32 = torch.bfloat16, torch.float32
    recs = []
    for g in grads:
        dt = g.dtype
        if dt is bf16:
            flags = _native.TM_GRAD_BF16
        elif dt is f32:
            flags = _native.TM_GRAD_F32
        else:
            flags = grad_flags(g, who)  # raises
        if g.layout != torch.strided:
            raise RuntimeError(f"{who}: {g.layout} grads are not supported (dense grads only)")
        if not g.is_cuda or not g.is_contiguous():
            require_device_tensor(g, who, "grad")  # raises with the reason
        recs.append((0, 0, 0, g.data_ptr(), 0, 0, g.numel(), 0, flags))
    return np.array(recs, dtype=_native.TENSOR_DTYPE) if recs else np.zeros(0, _native.TENSOR_DTYPE)
