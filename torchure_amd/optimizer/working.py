"""bf16 working copies of fp32 master params, and fp32 grad accumulation.

The reference keeps only fp32 params and lets autocast cast them to bf16 at
every forward (torchure/train/trainer.py:374). Here the bf16 copy is
materialised once per step by the optimizer kernel (RNE(master), the rounding
of torch/headeronly/util/BFloat16.h:100-114), so a bf16 forward reads 2 B/param
instead of casting 4 B/param, and its backward leaves bf16 grads on the copies.

All copies of one call live in a single flat bf16 buffer (one allocation,
16-byte aligned per tensor so the update kernel's vector path applies); each
copy is a separate autograd leaf aliasing its slice.
"""

from __future__ import annotations

import weakref

import numpy as np
import torch

from torchure_amd import _native
from torchure_amd.core import tables

_ALIGN_ELEMS = 8  # 16 bytes of bf16


def attach_bf16_working_params(params) -> list[torch.Tensor]:
    """Create bf16 working copies = RNE(master) for fp32 ``params`` and attach them.

    Each master gets ``p._tm_working``; the returned list is in ``params`` order.
    """
    params = list(params)
    if not params:
        return []
    device = params[0].device
    offsets, total = [], 0
    for p in params:
        tables.require_device_tensor(p, "attach_bf16_working_params", "param")
        if p.dtype != torch.float32 or p.device != device:
            raise RuntimeError("attach_bf16_working_params: params must be fp32 on one device")
        offsets.append(total)
        total += (p.numel() + _ALIGN_ELEMS - 1) // _ALIGN_ELEMS * _ALIGN_ELEMS
    flat = torch.empty(max(total, 1), dtype=torch.bfloat16, device=device)
    views = [flat[off : off + p.numel()].view(p.shape) for p, off in zip(params, offsets)]
    _cast_list(params, views, device)
    out = []
    for p, w in zip(params, views):
        w = w.detach().requires_grad_(p.requires_grad)
        p._tm_working = w
        mark_current(p, w)
        out.append(w)
    return out


_CAST_UPLOAD = tables.TableUploader()


def _cast_list(masters, copies, device) -> None:
    """copies[i] = RNE(masters[i]) for the whole list in one launch (tm_cast_bf16_list)."""
    rows = np.zeros(len(masters), dtype=_native.TENSOR_DTYPE)
    rows["master"] = _native.host().ptrs(masters)
    rows["param_bf16"] = _native.host().ptrs(copies)
    rows["numel"] = np.fromiter((m.numel() for m in masters), dtype=np.int64, count=len(masters))
    chunk_elems = tables.DEFAULT_CHUNK_ELEMS
    chunks, n_chunks = tables.CHUNKS.get(rows["numel"], chunk_elems, device)
    d_rows = _CAST_UPLOAD(rows, device)
    rc = _native.lib().tm_cast_bf16_list(d_rows.data_ptr(), len(masters), chunks.data_ptr(), n_chunks,
                                         chunk_elems, _native.stream_handle(device))
    _native.check(rc, "tm_cast_bf16_list")


def mark_current(p: torch.Tensor, w: torch.Tensor) -> None:
    """Record that ``w`` holds RNE(``p``) as of ``p``'s and ``w``'s current autograd versions."""
    w._tm_master_version = p._version
    w._tm_copy_version = w._version


def is_current(p: torch.Tensor, w: torch.Tensor) -> bool:
    """True if ``p`` has not been modified in place since ``w`` was last written from it."""
    return getattr(w, "_tm_master_version", None) == p._version


def current_copy(p: torch.Tensor) -> torch.Tensor | None:
    """``p``'s attached bf16 working copy if it holds RNE(``p``) now, else None: the copy has
    ``p``'s shape and device, and neither ``p`` nor the copy has been modified in place since
    the copy was last written (by attach, refresh or ``AdamW.step()``). Its bits are then those
    of ``p.to(torch.bfloat16)``, so a reader may take it instead of casting."""
    w = getattr(p, "_tm_working", None)
    if (w is None or p.dtype != torch.float32 or w.dtype != torch.bfloat16 or w.shape != p.shape
            or w.device != p.device or not w.is_contiguous() or not is_current(p, w)
            or getattr(w, "_tm_copy_version", None) != w._version):
        return None
    return w


def refresh_bf16_working_params(params) -> None:
    """Rewrite the attached bf16 working copies as RNE(master), in place.

    Needed after the fp32 masters change outside ``AdamW.step()``, e.g. after
    ``model.load_state_dict(...)`` on a resume (torchure/train/trainer.py:340-350), so
    that the next bf16 forward does not run on stale weights. ``AdamW.step()`` raises
    if it finds a master modified since its copy was last written."""
    per_dev: dict = {}
    for p in params:
        w = getattr(p, "_tm_working", None)
        if w is None:
            continue
        tables.require_device_tensor(p, "refresh_bf16_working_params", "param")
        per_dev.setdefault(p.device, []).append((p, w))
    for device, pairs in per_dev.items():  # one launch per device
        _cast_list([p for p, _ in pairs], [w for _, w in pairs], device)
        for p, w in pairs:
            torch.autograd.graph.increment_version(w)
            mark_current(p, w)


def accumulate_grad_(acc: torch.Tensor, micro: torch.Tensor) -> None:
    """acc (fp32) += micro (bf16), in place: one micro-step of grad accumulation
    (the fp32 .grad accumulation of torchure/train/trainer.py:383-390)."""
    who = "accumulate_grad_"
    tables.require_device_tensor(acc, who, "accumulator")
    tables.require_device_tensor(micro, who, "micro-step grad")
    if acc.dtype != torch.float32 or micro.dtype != torch.bfloat16:
        raise RuntimeError(f"{who}: accumulator must be float32 and micro grad bfloat16")
    if acc.numel() != micro.numel() or acc.device != micro.device:
        raise RuntimeError(f"{who}: size/device mismatch")
    rc = _native.lib().tm_grad_accumulate_bf16(
        acc.data_ptr(), micro.data_ptr(), acc.numel(), _native.stream_handle(acc.device)
    )
    _native.check(rc, "tm_grad_accumulate_bf16")
    torch.autograd.graph.increment_version(acc)


# device -> (norm tensor, [(weakref(grad), grad._version), ...]) of the last fused
# accumulate+norm call; clip_grad_norm reuses it when it sees exactly those grads,
# unmodified (torch bumps _version on every in-place op; this package's own kernels
# that write grads call increment_version or drop the entry).
_NORM_CACHE: dict = {}
_ACC_UPLOAD = tables.TableUploader()


def _stamp(grads):
    return [(weakref.ref(g), g._version) for g in grads]


def cached_norm(grads: list[torch.Tensor]):
    """The fused norm of exactly ``grads`` (same tensors, same order, unmodified), or None."""
    if not grads:
        return None
    hit = _NORM_CACHE.get(grads[0].device)
    if hit is None:
        return None
    norm, stamp = hit
    if len(stamp) != len(grads):
        return None
    for (ref, ver), g in zip(stamp, grads):
        if ref() is not g or g._version != ver:
            return None
    return norm


def drop_cached_norm(device=None) -> None:
    if device is None:
        _NORM_CACHE.clear()
    else:
        _NORM_CACHE.pop(device, None)


def accumulate_grads_(params, *, last: bool = False,
                      chunk_elems: int = tables.DEFAULT_CHUNK_ELEMS) -> torch.Tensor | None:
    """One micro-step of gradient accumulation for fp32 masters with bf16 working copies.

    For every param whose working copy carries a bf16 grad: ``p.grad`` (fp32) += that
    grad, in one launch over the whole list; the bf16 grad is then released. A param
    without ``p.grad`` gets one holding the widened grad itself (assigned, not added to
    zeros, as autograd's first backward assigns the grad). This is the fp32 ``.grad``
    accumulation autograd performs across micro-batches in
    torchure/train/trainer.py:383-390.

    With ``last=True`` the same pass also computes the global L2 norm of the
    accumulated fp32 grads of all ``params`` (returned as a 0-d fp32 device tensor).
    A following ``clip_grad_norm`` over the same params reuses it instead of reading
    every grad again; the value is bit-identical to what it would compute.
    """
    who = "accumulate_grads_"
    params = list(params)
    todo = []  # (param, its fp32 accumulator or None on a first micro-step, bf16 micro grad or None)
    for p in params:
        w = getattr(p, "_tm_working", None)
        mg = w.grad if w is not None else None
        g = p.grad
        if mg is None and (not last or g is None):
            continue
        tables.require_device_tensor(p, who, "param")
        dt = p.dtype if g is None else g.dtype
        if g is not None:
            tables.require_device_tensor(g, who, "fp32 accumulator")
        if dt != torch.float32:
            raise RuntimeError(f"{who}: the accumulator (p.grad) must be float32, got {dt}")
        if mg is not None:
            tables.require_device_tensor(mg, who, "bf16 micro-step grad")
            if mg.dtype != torch.bfloat16 or mg.numel() != p.numel() or mg.device != p.device:
                raise RuntimeError(f"{who}: micro-step grad must be bf16 of the param's size and device")
        todo.append((p, g, mg))
    if not todo:
        if last:
            raise AssertionError(f"{who}: no grads to accumulate or measure")
        return None
    device = todo[0][0].device
    if any(p.device != device for p, _, _ in todo):
        raise RuntimeError(f"{who}: all params must be on one device")
    # Every check has passed: only now give first micro-steps their accumulator, which the
    # kernel assigns (no zero fill, no read), so an error above leaves no p.grad behind.
    accs, micros, assign = [], [], []
    for p, g, mg in todo:
        fresh = g is None
        if fresh:
            g = p.grad = torch.empty_like(p, memory_format=torch.contiguous_format)
        accs.append(g)
        micros.append(mg)
        assign.append(fresh)
    drop_cached_norm(device)
    rows = np.zeros(len(accs), dtype=_native.ACCUM_DTYPE)
    rows["acc"] = np.asarray([a.data_ptr() for a in accs], dtype=np.uint64)
    rows["micro"] = np.asarray([m.data_ptr() if m is not None else 0 for m in micros], dtype=np.uint64)
    rows["numel"] = np.asarray([a.numel() for a in accs], dtype=np.int64)
    rows["flags"] = np.asarray(assign, dtype=np.int64) * _native.TM_ACCUM_ASSIGN
    chunk_elems = tables.check_chunk_elems(chunk_elems)
    chunks, n_chunks = tables.CHUNKS.get(rows["numel"], chunk_elems, device)
    d_rows = _ACC_UPLOAD(rows, device)
    norm = torch.empty((), dtype=torch.float32, device=device) if last else None
    ws = None
    if last:  # one fp64 partial per 256-element slice, reduced in a fixed order
        ws = torch.empty(int(_native.lib().tm_accum_norm_workspace_bytes(n_chunks, chunk_elems)),
                         dtype=torch.uint8, device=device)
    rc = _native.lib().tm_grad_accumulate_list(
        d_rows.data_ptr(), len(accs), chunks.data_ptr(), n_chunks, chunk_elems, int(last),
        ws.data_ptr() if last else None, ws.numel() if last else 0, norm.data_ptr() if last else None,
        _native.stream_handle(device))
    _native.check(rc, "tm_grad_accumulate_list")
    for a, m in zip(accs, micros):
        if m is not None:
            torch.autograd.graph.increment_version(a)
    for p in params:
        w = getattr(p, "_tm_working", None)
        if w is not None and w.grad is not None:
            w.grad = None
    if last:
        _NORM_CACHE[device] = (norm, _stamp(accs))
    return norm
