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
    out = []
    lib = _native.lib()
    stream = _native.stream_handle(device)
    for p, off in zip(params, offsets):
        w = flat[off : off + p.numel()].view(p.shape)
        _native.check(lib.tm_cast_bf16(w.data_ptr(), p.data_ptr(), p.numel(), stream), "tm_cast_bf16")
        w = w.detach().requires_grad_(p.requires_grad)
        p._tm_working = w
        out.append(w)
    return out


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
