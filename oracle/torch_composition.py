"""The reference's optimizer tail composed from the torch library on the CPU --
TEST INFRASTRUCTURE ONLY (golden vectors and bench.py's cpu_baseline leg).

Same torch calls, same order, as the reference step:
  clip  torchure/core/grad_helper.py:17-18,32-33
        (_foreach_norm -> stack -> vector_norm -> clamp(max_norm/(total+1e-6), max=1)
         -> _foreach_mul_)
  step  torch.optim.AdamW(groups, fused=True) with the two groups of
        torchure/optimizer/builder.py:37-43
  bf16  master.to(torch.bfloat16) (what autocast does at the next forward,
        torchure/train/trainer.py:374)
bf16 gradients are widened to fp32 first (exact), fp32 being the reference's
native grad dtype.
"""

from __future__ import annotations

import torch


def clip_grad_norm_reference(grads: list[torch.Tensor], max_norm: float | None) -> torch.Tensor:
    norms = torch._foreach_norm(grads, 2.0)
    total = torch.linalg.vector_norm(torch.stack(norms), 2.0)
    if max_norm is None:
        return total
    clip_coef = torch.clamp(max_norm / (total + 1e-6), max=1.0)
    torch._foreach_mul_(grads, clip_coef)
    return total


def make_reference_optimizer(params: list[torch.nn.Parameter], lr=3e-4, betas=(0.9, 0.95), eps=1e-8,
                             weight_decay=0.1) -> torch.optim.AdamW:
    groups = [
        {"params": [p for p in params if p.dim() >= 2], "weight_decay": weight_decay},
        {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0},
    ]
    return torch.optim.AdamW(groups, lr=lr, betas=betas, eps=eps, fused=True)


def reference_step(params, opt, max_norm=1.0, bf16_out=None) -> torch.Tensor:
    """One step: clip -> AdamW(fused) -> bf16 copies. grads must already be on p.grad (fp32)."""
    total = clip_grad_norm_reference([p.grad for p in params], max_norm)
    opt.step()
    if bf16_out is not None:
        for p, w in zip(params, bf16_out):
            w.copy_(p.detach().to(torch.bfloat16))
    return total
