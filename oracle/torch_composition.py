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


def chunk_fwd_reference(hidden, weight, labels, ignore_index):
    """Per-chunk math of torchure/loss/fused_linear_ce.py:31-59 with the same torch
    calls (without torch.compile): returns (loss_sum, grad_hidden, grad_weight)."""
    logits = (hidden @ weight.t()).float()
    valid = labels != ignore_index
    safe = torch.where(valid, labels, 0).unsqueeze(1)
    lse = torch.logsumexp(logits, dim=-1)
    target = logits.gather(1, safe).squeeze(1)
    loss_sum = ((lse - target) * valid).sum()
    probs = torch.exp(logits - lse.unsqueeze(1))
    probs = probs * valid.unsqueeze(1)
    probs.scatter_add_(1, safe, -valid.float().unsqueeze(1))
    grad_logits = probs.to(hidden.dtype)
    grad_hidden = grad_logits @ weight
    grad_weight = grad_logits.t() @ hidden
    return loss_sum, grad_hidden, grad_weight


def fused_linear_ce_reference(hidden, weight, labels, ignore_index=-100, chunk_size=1024,
                              chunk_fn=chunk_fwd_reference):
    """Forward + backward (grad_out = 1) of the reference op, fused_linear_ce.py:62-127.
    Returns (mean loss, grad_hidden, grad_weight fp32)."""
    n = hidden.shape[0]
    w = weight.to(hidden.dtype)
    loss_sum = torch.zeros((), dtype=torch.float32, device=hidden.device)
    grad_hidden = torch.empty_like(hidden)
    grad_weight = torch.zeros_like(weight, dtype=torch.float32)
    for s in range(0, n, chunk_size):
        e = min(s + chunk_size, n)
        chunk_loss, gh, gw = chunk_fn(hidden[s:e], w, labels[s:e], ignore_index)
        loss_sum += chunk_loss
        grad_hidden[s:e] = gh
        grad_weight += gw
    n_valid = (labels != ignore_index).sum().clamp_min(1)
    scale = 1.0 / n_valid
    grad_hidden.mul_(scale.to(grad_hidden.dtype))
    grad_weight.mul_(scale)
    return loss_sum / n_valid, grad_hidden, grad_weight
