"""Learning-rate schedules, same classes and formulas as torchure/optimizer/scheduler.py.

Host-only (python floats, i.e. double): the schedule writes ``group['lr']``
before each step and the fused kernel reads it as a double hyper-parameter.
The class name keeps the reference's spelling (``WarmupStableDecaySchedulder``)
so configs and imports resolve unchanged.
"""

from __future__ import annotations

from torch.optim.lr_scheduler import LRScheduler


def wsd_scale(step: int, total_steps: int, warmup_ratio: float, decay_ratio: float) -> float:
    """LR multiplier of the warmup-stable-decay schedule at step index ``step``.

    torchure/optimizer/scheduler.py:17-35:
      W = max(1, round(T * warmup_ratio)); decay starts at T * (1 - decay_ratio)
      step <  W           -> (step + 1) / W
      step >= decay start -> max(0, 1 - (step - start) / (decay_ratio * T))
      otherwise           -> 1.0
    """
    decay_phase_start = total_steps * (1 - decay_ratio)
    warmup_steps = max(1, round(total_steps * warmup_ratio))
    if step < warmup_steps:
        return (step + 1) / warmup_steps
    if step >= decay_phase_start:
        num_decay_steps = decay_ratio * total_steps
        return max(0, 1 - ((step - decay_phase_start) / num_decay_steps))
    return 1.0


class WarmupStableDecaySchedulder(LRScheduler):
    """Warmup-stable-decay; torchure/optimizer/scheduler.py:10-35."""

    def __init__(self, optimizer, total_steps, warmup_ratio, decay_ratio, last_epoch=-1):
        self.total_steps = total_steps
        self.warmup_ratio = warmup_ratio
        self.decay_ratio = decay_ratio
        super().__init__(optimizer, last_epoch)

    def get_lr(self):
        scale = wsd_scale(self.last_epoch, self.total_steps, self.warmup_ratio, self.decay_ratio)
        return [base_lr * scale for base_lr in self.base_lrs]


class CosineAnnealingScheduler(LRScheduler):
    """Placeholder kept for registry parity: torchure/optimizer/scheduler.py:38-47 is a
    stub whose get_lr returns 0, and build_scheduler refuses it."""

    def __init__(self, optimizer, total_steps, warmup_ratio, decay_phase, last_epoch):
        self.total_steps = total_steps
        self.warmup_ratio = warmup_ratio
        self.decay_phase = decay_phase
        super().__init__(optimizer, last_epoch)

    def get_lr(self):
        return [base_lr * 0 for base_lr in self.base_lrs]
