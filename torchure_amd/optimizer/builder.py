"""Optimizer / scheduler registry; same names and behaviour as torchure/optimizer/builder.py.

``build_optimizer`` splits params into the two groups of builder.py:31-46
(weight decay on >=2-D tensors, 0.0 on 1-D), in ``model.parameters()`` order,
and passes the remaining config keys (lr, betas, fused, ...) through. The
"adamw" entry is this package's fused gfx950 AdamW instead of torch.optim.AdamW.
"""

from __future__ import annotations

import torch.nn as nn
import torch.optim as optim

from torchure_amd.optimizer.adamw import AdamW
from torchure_amd.optimizer.scheduler import CosineAnnealingScheduler, WarmupStableDecaySchedulder

OPTIMIZER_REGISTRY = {
    "adamw": AdamW,
    "sgd": optim.SGD,
}

SCHEDULER_REGISTRY = {
    "wsd": WarmupStableDecaySchedulder,
    "cosine": CosineAnnealingScheduler,
}


def split_param_groups(params, weight_decay: float) -> list[dict]:
    """builder.py:37-43: decay group (dim >= 2) then no-decay group (dim < 2)."""
    params = [p for p in params if p.requires_grad]
    return [
        {"params": [p for p in params if p.dim() >= 2], "weight_decay": weight_decay},
        {"params": [p for p in params if p.dim() < 2], "weight_decay": 0.0},
    ]


def build_optimizer(model: nn.Module, optim_name: str, optim_config: dict) -> optim.Optimizer:
    cfg = dict(optim_config)
    weight_decay = cfg.pop("weight_decay", 0.0)
    param_groups = split_param_groups(model.parameters(), weight_decay)
    return OPTIMIZER_REGISTRY[optim_name](param_groups, **cfg)


def build_scheduler(optimizer: optim.Optimizer, scheduler_config: dict) -> optim.lr_scheduler.LRScheduler:
    scheduler_cfg = dict(scheduler_config)
    scheduler_type = scheduler_cfg["type"]
    if scheduler_type == "cosine":
        raise NotImplementedError("cosine scheduler is a stub (get_lr returns 0); use wsd")
    scheduler_cfg.pop("type")
    scheduler_cfg["optimizer"] = optimizer
    return SCHEDULER_REGISTRY[scheduler_type](**scheduler_cfg)
