from torchure_amd.optimizer.adamw import AdamW
from torchure_amd.optimizer.builder import (
    OPTIMIZER_REGISTRY,
    SCHEDULER_REGISTRY,
    build_optimizer,
    build_scheduler,
    split_param_groups,
)
from torchure_amd.optimizer.scheduler import (
    CosineAnnealingScheduler,
    WarmupStableDecaySchedulder,
    wsd_scale,
)
from torchure_amd.optimizer.working import (
    accumulate_grad_,
    accumulate_grads_,
    attach_bf16_working_params,
    refresh_bf16_working_params,
)

__all__ = [
    "AdamW",
    "OPTIMIZER_REGISTRY",
    "SCHEDULER_REGISTRY",
    "build_optimizer",
    "build_scheduler",
    "split_param_groups",
    "CosineAnnealingScheduler",
    "WarmupStableDecaySchedulder",
    "wsd_scale",
    "accumulate_grad_",
    "accumulate_grads_",
    "attach_bf16_working_params",
    "refresh_bf16_working_params",
]
