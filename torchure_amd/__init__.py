"""torchure_amd: MI355X-native mixed-precision optimizer step for torchure.

Drop-in for torchure's optimizer tail (clip_grad_norm -> AdamW.step ->
zero_grad -> scheduler.step) on hand-written gfx950 HIP kernels reached
through a C ABI (include/torchure_amd.h, libtorchure_amd.so).
"""

from torchure_amd import _native
from torchure_amd.core.grad_helper import clip_grad_norm
from torchure_amd.optimizer import (
    AdamW,
    WarmupStableDecaySchedulder,
    attach_bf16_working_params,
    build_optimizer,
    build_scheduler,
    refresh_bf16_working_params,
)

__all__ = [
    "_native",
    "clip_grad_norm",
    "AdamW",
    "WarmupStableDecaySchedulder",
    "attach_bf16_working_params",
    "build_optimizer",
    "build_scheduler",
    "refresh_bf16_working_params",
]
