from torchure_amd.core.grad_helper import clip_grad_norm

__all__ = ["clip_grad_norm"]
