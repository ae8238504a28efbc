from torchure_amd.loss.fused_linear_ce import fused_linear_cross_entropy

__all__ = ["fused_linear_cross_entropy"]
