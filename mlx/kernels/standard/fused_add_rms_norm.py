"""Residual add + RMSNorm, y = RMSNorm(x + residual) (spec of reference
mlx/kernels/standard/fused_add_rms_norm.py:5-12: nn.RMSNorm, unit gain at
init), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Residual + RMSNorm: y = RMSNorm(x + residual)."""

    def __init__(self, dim: int = 1024, eps: float = 1e-5):
        super().__init__()
        self.weight = torch.ones(dim)
        self.eps = eps

    def forward(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        v = x + residual
        return v * torch.rsqrt(torch.mean(v * v, dim=-1, keepdim=True) + self.eps) * self.weight
