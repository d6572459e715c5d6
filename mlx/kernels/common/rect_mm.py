"""Rectangular matrix multiplication C = A @ B (spec of reference
mlx/kernels/common/rect_mm.py:10-11, mx.matmul), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Rectangular matrix multiplication: C = A @ B  (M x K . K x N)."""

    def forward(self, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A, B)
