"""Square matrix multiplication C = A @ B (spec of reference
mlx/kernels/common/sqr_mm.py:5-11, mx.matmul), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Square matrix multiplication: C = A @ B  (N x N . N x N)."""

    def forward(self, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A, B)
