"""Batched matrix multiplication C[b] = A[b] @ B[b] (spec of reference
mlx/kernels/common/batch_mm.py:5-10, mx.matmul), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Batched matrix multiplication: C[b] = A[b] @ B[b]."""

    def forward(self, A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A, B)
