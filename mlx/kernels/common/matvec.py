"""Matrix-vector product y = A @ x (spec of reference mlx/kernels/common/matvec.py:5-10,
mx.matmul), run on the host CPU in fp32."""
import torch


class Model(torch.nn.Module):
    """Matrix-vector multiplication: y = A @ x  (M x K . K -> M)."""

    def forward(self, A: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        return torch.matmul(A, x)
