"""2D transpose B = A^T (spec of reference mlx/kernels/common/transpose_2d.py:5-11,
mx.transpose), run on the host CPU."""
import torch


class Model(torch.nn.Module):
    """2D transpose: B = A^T."""

    def forward(self, A: torch.Tensor) -> torch.Tensor:
        return A.t().contiguous()
