"""2D convolution, NHWC input x OHWI weight (spec of reference
mlx/kernels/common/conv2d.py:5-12, mx.conv2d: cross-correlation, dilation 1,
groups 1), run on the host CPU in fp32.  `padding` is new: the reference
Model hard-codes padding=0."""
import torch
import torch.nn.functional as F


class Model(torch.nn.Module):
    """2D convolution: out = conv2d(x, weight)."""

    def __init__(self, in_channels=64, out_channels=64, kernel_size=3, stride=1, padding=1):
        super().__init__()
        self.in_c, self.out_c, self.ks = in_channels, out_channels, kernel_size
        self.st, self.pad = stride, padding

    def forward(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        # NHWC -> NCHW and OHWI -> OIHW for torch, then back to NHWC.
        y = F.conv2d(x.permute(0, 3, 1, 2), w.permute(0, 3, 1, 2),
                     stride=self.st, padding=self.pad, dilation=1, groups=1)
        return y.permute(0, 2, 3, 1).contiguous()
