"""LLaMA decoder layer, prefill (spec of reference
mlx/kernels/full/llama_decoder_layer.py:5-64), run on the host CPU in fp32:
RMSNorm (no gain) -> x @ W_qkv -> RoPE on q, k (positions 0..S-1, interleaved
pairs, omega_i = base^(-2i/Dh)) -> GQA softmax attention over all S positions
(query head h reads kv head h // G) -> @ W_o + x -> RMSNorm -> SwiGLU over the
[gate | up] halves of W_gu -> @ W_down + residual.  Computed in float64: with
the reference's normal(0, 1) weights the outputs reach the thousands, where
fp32 rounding alone exceeds the registry's atol on near-zero outputs."""
import math

import torch
import torch.nn.functional as F


class Model(torch.nn.Module):
    """Full LLaMA decoder layer: (S, D) -> (S, D)."""

    def __init__(self, S=64, D=128, H=4, H_kv=2, FF=256, base=10000.0, eps=1e-5):
        super().__init__()
        self.S, self.D, self.H, self.H_kv, self.FF = S, D, H, H_kv, FF
        self.base, self.eps = base, eps
        self.D_head = D // H
        self.G = H // H_kv

    def _rms_norm(self, x):
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + self.eps)

    def _rope(self, t):
        heads, S, Dh = t.shape
        idx = torch.arange(Dh // 2, dtype=torch.float64)
        omega = 1.0 / (self.base ** (2.0 * idx / Dh))
        ang = torch.arange(S, dtype=torch.float64)[:, None] * omega[None, :]
        c, s = torch.cos(ang), torch.sin(ang)
        t0, t1 = t[..., 0::2], t[..., 1::2]
        return torch.stack([t0 * c - t1 * s, t0 * s + t1 * c], dim=-1).reshape(heads, S, Dh)

    def forward(self, x, W_qkv, W_o, W_gu, W_down):
        out_dtype = x.dtype
        x, W_qkv, W_o, W_gu, W_down = (t.double() for t in (x, W_qkv, W_o, W_gu, W_down))
        S, D, H, H_kv, Dh, FF = self.S, self.D, self.H, self.H_kv, self.D_head, self.FF
        qkv = self._rms_norm(x) @ W_qkv
        q = qkv[:, :D].reshape(S, H, Dh).transpose(0, 1)
        k = qkv[:, D:D + H_kv * Dh].reshape(S, H_kv, Dh).transpose(0, 1)
        v = qkv[:, D + H_kv * Dh:].reshape(S, H_kv, Dh).transpose(0, 1)
        q, k = self._rope(q), self._rope(k)
        k = k.repeat_interleave(self.G, dim=0)
        v = v.repeat_interleave(self.G, dim=0)
        attn = torch.softmax((q @ k.transpose(1, 2)) / math.sqrt(Dh), dim=-1) @ v
        x = x + attn.transpose(0, 1).reshape(S, D) @ W_o
        gu = self._rms_norm(x) @ W_gu
        return (x + (F.silu(gu[:, :FF]) * gu[:, FF:]) @ W_down).to(out_dtype)
