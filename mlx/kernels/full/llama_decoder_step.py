"""LLaMA decoder layer, one decode step: spec run on the host CPU in fp32.

The math follows reference mlx/kernels/full/llama_decoder_layer.py:24-64 —
RMSNorm without gain (:48-50), interleaved-pair RoPE with omega_i =
base^(-2i/Dh) (:52-64), GQA where query head h reads kv head h // G (mx.repeat
along the head axis, :34), softmax(q k^T / sqrt(Dh)) v, W_o + residual, RMSNorm,
SwiGLU (silu(gate) * up, :41-45), W_down + residual — applied to one new token
per sequence: its position is L (the cache length), and it attends to the L
cached (already rotated) keys plus its own.  bf16 inputs are widened to fp32.
"""
import math

import torch
import torch.nn.functional as F


class Model(torch.nn.Module):
    """One decode step of a LLaMA decoder layer.

    Inputs (QD = H * D_head; QD = D for a whole layer, QD < D for the work
    of one tensor-parallel shard at its real shapes -- a cost proxy: the full
    residual is added and the shard's own partial x1 normalised, so shards'
    outputs do not sum to the layer's):
        x        (B, D)
        W_qkv    (D, QD + 2*H_kv*D_head)  columns [Q | K | V]
        W_o      (QD, D)
        W_gu     (D, 2*FF)                columns [gate | up]
        W_down   (FF, D)
        K_cache  (B, H_kv, L, D_head)     rotated keys of positions 0..L-1
        V_cache  (B, H_kv, L, D_head)
    Outputs: y (B, D), k_new (B, H_kv, D_head), v_new (B, H_kv, D_head)
    """

    def __init__(self, B=16, D=4096, H=32, H_kv=8, FF=14336, L=2048, base=500000.0, eps=1e-5,
                 D_head=None):
        super().__init__()
        self.B, self.D, self.H, self.H_kv, self.FF, self.L = B, D, H, H_kv, FF, L
        self.base, self.eps = base, eps
        self.D_head = D // H if D_head is None else D_head
        self.QD = H * self.D_head
        self.G = H // H_kv

    def forward(self, x, W_qkv, W_o, W_gu, W_down, K_cache, V_cache):
        B, QD, H, H_kv, Dh, FF, G = self.B, self.QD, self.H, self.H_kv, self.D_head, self.FF, self.G
        x = x.float()

        # ---- attention ----
        h = self._rms_norm(x)
        qkv = h @ W_qkv.float()
        q = qkv[:, :QD].reshape(B, H, Dh)
        k = qkv[:, QD:QD + H_kv * Dh].reshape(B, H_kv, Dh)
        v = qkv[:, QD + H_kv * Dh:].reshape(B, H_kv, Dh)
        q = self._rope(q, self.L)
        k = self._rope(k, self.L)
        keys = torch.cat([K_cache.float(), k[:, :, None, :]], dim=2)     # (B, H_kv, L+1, Dh)
        vals = torch.cat([V_cache.float(), v[:, :, None, :]], dim=2)
        qg = q.reshape(B, H_kv, G, Dh)                                   # head h -> kv head h // G
        scores = (qg @ keys.transpose(2, 3)) / math.sqrt(Dh)             # (B, H_kv, G, L+1)
        attn = torch.softmax(scores, dim=-1)
        out = (attn @ vals).reshape(B, QD) @ W_o.float()
        x = x + out

        # ---- SwiGLU FFN ----
        h = self._rms_norm(x)
        gu = h @ W_gu.float()
        ff = (F.silu(gu[:, :FF]) * gu[:, FF:]) @ W_down.float()
        return x + ff, k, v

    def _rms_norm(self, x):
        v = torch.mean(x * x, dim=-1, keepdim=True)
        return x * torch.rsqrt(v + self.eps)

    def _rope(self, t, pos):
        half = self.D_head // 2
        idx = torch.arange(half, dtype=torch.float32)
        omega = 1.0 / (self.base ** (2.0 * idx / self.D_head))
        ang = float(pos) * omega
        c, s = torch.cos(ang), torch.sin(ang)
        t0, t1 = t[..., 0::2], t[..., 1::2]
        r0 = t0 * c - t1 * s
        r1 = t0 * s + t1 * c
        return torch.stack([r0, r1], dim=-1).reshape(t.shape)
