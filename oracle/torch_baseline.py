"""The reference's unfused composition in PyTorch on the host (TEST INFRASTRUCTURE ONLY).

Only ``bench.py``'s ``cpu_baseline`` leg and ``tests/`` use this module: it is
the CPU baseline the GPU op is reported next to, never part of the product.

It restates, with torch fp32 tensors on the CPU, the unfused path the
reference's own test composes (tests/test_fused_qkv_rope.py:244-259, the same
ops as attention.py:42-48): three projections ``x @ w.T``, per-head RMSNorm
``p * rsqrt(mean(p^2) + eps) * gamma`` on Q and K (fused_qkv_rope.py:98-100
arithmetic), then ``p * cos + rotate_half(p) * sin`` with ``rotate_half([x1,
x2]) = [-x2, x1]`` (mini_qwen/model/layers/rope.py:24-45), cos/sin broadcast
over heads.  Prefill mode: ``cos/sin [S, D]``.  BASELINE config 1 names this
path in fp32; the numpy oracle (qkv_rope_oracle.unfused_composition) computes
the same thing and pins it (tests/test_oracle.py).
"""
from __future__ import annotations

import torch


def unfused_composition_torch(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin, eps: float = 1e-6):
    """x [B, S, hidden], w_* [out, hidden], gammas [D], cos/sin [S, D] -> q, k, v [B, S, H, D]."""
    B, S, hidden = x.shape
    D = q_norm_w.shape[0]
    x2d = x.reshape(B * S, hidden)
    c = cos[None, :, None, :]
    s = sin[None, :, None, :]
    half = D // 2

    def norm_rope(p, gamma):
        p = p * torch.rsqrt(p.pow(2).mean(-1, keepdim=True) + eps) * gamma
        rot = torch.cat([-p[..., half:], p[..., :half]], dim=-1)
        return p * c + rot * s

    q = norm_rope((x2d @ w_q.T).view(B, S, -1, D), q_norm_w)
    k = norm_rope((x2d @ w_k.T).view(B, S, -1, D), k_norm_w)
    v = (x2d @ w_v.T).view(B, S, -1, D)
    return q, k, v
