"""W4A16 (int4 weights, bf16 activations) GEMM and the fused W4A16 QKV front.

``w4a16_gemm`` mirrors the reference's frozen signature
(mini_qwen/kernels/w4a16_gemm.py:8-15, :194-247):

    w4a16_gemm(x [M, K] bf16, qweight [K//8, N] int32, scales [K//g, N],
               qzeros [K//g, N//8] int32, group_size=128) -> [M, N] bf16

``LinearW4A16`` mirrors mini_qwen/model/layers/linear_w4a16.py (same buffers,
``from_float`` / ``from_gptq`` / ``forward``).  ``fused_qkv_rope_w4a16`` replaces
the reference's unfused W4A16 attention front (attention.py:102-109 prefill,
:136-148 decode: three w4a16_gemm launches, RMSNorm x2 and RoPE) with one
kernel whose weight stage dequantises in registers right before the MFMA.

Scales may be bf16 (the reference converts to bf16 at load,
linear_w4a16.py:95) or fp16 (AWQ checkpoints); the dequantised weight
``(q - z) * s`` is exact in fp32 and rounded once to bf16 for the MFMA.  The
kernels need K % 64 == 0 and group_size % 64 == 0.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch
import torch.nn as nn

from . import _native
from .fused_qkv_rope import EPS, _lead_shape, _positions, _require, _rope_tables, fused_ext, paged_kv
from .quantization import from_autoawq, gptq_zero_fix, per_group_minmax_quantize


def _scale_type(scales: torch.Tensor) -> int:
    if scales.dtype == torch.bfloat16:
        return _native.MQK_SCALE_BF16
    if scales.dtype == torch.float16:
        return _native.MQK_SCALE_FP16
    raise TypeError(f"scales must be bf16 or fp16, got {scales.dtype}")


def _check_int4(qweight, scales, qzeros, K, group_size, device, name):
    qweight = _require(qweight, f"{name}.qweight", device, torch.int32)
    qzeros = _require(qzeros, f"{name}.qzeros", device, torch.int32)
    scales = _require(scales, f"{name}.scales", device, None)
    st = _scale_type(scales)
    N = qweight.shape[1]
    G = K // group_size
    if qweight.shape != (K // 8, N) or scales.shape != (G, N) or qzeros.shape != (G, N // 8):
        raise ValueError(
            f"{name}: qweight {tuple(qweight.shape)}, scales {tuple(scales.shape)}, qzeros "
            f"{tuple(qzeros.shape)} do not match K={K}, N={N}, group={group_size}")
    return qweight, scales, qzeros, st


def w4a16_gemm(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor,
               qzeros: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """``x @ dequant(qweight)``: ``[M, K] bf16 -> [M, N] bf16``."""
    if x.dim() != 2:
        raise ValueError("x must be [M, K]")
    M, K = x.shape
    device = x.device
    x = _require(x, "x", device)
    if K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    qweight, scales, qzeros, st = _check_int4(qweight, scales, qzeros, K, group_size, device, "w4a16")
    N = qweight.shape[1]
    if N % 8 != 0:
        raise ValueError(f"N={N} must be a multiple of 8")
    out = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    if M == 0:
        return out
    lib = _native.library()
    stream = _native.stream_handle(device)
    ws = _native.workspace(device, stream, int(lib.mqk_w4a16_gemm_workspace_size(M, K, N)))
    status = _native.call(device, lib.mqk_w4a16_gemm_ex,
        x.data_ptr(), qweight.data_ptr(), scales.data_ptr(), qzeros.data_ptr(), M, K, N,
        group_size, st, out.data_ptr(), _native.ptr(ws), 0 if ws is None else ws.numel(), stream)
    _native.check(status, "mqk_w4a16_gemm_ex")
    return out


class LinearW4A16(nn.Module):
    """Quantized linear layer with packed int4 weights (linear_w4a16.py:8-106)."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 128,
                 scale_dtype=torch.bfloat16):
        super().__init__()
        if in_features % group_size != 0:
            raise ValueError(f"in_features={in_features} not divisible by group_size={group_size}")
        if out_features % 8 != 0:
            raise ValueError(f"out_features={out_features} must be a multiple of 8")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        G = in_features // group_size
        self.register_buffer("qweight", torch.zeros(in_features // 8, out_features, dtype=torch.int32))
        self.register_buffer("scales", torch.zeros(G, out_features, dtype=scale_dtype))
        self.register_buffer("qzeros", torch.zeros(G, out_features // 8, dtype=torch.int32))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        out = w4a16_gemm(x.reshape(-1, self.in_features), self.qweight, self.scales, self.qzeros,
                         self.group_size)
        return out.reshape(*lead, self.out_features)

    @classmethod
    def from_float(cls, linear: nn.Linear, group_size: int = 128) -> "LinearW4A16":
        """Quantize an ``nn.Linear`` (weight ``[N, K]``) with per-group min-max."""
        w = linear.weight.data.float().T.contiguous()
        K, N = w.shape
        qweight, scales, qzeros = per_group_minmax_quantize(w, group_size)
        layer = cls(K, N, group_size).to(w.device)
        layer.qweight.copy_(qweight)
        layer.scales.copy_(scales)
        layer.qzeros.copy_(qzeros)
        return layer

    @classmethod
    def from_gptq(cls, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                  group_size: int = 128, zero_plus_one: bool = True) -> "LinearW4A16":
        """Build from GPTQ buffers in this layout; v1 checkpoints store ``z - 1``."""
        K, N = qweight.shape[0] * 8, qweight.shape[1]
        layer = cls(K, N, group_size).to(qweight.device)
        layer.qweight.copy_(qweight.to(torch.int32))
        layer.scales.copy_(scales.to(torch.bfloat16))
        layer.qzeros.copy_(gptq_zero_fix(qzeros) if zero_plus_one else qzeros.to(torch.int32))
        return layer

    @classmethod
    def from_autoawq(cls, qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                     group_size: int = 128) -> "LinearW4A16":
        """Build from an AutoAWQ checkpoint (qweight [K, N/8] packed along N with the
        AWQ nibble order, fp16 scales).  The values are repacked, not requantised;
        the fp16 scales are kept (the kernels read fp16 or bf16 scales)."""
        qw, sc, qz = from_autoawq(qweight, qzeros, scales)
        K, N = qw.shape[0] * 8, qw.shape[1]
        layer = cls(K, N, group_size, scale_dtype=sc.dtype).to(qw.device)
        layer.qweight.copy_(qw)
        layer.scales.copy_(sc)
        layer.qzeros.copy_(qz)
        return layer

    def extra_repr(self) -> str:
        return f"in={self.in_features}, out={self.out_features}, group_size={self.group_size}"


Int4Weights = Tuple[torch.Tensor, torch.Tensor, torch.Tensor]  # (qweight, scales, qzeros)


def _as_int4(p) -> Int4Weights:
    if isinstance(p, LinearW4A16):
        return p.qweight, p.scales, p.qzeros
    qweight, scales, qzeros = p
    return qweight, scales, qzeros


def fused_qkv_rope_w4a16(
    x: torch.Tensor,
    q_proj,
    k_proj,
    v_proj,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
    group_size: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """W4A16 twin of :func:`mqk.fused_qkv_rope`.

    ``q_proj/k_proj/v_proj`` are ``LinearW4A16`` modules or ``(qweight, scales,
    qzeros)`` tuples.  Same layouts, position rules and outputs as the bf16 op.
    The norm is applied in fp32 to the accumulator (the reference's unfused
    front rounds to bf16 before multiplying by the norm weight,
    rms_norm.py:15-18; the difference is below one bf16 ulp of the output).
    """
    return _fused_w4a16(x, q_proj, k_proj, v_proj, q_norm_w, k_norm_w, cos, sin, positions, group_size)


def fused_qkv_rope_w4a16_paged(
    x: torch.Tensor,
    q_proj,
    k_proj,
    v_proj,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
    kv_seq: Optional[torch.Tensor] = None,
    kv_pos: Optional[torch.Tensor] = None,
    return_kv: bool = True,
    group_size: Optional[int] = None,
):
    """:func:`fused_qkv_rope_w4a16` that also writes K and V into a paged KV cache
    (see :func:`mqk.fused_qkv_rope_paged`)."""
    return _fused_w4a16(x, q_proj, k_proj, v_proj, q_norm_w, k_norm_w, cos, sin, positions, group_size,
                        paged=(k_cache, v_cache, block_table, kv_seq, kv_pos), return_kv=return_kv)


def fused_qkv_rope_w4a16_ex(
    x: torch.Tensor,
    q_proj,
    k_proj,
    v_proj,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
    *,
    group_size: Optional[int] = None,
    cu_seqlens: Optional[torch.Tensor] = None,
    seq_pos0: Optional[torch.Tensor] = None,
    input_norm_w: Optional[torch.Tensor] = None,
    input_eps: float = EPS,
    k_cache: Optional[torch.Tensor] = None,
    v_cache: Optional[torch.Tensor] = None,
    block_table: Optional[torch.Tensor] = None,
    kv_seq: Optional[torch.Tensor] = None,
    kv_pos: Optional[torch.Tensor] = None,
    return_kv: bool = True,
):
    """W4A16 twin of :func:`mqk.fused_qkv_rope_ex` (varlen positions, input RMSNorm,
    paged-KV-cache write)."""
    return _fused_w4a16(x, q_proj, k_proj, v_proj, q_norm_w, k_norm_w, cos, sin, positions, group_size,
                        return_kv=return_kv,
                        ext_args=dict(cu_seqlens=cu_seqlens, seq_pos0=seq_pos0, input_norm_w=input_norm_w,
                                      input_eps=input_eps, k_cache=k_cache, v_cache=v_cache,
                                      block_table=block_table, kv_seq=kv_seq, kv_pos=kv_pos))


def _fused_w4a16(x, q_proj, k_proj, v_proj, q_norm_w, k_norm_w, cos, sin, positions, group_size,
                 paged=None, return_kv=True, ext_args=None):
    lead, S = _lead_shape(x, None if ext_args is None else ext_args.get("cu_seqlens"))
    H = x.shape[-1]
    D = q_norm_w.shape[0]
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    if group_size is None:
        group_size = q_proj.group_size if isinstance(q_proj, LinearW4A16) else 128
    device = x.device
    x = _require(x, "x", device)
    q_norm_w = _require(q_norm_w, "q_norm_w", device)
    k_norm_w = _require(k_norm_w, "k_norm_w", device)
    parts = []
    sts = []
    for name, proj in (("q_proj", q_proj), ("k_proj", k_proj), ("v_proj", v_proj)):
        qw, sc, qz, st = _check_int4(*_as_int4(proj), H, group_size, device, name)
        parts.append((qw, sc, qz))
        sts.append(st)
    if len(set(sts)) != 1:
        raise TypeError("q/k/v scales must share one dtype")
    H_Q = parts[0][0].shape[1] // D
    H_KV = parts[1][0].shape[1] // D
    if parts[0][0].shape[1] != H_Q * D or parts[1][0].shape[1] != H_KV * D or \
            parts[2][0].shape[1] != H_KV * D:
        raise ValueError("projection widths must be whole heads (H_Q*D, H_KV*D, H_KV*D)")
    cos, sin = _rope_tables(cos, sin, D, device)
    T = x.numel() // H
    pos = _positions(positions, T, device)
    desc = keep = ext = None
    if paged is not None:
        desc, keep = paged_kv(*paged, T, H_KV, D, device, positions)
    if ext_args is not None:
        ext, keep = fused_ext(T, H_KV, D, H, device, positions, **ext_args)
        if not return_kv and not ext.kv:
            raise ValueError("return_kv=False needs a paged cache")
    q = torch.empty(*lead, H_Q, D, dtype=torch.bfloat16, device=device)
    k = torch.empty(*lead, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    v = torch.empty(*lead, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    if T == 0:
        return q, k, v
    lib = _native.library()
    stream = _native.stream_handle(device)
    if ext is not None:
        nbytes = _native.fused_workspace_bytes(T, H_Q, H_KV, H, D, ext)
    else:
        nbytes = _native.fused_workspace_bytes(T, H_Q, H_KV, H, D)
    ws = _native.workspace(device, stream, nbytes)
    flat = [t.data_ptr() for trio in parts for t in trio]
    head = (x.data_ptr(), *flat, group_size, sts[0],
            q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            _native.ptr(pos), T, S, H, H_Q, H_KV, D, cos.shape[0], EPS,
            q.data_ptr(), _native.ptr(k), _native.ptr(v))
    tail = (_native.ptr(ws), 0 if ws is None else ws.numel(), stream)
    if ext is not None:
        status = _native.call(device, lib.mqk_fused_qkv_rope_ex_w4a16, *head, ctypes.byref(ext), *tail)
        _native.check(status, "mqk_fused_qkv_rope_ex_w4a16")
    elif desc is None:
        status = _native.call(device, lib.mqk_fused_qkv_rope_w4a16, *head, *tail)
        _native.check(status, "mqk_fused_qkv_rope_w4a16")
    else:
        status = _native.call(device, lib.mqk_fused_qkv_rope_paged_w4a16, *head, ctypes.byref(desc), *tail)
        _native.check(status, "mqk_fused_qkv_rope_paged_w4a16")
    del keep
    return q, k, v
