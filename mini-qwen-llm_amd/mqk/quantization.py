"""int4 weight format of the W4A16 path (offline / load-time host utilities).

Format (reference mini_qwen/quantization/packing.py:1-9, w4a16_gemm.py:8-15):
  * qweight [K // 8, N] int32, packed along K: nibble i (bits 4i..4i+3) of
    qweight[j, n] is W[8j + i, n] (little-endian nibbles, no AutoAWQ interleave);
  * qzeros  [K // g, N // 8] int32, packed along N the same way;
  * scales  [K // g, N] (bf16 in the reference; fp16 accepted by the kernels);
  * dequant: W[k, n] = (q[k, n] - z[k // g, n]) * s[k // g, n].

These run in plain torch on any device; they are not on the per-token path.
"""
from __future__ import annotations

import torch
from torch import Tensor

_SHIFTS = (0, 4, 8, 12, 16, 20, 24, 28)


def _shifts(device) -> Tensor:
    return torch.tensor(_SHIFTS, dtype=torch.int32, device=device)


def pack_int4(x: Tensor) -> Tensor:
    """``[..., K]`` values in 0..15 -> ``[..., K // 8]`` int32 (packing.py:11-24)."""
    if x.shape[-1] % 8 != 0:
        raise ValueError(f"last dimension must be a multiple of 8, got {x.shape[-1]}")
    v = x.reshape(*x.shape[:-1], -1, 8).to(torch.int32) & 0xF
    # OR of disjoint nibbles in int64, then reinterpreted as int32 (the top
    # nibble lands in the sign bit, as in the reference's int32 arithmetic).
    acc = torch.zeros(v.shape[:-1], dtype=torch.int64, device=v.device)
    for i, s in enumerate(_SHIFTS):
        acc |= v[..., i].to(torch.int64) << s
    acc = torch.where(acc >= (1 << 31), acc - (1 << 32), acc)
    return acc.to(torch.int32)


def unpack_int4(packed: Tensor) -> Tensor:
    """Inverse of :func:`pack_int4` (packing.py:27-39): ``[..., K // 8]`` -> ``[..., K]``."""
    p = packed.to(torch.int32)
    v = (p.unsqueeze(-1) >> _shifts(packed.device)) & 0xF
    return v.reshape(*p.shape[:-1], -1).to(torch.int32)


def per_group_minmax_quantize(w: Tensor, group_size: int = 128, scale_dtype=torch.bfloat16):
    """Per-group min-max int4 quantization of ``w [K, N]`` (awq.py:14-58).

    scales = ((max - min) / 15).clamp(min=1e-8); zeros = round(-min / scales)
    clamped to 0..15; q = round(w / scales + zeros) clamped to 0..15.  Returns
    ``(qweight [K//8, N] int32, scales [K//g, N] scale_dtype, qzeros [K//g, N//8] int32)``.
    """
    K, N = w.shape
    if K % group_size != 0:
        raise ValueError(f"K={K} must be divisible by group_size={group_size}")
    if N % 8 != 0:
        raise ValueError(f"N={N} must be a multiple of 8 (qzeros packed along N)")
    wg = w.float().reshape(K // group_size, group_size, N)
    wmax = wg.amax(dim=1)
    wmin = wg.amin(dim=1)
    scales = ((wmax - wmin) / 15.0).clamp(min=1e-8)
    zeros = (-wmin / scales).round().clamp(0, 15).to(torch.int32)
    q = (wg / scales[:, None, :] + zeros[:, None, :].float()).round().clamp(0, 15).to(torch.int32)
    qweight = pack_int4(q.reshape(K, N).T.contiguous()).T.contiguous()
    qzeros = pack_int4(zeros)
    return qweight, scales.to(scale_dtype), qzeros


def dequantize(qweight: Tensor, scales: Tensor, qzeros: Tensor, group_size: int = 128) -> Tensor:
    """fp32 ``[K, N]`` = ``(q - z) * s`` (the format's definition; w4a16_gemm.py:90-92)."""
    q = unpack_int4(qweight.T.contiguous()).T.float()
    z = unpack_int4(qzeros).float()
    s = scales.float()
    K, N = q.shape
    G = K // group_size
    return ((q.reshape(G, group_size, N) - z[:, None, :]) * s[:, None, :]).reshape(K, N)


def gptq_zero_fix(qzeros: Tensor) -> Tensor:
    """GPTQ v1 stores ``z - 1``: add 1 and clamp to 0..15 (linear_w4a16.py:96-99)."""
    return pack_int4((unpack_int4(qzeros.to(torch.int32)) + 1).clamp(0, 15))


# AutoAWQ ("GEMM" kernels) checkpoint layout: qweight [K, N // 8] and qzeros
# [K // g, N // 8] int32 packed along N, nibble i of a word holding column
# 8*j + AWQ_ORDER[i] of its 8-column group; scales [K // g, N] fp16.
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _unpack_awq_cols(packed: Tensor) -> Tensor:
    """AutoAWQ words ``[R, N // 8]`` -> values ``[R, N]`` in natural column order."""
    nib = unpack_int4(packed.to(torch.int32))            # [R, N], nibble order
    R, N = nib.shape
    nib = nib.view(R, N // 8, 8)
    out = torch.empty_like(nib)
    for i, c in enumerate(AWQ_ORDER):
        out[:, :, c] = nib[:, :, i]
    return out.view(R, N)


def from_autoawq(qweight: Tensor, qzeros: Tensor, scales: Tensor):
    """Repack an AutoAWQ checkpoint tensor triple into this package's int4 format.

    AutoAWQ packs along N with the nibble order ``AWQ_ORDER``; this format packs
    qweight along K in natural order (packing.py:11-24) and qzeros along N in
    natural order.  The integer values and the scales are unchanged, so the
    dequantised weight is identical.  Returns ``(qweight [K//8, N], scales
    [K//g, N] (dtype kept), qzeros [K//g, N//8])``.
    """
    K, n8 = qweight.shape
    N = n8 * 8
    if qzeros.shape[1] != n8 or scales.shape[1] != N or scales.shape[0] != qzeros.shape[0]:
        raise ValueError(f"inconsistent AutoAWQ shapes: qweight {tuple(qweight.shape)}, "
                         f"qzeros {tuple(qzeros.shape)}, scales {tuple(scales.shape)}")
    if K % 8 != 0:
        raise ValueError(f"K={K} must be a multiple of 8")
    w = _unpack_awq_cols(qweight)                         # [K, N]
    z = _unpack_awq_cols(qzeros)                          # [K//g, N]
    new_qweight = pack_int4(w.T.contiguous()).T.contiguous()
    new_qzeros = pack_int4(z)
    return new_qweight, scales, new_qzeros
