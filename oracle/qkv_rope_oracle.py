"""CPU oracle for the fused QKV + QK-Norm + RoPE path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``mqk``) never calls into it and fails loudly
when its HIP library is missing.

It restates, in numpy, the arithmetic of the reference (mini-qwen-llm) for the
path ``x -> Q/K/V projection -> per-head RMSNorm over head_dim -> rotate-half
RoPE`` and its W4A16 twin.  Each function cites the reference file:line it
follows.  bf16 values are carried as ``uint16`` bit patterns and widened to
float32/float64 exactly; rounding back to bf16 is round-to-nearest-even.

Pinning (what checks each function against something other than itself):
  * bf16 helpers        -- exhaustive round trip of all 65536 patterns, known
                           RNE tie cases, ml_dtypes-free bit arithmetic.
  * rope_tables         -- closed form cos(p * theta^(-2i/D)) in float64, the
                           ``cat([f, f])`` layout (cos1 == cos2), position 0.
  * qk_norm / rope      -- closed forms (constant, one-hot, zero vectors),
                           norm preservation, p then -p identity, and an
                           independent complex-number formulation of RoPE.
  * projection          -- brute-force triple loop on tiny shapes.
  * row selection       -- prefill ``t % S`` vs positions mode, sentinel tables.
  * varlen_positions    -- hand-worked offsets with an empty sequence, and a
                           brute-force scan of cu_seqlens for every token.
  * paged_slot          -- hand-worked slots of a small block table, and a
                           brute-force scan of every slot of the cache.
  * int4 pack/unpack    -- hand-packed 0x76543210 known answer, round trips.
  * awq_unpack          -- hand-packed 0x75316420 known answer (AutoAWQ's
                           nibble order), brute-force per-nibble decode.
  * minmax quantizer    -- hand-computed group, error <= scale/2, zero exact.
  * dequant / w4a16     -- brute-force nibble-by-nibble restatement.
There is no function here marked "parity unpinned"; the GEMM's bf16 bit pattern
of the reference's vendor library (cuBLAS) is not reproducible anywhere, so V
parity is stated as a tolerance plus "within one bf16 ulp" (see tests).
"""
from __future__ import annotations

import numpy as np

HEAD_DIM = 128
DEFAULT_EPS = 1e-6
DEFAULT_THETA = 1.0e6


# ---------------------------------------------------------------------------
# bf16 <-> float helpers (bit-level, round-to-nearest-even)
# ---------------------------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 (or float64, first rounded to float32) to bf16 bits, RNE.

    NaN inputs map to the canonical quiet NaN 0x7FC0.
    """
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    rounded = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded = np.where(nan, np.uint16(0x7FC0), rounded)
    return rounded.reshape(f.shape)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Value of ``x`` after one rounding to bf16, as float32."""
    return bf16_to_f32(f32_to_bf16(x))


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen fp16 bit patterns (uint16) to float32 exactly."""
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------
# RoPE tables  (mini_qwen/model/layers/rope.py:6-21)
# ---------------------------------------------------------------------------

def rope_tables(head_dim: int, max_seq_len: int, theta: float = DEFAULT_THETA,
                dtype=np.float32):
    """cos/sin tables ``[max_seq_len, head_dim]``.

    rope.py:9   inv_freq = 1 / theta ** (arange(0, D, 2) / D)      (fp32)
    rope.py:14  freqs    = outer(arange(max_seq_len), inv_freq)
    rope.py:15  emb      = cat([freqs, freqs], -1)
    rope.py:16-17 cos/sin of emb.
    ``dtype=np.float64`` gives the exact-math table used to pin the fp32 one.
    """
    exps = np.arange(0, head_dim, 2, dtype=dtype) / dtype(head_dim)
    inv_freq = dtype(1.0) / (dtype(theta) ** exps)
    t = np.arange(max_seq_len, dtype=dtype)
    freqs = np.outer(t, inv_freq).astype(dtype)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(dtype), np.sin(emb).astype(dtype)


# ---------------------------------------------------------------------------
# Projection  (mini_qwen/kernels/fused_qkv_rope.py:164-169)
# ---------------------------------------------------------------------------

def projection(x2d: np.ndarray, w: np.ndarray, dtype=np.float64) -> np.ndarray:
    """``x2d @ w.T`` for ``x2d [T, hidden]``, ``w [out, hidden]`` (nn.Linear layout)."""
    return np.asarray(x2d, dtype=dtype) @ np.asarray(w, dtype=dtype).T


# ---------------------------------------------------------------------------
# Row selection for the RoPE tables  (fused_qkv_rope.py:106-111)
# ---------------------------------------------------------------------------

def rope_rows(T: int, S: int, positions=None) -> np.ndarray:
    """Row of cos/sin used by token ``t``.

    prefill (positions is None): ``t % S``          (fused_qkv_rope.py:109)
    positions mode:              ``positions[t]``   (fused_qkv_rope.py:107)
    """
    if positions is None:
        return np.arange(T, dtype=np.int64) % int(S)
    p = np.asarray(positions).astype(np.int64).reshape(-1)
    assert p.shape[0] == T
    return p


def varlen_positions(cu_seqlens, seq_pos0=None):
    """``(batch_ids, positions)`` of packed sequences, as paged_attn_prefill derives
    them from ``cu_seqlens`` (mini_qwen/kernels/paged_attn_prefill.py:188-199):
    ``batch_ids = repeat_interleave(arange(B), lengths)``,
    ``positions = arange(total) - cu_seqlens[batch_ids]``; with ``seq_pos0`` the
    position of each sequence's first token is added (continued sequences).
    """
    cu = np.asarray(cu_seqlens, dtype=np.int64).reshape(-1)
    lengths = cu[1:] - cu[:-1]
    batch = np.repeat(np.arange(lengths.shape[0], dtype=np.int64), lengths)
    pos = np.arange(batch.shape[0], dtype=np.int64) - cu[batch]
    if seq_pos0 is not None:
        pos = pos + np.asarray(seq_pos0, dtype=np.int64).reshape(-1)[batch]
    return batch, pos


# ---------------------------------------------------------------------------
# QK-Norm + RoPE on one projection  (fused_qkv_rope.py:84-118)
# ---------------------------------------------------------------------------

def qk_norm(raw: np.ndarray, gamma: np.ndarray, eps: float = DEFAULT_EPS,
            dtype=np.float64) -> np.ndarray:
    """Per-head RMSNorm over the last axis.

    fused_qkv_rope.py:98   rms = rsqrt((sum(x1^2) + sum(x2^2)) / D + EPS)
    fused_qkv_rope.py:99-100  x_n = x * rms * w
    """
    r = np.asarray(raw, dtype=dtype)
    D = r.shape[-1]
    ss = np.sum(r * r, axis=-1, keepdims=True)
    rms = 1.0 / np.sqrt(ss / D + eps)
    return r * rms * np.asarray(gamma, dtype=dtype)


def rope(xn: np.ndarray, cos_rows: np.ndarray, sin_rows: np.ndarray,
         dtype=np.float64) -> np.ndarray:
    """Rotate-half RoPE, ``xn [T, H, D]``, ``cos_rows/sin_rows [T, D]``.

    fused_qkv_rope.py:117  out1 = x1_n * cos1 - x2_n * sin1
    fused_qkv_rope.py:118  out2 = x2_n * cos2 + x1_n * sin2
    Both halves of cos/sin are read separately (cos1 = cos[:, :D/2],
    cos2 = cos[:, D/2:]), as the reference kernel does (:112-115).
    """
    x = np.asarray(xn, dtype=dtype)
    half = x.shape[-1] // 2
    c = np.asarray(cos_rows, dtype=dtype)[:, None, :]
    s = np.asarray(sin_rows, dtype=dtype)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    out1 = x1 * c[..., :half] - x2 * s[..., :half]
    out2 = x2 * c[..., half:] + x1 * s[..., half:]
    return np.concatenate([out1, out2], axis=-1)


def qk_norm_rope(raw: np.ndarray, gamma, cos, sin, S: int, positions=None,
                 eps: float = DEFAULT_EPS, dtype=np.float64) -> np.ndarray:
    """Norm then RoPE for ``raw [T, H, D]`` with tables ``cos/sin [R, D]``."""
    T = raw.shape[0]
    rows = rope_rows(T, S, positions)
    c = np.asarray(cos, dtype=dtype)[rows]
    s = np.asarray(sin, dtype=dtype)[rows]
    return rope(qk_norm(raw, gamma, eps, dtype), c, s, dtype)


# ---------------------------------------------------------------------------
# Whole fused op  (fused_qkv_rope.py:130-195)
# ---------------------------------------------------------------------------

def fused_qkv_rope(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin,
                   positions=None, eps: float = DEFAULT_EPS,
                   round_projection: bool = False, dtype=np.float64):
    """Oracle of ``fused_qkv_rope``; all inputs are float arrays (bf16 values).

    Shapes follow fused_qkv_rope.py:155-158: ``D = q_norm_w.shape[0]``,
    ``H_Q = w_q.shape[0] // D``, ``H_KV = w_k.shape[0] // D``; ``x [B, S, hidden]``.
    ``round_projection=True`` reproduces the reference's bf16 rounding of the
    GEMM output before the norm (torch.mm returns bf16, :167-169); False keeps
    the exact projection (the "fp32 composition" of the acceptance criteria).
    Returns unrounded ``q [B,S,H_Q,D]``, ``k [B,S,H_KV,D]``, ``v [B,S,H_KV,D]``.
    """
    x = np.asarray(x)
    B, S, H = x.shape
    D = int(np.asarray(q_norm_w).shape[0])
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    HQ = np.asarray(w_q).shape[0] // D
    HKV = np.asarray(w_k).shape[0] // D
    x2d = x.reshape(B * S, H)
    q = projection(x2d, w_q, dtype)
    k = projection(x2d, w_k, dtype)
    v = projection(x2d, w_v, dtype)
    if round_projection:
        q, k, v = (round_bf16(a).astype(dtype) for a in (q, k, v))
    q = q.reshape(B * S, HQ, D)
    k = k.reshape(B * S, HKV, D)
    v = v.reshape(B * S, HKV, D)
    qo = qk_norm_rope(q, q_norm_w, cos, sin, S, positions, eps, dtype)
    ko = qk_norm_rope(k, k_norm_w, cos, sin, S, positions, eps, dtype)
    return (qo.reshape(B, S, HQ, D), ko.reshape(B, S, HKV, D), v.reshape(B, S, HKV, D))


def unfused_composition(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin,
                        eps: float = DEFAULT_EPS, dtype=np.float32):
    """The reference's unfused composition, used as the CPU baseline.

    tests/test_fused_qkv_rope.py:244-259 (== attention.py:42-48 with the
    QK-Norm in fp32): three projections, per-head RMSNorm, then
    ``q * cos + rotate_half(q) * sin`` broadcast over heads (rope.py:24-45),
    all in ``dtype`` on the host.  Prefill mode, ``cos/sin [S, D]``.
    """
    B, S, H = x.shape
    D = q_norm_w.shape[0]
    x2d = x.reshape(B * S, H)
    outs = []
    for w, g in ((w_q, q_norm_w), (w_k, k_norm_w), (w_v, None)):
        p = (x2d @ w.T).reshape(B, S, -1, D)
        if g is not None:
            rms = 1.0 / np.sqrt(np.mean(p * p, axis=-1, keepdims=True) + dtype(eps))
            p = p * rms * g
            c = cos[None, :, None, :]
            s = sin[None, :, None, :]
            half = D // 2
            rot = np.concatenate([-p[..., half:], p[..., :half]], axis=-1)
            p = p * c + rot * s
        outs.append(p.astype(dtype, copy=False))
    return tuple(outs)


# ---------------------------------------------------------------------------
# HF-order RMSNorm used by the reference's unfused W4A16 front
# (mini_qwen/model/layers/rms_norm.py:11-18)
# ---------------------------------------------------------------------------

def rms_norm_hf(x, weight, eps: float = DEFAULT_EPS, round_to_bf16: bool = True, round_out: bool = False):
    """``weight * (x_fp32 * rms).to(input_dtype)`` -- rounds before the gamma multiply.

    With bf16 activations and weight (the model dtype) the product is a bf16
    tensor too: ``round_out=True`` rounds it, giving the bf16 input the decoder
    layer hands to the attention projections (qwen3.py:58-59).
    """
    xf = np.asarray(x, dtype=np.float32)
    rms = np.float32(1.0) / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + np.float32(eps))
    y = xf * rms
    if round_to_bf16:
        y = round_bf16(y)
    out = np.asarray(weight, dtype=np.float32) * y
    return round_bf16(out) if round_out else out


# ---------------------------------------------------------------------------
# int4 packing  (mini_qwen/quantization/packing.py:11-39)
# ---------------------------------------------------------------------------

_SHIFTS = np.arange(8, dtype=np.uint32) * np.uint32(4)


def pack_int4(vals: np.ndarray) -> np.ndarray:
    """``[..., K]`` values in 0..15 -> ``[..., K//8]`` int32, nibble i = vals[8j+i].

    packing.py:20-24: ``packed = sum(w[8i+k] << 4k)`` (little-endian nibbles).
    """
    v = np.asarray(vals).astype(np.uint32)
    assert v.shape[-1] % 8 == 0
    v = v.reshape(*v.shape[:-1], -1, 8)
    packed = np.bitwise_or.reduce(v << _SHIFTS, axis=-1)
    return packed.astype(np.uint32).view(np.int32)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pack_int4` (packing.py:27-39)."""
    p = np.asarray(packed).astype(np.int32).view(np.uint32)
    v = (p[..., None] >> _SHIFTS) & np.uint32(0xF)
    return v.reshape(*p.shape[:-1], -1).astype(np.int32)


# ---------------------------------------------------------------------------
# Paged KV cache addressing  (paged_attn_prefill.py:45-56, kv_cache.py:3-6)
# ---------------------------------------------------------------------------

def paged_slot(block_table, seq, pos, block_size: int = 16, num_blocks=None) -> np.ndarray:
    """Flat cache slot of each token: ``block_table[seq, pos // bs] * bs + pos % bs``.

    The cache is ``[num_blocks, block_size, H_kv, D]`` (kv_cache.py:3-6), so a
    token's K/V row of head h sits at row ``slot * H_kv + h`` of the flattened
    cache.  The scatter kernel computes ``page_idx = pos // PAGE_SIZE``,
    ``slot = pos % PAGE_SIZE``, ``phys = Block_table[batch_id, page_idx]``
    (paged_attn_prefill.py:47-51).  The reference does not bound-check; here a
    token whose sequence, page or block falls outside the table (or outside
    ``num_blocks``) gets -1: nothing is written for it.
    """
    bt = np.asarray(block_table, dtype=np.int64)
    seq = np.asarray(seq, dtype=np.int64)
    pos = np.asarray(pos, dtype=np.int64)
    rows, cols = bt.shape
    page = np.where(pos >= 0, pos // block_size, -1)
    ok = (seq >= 0) & (seq < rows) & (pos >= 0) & (page < cols)
    blk = np.where(ok, bt[np.clip(seq, 0, rows - 1), np.clip(page, 0, cols - 1)], -1)
    if num_blocks is not None:
        ok &= (blk >= 0) & (blk < num_blocks)
    ok &= blk >= 0
    return np.where(ok, blk * block_size + pos % block_size, -1)


# ---------------------------------------------------------------------------
# Per-group min-max quantizer  (mini_qwen/quantization/awq.py:14-58)
# ---------------------------------------------------------------------------

def minmax_quantize(w: np.ndarray, group_size: int = 128):
    """``w [K, N]`` -> (qweight [K//8, N] i32, scales [K//g, N] bf16 bits, qzeros [K//g, N//8] i32).

    awq.py:37-38  scales = ((max - min) / 15).clamp(min=1e-8)
    awq.py:41     zeros  = round(-min / scales).clamp(0, 15)
    awq.py:44-49  q      = round(w / scales + zeros).clamp(0, 15)
    awq.py:53,56  qweight packed along K, qzeros packed along N; scales -> bf16 (:58).
    numpy's round is half-to-even, as torch.round.
    """
    w = np.asarray(w, dtype=np.float32)
    K, N = w.shape
    assert K % group_size == 0 and N % 8 == 0
    wg = w.reshape(K // group_size, group_size, N)
    wmax = wg.max(axis=1)
    wmin = wg.min(axis=1)
    scales = np.maximum((wmax - wmin) / np.float32(15.0), np.float32(1e-8)).astype(np.float32)
    zeros = np.clip(np.round(-wmin / scales), 0, 15).astype(np.int32)
    q = np.clip(np.round(wg / scales[:, None, :] + zeros[:, None, :].astype(np.float32)), 0, 15)
    q = q.astype(np.int32).reshape(K, N)
    qweight = pack_int4(q.T).T.copy()
    qzeros = pack_int4(zeros)
    return qweight, f32_to_bf16(scales), qzeros


def dequant(qweight, scales_f32, qzeros, group_size: int = 128) -> np.ndarray:
    """fp32 weight ``[K, N]`` = ``(q - z) * s``  (tests/test_w4a16_gemm.py:19-44,
    w4a16_gemm.py:90-92).  ``scales_f32`` are the scale values as float32."""
    q = unpack_int4(np.asarray(qweight).T).T.astype(np.float32)  # [K, N]
    z = unpack_int4(qzeros).astype(np.float32)                    # [G, N]
    s = np.asarray(scales_f32, dtype=np.float32)                  # [G, N]
    K, N = q.shape
    G = K // group_size
    qg = q.reshape(G, group_size, N)
    return ((qg - z[:, None, :]) * s[:, None, :]).reshape(K, N)


# AutoAWQ checkpoints (the "GEMM" layout, AutoAWQ 0.2.x, awq/modules/linear/gemm.py,
# WQLinear_GEMM.from_linear; not vendored in the reference) pack 8 values along N
# into each int32 with the order map (0, 2, 4, 6, 1, 3, 5, 7): nibble i of word
# [r, j] holds column 8*j + AWQ_ORDER[i].  qweight is [K, N/8], qzeros [K/g, N/8],
# scales [K/g, N] fp16; the weight is (q - z) * s as in the reference's format.
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def awq_unpack(words: np.ndarray) -> np.ndarray:
    """AutoAWQ words ``[R, N/8]`` int32 -> values ``[R, N]`` in column order."""
    p = np.asarray(words).astype(np.int32).view(np.uint32)
    R, n8 = p.shape
    out = np.empty((R, n8, 8), dtype=np.int32)
    for i, c in enumerate(AWQ_ORDER):
        out[:, :, c] = ((p >> np.uint32(4 * i)) & np.uint32(0xF)).astype(np.int32)
    return out.reshape(R, n8 * 8)


def dequant_awq(qweight_awq, qzeros_awq, scales_f32, group_size: int = 128) -> np.ndarray:
    """fp32 ``[K, N]`` = ``(q - z) * s`` read straight from AutoAWQ words."""
    q = awq_unpack(qweight_awq).astype(np.float32)
    z = awq_unpack(qzeros_awq).astype(np.float32)
    s = np.asarray(scales_f32, dtype=np.float32)
    K, N = q.shape
    G = K // group_size
    return ((q.reshape(G, group_size, N) - z[:, None, :]) * s[:, None, :]).reshape(K, N)


def gptq_zero_fix(qzeros: np.ndarray) -> np.ndarray:
    """GPTQ v1 checkpoints store ``z - 1``; the loader adds 1 and clamps to 0..15
    (mini_qwen/model/layers/linear_w4a16.py:96-99)."""
    return pack_int4(np.clip(unpack_int4(qzeros) + 1, 0, 15))


def w4a16_gemm(x, qweight, scales_f32, qzeros, group_size: int = 128, dtype=np.float64,
               round_weight: bool = False):
    """``x [M, K] @ dequant(...)`` (w4a16_gemm.py:194-247), unrounded.

    ``round_weight=True`` rounds the fp32 dequantised weight to bf16 first: the
    numerics of an implementation that feeds bf16 matrix units (the reference's
    fp32 ``tl.dot`` is itself a reduced-precision product on tensor cores)."""
    w = dequant(qweight, scales_f32, qzeros, group_size)
    if round_weight:
        w = round_bf16(w)
    return np.asarray(x, dtype=dtype) @ w.astype(dtype)


def fused_qkv_rope_w4a16(x, qw, sc, qz, q_norm_w, k_norm_w, cos, sin, Hq, Hkv,
                         positions=None, group_size: int = 128, eps: float = DEFAULT_EPS,
                         dtype=np.float64, round_weight: bool = False):
    """W4A16 front (attention.py:102-109 / :136-148) with the norm kept in fp32.

    ``qw/sc/qz`` are 3-tuples (q, k, v projection) of packed weights, scale
    values (float32) and packed zeros.  ``x [B, S, hidden]``.
    """
    x = np.asarray(x)
    B, S, H = x.shape
    D = int(np.asarray(q_norm_w).shape[0])
    x2d = x.reshape(B * S, H)
    proj = [w4a16_gemm(x2d, qw[i], sc[i], qz[i], group_size, dtype, round_weight) for i in range(3)]
    q = proj[0].reshape(B * S, Hq, D)
    k = proj[1].reshape(B * S, Hkv, D)
    v = proj[2].reshape(B * S, Hkv, D)
    qo = qk_norm_rope(q, q_norm_w, cos, sin, S, positions, eps, dtype)
    ko = qk_norm_rope(k, k_norm_w, cos, sin, S, positions, eps, dtype)
    return (qo.reshape(B, S, Hq, D), ko.reshape(B, S, Hkv, D), v.reshape(B, S, Hkv, D))


# ---------------------------------------------------------------------------
# Comparison metrics used by every parity test
# ---------------------------------------------------------------------------

def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if np.size(a) else 0.0


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 ulps between two arrays of bf16 bit patterns (finite values)."""
    def ordered(u):
        u = np.asarray(u, dtype=np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - u, u)  # monotone map of the bf16 line
    return np.abs(ordered(a_bits) - ordered(b_bits))
