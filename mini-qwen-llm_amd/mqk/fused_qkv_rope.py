"""Fused QKV projection + QK-Norm + RoPE on MI355X (drop-in for the reference op).

Mirror of ``mini_qwen.kernels.fused_qkv_rope.fused_qkv_rope``
(mini_qwen/kernels/fused_qkv_rope.py:130-195, frozen signature :24-35):

    fused_qkv_rope(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin, positions=None)
        x         [B, S, hidden]           bf16
        w_q       [H_Q * D, hidden]        bf16 (nn.Linear layout)
        w_k, w_v  [H_KV * D, hidden]       bf16
        q_norm_w, k_norm_w [D]             bf16
        cos, sin  [S or rows, D]           bf16
        positions [B*S] int32 or None      None: prefill, token t uses row t % S;
                                           else row positions[t]
        -> q [B, S, H_Q, D], k [B, S, H_KV, D], v [B, S, H_KV, D]   bf16, contiguous

Shapes are inferred as the reference does (:155-158): ``D = q_norm_w.shape[0]``,
``H_Q = w_q.shape[0] // D``, ``H_KV = w_k.shape[0] // D``, and ``D`` must be even
(:160).  The whole op is one HIP kernel launch (libmqk.so): bf16 MFMA projection,
fp32 norm + RoPE applied to the accumulators, one bf16 store per output.

Differences from the reference, all deliberate:
  * the norm reads the fp32 accumulator, not a bf16-rounded GEMM output (head
    sizes other than 64 and 128 -- multiples of 8 up to 512 -- run the
    reference's own composition instead: GEMMs into bf16 q / k / v, then norm +
    RoPE; other head sizes raise);
  * ``v`` is our own MFMA projection (fp32 accumulate, one rounding), so it is
    not bit-identical to a vendor GEMM (test_fused_qkv_rope.py:165 demands
    bit-equality with torch's own GEMM, which no independent kernel can give);
  * positions outside ``[0, cos.shape[0])`` are clamped instead of read out of
    bounds; int64 positions are accepted and converted;
  * inputs must be CUDA/HIP tensors, all bf16, all fp32 or all fp16 (TypeError /
    ValueError otherwise); non-contiguous inputs are made contiguous.

fp32 inputs (the dtype of the reference's CPU-runnable fp32 layer) take a
separate kernel: an fp32 projection on the matrix cores (fp32 products and
sums), norm and RoPE in fp32, fp32 outputs.  fp16 inputs (a model loaded in
fp16) take the same kernel on the fp16 matrix cores (exact products, fp32
sums), with fp16 outputs.  Differences from the reference on these dtypes: its
Triton kernel rounds Q and K to bf16 before storing them into the fp32 / fp16
outputs (fused_qkv_rope.py:117-120), and on fp16 its GEMM output is rounded to
fp16 before the norm; here neither happens, so the outputs carry fp32 / fp16
precision (the unfused composition's values), not the fused reference's bits.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _native

EPS = 1e-6  # the reference hard-codes EPS=1e-6 (fused_qkv_rope.py:187)


def _require(t: torch.Tensor, name: str, device: torch.device, dtype=torch.bfloat16) -> torch.Tensor:
    # (integer device indices and no torch.device objects on the success path:
    # these checks run for every tensor of every call)
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU device, got {t.device}")
    if t.get_device() != device.index:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.data_ptr() & 15:
        # a view at an odd offset: the pipelined and decode kernels read every operand
        # with 16-byte loads, so take a (16-byte aligned) copy rather than the slower
        # kernels the C ABI keeps for unaligned pointers
        return t.clone(memory_format=torch.contiguous_format)
    return t if t.is_contiguous() else t.contiguous()


def _positions(positions: Optional[torch.Tensor], T: int, device) -> Optional[torch.Tensor]:
    if positions is None:
        return None
    if not isinstance(positions, torch.Tensor):
        raise TypeError("positions must be a torch.Tensor")
    if positions.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"positions must be int32 (or int64), got {positions.dtype}")
    positions = _require(positions, "positions", device, dtype=None)
    if positions.numel() != T:
        raise ValueError(f"positions has {positions.numel()} entries, expected B*S = {T}")
    # (a contiguous tensor is read as its T entries in order, whatever its shape)
    return positions if positions.dtype == torch.int32 else positions.to(torch.int32)


def _rope_tables(cos, sin, D, device, dtype=torch.bfloat16):
    cos = _require(cos, "cos", device, dtype)
    sin = _require(sin, "sin", device, dtype)
    if cos.dim() != 2 or cos.shape[1] != D or sin.shape != cos.shape:
        raise ValueError(f"cos/sin must both be [rows, {D}], got {tuple(cos.shape)} / {tuple(sin.shape)}")
    if cos.shape[0] < 1:
        raise ValueError("cos/sin need at least one row")
    return cos, sin


def fused_qkv_rope(
    x: torch.Tensor,
    w_q: torch.Tensor,
    w_k: torch.Tensor,
    w_v: torch.Tensor,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused QKV projection + QK-Norm + RoPE; see the module docstring."""
    B, S, H = x.shape
    D = q_norm_w.shape[0]
    H_Q = w_q.shape[0] // D
    H_KV = w_k.shape[0] // D
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    device = x.device
    dtype = x.dtype if isinstance(x, torch.Tensor) and x.dtype in (torch.float32, torch.float16) else torch.bfloat16
    x = _require(x, "x", device, dtype)
    w_q = _require(w_q, "w_q", device, dtype)
    w_k = _require(w_k, "w_k", device, dtype)
    w_v = _require(w_v, "w_v", device, dtype)
    q_norm_w = _require(q_norm_w, "q_norm_w", device, dtype)
    k_norm_w = _require(k_norm_w, "k_norm_w", device, dtype)
    if w_q.shape != (H_Q * D, H) or w_k.shape != (H_KV * D, H) or w_v.shape != (H_KV * D, H):
        raise ValueError(
            f"weight shapes {tuple(w_q.shape)}, {tuple(w_k.shape)}, {tuple(w_v.shape)} do not match "
            f"H_Q={H_Q}, H_KV={H_KV}, D={D}, hidden={H}")
    if k_norm_w.shape != (D,):
        raise ValueError(f"k_norm_w must be [{D}], got {tuple(k_norm_w.shape)}")
    cos, sin = _rope_tables(cos, sin, D, device, dtype)
    T = B * S
    pos = _positions(positions, T, device)

    q = torch.empty(B, S, H_Q, D, dtype=dtype, device=device)
    k = torch.empty(B, S, H_KV, D, dtype=dtype, device=device)
    v = torch.empty(B, S, H_KV, D, dtype=dtype, device=device)
    if T == 0:
        return q, k, v

    lib = _native.library()
    stream = _native.stream_handle(device)
    if dtype != torch.bfloat16:
        entry = "mqk_fused_qkv_rope_f32" if dtype == torch.float32 else "mqk_fused_qkv_rope_f16"
        status = _native.call(
            device, getattr(lib, entry),
            x.data_ptr(), w_q.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
            q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), _native.ptr(pos),
            T, S, H, H_Q, H_KV, D, cos.shape[0], EPS,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), stream)
        _native.check(status, entry)
        return q, k, v
    nbytes = _native.fused_workspace_bytes(T, H_Q, H_KV, H, D)
    ws = _native.workspace(device, stream, nbytes)
    status = _native.call(
        device, lib.mqk_fused_qkv_rope_bf16,
        x.data_ptr(), w_q.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), _native.ptr(pos),
        T, S, H, H_Q, H_KV, D, cos.shape[0], EPS,
        q.data_ptr(), k.data_ptr(), v.data_ptr(),
        _native.ptr(ws), 0 if ws is None else ws.numel(), stream)
    _native.check(status, "mqk_fused_qkv_rope_bf16")
    return q, k, v


def paged_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
             kv_seq: Optional[torch.Tensor], kv_pos: Optional[torch.Tensor], T: int, H_KV: int, D: int,
             device, positions: Optional[torch.Tensor]):
    """Validated ``mqk_paged_kv`` descriptor and the tensors it points to (kept alive
    by the caller for the duration of the launch).

    Caches: ``[num_blocks, block_size, H_KV, D]`` bf16, contiguous (written in
    place, so never copied).  ``block_table [rows, cols]`` int32.  ``kv_seq`` /
    ``kv_pos`` ``[T]``: the token's sequence (row of block_table) and position in
    it; both default to ``t // S`` and ``t % S`` and are required in positions mode.
    """
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if not isinstance(c, torch.Tensor) or c.device != device or c.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be a bf16 tensor on {device}")
        if c.dim() != 4 or c.shape[2] != H_KV or c.shape[3] != D:
            raise ValueError(f"{name} must be [num_blocks, block_size, {H_KV}, {D}], got {tuple(c.shape)}")
        if not c.is_contiguous():
            raise ValueError(f"{name} must be contiguous (it is written in place)")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    if block_table.dtype not in (torch.int32, torch.int64) or block_table.dim() != 2:
        raise TypeError("block_table must be a 2-D int32 tensor")
    bt = _require(block_table, "block_table", device, dtype=None).to(torch.int32).contiguous()
    if positions is not None and (kv_seq is None or kv_pos is None):
        raise ValueError("positions mode needs kv_seq and kv_pos (the cache slot of each token)")
    seq = None if kv_seq is None else _positions(kv_seq, T, device)
    pos = None if kv_pos is None else _positions(kv_pos, T, device)
    desc = _native.PagedKV(k_cache.data_ptr(), v_cache.data_ptr(), bt.data_ptr(), bt.shape[0], bt.shape[1],
                           k_cache.shape[0], k_cache.shape[1], _native.ptr(seq), _native.ptr(pos))
    return desc, (bt, seq, pos)


def fused_qkv_rope_paged(
    x: torch.Tensor,
    w_q: torch.Tensor,
    w_k: torch.Tensor,
    w_v: torch.Tensor,
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
):
    """:func:`fused_qkv_rope` that also writes K and V into a paged KV cache.

    Fuses the reference's separate cache scatter (``write_kv_decode`` and the
    prefill scatter, mini_qwen/kernels/paged_attn_prefill.py:27-56, :203-213,
    :232-254) into the same kernel: the K/V rows are stored once to ``k``/``v``
    (unless ``return_kv`` is False) and once to their cache slot.  Returns
    ``(q, k, v)``, with ``k``/``v`` None when ``return_kv`` is False.
    """
    B, S, H = x.shape
    D = q_norm_w.shape[0]
    H_Q = w_q.shape[0] // D
    H_KV = w_k.shape[0] // D
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    device = x.device
    dtype = torch.bfloat16  # (the paged and extended forms run the bf16 kernels only)
    x = _require(x, "x", device, dtype)
    w_q = _require(w_q, "w_q", device, dtype)
    w_k = _require(w_k, "w_k", device, dtype)
    w_v = _require(w_v, "w_v", device, dtype)
    q_norm_w = _require(q_norm_w, "q_norm_w", device, dtype)
    k_norm_w = _require(k_norm_w, "k_norm_w", device, dtype)
    if w_q.shape != (H_Q * D, H) or w_k.shape != (H_KV * D, H) or w_v.shape != (H_KV * D, H):
        raise ValueError(
            f"weight shapes {tuple(w_q.shape)}, {tuple(w_k.shape)}, {tuple(w_v.shape)} do not match "
            f"H_Q={H_Q}, H_KV={H_KV}, D={D}, hidden={H}")
    cos, sin = _rope_tables(cos, sin, D, device)
    T = B * S
    pos = _positions(positions, T, device)
    desc, keep = paged_kv(k_cache, v_cache, block_table, kv_seq, kv_pos, T, H_KV, D, device, positions)

    q = torch.empty(B, S, H_Q, D, dtype=torch.bfloat16, device=device)
    k = torch.empty(B, S, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    v = torch.empty(B, S, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    if T == 0:
        return q, k, v
    lib = _native.library()
    stream = _native.stream_handle(device)
    nbytes = _native.fused_workspace_bytes(T, H_Q, H_KV, H, D)
    ws = _native.workspace(device, stream, nbytes)
    status = _native.call(device, lib.mqk_fused_qkv_rope_paged_bf16,
        x.data_ptr(), w_q.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), _native.ptr(pos),
        T, S, H, H_Q, H_KV, D, cos.shape[0], EPS,
        q.data_ptr(), _native.ptr(k), _native.ptr(v), ctypes.byref(desc),
        _native.ptr(ws), 0 if ws is None else ws.numel(), stream)
    _native.check(status, "mqk_fused_qkv_rope_paged_bf16")
    del keep
    return q, k, v


def fused_ext(T: int, H_KV: int, D: int, hidden: int, device, positions=None, cu_seqlens=None,
              seq_pos0=None, input_norm_w=None, input_eps: float = EPS, k_cache=None, v_cache=None,
              block_table=None, kv_seq=None, kv_pos=None):
    """Validated ``mqk_fused_ext`` descriptor of the optional features and the
    tensors it points to (kept alive by the caller for the duration of the launch).

    ``cu_seqlens [n_seqs + 1]`` int32 (varlen mode, exclusive with ``positions``),
    ``seq_pos0 [n_seqs]`` (position of each sequence's first token, default 0),
    ``input_norm_w [hidden]`` bf16 (input RMSNorm), and the paged cache
    (``k_cache``/``v_cache``/``block_table`` together, see :func:`paged_kv`).
    """
    keep = []
    ext = _native.FusedExt()
    if cu_seqlens is not None:
        if positions is not None:
            raise ValueError("cu_seqlens (varlen) and positions are exclusive")
        if cu_seqlens.dtype not in (torch.int32, torch.int64) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
            raise ValueError("cu_seqlens must be a 1-D int32 tensor of n_seqs + 1 >= 2 offsets")
        cu = _require(cu_seqlens, "cu_seqlens", device, dtype=None).to(torch.int32)
        keep.append(cu)
        ext.cu_seqlens = cu.data_ptr()
        ext.n_seqs = cu.numel() - 1
        if seq_pos0 is not None:
            if seq_pos0.numel() != ext.n_seqs:
                raise ValueError(f"seq_pos0 has {seq_pos0.numel()} entries, expected n_seqs = {ext.n_seqs}")
            p0 = _require(seq_pos0, "seq_pos0", device, dtype=None).reshape(-1).to(torch.int32)
            keep.append(p0)
            ext.seq_pos0 = p0.data_ptr()
    elif seq_pos0 is not None:
        raise ValueError("seq_pos0 needs cu_seqlens")
    if input_norm_w is not None:
        g = _require(input_norm_w, "input_norm_w", device)
        if g.shape != (hidden,):
            raise ValueError(f"input_norm_w must be [{hidden}], got {tuple(g.shape)}")
        keep.append(g)
        ext.in_gamma = g.data_ptr()
        ext.in_eps = float(input_eps)
    if k_cache is not None or v_cache is not None or block_table is not None:
        if k_cache is None or v_cache is None or block_table is None:
            raise ValueError("k_cache, v_cache and block_table go together")
        desc, kv_keep = paged_kv(k_cache, v_cache, block_table, kv_seq, kv_pos, T, H_KV, D, device, positions)
        keep.append((desc, kv_keep))
        ext.kv = ctypes.pointer(desc)
    elif kv_seq is not None or kv_pos is not None:
        raise ValueError("kv_seq / kv_pos need a paged cache")
    return ext, keep


def _lead_shape(x: torch.Tensor, cu_seqlens) -> Tuple[tuple, int]:
    """Leading output dims and S for x [B, S, hidden] or (varlen) [T, hidden]."""
    if x.dim() == 3:
        return tuple(x.shape[:2]), x.shape[1]
    if x.dim() == 2 and cu_seqlens is not None:
        return (x.shape[0],), x.shape[0]
    raise ValueError(f"x must be [B, S, hidden] (or [T, hidden] with cu_seqlens), got {tuple(x.shape)}")


def fused_qkv_rope_ex(
    x: torch.Tensor,
    w_q: torch.Tensor,
    w_k: torch.Tensor,
    w_v: torch.Tensor,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
    *,
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
    """:func:`fused_qkv_rope` with the optional features of ``mqk_fused_qkv_rope_ex_bf16``.

    * ``cu_seqlens`` (varlen prefill): ``x`` is ``[T, hidden]`` (or ``[1, T, hidden]``)
      holding packed sequences; token t of sequence s uses RoPE row / cache
      position ``t - cu_seqlens[s] (+ seq_pos0[s])`` and block-table row s, the
      batch_ids / positions of paged_attn_prefill.py:188-199.
    * ``input_norm_w``: the decoder's input RMSNorm (rms_norm.py:11-18) is applied
      to ``x`` inside the op.
    * ``k_cache``/``v_cache``/``block_table``: the paged-KV-cache write of
      :func:`fused_qkv_rope_paged` (``return_kv=False`` writes the cache only).

    Outputs are shaped ``x.shape[:-1] + (H, D)``.
    """
    lead, S = _lead_shape(x, cu_seqlens)
    H = x.shape[-1]
    D = q_norm_w.shape[0]
    H_Q = w_q.shape[0] // D
    H_KV = w_k.shape[0] // D
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    device = x.device
    dtype = torch.bfloat16  # (the paged and extended forms run the bf16 kernels only)
    x = _require(x, "x", device, dtype)
    w_q = _require(w_q, "w_q", device, dtype)
    w_k = _require(w_k, "w_k", device, dtype)
    w_v = _require(w_v, "w_v", device, dtype)
    q_norm_w = _require(q_norm_w, "q_norm_w", device, dtype)
    k_norm_w = _require(k_norm_w, "k_norm_w", device, dtype)
    if w_q.shape != (H_Q * D, H) or w_k.shape != (H_KV * D, H) or w_v.shape != (H_KV * D, H):
        raise ValueError(
            f"weight shapes {tuple(w_q.shape)}, {tuple(w_k.shape)}, {tuple(w_v.shape)} do not match "
            f"H_Q={H_Q}, H_KV={H_KV}, D={D}, hidden={H}")
    cos, sin = _rope_tables(cos, sin, D, device)
    T = x.numel() // H
    pos = _positions(positions, T, device)
    ext, keep = fused_ext(T, H_KV, D, H, device, positions, cu_seqlens, seq_pos0, input_norm_w, input_eps,
                          k_cache, v_cache, block_table, kv_seq, kv_pos)
    if not return_kv and not ext.kv:
        raise ValueError("return_kv=False needs a paged cache")
    q = torch.empty(*lead, H_Q, D, dtype=torch.bfloat16, device=device)
    k = torch.empty(*lead, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    v = torch.empty(*lead, H_KV, D, dtype=torch.bfloat16, device=device) if return_kv else None
    if T == 0:
        return q, k, v
    lib = _native.library()
    stream = _native.stream_handle(device)
    nbytes = _native.fused_workspace_bytes(T, H_Q, H_KV, H, D, ext)
    ws = _native.workspace(device, stream, nbytes)
    status = _native.call(device, lib.mqk_fused_qkv_rope_ex_bf16,
        x.data_ptr(), w_q.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), _native.ptr(pos),
        T, S, H, H_Q, H_KV, D, cos.shape[0], EPS,
        q.data_ptr(), _native.ptr(k), _native.ptr(v), ctypes.byref(ext),
        _native.ptr(ws), 0 if ws is None else ws.numel(), stream)
    _native.check(status, "mqk_fused_qkv_rope_ex_bf16")
    del keep
    return q, k, v


def fused_qkv_rope_varlen(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin, cu_seqlens, seq_pos0=None,
                          **kwargs):
    """Varlen prefill: ``x [T, hidden]`` packed sequences delimited by ``cu_seqlens``;
    returns ``q [T, H_Q, D]``, ``k``/``v [T, H_KV, D]`` (the layout paged_attn_prefill
    takes).  Keyword arguments as :func:`fused_qkv_rope_ex`."""
    return fused_qkv_rope_ex(x, w_q, w_k, w_v, q_norm_w, k_norm_w, cos, sin, cu_seqlens=cu_seqlens,
                             seq_pos0=seq_pos0, **kwargs)


def qk_norm_rope(
    q_raw: torch.Tensor,
    k_raw: torch.Tensor,
    q_norm_w: torch.Tensor,
    k_norm_w: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: Optional[torch.Tensor] = None,
    eps: float = EPS,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """QK-Norm + RoPE on already-projected ``q_raw [B, S, H_Q, D]`` / ``k_raw [B, S, H_KV, D]``.

    The standalone twin of ``_qk_norm_rope_kernel`` (fused_qkv_rope.py:46-127),
    with the same position rules (prefill: row ``t % S``; else ``positions[t]``).
    """
    if q_raw.dim() != 4 or k_raw.dim() != 4:
        raise ValueError("q_raw/k_raw must be [B, S, H, D]")
    B, S, H_Q, D = q_raw.shape
    H_KV = k_raw.shape[2]
    assert D % 2 == 0, "head_dim must be even (RoPE rotate_half)"
    if k_raw.shape[:2] != (B, S) or k_raw.shape[3] != D:
        raise ValueError(f"k_raw shape {tuple(k_raw.shape)} does not match q_raw {tuple(q_raw.shape)}")
    device = q_raw.device
    q_raw = _require(q_raw, "q_raw", device)
    k_raw = _require(k_raw, "k_raw", device)
    q_norm_w = _require(q_norm_w, "q_norm_w", device)
    k_norm_w = _require(k_norm_w, "k_norm_w", device)
    cos, sin = _rope_tables(cos, sin, D, device)
    T = B * S
    pos = _positions(positions, T, device)
    q_out = torch.empty_like(q_raw)
    k_out = torch.empty_like(k_raw)
    if T == 0:
        return q_out, k_out
    stream = _native.stream_handle(device)
    status = _native.call(device, _native.library().mqk_qk_norm_rope_bf16,
        q_raw.data_ptr(), k_raw.data_ptr(), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), _native.ptr(pos), T, S, H_Q, H_KV, D, cos.shape[0],
        float(eps), q_out.data_ptr(), k_out.data_ptr(), stream)
    _native.check(status, "mqk_qk_norm_rope_bf16")
    return q_out, k_out
