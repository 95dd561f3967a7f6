"""Bit-level invariance of the pipelined prefill tiles.

Every direct-to-LDS tile variant accumulates each output element over the same
16-wide k-steps in the same order, whatever the tile's shape, its wave layout or
the depth of its stage ring, and applies the same epilogue.  Their outputs must
therefore be identical bit for bit: a tile-edge, row-tail or head-split bug in
one shape shows up as a mismatch against the others, independently of the
oracle's tolerance.  (The register-staged variants sum their QK-norm squares in
another order, and the KZ = 2 ones split K inside the workgroup, so they are only
held to the oracle, in test_fused_qkv_rope_gpu.py and test_w4a16_gpu.py.)
"""
from __future__ import annotations

import pytest
import torch

from conftest import HEAD_DIM, Case

pytestmark = pytest.mark.gpu

D = HEAD_DIM
BF16_DMA_VARIANTS = [10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23]
INT4_DMA_VARIANTS = [30, 31, 32, 33, 34, 35]


def _with_variant(variant, fn):
    import mqk
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", variant)
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        mqk.set_option("prefill_tile", old)


@pytest.mark.parametrize("positions", [False, True])
def test_bf16_dma_variants_bit_identical(positions, device):
    import mqk
    T, hidden, Hq, Hkv = 600, 2048, 16, 4  # row tail in every tile height; 24 heads tile as 1, 2 or 3
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(5), dtype=torch.int32) \
        if positions else None
    case = Case(1, T, hidden, Hq, Hkv, seed=710, rows=4096 if positions else None, positions=pos)
    args = case.args(device)
    ref = _with_variant(16, lambda: mqk.fused_qkv_rope(*args))
    for v in BF16_DMA_VARIANTS:
        out = _with_variant(v, lambda: mqk.fused_qkv_rope(*args))
        for name, a, b in zip("qkv", out, ref):
            assert torch.equal(a, b), f"variant {v}: {name} differs from variant 16"


def test_int4_dma_variants_bit_identical(device):
    import mqk
    from test_w4a16_gpu import _int4_case
    B, S, hidden, Hq, Hkv = 1, 600, 1024, 16, 4
    x, projs, gq, gk = _int4_case(B, S, hidden, Hq, Hkv, seed=930, scale_dtype=torch.float16)
    c, s = mqk.rope_tables(D, 4096)
    pos = torch.randint(0, 4096, (S,), generator=torch.Generator().manual_seed(6), dtype=torch.int32)
    dp = [tuple(t.to(device) for t in p) for p in projs]
    args = (x.to(device), *dp, gq.to(device), gk.to(device), c.bfloat16().to(device), s.bfloat16().to(device),
            pos.to(device))
    ref = _with_variant(31, lambda: mqk.fused_qkv_rope_w4a16(*args))
    for v in INT4_DMA_VARIANTS:
        out = _with_variant(v, lambda: mqk.fused_qkv_rope_w4a16(*args))
        for name, a, b in zip("qkv", out, ref):
            assert torch.equal(a, b), f"int4 variant {v}: {name} differs from variant 31"


def _ex_case(hidden, seed):
    """Varlen batch of four sequences (one empty) with start offsets, a paged KV
    cache behind a shuffled block table, and the decoder's input RMSNorm."""
    g = torch.Generator().manual_seed(seed)
    lens = [150, 0, 230, 220]
    cu = torch.tensor([0, 150, 150, 380, 600], dtype=torch.int32)
    start = torch.tensor([3, 0, 700, 40], dtype=torch.int32)
    bs, per_seq = 16, 59  # covers position 700 + 230
    bt = torch.randperm(4 * per_seq + 8, generator=g)[: 4 * per_seq].view(4, per_seq).to(torch.int32)
    in_w = (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16()
    return sum(lens), cu, start, bs, bt, 4 * per_seq + 8, in_w


def _ex_run(fn, variant, device, Hkv, num_blocks, bs):
    """One call with tile variant `variant` (no tail split) on fresh sentinel caches
    (the sentinel's bits are a NaN in bf16, so results are compared as int16 bits)."""
    import mqk
    kc = torch.full((num_blocks, bs, Hkv, D), -7, dtype=torch.int16, device=device).view(torch.bfloat16)
    vc = kc.clone()
    old_tail = mqk.get_option("tail_split")
    mqk.set_option("tail_split", 0)
    try:
        out = _with_variant(variant, lambda: fn(kc, vc))
    finally:
        mqk.set_option("tail_split", old_tail)
    return list(out) + [kc, vc]


def test_bf16_dma_variants_bit_identical_with_ex_features(device):
    """The single-head and 8-wave 128 x 256 tiles through varlen positions, the
    input RMSNorm and the paged-cache write: outputs and cache contents equal
    variant 16's bit for bit."""
    import mqk
    hidden, Hq, Hkv = 2048, 16, 4
    T, cu, start, bs, bt, nb, in_w = _ex_case(hidden, 950)
    case = Case(1, T, hidden, Hq, Hkv, seed=951, rows=1024)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    cu_d, st_d, bt_d, inw_d = cu.to(device), start.to(device), bt.to(device), in_w.to(device)

    def fn(kc, vc):
        return mqk.fused_qkv_rope_ex(x.view(T, hidden), wq, wk, wv, gq, gk, cos, sin, cu_seqlens=cu_d,
                                     seq_pos0=st_d, input_norm_w=inw_d, k_cache=kc, v_cache=vc,
                                     block_table=bt_d)
    ref = _ex_run(fn, 16, device, Hkv, nb, bs)
    assert (ref[3].view(torch.int16) != -7).any()  # the cache was written
    for v in (19, 20, 21, 22, 23):
        out = _ex_run(fn, v, device, Hkv, nb, bs)
        for name, a, b in zip(["q", "k", "v", "k_cache", "v_cache"], out, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"variant {v}: {name} differs from variant 16"


def test_int4_dma_variants_bit_identical_with_ex_features(device):
    """The int4 single-head tiles (34, 35) likewise against variant 31."""
    import mqk
    from test_w4a16_gpu import _int4_case
    hidden, Hq, Hkv = 1024, 16, 4
    T, cu, start, bs, bt, nb, in_w = _ex_case(hidden, 960)
    x, projs, gq, gk = _int4_case(1, T, hidden, Hq, Hkv, seed=961, scale_dtype=torch.float16)
    c, s = mqk.rope_tables(D, 1024)
    dp = [tuple(t.to(device) for t in p) for p in projs]
    xd = x.to(device).view(T, hidden)
    rest = (gq.to(device), gk.to(device), c.bfloat16().to(device), s.bfloat16().to(device))
    cu_d, st_d, bt_d, inw_d = cu.to(device), start.to(device), bt.to(device), in_w.to(device)

    def fn(kc, vc):
        return mqk.fused_qkv_rope_w4a16_ex(xd, *dp, *rest, cu_seqlens=cu_d, seq_pos0=st_d, input_norm_w=inw_d,
                                           k_cache=kc, v_cache=vc, block_table=bt_d)
    ref = _ex_run(fn, 31, device, Hkv, nb, bs)
    for v in (34, 35):
        out = _ex_run(fn, v, device, Hkv, nb, bs)
        for name, a, b in zip(["q", "k", "v", "k_cache", "v_cache"], out, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), \
                f"int4 variant {v}: {name} differs from variant 31"
