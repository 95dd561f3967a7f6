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
