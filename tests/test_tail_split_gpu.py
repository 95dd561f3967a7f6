"""GPU tests of the tail split: when the rows of a tile kernel's last, partial row
tile (at most 64) would cost a whole extra round of tiles over the CUs, the op
runs the tile kernel on the other rows and the split-K decode kernel on those
(two launches).  Outputs must match the oracle, the tile rows must be bit-equal
to the unsplit op, and the tail rows bit-equal to the decode kernel run on them
alone.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

D = HEAD_DIM


def _opt(name, value):
    import mqk
    old = mqk.get_option(name)
    mqk.set_option(name, value)
    return old


@pytest.mark.parametrize("positions", [False, True])
def test_tail_split_bf16(positions, device):
    import mqk
    T, hidden, Hq, Hkv = 8192 + 22, 512, 32, 8  # 128x384 tiles: 1040 -> 1024 tiles + 22 rows
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(3), dtype=torch.int32) \
        if positions else None
    case = Case(1, T, hidden, Hq, Hkv, seed=901, rows=4096 if positions else None, positions=pos)
    x, wq, wk, wv, gq, gk, cos, sin, p = case.args(device)
    old = _opt("tail_split", 0)
    try:
        ref = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, p)
        mqk.set_option("tail_split", 1)
        out = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, p)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("tail_split", old)
    t0 = T - 22
    for a, b in zip(out, ref):
        assert torch.equal(a[:, :t0], b[:, :t0])  # the tile kernel's rows are untouched
    # tail rows == the decode kernel on those rows alone
    tail_pos = p[t0:] if positions else (torch.arange(t0, T, dtype=torch.int32) % T).to(device)
    alone = mqk.fused_qkv_rope(x[:, t0:].contiguous(), wq, wk, wv, gq, gk, cos, sin, tail_pos)
    torch.cuda.synchronize()
    for a, b in zip(out, alone):
        assert torch.equal(a[:, t0:], b)
    idx = np.concatenate([np.arange(0, 40), np.arange(t0 - 8, T)])
    want = case.oracle(token_idx=idx)
    for got, w_ in zip(out, want):
        g_ = f32(got)[0, idx].reshape(w_.shape)
        assert orc.max_abs(g_, w_) <= 2e-2 and orc.rel_l2(g_, w_) <= 1e-2


def test_tail_split_w4a16_paged(device):
    import mqk
    T, hidden, Hq, Hkv = 8192 + 22, 512, 32, 8  # 256x256 int4 tiles: 792 -> 768 tiles + 22 rows
    g = torch.Generator().manual_seed(5)
    projs = []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w, 128)))
    x = torch.randn(1, T, hidden, generator=g).bfloat16().to(device)
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    c, s_ = mqk.rope_tables(D, T)
    cos, sin = c.bfloat16().to(device), s_.bfloat16().to(device)
    bs = 16
    nb = T // bs + 8
    bt = torch.randperm(nb, generator=g)[: (T + bs - 1) // bs].view(1, -1).to(torch.int32).to(device)
    kc = torch.zeros(nb, bs, Hkv, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    old = _opt("tail_split", 0)
    try:
        ref = mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin)
        mqk.set_option("tail_split", 1)
        q, k, v = mqk.fused_qkv_rope_w4a16_paged(x, *projs, gq, gk, cos, sin, kc, vc, bt)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("tail_split", old)
    t0 = T - 22
    for a, b in zip((q, k, v), ref):
        assert torch.equal(a[:, :t0], b[:, :t0])
        d = (a[:, t0:].float() - b[:, t0:].float()).abs().max().item()
        assert d <= 2e-2  # the tail rows come from the decode kernel: same math, other summation order
    t = np.arange(T)
    slots = bt.cpu().numpy()[0, t // bs].astype(np.int64) * bs + t % bs
    for cache, rows in ((kc, k), (vc, v)):
        flat = cache.view(torch.int16).reshape(-1, Hkv, D).cpu()
        assert torch.equal(flat[torch.from_numpy(slots)], rows[0].view(torch.int16).cpu())


def test_no_tail_split_when_no_round_is_saved(device):
    """Few tiles: every row stays in the tile kernel (bit-equal with the option off)."""
    import mqk
    case = Case(1, 300, 512, 4, 2, seed=11)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    a = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
    old = _opt("tail_split", 0)
    try:
        b = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("tail_split", old)
    assert all(torch.equal(u, w_) for u, w_ in zip(a, b))
