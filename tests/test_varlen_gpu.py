"""GPU tests of the varlen (cu_seqlens) mode of mqk_fused_qkv_rope_ex_*.

Token t of packed sequence s uses RoPE row / cache position t - cu_seqlens[s]
(+ seq_pos0[s]) and block-table row s, the batch_ids / positions that
paged_attn_prefill derives from cu_seqlens (mini_qwen/kernels/paged_attn_prefill.py
:188-199; restated in oracle.varlen_positions).  The varlen op must equal the
positions-mode op fed those positions bit for bit (same kernels, same rows), match
the oracle within the fused op's tolerance, and write the same cache slots.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

D = HEAD_DIM
SENTINEL = 0x7F7F


def _lengths(n, lo, hi, seed, zeros=True):
    g = np.random.default_rng(seed)
    lens = g.integers(lo, hi + 1, n)
    if zeros:
        lens[1] = 0  # an empty sequence in the batch
    return lens


def _case(lens, hidden, Hq, Hkv, seed, start=None, rows=4096):
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _, pos = orc.varlen_positions(cu, start)
    case = Case(1, T, hidden, Hq, Hkv, seed, rows=rows, positions=torch.from_numpy(pos.astype(np.int32)))
    return case, torch.from_numpy(cu), pos


@pytest.mark.parametrize("n,lo,hi,with_start", [(5, 1, 12, False), (9, 1, 70, True), (16, 1, 300, True)])
def test_varlen_equals_positions_mode(n, lo, hi, with_start, device):
    import mqk
    lens = _lengths(n, lo, hi, seed=n)
    start = np.random.default_rng(n + 1).integers(0, 1000, n) if with_start else None
    case, cu, pos = _case(lens, 1024, 16, 8, seed=900 + n, start=start)
    x, wq, wk, wv, gq, gk, cos, sin, p = case.args(device)
    s0 = None if start is None else torch.from_numpy(start.astype(np.int32)).to(device)
    q, k, v = mqk.fused_qkv_rope_varlen(x[0], wq, wk, wv, gq, gk, cos, sin, cu.to(device), seq_pos0=s0)
    q0, k0, v0 = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, p)
    torch.cuda.synchronize()
    T = x.shape[1]
    assert q.shape == (T, 16, D) and k.shape == (T, 8, D)
    assert torch.equal(q, q0[0]) and torch.equal(k, k0[0]) and torch.equal(v, v0[0])


def test_varlen_matches_oracle(device):
    import mqk
    lens = _lengths(6, 1, 40, seed=3)
    start = np.random.default_rng(4).integers(0, 3000, 6)
    case, cu, pos = _case(lens, 512, 4, 2, seed=77, start=start)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    q, k, v = mqk.fused_qkv_rope_varlen(x[0], wq, wk, wv, gq, gk, cos, sin, cu.to(device),
                                        seq_pos0=torch.from_numpy(start.astype(np.int32)).to(device))
    torch.cuda.synchronize()
    oq, ok, ov = case.oracle()
    for got, want in ((q, oq), (k, ok), (v, ov)):
        got = f32(got).reshape(want.shape)
        assert orc.max_abs(got, want) <= 2e-2 and orc.rel_l2(got, want) <= 1e-2


def test_varlen_row_indexing_exact(device):
    """Sentinel tables (cos row r encodes r, sin = 0, gamma = 1, one-hot norm input):
    the output reveals exactly which row every token used."""
    import mqk
    lens = np.array([3, 0, 5, 2, 7])
    start = np.array([0, 9, 17, 100, 250])
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _, pos = orc.varlen_positions(cu, start)
    hidden, rows = 64, 512
    x = torch.zeros(1, T, hidden)
    x[0, :, 0] = 1.0
    w = torch.zeros(D, hidden)
    w[:, 0] = 1.0  # every channel of the head = x[:, 0] = 1, which the norm leaves at 1 (to 5e-7)
    cos = torch.zeros(rows, D)
    cos[:, 0] = torch.arange(rows) / 1024.0  # exactly representable in bf16
    sin = torch.zeros(rows, D)
    ones = torch.ones(D)
    dev = lambda t: t.bfloat16().to(device)
    q, k, _ = mqk.fused_qkv_rope_varlen(dev(x[0]), dev(w), dev(w), dev(w), dev(ones), dev(ones), dev(cos),
                                        dev(sin), torch.from_numpy(cu).to(device),
                                        seq_pos0=torch.from_numpy(start.astype(np.int32)).to(device))
    torch.cuda.synchronize()
    got = q[:, 0, 0].float().cpu().numpy() * 1024.0
    got_rows = np.round(got).astype(np.int64)
    assert np.array_equal(got, got_rows)  # cos[row, 0] = row / 1024 came through exactly
    assert got_rows.tolist() == pos.tolist()


def _caches(nb, bs, Hkv, device):
    k = torch.full((nb, bs, Hkv, D), SENTINEL, dtype=torch.int16, device=device)
    return k.view(torch.bfloat16), k.clone().view(torch.bfloat16)


@pytest.mark.parametrize("n,hi", [(4, 30), (12, 200)])
def test_varlen_paged_write(n, hi, device):
    import mqk
    lens = _lengths(n, 1, hi, seed=50 + n)
    start = np.random.default_rng(n).integers(0, 64, n)
    case, cu, pos = _case(lens, 512, 4, 2, seed=60 + n, start=start)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    bs = 16
    pages = int((pos.max() + 1 + bs - 1) // bs) if pos.size else 1
    nb = n * pages + 3
    bt = torch.randperm(nb, generator=torch.Generator().manual_seed(n))[: n * pages].view(n, pages).to(torch.int32)
    kc, vc = _caches(nb, bs, 2, device)
    q, k, v = mqk.fused_qkv_rope_varlen(x[0], wq, wk, wv, gq, gk, cos, sin, cu.to(device),
                                        seq_pos0=torch.from_numpy(start.astype(np.int32)).to(device),
                                        k_cache=kc, v_cache=vc, block_table=bt.to(device))
    torch.cuda.synchronize()
    batch, pos2 = orc.varlen_positions(cu.numpy(), start)
    slots = bt.numpy()[batch, pos2 // bs].astype(np.int64) * bs + pos2 % bs
    for cache, rows in ((kc, k), (vc, v)):
        flat = cache.view(torch.int16).reshape(-1, 2, D).cpu()
        assert torch.equal(flat[torch.from_numpy(slots)], rows.view(torch.int16).cpu())
        mask = torch.ones(flat.shape[0], dtype=torch.bool)
        mask[torch.from_numpy(slots)] = False
        assert bool((flat[mask] == SENTINEL).all())


def test_varlen_w4a16_equals_positions_mode(device):
    import mqk
    lens = _lengths(7, 1, 90, seed=11)
    start = np.random.default_rng(12).integers(0, 500, 7)
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    _, pos = orc.varlen_positions(cu, start)
    hidden, Hq, Hkv = 512, 4, 2
    g = torch.Generator().manual_seed(13)
    projs = []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w, 128)))
    x = torch.randn(1, T, hidden, generator=g).bfloat16().to(device)
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    c, s_ = mqk.rope_tables(D, 1024)
    cos, sin = c.bfloat16().to(device), s_.bfloat16().to(device)
    q, k, v = mqk.fused_qkv_rope_w4a16_ex(x[0], *projs, gq, gk, cos, sin,
                                          cu_seqlens=torch.from_numpy(cu).to(device),
                                          seq_pos0=torch.from_numpy(start.astype(np.int32)).to(device))
    q0, k0, v0 = mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin,
                                          torch.from_numpy(pos.astype(np.int32)).to(device))
    torch.cuda.synchronize()
    assert torch.equal(q, q0[0]) and torch.equal(k, k0[0]) and torch.equal(v, v0[0])
