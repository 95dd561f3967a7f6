"""Decode splits longer than one x slice (bf16, T <= 64).

The decode kernel stages a split's x slice (64 rows x up to 16 k tiles) in LDS.
Wider models need more: hidden 5120 with 56 heads (Qwen3-14B) takes 4 splits of
20 tiles per head to keep one workgroup per CU, and 72 heads at hidden 4096
(Qwen3-235B-A22B) 3 splits of 21-22.  Such launches run `decode_long_kernel`:
each split stages its range in two slices and accumulates the tiles in order,
and its recompute path slices the same way, so the recompute and hand-off
paths stay bit-identical.  A launch whose longest split exceeds one slice can
hold a split of exactly 16 tiles (balanced ranges), covered here with hidden
2112 (33 tiles) in two splits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import Case, f32, launched_kernels
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu


def _opts(opts, fn):
    import mqk
    old = {k: mqk.get_option(k) for k in opts}
    try:
        for k, v in opts.items():
            mqk.set_option(k, v)
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        for k, v in old.items():
            mqk.set_option(k, v)


def _case(T, hidden, hq, hkv, seed):
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    return Case(T, 1, hidden, hq, hkv, seed=seed, rows=8192, positions=pos)


def _check(out, case, label):
    ref = case.oracle()
    for name, o, r in zip("qkv", out, ref):
        o = f32(o).reshape(r.shape)
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        assert ma <= 2e-2 and rl <= 1e-2, f"{label} {name}: {ma:.4f} {rl:.2e}"


@pytest.mark.parametrize("T,hidden,hq,hkv,splits", [
    (64, 5120, 40, 8, {}), (1, 5120, 40, 8, {}), (37, 5120, 64, 8, {}), (64, 4096, 64, 4, {}),
    (64, 2112, 16, 8, {"decode_splits": 2})])
def test_long_splits_match_oracle_and_recompute(T, hidden, hq, hkv, splits, device):
    import mqk
    case = _case(T, hidden, hq, hkv, seed=4000 + T + hidden)
    args = case.args(device)
    call = lambda: mqk.fused_qkv_rope(*args)
    assert _opts(splits, lambda: launched_kernels(call)) == ["decode"]
    want = _opts(splits, call)
    _check(want, case, f"T={T} hidden={hidden}")
    for extra in ({"decode_force_recompute": 1}, {"decode_max_spins": 0}, {"decode_max_spins": 1}):
        got = _opts({**splits, **extra}, call)
        assert all(torch.equal(a, b) for a, b in zip(got, want)), extra
    again = _opts(splits, call)  # the counters were re-armed
    assert all(torch.equal(a, b) for a, b in zip(again, want))


def test_long_splits_with_input_norm(device):
    """The input-norm form of the long-split kernel against the tile kernel on
    the same call (both meet the bar; they differ only in summation order)."""
    import mqk
    case = _case(48, 5120, 40, 8, seed=4100)
    args = case.args(device)
    gam = (1 + 0.1 * torch.randn(5120, generator=torch.Generator().manual_seed(4101))).bfloat16().to(device)
    call = lambda: mqk.fused_qkv_rope_ex(*args[:8], positions=args[8], input_norm_w=gam)
    assert launched_kernels(call) == ["row_scale", "decode"]
    got = _opts({}, call)
    ref = _opts({"decode_max_t": 0, "decode_blocks": 0, "tile_ksplit": 0}, call)
    rec = _opts({"decode_force_recompute": 1}, call)
    for a, b, c in zip(got, ref, rec):
        assert torch.equal(a, c)
        assert orc.max_abs(f32(a), f32(b)) <= 2e-2 and orc.rel_l2(f32(a), f32(b)) <= 1e-2


@pytest.mark.parametrize("T,hidden,hq,hkv", [(64, 5120, 40, 8), (17, 4096, 64, 4)])
def test_long_splits_int4(T, hidden, hq, hkv, device):
    """int4 weights (dequantised per tile, splits run in two halves) against the
    oracle, with the recompute and hand-off paths bit-identical."""
    import mqk
    case = _case(T, hidden, hq, hkv, seed=4200 + T)
    args = case.args(device)
    projs = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128, torch.bfloat16))
             for w in (case.w_q, case.w_k, case.w_v)]
    call = lambda: mqk.fused_qkv_rope_w4a16(args[0], *projs, *args[4:])
    assert launched_kernels(call) == ["decode"]
    want = _opts({}, call)
    ref = orc.fused_qkv_rope_w4a16(f32(case.x).reshape(1, T, hidden), [p[0].cpu().numpy() for p in projs],
                                   [p[1].float().cpu().numpy() for p in projs], [p[2].cpu().numpy() for p in projs],
                                   f32(case.q_norm_w), f32(case.k_norm_w), f32(case.cos), f32(case.sin), hq, hkv,
                                   positions=case.positions.numpy(), round_weight=True)
    for name, o, r in zip("qkv", want, ref):
        o = f32(o).reshape(r.shape)
        assert orc.max_abs(o, r) <= 2e-2 and orc.rel_l2(o, r) <= 1e-2, name
    for extra in ({"decode_force_recompute": 1}, {"decode_max_spins": 0}):
        got = _opts(extra, call)
        assert all(torch.equal(a, b) for a, b in zip(got, want)), extra
