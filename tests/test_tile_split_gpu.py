"""GPU tests of the split-K tile launch.

With fewer tiles than CUs (64 < T up to about a thousand tokens at hidden
4096), the pipelined tile kernel can cut each tile's K range over several
workgroups of one XCD: each publishes its fp32 partial and counts its arrival;
once all have arrived, each sums its share of the tile's rows over the
partials in split order and runs the usual epilogue on them.  Results must
meet the oracle bar for every split count and both split shapes (128 x 384
when the heads tile by 3, 256 x 256 otherwise), with positions, varlen
offsets, the paged-cache write and the input norm; the recompute fallback (a
split on an unexpected XCD) and the hand-off of a split's rows to the last
arrival (its bounded wait run out) must give identical bits; one call is one
launch.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32, launched_kernels
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

D = HEAD_DIM
MAX_ABS, REL_L2 = 2e-2, 1e-2


def _with_options(opts, fn):
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


def _check_oracle(out, case, T, label):
    idx = np.unique(np.concatenate([np.arange(0, 6), np.arange(120, 136), np.arange(250, 260),
                                    np.arange(T - 6, T)]).clip(0, T - 1))
    ref = case.oracle(token_idx=idx)
    for name, o, r in zip("qkv", out, ref):
        o = f32(o)[0, idx].reshape(r.shape)
        assert orc.max_abs(o, r) <= MAX_ABS and orc.rel_l2(o, r) <= REL_L2, f"{label} {name} vs oracle"


@pytest.mark.parametrize("T,hidden,Hq,Hkv,ksplit", [
    (129, 4096, 32, 8, 2), (256, 4096, 32, 8, 4), (512, 4096, 32, 8, 4), (512, 4096, 32, 8, 3),
    (1000, 4096, 32, 8, 2), (300, 2048, 32, 4, 4), (700, 2048, 32, 4, 2), (200, 1024, 16, 8, 4), (256, 4096, 32, 8, 8), (384, 4096, 32, 8, 5)])
def test_split_tile_matches_oracle(T, hidden, Hq, Hkv, ksplit, device):
    import mqk
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(T + ksplit), dtype=torch.int32)
    case = Case(1, T, hidden, Hq, Hkv, seed=2100 + T + ksplit, rows=8192, positions=pos)
    args = case.args(device)
    call = lambda: mqk.fused_qkv_rope(*args)
    assert launched_kernels(lambda: _with_options({"tile_ksplit": ksplit}, call)) == ["tile_split"]
    out = _with_options({"tile_ksplit": ksplit}, call)
    _check_oracle(out, case, T, f"T={T} hidden={hidden} ksplit={ksplit}")
    # the recompute fallback: every tile recomputed by its last arrival, same bits
    again = _with_options({"tile_ksplit": ksplit, "decode_force_recompute": 1}, call)
    assert all(torch.equal(a, b) for a, b in zip(out, again)), f"T={T}: recompute path differs"
    # every split's wait cut short: its rows handed to the last arrival, same bits
    handed = _with_options({"tile_ksplit": ksplit, "decode_max_spins": 0}, call)
    assert all(torch.equal(a, b) for a, b in zip(out, handed)), f"T={T}: hand-off path differs"
    # repeated calls reuse the workspace: the last split to leave re-armed every word
    once_more = _with_options({"tile_ksplit": ksplit}, call)
    assert all(torch.equal(a, b) for a, b in zip(out, once_more))


def test_split_tile_prefill_mode_and_default_plan(device):
    """Prefill mode (no positions) at the reference's (B, S) = (1, 512) point, as
    the default plan runs it, and B = 2 x S = 200 with the rows of two sequences
    in one tile."""
    import mqk
    for B, S in ((1, 512), (2, 200)):
        case = Case(B, S, 4096, 32, 8, seed=2200 + S)
        args = case.args(device)
        out = mqk.fused_qkv_rope(*args)
        torch.cuda.synchronize()
        T = B * S
        idx = np.unique(np.concatenate([np.arange(0, 5), np.arange(S - 5, S + 5), np.arange(T - 5, T)]).clip(0, T - 1))
        ref = case.oracle(token_idx=idx)
        forced = _with_options({"tile_ksplit": 4}, lambda: mqk.fused_qkv_rope(*args))
        for label, got in (("default plan", out), ("split 4", forced)):
            for name, o, r in zip("qkv", got, ref):
                o = f32(o).reshape(T, -1, D)[idx].reshape(r.shape)
                assert orc.max_abs(o, r) <= MAX_ABS and orc.rel_l2(o, r) <= REL_L2, f"B={B} S={S} {name} {label}"


def test_split_tile_varlen_paged_input_norm(device):
    """Varlen offsets, paged-cache slots and the input-norm scales in a split-K
    launch: within the bar of the one-workgroup-per-tile launch, every cache
    slot holding the returned K/V."""
    import mqk
    from test_decode_blocks_gpu import _close
    from test_paged_gpu import _block_table, _caches, _check_cache, _expected_slots
    lens = np.array([170, 0, 145, 135])
    T, hidden, Hq, Hkv, bs = int(lens.sum()), 4096, 32, 8, 16
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    start = np.array([5, 0, 300, 17])
    seq, posv = orc.varlen_positions(cu, start)
    case = Case(1, T, hidden, Hq, Hkv, seed=2300, rows=4096)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    x = x.reshape(T, hidden)
    g_in = (1 + 0.3 * torch.randn(hidden, generator=torch.Generator().manual_seed(9))).bfloat16().to(device)
    bt = _block_table(len(lens), 32, 256, seed=3)
    cu_d, st_d = torch.from_numpy(cu).to(device), torch.from_numpy(start.astype(np.int32)).to(device)

    def run():
        kc, vc = _caches(256, bs, Hkv, device)
        out = mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, cu_seqlens=cu_d, seq_pos0=st_d,
                                    input_norm_w=g_in, k_cache=kc, v_cache=vc, block_table=bt.to(device))
        return out, kc, vc

    (q, k, v), kc, vc = _with_options({"tile_ksplit": 4}, run)
    assert launched_kernels(lambda: _with_options({"tile_ksplit": 4}, run)) == ["row_scale", "tile_split"]
    (qt, kt, vt), _, _ = _with_options({"tile_ksplit": 0, "decode_blocks": 0}, run)
    _close((q, k, v), (qt, kt, vt), "varlen + paged + input norm, split tile vs tile")
    slots = _expected_slots(seq, posv, bt.numpy(), bs)
    _check_cache(kc, k, slots, "k cache")
    _check_cache(vc, v, slots, "v cache")


@pytest.mark.parametrize("T,hidden,Hq,Hkv,plan", [
    (128, 5120, 40, 8, "tile_split"), (768, 5120, 40, 8, "tile_split"), (1024, 5120, 40, 8, "tile_split"),
    (512, 2048, 32, 4, "tile_head"), (1024, 2048, 32, 4, "tile_split"), (256, 1024, 16, 8, "tile_head"),
    (384, 1024, 16, 8, "tile_head"), (320, 4096, 32, 8, "tile_head"), (640, 4096, 32, 8, "tile_head"),
    (512, 5120, 40, 8, "tile_head")])
def test_default_plan_other_shapes_matches_oracle(T, hidden, Hq, Hkv, plan, device):
    """The planner's own choices at the other Qwen3 attention shapes (Qwen3-14B
    heads at hidden 5120, 30B-A3B at 2048, 0.6B at 1024), decode-style positions,
    against the oracle; the plan is the one the refitted cost model picks there."""
    import mqk
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(T + hidden), dtype=torch.int32)
    case = Case(1, T, hidden, Hq, Hkv, seed=2300 + T + hidden, rows=8192, positions=pos)
    args = case.args(device)
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*args)) == [plan]
    out = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    _check_oracle(out, case, T, f"default plan T={T} hidden={hidden}")


def test_split_tile_counts_recomputed_tiles(device):
    """The statistics word counts the tiles a split-K launch finished on its
    recompute path: none when every split ran on the XCD the grid assumes (an
    unpartitioned MI355X), one per tile per call when the path is forced."""
    import mqk
    T, hidden, Hq, Hkv = 512, 4096, 32, 8
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(77), dtype=torch.int32)
    case = Case(1, T, hidden, Hq, Hkv, seed=2400, rows=8192, positions=pos)
    args = case.args(device)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        # (torch pools its streams, so this stream's workspace may carry counts of
        # earlier calls: the test counts differences)
        start = mqk.decode_recomputes(device, stream)
        split = {"head_tiles": 0}  # (single-head tiles would take this call)
        assert launched_kernels(lambda: _with_options(split, lambda: mqk.fused_qkv_rope(*args))) == ["tile_split"]
        want = _with_options(split, lambda: mqk.fused_qkv_rope(*args))
        natural = mqk.decode_recomputes(device, stream)
        got = _with_options({"decode_force_recompute": 1, "head_tiles": 0},
                            lambda: [mqk.fused_qkv_rope(*args) for _ in range(2)])
        after = mqk.decode_recomputes(device, stream)
    assert natural == start
    assert after - natural == 2 * (T // 128) * ((Hq + 2 * Hkv) // 3)  # 4 row tiles x 16 head tiles per call
    for g in got:
        assert all(torch.equal(a, b) for a, b in zip(g, want))
