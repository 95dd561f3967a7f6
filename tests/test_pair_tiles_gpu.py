"""Pair tiles (variants 24-28): two workgroups share one head.

A pair of 256-row (24, 25), 128-row (26, 27) or 192-row (28) workgroups covers
2 * hpt + 1 heads (3 for variants 24, 26 and 28, 256 x 192 / 128 x 192 / 192 x 192
each; 5 for variants 25 and 27, 256 x 320 / 128 x 320 each).  Each side holds hpt whole heads and half
of the head they share: head dims 32*side + [0, 32) and + [64, 96), so every RoPE
pair (d, d + 64) stays on one side.  The shared head's RMSNorm needs both halves'
sums of squares, which the sides exchange through the workspace (a side whose
bounded wait runs out hands its fp32 half to the partner instead).

The sums are formed in the whole-head epilogue's order (each side adds its four
16-dim runs with the first two butterfly levels; own + other is the third), and
every accumulator sums the same k-steps in the same order as any other pipelined
tile, so the outputs must equal variant 16's / 18's bit for bit -- through both
exchange paths, with RoPE positions, varlen offsets, the input RMSNorm and the
paged-cache write, under graph replay and on many streams.  The oracle bar of
test_fused_qkv_rope_gpu.py (max-abs 2e-2, rel-L2 1e-2) is checked at BASELINE
config 4's dims, where the planner takes variant 25, and at the mid token counts
where it takes the 128-row pairs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32, launched_kernels

pytestmark = pytest.mark.gpu

D = HEAD_DIM
MAX_ABS = 2e-2
REL_L2 = 1e-2
# (variant, Hq, Hkv, whole-head variant of the same heads): 48 heads tile as pairs of
# 3 and as 128 x 384; 40 heads as pairs of 5 and as 256 x 256.  The shared heads
# are Q, K and V heads in both (48: 1, 4, .., 34, 37 (K), 40, 43, 46 (V);
# 40: 2, 7, .., 27, 32 (K), 37 (V)).
PAIRS = [(24, 32, 8, 16), (25, 32, 4, 18), (26, 32, 8, 16), (27, 32, 4, 18), (28, 32, 8, 16)]


def _opts(**kv):
    import mqk
    old = {k: mqk.get_option(k) for k in kv}
    for k, v in kv.items():
        mqk.set_option(k, v)
    return old


def _run(fn, **kv):
    import mqk
    old = _opts(**kv)
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        for k, v in old.items():
            mqk.set_option(k, v)


def _same(out, ref, label):
    for name, a, b in zip("qkv", out, ref):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{label}: {name} differs"


@pytest.mark.parametrize("variant,Hq,Hkv,whole", PAIRS)
@pytest.mark.parametrize("positions", [False, True])
def test_pair_tiles_bit_identical(variant, Hq, Hkv, whole, positions, device):
    """T = 600: two full row tiles and an 88-row tail; prefill and positions modes."""
    import mqk
    T, hidden = 600, 1024
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(41), dtype=torch.int32) \
        if positions else None
    case = Case(1, T, hidden, Hq, Hkv, seed=4100 + variant, rows=4096 if positions else None, positions=pos)
    args = case.args(device)
    ref = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=whole, tail_split=0)
    out = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant, tail_split=0)
    _same(out, ref, f"variant {variant}")


@pytest.mark.parametrize("variant,Hq,Hkv,whole", PAIRS)
def test_pair_tiles_hand_over(variant, Hq, Hkv, whole, device):
    """Side 1 of every pair holds back before publishing and side 0 polls once
    (pair_max_spins = 0), so every side 0 of a Q or K head hands its fp32 half
    over and side 1 finishes both halves: the same bits.  The next call, with
    the exchange back to normal, finds every pair word cleared."""
    import mqk
    T, hidden = 512, 1024
    case = Case(1, T, hidden, Hq, Hkv, seed=4200 + variant)
    args = case.args(device)
    ref = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=whole)
    out = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant, pair_max_spins=0, pair_hold=25)
    _same(out, ref, f"variant {variant} (hand-over)")
    again = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant)
    _same(again, ref, f"variant {variant} (after a hand-over)")


def _ex_case(hidden, seed):
    """Varlen batch of four sequences (one empty) with start offsets, a paged KV
    cache behind a shuffled block table, and the decoder's input RMSNorm."""
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor([0, 150, 150, 380, 600], dtype=torch.int32)
    start = torch.tensor([3, 0, 700, 40], dtype=torch.int32)
    bs, per_seq = 16, 59  # covers position 700 + 230
    bt = torch.randperm(4 * per_seq + 8, generator=g)[: 4 * per_seq].view(4, per_seq).to(torch.int32)
    in_w = (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16()
    return 600, cu, start, bs, bt, 4 * per_seq + 8, in_w


@pytest.mark.parametrize("variant,Hq,Hkv,whole", PAIRS)
def test_pair_tiles_ex_features(variant, Hq, Hkv, whole, device):
    """Varlen positions, the input RMSNorm and the paged-cache write: outputs and
    cache contents (sentinel-filled, so unwritten rows stay visible) equal the
    whole-head variant's bit for bit."""
    import mqk
    hidden = 1024
    T, cu, start, bs, bt, nb, in_w = _ex_case(hidden, 4300 + variant)
    case = Case(1, T, hidden, Hq, Hkv, seed=4301 + variant, rows=1024)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    cu_d, st_d, bt_d, inw_d = cu.to(device), start.to(device), bt.to(device), in_w.to(device)

    def call(v):
        kc = torch.full((nb, bs, Hkv, D), -7, dtype=torch.int16, device=device).view(torch.bfloat16)
        vc = kc.clone()
        out = _run(lambda: mqk.fused_qkv_rope_ex(x.view(T, hidden), wq, wk, wv, gq, gk, cos, sin,
                                                 cu_seqlens=cu_d, seq_pos0=st_d, input_norm_w=inw_d,
                                                 k_cache=kc, v_cache=vc, block_table=bt_d),
                   prefill_tile=v, tail_split=0)
        return list(out) + [kc, vc]

    ref, out = call(whole), call(variant)
    assert (ref[3].view(torch.int16) != -7).any()  # the cache was written
    for name, a, b in zip(["q", "k", "v", "k_cache", "v_cache"], out, ref):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"variant {variant}: {name} differs"


@pytest.mark.parametrize("variant,Hkv", [(25, 4), (26, 8), (28, 8)])
def test_pair_tiles_graph_replay(variant, Hkv, device):
    """Pair tiles in a HIP graph: the pair words are cleared by the launch itself,
    so replays, with eager calls of the same and another plan in between, stay
    bit-exact."""
    import mqk
    case = Case(1, 1024, 2048, 32, Hkv, seed=4400)
    args = case.args(device)
    small = Case(1, 64, 2048, 32, Hkv, seed=4401).args(device)
    old = _opts(prefill_tile=variant)
    try:
        stream = torch.cuda.Stream(device)
        with torch.cuda.stream(stream):
            eager = mqk.fused_qkv_rope(*args)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                out = mqk.fused_qkv_rope(*args)
        for rep in range(4):
            for t in out:
                t.fill_(0)
            graph.replay()
            torch.cuda.synchronize()
            assert all(torch.equal(a, b) for a, b in zip(out, eager)), f"replay {rep}"
            with torch.cuda.stream(stream):
                mqk.fused_qkv_rope(*small)
                mqk.fused_qkv_rope(*args)
            torch.cuda.synchronize()
    finally:
        for k, v in old.items():
            mqk.set_option(k, v)


@pytest.mark.parametrize("variant,Hq,Hkv,whole", PAIRS)
def test_pair_tiles_across_xcds(variant, Hq, Hkv, whole, device):
    """The two sides of every pair on different XCDs (adjacent workgroup ids), in
    the normal exchange and through the hand-over path: the device-coherent
    exchange gives the same bits as the whole-head tiles."""
    import mqk
    case = Case(1, 512, 1024, Hq, Hkv, seed=4800 + variant)
    args = case.args(device)
    ref = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=whole)
    out = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant, pair_cross_xcd=1)
    _same(out, ref, f"variant {variant} across XCDs")
    out = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant, pair_cross_xcd=1, pair_max_spins=0,
               pair_hold=25)
    _same(out, ref, f"variant {variant} across XCDs (hand-over)")


@pytest.mark.parametrize("variant", [24, 26, 28])
def test_pair_tiles_on_many_streams(variant, device):
    """The exchange uses device-coherent accesses, so a pair whose sides land on
    different XCDs (whatever the hardware queue's starting XCD) still agrees."""
    import mqk
    case = Case(1, 512, 1024, 32, 8, seed=4500)
    args = case.args(device)
    ref = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=16)
    old = _opts(prefill_tile=variant)
    try:
        streams = [torch.cuda.Stream(device) for _ in range(8)]
        for i, st in enumerate(streams):
            with torch.cuda.stream(st):
                got = [mqk.fused_qkv_rope(*args) for _ in range(2)]
                st.synchronize()
            for g in got:
                _same(g, ref, f"stream {i}")
    finally:
        for k, v in old.items():
            mqk.set_option(k, v)


def test_config4_takes_pair_tiles_and_meets_the_oracle(device):
    """BASELINE config 4 (Qwen3-30B-A3B attention, B=1 x S=8192, hidden 2048,
    32 / 4 heads): the planner's one launch is variant 25 (512 workgroups, two
    rounds); sampled tokens against the oracle at the acceptance bar, and every
    token against variant 18 bit for bit."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    case = Case(1, 8192, 2048, 32, 4, seed=4600)
    args = case.args(device)
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*args)) == ["tile_pair"]
    q, k, v = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    idx = np.sort(np.random.default_rng(46).choice(8192, 96, replace=False))
    ref = case.oracle(token_idx=idx)
    for name, o, r in zip("qkv", (q, k, v), ref):
        o = f32(o).reshape(8192, -1, D)[idx].reshape(r.shape)
        assert np.isfinite(o).all()
        assert orc.max_abs(o, r) <= MAX_ABS, name
        assert orc.rel_l2(o, r) <= REL_L2, name
    whole = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=18)
    _same((q, k, v), whole, "config 4")


def test_pair_tiles_not_taken_without_workspace_room_or_for_head_dim_64(device):
    """A head_dim 64 call never plans pair tiles (its heads do not split into the
    32-dim runs), and an explicit pair variant is refused for it."""
    import mqk
    case = Case(1, 1024, 2048, 64, 8, seed=4700, head_dim=64)
    args = case.args(device)
    kernels = launched_kernels(lambda: mqk.fused_qkv_rope(*args))
    assert "tile_pair" not in kernels
    old = _opts(prefill_tile=25)
    try:
        with pytest.raises(Exception):
            mqk.fused_qkv_rope(*args)
            torch.cuda.synchronize()
    finally:
        for k, v in old.items():
            mqk.set_option(k, v)


@pytest.mark.parametrize("T,hidden,Hq,Hkv,variant,whole", [(1024, 4096, 32, 8, 26, 16), (768, 2560, 32, 8, 26, 16),
                                                          (2048, 2048, 32, 4, 27, 18), (1536, 4096, 32, 8, 28, 16),
                                                          (1400, 2560, 32, 8, 28, 16)])
def test_mid_t_takes_pair_tiles_and_meets_the_oracle(T, hidden, Hq, Hkv, variant, whole, device):
    """One round of pair tiles where no whole-head shape fills the CUs: Qwen3-8B
    at T = 1024 (8 x 16 pairs of 2 x 128 x 192, where the split-K launch ran
    before) and T = 1536 (8 x 16 pairs of 2 x 192 x 192), Qwen3-4B dims at T = 768
    (6 x 16 pairs of 128-row tiles) and T = 1400 (8 x 16 pairs of 192-row tiles,
    the last one partial), Qwen3-30B-A3B attention dims at T = 2048 (16 x 8 pairs
    of 2 x 128 x 320).  The planner's one launch is the pair kernel; sampled tokens
    against the oracle at the acceptance bar, every token against the whole-head
    tiles bit for bit."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    case = Case(1, T, hidden, Hq, Hkv, seed=4900 + T)
    args = case.args(device)
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*args)) == ["tile_pair"]
    got = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    idx = np.sort(np.random.default_rng(T).choice(T, 64, replace=False))
    ref = case.oracle(token_idx=idx)
    for name, o, r in zip("qkv", got, ref):
        o = f32(o).reshape(T, -1, D)[idx].reshape(r.shape)
        assert np.isfinite(o).all()
        assert orc.max_abs(o, r) <= MAX_ABS, name
        assert orc.rel_l2(o, r) <= REL_L2, name
    forced = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=variant)
    _same(got, forced, f"planner against variant {variant}")
    whole_out = _run(lambda: mqk.fused_qkv_rope(*args), prefill_tile=whole)
    _same(got, whole_out, f"T = {T}, hidden {hidden}")
