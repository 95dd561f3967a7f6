"""GPU tests of the decode-block plan.

A call of 64 < T tokens whose tile launch would leave most CUs idle (few row
tiles, long K) runs instead as a launch of the split-K decode kernel that
streams the weights over every CU once for all its 64-row blocks (up to
sixteen; option decode_passes caps the blocks per launch, and row 0 of a
further launch is the call's token 64 * (blocks before it), so positions,
cache slots and varlen offsets keep the call's token index).  Block b is
finished by its designated split b % splits, or, when that split's bounded
wait runs out, by the last split to arrive.  Each block must equal the decode
kernel run on those 64 rows alone, bit for bit, whatever the blocks per launch
and whoever finishes it; the whole call must match the oracle and, within the
acceptance bar, the tile path (option decode_blocks = 0).
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


def _with_option(name, value, fn):
    import mqk
    old = mqk.get_option(name)
    try:
        mqk.set_option(name, value)
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        mqk.set_option(name, old)


def _blocks(fn):
    """fn with the decode blocks forced (the planner takes them whenever eligible)."""
    return _with_option("decode_cost_model", 0, fn)


def _close(a, b, label):
    """Two kernel families against each other (each is held to the oracle bar
    separately): they may round an element to neighbouring bf16 values, one ulp
    apart, which above |v| = 4 exceeds 2e-2; the bound is the larger of the two."""
    for name, x, y in zip("qkv", a, b):
        x, y = f32(x), f32(y)
        ma, rl = orc.max_abs(x, y), orc.rel_l2(x, y)
        excess = np.abs(x - y) - np.maximum(MAX_ABS, 2.0 ** -7 * np.abs(y))
        assert float(excess.max()) <= 0 and rl <= REL_L2, f"{label} {name}: {ma} {rl}"


@pytest.mark.parametrize("T", [65, 128, 200, 256, 300, 448, 832, 1024])
def test_decode_blocks_bf16(T, device):
    import mqk
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = Case(1, T, 4096, 32, 8, seed=1100 + T, rows=8192, positions=pos)
    x, wq, wk, wv, gq, gk, cos, sin, p = case.args(device)
    call = lambda: mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, p)
    # decode blocks whatever the cost model prefers (1024 tokens at hidden 4096
    # run as a tile launch by default)
    out = _with_option("decode_cost_model", 0, call)
    for t0 in range(0, T, 64):
        alone = mqk.fused_qkv_rope(x[:, t0:t0 + 64].contiguous(), wq, wk, wv, gq, gk, cos, sin, p[t0:t0 + 64])
        torch.cuda.synchronize()
        for a, b in zip(out, alone):
            assert torch.equal(a[:, t0:t0 + 64], b), f"T={T}: block at {t0} differs from the decode kernel alone"
    for passes in (3, 1):  # several launches sharing the workspace in stream order
        more = _with_option("decode_passes", passes, lambda: _with_option("decode_cost_model", 0, call))
        assert all(torch.equal(a, b) for a, b in zip(out, more)), f"T={T}: {passes} blocks per launch"
    tile = _with_option("decode_blocks", 0, call)
    _close(out, tile, f"T={T} blocks vs tile")
    idx = np.unique(np.concatenate([np.arange(0, 4), np.arange(60, 70), np.arange(T - 4, T)]).clip(0, T - 1))
    ref = case.oracle(token_idx=idx)
    for name, o, r in zip("qkv", out, ref):
        o = f32(o)[0, idx].reshape(r.shape)
        assert orc.max_abs(o, r) <= MAX_ABS and orc.rel_l2(o, r) <= REL_L2, f"T={T} {name} vs oracle"


def test_decode_blocks_w4a16(device):
    import mqk
    from test_w4a16_gpu import _check_w4, _int4_case
    T, hidden, Hq, Hkv = 200, 1024, 16, 8
    x, projs, gq, gk = _int4_case(1, T, hidden, Hq, Hkv, seed=1201, scale_dtype=torch.float16)
    c, s = mqk.rope_tables(D, 4096)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(7), dtype=torch.int32)
    dp = [tuple(t.to(device) for t in pr) for pr in projs]
    xd, args = x.to(device), (gq.to(device), gk.to(device), cos.to(device), sin.to(device))
    mqk.set_option("head_tiles", 0)  # (one round of int4 single-head tiles would take this call)
    try:
        out = mqk.fused_qkv_rope_w4a16(xd, *dp, *args, pos.to(device))
        torch.cuda.synchronize()
    finally:
        mqk.set_option("head_tiles", 1)
    for t0 in range(0, T, 64):
        alone = mqk.fused_qkv_rope_w4a16(xd[:, t0:t0 + 64].contiguous(), *dp, *args, pos[t0:t0 + 64].to(device))
        torch.cuda.synchronize()
        for a, b in zip(out, alone):
            assert torch.equal(a[:, t0:t0 + 64], b), f"int4 block at {t0} differs from the decode kernel alone"
    _check_w4(out, x, projs, gq, gk, cos, sin, Hq, Hkv, pos.numpy(), "w4a16 decode blocks")


def test_decode_blocks_varlen_paged_input_norm(device):
    """Varlen offsets, paged-cache slots and the input-norm scales follow the
    call's token index across block launches: equal to the tile path within the
    bar, with every cache slot holding the returned K/V."""
    import mqk
    from test_paged_gpu import _block_table, _caches, _check_cache, _expected_slots
    lens = np.array([70, 0, 45, 35])
    T, hidden, Hq, Hkv, bs = int(lens.sum()), 4096, 32, 8, 16
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    start = np.array([5, 0, 300, 17])
    seq, posv = orc.varlen_positions(cu, start)
    case = Case(1, T, hidden, Hq, Hkv, seed=1300, rows=4096)
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

    (q, k, v), kc, vc = run()
    torch.cuda.synchronize()
    (qt, kt, vt), _, _ = _with_option("decode_blocks", 0, run)
    _close((q, k, v), (qt, kt, vt), "varlen + paged + input norm, blocks vs tile")
    slots = _expected_slots(seq, posv, bt.numpy(), bs)
    _check_cache(kc, k, slots, "k cache")
    _check_cache(vc, v, slots, "v cache")


def test_decode_blocks_recompute_path(device):
    """The recompute fallback (a split on an unexpected XCD) over a four-block
    launch: every block recomputed by the last arrival, bit-identical."""
    import mqk
    T = 256
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(3), dtype=torch.int32)
    case = Case(1, T, 4096, 32, 8, seed=1400, rows=8192, positions=pos)
    args = case.args(device)
    call = lambda: _blocks(lambda: mqk.fused_qkv_rope(*args))
    assert launched_kernels(call) == ["decode_multi"]
    out = call()
    again = _with_option("decode_force_recompute", 1, call)
    for a, b in zip(out, again):
        assert torch.equal(a, b)


@pytest.mark.parametrize("spins", [0, 1, 64])
def test_decode_blocks_finisher_hand_off(spins, device):
    """A designated finisher whose (host-shortened) wait runs out marks its block
    abandoned and the block's last split to arrive finishes it instead: every
    block is finished exactly once, bit-identical to the default."""
    import mqk
    T = 512
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(12), dtype=torch.int32)
    case = Case(1, T, 4096, 32, 8, seed=1450, rows=8192, positions=pos)
    args = case.args(device)
    call = lambda: _blocks(lambda: mqk.fused_qkv_rope(*args))
    assert launched_kernels(call) == ["decode_multi"]
    want = call()
    for rep in range(3):
        got = _with_option("decode_max_spins", spins, call)
        assert all(torch.equal(a, b) for a, b in zip(got, want)), f"spins={spins} rep={rep}"
    again = call()  # the counters were left at zero
    assert all(torch.equal(a, b) for a, b in zip(again, want))


def test_decode_blocks_input_norm_four_blocks(device):
    """The fused input RMSNorm across a four-block launch: each block equals the
    same op on its 64 rows alone."""
    import mqk
    T, hidden = 256, 4096
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(4), dtype=torch.int32)
    case = Case(1, T, hidden, 32, 8, seed=1500, rows=8192, positions=pos)
    x, wq, wk, wv, gq, gk, cos, sin, p = case.args(device)
    g_in = (1 + 0.3 * torch.randn(hidden, generator=torch.Generator().manual_seed(5))).bfloat16().to(device)
    call = lambda: _blocks(lambda: mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, p, input_norm_w=g_in))
    assert launched_kernels(call) == ["row_scale", "decode_multi"]
    out = call()
    for t0 in range(0, T, 64):
        alone = mqk.fused_qkv_rope_ex(x[:, t0:t0 + 64].contiguous(), wq, wk, wv, gq, gk, cos, sin,
                                      p[t0:t0 + 64], input_norm_w=g_in)
        torch.cuda.synchronize()
        for a, b in zip(out, alone):
            assert torch.equal(a[:, t0:t0 + 64], b), f"input-norm block at {t0} differs"


def test_topology_and_recompute_statistic(device):
    """The planner's topology comes from the device (all CUs; 8 XCDs on an
    unpartitioned MI355X), and every head finished on the recompute path is
    counted in the workspace's statistics word."""
    import mqk
    assert mqk.get_option("device_cus") == torch.cuda.get_device_properties(device).multi_processor_count
    xcds = mqk.get_option("device_xcds")
    assert xcds >= 1 and mqk.get_option("device_cus") % xcds == 0
    print(f"  device: {mqk.get_option('device_cus')} CUs in {xcds} XCDs")
    case = Case(16, 1, 1024, 16, 8, seed=4711, rows=4096,
                positions=torch.arange(16, dtype=torch.int32) * 3)
    args = case.args(device)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        want = mqk.fused_qkv_rope(*args)
        natural = mqk.decode_recomputes(device, stream)
        print(f"  heads finished on the recompute path without forcing: {natural}")
        mqk.set_option("decode_force_recompute", 1)
        try:
            got = [mqk.fused_qkv_rope(*args) for _ in range(3)]
        finally:
            mqk.set_option("decode_force_recompute", 0)
        after = mqk.decode_recomputes(device, stream)
    assert after - natural == 3 * (16 + 2 * 8)
    for g in got:
        assert all(torch.equal(a, b) for a, b in zip(g, want))
