"""GPU tests of the fused paged-KV-cache write (mqk_fused_qkv_rope_paged_*).

The cache layout and addressing follow the reference's KVCache
(mini_qwen/cache/kv_cache.py:3-6: [num_blocks, block_size, H_kv, D]) and its
scatter kernel (mini_qwen/kernels/paged_attn_prefill.py:45-56: block =
block_table[seq][pos // block_size], slot = pos % block_size).  The fused op
must leave, in every addressed slot, exactly the K / V rows it returns (bit for
bit: the same bf16 values are stored twice), leave every other slot untouched,
and return q / k / v identical to the unpaged op.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case

pytestmark = pytest.mark.gpu

D = HEAD_DIM
SENTINEL = 0x7F7F  # bf16 bit pattern no kernel output here takes (a huge finite value)


def _caches(num_blocks, block_size, Hkv, device):
    k = torch.full((num_blocks, block_size, Hkv, D), SENTINEL, dtype=torch.int16, device=device)
    v = torch.full_like(k, SENTINEL)
    return k.view(torch.bfloat16), v.view(torch.bfloat16)


def _block_table(n_seq, blocks_per_seq, num_blocks, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(num_blocks, generator=g)[: n_seq * blocks_per_seq]
    return perm.view(n_seq, blocks_per_seq).to(torch.int32)


def _expected_slots(seq, pos, bt, block_size, num_blocks=None):
    """Flat cache slot of every token, from the oracle's restatement of the
    reference scatter (paged_attn_prefill.py:47-51); -1 = not written."""
    from oracle import qkv_rope_oracle as orc
    return orc.paged_slot(bt, seq, pos, block_size, num_blocks)


def _check_cache(cache, rows, slots, label):
    """cache [NB, bs, H, D]; rows [T, H, D] expected at flat slots [T]; all else sentinel."""
    flat = cache.view(torch.int16).reshape(-1, cache.shape[2], D).cpu()
    want = rows.view(torch.int16).reshape(-1, cache.shape[2], D).cpu()
    slots = torch.as_tensor(slots, dtype=torch.int64)
    assert torch.equal(flat[slots], want), f"{label}: cache rows differ from the returned K/V"
    mask = torch.ones(flat.shape[0], dtype=torch.bool)
    mask[slots] = False
    assert bool((flat[mask] == SENTINEL).all()), f"{label}: a slot outside the table was written"


@pytest.mark.parametrize("variant", [0, 1, 18])
def test_paged_prefill(variant, device):
    import mqk
    B, S, hidden, Hq, Hkv, bs = 2, 100, 1024, 16, 8, 16
    case = Case(B, S, hidden, Hq, Hkv, seed=1200 + variant)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    nb = 40
    bt = _block_table(B, 8, nb, seed=variant)
    kc, vc = _caches(nb, bs, Hkv, device)
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", variant)
        q, k, v = mqk.fused_qkv_rope_paged(x, wq, wk, wv, gq, gk, cos, sin, kc, vc, bt.to(device))
        q0, k0, v0 = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)
    t = np.arange(B * S)
    slots = _expected_slots(t // S, t % S, bt.numpy(), bs)
    _check_cache(kc, k.reshape(B * S, Hkv, D), slots, f"prefill k (tile {variant})")
    _check_cache(vc, v.reshape(B * S, Hkv, D), slots, f"prefill v (tile {variant})")


@pytest.mark.parametrize("B", [1, 8, 64])
def test_paged_decode_cache_only(B, device):
    """The decode step (one token per sequence, positions mode): K/V go to the cache
    only, as write_kv_decode does after fused_qkv_rope (attention.py:150-153)."""
    import mqk
    hidden, Hq, Hkv, bs = 1024, 16, 8, 16
    g = torch.Generator().manual_seed(B)
    positions = torch.randint(0, 2000, (B,), generator=g, dtype=torch.int32)
    case = Case(B, 1, hidden, Hq, Hkv, seed=1300 + B, rows=2048, positions=positions)
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    nb = B * 128 + 7
    bt = _block_table(B, 125, nb, seed=B)
    kc, vc = _caches(nb, bs, Hkv, device)
    seq = torch.arange(B, dtype=torch.int32)
    q, k, v = mqk.fused_qkv_rope_paged(x, wq, wk, wv, gq, gk, cos, sin, kc, vc, bt.to(device),
                                       positions=pos, kv_seq=seq.to(device), kv_pos=pos, return_kv=False)
    q0, k0, v0 = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
    torch.cuda.synchronize()
    assert k is None and v is None and torch.equal(q, q0)
    slots = _expected_slots(seq.numpy(), positions.numpy(), bt.numpy(), bs)
    _check_cache(kc, k0.reshape(B, Hkv, D), slots, f"decode k B={B}")
    _check_cache(vc, v0.reshape(B, Hkv, D), slots, f"decode v B={B}")


def test_paged_out_of_range_entries_skipped(device):
    """Entries whose block is -1 / past num_blocks, whose page is past the table, or
    whose sequence is past the table are not written (and nothing faults)."""
    import mqk
    B, S, hidden, Hq, Hkv, bs = 1, 64 + 16, 512, 4, 2, 16
    case = Case(B, S, hidden, Hq, Hkv, seed=77)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    nb = 6
    bt = torch.tensor([[3, -1, 99, 0]], dtype=torch.int32)  # pages 1, 2 invalid; page 4 past the table
    kc, vc = _caches(nb, bs, Hkv, device)
    q, k, v = mqk.fused_qkv_rope_paged(x, wq, wk, wv, gq, gk, cos, sin, kc, vc, bt.to(device))
    torch.cuda.synchronize()
    t = np.arange(S)
    all_slots = _expected_slots(np.zeros(S, dtype=np.int64), t, bt.numpy(), bs, nb)
    ok = all_slots >= 0
    assert np.array_equal(ok, (t // bs == 0) | (t // bs == 3))  # pages 0 and 3 only
    _check_cache(kc, k.reshape(S, Hkv, D)[torch.from_numpy(ok)], all_slots[ok], "partial table k")
    # a sequence index past the table
    seq = torch.full((S,), 5, dtype=torch.int32)
    kc2, vc2 = _caches(nb, bs, Hkv, device)
    mqk.fused_qkv_rope_paged(x, wq, wk, wv, gq, gk, cos, sin, kc2, vc2, bt.to(device),
                             kv_seq=seq.to(device))
    torch.cuda.synchronize()
    assert (_expected_slots(seq.numpy(), t, bt.numpy(), bs, nb) == -1).all()
    assert bool((kc2.view(torch.int16) == SENTINEL).all())


def test_paged_positions_mode_needs_slots(device):
    import mqk
    case = Case(1, 4, 256, 2, 1, seed=3, positions=torch.arange(4, dtype=torch.int32))
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    kc, vc = _caches(4, 16, 1, device)
    with pytest.raises(ValueError, match="kv_seq and kv_pos"):
        mqk.fused_qkv_rope_paged(x, wq, wk, wv, gq, gk, cos, sin, kc, vc,
                                 torch.zeros(1, 1, dtype=torch.int32, device=device), positions=pos)


@pytest.mark.parametrize("S,variant", [(1, 0), (200, 0), (200, 4)])
def test_paged_w4a16(S, variant, device):
    import mqk
    hidden, Hq, Hkv, bs = 512, 4, 2, 16
    B = 3
    g = torch.Generator().manual_seed(S + variant)
    projs = []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w, 128)))
    x = torch.randn(B, S, hidden, generator=g).bfloat16().to(device)
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    c, s_ = mqk.rope_tables(D, max(S, 16))
    cos, sin = c.bfloat16().to(device), s_.bfloat16().to(device)
    nb = B * ((S + bs - 1) // bs) + 5
    bt = _block_table(B, (S + bs - 1) // bs, nb, seed=S)
    kc, vc = _caches(nb, bs, Hkv, device)
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", variant)
        q, k, v = mqk.fused_qkv_rope_w4a16_paged(x, *projs, gq, gk, cos, sin, kc, vc, bt.to(device))
        q0, k0, v0 = mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)
    t = np.arange(B * S)
    slots = _expected_slots(t // S, t % S, bt.numpy(), bs)
    _check_cache(kc, k.reshape(B * S, Hkv, D), slots, f"w4a16 k S={S}")
    _check_cache(vc, v.reshape(B * S, Hkv, D), slots, f"w4a16 v S={S}")
