"""Head sizes the fused kernels do not tile: a multiple of 8 up to 512, other than 64 and 128.

The reference op takes any even head_dim D (mini_qwen/kernels/fused_qkv_rope.py:155-160).
mqk runs D = 64 and 128 fused; other multiples of 8 up to 512 run as the reference
itself composes the op (fused_qkv_rope.py:166-190): the three projections as plain
GEMMs on the tile kernels, written into q, k and v (so rounded to bf16), then one
norm + RoPE launch in place on q and k.  The reference's own test holds its op to
that composition (test_fused_qkv_rope.py:39-72: bf16 projections, fp32 norm and
RoPE), so the outputs are held to the oracle with the same bf16 rounding of the
projection (``round_projection=True``) at the acceptance bar (max-abs 2e-2, rel-L2
1e-2); against the exact projection the rel-L2 bar holds too (the projection's
rounding moves single elements of |q| ~ 2 by up to ~2.1e-2), in prefill, positions
and varlen modes, with the paged-cache write and with the fused input RMSNorm.  (The
cases here meet 2e-2 exactly; an element whose fp32 sum sits within summation-order
error of a bf16 boundary can round the other way here than in the oracle, which
test_random_shapes_gpu.py bounds per element.)
Head sizes it cannot take raise.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import Case, f32, launched_kernels
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-2


def _check(out, case, idx, label):
    T = case.B * case.S
    for round_projection in (True, False):
        ref = case.oracle(token_idx=idx, round_projection=round_projection)
        for name, o, r in zip("qkv", out, ref):
            o = f32(o).reshape(T, -1, case.D)[idx].reshape(r.shape)
            assert np.isfinite(o).all(), f"{label}: {name}"
            if round_projection:
                assert orc.max_abs(o, r) <= MAX_ABS, f"{label}: {name} max-abs {orc.max_abs(o, r)}"
            assert orc.rel_l2(o, r) <= REL_L2, f"{label}: {name} rel-L2 {orc.rel_l2(o, r)} ({round_projection})"


@pytest.mark.parametrize("D,Hq,Hkv,hidden,B,S,positions", [
    (256, 16, 4, 2048, 2, 150, False),   # a 256-wide head, prefill
    (256, 8, 2, 1024, 64, 1, True),      # decode-style: one token per sequence
    (96, 32, 8, 2048, 1, 520, False),
    (80, 20, 4, 1024, 33, 1, True),      # Hkv * D = 320: a partial 128-column tile
    (192, 12, 4, 1536, 4, 50, False),
    (512, 4, 1, 2048, 1, 17, True),
])
def test_any_head_dim_matches_oracle(D, Hq, Hkv, hidden, B, S, positions, device):
    import mqk
    T = B * S
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(D), dtype=torch.int32) \
        if positions else None
    case = Case(B, S, hidden, Hq, Hkv, seed=9000 + D, head_dim=D, rows=4096 if positions else None, positions=pos)
    args = case.args(device)
    kernels = launched_kernels(lambda: mqk.fused_qkv_rope(*args))
    # (the projections: one launch of the fused kernels' plan, or each its own;
    # a plan may add a tail launch)
    assert len(kernels) >= 2 and kernels[-1] == "norm_rope_any" and "norm_rope_any" not in kernels[:-1], kernels
    out = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    idx = np.unique(np.concatenate([[0, T - 1], np.random.default_rng(D).choice(T, min(T, 24), replace=False)]))
    _check(out, case, idx, f"D={D} Hq={Hq} Hkv={Hkv} T={T}")


@pytest.mark.parametrize("D,Hq,Hkv,T,expect", [
    (256, 16, 4, 8, ["decode"]),                 # q 4096 / k, v 1024 columns: one launch for all three
    (256, 16, 4, 48, ["decode"]),
    (256, 16, 4, 600, None),
    (96, 32, 2, 8, ["decode", "tile*", "tile*"]),  # k, v 192 columns: q planned, k and v on the tiles
])
def test_any_head_dim_planned_projections(D, Hq, Hkv, T, expect, device):
    """Where the q and k / v widths are whole 128-column blocks, the three
    projections run as one launch of the fused op's plan over those blocks with q
    and k stored as projected (at decode sizes the split-K decode kernel streams
    all the weights over every CU once), then the norm + RoPE launch.  Otherwise
    each projection of whole blocks takes its own plan and the others the tile
    kernels.  Held to the oracle as above."""
    import mqk
    hidden = 4096
    pos = torch.randint(0, 4096, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = Case(T, 1, hidden, Hq, Hkv, seed=9050 + T + D, head_dim=D, rows=4096, positions=pos)
    args = case.args(device)
    kernels = launched_kernels(lambda: mqk.fused_qkv_rope(*args))
    assert kernels[-1] == "norm_rope_any" and "norm_rope_any" not in kernels[:-1], kernels
    if expect:
        got = kernels[:-1]
        assert len(got) == len(expect) and all(
            g.startswith(x[:-1]) if x.endswith("*") else g == x for g, x in zip(got, expect)), kernels
    else:
        assert 1 <= len(kernels) - 1 <= 2, kernels  # one launch, perhaps with a tail
    out = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    idx = np.unique(np.concatenate([[0, T - 1], np.random.default_rng(T).choice(T, min(T, 24), replace=False)]))
    _check(out, case, idx, f"planned D={D} Hq={Hq} Hkv={Hkv} T={T}")


def test_any_head_dim_varlen(device):
    """Varlen positions (cu_seqlens with start offsets) at head_dim 256."""
    import mqk
    D, Hq, Hkv, hidden = 256, 8, 2, 1024
    cu = torch.tensor([0, 40, 40, 130], dtype=torch.int32)
    start = torch.tensor([5, 0, 300], dtype=torch.int32)
    seq, posv = orc.varlen_positions(cu.numpy(), start.numpy())
    T = int(cu[-1])
    case = Case(1, T, hidden, Hq, Hkv, seed=9100, head_dim=D, rows=1024,
                positions=torch.from_numpy(posv.astype(np.int32)))
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    out = mqk.fused_qkv_rope_ex(x.view(T, hidden), wq, wk, wv, gq, gk, cos, sin,
                                cu_seqlens=cu.to(device), seq_pos0=start.to(device))
    torch.cuda.synchronize()
    out = [o.reshape(1, T, -1, D) for o in out]
    _check(out, case, np.arange(T), "varlen D=256")


def test_any_head_dim_refusals(device):
    """Head sizes outside the generic path raise (odd multiples of 2, above 512)."""
    import mqk
    for D in (66, 1024):
        case = Case(1, 8, 1024, 4, 2, seed=9200 + D, head_dim=D)
        with pytest.raises(mqk.MqkNativeError, match=f"head_dim {D} not supported"):
            mqk.fused_qkv_rope(*case.args(device))
            torch.cuda.synchronize()


@pytest.mark.parametrize("T,Hkv,round_weight,expect", [(8, 4, True, ["decode"]), (40, 4, True, ["decode"]),
                                                       (8, 2, False, ["gemv"] * 3)])
def test_any_head_dim_w4a16(T, Hkv, round_weight, expect, device):
    """The W4A16 front at head_dim 96: the projections into q / k / v, then the
    norm + RoPE launch, against the oracle with the same weight and projection
    rounding.  With 4 KV heads (q 1536, k / v 384 columns: whole 128-column
    blocks) one launch of the fused int4 plan, which rounds the dequantised
    weight to bf16, with q and k stored as projected; with 2 (k / v 192 columns)
    at T = 8, three column-parallel GEMMs, which keep it exact."""
    import mqk
    D, Hq, hidden = 96, 16, 1024
    pos = torch.randint(0, 2048, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = Case(T, 1, hidden, Hq, Hkv, seed=9400 + T + Hkv, head_dim=D, rows=2048, positions=pos)
    args = case.args(device)
    projs = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128, torch.bfloat16))
             for w in (case.w_q, case.w_k, case.w_v)]
    kernels = launched_kernels(lambda: mqk.fused_qkv_rope_w4a16(args[0], *projs, *args[4:]))
    assert kernels[-1] == "norm_rope_any" and "norm_rope_any" not in kernels[:-1], kernels
    assert kernels[:-1] == expect, kernels
    out = mqk.fused_qkv_rope_w4a16(args[0], *projs, *args[4:])
    torch.cuda.synchronize()
    x2 = f32(case.x).reshape(T, hidden)
    raw = [orc.round_bf16(orc.w4a16_gemm(x2, p[0].cpu().numpy(), p[1].float().cpu().numpy(), p[2].cpu().numpy(),
                                         128, np.float64, round_weight)) for p in projs]
    rows = pos.numpy()
    q = orc.qk_norm_rope(raw[0].reshape(T, Hq, D), f32(case.q_norm_w), f32(case.cos), f32(case.sin), 1, rows)
    k = orc.qk_norm_rope(raw[1].reshape(T, Hkv, D), f32(case.k_norm_w), f32(case.cos), f32(case.sin), 1, rows)
    for name, o, r in zip("qkv", out, (q, k, raw[2].reshape(T, Hkv, D))):
        o = f32(o).reshape(r.shape)
        assert np.isfinite(o).all(), name
        assert orc.max_abs(o, r) <= MAX_ABS, f"{name} max-abs {orc.max_abs(o, r)}"
        assert orc.rel_l2(o, r) <= REL_L2, f"{name} rel-L2 {orc.rel_l2(o, r)}"


def test_any_head_dim_paged_cache(device):
    """The paged-cache write at head_dim 256 (prefill, two sequences): every cache
    slot the block table maps holds the returned K / V row bit for bit; the rest
    of the (sentinel-filled) caches stays untouched."""
    import mqk
    D, Hq, Hkv, hidden, B, S, bs = 256, 8, 2, 1024, 2, 40, 16
    SENTINEL = -7
    nb = 12
    g = torch.Generator().manual_seed(9500)
    bt = torch.randperm(nb, generator=g)[: B * 3].view(B, 3).to(torch.int32)
    case = Case(B, S, hidden, Hq, Hkv, seed=9501, head_dim=D)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    kc = torch.full((nb, bs, Hkv, D), SENTINEL, dtype=torch.int16, device=device).view(torch.bfloat16)
    vc = kc.clone()
    q, k, v = mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, k_cache=kc, v_cache=vc,
                                    block_table=bt.to(device))
    torch.cuda.synchronize()
    T = B * S
    seq = np.repeat(np.arange(B), S)
    pos = np.tile(np.arange(S), B)
    slots = torch.as_tensor(orc.paged_slot(bt.numpy(), seq, pos, bs, nb), dtype=torch.int64)
    for name, cache, rows in (("k", kc, k), ("v", vc, v)):
        flat = cache.view(torch.int16).reshape(-1, Hkv, D).cpu()
        want = rows.view(torch.int16).reshape(T, Hkv, D).cpu()
        assert torch.equal(flat[slots], want), f"{name} cache rows differ from the returned rows"
        mask = torch.ones(flat.shape[0], dtype=torch.bool)
        mask[slots] = False
        assert bool((flat[mask] == SENTINEL).all()), f"{name}: a slot outside the table was written"
    _check((q, k, v), case, np.arange(T), "paged D=256")


def test_any_head_dim_input_norm(device):
    """The fused input RMSNorm at head_dim 96: the op on x equals the op on the
    oracle-normalised activations, within the acceptance bar."""
    import mqk
    D, Hq, Hkv, hidden, T = 96, 16, 4, 2048, 150
    case = Case(1, T, hidden, Hq, Hkv, seed=9600, head_dim=D, x_std=3.0)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    gam = (1 + 0.3 * torch.randn(hidden, generator=torch.Generator().manual_seed(96))).bfloat16()
    out = mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, input_norm_w=gam.to(device))
    torch.cuda.synchronize()
    xn = orc.rms_norm_hf(f32(case.x).reshape(T, hidden), f32(gam), 1e-6, round_out=True)
    normed = Case(1, T, hidden, Hq, Hkv, seed=9600, head_dim=D, x_std=3.0)
    normed.x = torch.from_numpy(xn.astype(np.float32)).reshape(1, T, hidden).bfloat16()
    _check([o.reshape(1, T, -1, D) for o in out], normed, np.arange(0, T, 7), "input norm D=96")


@pytest.mark.parametrize("T", [8, 150])
def test_any_head_dim_w4a16_input_norm(T, device):
    """The W4A16 front's fused input RMSNorm at head_dim 96 (q 1536 and k / v 384
    columns: one launch of the fused int4 plan, its per-token scales from the
    pre-pass): against the oracle on the normalised activations, the weight
    dequantised and rounded to bf16 as the int4 kernels do, the projection
    rounded to bf16.  With k / v widths that are not whole 128-column blocks it
    raises."""
    import mqk
    D, Hq, Hkv, hidden = 96, 16, 4, 1024
    pos = torch.randint(0, 2048, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = Case(T, 1, hidden, Hq, Hkv, seed=9700 + T, head_dim=D, rows=2048, positions=pos, x_std=3.0)
    args = case.args(device)
    projs = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128, torch.bfloat16))
             for w in (case.w_q, case.w_k, case.w_v)]
    gam = (1 + 0.3 * torch.randn(hidden, generator=torch.Generator().manual_seed(97))).bfloat16()
    out = mqk.fused_qkv_rope_w4a16_ex(args[0], *projs, *args[4:8], positions=args[8], input_norm_w=gam.to(device))
    torch.cuda.synchronize()
    xn = orc.rms_norm_hf(f32(case.x).reshape(T, hidden), f32(gam), 1e-6, round_out=True)
    raw = [orc.round_bf16(orc.w4a16_gemm(xn, p[0].cpu().numpy(), p[1].float().cpu().numpy(), p[2].cpu().numpy(),
                                         128, np.float64, True)) for p in projs]
    rows = pos.numpy()
    q = orc.qk_norm_rope(raw[0].reshape(T, Hq, D), f32(case.q_norm_w), f32(case.cos), f32(case.sin), 1, rows)
    k = orc.qk_norm_rope(raw[1].reshape(T, Hkv, D), f32(case.k_norm_w), f32(case.cos), f32(case.sin), 1, rows)
    for name, o, r in zip("qkv", out, (q, k, raw[2].reshape(T, Hkv, D))):
        o = f32(o).reshape(r.shape)
        assert np.isfinite(o).all(), name
        assert orc.max_abs(o, r) <= MAX_ABS, f"{name} max-abs {orc.max_abs(o, r)}"
        assert orc.rel_l2(o, r) <= REL_L2, f"{name} rel-L2 {orc.rel_l2(o, r)}"
    # k / v of 2 heads x 96 = 192 columns: the per-projection GEMMs take no input norm
    case2 = Case(T, 1, hidden, Hq, 2, seed=9800 + T, head_dim=D, rows=2048, positions=pos)
    a2 = case2.args(device)
    p2 = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128, torch.bfloat16))
          for w in (case2.w_q, case2.w_k, case2.w_v)]
    with pytest.raises(mqk.MqkNativeError, match="input RMSNorm needs"):
        mqk.fused_qkv_rope_w4a16_ex(a2[0], *p2, *a2[4:8], positions=a2[8],
                                    input_norm_w=gam.to(device))
        torch.cuda.synchronize()
