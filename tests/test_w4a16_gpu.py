"""GPU parity of the W4A16 entry points and of the standalone QK-Norm + RoPE.

W4A16 numerics: the kernel dequantises ``(q - z) * s`` exactly in fp32 and
rounds the weight once to bf16 for the MFMA.  Two oracles bound it:
  * against the oracle GEMM on the bf16-rounded dequantised weight the only
    differences are fp32 summation order and the output's bf16 rounding:
    |out - ref| <= 2^-8 |ref| + 1e-3 * rms(ref);
  * against the exact fp32 dequant (the reference's test oracle,
    tests/test_w4a16_gemm.py:19-44) the bf16 weight rounding adds a random
    2^-9 relative error per weight: rel-L2 <= 1e-2.
The fused W4A16 front is held to the bf16 path's bar (max-abs 2e-2, rel-L2
1e-2) against norm + RoPE of the projection with the dequantised weight rounded
to bf16 (what a bf16 matrix unit consumes); against the exact fp32 dequant the
per-weight 2^-9 rounding adds up to ~1 bf16 ulp of a normalised output, so that
comparison is held to max-abs 4e-2, rel-L2 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, f32

pytestmark = pytest.mark.gpu

D = HEAD_DIM


def _quant(K, N, seed, scale_dtype=torch.bfloat16, group=128):
    import mqk
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(K, N, generator=g) * 0.02
    qw, sc, qz = mqk.per_group_minmax_quantize(w, group, scale_dtype)
    return qw, sc, qz


def _oracle_gemm(x, qw, sc, qz, group, round_w):
    from oracle import qkv_rope_oracle as orc
    w = orc.dequant(qw.numpy(), sc.float().numpy(), qz.numpy(), group)
    if round_w:
        w = orc.round_bf16(w)
    return f32(x).astype(np.float64) @ w.astype(np.float64)


def _check_gemm(out, x, qw, sc, qz, group, label):
    from oracle import qkv_rope_oracle as orc
    o = f32(out).astype(np.float64)
    tight = _oracle_gemm(x, qw, sc, qz, group, True)
    exact = _oracle_gemm(x, qw, sc, qz, group, False)
    rms = float(np.sqrt(np.mean(tight ** 2))) if tight.size else 0.0
    bound = 2.0 ** -8 * np.abs(tight) + 1e-3 * rms
    worst = float(np.max(np.abs(o - tight) - bound)) if o.size else -1.0
    rl = orc.rel_l2(o, exact)
    print(f"  {label}: worst excess={worst:.3e} rel_l2(exact)={rl:.2e}")
    assert np.isfinite(o).all()
    assert worst <= 0, f"{label}: exceeds 2^-8|ref| + 1e-3 rms by {worst}"
    assert rl <= 1e-2, f"{label}: rel L2 vs exact dequant {rl}"


@pytest.mark.parametrize("M,K,N", [(1, 128, 8), (1, 1024, 4096), (4, 1024, 4096), (16, 1024, 4096),
                                   (200, 1024, 1000), (300, 512, 264)])
def test_w4a16_gemm(M, K, N, device):
    import mqk
    qw, sc, qz = _quant(K, N, seed=M + N)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M)) ).bfloat16()
    out = mqk.w4a16_gemm(x.to(device), qw.to(device), sc.to(device), qz.to(device), 128)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    _check_gemm(out, x, qw, sc, qz, 128, f"M={M} K={K} N={N}")


def test_w4a16_gemm_fp16_scales_and_group64(device):
    import mqk
    qw, sc, qz = _quant(512, 256, seed=5, scale_dtype=torch.float16, group=64)
    x = torch.randn(33, 512, generator=torch.Generator().manual_seed(6)).bfloat16()
    out = mqk.w4a16_gemm(x.to(device), qw.to(device), sc.to(device), qz.to(device), 64)
    _check_gemm(out, x, qw, sc, qz, 64, "fp16 scales, group 64")


def test_w4a16_known_answer(device):
    """All nibbles 9, zero 8, scale 0.5 -> W = 0.5 everywhere; x = 1 -> K/2."""
    import mqk
    K, N = 256, 128
    qw = torch.full((K // 8, N), 0x99999999 - (1 << 32), dtype=torch.int32)
    qz = torch.full((K // 128, N // 8), 0x88888888 - (1 << 32), dtype=torch.int32)
    sc = torch.full((K // 128, N), 0.5, dtype=torch.bfloat16)
    x = torch.ones(3, K, dtype=torch.bfloat16)
    out = mqk.w4a16_gemm(x.to(device), qw.to(device), sc.to(device), qz.to(device), 128)
    assert torch.all(out.float().cpu() == K * 0.5)


def test_linear_w4a16_from_float_and_gptq(device):
    import mqk
    lin = torch.nn.Linear(512, 384, bias=False)
    torch.nn.init.normal_(lin.weight, std=0.02, generator=torch.Generator().manual_seed(9))
    layer = mqk.LinearW4A16.from_float(lin, 128).to(device)
    x = torch.randn(2, 7, 512, generator=torch.Generator().manual_seed(10)).bfloat16()
    y = layer(x.to(device))
    assert y.shape == (2, 7, 384)
    _check_gemm(y.reshape(14, 384), x.reshape(14, 512), layer.qweight.cpu(), layer.scales.cpu(),
                layer.qzeros.cpu(), 128, "LinearW4A16.from_float")
    # GPTQ v1 stores z - 1: from_gptq adds it back and reproduces the same layer
    from oracle import qkv_rope_oracle as orc
    z = orc.unpack_int4(layer.qzeros.cpu().numpy())
    qz_v1 = torch.from_numpy(orc.pack_int4(np.clip(z - 1, 0, 15)))
    g = mqk.LinearW4A16.from_gptq(layer.qweight, qz_v1.to(device), layer.scales, 128)
    fixed = orc.unpack_int4(g.qzeros.cpu().numpy())
    assert np.array_equal(fixed, np.where(z == 0, 1, z))


def _int4_case(B, S, hidden, Hq, Hkv, seed, scale_dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    projs = [_quant(hidden, h * D, seed + i, scale_dtype) for i, h in enumerate((Hq, Hkv, Hkv))]
    x = torch.randn(B, S, hidden, generator=g).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    return x, projs, gq, gk


def _oracle_w4a16(x, projs, gq, gk, cos, sin, Hq, Hkv, positions, round_weight=True):
    from oracle import qkv_rope_oracle as orc
    qw = [p[0].numpy() for p in projs]
    sc = [p[1].float().numpy() for p in projs]
    qz = [p[2].numpy() for p in projs]
    return orc.fused_qkv_rope_w4a16(f32(x), qw, sc, qz, f32(gq), f32(gk), f32(cos), f32(sin),
                                    Hq, Hkv, positions=positions, round_weight=round_weight)


def _check_w4(out, x, projs, gq, gk, cos, sin, Hq, Hkv, positions, label):
    from oracle import qkv_rope_oracle as orc
    for round_weight, bound in ((True, 2e-2), (False, 4e-2)):
        ref = _oracle_w4a16(x, projs, gq, gk, cos, sin, Hq, Hkv, positions, round_weight)
        for name, o, r in zip("qkv", out, ref):
            o = f32(o).reshape(r.shape)
            ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
            print(f"  {label} {name} (bf16 weight ref={round_weight}): max_abs={ma:.5f} rel_l2={rl:.2e}")
            assert ma <= bound and rl <= 1e-2, f"{label} {name}: {ma} {rl}"


@pytest.mark.parametrize("B,S,positions_mode,scale_dtype", [
    (2, 100, False, torch.bfloat16),   # prefill, tile kernel
    (1, 8, True, torch.bfloat16),      # decode kernel, int4 loader
    (1, 64, True, torch.float16),      # decode boundary, fp16 scales
    (1, 77, True, torch.bfloat16),     # ragged continuous batch, tile kernel
])
def test_fused_w4a16(B, S, positions_mode, scale_dtype, device):
    import mqk
    from oracle import qkv_rope_oracle as orc
    hidden, Hq, Hkv = 1024, 16, 8
    x, projs, gq, gk = _int4_case(B, S, hidden, Hq, Hkv, seed=S, scale_dtype=scale_dtype)
    rows = 4096 if positions_mode else S
    c, s = mqk.rope_tables(D, rows)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = None
    if positions_mode:
        pos = torch.randint(0, rows, (B * S,), generator=torch.Generator().manual_seed(S), dtype=torch.int32)
    dp = [tuple(t.to(device) for t in p) for p in projs]
    q, k, v = mqk.fused_qkv_rope_w4a16(x.to(device), *dp, gq.to(device), gk.to(device), cos.to(device),
                                       sin.to(device), None if pos is None else pos.to(device))
    torch.cuda.synchronize()
    _check_w4((q, k, v), x, projs, gq, gk, cos, sin, Hq, Hkv, None if pos is None else pos.numpy(),
              f"w4a16 B={B} S={S}")


def test_config5_w4a16_ragged_full_size(device):
    """BASELINE config 5 at full size: Qwen3-8B dims (hidden 4096, 32/8 heads), AWQ
    int4 weights with random nibbles U{0..15}, fp16 scales U(0.005, 0.02), random
    zeros; 16 packed sequences of lengths U[1, 1024] starting at positions
    U[0, 4096), read from an 8192-row table.  The tile launch and the decode-kernel
    tail launch both run (T is not a multiple of 256).  Checked against the oracle
    on 192 tokens: each sequence's first and last token plus a seeded sample."""
    import mqk
    hidden, Hq, Hkv = 4096, 32, 8
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(1, 1025, (16,), generator=g)
    starts = torch.randint(0, 4096, (16,), generator=g)
    pos = torch.cat([s + torch.arange(int(n)) for s, n in zip(starts, lens)]).to(torch.int32)
    T = int(lens.sum())
    projs = []
    for h in (Hq, Hkv, Hkv):
        N = h * D
        qw = torch.randint(-2**31, 2**31 - 1, (hidden // 8, N), generator=g, dtype=torch.int64).to(torch.int32)
        sc = (0.005 + 0.015 * torch.rand(hidden // 128, N, generator=g)).half()
        qz = torch.randint(-2**31, 2**31 - 1, (hidden // 128, N // 8), generator=g,
                           dtype=torch.int64).to(torch.int32)
        projs.append((qw, sc, qz))
    x = torch.randn(1, T, hidden, generator=g).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    c, s = mqk.rope_tables(D, 8192)
    cos, sin = c.bfloat16(), s.bfloat16()
    dp = [tuple(t.to(device) for t in p) for p in projs]
    q, k, v = mqk.fused_qkv_rope_w4a16(x.to(device), *dp, gq.to(device), gk.to(device), cos.to(device),
                                       sin.to(device), pos.to(device))
    torch.cuda.synchronize()
    assert q.shape == (1, T, Hq, D) and k.shape == (1, T, Hkv, D) and v.shape == (1, T, Hkv, D)
    ends = torch.cumsum(lens, 0)
    edge = torch.cat([ends - lens, ends - 1]).numpy()
    rest = np.random.default_rng(4).choice(T, size=160, replace=False)
    idx = np.unique(np.concatenate([edge, rest]))
    ti = torch.as_tensor(idx)
    out = tuple(t[0, ti].cpu()[None] for t in (q, k, v))
    # q / k are normalised (rms ~ 1): the absolute bar of the other tests.  v is
    # the plain projection, which with these int4 weights has rms ~ 5.5 and
    # reaches |v| ~ 30, where one bf16 ulp is 0.125: its max-abs bar is the same
    # one in units of rms(ref).
    from oracle import qkv_rope_oracle as orc
    for round_weight, bound in ((True, 2e-2), (False, 4e-2)):
        ref = _oracle_w4a16(x[:, ti], projs, gq, gk, cos, sin, Hq, Hkv, pos.numpy()[idx], round_weight)
        for name, o, r in zip("qkv", out, ref):
            o = f32(o).reshape(r.shape).astype(np.float64)
            scale = float(np.sqrt(np.mean(r ** 2))) if name == "v" else 1.0
            ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
            print(f"  C5 T={T} {name} (bf16 weight ref={round_weight}): max_abs={ma:.5f} "
                  f"(bar scale {scale:.2f}) rel_l2={rl:.2e}")
            assert np.isfinite(o).all()
            assert ma <= bound * scale and rl <= 1e-2, f"C5 {name}: {ma} {rl}"


def test_fused_w4a16_accepts_modules(device):
    import mqk
    hidden, Hq, Hkv = 512, 4, 2
    mods = []
    for h in (Hq, Hkv, Hkv):
        lin = torch.nn.Linear(hidden, h * D, bias=False)
        mods.append(mqk.LinearW4A16.from_float(lin, 128).to(device))
    x = torch.randn(1, 5, hidden).bfloat16().to(device)
    g = torch.ones(D, dtype=torch.bfloat16, device=device)
    c, s = mqk.rope_tables(D, 5)
    a = mqk.fused_qkv_rope_w4a16(x, *mods, g, g, c.bfloat16().to(device), s.bfloat16().to(device))
    b = mqk.fused_qkv_rope_w4a16(x, *[(m.qweight, m.scales, m.qzeros) for m in mods], g, g,
                                 c.bfloat16().to(device), s.bfloat16().to(device))
    for u, w in zip(a, b):
        assert torch.equal(u, w)


# ── standalone QK-Norm + RoPE (fused_qkv_rope.py:46-127) ─────────────────────

@pytest.mark.parametrize("B,S,Hq,Hkv,positions_mode", [(2, 33, 16, 8, False), (1, 9, 32, 8, True),
                                                       (3, 1, 4, 4, True)])
def test_qk_norm_rope(B, S, Hq, Hkv, positions_mode, device):
    import mqk
    from oracle import qkv_rope_oracle as orc
    g = torch.Generator().manual_seed(B * 100 + S)
    q_raw = (torch.randn(B, S, Hq, D, generator=g) * 3).bfloat16()
    k_raw = (torch.randn(B, S, Hkv, D, generator=g) * 3).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    rows = 2048 if positions_mode else S
    c, s = mqk.rope_tables(D, rows)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = torch.randint(0, rows, (B * S,), generator=g, dtype=torch.int32) if positions_mode else None
    qo, ko = mqk.qk_norm_rope(q_raw.to(device), k_raw.to(device), gq.to(device), gk.to(device),
                              cos.to(device), sin.to(device), None if pos is None else pos.to(device))
    torch.cuda.synchronize()
    pn = None if pos is None else pos.numpy()
    for name, o, raw, gam, H in (("q", qo, q_raw, gq, Hq), ("k", ko, k_raw, gk, Hkv)):
        r = orc.qk_norm_rope(f32(raw).reshape(B * S, H, D), f32(gam), f32(cos), f32(sin), S, pn)
        o = f32(o).reshape(r.shape)
        # one bf16 rounding of the output plus fp32 arithmetic
        excess = np.abs(o - r) - (2.0 ** -8 * np.abs(r) + 1e-5)
        assert float(excess.max()) <= 0, f"{name}: {float(excess.max())}"


def test_qk_norm_rope_matches_fused(device):
    """Norm + RoPE of a bf16-rounded projection == the standalone kernel on it."""
    import mqk
    from conftest import Case
    case = Case(1, 16, 512, 4, 2, seed=21)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    q_raw = (x.reshape(16, 512) @ wq.T).reshape(1, 16, 4, D)
    k_raw = (x.reshape(16, 512) @ wk.T).reshape(1, 16, 2, D)
    qo, ko = mqk.qk_norm_rope(q_raw, k_raw, gq, gk, cos, sin)
    qf, kf, _ = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
    # differ only by the bf16 rounding of the projection (|out| <= ~8 -> <= 0.04)
    assert (qo.float() - qf.float()).abs().max().item() <= 4e-2
    assert (ko.float() - kf.float()).abs().max().item() <= 4e-2


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 30, 31, 32])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
def test_fused_w4a16_tile_variants(variant, scale_dtype, device):
    """Every int4 tile variant on a ragged-length shape (T = 600: row tail), 24 heads,
    two quantisation groups per 256 k (group 128)."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    B, S, hidden, Hq, Hkv = 1, 600, 1024, 16, 4
    x, projs, gq, gk = _int4_case(B, S, hidden, Hq, Hkv, seed=900 + variant, scale_dtype=scale_dtype)
    c, s = mqk.rope_tables(D, 4096)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = torch.randint(0, 4096, (S,), generator=torch.Generator().manual_seed(variant), dtype=torch.int32)
    dp = [tuple(t.to(device) for t in p) for p in projs]
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", variant)
        q, k, v = mqk.fused_qkv_rope_w4a16(x.to(device), *dp, gq.to(device), gk.to(device), cos.to(device),
                                           sin.to(device), pos.to(device))
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    _check_w4((q, k, v), x, projs, gq, gk, cos, sin, Hq, Hkv, pos.numpy(), f"w4a16 tile {variant}")
