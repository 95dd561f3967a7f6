"""GPU parity of the W4A16 entry points and of the standalone QK-Norm + RoPE.

W4A16 numerics: the kernel dequantises ``(q - z) * s`` exactly in fp32 and
rounds the weight once to bf16 for the MFMA.  Two oracles bound it:
  * against the oracle GEMM on the bf16-rounded dequantised weight the only
    differences are fp32 summation order and the output's bf16 rounding:
    |out - ref| <= 2^-8 |ref| + 1e-3 * rms(ref);
  * against the exact fp32 dequant (the reference's test oracle,
    tests/test_w4a16_gemm.py:19-44) the bf16 weight rounding adds a random
    error of at most 2^-8 relative per weight: rel-L2 <= 1e-2.
The fused W4A16 front is held to the bf16 path's bar (max-abs 2e-2, rel-L2
1e-2) against norm + RoPE of the projection with the dequantised weight rounded
to bf16 (what a bf16 matrix unit consumes); against the exact fp32 dequant the
per-weight rounding (at most 2^-8 relative) adds up to ~1 bf16 ulp of a normalised output, so that
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


def _check_gemm(out, x, qw, sc, qz, group, label, exact_weight=None):
    """exact_weight (default: M <= 16, the column-parallel kernel's range): the
    kernel multiplies the exact fp32 weight (q - z) * s, so it is held to the
    exact oracle within the output's rounding plus the fp32 summation bound,
    |out - ref| <= 2^-8 |ref| + K * 2^-24 * sum_k |x_k w_k|; otherwise (MFMA
    kernels, bf16 weight) to the bf16-weight oracle as described above."""
    from oracle import qkv_rope_oracle as orc
    o = f32(out).astype(np.float64)
    if exact_weight is None:
        exact_weight = o.shape[0] <= 16
    tight = _oracle_gemm(x, qw, sc, qz, group, not exact_weight)
    exact = _oracle_gemm(x, qw, sc, qz, group, False)
    rms = float(np.sqrt(np.mean(tight ** 2))) if tight.size else 0.0
    if exact_weight:
        w = orc.dequant(qw.numpy(), sc.float().numpy(), qz.numpy(), group).astype(np.float64)
        absdot = np.abs(f32(x).astype(np.float64)) @ np.abs(w)
        bound = 2.0 ** -8 * np.abs(tight) + x.shape[1] * 2.0 ** -24 * absdot
    else:
        bound = 2.0 ** -8 * np.abs(tight) + 1e-3 * rms
    worst = float(np.max(np.abs(o - tight) - bound)) if o.size else -1.0
    rl = orc.rel_l2(o, exact)
    print(f"  {label}: worst excess={worst:.3e} rel_l2(exact)={rl:.2e}")
    assert np.isfinite(o).all()
    assert worst <= 0, f"{label}: exceeds the bound by {worst}"
    assert rl <= 1e-2, f"{label}: rel L2 vs exact dequant {rl}"


@pytest.mark.parametrize("M,K,N", [(1, 128, 8), (1, 1024, 4096), (4, 1024, 4096), (8, 1024, 4096),
                                   (16, 1024, 4096), (64, 1024, 4096), (65, 1024, 4096), (300, 4096, 1024),
                                   (1024, 1024, 4096), (200, 1024, 1000), (300, 512, 264)])
def test_w4a16_gemm(M, K, N, device):
    import mqk
    qw, sc, qz = _quant(K, N, seed=M + N)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M)) ).bfloat16()
    out = mqk.w4a16_gemm(x.to(device), qw.to(device), sc.to(device), qz.to(device), 128)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    _check_gemm(out, x, qw, sc, qz, 128, f"M={M} K={K} N={N}")


@pytest.mark.parametrize("M", [1, 16, 200])
@pytest.mark.usefixtures("no_head_tiles")
def test_w4a16_gemm_decode_path_matches_tile(M, device):
    """Small M runs on the split-K decode kernel (the reference's decode GEMV
    regime, w4a16_gemm.py:110-189): it must agree with the tile kernel (forced
    with decode_max_t = 0 and decode_blocks = 0) within the fp32 summation-order
    bound, and launch one decode kernel, no tile kernel."""
    import mqk
    from conftest import launched_kernels
    K, N = 1024, 4096
    qw, sc, qz = (t.to(device) for t in _quant(K, N, seed=40 + M))
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(41 + M)).bfloat16().to(device)
    run = lambda: mqk.w4a16_gemm(x, qw, sc, qz, 128)
    mqk.set_option("gemv_max_m", 0)  # (M <= 16 otherwise runs the column-parallel kernel)
    try:
        assert launched_kernels(run) == (["decode"] if M <= 64 else ["decode_multi"])
        dec = run()
        mqk.set_option("decode_max_t", 0)
        mqk.set_option("decode_blocks", 0)
        tile = run()
        torch.cuda.synchronize()
        assert launched_kernels(run) in (["tile_w4"], ["tile_reg"])
    finally:
        mqk.set_option("decode_max_t", 64)
        mqk.set_option("decode_blocks", 16)
        mqk.set_option("gemv_max_m", 16)
    a, b = dec.float(), tile.float()
    assert float((a - b).abs().max()) <= float(2.0 ** -7 * b.abs().max() + 1e-3)
    _check_gemm(dec.cpu(), x.cpu(), qw.cpu(), sc.cpu(), qz.cpu(), 128, f"decode path M={M}", exact_weight=False)


@pytest.mark.parametrize("M,K,N,scale_dtype", [
    (1, 1024, 4096, torch.bfloat16), (4, 1024, 4096, torch.float16), (8, 1024, 4096, torch.bfloat16),
    (16, 1024, 4096, torch.float16), (3, 4096, 1000, torch.bfloat16), (16, 2048, 8, torch.bfloat16),
    (5, 128, 264, torch.float16), (2, 12288, 1024, torch.bfloat16)])
def test_w4a16_gemv_small_m(M, K, N, scale_dtype, device):
    """M <= 16 (the reference's decode GEMV regime, w4a16_gemm.py:110-189, and its
    published shapes M in {1, 4, 8, 16}, K = 1024, N = 4096): one launch of the
    column-parallel kernel, any N % 8 == 0, exact fp32 dequantisation and
    accumulation, held to the exact oracle; within the MFMA paths' bound of the
    split-K decode kernel's result where that kernel runs (N % 128 == 0)."""
    import mqk
    from conftest import launched_kernels
    qw, sc, qz = _quant(K, N, seed=M + K + N, scale_dtype=scale_dtype)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M + 1)).bfloat16()
    d = [t.to(device) for t in (x, qw, sc, qz)]
    run = lambda: mqk.w4a16_gemm(*d, 128)
    assert launched_kernels(run) == ["gemv"]
    out = run()
    torch.cuda.synchronize()
    _check_gemm(out, x, qw, sc, qz, 128, f"gemv M={M} K={K} N={N}", exact_weight=True)
    if N % 128 == 0:
        mqk.set_option("gemv_max_m", 0)
        try:
            dec = run()
        finally:
            mqk.set_option("gemv_max_m", 16)
        a, b = out.float(), dec.float()
        assert float((a - b).abs().max()) <= float(2.0 ** -7 * b.abs().max() + 1e-3)


def test_w4a16_gemv_unaligned_operands(device):
    """Operands that are not 16-byte aligned (views at odd element offsets) take
    the same kernel: it reads the packed weights, scales and zeros with scalar loads."""
    import mqk
    M, K, N = 4, 512, 264
    qw, sc, qz = _quant(K, N, seed=77)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(78)).bfloat16()
    def off(t):  # same values, storage offset of one element
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=device)
        v = buf[1:].view(t.shape)
        v.copy_(t.to(device))
        return v
    out = mqk.w4a16_gemm(x.to(device), off(qw), off(sc), off(qz), 128)
    _check_gemm(out, x, qw, sc, qz, 128, "gemv unaligned weights", exact_weight=True)


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


@pytest.mark.parametrize("S,hidden,Hq,Hkv,plan", [
    (256, 5120, 40, 8, ["decode"] * 4), (512, 5120, 40, 8, ["tile_w4_head"]), (768, 5120, 40, 8, ["tile_w4"]),
    (1024, 1024, 16, 8, ["tile_w4_head"]), (512, 1024, 16, 8, ["tile_w4_head"]), (640, 2048, 32, 4, ["tile_w4_head"])])
def test_fused_w4a16_default_plan_other_shapes(S, hidden, Hq, Hkv, plan, device):
    """The int4 planner's choices at the other Qwen3 attention shapes, with
    decode-style positions, against the oracle."""
    import mqk
    from conftest import launched_kernels
    x, projs, gq, gk = _int4_case(1, S, hidden, Hq, Hkv, seed=S + hidden)
    c, s = mqk.rope_tables(D, 8192)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = torch.randint(0, 8192, (S,), generator=torch.Generator().manual_seed(S + 1), dtype=torch.int32)
    dp = [tuple(t.to(device) for t in p) for p in projs]
    args = (x.to(device), *dp, gq.to(device), gk.to(device), cos.to(device), sin.to(device), pos.to(device))
    assert launched_kernels(lambda: mqk.fused_qkv_rope_w4a16(*args)) == plan
    out = mqk.fused_qkv_rope_w4a16(*args)
    torch.cuda.synchronize()
    _check_w4(out, x, projs, gq, gk, cos, sin, Hq, Hkv, pos.numpy(), f"w4a16 default plan S={S} hidden={hidden}")


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
    from oracle import qkv_rope_oracle as orc
    Ws = [orc.dequant(qw.numpy(), sc.float().numpy(), qz.numpy(), 128) for qw, sc, qz in projs]
    _check_w4_bounds(out, f32(x[0, ti]), Ws, gq, gk, cos, sin, Hq, Hkv, pos.numpy()[idx], f"C5 T={T}")


def _check_w4_bounds(out, x2d, Ws, gq, gk, cos, sin, Hq, Hkv, rows, label):
    """The W4A16 front against two oracles, with bounds derived from the data.

    The kernel computes p' = sum_k x_k * bf16(w_k) in fp32 (w = (q - z) * s is
    exact in fp32), then norm + RoPE in fp32 and one bf16 rounding of the output.
    bf16 has 8 significand bits, so a rounding is off by at most 2^-8 relative.
    Per output column i, with A_i = sum_k |x_k w_ki| and Q_i = sqrt(sum_k (x_k w_ki)^2):
      * fp32 summation: |p'_i - p_bw_i| <= 6 sqrt(K) 2^-24 A_i, p_bw = the
        projection with bf16-rounded weights (the probabilistic rounding-error
        bound of Higham and Mary, SIAM J. Sci. Comput. 41(5), 2019, with
        lambda = 6; the worst-case K 2^-24 A_i exceeds half a bf16 ulp almost
        everywhere and would leave the ulp check below empty);
      * weight rounding: p_bw_i - p_i = sum_k x_k w_ki d_k, d_k independent and
        uniform in [-2^-8, 2^-8] (variance 2^-16 / 3): six standard deviations
        bound it, e_i = 6 * 2^-8 / sqrt(3) * Q_i.
    Checks:
      V  vs bf16(p_bw): at most 1 bf16 ulp wherever the summation bound is under
         half an ulp (everywhere but near-cancelling columns, which are counted);
      V  vs p (exact dequant): |v - p| <= E_i + 2^-8 (|p| + E_i), E_i = e_i + 6 sqrt(K) 2^-24 A_i;
      Q/K vs both oracles: the acceptance bar, max-abs 2e-2, rel-L2 1e-2;
      Q/K vs the exact dequant, per head h: the map p -> p / rms(p) moves by at
         most 2 sqrt(D) |dp|_2 / |p|_2 (2-norms over the head's 128 values); times
         max|gamma| and the RoPE pair gain max sqrt(cos^2 + sin^2) of the bf16
         tables, plus the output rounding 2^-8 |ref| and 1e-5 of fp32 epilogue
         arithmetic; and rel-L2 <= 1e-2.
    """
    from oracle import qkv_rope_oracle as orc
    T = x2d.shape[0]
    x = x2d.astype(np.float64)
    K = x.shape[1]
    refs_bw = orc.fused_qkv_rope(x.reshape(1, T, K), *[orc.round_bf16(W).T for W in Ws], f32(gq), f32(gk),
                                 f32(cos), f32(sin), positions=rows)
    refs_ex = orc.fused_qkv_rope(x.reshape(1, T, K), *[W.T for W in Ws], f32(gq), f32(gk), f32(cos),
                                 f32(sin), positions=rows)
    c, s_ = f32(cos)[rows].astype(np.float64), f32(sin)[rows].astype(np.float64)
    rope_gain = float(np.sqrt(c ** 2 + s_ ** 2).max())
    for i, (name, H, gam) in enumerate((("q", Hq, gq), ("k", Hkv, gk), ("v", Hkv, None))):
        W = Ws[i].astype(np.float64)
        o = f32(out[i]).reshape(T, H * D).astype(np.float64)
        A = np.abs(x) @ np.abs(W)
        e = 6 * 2.0 ** -8 / np.sqrt(3) * np.sqrt((x * x) @ (W * W))
        summ = 6 * np.sqrt(K) * 2.0 ** -24 * A
        E = e + summ
        r_bw = refs_bw[i].reshape(T, H * D)
        r_ex = refs_ex[i].reshape(T, H * D)
        if name == "v":
            rb = orc.f32_to_bf16(r_bw)
            ob = orc.f32_to_bf16(o)
            ulps = orc.bf16_ulp_distance(ob, rb)
            half_ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(r_bw), 1e-30))) - 8)
            clean = summ < half_ulp
            bound = E + 2.0 ** -8 * (np.abs(r_ex) + E)
            excess = float((np.abs(o - r_ex) - bound).max())
            print(f"  {label} v: max ulps vs bf16(bw ref)={int(ulps[clean].max())}, all elements "
                  f"{int(ulps.max())} "
                  f"({int((~clean).sum())} near-cancelling of {clean.size}); "
                  f"max |v - exact|={orc.max_abs(o, r_ex):.4f}, worst excess over bound={excess:.4f}")
            assert int(ulps[clean].max()) <= 1, f"{label} v: more than 1 bf16 ulp"
            assert excess <= 0, f"{label} v: exceeds the exact-dequant bound by {excess}"
        else:
            ma, rl = orc.max_abs(o, r_bw), orc.rel_l2(o, r_bw)
            assert ma <= 2e-2 and rl <= 1e-2, f"{label} {name} vs bf16-weight oracle: {ma} {rl}"
            p = (x @ W).reshape(T, H, D)
            En = np.linalg.norm(E.reshape(T, H, D), axis=-1)
            pn = np.linalg.norm(p, axis=-1)
            head_bound = float(np.abs(f32(gam)).max()) * rope_gain * 2 * np.sqrt(D) * En / pn
            bound = head_bound[..., None] + 2.0 ** -8 * np.abs(r_ex.reshape(T, H, D)) + 1e-5
            err = np.abs(o - r_ex).reshape(T, H, D)
            excess = float((err - bound).max())
            rl_ex = orc.rel_l2(o, r_ex)
            print(f"  {label} {name}: vs bf16-weight ref max_abs={ma:.4f} rel_l2={rl:.2e}; vs exact "
                  f"max_abs={float(err.max()):.4f} (bound median {float(np.median(bound)):.3f}) rel_l2={rl_ex:.2e}")
            assert excess <= 0 and rl_ex <= 1e-2, f"{label} {name} vs exact dequant: {excess} {rl_ex}"
            assert float(err.max()) <= 2e-2, f"{label} {name} vs exact dequant: max-abs {float(err.max())}"


def _awq_pack(vals: np.ndarray) -> np.ndarray:
    """[R, N] values 0..15 -> AutoAWQ words [R, N/8]: nibble i holds column 8j + (0,2,4,6,1,3,5,7)[i]
    (written here from the order map, independently of the repacker under test)."""
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    v = vals.astype(np.uint32).reshape(vals.shape[0], -1, 8)
    out = np.zeros(v.shape[:2], dtype=np.uint32)
    for i, c in enumerate(order):
        out |= v[:, :, c] << np.uint32(4 * i)
    return out.view(np.int32)


def test_autoawq_checkpoint_c5_dims(device):
    """An AutoAWQ checkpoint (qweight [K, N/8] and qzeros [K/g, N/8] packed along N
    in AWQ nibble order, fp16 scales) at Qwen3-8B dims goes through
    LinearW4A16.from_autoawq into the fused W4A16 front; the oracle reads the AWQ
    words directly (dequant_awq).  A ragged continuous batch in positions mode,
    as BASELINE config 5, checked on every sequence's first and last token plus
    a seeded sample."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    hidden, Hq, Hkv, g = 4096, 32, 8, 128
    rng = np.random.default_rng(31)
    lens = rng.integers(1, 257, 8)
    starts = rng.integers(0, 4096, 8)
    pos = np.concatenate([st + np.arange(n) for st, n in zip(starts, lens)]).astype(np.int32)
    T = int(lens.sum())
    mods, Ws = [], []
    for h in (Hq, Hkv, Hkv):
        N = h * D
        qw = _awq_pack(rng.integers(0, 16, (hidden, N)))
        qz = _awq_pack(rng.integers(0, 16, (hidden // g, N)))
        sc = rng.uniform(0.005, 0.02, (hidden // g, N)).astype(np.float16)
        mods.append(mqk.LinearW4A16.from_autoawq(torch.from_numpy(qw).to(device), torch.from_numpy(qz).to(device),
                                                 torch.from_numpy(sc).to(device), g))
        Ws.append(orc.dequant_awq(qw, qz, sc.astype(np.float32), g))
    tg = torch.Generator().manual_seed(31)
    x = torch.randn(1, T, hidden, generator=tg).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=tg)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=tg)).bfloat16()
    c, s = mqk.rope_tables(D, 8192)
    cos, sin = c.bfloat16(), s.bfloat16()
    q, k, v = mqk.fused_qkv_rope_w4a16(x.to(device), *mods, gq.to(device), gk.to(device), cos.to(device),
                                       sin.to(device), torch.from_numpy(pos).to(device))
    torch.cuda.synchronize()
    ends = np.cumsum(lens)
    idx = np.unique(np.concatenate([ends - lens, ends - 1, rng.choice(T, size=64, replace=False)]))
    ti = torch.as_tensor(idx)
    out = tuple(t[0, ti].cpu() for t in (q, k, v))
    _check_w4_bounds(out, f32(x[0, ti]), Ws, gq, gk, cos, sin, Hq, Hkv, pos[idx], f"AutoAWQ T={T}")


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


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 30, 31, 32, 33, 34, 35])
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


@pytest.mark.parametrize("M,K,N", [(300, 1024, 1000), (200, 512, 264), (1024, 2048, 4088)])
def test_w4a16_gemm_partial_last_tile_pipelined(M, K, N, device):
    """N not a multiple of 128: the pipelined int4 tile kernel runs the partial last
    tile (its columns past N re-read in-range chunks and are never stored, the zeros
    come with 4-byte loads), not the register-staged fallback."""
    import mqk
    from conftest import launched_kernels
    qw, sc, qz = _quant(K, N, seed=M + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).bfloat16()
    d = [t.to(device) for t in (x, qw, sc, qz)]
    run = lambda: mqk.w4a16_gemm(*d, 128)
    assert launched_kernels(run) in (["tile_w4"], ["tile_w4_head"])
    out = run()
    torch.cuda.synchronize()
    _check_gemm(out, x, qw, sc, qz, 128, f"partial tile M={M} K={K} N={N}")
