"""fp32 callers: mqk.fused_qkv_rope on fp32 tensors against the CPU oracle.

The reference op runs on fp32 tensors too (its fp32 layer is the
CPU-runnable configuration, Qwen3-0.6B dims, B=1 x S=128): an fp32 GEMM
(fused_qkv_rope.py:167-169), then the norm and RoPE of :84-127 in fp32 with
fp32 stores.  The HIP path computes the projection on the fp32 matrix cores
and the norm and RoPE in fp32, in 32-row tiles (v_mfma_f32_32x32x2_f32) or,
when those would leave CUs idle, 16-row tiles (v_mfma_f32_16x16x4_f32).

Tolerance, against the oracle in float64 on the same fp32 inputs: every
product and partial sum of the projection rounds to fp32 (2^-24 relative), so
with K <= 4096 terms of these magnitudes the projection is within ~1e-6 of the
exact value; the norm (1/rms ~ 1.5) and RoPE scale that to a few 1e-6 at
outputs of magnitude ~4.  Bar: max-abs <= 5e-5 and rel-L2 <= 5e-6 for q, k, v
(the reference's own test allows 1e-2, test_fused_qkv_rope.py:143-144).
Against the reference's unfused fp32 composition on the CPU (all in fp32,
test_fused_qkv_rope.py:244-259) the same bar holds.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM

pytestmark = pytest.mark.gpu

MAX_ABS = 5e-5
REL_L2 = 5e-6


def _inputs(B, S, hidden, Hq, Hkv, seed, rows=None, positions=None):
    from mqk.rope import rope_tables
    g = torch.Generator().manual_seed(seed)
    D = HEAD_DIM
    x = torch.randn(B, S, hidden, generator=g)
    w_q = torch.randn(Hq * D, hidden, generator=g) * 0.02
    w_k = torch.randn(Hkv * D, hidden, generator=g) * 0.02
    w_v = torch.randn(Hkv * D, hidden, generator=g) * 0.02
    gq = 1 + 0.1 * torch.randn(D, generator=g)
    gk = 1 + 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(D, rows if rows is not None else S, 1e6)
    return [x, w_q, w_k, w_v, gq, gk, cos.float(), sin.float()], positions


def _oracle(args, positions, S):
    from oracle import qkv_rope_oracle as orc
    x = args[0].numpy()
    B, S_, H = x.shape
    T = B * S_
    rows = np.arange(T) % S if positions is None else positions.numpy().astype(np.int64)
    return orc.fused_qkv_rope(x.reshape(1, T, H), *(a.numpy() for a in args[1:]), positions=rows)


def _check(out, ref, label):
    from oracle import qkv_rope_oracle as orc
    for name, o, r in zip("qkv", out, ref):
        assert o.dtype == torch.float32, f"{label} {name}: dtype {o.dtype}"
        o = o.detach().cpu().numpy().reshape(r.shape)
        assert np.isfinite(o).all(), f"{label} {name}: non-finite values"
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        print(f"  {label} {name}: max_abs={ma:.2e} rel_l2={rl:.2e}")
        assert ma <= MAX_ABS, f"{label} {name}: max abs {ma:.3e} > {MAX_ABS}"
        assert rl <= REL_L2, f"{label} {name}: rel L2 {rl:.3e} > {REL_L2}"


@pytest.mark.parametrize("B,S,hidden,Hq,Hkv", [
    (1, 128, 1024, 16, 8),   # the reference's fp32 configuration (Qwen3-0.6B layer)
    (2, 37, 1024, 16, 8),    # rows that do not fill the 32-row tiles
    (1, 40, 4096, 32, 8),    # Qwen3-8B dims
    (1, 64, 2048, 32, 4),    # GQA 8:1
    (3, 5, 2080, 2, 1),      # hidden a multiple of 32 only
    (4, 128, 1024, 16, 8),   # enough 32-row tiles to fill the CUs (the others run 16-row tiles)
    (1, 300, 2048, 32, 4),
])
def test_f32_prefill(B, S, hidden, Hq, Hkv, device):
    import mqk
    args, _ = _inputs(B, S, hidden, Hq, Hkv, seed=300 + S)
    q, k, v = mqk.fused_qkv_rope(*(a.to(device) for a in args))
    torch.cuda.synchronize()
    assert q.shape == (B, S, Hq, HEAD_DIM) and k.shape == (B, S, Hkv, HEAD_DIM) and v.shape == k.shape
    _check((q, k, v), _oracle(args, None, S), f"f32 prefill B={B} S={S} hidden={hidden}")


def test_f32_decode_positions(device):
    """Positions mode (the decoder's decode call): 64 sequences, one token each,
    rows picked from a full 8192-row table."""
    import mqk
    g = torch.Generator().manual_seed(311)
    pos = torch.randint(0, 8192, (64,), generator=g, dtype=torch.int32)
    args, pos = _inputs(64, 1, 1024, 16, 8, seed=312, rows=8192, positions=pos)
    q, k, v = mqk.fused_qkv_rope(*(a.to(device) for a in args), positions=pos.to(device))
    torch.cuda.synchronize()
    _check((q, k, v), _oracle(args, pos, 1), "f32 decode")


def test_f32_matches_unfused_composition(device):
    """The reference's unfused fp32 composition (projections, per-head RMSNorm,
    rotate-half RoPE, all fp32 on the host) at its fp32 configuration."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    args, _ = _inputs(1, 128, 1024, 16, 8, seed=313)
    out = mqk.fused_qkv_rope(*(a.to(device) for a in args))
    torch.cuda.synchronize()
    ref = orc.unfused_composition(*(a.numpy() for a in args), dtype=np.float32)
    _check(out, ref, "f32 vs unfused fp32")


def test_f32_v_is_the_projection(device):
    """V passthrough (fused_qkv_rope.py:169, :194): v equals x @ w_v.T, here
    within fp32 accumulation of the float64 product."""
    import mqk
    args, _ = _inputs(2, 64, 1024, 16, 8, seed=314)
    _, _, v = mqk.fused_qkv_rope(*(a.to(device) for a in args))
    torch.cuda.synchronize()
    ref = args[0].double().reshape(128, 1024) @ args[3].double().T
    err = (v.double().cpu().reshape(128, -1) - ref).abs().max().item()
    assert err <= 1e-5, err


def test_f32_mixed_dtypes_rejected(device):
    import mqk
    args, _ = _inputs(1, 8, 1024, 16, 8, seed=315)
    dev = [a.to(device) for a in args]
    dev[1] = dev[1].bfloat16()
    with pytest.raises(TypeError, match="w_q must be torch.float32"):  # (fp32 x, bf16 w_q)
        mqk.fused_qkv_rope(*dev)
    dev = [a.to(device) for a in args]
    dev[6] = dev[6].bfloat16()
    with pytest.raises(TypeError, match="cos must be torch.float32"):
        mqk.fused_qkv_rope(*dev)


def test_f32_is_one_native_launch(device):
    import mqk
    from conftest import launched_kernels
    args, _ = _inputs(1, 128, 1024, 16, 8, seed=316)
    dev = [a.to(device) for a in args]
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*dev)) == ["f32"]


# ── fp16 tensors (a model loaded with dtype=float16, loader.py:12-52) ────────

@pytest.mark.parametrize("B,S,hidden,Hq,Hkv,positions", [
    (1, 128, 1024, 16, 8, False), (64, 1, 4096, 32, 8, True), (4, 128, 1024, 16, 8, False)])
def test_f16_matches_oracle(B, S, hidden, Hq, Hkv, positions, device):
    """fp16 inputs on the fp16 matrix cores (exact products), fp32 sums, norm
    and RoPE, one fp16 rounding per output: against the oracle on the same fp16
    values, within half an fp16 ulp of the output plus the fp32 summation error
    (max-abs <= 4e-3 at outputs below 8; rel-L2 <= 1e-3)."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    g = torch.Generator().manual_seed(320 + B)
    rows = 8192 if positions else S
    pos = torch.randint(0, rows, (B * S,), generator=g, dtype=torch.int32) if positions else None
    args, _ = _inputs(B, S, hidden, Hq, Hkv, seed=321 + B, rows=rows)
    args = [a.half() for a in args]
    out = mqk.fused_qkv_rope(*(a.to(device) for a in args), None if pos is None else pos.to(device))
    torch.cuda.synchronize()
    ref = _oracle([a.float() for a in args], pos, S)
    for name, o, r in zip("qkv", out, ref):
        assert o.dtype == torch.float16
        o = o.float().cpu().numpy().reshape(r.shape)
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        assert np.abs(r).max() < 8 and ma <= 4e-3 and rl <= 1e-3, f"{name}: {ma:.2e} {rl:.2e}"


def test_f32_and_f16_rejected_by_the_bf16_only_forms(device):
    """The paged and extended forms run bf16 kernels only: fp32 or fp16 inputs
    raise TypeError there, whatever the dtype of cos / sin."""
    import mqk
    args, _ = _inputs(1, 8, 1024, 16, 8, seed=322)
    for dt in (torch.float32, torch.float16):
        dev = [a.to(device).to(dt) for a in args]
        dev[6], dev[7] = dev[6].bfloat16(), dev[7].bfloat16()
        with pytest.raises(TypeError, match="x must be torch.bfloat16"):
            mqk.fused_qkv_rope_ex(*dev)
