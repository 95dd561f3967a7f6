"""GPU tests of the fused input RMSNorm (mqk_fused_qkv_rope_ex_*, ext->in_gamma).

The op must compute the projections of bf16(gamma * bf16(x * rsqrt(mean(x^2) + eps)))
-- the decoder's input_layernorm (mini_qwen/model/layers/rms_norm.py:15-18, applied
at qwen3.py:58-59; oracle.rms_norm_hf(..., round_out=True)) -- without writing the
normalised activations to HBM.

* Exactness: V heads whose weight rows are one-hot copy single normalised
  activations through the MFMA unchanged, so ``v`` exposes the kernel's normalised
  x bit for bit.  It must equal the oracle's, except where the per-token scale
  (rsqrt on the GPU, 1/sqrt on the host) differs in its last bit and flips a
  bf16 rounding: at most one bf16 ulp, on under 0.5 % of the elements.
* Parity: the full op against the oracle composition (RMSNorm -> fused op) within
  the fused op's tolerance, for every kernel family (pipelined tile variants, the
  register-staged tile kernel, the split-K decode kernel, int4 weights).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

D = HEAD_DIM
EPS = 1e-6


def _gamma(hidden, seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.3 * torch.randn(hidden, generator=g)).bfloat16()


def _onehot_v(hidden, Hkv, seed):
    """w_v [Hkv*D, hidden] whose row r picks activation k_r (distinct, spread over hidden)."""
    g = torch.Generator().manual_seed(seed)
    ks = torch.randperm(hidden, generator=g)[: Hkv * D]
    w = torch.zeros(Hkv * D, hidden)
    w[torch.arange(Hkv * D), ks] = 1.0
    return w.bfloat16(), ks.numpy()


def _check_normed_copy(v, x, gamma, ks):
    want = orc.f32_to_bf16(orc.rms_norm_hf(f32(x), f32(gamma), EPS, round_out=True))[:, ks]
    got = v.reshape(v.shape[0], -1).view(torch.int16).cpu().numpy().view(np.uint16)
    ulps = orc.bf16_ulp_distance(got, want)
    assert ulps.max() <= 1, f"normalised x differs by {ulps.max()} bf16 ulps"
    assert (ulps > 0).mean() < 5e-3, f"{(ulps > 0).mean():.4f} of the normalised x differ by one ulp"


@pytest.mark.parametrize("T,tile", [(2048, 0), (300, 16), (300, 18), (300, 1), (300, 4), (37, 0), (64, 0)])
def test_input_norm_exact_copy(T, tile, device):
    import mqk
    hidden, Hq, Hkv = 1024, 10, 4  # 18 heads: whole tiles for the 3- and 2-head variants
    case = Case(1, T, hidden, Hq, Hkv, seed=500 + T + tile, x_std=3.0)
    x, wq, wk, _, gq, gk, cos, sin, _ = case.args(device)
    wv, ks = _onehot_v(hidden, Hkv, seed=T)
    gam = _gamma(hidden, seed=T + 1)
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", tile)
        _, _, v = mqk.fused_qkv_rope_ex(x, wq, wk, wv.to(device), gq, gk, cos, sin,
                                        input_norm_w=gam.to(device), input_eps=EPS)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    _check_normed_copy(v[0], case.x[0], gam, ks)


@pytest.mark.parametrize("B,S,tile", [(2, 100, 0), (1, 300, 1), (8, 1, 0)])
def test_input_norm_matches_oracle(B, S, tile, device):
    import mqk
    hidden, Hq, Hkv = 512, 4, 2
    case = Case(B, S, hidden, Hq, Hkv, seed=610 + S)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    gam = _gamma(hidden, seed=S)
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", tile)
        q, k, v = mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, input_norm_w=gam.to(device))
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    xn = orc.rms_norm_hf(f32(case.x), f32(gam), EPS, round_out=True).reshape(1, B * S, hidden)
    want = orc.fused_qkv_rope(xn, f32(case.w_q), f32(case.w_k), f32(case.w_v), f32(case.q_norm_w),
                              f32(case.k_norm_w), f32(case.cos), f32(case.sin),
                              positions=np.arange(B * S) % S)
    for got, w_ in zip((q, k, v), want):
        g_ = f32(got).reshape(w_.shape)
        assert orc.max_abs(g_, w_) <= 2e-2 and orc.rel_l2(g_, w_) <= 1e-2


def test_input_norm_decode_recompute_path(device):
    """The split-K decode kernel's recompute path re-stages x and must normalise it again."""
    import mqk
    hidden, Hq, Hkv = 1024, 8, 4
    case = Case(1, 16, hidden, Hq, Hkv, seed=700, x_std=2.0)
    x, wq, wk, _, gq, gk, cos, sin, _ = case.args(device)
    wv, ks = _onehot_v(hidden, Hkv, seed=7)
    gam = _gamma(hidden, seed=8).to(device)
    q0, k0, v0 = mqk.fused_qkv_rope_ex(x, wq, wk, wv.to(device), gq, gk, cos, sin, input_norm_w=gam)
    mqk.set_option("decode_force_recompute", 1)
    try:
        q1, k1, v1 = mqk.fused_qkv_rope_ex(x, wq, wk, wv.to(device), gq, gk, cos, sin, input_norm_w=gam)
        torch.cuda.synchronize()
    finally:
        mqk.set_option("decode_force_recompute", 0)
    assert torch.equal(q0, q1) and torch.equal(k0, k1) and torch.equal(v0, v1)
    _check_normed_copy(v1[0], case.x[0], gam.cpu(), ks)


@pytest.mark.parametrize("S,tile", [(1, 0), (16, 0), (300, 0), (300, 4), (300, 31), (300, 32), (300, 33)])
def test_input_norm_w4a16(S, tile, device):
    import mqk
    hidden, Hq, Hkv, B = 512, 4, 2, 3
    g = torch.Generator().manual_seed(S + tile)
    projs, wf = [], []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        qw, sc, qz = mqk.per_group_minmax_quantize(w, 128)
        projs.append((qw.to(device), sc.to(device), qz.to(device)))
        wf.append(mqk.dequantize(qw, sc, qz, 128).float().numpy().T)  # [N, hidden]
    x = (torch.randn(B, S, hidden, generator=g) * 2).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gam = _gamma(hidden, seed=S)
    c, s_ = mqk.rope_tables(D, max(S, 16))
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", tile)
        q, k, v = mqk.fused_qkv_rope_w4a16_ex(x.to(device), *projs, gq.to(device), gk.to(device),
                                              c.bfloat16().to(device), s_.bfloat16().to(device),
                                              input_norm_w=gam.to(device))
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", old)
    xn = orc.rms_norm_hf(f32(x), f32(gam), EPS, round_out=True).reshape(1, B * S, hidden)
    wbf = [orc.round_bf16(w_.astype(np.float32)) for w_ in wf]  # the kernels' bf16-rounded weights
    want = orc.fused_qkv_rope(xn, *wbf, f32(gq), f32(gk), f32(c.bfloat16()), f32(s_.bfloat16()),
                              positions=np.arange(B * S) % S)
    for got, w_ in zip((q, k, v), want):
        g_ = f32(got).reshape(w_.shape)
        assert orc.max_abs(g_, w_) <= 2e-2 and orc.rel_l2(g_, w_) <= 1e-2


def test_input_norm_prefill_then_decode_same_workspace(device):
    """A prefill call with the input norm writes its per-token scales into the
    stream's workspace; they must not land on the decode kernel's arrival counters
    (which open the workspace and must stay zero), or a later decode call breaks."""
    import mqk
    hidden, Hq, Hkv = 512, 4, 2
    pre = Case(1, 500, hidden, Hq, Hkv, seed=801)
    x, wq, wk, wv, gq, gk, cos, sin, _ = pre.args(device)
    mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, input_norm_w=_gamma(hidden, 1).to(device))
    dec = Case(8, 1, hidden, Hq, Hkv, seed=802)
    x, wq, wk, wv, gq, gk, cos, sin, _ = dec.args(device)
    q, k, v = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
    torch.cuda.synchronize()
    for got, want in zip((q, k, v), dec.oracle()):
        g_ = f32(got).reshape(want.shape)
        assert orc.max_abs(g_, want) <= 2e-2 and orc.rel_l2(g_, want) <= 1e-2


@pytest.mark.parametrize("T,hidden,plan", [(1536, 8192, ["row_scale", "tile"]), (1536, 4096, ["row_scale", "tile_pair"])])
def test_input_norm_pair_tiles_need_lds_room(T, hidden, plan, device):
    """With the input norm, gamma (hidden x 2 bytes) sits in the LDS beside the
    ring.  At hidden 8192 it does not fit beside the 192-row pair tiles' ring and
    exchange word (144 KiB + 16 B + 16 KiB), so the planner takes whole-head tiles
    there; at hidden 4096 the pair tiles run.  Either way the result is the
    variant-16 launch's, bit for bit."""
    from conftest import launched_kernels
    import mqk
    case = Case(1, T, hidden, 32, 8, seed=5200 + hidden)
    x, wq, wk, wv, gq, gk, cos, sin, _ = case.args(device)
    gam = _gamma(hidden, 52).to(device)
    call = lambda: mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, input_norm_w=gam)
    assert launched_kernels(call) == plan
    out = call()
    torch.cuda.synchronize()
    mqk.set_option("prefill_tile", 16)
    try:
        ref = call()
        torch.cuda.synchronize()
    finally:
        mqk.set_option("prefill_tile", 0)
    for name, a, b in zip("qkv", out, ref):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), name
