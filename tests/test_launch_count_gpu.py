"""Kernel launches per call, counted with torch.profiler.

The reference counts device kernels of the unfused and the fused front the
same way (tests/test_fused_qkv_rope.py:287-311; 33 unfused against 6 fused,
docs/02_fused_qkv_rope.md:65-67).  Here the whole front is one launch in the
common cases; a split-off tail adds a decode launch, the fused input RMSNorm
adds its pre-pass, and mid token counts run as one decode launch covering all
their 64-row blocks ("decode_multi") or as one split-K tile launch
("tile_split").  Each case names the plan it expects, so
a change of the planner shows up here as well as in the timings.
"""
from __future__ import annotations

import pytest
import torch

from conftest import Case, launched_kernels

pytestmark = pytest.mark.gpu

HID, HQ, HKV = 4096, 32, 8  # Qwen3-8B attention shapes (BASELINE configs 2 and 3)


def _bf16_call(case, device, **ext):
    import mqk
    args = case.args(device)
    if ext:
        return lambda: mqk.fused_qkv_rope_ex(*args, **ext)
    return lambda: mqk.fused_qkv_rope(*args)


def test_prefill_c2_is_one_tile_launch(device):
    case = Case(4, 512, HID, HQ, HKV, seed=11)
    assert launched_kernels(_bf16_call(case, device)) == ["tile"]


def test_decode_c3_is_one_decode_launch(device):
    pos = torch.randint(0, 8192, (64,), generator=torch.Generator().manual_seed(3), dtype=torch.int32)
    case = Case(64, 1, HID, HQ, HKV, seed=12, rows=8192, positions=pos)
    assert launched_kernels(_bf16_call(case, device)) == ["decode"]


@pytest.mark.parametrize("T,plan", [(128, ["decode_multi"]), (256, ["decode_multi"]),
                                    (448, ["decode_multi"])])
def test_mid_t_decode_block_launches(T, plan, device):
    import mqk
    mqk.set_option("decode_cost_model", 0)  # the planner's choice is pinned elsewhere
    try:
        case = Case(1, T, HID, HQ, HKV, seed=13 + T)
        assert launched_kernels(_bf16_call(case, device)) == plan
    finally:
        mqk.set_option("decode_cost_model", 1)


@pytest.mark.parametrize("T,plan", [(128, ["decode_multi"]), (192, ["decode_multi"]), (256, ["tile_head"]),
                                    (512, ["tile_head"]), (640, ["tile_head"]), (768, ["tile_pair"]),
                                    (1024, ["tile_pair"]), (1152, ["tile"]), (1536, ["tile_pair"]),
                                    (2048, ["tile"])])
def test_default_plan_by_token_count(T, plan, device):
    """The default planner at hidden 4096 (bf16): decode blocks for a few 64-row
    blocks, one round of single-head tiles from about 200 tokens while those fit
    the CUs, one round of 128-row pair tiles beyond, whole-head tiles, then nearly
    a round of 192-row pair tiles, one tile per workgroup once the tiles fill the
    CUs."""
    case = Case(1, T, HID, HQ, HKV, seed=15 + T)
    assert launched_kernels(_bf16_call(case, device)) == plan


def test_config4_is_one_pair_tile_launch(device):
    """BASELINE config 4 (hidden 2048, 32 / 4 heads, T = 8192): 512 pair tiles of
    256 x 320 in two rounds, one launch."""
    case = Case(1, 8192, 2048, 32, 4, seed=19)
    assert launched_kernels(_bf16_call(case, device)) == ["tile_pair"]


@pytest.mark.parametrize("hidden,hq,hkv,T,plan", [
    (1024, 16, 8, 128, ["tile_head"]), (1024, 16, 8, 1024, ["tile_head"]), (1024, 16, 8, 2048, ["tile"]),
    (2048, 32, 4, 128, ["tile_head"]), (2048, 32, 4, 512, ["tile_head"]), (2048, 32, 4, 1536, ["tile"]),
    (5120, 40, 8, 512, ["tile_head"]), (5120, 40, 8, 1024, ["tile_split"])])
def test_default_plan_other_shapes(hidden, hq, hkv, T, plan, device):
    """The planner at the other Qwen3 attention shapes takes the kernel family
    measured fastest on MI355X (bf16): e.g. hidden 2048 at T = 512 as one round of
    128 x 128 single-head tiles (22.9 us against 31.9 for split-K tiles), hidden
    5120 at T = 1024 as split-K tiles (94.6 us against 117.2 for one tile per
    workgroup)."""
    case = Case(1, T, hidden, hq, hkv, seed=17 + T)
    assert launched_kernels(_bf16_call(case, device)) == plan


def test_tail_split_adds_one_decode_launch(device):
    """2080 tokens in 128 x 384 tiles: 16 full row tiles fill the 256 CUs once,
    and the last 32 rows go to the decode kernel instead of a second round."""
    import mqk
    case = Case(1, 2080, HID, HQ, HKV, seed=14)
    mqk.set_option("prefill_tile", 16)
    try:
        assert launched_kernels(_bf16_call(case, device)) == ["tile", "decode"]
        mqk.set_option("tail_split", 0)
        assert launched_kernels(_bf16_call(case, device)) == ["tile"]
    finally:
        mqk.set_option("tail_split", 1)
        mqk.set_option("prefill_tile", 0)


@pytest.mark.parametrize("B,S,plan", [(64, 1, ["row_scale", "decode"]), (4, 512, ["row_scale", "tile"]),
                                      (1, 128, ["row_scale", "decode_multi"]), (1, 256, ["row_scale", "tile_head"])])
def test_input_norm_adds_its_pre_pass(B, S, plan, device):
    g = torch.Generator().manual_seed(15)
    pos = torch.randint(0, 4096, (B * S,), generator=g, dtype=torch.int32) if S == 1 else None
    case = Case(B, S, HID, HQ, HKV, seed=15, rows=4096 if S == 1 else S, positions=pos)
    in_w = (1 + 0.1 * torch.randn(HID, generator=g)).bfloat16().to(device)
    assert launched_kernels(_bf16_call(case, device, input_norm_w=in_w)) == plan


def test_w4a16_front_is_one_launch(device):
    import mqk
    g = torch.Generator().manual_seed(16)
    hidden, Hq, Hkv, D, T = 1024, 16, 8, 128, 2048
    projs = []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w, 128, torch.float16)))
    x = torch.randn(1, T, hidden, generator=g).bfloat16().to(device)
    gq = torch.ones(D, dtype=torch.bfloat16, device=device)
    c, s = mqk.rope_tables(D, T)
    cos, sin = c.bfloat16().to(device), s.bfloat16().to(device)
    run = lambda: mqk.fused_qkv_rope_w4a16(x, *projs, gq, gq, cos, sin)
    assert launched_kernels(run) == ["tile_w4"]


@pytest.mark.parametrize("hidden,hq,hkv,T,plan", [
    (1024, 16, 8, 512, ["tile_w4_head"]), (1024, 16, 8, 1024, ["tile_w4_head"]),
    (2048, 32, 4, 1024, ["decode_multi"]),
    (5120, 40, 8, 256, ["decode"] * 4), (5120, 40, 8, 512, ["tile_w4_head"]), (5120, 40, 8, 768, ["tile_w4"])])
def test_w4a16_plan_other_shapes(hidden, hq, hkv, T, plan, device):
    """The int4 planner at the other Qwen3 attention shapes takes the kernel family
    measured fastest on MI355X: e.g. hidden 1024 at T = 512 and 1024 as one round
    of int4 single-head tiles (22.7 / 26.0 us against 34.4 / 41.7); hidden 5120,
    whose decode launches hold one 64-row block each, as four decode launches at
    T = 256 (83 us against 170), single-head tiles at T = 512 (98.7 us against
    158.4) and the tile kernel at T = 768 (174 us against 241)."""
    import mqk
    g = torch.Generator(device=device).manual_seed(18 + T)
    D = 128
    projs = []
    for h in (hq, hkv, hkv):
        N = h * D
        projs.append((torch.randint(-2**31, 2**31 - 1, (hidden // 8, N), generator=g, device=device, dtype=torch.int32),
                      (0.005 + 0.015 * torch.rand(hidden // 128, N, generator=g, device=device)).bfloat16(),
                      torch.randint(-2**31, 2**31 - 1, (hidden // 128, N // 8), generator=g, device=device,
                                    dtype=torch.int32)))
    x = torch.randn(1, T, hidden, generator=g, device=device).bfloat16()
    gq = torch.ones(D, dtype=torch.bfloat16, device=device)
    c, s = mqk.rope_tables(D, T)
    cos, sin = c.bfloat16().to(device), s.bfloat16().to(device)
    run = lambda: mqk.fused_qkv_rope_w4a16(x, *projs, gq, gq, cos, sin)
    assert launched_kernels(run) == plan
