"""Seeded random calls through the default planner against the oracle.

Each case draws a Qwen3 attention shape (hidden 1024 ... 5120, 16 ... 64 query
heads), a token count from one of three ranges (decode, mid, prefill), prefill
or positions mode, and bf16 or int4 weights, and checks sampled rows of q, k
and v against the oracle at the north-star bar (max-abs <= 2e-2, rel-L2 <=
1e-2; int4 against the bf16-rounded dequantised weights).  Whatever kernels the
planner picks for the case (decode, decode blocks, split-K tiles, tiles, tile
plus tail) are exercised with their real sizes.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32
from oracle import qkv_rope_oracle as orc

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 16, 8), (2048, 16, 8), (2048, 32, 4), (2560, 32, 8), (4096, 32, 8), (4096, 32, 4),
          (5120, 40, 8), (5120, 64, 8)]


def _draw(i):
    rng = random.Random(7000 + i)
    hidden, hq, hkv = rng.choice(SHAPES)
    T = rng.choice([rng.randint(1, 64), rng.randint(65, 700), rng.randint(700, 3000)])
    int4 = rng.random() < 0.35
    prefill = rng.random() < 0.5
    idx = np.unique(np.array([0, 1, T // 3, T // 2, T - 2, T - 1] + [rng.randrange(T) for _ in range(10)]).clip(0, T - 1))
    return hidden, hq, hkv, T, int4, prefill, idx


@pytest.mark.parametrize("i", range(16))
def test_random_call_matches_oracle(i, device):
    import mqk
    hidden, hq, hkv, T, int4, prefill, idx = _draw(i)
    if prefill:
        B = max(b for b in (1, 2, 3, 4) if T % b == 0)
        case = Case(B, T // B, hidden, hq, hkv, seed=8000 + i)
    else:
        pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(i), dtype=torch.int32)
        case = Case(T, 1, hidden, hq, hkv, seed=8000 + i, rows=8192, positions=pos)
    args = case.args(device)
    label = f"hidden {hidden} heads {hq}/{hkv} T {T} {'prefill' if prefill else 'positions'} {'int4' if int4 else 'bf16'}"
    if int4:
        projs = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128,
                                                                            torch.bfloat16))
                 for w in (case.w_q, case.w_k, case.w_v)]
        out = mqk.fused_qkv_rope_w4a16(args[0], *projs, *args[4:])
        torch.cuda.synchronize()
        x2 = f32(case.x).reshape(T, hidden)[idx]
        rows = (np.arange(T) % case.S if case.positions is None else case.positions.numpy())[idx]
        ref = orc.fused_qkv_rope_w4a16(x2.reshape(1, len(idx), hidden), [p[0].cpu().numpy() for p in projs],
                                       [p[1].float().cpu().numpy() for p in projs], [p[2].cpu().numpy() for p in projs],
                                       f32(case.q_norm_w), f32(case.k_norm_w), f32(case.cos), f32(case.sin), hq, hkv,
                                       positions=rows, round_weight=True)
    else:
        out = mqk.fused_qkv_rope(*args)
        torch.cuda.synchronize()
        ref = case.oracle(token_idx=idx)
    for name, o, r in zip("qkv", out, ref):
        o = f32(o).reshape(T, -1, HEAD_DIM)[idx].reshape(r.shape)
        assert np.isfinite(o).all(), f"{label}: {name} not finite"
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        assert ma <= 2e-2 and rl <= 1e-2, f"{label}: {name} max-abs {ma:.4f} rel-L2 {rl:.2e}"
