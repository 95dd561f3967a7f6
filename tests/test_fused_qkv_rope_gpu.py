"""GPU parity of mqk.fused_qkv_rope against the CPU oracle.

Mirrors the reference's acceptance tests (tests/test_fused_qkv_rope.py:112-223:
prefill correctness, V passthrough, decode mode) with the gaps noted there
closed: every input is seeded, the QK-norm gammas are random (1 + N(0, 0.1)) so
a swapped or skipped gamma fails, and both max-abs and rel-L2 are checked.

Tolerance (north-star acceptance bar), against the oracle's exact projection
followed by norm + RoPE in float64 (the "fp32 composition"):
max|out - ref| <= 2e-2  and  ||out - ref|| / ||ref|| <= 1e-2, for q, k and v.

The reference's own numerics (projection rounded to bf16 before the norm,
fused_qkv_rope.py:167-169) are a second, independent approximation of the same
composition: that rounding alone moves a normalised output by up to one bf16
ulp of the projection (2^-8 relative), i.e. ~0.016-0.03 at |out| in [4, 8).
Against that variant the bound is the sum of the two implementations' errors,
max-abs <= 4e-2 (rel-L2 stays <= 1e-2).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import HEAD_DIM, Case, f32

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-2


def _run(case: Case, device, **kw):
    import mqk
    return mqk.fused_qkv_rope(*case.args(device), **kw)


def _check(out, ref, label, max_abs=MAX_ABS):
    from oracle import qkv_rope_oracle as orc
    names = "qkv" if len(out) == 3 else ("qk" if len(out) == 2 else "v")
    for name, o, r in zip(names, out, ref):
        o = f32(o).reshape(r.shape)
        assert np.isfinite(o).all(), f"{label}: {name} has non-finite values"
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        print(f"  {label} {name}: max_abs={ma:.5f} rel_l2={rl:.2e}")
        assert ma <= max_abs, f"{label} {name}: max abs {ma:.5f} > {max_abs}"
        assert rl <= REL_L2, f"{label} {name}: rel L2 {rl:.3e} > {REL_L2}"


# ── reference acceptance shapes (test_fused_qkv_rope.py:112-116) ─────────────

@pytest.mark.parametrize("B,S,hidden,Hq,Hkv", [
    (1, 32, 1024, 16, 8),
    (2, 64, 1024, 16, 8),
    (4, 128, 1024, 16, 8),
])
def test_prefill_correctness(B, S, hidden, Hq, Hkv, device):
    case = Case(B, S, hidden, Hq, Hkv, seed=100 + B)
    q, k, v = _run(case, device)
    torch.cuda.synchronize()
    assert q.shape == (B, S, Hq, HEAD_DIM) and q.is_contiguous()
    assert k.shape == (B, S, Hkv, HEAD_DIM) and k.is_contiguous()
    assert v.shape == (B, S, Hkv, HEAD_DIM) and v.is_contiguous()
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16
    _check((q, k, v), case.oracle(), f"B={B} S={S}")
    _check((q, k, v), case.oracle(round_projection=True), f"B={B} S={S} (bf16-rounded GEMM ref)",
           max_abs=2 * MAX_ABS)


def test_reference_gamma_ones_shape(device):
    """The reference's own inputs (unit gammas, table of S+1 rows) at its perf shape."""
    case = Case(4, 512, 1024, 16, 8, seed=7, gamma_ones=True, rows=513)
    q, k, v = _run(case, device)
    _check((q, k, v), case.oracle(), "B=4 S=512 gamma=1")


def test_v_passthrough(device):
    """V is the plain projection.  The reference demands bit-equality with torch's
    own GEMM (test_fused_qkv_rope.py:147-165), which an independent MFMA kernel
    cannot reproduce.  Restated: v equals the correctly rounded exact projection
    except where the fp32 accumulation error can move it across a bf16 rounding
    boundary, and never differs by more than that error bound plus one ulp:
      |v - bf16(exact)| <= ulp(exact) + K * 2^-24 * sum_k |x_k w_k|."""
    from oracle import qkv_rope_oracle as orc
    case = Case(2, 64, 1024, 16, 8, seed=3)
    _, _, v = _run(case, device)
    ref = case.oracle()[2]
    v_f = f32(v).reshape(ref.shape).astype(np.float64)
    ref_bf = orc.round_bf16(ref.astype(np.float32)).astype(np.float64)
    x2 = np.abs(f32(case.x).reshape(-1, case.hidden)).astype(np.float64)
    absdot = (x2 @ np.abs(f32(case.w_v)).astype(np.float64).T).reshape(ref.shape)
    ulp = np.maximum(np.abs(ref_bf), 2.0 ** -126) * 2.0 ** -7
    bound = ulp + case.hidden * 2.0 ** -24 * absdot
    exact = np.mean(v_f == ref_bf)
    print(f"  V exact-match fraction={exact:.5f}, max excess={np.max(np.abs(v_f - ref_bf) - bound):.3g}")
    assert np.all(np.abs(v_f - ref_bf) <= bound)
    assert exact > 0.99


@pytest.mark.parametrize("B", [1, 4, 8])
def test_decode_mode_preindexed(B, device):
    """Decoder convention (attention.py:128-135): cos/sin [B, D] pre-indexed by the
    sequence positions, positions = arange(B)."""
    from mqk.rope import rope_tables
    g = torch.Generator().manual_seed(200 + B)
    case = Case(B, 1, 1024, 16, 8, seed=200 + B, positions=torch.arange(B, dtype=torch.int32))
    pos_vals = torch.randint(0, 2048, (B,), generator=g)
    cos_full, sin_full = rope_tables(HEAD_DIM, 2048)
    case.cos = cos_full[pos_vals].bfloat16()
    case.sin = sin_full[pos_vals].bfloat16()
    q, k, v = _run(case, device)
    assert q.shape == (B, 1, 16, HEAD_DIM) and k.shape == (B, 1, 8, HEAD_DIM)
    _check((q, k, v), case.oracle(), f"decode B={B}")


@pytest.mark.parametrize("B", [1, 7, 64])
def test_decode_mode_full_table(B, device):
    """Positions index a full [8192, D] table directly (BASELINE config 3 style)."""
    g = torch.Generator().manual_seed(300 + B)
    pos = torch.randint(0, 8192, (B,), generator=g, dtype=torch.int64).to(torch.int32)
    case = Case(B, 1, 4096, 32, 8, seed=300 + B, rows=8192, positions=pos)
    q, k, v = _run(case, device)
    _check((q, k, v), case.oracle(), f"decode full-table B={B}")


@pytest.mark.parametrize("blocks", [16, 0])
@pytest.mark.parametrize("T", [63, 64, 65, 129, 200])
def test_tile_boundaries(T, blocks, device):
    """Token counts around the decode/tile-kernel switch and the 128-row tile,
    with 64-row decode blocks allowed (the default) and off (tile kernel)."""
    import mqk
    case = Case(1, T, 2048, 16, 4, seed=400 + T)
    old = mqk.get_option("decode_blocks")
    try:
        mqk.set_option("decode_blocks", blocks)
        q, k, v = _run(case, device)
    finally:
        mqk.set_option("decode_blocks", old)
    _check((q, k, v), case.oracle(), f"T={T} decode_blocks={blocks}")


def test_decode_and_tile_paths_agree(device):
    """The split-K decode kernel and the tile kernel compute the same op."""
    import mqk
    case = Case(1, 48, 4096, 32, 8, seed=11, rows=4096,
                positions=torch.randint(0, 4096, (48,), generator=torch.Generator().manual_seed(5),
                                        dtype=torch.int64).to(torch.int32))
    a = _run(case, device)
    old = mqk.get_option("decode_max_t")
    try:
        mqk.set_option("decode_max_t", 0)
        b = _run(case, device)
    finally:
        mqk.set_option("decode_max_t", old)
    for x, y in zip(a, b):
        d = (x.float() - y.float()).abs().max().item()
        assert d <= 2 * MAX_ABS, d
    _check(a, case.oracle(), "decode path")
    _check(b, case.oracle(), "tile path")


@pytest.mark.parametrize("splits,recompute", [(0, 0), (0, 1), (4, 0), (8, 0), (16, 0), (16, 1), (7, 0)])
def test_decode_variants(splits, recompute, device):
    """Split counts of the decode kernel, and its recompute path (taken when a
    split runs on an unexpected XCD), which must give bit-identical results."""
    import mqk
    g = torch.Generator().manual_seed(600 + splits)
    pos = torch.randint(0, 8192, (64,), generator=g).to(torch.int32)
    case = Case(64, 1, 4096, 32, 8, seed=600 + splits, rows=8192, positions=pos)
    names = ("decode_splits", "decode_force_recompute")
    old = [mqk.get_option(n) for n in names]
    try:
        mqk.set_option("decode_splits", splits)
        ref_path = _run(case, device)
        mqk.set_option("decode_force_recompute", recompute)
        out = _run(case, device)
        again = _run(case, device)
    finally:
        for n, val in zip(names, old):
            mqk.set_option(n, val)
    for a, b, c in zip(out, again, ref_path):
        assert torch.equal(a, b)
        assert torch.equal(a, c)
    _check(out, case.oracle(), f"decode splits={splits} recompute={recompute}")


def test_decode_repeatable(device):
    """Arrival counters are reset by each call: repeated calls give identical bits."""
    case = Case(32, 1, 4096, 32, 8, seed=12, rows=8192,
                positions=torch.arange(32, dtype=torch.int32) * 200)
    first = _run(case, device)
    for _ in range(3):
        again = _run(case, device)
        for x, y in zip(first, again):
            assert torch.equal(x, y)


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23])
def test_tile_variants(variant, device):
    """Every prefill tile variant, on a shape with a row tail (M = 600) and a
    head count (24) that all of them can tile."""
    import mqk
    case = Case(2, 300, 2048, 16, 4, seed=700 + variant)
    old = mqk.get_option("prefill_tile")
    try:
        mqk.set_option("prefill_tile", variant)
        out = _run(case, device)
    finally:
        mqk.set_option("prefill_tile", old)
    _check(out, case.oracle(), f"tile variant {variant}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 4), (40, 8), (12, 2)])
def test_gqa_ratios(Hq, Hkv, device):
    case = Case(2, 96, 1024, Hq, Hkv, seed=500 + Hq)
    _check(_run(case, device), case.oracle(), f"Hq={Hq} Hkv={Hkv}")


# Attention shapes of the other Qwen3 models (hidden, Q heads, KV heads), each as a
# prefill (tile kernel, a partial last row tile) and as a decode step (split-K
# kernel, random positions into an 8192-row table).
QWEN3_FAMILY = [
    ("Qwen3-1.7B", 2048, 16, 8),
    ("Qwen3-4B", 2560, 32, 8),
    ("Qwen3-14B", 5120, 40, 8),
    ("Qwen3-32B", 5120, 64, 8),
    ("Qwen3-235B-A22B", 4096, 64, 4),
]


@pytest.mark.parametrize("name,hidden,Hq,Hkv", QWEN3_FAMILY)
def test_qwen3_family_shapes(name, hidden, Hq, Hkv, device):
    case = Case(1, 200, hidden, Hq, Hkv, seed=hidden + Hq)
    _check(_run(case, device), case.oracle(), f"{name} prefill T=200")
    pos = torch.randint(0, 8192, (48,), generator=torch.Generator().manual_seed(Hq), dtype=torch.int32)
    case = Case(48, 1, hidden, Hq, Hkv, seed=hidden + Hq + 1, rows=8192, positions=pos)
    _check(_run(case, device), case.oracle(), f"{name} decode B=48")


def test_theta_and_scale(device):
    """theta != 1e6 and larger activations (checks no hidden theta/scale assumption).

    Here |v| reaches ~40, where bf16 itself is 0.125 apart, so v is held to
    its own resolution: max-abs <= 2^-8 * max|v| (one ulp of the largest value)."""
    case = Case(1, 256, 2048, 16, 8, seed=21, theta=10000.0, x_std=3.0, w_std=0.05)
    q, k, v = _run(case, device)
    ref = case.oracle()
    _check((q, k), ref[:2], "theta=1e4")
    _check((v,), ref[2:], "theta=1e4 (v)", max_abs=2.0 ** -8 * float(np.abs(ref[2]).max()))


def test_empty_and_single(device):
    import mqk
    case = Case(1, 1, 1024, 16, 8, seed=1)
    _check(_run(case, device), case.oracle(), "T=1 prefill")
    x, wq, wk, wv, gq, gk, c, s, _ = case.args(device)
    q, k, v = mqk.fused_qkv_rope(x[:, :0], wq, wk, wv, gq, gk, c, s)
    assert q.shape == (1, 0, 16, HEAD_DIM) and v.shape == (1, 0, 8, HEAD_DIM)


def test_non_default_stream(device):
    case = Case(2, 64, 1024, 16, 8, seed=31)
    s = torch.cuda.Stream()
    args = case.args(device)
    torch.cuda.synchronize()
    import mqk
    with torch.cuda.stream(s):
        out = mqk.fused_qkv_rope(*args)
    s.synchronize()
    _check(out, case.oracle(), "side stream")


# ── RoPE row indexing, bit-exact ─────────────────────────────────────────────

def _sentinel_case(T, rows, positions, seed):
    """Inputs whose expected output is exactly representable.

    x = e_0 (one-hot on hidden index 0) and W[:, 0] = 1, so every head's
    projection is the constant vector 1; gamma = 1 -> normalised value
    k = 1/sqrt(1 + eps).  Table entries are multiples of 1/64 that encode the
    row index r in 5-bit fields:
      cos[r, d] = 1 + ((r >> 5*(d % 4)) & 31) / 64
      sin[r, d] = ((r >> 5*((d // 4) % 4)) & 31) / 64
    so out[d] = (cos - sin) * k and out[d+64] = (cos + sin) * k round back to
    the exact bf16 values cos -/+ sin, and every row (up to 2^20) gives a
    different output: the test reveals exactly which row each token read, for
    cos and sin and for both halves separately.
    """
    hidden, Hq, Hkv = 256, 2, 1
    case = Case(1, T, hidden, Hq, Hkv, seed=seed, gamma_ones=True, rows=rows, positions=positions)
    x = torch.zeros(1, T, hidden)
    x[..., 0] = 1.0
    case.x = x.bfloat16()
    for name in ("w_q", "w_k", "w_v"):
        w = getattr(case, name).float()
        w[:, 0] = 1.0
        w[:, 1:] = 0.0
        setattr(case, name, w.bfloat16())
    ri = torch.arange(rows)[:, None]
    di = torch.arange(HEAD_DIM)[None, :]
    case.cos = (1.0 + ((ri >> (5 * (di % 4))) & 31).float() / 64.0).bfloat16()
    case.sin = (((ri >> (5 * ((di // 4) % 4))) & 31).float() / 64.0).bfloat16()
    return case


def _expected_sentinel(case, row_of_token):
    from oracle import qkv_rope_oracle as orc
    c = f32(case.cos)[row_of_token]
    s = f32(case.sin)[row_of_token]
    half = HEAD_DIM // 2
    k = np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(1e-6))
    lo = (c[:, :half] - s[:, :half]) * k
    hi = (c[:, half:] + s[:, half:]) * k
    return orc.round_bf16(np.concatenate([lo, hi], axis=-1))


@pytest.mark.parametrize("T", [5, 64, 300])
def test_rope_rows_prefill_bitexact(T, device):
    """Prefill: token t reads row t % S (fused_qkv_rope.py:109); batch of B=3."""
    S = T
    case = _sentinel_case(T, rows=S, positions=None, seed=41)
    # three sequences of length S: rows repeat t % S
    case.x = case.x.repeat(3, 1, 1)
    case.B = 3
    q, k, v = _run(case, device)
    rows = np.arange(3 * S) % S
    exp = _expected_sentinel(case, rows)
    qf = f32(q).reshape(3 * S, 2, HEAD_DIM)
    kf = f32(k).reshape(3 * S, 1, HEAD_DIM)
    assert np.array_equal(qf[:, 0], exp) and np.array_equal(qf[:, 1], exp)
    assert np.array_equal(kf[:, 0], exp)
    assert np.all(f32(v) == 1.0)


@pytest.mark.parametrize("T", [1, 33, 64, 257])
def test_rope_rows_positions_bitexact(T, device):
    """Positions mode: token t reads row positions[t] (fused_qkv_rope.py:107)."""
    g = torch.Generator().manual_seed(T)
    pos = torch.randint(0, 8192, (T,), generator=g).to(torch.int32)
    case = _sentinel_case(T, rows=8192, positions=pos, seed=42)
    q, k, _ = _run(case, device)
    exp = _expected_sentinel(case, pos.numpy().astype(np.int64))
    assert np.array_equal(f32(q).reshape(T, 2, HEAD_DIM)[:, 1], exp)
    assert np.array_equal(f32(k).reshape(T, 1, HEAD_DIM)[:, 0], exp)


def test_positions_out_of_range_clamped(device):
    """Rows outside the table are clamped (the reference reads out of bounds)."""
    pos = torch.tensor([-5, 0, 3, 10, 1000], dtype=torch.int32)
    case = _sentinel_case(5, rows=8, positions=pos, seed=43)
    q, _, _ = _run(case, device)
    exp = _expected_sentinel(case, np.array([0, 0, 3, 7, 7]))
    assert np.array_equal(f32(q).reshape(5, 2, HEAD_DIM)[:, 0], exp)


# ── BASELINE configurations (token sample checked against the oracle) ─────────

def _sample(T, n, seed):
    idx = np.random.default_rng(seed).choice(T, size=min(n, T), replace=False)
    idx.sort()
    return idx


def test_config2_qwen3_8b_prefill(device):
    case = Case(4, 512, 4096, 32, 8, seed=1)
    q, k, v = _run(case, device)
    idx = _sample(2048, 192, 1)
    ref = case.oracle(token_idx=idx)
    out = tuple(t.reshape(2048, *t.shape[2:])[torch.as_tensor(idx)] for t in (q, k, v))
    _check(out, tuple(r[0] for r in ref), "C2 8B prefill")


def test_config3_qwen3_8b_decode(device):
    g = torch.Generator().manual_seed(2)
    pos = torch.randint(0, 8192, (64,), generator=g).to(torch.int32)
    case = Case(64, 1, 4096, 32, 8, seed=2, rows=8192, positions=pos)
    _check(_run(case, device), case.oracle(), "C3 8B decode")


def test_config4_30b_a3b_long_prefill(device):
    case = Case(1, 8192, 2048, 32, 4, seed=3)
    q, k, v = _run(case, device)
    idx = _sample(8192, 160, 3)
    ref = case.oracle(token_idx=idx)
    out = tuple(t.reshape(8192, *t.shape[2:])[torch.as_tensor(idx)] for t in (q, k, v))
    _check(out, tuple(r[0] for r in ref), "C4 30B-A3B S=8192")


def test_large_t_64bit_offsets(device):
    """Maximum-size addressing: T = 270000 tokens with 32 query heads puts q's
    byte offsets past 2^31 (t * Hq * 128 * 2), so every output, x and table index
    must be 64-bit.  Checked against the oracle on the first and last tokens."""
    T, hidden, Hq, Hkv = 270000, 64, 32, 4
    pos = (torch.arange(T) % 4096).to(torch.int32)
    case = Case(1, T, hidden, Hq, Hkv, seed=11, rows=4096, positions=pos)
    q, k, v = _run(case, device)
    torch.cuda.synchronize()
    assert q.numel() * q.element_size() > 2 ** 31
    idx = np.concatenate([np.arange(0, 8), np.arange(T - 24, T)])
    ref = case.oracle(token_idx=idx)
    out = tuple(t.reshape(T, *t.shape[2:])[torch.as_tensor(idx)] for t in (q, k, v))
    _check(out, tuple(r[0] for r in ref), "T=270000")


# ── argument checks of the Python shim (the reference asserts only an even D) ──

def test_shim_rejects_bad_arguments(device):
    import mqk
    case = Case(1, 8, 1024, 16, 8, seed=140)
    args = list(case.args(device))
    bad = list(args)
    bad[0] = case.x  # host tensor
    with pytest.raises(ValueError, match="x must be on a GPU device"):
        mqk.fused_qkv_rope(*bad)
    bad = list(args)
    bad[2] = bad[2].half()
    with pytest.raises(TypeError, match="w_k must be torch.bfloat16"):
        mqk.fused_qkv_rope(*bad)
    with pytest.raises(TypeError, match="positions must be int32"):
        mqk.fused_qkv_rope(*args[:8], torch.zeros(8, device=device))
    with pytest.raises(ValueError, match="positions has 7 entries"):
        mqk.fused_qkv_rope(*args[:8], torch.zeros(7, dtype=torch.int32, device=device))
    with pytest.raises(ValueError, match="weight shapes"):
        mqk.fused_qkv_rope(args[0], args[1][:, :512], *args[2:8])


def test_shim_accepts_strided_and_int64_inputs(device):
    """Non-contiguous inputs are made contiguous and int64 positions converted:
    the result equals the call on contiguous int32 inputs bit for bit."""
    import mqk
    g = torch.Generator().manual_seed(141)
    pos = torch.randint(0, 64, (16,), generator=g, dtype=torch.int32)
    case = Case(16, 1, 1024, 16, 8, seed=141, rows=64, positions=pos)
    args = list(case.args(device))
    ref = mqk.fused_qkv_rope(*args)
    strided = list(args)
    strided[1] = args[1].t().contiguous().t()          # column-major w_q
    strided[6] = torch.cat([args[6], args[6]], 1)[:, :HEAD_DIM]  # cos with row stride 2 * D
    strided[8] = args[8].long()
    assert not strided[1].is_contiguous() and not strided[6].is_contiguous()
    out = mqk.fused_qkv_rope(*strided)
    torch.cuda.synchronize()
    for a, b in zip(out, ref):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,S", [(16, 1), (1, 300)])
def test_unaligned_views_take_the_fast_path(B, S, device):
    """x and w_k passed as views at an odd element offset: the shim copies them to
    aligned storage, so the call runs the same kernels (the decode kernel, a tile
    plan) as with aligned operands and returns the same bits."""
    import mqk
    from conftest import launched_kernels
    pos = torch.randint(0, 4096, (B * S,), generator=torch.Generator().manual_seed(B), dtype=torch.int32)
    case = Case(B, S, 1024, 16, 8, seed=150 + B, rows=4096, positions=pos)
    args = list(case.args(device))

    def odd(t):  # same values, storage offset of one element (2 bytes)
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=device)
        v = buf[1:].view(t.shape)
        v.copy_(t)
        return v
    shifted = list(args)
    shifted[0], shifted[2] = odd(args[0]), odd(args[2])
    assert shifted[0].data_ptr() % 16 and shifted[2].data_ptr() % 16
    ref_kernels = launched_kernels(lambda: mqk.fused_qkv_rope(*args))
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*shifted)) == ref_kernels
    assert "tile_reg" not in ref_kernels
    for a, b in zip(mqk.fused_qkv_rope(*args), mqk.fused_qkv_rope(*shifted)):
        assert torch.equal(a, b)
