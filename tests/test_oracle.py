"""Pins the CPU oracle (oracle/qkv_rope_oracle.py) against checks that do not
restate its own formulas: exhaustive bit-level round trips, closed forms,
special inputs, an independent complex-number formulation of RoPE, brute force
on tiny shapes, and hand-computed known answers.

The reference ships no golden vectors or fixtures for this path (its fused
tests are unseeded and compare against an oracle kept in the test file), so
these checks are the oracle's pinning; each names the reference line it
protects.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import qkv_rope_oracle as orc

D = 128


# ── bf16 helpers ──────────────────────────────────────────────────────────────

def test_bf16_roundtrip_exhaustive():
    """Every finite bf16 pattern widens and narrows back to itself."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.bf16_to_f32(bits)
    finite = np.isfinite(f)
    back = orc.f32_to_bf16(f[finite])
    assert np.array_equal(back, bits[finite])


def test_bf16_round_to_nearest_even():
    # 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7: ties to even (1.0)
    assert orc.f32_to_bf16(np.float32(1 + 2 ** -8)) == 0x3F80
    # 1 + 3 * 2^-8 is halfway between 1 + 2^-7 (odd) and 1 + 2^-6: rounds up
    assert orc.f32_to_bf16(np.float32(1 + 3 * 2 ** -8)) == 0x3F82
    # just above a tie rounds up
    assert orc.f32_to_bf16(np.float32(1 + 2 ** -8 + 2 ** -20)) == 0x3F81
    assert orc.f32_to_bf16(np.float32(-2.0)) == 0xC000
    assert orc.f32_to_bf16(np.float32(np.nan)) == 0x7FC0


def test_bf16_matches_torch():
    """Same rounding as torch's float32 -> bfloat16 cast on random data."""
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(0).standard_normal(100_000).astype(np.float32) * 37
    t = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), t)


# ── RoPE tables (rope.py:6-21) ────────────────────────────────────────────────

@pytest.mark.parametrize("theta", [1e6, 1e4])
def test_rope_tables_closed_form(theta):
    """fp32 tables match cos/sin(p * theta^(-2i/D)) to the fp32 angle error."""
    n = 8192
    cos, sin = orc.rope_tables(D, n, theta)
    p = np.arange(n, dtype=np.float64)[:, None]
    i = np.arange(D // 2, dtype=np.float64)[None, :]
    ang = p * theta ** (-2 * i / D)
    ang = np.concatenate([ang, ang], axis=1)
    # fp32 angle = p * inv_freq carries ~|angle| * 2^-23 absolute error
    tol = np.abs(ang) * 2.0 ** -22 + 1e-6
    assert np.all(np.abs(cos - np.cos(ang)) <= tol)
    assert np.all(np.abs(sin - np.sin(ang)) <= tol)


def test_rope_tables_layout():
    cos, sin = orc.rope_tables(D, 64)
    assert cos.shape == (64, D) and cos.dtype == np.float32
    assert np.array_equal(cos[:, : D // 2], cos[:, D // 2:])  # cat([f, f]) (rope.py:15)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)     # position 0 = identity


# ── QK-Norm (fused_qkv_rope.py:98-100) ───────────────────────────────────────

@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_norm_constant_vector(D):
    """x = c * ones  ->  sign(c) * gamma / sqrt(1 + eps / c^2)."""
    g = np.random.default_rng(1).uniform(0.5, 1.5, D)
    for c in (3.0, -0.25, 1e-2):
        out = orc.qk_norm(np.full((1, 1, D), c), g, eps=1e-6)
        exp = np.sign(c) * g / math.sqrt(1 + 1e-6 / c ** 2)
        np.testing.assert_allclose(out[0, 0], exp, rtol=1e-12)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_norm_one_hot_and_zero(D):
    g = np.linspace(0.5, 1.5, D)
    x = np.zeros((1, 1, D))
    x[0, 0, 17] = 5.0
    out = orc.qk_norm(x, g, eps=0.0)
    exp = np.zeros(D)
    exp[17] = math.sqrt(D) * g[17]
    np.testing.assert_allclose(out[0, 0], exp, rtol=1e-12, atol=1e-12)
    assert np.all(orc.qk_norm(np.zeros((2, 3, D)), g) == 0.0)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_norm_scale_invariant_and_gamma_per_dim(D):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 3, D))
    g = rng.uniform(0.5, 1.5, D)
    a = orc.qk_norm(x, g, eps=0.0)
    np.testing.assert_allclose(orc.qk_norm(7.5 * x, g, eps=0.0), a, rtol=1e-12)
    # unit RMS after removing gamma
    np.testing.assert_allclose(np.sqrt(np.mean((a / g) ** 2, axis=-1)), 1.0, rtol=1e-12)


# ── RoPE (fused_qkv_rope.py:102-118) ─────────────────────────────────────────

def _tables64(n, theta=1e6, D=D):
    return orc.rope_tables(D, n, theta, np.float64)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_rope_matches_complex_rotation(D):
    """Independent formulation: (x1 + i x2) * e^{i angle} = out1 + i out2, which
    fixes the sign convention and the half pairing of rotate_half."""
    rng = np.random.default_rng(3)
    T, H = 37, 3
    x = rng.standard_normal((T, H, D))
    cos, sin = _tables64(4096, D=D)
    rows = rng.integers(0, 4096, T)
    out = orc.rope(x, cos[rows], sin[rows])
    z = (x[..., : D // 2] + 1j * x[..., D // 2:]) * np.exp(1j * np.arctan2(sin[rows, : D // 2], cos[rows, : D // 2]))[:, None, :]
    np.testing.assert_allclose(out[..., : D // 2], z.real, atol=1e-12)
    np.testing.assert_allclose(out[..., D // 2:], z.imag, atol=1e-12)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_rope_identity_norm_and_inverse(D):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((16, 2, D))
    cos, sin = _tables64(512, D=D)
    np.testing.assert_array_equal(orc.rope(x, cos[[0] * 16], sin[[0] * 16]), x)
    rows = rng.integers(0, 512, 16)
    y = orc.rope(x, cos[rows], sin[rows])
    pair = lambda a: a[..., : D // 2] ** 2 + a[..., D // 2:] ** 2
    np.testing.assert_allclose(pair(y), pair(x), rtol=1e-10)
    back = orc.rope(y, cos[rows], -sin[rows])  # rotate by -angle
    np.testing.assert_allclose(back, x, atol=1e-12)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_rope_uses_both_table_halves(D):
    """The kernel reads cos/sin halves separately (:112-115): tables whose halves
    differ must give different results for the two output halves."""
    x = np.ones((1, 1, D))
    c = np.zeros((1, D)); c[0, : D // 2] = 1.0; c[0, D // 2:] = 2.0
    s = np.zeros((1, D)); s[0, : D // 2] = 0.5; s[0, D // 2:] = 0.25
    out = orc.rope(x, c, s)[0, 0]
    assert np.all(out[: D // 2] == 1.0 - 0.5) and np.all(out[D // 2:] == 2.0 + 0.25)


def test_row_selection():
    """prefill: t % S (:109); positions mode: positions[t] (:107)."""
    assert list(orc.rope_rows(10, 4)) == [0, 1, 2, 3, 0, 1, 2, 3, 0, 1]
    assert list(orc.rope_rows(3, 99, np.array([7, 0, 5]))) == [7, 0, 5]


# ── projection and the whole op ───────────────────────────────────────────────

def test_projection_brute_force():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 5))
    w = rng.standard_normal((4, 5))
    ref = [[sum(x[i, k] * w[j, k] for k in range(5)) for j in range(4)] for i in range(3)]
    np.testing.assert_allclose(orc.projection(x, w), ref, rtol=1e-12)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_fused_shapes_and_v_passthrough(D):
    rng = np.random.default_rng(6)
    B, S, H, Hq, Hkv = 2, 5, 256, 4, 2
    x = rng.standard_normal((B, S, H))
    wq, wk, wv = (rng.standard_normal((h * D, H)) * 0.05 for h in (Hq, Hkv, Hkv))
    g = np.ones(D)
    cos, sin = _tables64(S, D=D)
    q, k, v = orc.fused_qkv_rope(x, wq, wk, wv, g, g, cos, sin)
    assert q.shape == (B, S, Hq, D) and k.shape == (B, S, Hkv, D) and v.shape == (B, S, Hkv, D)
    np.testing.assert_allclose(v.reshape(B * S, -1), x.reshape(B * S, H) @ wv.T, rtol=1e-12)


@pytest.mark.parametrize("D", [128, 64])  # head_dim: Qwen3 checkpoints / the reference's default config
def test_fused_equals_unfused_composition(D):
    """The fused oracle agrees with the reference's unfused composition
    (test_fused_qkv_rope.py:244-259) evaluated in float64."""
    rng = np.random.default_rng(7)
    B, S, H, Hq, Hkv = 1, 9, 256, 2, 1
    x = rng.standard_normal((B, S, H))
    wq, wk, wv = (rng.standard_normal((h * D, H)) * 0.05 for h in (Hq, Hkv, Hkv))
    gq, gk = rng.uniform(0.8, 1.2, D), rng.uniform(0.8, 1.2, D)
    cos, sin = _tables64(S, D=D)
    a = orc.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
    b = orc.unfused_composition(x, wq, wk, wv, gq, gk, cos, sin, dtype=np.float64)
    for u, w_ in zip(a, b):
        np.testing.assert_allclose(u, w_, rtol=1e-10, atol=1e-12)


def test_torch_cpu_baseline_equals_fused_oracle():
    """The torch restatement bench.py times as the CPU baseline computes the same
    function as the fused oracle (float64 on both sides), GQA shapes and S > 1."""
    import torch
    from oracle.torch_baseline import unfused_composition_torch
    rng = np.random.default_rng(17)
    B, S, H, Hq, Hkv = 2, 7, 256, 4, 2
    x = rng.standard_normal((B, S, H))
    wq, wk, wv = (rng.standard_normal((h * D, H)) * 0.05 for h in (Hq, Hkv, Hkv))
    gq, gk = rng.uniform(0.8, 1.2, D), rng.uniform(0.8, 1.2, D)
    cos, sin = _tables64(S, D=D)
    a = orc.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin)
    t = lambda v: torch.from_numpy(np.ascontiguousarray(v))
    b = unfused_composition_torch(t(x), t(wq), t(wk), t(wv), t(gq), t(gk), t(cos), t(sin))
    for u, w_ in zip(a, b):
        assert tuple(w_.shape) == u.shape
        np.testing.assert_allclose(w_.numpy(), u, rtol=1e-10, atol=1e-12)


def test_round_projection_changes_only_by_bf16_rounding():
    rng = np.random.default_rng(8)
    x = orc.round_bf16(rng.standard_normal((1, 4, 256)).astype(np.float32))
    w = orc.round_bf16((rng.standard_normal((D, 256)) * 0.05).astype(np.float32))
    g = np.ones(D, np.float32)
    cos, sin = orc.rope_tables(D, 4)
    exact = orc.fused_qkv_rope(x, w, w, w, g, g, cos, sin)
    rounded = orc.fused_qkv_rope(x, w, w, w, g, g, cos, sin, round_projection=True)
    assert np.array_equal(rounded[2], orc.round_bf16(exact[2].astype(np.float32)))
    assert orc.max_abs(rounded[0], exact[0]) < 0.05


def test_rms_norm_hf_rounds_before_gamma():
    """rms_norm.py:15-18 rounds x*rms to the input dtype before the gamma multiply."""
    x = np.full((1, D), 3.0, np.float32)
    x[0, 0] = 1.0
    g = np.full(D, 1.5, np.float32)
    y = orc.rms_norm_hf(x, g)
    rms = 1 / np.sqrt(np.mean(x * x) + 1e-6)
    assert y[0, 0] == np.float32(1.5) * orc.round_bf16(np.float32(1.0) * np.float32(rms))


def test_rms_norm_hf_round_out_closed_form():
    """bf16 model: weight * y is a bf16 product.  x = 2 everywhere gives y = bf16(0.99999988)
    = 1 exactly, so the output is the weight rounded to bf16: 1 + 2^-8 is a tie that
    rounds to even (1.0)."""
    x = np.full((2, 64), 2.0, np.float32)
    g = np.full(64, 1.0 + 2.0 ** -8, np.float32)
    assert np.all(orc.rms_norm_hf(x, g, round_out=True) == 1.0)
    assert np.all(orc.rms_norm_hf(x, g) == np.float32(1.0 + 2.0 ** -8))
    g2 = np.full(64, 1.0 + 3 * 2.0 ** -8, np.float32)  # tie between 1+2^-7 and 1+2^-6: even is 1+2^-6
    assert np.all(orc.rms_norm_hf(x, g2, round_out=True) == np.float32(1.0 + 2.0 ** -6))


# ── int4 format (packing.py, awq.py, linear_w4a16.py) ─────────────────────────

def test_pack_known_answer():
    """packed = sum(v[i] << 4i): 0..7 -> 0x76543210 (packing.py:20-24)."""
    assert orc.pack_int4(np.arange(8))[0] == 0x76543210
    v = np.array([15, 0, 0, 0, 0, 0, 0, 8])
    assert orc.pack_int4(v).view(np.uint32)[0] == 0x8000000F
    assert list(orc.unpack_int4(np.array([0x76543210], np.int32))) == list(range(8))


def test_pack_roundtrips_along_k_and_n():
    rng = np.random.default_rng(9)
    w = rng.integers(0, 16, (128, 64))
    qw = orc.pack_int4(w.T).T            # [K/8, N], along K (test_w4a16_gemm.py:67-74)
    assert qw.shape == (16, 64)
    assert np.array_equal(orc.unpack_int4(qw.T).T, w)
    z = rng.integers(0, 16, (8, 64))
    qz = orc.pack_int4(z)                # [G, N/8], along N (:77-84)
    assert np.array_equal(orc.unpack_int4(qz), z)


def test_minmax_quantizer_hand_example():
    """One group of 128 values in [-1, 2] with a known exact grid."""
    col = np.linspace(-1.0, 2.0, 128).astype(np.float32)
    w = np.stack([col] * 8, axis=1)                   # [128, 8]
    qw, sc_bits, qz = orc.minmax_quantize(w, 128)
    s = orc.bf16_to_f32(sc_bits)
    np.testing.assert_allclose(s, orc.round_bf16(np.float32(3.0 / 15.0)))
    z = orc.unpack_int4(qz)
    assert np.all(z == 5)                             # round(1 / 0.2) = 5
    q = orc.unpack_int4(qw.T).T
    exp = np.clip(np.round(col / np.float32(0.2) + 5), 0, 15)
    assert np.array_equal(q[:, 0], exp.astype(np.int32))


def test_quantizer_error_bound_and_zero_exact():
    rng = np.random.default_rng(10)
    w = rng.standard_normal((256, 16)).astype(np.float32)
    w[5, 3] = 0.0
    qw, sc_bits, qz = orc.minmax_quantize(w, 128)
    sq = (w.reshape(2, 128, 16).max(1) - w.reshape(2, 128, 16).min(1)) / 15
    deq = orc.dequant(qw, sq, qz, 128)          # exact-fp32 scales: error <= s/2 (+ clamp)
    err = np.abs(deq - w).reshape(2, 128, 16)
    assert np.all(err <= sq[:, None, :] * 0.5 + 1e-6)


def test_dequant_brute_force():
    rng = np.random.default_rng(11)
    K, N, g = 256, 16, 128
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(0, 16, (K // g, N))
    s = rng.uniform(0.005, 0.02, (K // g, N)).astype(np.float32)
    deq = orc.dequant(orc.pack_int4(q.T).T, s, orc.pack_int4(z), g)
    for k in range(0, K, 37):
        for n in range(N):
            assert deq[k, n] == np.float32((q[k, n] - z[k // g, n])) * s[k // g, n]


def test_gptq_zero_fix():
    z = np.array([[0, 1, 14, 15, 3, 4, 5, 6]])
    fixed = orc.unpack_int4(orc.gptq_zero_fix(orc.pack_int4(z)))
    assert list(fixed[0]) == [1, 2, 15, 15, 4, 5, 6, 7]


def test_w4a16_gemm_brute_force():
    rng = np.random.default_rng(12)
    M, K, N = 2, 128, 8
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(0, 16, (1, N))
    s = rng.uniform(0.01, 0.02, (1, N)).astype(np.float32)
    x = rng.standard_normal((M, K))
    out = orc.w4a16_gemm(x, orc.pack_int4(q.T).T, s, orc.pack_int4(z), 128)
    ref = np.array([[sum(x[m, k] * float(np.float32(q[k, n] - z[0, n]) * s[0, n]) for k in range(K))
                     for n in range(N)] for m in range(M)])
    np.testing.assert_allclose(out, ref, rtol=1e-10)


def test_metrics():
    a = np.array([1.0, 2.0, 3.0])
    assert orc.max_abs(a, a + [0, 0.5, 0]) == 0.5
    assert abs(orc.rel_l2(a * 1.01, a) - 0.01) < 1e-12
    one = orc.f32_to_bf16(np.float32(1.0))
    nxt = np.uint16(one + 1)
    neg = orc.f32_to_bf16(np.float32(-0.0))
    assert orc.bf16_ulp_distance(one, nxt) == 1
    assert orc.bf16_ulp_distance(neg, orc.f32_to_bf16(np.float32(0.0))) == 0


def test_varlen_positions_known_answer():
    b, p = orc.varlen_positions([0, 3, 3, 7])
    assert b.tolist() == [0, 0, 0, 2, 2, 2, 2]
    assert p.tolist() == [0, 1, 2, 0, 1, 2, 3]
    b, p = orc.varlen_positions([0, 2, 5], seq_pos0=[10, 100])
    assert b.tolist() == [0, 0, 1, 1, 1] and p.tolist() == [10, 11, 100, 101, 102]


def test_varlen_positions_brute_force():
    rng = np.random.default_rng(7)
    lengths = rng.integers(0, 9, 13)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    start = rng.integers(0, 50, 13)
    b, p = orc.varlen_positions(cu, start)
    for t in range(int(cu[-1])):
        s = [i for i in range(13) if cu[i] <= t < cu[i + 1]]
        assert len(s) == 1 and b[t] == s[0] and p[t] == t - cu[s[0]] + start[s[0]]


# ── paged-cache slots (paged_attn_prefill.py:45-56, kv_cache.py:3-6) ─────────

def test_paged_slot_known_answer():
    """Block size 4, two sequences: seq 0 owns blocks (5, 2), seq 1 owns (0, 7).
    pos 0 of seq 0 -> block 5, slot 0 -> 20; pos 6 of seq 0 -> page 1 = block 2,
    slot 2 -> 10; pos 3 of seq 1 -> block 0, slot 3 -> 3; pos 5 of seq 1 ->
    block 7, slot 1 -> 29.  Out of the table: pos 8 (page 2), seq 2, pos -1,
    and a block id beyond num_blocks."""
    bt = np.array([[5, 2], [0, 7]])
    got = orc.paged_slot(bt, [0, 0, 1, 1, 0, 2, 1], [0, 6, 3, 5, 8, 0, -1], block_size=4, num_blocks=8)
    assert got.tolist() == [20, 10, 3, 29, -1, -1, -1]
    assert orc.paged_slot(np.array([[9]]), [0], [1], 4, num_blocks=8).tolist() == [-1]


def test_paged_slot_brute_force():
    """Every (seq, pos) of a random table: the slot is the unique cache position
    whose (block, offset) pair the table assigns to that token."""
    rng = np.random.default_rng(8)
    bs, rows, cols = 16, 3, 5
    nb = rows * cols + 4
    bt = rng.permutation(nb)[: rows * cols].reshape(rows, cols)
    owner = {}  # cache slot -> (seq, pos), by walking the cache
    for blk in range(nb):
        for off in range(bs):
            hit = [(s, c) for s in range(rows) for c in range(cols) if bt[s, c] == blk]
            if hit:
                s, c = hit[0]
                owner[blk * bs + off] = (s, c * bs + off)
    seqs, poss = np.meshgrid(np.arange(rows), np.arange(cols * bs), indexing="ij")
    got = orc.paged_slot(bt, seqs.ravel(), poss.ravel(), bs, nb)
    for slot, s, p in zip(got, seqs.ravel(), poss.ravel()):
        assert owner[int(slot)] == (s, p)
    assert len(set(got.tolist())) == got.size


# ── AutoAWQ words (AWQ order 0,2,4,6,1,3,5,7) ─────────────────────────────────

def test_awq_unpack_known_answer():
    """Column c of an 8-column group holding value c packs to 0x75316420: nibble
    i holds column (0,2,4,6,1,3,5,7)[i], so nibbles read 0,2,4,6,1,3,5,7."""
    w = np.array([[0x75316420, 0x00000000, 0x11111111]], dtype=np.uint32).view(np.int32)
    got = orc.awq_unpack(w)
    assert got[0, :8].tolist() == list(range(8))
    assert got[0, 8:16].tolist() == [0] * 8 and got[0, 16:].tolist() == [1] * 8
    hi = np.array([[np.uint32(0xF0000000)]]).view(np.int32)   # top nibble = nibble 7 -> column 7
    assert orc.awq_unpack(hi)[0].tolist() == [0] * 7 + [15]


def test_dequant_awq_brute_force():
    rng = np.random.default_rng(9)
    K, N, g = 256, 16, 128
    words = rng.integers(0, 2**32, (K, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    zw = rng.integers(0, 2**32, (K // g, N // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    s = rng.uniform(0.005, 0.02, (K // g, N)).astype(np.float32)
    got = orc.dequant_awq(words, zw, s, g)
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    for k in range(0, K, 37):
        for n in range(N):
            i = order.index(n % 8)  # nibble holding column n
            q = (int(words.view(np.uint32)[k, n // 8]) >> (4 * i)) & 0xF
            z = (int(zw.view(np.uint32)[k // g, n // 8]) >> (4 * i)) & 0xF
            assert got[k, n] == np.float32((q - z) * s[k // g, n])
