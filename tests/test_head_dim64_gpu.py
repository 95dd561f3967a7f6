"""GPU parity at head_dim 64, the head size of the reference's default model
config (mini_qwen/config.py:13: Qwen3Config.head_dim = 64, with 16 query and 8
KV heads over hidden 1024).  The reference op infers D from q_norm_w
(mini_qwen/kernels/fused_qkv_rope.py:155-160) and accepts it.

The kernels tile the projection in 128-column blocks; at head_dim 64 a block
holds two heads, each normalised over its own 64 dims and rotated with pairs
(d, d + 32).  Every kernel family is exercised here against the oracle, which
is written for any D (tests/test_oracle.py pins it at D = 64 as well): the
pipelined tile kernel, the register-staged tiles, the single-head and split-K
tiles of mid token counts, the decode kernel (one block, several blocks, long
splits), the int4 tiles and decode, the fp32 / fp16 front, the standalone
QK-Norm + RoPE and the paged-cache write.  Row selection is checked bit for bit
with sentinel tables, in prefill and positions modes.

Bars as for head_dim 128: max-abs 2e-2 and rel-L2 1e-2 against the oracle's
exact projection followed by norm and RoPE in float64.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import Case, f32, launched_kernels

pytestmark = pytest.mark.gpu

D = 64
MAX_ABS = 2e-2
REL_L2 = 1e-2


def _run(case, device, **kw):
    import mqk
    return mqk.fused_qkv_rope(*case.args(device), **kw)


def _check(out, ref, label, max_abs=MAX_ABS, rel_l2=REL_L2):
    from oracle import qkv_rope_oracle as orc
    for name, o, r in zip("qkv", out, ref):
        o = f32(o).reshape(r.shape)
        assert np.isfinite(o).all(), f"{label}: {name} has non-finite values"
        ma, rl = orc.max_abs(o, r), orc.rel_l2(o, r)
        print(f"  {label} {name}: max_abs={ma:.5f} rel_l2={rl:.2e}")
        assert ma <= max_abs, f"{label} {name}: max abs {ma:.5f} > {max_abs}"
        assert rl <= rel_l2, f"{label} {name}: rel L2 {rl:.3e} > {rel_l2}"


class _Options:
    """Sets mqk options for the duration of a with-block."""

    def __init__(self, **opts):
        self.opts = opts

    def __enter__(self):
        import mqk
        self.old = {k: mqk.get_option(k) for k in self.opts}
        for k, v in self.opts.items():
            mqk.set_option(k, v)

    def __exit__(self, *exc):
        import mqk
        for k, v in self.old.items():
            mqk.set_option(k, v)


# ── the reference's default config and its shapes ─────────────────────────────

@pytest.mark.parametrize("B,S", [(1, 32), (2, 64), (4, 128), (4, 512)])
def test_default_config_prefill(B, S, device):
    """Qwen3Config() (hidden 1024, 16 / 8 heads of 64): prefill over the decode,
    mid-T and tile plans, against the oracle and its bf16-rounded-GEMM variant."""
    case = Case(B, S, 1024, 16, 8, seed=6400 + S, head_dim=D)
    q, k, v = _run(case, device)
    torch.cuda.synchronize()
    assert q.shape == (B, S, 16, D) and k.shape == (B, S, 8, D) and v.shape == (B, S, 8, D)
    assert q.is_contiguous() and k.is_contiguous() and v.is_contiguous()
    _check((q, k, v), case.oracle(), f"D=64 B={B} S={S}")
    _check((q, k, v), case.oracle(round_projection=True), f"D=64 B={B} S={S} (bf16 GEMM ref)",
           max_abs=2 * MAX_ABS)


@pytest.mark.parametrize("B,hidden,Hq,Hkv", [(1, 1024, 16, 8), (8, 1024, 16, 8), (64, 1024, 16, 8),
                                             (64, 4096, 64, 16), (48, 5120, 80, 16)])
def test_decode_positions(B, hidden, Hq, Hkv, device):
    """Decode steps (positions into an 8192-row table): the split-K decode kernel,
    including the long splits of a wide model (hidden 5120)."""
    pos = torch.randint(0, 8192, (B,), generator=torch.Generator().manual_seed(B + Hq), dtype=torch.int32)
    case = Case(B, 1, hidden, Hq, Hkv, seed=6500 + B, rows=8192, positions=pos, head_dim=D)
    _check(_run(case, device), case.oracle(), f"D=64 decode B={B} hidden={hidden}")


@pytest.mark.parametrize("splits", [0, 4, 7])
def test_decode_splits_and_recompute(splits, device):
    """Other split counts against the oracle, and the recompute path (taken when
    a split runs on an unexpected XCD) bit-identical to the finish from partials
    at the same split count."""
    pos = torch.randint(0, 8192, (64,), generator=torch.Generator().manual_seed(splits), dtype=torch.int32)
    case = Case(64, 1, 4096, 64, 16, seed=6600 + splits, rows=8192, positions=pos, head_dim=D)
    with _Options(decode_splits=splits):
        ref = _run(case, device)
        with _Options(decode_force_recompute=1):
            out = _run(case, device)
    for a, b in zip(ref, out):
        assert torch.equal(a, b)
    _check(out, case.oracle(), f"D=64 decode splits={splits}")


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23])
def test_tile_variants(variant, device):
    """Every prefill tile variant (pipelined and register-staged) on 24 blocks
    of 128 columns (32 / 8 heads of 64), with a partial last row tile."""
    case = Case(2, 300, 2048, 32, 8, seed=6700 + variant, head_dim=D)
    with _Options(prefill_tile=variant):
        out = _run(case, device)
    _check(out, case.oracle(), f"D=64 tile variant {variant}")


@pytest.mark.parametrize("T,opts,plan", [
    (256, dict(), None),                                          # default plan
    (256, dict(head_tiles=0), ["tile_split"]),                    # split-K tiles
    (200, dict(head_tiles=0, tile_ksplit=0), ["decode_multi"]),   # several decode blocks in one launch
    (512, dict(), None),
])
def test_mid_token_counts(T, opts, plan, device):
    """Mid token counts at Qwen3-8B width with head_dim 64 (64 / 16 heads): the
    single-head tiles, the split-K tile launch and the decode blocks."""
    import mqk
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = Case(1, T, 4096, 64, 16, seed=6800 + T, rows=8192, positions=pos, head_dim=D)
    with _Options(**opts):
        if plan is not None:
            args = case.args(device)
            assert launched_kernels(lambda: mqk.fused_qkv_rope(*args)) == plan
        out = _run(case, device)
    _check(out, case.oracle(), f"D=64 T={T} {opts}")


def test_config2_shape_at_head_dim_64(device):
    """BASELINE config 2's projection (hidden 4096, N = 6144) as 96 / 24 heads of
    64: the 128 x 384 tiles, sampled tokens against the oracle."""
    case = Case(4, 512, 4096, 64, 16, seed=6900, head_dim=D)
    q, k, v = _run(case, device)
    idx = np.sort(np.random.default_rng(1).choice(2048, 128, replace=False))
    ref = case.oracle(token_idx=idx)
    out = tuple(t.reshape(2048, *t.shape[2:])[torch.as_tensor(idx)] for t in (q, k, v))
    _check(out, tuple(r[0] for r in ref), "D=64 C2 shape")


# ── row selection, bit-exact (sentinel tables, as at head_dim 128) ─────────────

def _sentinel_case(T, rows, positions, seed):
    """x = e_0 and W[:, 0] = 1, so every head's projection is the constant 1 and,
    with gamma = 1, the normalised value is k = 1/sqrt(1 + eps); cos / sin entries
    encode the row in 5-bit fields (multiples of 1/64), so the output reveals the
    row each token read, for both tables and both halves (d < 32, d >= 32)."""
    hidden, Hq, Hkv = 256, 2, 2
    case = Case(1, T, hidden, Hq, Hkv, seed=seed, gamma_ones=True, rows=rows, positions=positions, head_dim=D)
    x = torch.zeros(1, T, hidden)
    x[..., 0] = 1.0
    case.x = x.bfloat16()
    for name in ("w_q", "w_k", "w_v"):
        w = getattr(case, name).float()
        w[:, 0] = 1.0
        w[:, 1:] = 0.0
        setattr(case, name, w.bfloat16())
    ri = torch.arange(rows)[:, None]
    di = torch.arange(D)[None, :]
    case.cos = (1.0 + ((ri >> (5 * (di % 4))) & 31).float() / 64.0).bfloat16()
    case.sin = (((ri >> (5 * ((di // 4) % 4))) & 31).float() / 64.0).bfloat16()
    return case


def _expected_sentinel(case, row_of_token):
    from oracle import qkv_rope_oracle as orc
    c = f32(case.cos)[row_of_token]
    s = f32(case.sin)[row_of_token]
    half = D // 2
    k = np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(1e-6))
    lo = (c[:, :half] - s[:, :half]) * k
    hi = (c[:, half:] + s[:, half:]) * k
    return orc.round_bf16(np.concatenate([lo, hi], axis=-1))


@pytest.mark.parametrize("T", [5, 64, 300])
def test_rope_rows_prefill_bitexact(T, device):
    """Prefill: token t reads row t % S (fused_qkv_rope.py:109), batch of 3."""
    case = _sentinel_case(T, rows=T, positions=None, seed=71)
    case.x = case.x.repeat(3, 1, 1)
    case.B = 3
    q, k, v = _run(case, device)
    exp = _expected_sentinel(case, np.arange(3 * T) % T)
    qf = f32(q).reshape(3 * T, 2, D)
    kf = f32(k).reshape(3 * T, 2, D)
    for h in range(2):
        assert np.array_equal(qf[:, h], exp), f"q head {h}"
        assert np.array_equal(kf[:, h], exp), f"k head {h}"
    assert np.all(f32(v) == 1.0)


@pytest.mark.parametrize("T", [1, 33, 64, 257])
def test_rope_rows_positions_bitexact(T, device):
    """Positions mode: token t reads row positions[t] (fused_qkv_rope.py:107);
    T = 1..64 run the decode kernel, 257 a tile plan."""
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(T), dtype=torch.int32)
    case = _sentinel_case(T, rows=8192, positions=pos, seed=72)
    q, k, _ = _run(case, device)
    exp = _expected_sentinel(case, pos.numpy().astype(np.int64))
    for h in range(2):
        assert np.array_equal(f32(q).reshape(T, 2, D)[:, h], exp), f"q head {h}"
        assert np.array_equal(f32(k).reshape(T, 2, D)[:, h], exp), f"k head {h}"


# ── the other entry points ───────────────────────────────────────────────────

@pytest.mark.parametrize("B,S,positions_mode", [(2, 100, False), (1, 8, True), (1, 300, True)])
def test_w4a16_front(B, S, positions_mode, device):
    """The fused W4A16 front (int4 tiles, int4 decode) at head_dim 64, against
    norm + RoPE of the projection with the dequantised weight rounded to bf16."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    hidden, Hq, Hkv = 1024, 16, 8
    g = torch.Generator().manual_seed(S)
    projs = []
    for i, h in enumerate((Hq, Hkv, Hkv)):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(mqk.per_group_minmax_quantize(w, 128, torch.bfloat16))
    x = torch.randn(B, S, hidden, generator=g).bfloat16()
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    rows = 4096 if positions_mode else S
    c, s = mqk.rope_tables(D, rows)
    cos, sin = c.bfloat16(), s.bfloat16()
    pos = torch.randint(0, rows, (B * S,), generator=g, dtype=torch.int32) if positions_mode else None
    dp = [tuple(t.to(device) for t in p) for p in projs]
    out = mqk.fused_qkv_rope_w4a16(x.to(device), *dp, gq.to(device), gk.to(device), cos.to(device),
                                   sin.to(device), None if pos is None else pos.to(device))
    ref = orc.fused_qkv_rope_w4a16(f32(x), [p[0].numpy() for p in projs], [p[1].float().numpy() for p in projs],
                                   [p[2].numpy() for p in projs], f32(gq), f32(gk), f32(cos), f32(sin), Hq, Hkv,
                                   positions=None if pos is None else pos.numpy(), round_weight=True)
    _check(out, ref, f"D=64 w4a16 B={B} S={S}")


@pytest.mark.parametrize("dtype,max_abs,rel_l2", [(torch.float32, 2e-4, 5e-6), (torch.float16, 4e-3, 1e-3)])
def test_f32_and_f16_fronts(dtype, max_abs, rel_l2, device):
    """The fp32 / fp16 front at head_dim 64 (bars of its head_dim-128 tests)."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    B, S, hidden, Hq, Hkv = 2, 40, 1024, 16, 8
    g = torch.Generator().manual_seed(73)
    x = torch.randn(B, S, hidden, generator=g)
    ws = [torch.randn(h * D, hidden, generator=g) * 0.02 for h in (Hq, Hkv, Hkv)]
    gq, gk = (1 + 0.1 * torch.randn(D, generator=g) for _ in range(2))
    cos, sin = mqk.rope_tables(D, S)
    args = [t.to(dtype) for t in (x, *ws, gq, gk, cos.float(), sin.float())]
    out = mqk.fused_qkv_rope(*(a.to(device) for a in args))
    assert all(o.dtype == dtype for o in out)
    ref = orc.fused_qkv_rope(*(a.float().numpy() for a in args))
    _check(out, ref, f"D=64 {dtype}", max_abs=max_abs, rel_l2=rel_l2)


def test_standalone_qk_norm_rope(device):
    """mqk.qk_norm_rope (the twin of _qk_norm_rope_kernel) on [B, S, H, 64]."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    B, S, Hq, Hkv = 3, 50, 16, 8
    g = torch.Generator().manual_seed(74)
    q = torch.randn(B, S, Hq, D, generator=g).bfloat16()
    k = torch.randn(B, S, Hkv, D, generator=g).bfloat16()
    gq, gk = ((1 + 0.1 * torch.randn(D, generator=g)).bfloat16() for _ in range(2))
    cos, sin = (t.bfloat16() for t in mqk.rope_tables(D, S))
    qo, ko = mqk.qk_norm_rope(q.to(device), k.to(device), gq.to(device), gk.to(device), cos.to(device),
                              sin.to(device))
    for name, o, raw, gam in (("q", qo, q, gq), ("k", ko, k, gk)):
        ref = orc.qk_norm_rope(f32(raw).reshape(B * S, -1, D), f32(gam), f32(cos), f32(sin), S)
        o = f32(o).reshape(ref.shape)
        ma, rl = orc.max_abs(o, ref), orc.rel_l2(o, ref)
        print(f"  D=64 norm_rope {name}: max_abs={ma:.5f} rel_l2={rl:.2e}")
        assert ma <= MAX_ABS and rl <= REL_L2


@pytest.mark.parametrize("S", [1, 100])
def test_paged_cache_write(S, device):
    """The fused paged-KV write at head_dim 64: cache [blocks, 16, Hkv, 64]; every
    addressed slot holds the returned K / V rows bit for bit, q / k / v equal
    the unpaged op."""
    import mqk
    from oracle import qkv_rope_oracle as orc
    B, hidden, Hq, Hkv, bs, nb = 2, 1024, 16, 8, 16, 64
    pos = None if S > 1 else torch.tensor([37, 400], dtype=torch.int32)
    case = Case(B, S, hidden, Hq, Hkv, seed=75 + S, rows=512, positions=pos, head_dim=D)
    args = case.args(device)
    kc = torch.zeros(nb, bs, Hkv, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    bt = torch.randperm(nb, generator=torch.Generator().manual_seed(S))[: B * 32].view(B, 32).to(torch.int32)
    kw = {}
    if pos is not None:
        seq, p = torch.arange(B, dtype=torch.int32), pos
        kw = dict(kv_seq=seq.to(device), kv_pos=p.to(device))
    else:
        seq = torch.arange(B * S) // S
        p = torch.arange(B * S) % S
    q, k, v = mqk.fused_qkv_rope_paged(*args[:8], kc, vc, bt.to(device), positions=args[8], **kw)
    ref = _run(case, device)
    for a, b in zip((q, k, v), ref):
        assert torch.equal(a, b)
    slots = torch.as_tensor(orc.paged_slot(bt.numpy(), seq.numpy(), p.numpy(), bs, nb))
    assert bool((slots >= 0).all())
    for cache, rows in ((kc, k), (vc, v)):
        flat = cache.view(-1, Hkv, D)
        assert torch.equal(flat[slots.to(device)], rows.reshape(-1, Hkv, D))


# ── shapes the kernels do not take fail cleanly ──────────────────────────────

@pytest.mark.parametrize("D_,Hq,Hkv,match", [(64, 15, 8, "even head counts"), (64, 16, 3, "even head counts"),
                                            (66, 8, 4, "head_dim 66 not supported"),
                                            (1024, 2, 1, "head_dim 1024 not supported")])
def test_unsupported_head_shapes(D_, Hq, Hkv, match, device):
    import mqk
    case = Case(1, 8, 1024, Hq, Hkv, seed=76, head_dim=D_)
    with pytest.raises(mqk.MqkNativeError, match=match):
        _run(case, device)
