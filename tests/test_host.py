"""Host-side checks that need no GPU: the C ABI library loads and exports every
entry point include/mqk.h declares, argument validation returns the documented
error codes before anything is launched, the option knobs, the no-fallback
rule, and the torch-side format utilities against the oracle.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import qkv_rope_oracle as orc

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mqk.h"
LIB = ROOT / "mini-qwen-llm_amd" / "mqk" / "libmqk.so"

needs_lib = pytest.mark.skipif(not LIB.exists(), reason="libmqk.so not built (run __graft_entry__.build())")


def header_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mqk_[a-z0-9_]+)\s*\(", text)))


# ── symbols ───────────────────────────────────────────────────────────────────

def test_header_lists_expected_entry_points():
    names = header_functions()
    for n in ("mqk_fused_qkv_rope_bf16", "mqk_qk_norm_rope_bf16", "mqk_w4a16_gemm",
              "mqk_fused_qkv_rope_w4a16", "mqk_fused_qkv_rope_workspace_size"):
        assert n in names


@needs_lib
def test_library_exports_every_header_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, f"libmqk.so lacks {missing}"


@needs_lib
def test_ctypes_signatures_cover_header():
    from mqk import _native
    assert sorted(_native.SIGNATURES) == header_functions()


# ── calls that never reach a kernel ──────────────────────────────────────────

@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.skip("libmqk.so not built")
    from mqk import _native
    return _native.library()


def test_version_and_error_strings(lib):
    assert lib.mqk_version() >= 100
    for code, text in ((0, "ok"), (-1, "null"), (-2, "shape"), (-3, "unsupported"), (-4, "aligned"),
                       (-5, "workspace"), (-6, "HIP"), (-7, "option")):
        assert text in lib.mqk_error_string(code).decode()
    assert "unknown" in lib.mqk_error_string(-99).decode()


def _fused(lib, **kw):
    """Call mqk_fused_qkv_rope_bf16 with fake (never dereferenced) pointers."""
    fake = 1 << 20  # 16-byte aligned, never touched: every case fails validation first
    a = dict(x=fake, w_q=fake, w_k=fake, w_v=fake, q_gamma=fake, k_gamma=fake, cos=fake, sin=fake,
             positions=None, T=4, S=4, hidden=256, Hq=2, Hkv=1, D=128, cos_rows=4, eps=1e-6,
             q=fake, k=fake, v=fake, ws=None, ws_bytes=0, stream=None)
    a.update(kw)
    return lib.mqk_fused_qkv_rope_bf16(a["x"], a["w_q"], a["w_k"], a["w_v"], a["q_gamma"], a["k_gamma"],
                                       a["cos"], a["sin"], a["positions"], a["T"], a["S"], a["hidden"],
                                       a["Hq"], a["Hkv"], a["D"], a["cos_rows"], a["eps"], a["q"], a["k"],
                                       a["v"], a["ws"], a["ws_bytes"], a["stream"])


@pytest.mark.parametrize("kw,code,detail", [
    (dict(D=64), -3, "head_dim 64"),
    (dict(D=127), -2, "even"),
    (dict(hidden=96), -3, "multiple of 64"),
    (dict(T=-1), -2, "T >= 0"),
    (dict(Hkv=0), -2, "Hkv > 0"),
    (dict(x=None), -1, "x/q must"),
    (dict(v=None), -1, "x/q/k/v"),
    (dict(w_v=None), -1, "w_q/w_k/w_v"),
    (dict(cos=None), -1, "cos"),
    (dict(q=(1 << 20) + 2), -4, "aligned"),
    (dict(cos_rows=0), -2, "cos_rows"),
    (dict(S=0), -2, "S > 0"),
    (dict(eps=-1.0), -2, "eps"),
    (dict(Hq=1100), -3, "<= 1024"),
])
def test_fused_validation(lib, kw, code, detail):
    assert _fused(lib, **kw) == code
    assert detail in lib.mqk_last_error_detail().decode()


def test_fused_empty_is_noop(lib):
    assert _fused(lib, T=0, x=None, q=None, k=None, v=None) == 0
    assert lib.mqk_last_error_detail().decode() == ""


def test_decode_needs_workspace(lib):
    """T <= 64 routes to the split-K kernel, which needs its workspace."""
    assert _fused(lib, T=8, ws=None) == -5
    assert "workspace" in lib.mqk_last_error_detail().decode()


def test_head_tile_plan(lib):
    """With single-head tiles (the default) a bf16 call whose 64 x 128 or
    128 x 128 tiles fit one round over the CUs takes that launch and needs no
    workspace: T = 256 and 512 at Qwen3-8B dims (48 heads: 192 tiles), and
    hidden 2048 at T = 768 (40 heads, 6 x 40 = 240 tiles of 128 x 128).  At
    T = 1024 (8 x 48 = 384 single-head tiles, two rounds) one round of 128-row
    pair tiles takes the call (8 x 16 pairs of 2 x 128 x 192): the counters, then
    per pair 2 x 128 floats of row sums of squares and a 128 x 64 float hand-over
    area.  With pair tiles off, the split-K launch keeps it.  Further up, nearly a
    round of 192-row pairs takes T = 1536 (but not T = 1152, 7 workgroups per 8
    CUs), and 128 x 320 pairs take hidden 2048 with 40 heads at T = 2048."""
    from mqk import _native
    if _native.get_option("device_cus") != 256:
        pytest.skip("the plan depends on the device's CU count (256 on MI355X)")
    C = 4096 + 256 + 512 * 128
    part = 128 * 384 * 4
    _native.set_option("decode_blocks", 0)  # int4 then takes its tile kernel: no workspace
    try:
        assert lib.mqk_fused_qkv_rope_workspace_size(256, 32, 8, 4096) == 0
        assert lib.mqk_fused_qkv_rope_workspace_size(512, 32, 8, 4096) == 0
        assert lib.mqk_fused_qkv_rope_workspace_size(768, 32, 4, 2048) == 0
        assert lib.mqk_fused_qkv_rope_workspace_size(1024, 32, 8, 4096) == C + 128 * (2 * 128 + 128 * 64) * 4
        # T = 1536: 8 x 16 pairs of 192-row tiles (2 x 192 x 192 per 3 heads): per pair
        # 2 x 192 floats of sums and a 192 x 64 float hand-over area
        assert lib.mqk_fused_qkv_rope_workspace_size(1536, 32, 8, 4096) == C + 128 * (2 * 192 + 192 * 64) * 4
        # T = 1152 (7 workgroups per 8 CUs as 192-row pairs): whole-head tiles, no workspace
        assert lib.mqk_fused_qkv_rope_workspace_size(1152, 32, 8, 4096) == 0
        # hidden 2048 with 40 heads at T = 2048: 16 x 8 pairs of 128 x 320 tiles (2 x 128 floats
        # of sums and a 128 x 64 hand-over area each)
        assert lib.mqk_fused_qkv_rope_workspace_size(2048, 32, 4, 2048) == C + 128 * (2 * 128 + 128 * 64) * 4
        _native.set_option("pair_tiles", 0)
        assert lib.mqk_fused_qkv_rope_workspace_size(1024, 32, 8, 4096) == C + 128 * 2 * part
        assert lib.mqk_fused_qkv_rope_workspace_size(1536, 32, 8, 4096) == 0
    finally:
        _native.set_option("decode_blocks", 16)
        _native.set_option("pair_tiles", 1)


@pytest.mark.usefixtures("no_head_tiles")
def test_workspace_size(lib):
    from mqk import _native
    C = 4096 + 256 + 512 * 128  # 1024 arrival counters, the statistics line, a line per split-K tile
    # BASELINE config 4 (T = 8192, hidden 2048, 40 heads) in pair tiles of 2 x 256 x 320 per 5
    # heads: the counters (the pair words reuse the split-K tile lines), then per pair
    # 2 x 256 floats of row sums of squares and a 256 x 64 float hand-over area
    assert lib.mqk_fused_qkv_rope_workspace_size(8192, 32, 4, 2048) == C + 32 * 8 * (2 * 256 + 256 * 64) * 4
    # at most 512 pairs (one exchange word each in the counters' 512 tile lines): T = 16384
    # still runs as pairs, 16640 (520 pairs) as 256 x 256 tiles without a workspace
    assert lib.mqk_fused_qkv_rope_workspace_size(16384, 32, 4, 2048) == C + 512 * (2 * 256 + 256 * 64) * 4
    assert lib.mqk_fused_qkv_rope_workspace_size(16640, 32, 4, 2048) == 0
    _native.set_option("pair_tiles", 0)
    try:
        assert lib.mqk_fused_qkv_rope_workspace_size(8192, 32, 4, 2048) == 0   # tile kernel only
        assert lib.mqk_fused_qkv_rope_workspace_size(2048, 32, 8, 4096) == 0   # tile kernel only
    finally:
        _native.set_option("pair_tiles", 1)
    assert lib.mqk_fused_qkv_rope_workspace_size(0, 32, 8, 4096) == 0
    n = lib.mqk_fused_qkv_rope_workspace_size(64, 32, 8, 4096)
    assert n >= C + 48 * 64 * 128 * 4  # counters + at least one fp32 partial per head
    _native.set_option("tile_ksplit", 0)  # decode blocks or the one-workgroup-per-tile launch only
    try:
        # 64 < T: one decode launch covers every 64-row block; each block has its own
        # partials, so four blocks need four times the partial region
        assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 8, 4096) == C + 4 * (n - C)
        _native.set_option("decode_passes", 1)
        try:  # one block per launch: the launches share one block's region
            assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 8, 4096) == n
        finally:
            _native.set_option("decode_passes", 16)
        _native.set_option("decode_blocks", 0)
        try:
            assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 8, 4096) == 0
        finally:
            _native.set_option("decode_blocks", 16)
    finally:
        _native.set_option("tile_ksplit", 1)
    # Without decode blocks, bf16 T = 200 (2 x 16 tiles of 128 x 384) runs as a
    # split-K tile launch of 7 splits (the planner's model; 6 and 8 measured within
    # 1 us of each other): the counters, then one fp32 partial of a tile per
    # (tile, split); int4 takes the tile kernel, which needs none.
    _native.set_option("decode_blocks", 0)
    try:
        assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 8, 4096) == C + 32 * 7 * 128 * 384 * 4
        _native.set_option("tile_ksplit", 2)  # a forced split count
        try:
            assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 8, 4096) == C + 32 * 2 * 128 * 384 * 4
        finally:
            _native.set_option("tile_ksplit", 1)
        # 40 heads (no 3-head tiling): 1 x 20 tiles of 256 x 256 (8 row units each);
        # at hidden 2048 (32 stages) the model's best split count is 8
        assert lib.mqk_fused_qkv_rope_workspace_size(200, 32, 4, 2048) == C + 20 * 8 * 256 * 256 * 4
    finally:
        _native.set_option("decode_blocks", 16)


@pytest.mark.usefixtures("no_head_tiles")
@pytest.mark.usefixtures("no_pair_tiles")
def test_split_tile_plan(lib):
    """The planner's split-K tile model at Qwen3-8B dims (bf16 needs the split
    workspace; int4 keeps its decode blocks, so the size is the larger need):
    512 tokens as 4 x 16 tiles of 128 x 384 in 4 splits, 1024 tokens as 8 x 16
    tiles in 2 splits; both fit the CUs once (tiles x splits <= 256)."""
    from mqk import _native
    C = 4096 + 256 + 512 * 128
    part = 128 * 384 * 4  # one tile's fp32 partial
    _native.set_option("decode_blocks", 0)  # int4 then takes its tile kernel: no workspace
    try:
        assert lib.mqk_fused_qkv_rope_workspace_size(512, 32, 8, 4096) == C + 64 * 4 * part
        assert lib.mqk_fused_qkv_rope_workspace_size(1024, 32, 8, 4096) == C + 128 * 2 * part
        assert lib.mqk_fused_qkv_rope_workspace_size(2048, 32, 8, 4096) == 0  # 256 tiles: one each
        _native.set_option("tile_ksplit", 0)
        try:
            assert lib.mqk_fused_qkv_rope_workspace_size(512, 32, 8, 4096) == 0
        finally:
            _native.set_option("tile_ksplit", 1)
    finally:
        _native.set_option("decode_blocks", 16)


@pytest.mark.usefixtures("no_head_tiles")
def test_split_tile_plan_other_shapes(lib):
    """The split-K model for 256 x 256 tiles, refitted on MI355X measurements at
    hidden 1024 / 2048 / 5120: the split counts it picks (shown by the partials'
    size) are the fastest measured, or within ~2 us of it.  Hidden 5120 (Qwen3-14B
    heads) at T = 768 / 1024: 2 splits, 86.7 / 94.6 us against 110.5 / 117.2 us for
    one tile per workgroup; hidden 2048 (30B-A3B heads) at T = 512: 4 splits,
    32.7 us against 42.0 us for decode blocks."""
    from mqk import _native
    C = 4096 + 256 + 512 * 128
    part = 256 * 256 * 4
    size = lambda T, hq, hkv, h: lib.mqk_fused_qkv_rope_workspace_size(T, hq, hkv, h)
    _native.set_option("decode_blocks", 0)  # int4 then takes its tile kernel: no workspace
    try:
        for T, hq, hkv, h, tiles, s in ((128, 32, 4, 2048, 20, 8), (512, 32, 4, 2048, 40, 4),
                                        (768, 32, 4, 2048, 60, 4), (1024, 32, 4, 2048, 80, 3),
                                        (128, 40, 8, 5120, 28, 8), (512, 40, 8, 5120, 56, 4),
                                        (768, 40, 8, 5120, 84, 2), (1024, 40, 8, 5120, 112, 2),
                                        (256, 16, 8, 1024, 16, 4)):
            assert size(T, hq, hkv, h) == C + tiles * s * part, (T, h)
        for T, hq, hkv, h in ((1536, 32, 4, 2048), (1536, 40, 8, 5120), (1024, 16, 8, 1024)):
            assert size(T, hq, hkv, h) == 0, (T, h)  # one tile per workgroup
    finally:
        _native.set_option("decode_blocks", 16)


def test_decode_block_crossovers(lib):
    """The plan's cost model reproduces the crossovers measured on MI355X at hidden
    4096 (Qwen3-8B heads): a workspace is needed exactly when decode launches run.
    int4 runs as decode blocks up to T = 1024 (92 us against 138 for the tile
    kernel), and beyond sixteen blocks (T > 1024) it runs the tile kernel.  One
    launch covers every block, each with its own partials.  (bf16 takes the
    split-K tile launch from T ~ 400, whose partials are smaller; the size is the
    larger of the two formats' needs.)"""
    from mqk import _native
    size = lambda T: lib.mqk_fused_qkv_rope_workspace_size(T, 32, 8, 4096)
    C = 4096 + 256 + 512 * 128  # arrival counters, the statistics line, a line per split-K tile
    one = size(64) - C  # partials of one 64-row block
    for T in (128, 512, 768, 896, 1024):
        assert size(T) == C + (T // 64) * one, T
    assert size(1088) == 0
    _native.set_option("decode_passes", 4)
    _native.set_option("tile_ksplit", 0)  # (bf16's split-K partials at T = 1024 exceed four blocks')
    try:  # at most four blocks per launch: the launches reuse four blocks' partials
        assert size(1024) == C + 4 * one
    finally:
        _native.set_option("decode_passes", 16)
        _native.set_option("tile_ksplit", 1)


def test_w4a16_validation(lib):
    fake = 1 << 20
    call = lambda M=4, K=256, N=64, g=128, st=0, qw=fake: lib.mqk_w4a16_gemm(
        fake, qw, fake, fake, M, K, N, g, st, fake, None)
    assert call(N=12) == -2
    assert call(g=96) == -2         # K % group
    assert call(st=5) == -2
    assert call(qw=None) == -1
    assert call(K=96, g=32) == -3
    assert call(M=0) == 0


def test_f32_validation(lib):
    """The fp32 entry point's checks run before any launch (fake pointers)."""
    fake = 1 << 20
    f = lambda T=4, hidden=1024, D=128, x=fake, q=fake, wq=fake, cr=8, S=4: lib.mqk_fused_qkv_rope_f32(
        x, wq, fake, fake, fake, fake, fake, fake, None, T, S, hidden, 2, 1, D, cr, 1e-6, q, fake, fake, None)
    assert f(D=96) == -3
    assert f(D=127) == -2
    assert f(hidden=48) == -3      # hidden % 32
    assert f(x=None) == -1
    assert f(wq=None) == -1
    assert f(q=fake + 4) == -4
    assert f(cr=0) == -2
    assert f(S=0) == -2            # prefill mode needs S
    assert f(T=0) == 0
    assert f(T=-1) == -2


def test_qk_norm_rope_validation(lib):
    fake = 1 << 20
    f = lambda T=4, Hq=2, Hkv=1, D=128, qr=fake: lib.mqk_qk_norm_rope_bf16(
        qr, fake, fake, fake, fake, fake, None, T, 4, Hq, Hkv, D, 4, 1e-6, fake, fake, None)
    assert f(D=96) == -3
    assert f(qr=None) == -1
    assert f(T=0) == 0
    assert f(Hq=0, Hkv=0) == 0


def test_options_roundtrip(lib):
    from mqk import _native
    assert _native.get_option("decode_max_t") == 64
    for name, val in (("prefill_tile", 11), ("decode_max_t", 16), ("decode_splits", 4), ("group_m", 8),
                      ("decode_force_recompute", 1), ("decode_blocks", 3), ("tail_split", 0)):
        old = _native.get_option(name)
        _native.set_option(name, val)
        assert _native.get_option(name) == val
        _native.set_option(name, old)
    with pytest.raises(_native.MqkNativeError, match="unknown prefill_tile"):
        _native.set_option("prefill_tile", 999)
    with pytest.raises(_native.MqkNativeError, match="unknown option"):
        _native.set_option("no_such_knob", 1)
    assert _native.get_option("no_such_knob") == -1
    assert re.fullmatch(r"(\d+:\d+x\d+/\d+w;?)+", _native.tile_variants())


def test_missing_library_fails_loudly(tmp_path):
    """No fallback: pointing the loader at a missing library raises on use."""
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import torch, mqk\n"
            "x = torch.zeros(1, 2, 128, dtype=torch.bfloat16)\n"
            "try:\n"
            "    mqk.version()\n"
            "except mqk.MqkNativeError as e:\n"
            "    print('RAISED', e)\n") % str(ROOT / "mini-qwen-llm_amd")
    env = {"MQK_LIBRARY": str(tmp_path / "nope.so"), "PATH": "/usr/bin:/bin",
           "HOME": str(tmp_path)}
    import os
    env = {**os.environ, **env}
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert "RAISED" in r.stdout and "not found" in r.stdout, r.stdout + r.stderr


def test_fused_op_rejects_cpu_tensors():
    """The Python drop-in never computes on the host."""
    import mqk
    from mqk import _native
    x = torch.zeros(1, 4, 256, dtype=torch.bfloat16)
    w = torch.zeros(256, 256, dtype=torch.bfloat16)
    wk = torch.zeros(128, 256, dtype=torch.bfloat16)
    g = torch.ones(128, dtype=torch.bfloat16)
    c = torch.ones(4, 128, dtype=torch.bfloat16)
    with pytest.raises((ValueError, RuntimeError, _native.MqkNativeError)):
        mqk.fused_qkv_rope(x, w, wk, wk, g, g, c, c)


# ── torch host utilities vs the oracle ────────────────────────────────────────

def test_torch_rope_tables_match_oracle():
    import mqk
    for theta in (1e6, 1e4):
        c, s = mqk.rope_tables(128, 4096, theta)
        oc, os_ = orc.rope_tables(128, 4096, theta)
        # same fp32 operation sequence; torch's and numpy's pow/cos/sin may differ
        # by an ulp, i.e. an angle error of ~|angle| * 2^-23
        tol = np.arange(4096, dtype=np.float64)[:, None] * 2.0 ** -22 + 2e-6
        assert np.all(np.abs(c.numpy() - oc) <= tol) and np.all(np.abs(s.numpy() - os_) <= tol)


def test_torch_rotary_rows_and_apply():
    import mqk
    rope = mqk.RotaryEmbedding(128, 64)
    pos = torch.tensor([5, 0, 63])
    c, s = rope.rows(pos, torch.float32)
    assert torch.equal(c, rope.cos_cached[pos])
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 64, 2, 128)).astype(np.float32)
    cc, ss = rope(64)
    qo, _ = mqk.apply_rotary_emb(torch.from_numpy(q), torch.from_numpy(q), cc, ss)
    ref = orc.rope(q.reshape(64, 2, 128), cc.numpy(), ss.numpy()).reshape(1, 64, 2, 128)
    np.testing.assert_allclose(qo.numpy(), ref, atol=1e-5)


def test_torch_pack_matches_oracle():
    import mqk
    rng = np.random.default_rng(1)
    v = rng.integers(0, 16, (64, 256))
    t = mqk.pack_int4(torch.from_numpy(v))
    assert np.array_equal(t.numpy(), orc.pack_int4(v))
    assert np.array_equal(mqk.unpack_int4(t).numpy(), v)


def test_torch_quantizer_matches_oracle():
    import mqk
    rng = np.random.default_rng(2)
    w = rng.standard_normal((512, 64)).astype(np.float32)
    qw, sc, qz = mqk.per_group_minmax_quantize(torch.from_numpy(w), 128)
    oqw, osc, oqz = orc.minmax_quantize(w, 128)
    assert np.array_equal(qw.numpy(), oqw) and np.array_equal(qz.numpy(), oqz)
    assert np.array_equal(sc.view(torch.int16).numpy().view(np.uint16), osc)
    deq = mqk.dequantize(qw, sc, qz, 128).numpy()
    np.testing.assert_array_equal(deq, orc.dequant(oqw, orc.bf16_to_f32(osc), oqz, 128))


def test_torch_gptq_fix_matches_oracle():
    import mqk
    z = np.random.default_rng(3).integers(0, 16, (4, 32))
    pz = orc.pack_int4(z)
    assert np.array_equal(mqk.gptq_zero_fix(torch.from_numpy(pz)).numpy(), orc.gptq_zero_fix(pz))


# ── AutoAWQ ingest (format conversion, exact) ─────────────────────────────────

def test_autoawq_known_answer():
    """One 8-column group with column c holding value c: AutoAWQ packs nibble i =
    column AWQ_ORDER[i] = (0,2,4,6,1,3,5,7)[i], i.e. the word 0x75316420."""
    import mqk
    word = torch.tensor([[0x75316420]], dtype=torch.int32).repeat(8, 1)   # K = 8 rows, N = 8
    zeros = torch.tensor([[0x75316420]], dtype=torch.int32)                # one group
    scales = torch.full((1, 8), 0.5, dtype=torch.float16)
    qw, sc, qz = mqk.from_autoawq(word, zeros, scales)
    w = mqk.unpack_int4(qw.T.contiguous()).T                               # [K, N]
    assert torch.equal(w, torch.arange(8, dtype=torch.int32).repeat(8, 1))
    assert torch.equal(mqk.unpack_int4(qz), torch.arange(8, dtype=torch.int32)[None])
    assert sc.dtype == torch.float16 and torch.equal(sc, scales)


def test_autoawq_roundtrip_dequant_equal():
    """Repacking keeps every integer: dequant of the repacked triple equals the
    dequant read directly from the AutoAWQ words."""
    import mqk
    from mqk.quantization import AWQ_ORDER
    rng = np.random.default_rng(5)
    K, N, g = 256, 64, 128
    W = rng.integers(0, 16, (K, N))
    Z = rng.integers(0, 16, (K // g, N))
    def awq_pack(v):                     # independent restatement of the AutoAWQ packer
        out = np.zeros((v.shape[0], v.shape[1] // 8), dtype=np.uint32)
        for col in range(v.shape[1] // 8):
            for i, c in enumerate(AWQ_ORDER):
                out[:, col] |= (v[:, col * 8 + c].astype(np.uint32) << np.uint32(4 * i))
        return torch.from_numpy(out.view(np.int32))
    s = torch.from_numpy(rng.uniform(0.01, 0.02, (K // g, N)).astype(np.float16))
    qw, sc, qz = mqk.from_autoawq(awq_pack(W), awq_pack(Z), s)
    deq = mqk.dequantize(qw, sc, qz, g).numpy()
    ref = (W - np.repeat(Z, g, axis=0)).astype(np.float32) * np.repeat(s.float().numpy(), g, axis=0)
    np.testing.assert_array_equal(deq, ref)


def test_paged_validation(lib):
    """mqk_fused_qkv_rope_paged_bf16 argument checks (fake pointers, never launched)."""
    import ctypes
    from mqk import _native
    fake = 1 << 20

    def call(kv, positions=None, T=100, k=fake):
        return lib.mqk_fused_qkv_rope_paged_bf16(
            fake, fake, fake, fake, fake, fake, fake, fake, positions, T, 100, 256, 2, 1, 128, 100, 1e-6,
            fake, k, fake, kv, None, 0, None)

    good = dict(k_cache=fake, v_cache=fake, block_table=fake, bt_rows=1, bt_cols=8, num_blocks=8,
                block_size=16, kv_seq=None, kv_pos=None)
    def desc(**kw):
        d = dict(good); d.update(kw)
        return ctypes.byref(_native.PagedKV(**d))
    assert call(None) == -1 and "descriptor" in lib.mqk_last_error_detail().decode()
    assert call(desc(k_cache=None)) == -1
    assert call(desc(v_cache=fake + 8)) == -4
    assert call(desc(block_size=0)) == -2
    assert call(desc(), positions=fake) == -1
    assert "kv_seq" in lib.mqk_last_error_detail().decode()
    assert call(desc(), T=0) == 0


def test_ext_validation(lib):
    """mqk_fused_qkv_rope_ex_bf16 checks of the optional features (fake pointers,
    never launched) and the input-norm workspace size."""
    import ctypes
    from mqk import _native
    fake = 1 << 20

    def call(ext, positions=None, T=100, S=100):
        return lib.mqk_fused_qkv_rope_ex_bf16(
            fake, fake, fake, fake, fake, fake, fake, fake, positions, T, S, 256, 2, 1, 128, 100, 1e-6,
            fake, fake, fake, None if ext is None else ctypes.byref(ext), None, 0, None)

    assert call(_native.FusedExt(), T=0) == 0
    assert call(_native.FusedExt(cu_seqlens=fake, n_seqs=3), positions=fake) == -2
    assert "exclusive" in lib.mqk_last_error_detail().decode()
    assert call(_native.FusedExt(cu_seqlens=fake, n_seqs=0)) == -2
    assert call(_native.FusedExt(seq_pos0=fake)) == -2
    assert "cu_seqlens" in lib.mqk_last_error_detail().decode()
    # prefill mode without varlen still needs S > 0
    assert call(_native.FusedExt(), S=0) == -2 and "S > 0" in lib.mqk_last_error_detail().decode()
    assert call(_native.FusedExt(in_gamma=fake + 2, in_eps=1e-6)) == -4
    assert call(_native.FusedExt(in_gamma=fake, in_eps=-1.0)) == -2
    plain = lib.mqk_fused_qkv_rope_ex_workspace_size(1000, 32, 8, 4096, None)
    assert plain == lib.mqk_fused_qkv_rope_workspace_size(1000, 32, 8, 4096)
    normed = lib.mqk_fused_qkv_rope_ex_workspace_size(1000, 32, 8, 4096,
                                                       ctypes.byref(_native.FusedExt(in_gamma=fake)))
    assert normed >= plain + 4000


def test_native_call_makes_the_tensor_device_current(monkeypatch):
    """libmqk launches on the current HIP device: every launch goes through
    _native.call, which enters torch.cuda.device(<the tensors' device>) around it
    when another device is current, and calls straight through otherwise."""
    from mqk import _native
    seen = []
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)

    class Recorder:
        def __init__(self, dev):
            self.dev = dev

        def __enter__(self):
            seen.append(("enter", str(self.dev)))

        def __exit__(self, *exc):
            seen.append(("exit", str(self.dev)))

    monkeypatch.setattr(torch.cuda, "device", Recorder)
    r = _native.call(torch.device("cuda", 1), lambda a, b: seen.append(("launch", a, b)) or 7, 3, 4)
    assert r == 7
    assert seen == [("enter", "cuda:1"), ("launch", 3, 4), ("exit", "cuda:1")]
    seen.clear()
    assert _native.call(torch.device("cuda", 0), lambda a: seen.append(("launch", a)) or 8, 5) == 8
    assert seen == [("launch", 5)]


def test_every_launch_goes_through_native_call():
    """No entry point that launches kernels is called directly from the package."""
    import re
    pkg = ROOT / "mini-qwen-llm_amd" / "mqk"
    launching = re.compile(
        r"\.(mqk_fused_qkv_rope(_paged|_ex)?_(bf16|w4a16|f32)|mqk_w4a16_gemm(_ex)?|mqk_qk_norm_rope_bf16)\b")
    launches = 0
    for f in pkg.glob("*.py"):
        if f.name == "_native.py":  # the ctypes signature table names every entry point
            continue
        for ln in f.read_text().splitlines():
            if launching.search(ln) and not ln.strip().startswith(("#", '"')):
                launches += 1
                assert "_native.call(device, " in ln or ln.strip().startswith("device, lib."), f"{f.name}: {ln.strip()}"
    assert launches >= 8  # bf16 / paged / ex / qk-norm, int4 GEMM / plain / paged / ex


def test_stream_handle_falls_back_to_the_public_api(monkeypatch):
    """Without torch's raw-stream accessor the handle comes from
    torch.cuda.current_stream(device).cuda_stream."""
    from mqk import _native

    class FakeStream:
        cuda_stream = 12345

    monkeypatch.setattr(_native, "_raw_stream", None)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda dev=None: FakeStream())
    assert _native.stream_handle(torch.device("cuda", 0)) == 12345
    monkeypatch.setattr(_native, "_raw_stream", lambda idx: 777 + idx)
    assert _native.stream_handle(torch.device("cuda", 1)) == 778


def test_f16_validation(lib):
    """The fp16 entry point's checks run before any launch (fake pointers)."""
    fake = 1 << 20
    f = lambda T=4, hidden=1024, D=128, x=fake: lib.mqk_fused_qkv_rope_f16(
        x, fake, fake, fake, fake, fake, fake, fake, None, T, 4, hidden, 2, 1, D, 8, 1e-6, fake, fake, fake, None)
    assert f(D=96) == -3
    assert f(hidden=48) == -3
    assert f(x=None) == -1
    assert f(T=0) == 0


def test_workspace_size_any_head_dim(lib):
    """mqk_fused_qkv_rope_workspace_size_hd: at head_dim 128 and 64 the fused
    plan's bytes over 128-column blocks; at other head sizes what the three
    projections' own plans need (the decode kernel's counters and partials at
    decode sizes, none where single-head tiles take every projection)."""
    from mqk import _native
    for T in (1, 8, 256, 2048):
        assert lib.mqk_fused_qkv_rope_workspace_size_hd(T, 32, 8, 4096, 128) == \
            lib.mqk_fused_qkv_rope_workspace_size(T, 32, 8, 4096)
        assert lib.mqk_fused_qkv_rope_workspace_size_hd(T, 32, 8, 4096, 64) == \
            lib.mqk_fused_qkv_rope_workspace_size(T, 16, 4, 4096)
    assert lib.mqk_fused_qkv_rope_workspace_size_hd(0, 16, 4, 4096, 256) == 0
    assert lib.mqk_fused_qkv_rope_workspace_size_hd(8, 16, 4, 4000, 256) == 0  # hidden % 64 != 0
    if _native.get_option("device_cus") != 256:
        pytest.skip("the plan depends on the device's CU count (256 on MI355X)")
    # T = 8, head_dim 256: each projection runs on the split-K decode kernel, whose
    # counters and partials the workspace holds
    n = lib.mqk_fused_qkv_rope_workspace_size_hd(8, 16, 4, 4096, 256)
    assert n >= 4096 + 256 + 512 * 128
    # the Python front takes the larger of the fused and the per-projection sizes
    assert _native.fused_workspace_bytes(8, 16, 4, 4096, 256) >= n
    assert _native.fused_workspace_bytes(8, 32, 8, 4096, 128) == lib.mqk_fused_qkv_rope_workspace_size(8, 32, 8, 4096)
