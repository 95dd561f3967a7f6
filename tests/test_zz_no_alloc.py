"""mqk_fused_qkv_rope_bf16_noalloc (the entry point that allocates nothing)
against mqk_fused_qkv_rope_bf16 with a caller workspace, through the C ABI.

Both run the same kernels on the same inputs, so their outputs must be equal
bit for bit (integer-exact comparison of the bf16 patterns), on consecutive
calls whose sizes shrink (the fixed scratch keeps the previous call's partials;
only its counters must be zero at a call's start, and every call leaves them
so).  A call too large for the fixed scratch is rejected before any launch.
"""
from __future__ import annotations

import pytest
import torch

from conftest import Case

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _run(entry, case, device, with_ws):
    from mqk import _native
    lib = _native.library()
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    B, S, H = x.shape
    T = B * S
    D = 128
    q = torch.full((T, case.Hq, D), -7.0, dtype=torch.bfloat16, device=device)
    k = torch.full((T, case.Hkv, D), -7.0, dtype=torch.bfloat16, device=device)
    v = torch.full((T, case.Hkv, D), -7.0, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.current_stream(device)
    common = (x.data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(), gq.data_ptr(), gk.data_ptr(),
              cos.data_ptr(), sin.data_ptr(), _native.ptr(pos), T, S, H, case.Hq, case.Hkv, D,
              cos.shape[0], EPS, q.data_ptr(), k.data_ptr(), v.data_ptr())
    if with_ws:
        n = int(lib.mqk_fused_qkv_rope_workspace_size(T, case.Hq, case.Hkv, H))
        ws = _native.workspace(device, stream, n)
        st = entry(*common, _native.ptr(ws), 0 if ws is None else ws.numel(), stream.cuda_stream)
    else:
        st = entry(*common, stream.cuda_stream)
    return st, (q, k, v)


def _pair(case, device):
    from mqk import _native
    lib = _native.library()
    st, want = _run(lib.mqk_fused_qkv_rope_bf16, case, device, True)
    _native.check(st, "mqk_fused_qkv_rope_bf16")
    st, got = _run(lib.mqk_fused_qkv_rope_bf16_noalloc, case, device, False)
    _native.check(st, "mqk_fused_qkv_rope_bf16_noalloc")
    torch.cuda.synchronize()
    for name, a, b in zip("qkv", got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{name} differs"


def _decode_case(B, seed, hidden=4096, Hq=32, Hkv=8):
    pos = torch.randint(0, 8192, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    return Case(B, 1, hidden, Hq, Hkv, seed=seed, rows=8192, positions=pos)


def test_noalloc_decode_then_smaller_decode(device):
    """BASELINE config 3 (64 tokens, Qwen3-8B heads), then 16 tokens."""
    _pair(_decode_case(64, 501), device)
    _pair(_decode_case(16, 502), device)


def test_noalloc_mid_t_then_single_token(device):
    """256 tokens (decode launches of one 64-row block each: the four-block
    launch needs more than the fixed scratch), then a single token.  The split-K
    tile launch, which the workspace entry point would take at this size, is off:
    its partials exceed the fixed scratch, so the allocation-free entry point
    plans without it and the two would not run the same kernels."""
    from mqk import _native
    _native.set_option("tile_ksplit", 0)
    try:
        _pair(Case(1, 256, 4096, 32, 8, seed=503), device)
    finally:
        _native.set_option("tile_ksplit", 1)
    _pair(_decode_case(1, 504), device)


def test_noalloc_prefill_then_decode(device):
    """A tile launch (which needs no scratch), then a decode step
    at hidden 1024."""
    _pair(Case(2, 600, 1024, 16, 8, seed=505), device)
    _pair(_decode_case(40, 506, hidden=1024, Hq=16, Hkv=8), device)


def test_noalloc_wide_model_decode(device):
    """Qwen3-14B heads at hidden 5120 (the decode launch with splits of two x
    slices: 56 heads x 4 splits, 7 MiB of partials, within the fixed scratch),
    then a smaller call."""
    _pair(_decode_case(64, 508, hidden=5120, Hq=40, Hkv=8), device)
    _pair(_decode_case(9, 509, hidden=5120, Hq=40, Hkv=8), device)


def test_noalloc_rejects_oversized_decode(device):
    """1024 heads at hidden 1024: one split each, 32 MiB of partials: rejected
    with MQK_ERR_WORKSPACE before any launch; the outputs stay untouched."""
    from mqk import _native
    lib = _native.library()
    case = _decode_case(2, 507, hidden=1024, Hq=512, Hkv=256)
    st, out = _run(lib.mqk_fused_qkv_rope_bf16_noalloc, case, device, False)
    assert st == -5
    assert b"fixed scratch" in lib.mqk_last_error_detail()
    torch.cuda.synchronize()
    assert all(bool((t == -7.0).all()) for t in out)
