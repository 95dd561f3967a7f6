"""Shared test setup: import paths, the ``gpu`` marker, seeded input builders."""
from __future__ import annotations

import re
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "mini-qwen-llm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HEAD_DIM = 128


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmqk.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def f32(t: torch.Tensor) -> np.ndarray:
    """Exact float32 values of a (bf16) tensor, on the host."""
    return t.detach().float().cpu().numpy()


class Case:
    """Seeded inputs of one fused_qkv_rope call (host copies; .to(dev) moves them)."""

    def __init__(self, B, S, hidden, Hq, Hkv, seed, *, rows=None, theta=1e6, gamma_ones=False,
                 positions=None, w_std=0.02, x_std=1.0, head_dim=HEAD_DIM):
        g = torch.Generator().manual_seed(seed)
        D = self.D = head_dim
        self.B, self.S, self.hidden, self.Hq, self.Hkv = B, S, hidden, Hq, Hkv
        self.x = (torch.randn(B, S, hidden, generator=g) * x_std).bfloat16()
        self.w_q = (torch.randn(Hq * D, hidden, generator=g) * w_std).bfloat16()
        self.w_k = (torch.randn(Hkv * D, hidden, generator=g) * w_std).bfloat16()
        self.w_v = (torch.randn(Hkv * D, hidden, generator=g) * w_std).bfloat16()
        if gamma_ones:
            self.q_norm_w = torch.ones(D).bfloat16()
            self.k_norm_w = torch.ones(D).bfloat16()
        else:
            self.q_norm_w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
            self.k_norm_w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
        from mqk.rope import rope_tables
        n_rows = rows if rows is not None else S
        cos, sin = rope_tables(D, n_rows, theta)
        self.cos, self.sin = cos.bfloat16(), sin.bfloat16()
        self.positions = positions

    def args(self, device):
        pos = None if self.positions is None else self.positions.to(device)
        return (self.x.to(device), self.w_q.to(device), self.w_k.to(device), self.w_v.to(device),
                self.q_norm_w.to(device), self.k_norm_w.to(device), self.cos.to(device),
                self.sin.to(device), pos)

    def oracle(self, token_idx=None, round_projection=False):
        """Oracle outputs (float64) for all tokens or the given flat token indices."""
        from oracle import qkv_rope_oracle as orc
        T = self.B * self.S
        x2 = f32(self.x).reshape(T, self.hidden)
        if self.positions is None:
            rows = np.arange(T) % self.S
        else:
            rows = self.positions.cpu().numpy().astype(np.int64)
        if token_idx is not None:
            x2 = x2[token_idx]
            rows = rows[token_idx]
        n = x2.shape[0]
        return orc.fused_qkv_rope(x2.reshape(1, n, self.hidden), f32(self.w_q), f32(self.w_k),
                                  f32(self.w_v), f32(self.q_norm_w), f32(self.k_norm_w),
                                  f32(self.cos), f32(self.sin), positions=rows,
                                  round_projection=round_projection)


@pytest.fixture(scope="session")
def device():
    return torch.device("cuda:0")


@pytest.fixture
def no_head_tiles():
    """Plan without single-head tiles, so a test of the decode-block or split-K
    launches keeps the call on the path it is about."""
    from mqk import _native
    _native.set_option("head_tiles", 0)
    yield
    _native.set_option("head_tiles", 1)


@pytest.fixture
def no_pair_tiles():
    """Plan without pair tiles (their 128-row form takes some mid token counts
    that the split-K launch runs otherwise), so a test of another launch keeps
    the call on the path it is about."""
    from mqk import _native
    _native.set_option("pair_tiles", 0)
    yield
    _native.set_option("pair_tiles", 1)


# Short names of the library's kernels, by (demangled or mangled) kernel name.
_KERNEL_NAMES = (("decode_multi_kernel", "decode_multi"), ("decode_long_kernel", "decode"), ("decode_kernel", "decode"),
                 ("tile_dma_w4_kernel", "tile_w4"), ("tile_dma_split_kernel", "tile_split"), ("tile_dma_kernel", "tile"), ("tile_kernel", "tile_reg"),
                 ("row_scale_kernel", "row_scale"), ("norm_rope_any_kernel", "norm_rope_any"), ("norm_rope_kernel", "norm_rope"),
                 ("f32_qkv_kernel", "f32"), ("w4_gemv", "gemv"))


def _short_kernel_name(name: str):
    if re.search(r"tile_dma_kernel(<\d+, \d+, \d+, \d+, \d+, \d+, 64>|I(Li\d+E){6}Li64EE)", name):
        return "tile_pair"  # pair tiles (256 x 192 or 256 x 320, two workgroups per 3 or 5 heads)
    if re.search(r"tile_dma_kernel(<\d+, 1,|ILi\d+ELi1E)", name):
        return "tile_head"  # single-head tiles (64 x 128 or 128 x 128)
    if re.search(r"tile_dma_w4_kernel(<\d+, 1,|ILi\d+ELi1E)", name):
        return "tile_w4_head"  # their int4 twins
    for key, short in _KERNEL_NAMES:
        if key in name:
            return short
    return None


def launched_kernels(fn, *, warm=True):
    """The library kernels one call of ``fn`` launches, in launch order, as
    short names ("decode" = one 64-row block, "decode_multi" = several blocks,
    "tile", "tile_head" = single-head tiles, "tile_pair" = pair tiles, "tile_split" = split-K tile, "tile_w4", "tile_w4_head", "tile_reg", "row_scale", "norm_rope",
    "f32" = the fp32 front, "gemv" = the small-M W4A16 GEMM), recorded with torch.profiler (the reference counts its
    kernels the same way, tests/test_fused_qkv_rope.py:287-311).  Other
    kernels (torch's own fills and copies) are left out."""
    from torch.profiler import ProfilerActivity, profile
    if warm:
        fn()  # workspace allocation and first-call set-up out of the recorded call
        torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    evs = [e for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    evs.sort(key=lambda e: e.time_range.start)
    names = [_short_kernel_name(e.name) for e in evs]
    return [n for n in names if n is not None]
