"""Calls on many streams: no recompute path from the hardware queue's starting XCD.

Workgroups are dispatched round-robin over the XCDs, but the XCD that takes
workgroup 0 depends on the hardware queue behind the stream (measured on MI355X:
0, 5, 6 or 7 for different streams of one process, constant per queue).  The
decode and split-K tile kernels need all splits of a head (tile) on one XCD,
which round-robin dispatch gives whatever the starting XCD; they check exactly
that (sums of the splits' XCDs and their squares in the arrival word), so a
stream whose queue starts elsewhere must not send any head or tile down the
recompute path.  (A check against blockIdx % 8 once did, on 3 of 9 streams:
65 us per C3 call instead of 18.7.)
"""
from __future__ import annotations

import pytest
import torch

from conftest import Case

pytestmark = pytest.mark.gpu


def test_no_recompute_on_any_stream(device):
    import mqk
    pos = torch.randint(0, 8192, (512,), generator=torch.Generator().manual_seed(31), dtype=torch.int32)
    decode = Case(64, 1, 4096, 32, 8, seed=31, rows=8192, positions=pos[:64]).args(device)
    mid = Case(1, 512, 4096, 32, 8, seed=32, rows=8192, positions=pos).args(device)
    wide = Case(64, 1, 5120, 40, 8, seed=33, rows=8192, positions=pos[:64]).args(device)
    streams = [torch.cuda.Stream(device) for _ in range(10)]
    for i, st in enumerate(streams):
        with torch.cuda.stream(st):
            want = [mqk.fused_qkv_rope(*a) for a in (decode, mid, wide)]  # (workspaces sized)
            st.synchronize()
            before = mqk.decode_recomputes(device, st)
            got = [mqk.fused_qkv_rope(*a) for a in (decode, mid, wide) for _ in range(2)]
            after = mqk.decode_recomputes(device, st)
        assert after == before, f"stream {i}: {after - before} heads / tiles recomputed"
        for j, g in enumerate(got):
            assert all(torch.equal(a, b) for a, b in zip(g, want[j // 2]))
