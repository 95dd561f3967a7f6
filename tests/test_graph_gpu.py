"""HIP-graph capture of the fused ops (the serving loop's replay path).

The decode kernel's arrival counters are left at zero by every launch and no
memset is recorded, so a captured launch replays correctly.  Each replay is
compared with the eager result, with eager work and synchronisations between
the replays (graph nodes that misbehave only on replays after the first are
caught that way).
"""
from __future__ import annotations

import pytest
import torch

from conftest import Case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,S", [(64, 1), (8, 1), (2, 300)])
def test_graph_replay_matches_eager(B, S, device):
    import mqk
    case = Case(B, S, 1024, 16, 8, seed=990 + B + S, rows=4096,
                positions=torch.randint(0, 4096, (B * S,), generator=torch.Generator().manual_seed(B),
                                        dtype=torch.int32))
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)  # also creates the workspace
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
    for _ in range(3):
        for t in out:
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager))
        mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)  # eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_new_inputs(device):
    """Replays read the captured input buffers: new values copied in give new outputs."""
    import mqk
    case = Case(16, 1, 1024, 16, 8, seed=995, rows=4096, positions=torch.arange(16, dtype=torch.int32) * 7)
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
    for seed in range(3):
        g = torch.Generator(device=device).manual_seed(seed)
        x.copy_(torch.randn(x.shape, generator=g, device=device).bfloat16())
        graph.replay()
        torch.cuda.synchronize()
        want = mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, want))


def test_two_streams_concurrently(device):
    """Calls on two streams may overlap: each stream gets its own workspace (the
    decode kernel's counters and partials), so concurrent decode steps stay correct."""
    import mqk
    cases = [Case(64, 1, 1024, 16, 8, seed=1001 + i, rows=4096,
                  positions=torch.randint(0, 4096, (64,), generator=torch.Generator().manual_seed(i),
                                          dtype=torch.int32)) for i in range(2)]
    args = [c.args(device) for c in cases]
    want = [mqk.fused_qkv_rope(*a) for a in args]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device) for _ in range(2)]
    outs = [[], []]
    for rep in range(20):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                outs[i].append(mqk.fused_qkv_rope(*args[i]))
    torch.cuda.synchronize()
    for i in range(2):
        for o in outs[i]:
            assert all(torch.equal(a, b) for a, b in zip(o, want[i]))
