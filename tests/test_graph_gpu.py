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


def _replay_checks(graph, outs, want, rerun):
    """Three replays, each compared with the eager result, eager work in between."""
    for _ in range(3):
        for t in outs:
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(outs, want))
        rerun()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("T", [32, 200])
def test_graph_replay_w4a16(T, device):
    """The W4A16 front (decode kernel at T = 32, tile + tail launches at T = 200)."""
    import mqk
    hidden, Hq, Hkv, D = 1024, 16, 8, 128
    g = torch.Generator().manual_seed(T)
    projs = []
    for h in (Hq, Hkv, Hkv):
        w = torch.randn(hidden, h * D, generator=g) * 0.02
        projs.append(tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w, 128, torch.float16)))
    x = torch.randn(1, T, hidden, generator=g).bfloat16().to(device)
    gq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    gk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(device)
    c, s = mqk.rope_tables(D, 4096)
    cos, sin = c.bfloat16().to(device), s.bfloat16().to(device)
    pos = torch.randint(0, 4096, (T,), generator=g, dtype=torch.int32).to(device)
    run = lambda: mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin, pos)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = run()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = run()
    _replay_checks(graph, out, eager, run)


def test_graph_replay_paged_input_norm_decode(device):
    """Decode step with the fused input RMSNorm (a pre-pass kernel writing the
    workspace) and the paged-KV-cache write: outputs and cache contents replay."""
    import mqk
    B, hidden, Hq, Hkv, D, bs = 24, 1024, 16, 8, 128, 16
    g = torch.Generator().manual_seed(77)
    case = Case(B, 1, hidden, Hq, Hkv, seed=77, rows=4096,
                positions=torch.randint(0, 4096, (B,), generator=g, dtype=torch.int32))
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    in_w = (1 + 0.1 * torch.randn(hidden, generator=g)).bfloat16().to(device)
    nblocks = B * 4096 // bs
    kc = torch.zeros(nblocks, bs, Hkv, D, dtype=torch.bfloat16, device=device)
    vc = torch.zeros_like(kc)
    bt = torch.arange(nblocks, dtype=torch.int32, device=device).view(B, 4096 // bs)
    kv_seq = torch.arange(B, dtype=torch.int32, device=device)

    def run():
        return mqk.fused_qkv_rope_ex(x, wq, wk, wv, gq, gk, cos, sin, pos, input_norm_w=in_w,
                                     k_cache=kc, v_cache=vc, block_table=bt, kv_seq=kv_seq, kv_pos=pos)

    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = run()
        stream.synchronize()
        eager_caches = (kc.clone(), vc.clone())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = run()
    _replay_checks(graph, tuple(out) + (kc, vc), tuple(eager) + eager_caches, run)
