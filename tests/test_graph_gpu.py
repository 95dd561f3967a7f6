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


@pytest.mark.parametrize("int4", [False, True])
def test_graph_replay_long_split_decode(int4, device):
    """A decode step at Qwen3-14B dims (splits of two x slices, `decode_long_kernel`)
    captured and replayed, bf16 and int4 weights."""
    import mqk
    from conftest import launched_kernels
    case = Case(32, 1, 5120, 40, 8, seed=1990 + int4, rows=4096,
                positions=torch.randint(0, 4096, (32,), generator=torch.Generator().manual_seed(7), dtype=torch.int32))
    x, wq, wk, wv, gq, gk, cos, sin, pos = case.args(device)
    if int4:
        projs = [tuple(t.to(device) for t in mqk.per_group_minmax_quantize(w.float().T.contiguous(), 128,
                                                                            torch.bfloat16))
                 for w in (case.w_q, case.w_k, case.w_v)]
        call = lambda: mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin, pos)
    else:
        call = lambda: mqk.fused_qkv_rope(x, wq, wk, wv, gq, gk, cos, sin, pos)
    assert launched_kernels(call) == ["decode"]
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = call()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = call()
    for _ in range(3):
        for t in out:
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager))
        call()  # eager work between replays
        torch.cuda.synchronize()


def test_graph_replay_split_tile(device):
    """The split-K tile launch (a bf16 call of 512 tokens at hidden 4096) in a graph:
    its arrival and exit words are re-armed by the launch itself, so replays, with
    eager calls of the same and of another plan in between, stay bit-exact."""
    import mqk
    from conftest import launched_kernels
    T = 512
    case = Case(1, T, 4096, 32, 8, seed=997, rows=8192,
                positions=torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(4), dtype=torch.int32))
    args = case.args(device)
    small = Case(1, 64, 4096, 32, 8, seed=998, rows=8192,
                 positions=torch.arange(64, dtype=torch.int32)).args(device)
    mqk.set_option("head_tiles", 0)  # (one round of single-head tiles would take this call)
    try:
        _replay_split_tile(mqk, launched_kernels, args, small, device)
    finally:
        mqk.set_option("head_tiles", 1)


def _replay_split_tile(mqk, launched_kernels, args, small, device):
    assert launched_kernels(lambda: mqk.fused_qkv_rope(*args)) == ["tile_split"]
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = mqk.fused_qkv_rope(*args)  # also sizes the stream's workspace
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = mqk.fused_qkv_rope(*args)
    for rep in range(4):
        for t in out:
            t.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager)), f"replay {rep}"
        with torch.cuda.stream(stream):  # eager work on the graph's stream (same workspace)
            mqk.fused_qkv_rope(*small)
            mqk.fused_qkv_rope(*args)
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


@pytest.mark.parametrize("T,head_tiles,plan", [(32, 1, ["decode"]), (200, 1, ["tile_w4_head"]),
                                               (200, 0, ["decode_multi"]), (4128, 1, ["tile_w4", "decode"])])
def test_graph_replay_w4a16(T, head_tiles, plan, device):
    """The W4A16 front under capture, one case per launch plan: the decode kernel
    (T = 32), one round of int4 single-head tiles (T = 200, the default plan),
    one four-block decode launch (T = 200 without single-head tiles), and the tile
    launch plus the decode-kernel tail launch (T = 4128 = 16 row tiles of 256 +
    32 rows, whose 17th row tile would cost a second round over the CUs).  The
    plan is checked from the kernels the eager call launches."""
    import mqk
    from conftest import launched_kernels
    run = _w4a16_case(T, device)
    mqk.set_option("head_tiles", head_tiles)
    try:
        assert launched_kernels(run) == plan
        _graph_replay(run, device)
    finally:
        mqk.set_option("head_tiles", 1)


def _w4a16_case(T, device):
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
    return lambda: mqk.fused_qkv_rope_w4a16(x, *projs, gq, gk, cos, sin, pos)


def _graph_replay(run, device):
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = run()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = run()
    _replay_checks(graph, out, eager, run)


@pytest.mark.usefixtures("no_head_tiles")
def test_graph_survives_workspace_growth(device):
    """A graph captured with a small workspace replays correctly after a later
    eager call on the same stream needed a larger one.

    The decode step (T = 64) is captured with the one-block workspace; an eager
    T = 256 call (one four-block decode launch) then needs four times the
    partials.  The stream gets a new workspace and the old one stays allocated,
    so the replayed decode kernel still writes its partials and counters into
    memory nothing else owns.  Freed and refilled allocator blocks would expose a
    replay into released memory: stale counters would leave no finisher, and the
    outputs would keep the zeros written before each replay."""
    import mqk
    from mqk import _native
    hidden, Hq, Hkv = 1024, 16, 8
    small = Case(64, 1, hidden, Hq, Hkv, seed=4242, rows=4096,
                 positions=torch.randint(0, 4096, (64,), generator=torch.Generator().manual_seed(1),
                                         dtype=torch.int32))
    big = Case(1, 256, hidden, Hq, Hkv, seed=4243)
    lib = _native.library()
    assert lib.mqk_fused_qkv_rope_workspace_size(256, Hq, Hkv, hidden) > \
        2 * lib.mqk_fused_qkv_rope_workspace_size(64, Hq, Hkv, hidden)
    a_small, a_big = small.args(device), big.args(device)
    stream = torch.cuda.Stream(device)
    with torch.cuda.stream(stream):
        eager = mqk.fused_qkv_rope(*a_small)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = mqk.fused_qkv_rope(*a_small)
        retired = _native.retired_workspaces()
        want_big = mqk.fused_qkv_rope(*a_big)  # grows this stream's workspace
        stream.synchronize()
    assert _native.retired_workspaces() == retired + 1
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 22,), -1, dtype=torch.int32, device=device) for _ in range(16)]
    for rep in range(3):
        for t in out:
            t.fill_(0)
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager)), f"replay {rep}"
        with torch.cuda.stream(stream):
            again = mqk.fused_qkv_rope(*a_big)  # eager work on the grown workspace between replays
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(again, want_big))
    del junk


def test_workspace_growth_during_capture_raises(device):
    """A stream whose workspace would have to grow inside a capture raises (its
    zero fill would only run at replay) instead of capturing a wrong launch."""
    import mqk
    case = Case(48, 1, 1024, 16, 8, seed=4244, rows=4096,
                positions=torch.arange(48, dtype=torch.int32))
    args = case.args(device)
    stream = torch.cuda.Stream(device)  # fresh stream: no workspace yet
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(mqk.MqkNativeError, match="before capturing"):
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                mqk.fused_qkv_rope(*args)


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


def test_graph_replay_on_another_stream(device):
    """A graph captured on stream A replays on stream B into A's workspace; with
    B ordered after A's eager work by an event (and A's next work after the
    replay), the replays equal the eager call bit for bit.  This is the supported
    pattern; overlapping them would race on the shared workspace."""
    import mqk
    case = Case(32, 1, 1024, 16, 8, seed=4250, rows=4096,
                positions=torch.randint(0, 4096, (32,), generator=torch.Generator().manual_seed(3),
                                        dtype=torch.int32))
    args = case.args(device)
    sa, sb = torch.cuda.Stream(device), torch.cuda.Stream(device)
    with torch.cuda.stream(sa):
        eager = mqk.fused_qkv_rope(*args)
        sa.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=sa):
            out = mqk.fused_qkv_rope(*args)
    for rep in range(3):
        with torch.cuda.stream(sa):
            again = mqk.fused_qkv_rope(*args)  # eager work on A's workspace
        done_a = torch.cuda.Event()
        done_a.record(sa)
        for t in out:
            t.fill_(0)
        sb.wait_stream(torch.cuda.current_stream(device))
        sb.wait_event(done_a)
        with torch.cuda.stream(sb):
            graph.replay()
        sa.wait_stream(sb)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(out, eager)), f"replay {rep}"
        assert all(torch.equal(a, b) for a, b in zip(again, eager))


def test_workspace_bytes_and_release(device):
    """workspace_bytes() reports what the workspaces hold; release_workspaces()
    frees the retired ones (or all), and the next call allocates a fresh, zeroed
    workspace and gives the same bits."""
    import mqk
    case = Case(48, 1, 1024, 16, 8, seed=4251, rows=4096,
                positions=torch.randint(0, 4096, (48,), generator=torch.Generator().manual_seed(4),
                                        dtype=torch.int32))
    args = case.args(device)
    ref = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    held = mqk.workspace_bytes()
    assert held["current"] > 0
    assert mqk.release_workspaces() == held["retired"]
    assert mqk.workspace_bytes()["retired"] == 0
    released = mqk.release_workspaces(retired_only=False)
    assert released == held["current"] and mqk.workspace_bytes() == {"current": 0, "retired": 0}
    out = mqk.fused_qkv_rope(*args)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(out, ref))
    assert mqk.workspace_bytes()["current"] > 0
