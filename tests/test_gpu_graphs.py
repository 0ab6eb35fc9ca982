"""Projection groups captured in a HIP graph (torch.cuda.CUDAGraph) replay exactly as they run eagerly.

A decode step of the fused path — the Gemma norm producer feeding a merged Q4_K/Q6_K
projection, a SwiGLU down projection and a projection read through an input view — and
the batched path (the small-M, persistent and tiled GEMMs with their scratch) are captured once,
then replayed with new inputs written into the captured buffers. Between replays the same
step runs eagerly on the same inputs, and every replay must equal it bit for bit (the
kernels have fixed reduction orders; the decode tile's K pieces count their arrivals with
atomics but add the pieces in K order). The library issues no memset and no allocation of its
own; torch's graph pool holds every buffer.
"""
import numpy as np
import pytest
import torch

import _oracle as O
from test_gpu_parity import DEV, TOL_BF16, to_dev

pytestmark = pytest.mark.gpu


def _layer(parts_np, dtype=torch.bfloat16):
    from kaillm_amd.linear import PackedGGUFLinear

    layer = torch.nn.Module()
    layer.gguf_compact = torch.nn.ModuleList([PackedGGUFLinear(to_dev(w), t, dtype) for t, w in parts_np])
    return layer


@pytest.mark.parametrize("m", [1, 4, 8, 16, 64])
def test_decode_step_graph_replays_equal_eager(kai, m, monkeypatch):
    from kaillm_amd import native_fused
    from kaillm_amd.linear import GGUFLinearMethod

    print(f"graph step m={m}", flush=True)
    monkeypatch.setattr(native_fused, "CONSUMER_OF", {})
    monkeypatch.setattr(native_fused, "STASH", {})
    rng = np.random.default_rng(900 + m)
    k, kf = 2048, 1536
    a, b, s = 4, 8, 64
    method = GGUFLinearMethod()
    qkv = _layer([(O.Q4_K, O.random_blocks(O.Q4_K, 384, k, rng)), (O.Q6_K, O.random_blocks(O.Q6_K, 128, k, rng))])
    producer = 4242
    qkv._kai_act_producer = producer
    down = _layer([(O.Q6_K, O.random_blocks(O.Q6_K, 256, kf, rng))])
    viewed = _layer([(O.Q4_K, O.random_blocks(O.Q4_K, 256, k, rng))])
    viewed._kai_input_gather = torch.arange(k, device=DEV).reshape(a, b, s).transpose(0, 1).reshape(k)
    viewed._kai_input_view = (a, b, s)
    w32 = to_dev((1 + 0.1 * rng.standard_normal(k)).astype(np.float32))

    x = torch.empty((m, k), dtype=torch.bfloat16, device=DEV)
    res = torch.empty((m, k), dtype=torch.float32, device=DEV)
    gu = torch.empty((m, 2 * kf), dtype=torch.bfloat16, device=DEV)
    xv = torch.empty((m, k), dtype=torch.bfloat16, device=DEV)

    def act_fn(t):
        return torch.nn.functional.silu(t[..., :kf]) * t[..., kf:]

    def step():
        fused = native_fused.norm_prepare(producer, x, res, w32, 1e-6) if m <= 8 else None
        y, r_out = fused if fused is not None else (x, res)
        return [method.apply(qkv, y), method.apply_swiglu(down, gu, act_fn), method.apply(viewed, xv), r_out]

    def fill(seed):
        g = np.random.default_rng(seed)
        x.copy_(to_dev(g.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16))
        res.copy_(to_dev(g.standard_normal((m, k)).astype(np.float32)))
        gu.copy_(to_dev(g.standard_normal((m, 2 * kf)).astype(np.float32)).to(torch.bfloat16))
        xv.copy_(to_dev(g.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16))

    fill(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = step()
    torch.cuda.synchronize()
    if m <= 8:
        assert native_fused.CONSUMER_OF  # the qkv consumer was registered for the producer
    for replay in range(3):
        fill(10 + replay)
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(static_out, eager):
            assert torch.equal(got, want), f"replay {replay}"
    del graph


@pytest.mark.parametrize("m", [5, 8])
def test_decode_k_pieces_graph_replays_equal_eager(kai, m):
    """Two decode projections whose tiled paired kernel splits K across workgroups (320 row
    sets of long rows) captured in one graph: each launch took its slot of partial sums at
    capture, and every replay, with eager calls of the same projections in between, must
    equal the eager result bit for bit (the arrival counts are back at zero after each
    launch)."""
    from kaillm_amd.linear import GGUFLinearMethod

    print(f"graph K pieces m={m}", flush=True)
    rng = np.random.default_rng(950 + m)
    k = 8192
    method = GGUFLinearMethod()
    first = _layer([(O.Q6_K, O.random_blocks(O.Q6_K, 5120, k, rng))])
    second = _layer([(O.Q6_K, O.random_blocks(O.Q6_K, 5120, k, rng))])
    x = torch.empty((m, k), dtype=torch.bfloat16, device=DEV)

    def step():
        return [method.apply(first, x), method.apply(second, x)]

    def fill(seed):
        g = np.random.default_rng(seed)
        x.copy_(to_dev(g.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16))

    fill(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = step()
    torch.cuda.synchronize()
    for replay in range(3):
        fill(20 + replay)
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(static_out, eager):
            assert torch.equal(got, want), f"replay {replay}"
    del graph


@pytest.mark.parametrize("m", [9, 16])
def test_small_m_pieces_graph_replays_equal_eager(kai, m):
    """The small-M GEMM on long and short Q6_K rows (5120 x 17408 and 5120 x 6144, the C3 down
    and o_proj shapes), whose row sets are cut into pieces across waves and workgroups and
    added by its reduction launch: captured in one graph, every replay, with eager calls in
    between, must equal the eager result bit for bit, and the eager result must match the
    oracle."""
    from kaillm_amd.linear import GGUFLinearMethod

    print(f"graph small-M pieces m={m}", flush=True)
    rng = np.random.default_rng(970 + m)
    method = GGUFLinearMethod()
    shapes = [(5120, 17408), (5120, 6144)]
    parts = [O.random_blocks(O.Q6_K, n, k, rng) for n, k in shapes]
    layers = [_layer([(O.Q6_K, w)], torch.float16) for w in parts]
    xs = [torch.empty((m, k), dtype=torch.float16, device=DEV) for _, k in shapes]

    def step():
        return [method.apply(layer, x) for layer, x in zip(layers, xs)]

    def fill(seed):
        g = np.random.default_rng(seed)
        for x in xs:
            x.copy_(to_dev(g.standard_normal(tuple(x.shape)).astype(np.float32)).to(torch.float16))

    fill(1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = step()
    torch.cuda.synchronize()
    for replay in range(3):
        fill(30 + replay)
        eager = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(static_out, eager):
            assert torch.equal(got, want), f"replay {replay}"
    cols = np.arange(0, 5120, 37)
    for w, (n, k), x, got in zip(parts, shapes, xs, eager):
        want = O.mmq_reference(O.Q6_K, w[cols], x.cpu().numpy(), threads=16)
        err = O.normwise_rel(got.float().cpu().numpy()[:, cols], want)
        print(f"  {n}x{k} normwise rel err {err:.3e}")
        assert err <= TOL_BF16  # the projection writes bf16 for a 16-bit layer
    del graph
