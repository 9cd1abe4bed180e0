"""Capture of the library's launches in a HIP graph (torch.cuda.CUDAGraph):
GEMV plans (one decode layer as four dependent launches) and a grouped GEMM
plan replay to the same bits as their eager runs. Each graph is replayed
several times, with unrelated eager work and synchronisations between the
replays, and every replay is checked. Plans upload their tables at creation,
so a run is a kernel launch only (no allocation, memset or host copy)."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
DEV = "cuda:0"


def _w(rq, ty, n, k, seed):
    return rq.Weight.from_blocks(ty, synth.weights(ty, n, k, seed), k, n, device=DEV)


def _x(n, seed):
    return torch.from_numpy(synth.activations(n, seed)).to(DEV)


def _replays(graph, outs, want, other):
    for r in range(3):
        for y in outs:
            y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for y, ref in zip(outs, want):
            assert torch.equal(y, ref), f"replay {r}"
        other()  # eager work between replays
        torch.cuda.synchronize()


def _other_work():
    a = torch.randn(512, 512, device=DEV)
    (a @ a).sum().item()


def test_gemv_plans_in_graph(rq):
    layer = synth.QWEN3_06B_LAYER
    layers = 3
    xs = {k: _x(k, 100 + k) for k in {k for *_, k in layer}}
    groups = [(0, 1, 2), (3,), (4, 5), (6,)]
    plans, outs = [], []
    for li in range(layers):
        ws = {p: _w(rq, layer[p][1], layer[p][2], layer[p][3], 16 * li + p) for p in range(len(layer))}
        for g in groups:
            items = [(xs[layer[p][3]], ws[p], torch.empty(layer[p][2], device=DEV)) for p in g]
            outs += [y for _, _, y in items]
            plans.append(rq.GemvPlan(items))
    for p in plans:
        p.run()
    torch.cuda.synchronize()
    want = [y.clone() for y in outs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for p in plans:
                p.run()
    torch.cuda.synchronize()
    _replays(g, outs, want, _other_work)


def test_gemm_plan_in_graph(rq):
    rows = 96
    shapes = [(Q4K, 512, 1024), (Q6K, 256, 1024), (Q4K, 384, 2048)]
    xa, xb = _x(rows * 1024, 7), _x(rows * 2048, 8)
    items = []
    for i, (ty, n, k) in enumerate(shapes):
        items.append((xa if k == 1024 else xb, _w(rq, ty, n, k, 30 + i), torch.empty(rows * n, device=DEV)))
    plan = rq.GemmPlan(items, rows)
    plan.run()
    torch.cuda.synchronize()
    want = [y.clone() for _, _, y in items]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.run()
    torch.cuda.synchronize()
    _replays(g, [y for _, _, y in items], want, _other_work)


def test_gemv_large_plan_twice_in_graph(rq):
    """A 62 MB plan captured twice in one graph, and run eagerly between the
    replays, replays to the eager bits."""
    shapes = [(Q6K, 32768, 1024), (Q4K, 14336, 4096)]
    items = [(_x(k, 200 + i), _w(rq, ty, n, k, 210 + i), torch.empty(n, device=DEV)) for i, (ty, n, k) in enumerate(shapes)]
    plan = rq.GemvPlan(items)
    plan.run()
    torch.cuda.synchronize()
    want = [y.clone() for _, _, y in items]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.run()
            plan.run()
    torch.cuda.synchronize()
    _replays(g, [y for _, _, y in items], want, lambda: (plan.run(), _other_work()))
