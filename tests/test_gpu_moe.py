"""GPU parity of the MoE pieces: gather / scatter-add / SiLU*up against their
definitions (src/kernels_cuda/elementwise.cu:175-222, silu_and_mul.cu:7-23),
expert slicing, and the grouped expert FFN (dense.rs:1509-1559) against the
host reference (per-expert dequant + f64 matmuls, weighted sum)."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
DEV = "cuda:0"
TOL = 1e-3   # the north star's bound (row-L2 normalised max error), for the layer's final output


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def test_gather_scatter_exact(rq):
    rng = np.random.default_rng(1)
    rows, hidden = 50, 96
    src = rng.standard_normal((rows, hidden)).astype(np.float32)
    perm = rng.choice(rows, 17, replace=False).astype(np.uint32)
    g = rq.moe_gather(_dev(src), _dev(perm), hidden).cpu().numpy().reshape(17, hidden)
    assert np.array_equal(g, src[perm])
    dst0 = rng.standard_normal((rows, hidden)).astype(np.float32)
    wts = rng.standard_normal(17).astype(np.float32)
    d = _dev(dst0)
    rq.moe_scatter_add(_dev(g), _dev(perm), _dev(wts), d, hidden)
    want = dst0.copy()
    want[perm] = (want[perm].astype(np.float64) + wts[:, None].astype(np.float64) * g.astype(np.float64)).astype(np.float32)
    assert np.allclose(d.cpu().numpy(), want, rtol=1e-6, atol=1e-6)


def test_silu_and_mul(rq, orc):
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(10000) * 4).astype(np.float32)
    u = rng.standard_normal(10000).astype(np.float32)
    got = rq.silu_and_mul(_dev(g), _dev(u)).cpu().numpy()
    assert np.allclose(got, orc.silu_and_mul(g, u), rtol=2e-6, atol=1e-7)


def test_expert_gemv_is_gemv_of_slice(rq, orc):
    e_cnt, hidden, ffn = 8, 1024, 256
    w_np = synth.weights(Q4K, e_cnt * ffn, hidden, 3)
    w = rq.Weight(rq.GgmlType.Q4K, _dev(w_np), [hidden, ffn, e_cnt])
    x = _dev(synth.activations(hidden, 4))
    per = w_np.size // e_cnt
    for e in (0, 5, 7):
        y = rq.expert_gemv(x, w, e).cpu().numpy()
        ref = orc.reference_gemm(Q4K, w_np[e * per:(e + 1) * per], ffn, hidden, x.cpu().numpy())[0]
        assert orc.rel_err_row_l2(y[None], ref[None]) < 1e-4
        ew = rq.quant_expert_weight(w, e)
        assert np.array_equal(rq.gemv(x, ew).cpu().numpy(), y)


def _moe_case(rq, orc, tokens, experts, hidden, ffn, top_k, seed):
    gate = synth.weights(Q4K, experts * ffn, hidden, seed)
    up = synth.weights(Q4K, experts * ffn, hidden, seed + 1)
    down = synth.weights(Q4K, experts * hidden, ffn, seed + 2)
    x = synth.activations(tokens * hidden, seed + 3).reshape(tokens, hidden)
    logits = synth.normals(seed + 4, tokens * experts).reshape(tokens, experts)
    W = lambda a, i, o: rq.Weight(rq.GgmlType.Q4K, _dev(a), [i, o, experts])  # noqa: E731
    out = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped(_dev(x), tokens, hidden, logits, experts, top_k, True, 1.0,
                       W(gate, hidden, ffn), W(up, hidden, ffn), W(down, ffn, hidden), out)
    routes = [orc.route_top_k(logits[t], top_k) for t in range(tokens)]
    ref = orc.moe_ffn_grouped_reference(x, routes, gate, up, down, Q4K, hidden, ffn, experts)
    return out.cpu().numpy().reshape(tokens, hidden), ref, routes


def test_moe_ffn_grouped_small(rq, orc):
    y, ref, routes = _moe_case(rq, orc, 64, 16, 512, 256, 4, 100)
    counts = np.bincount([e for r in routes for e, _ in r], minlength=16)
    assert counts.sum() == 64 * 4 and counts.max() > counts.min()  # uneven groups
    assert orc.rel_err_row_l2(y, ref) < TOL


def test_moe_ffn_grouped_config5_full(rq, orc):
    """BASELINE config 5 in full: 128 experts, hidden 2048, ffn 768, 512 tokens
    routed top-8 (4096 token-expert pairs, uneven per-expert counts), every
    token checked against the host reference."""
    y, ref, routes = _moe_case(rq, orc, 512, 128, 2048, 768, 8, 200)
    counts = np.bincount([e for r in routes for e, _ in r], minlength=128)
    assert counts.sum() == 4096 and counts.max() > 2 * counts.min()
    e = orc.rel_err_row_l2(y, ref)
    print(f"config 5 MoE prefill, 512 tokens: row-L2 error {e:.2e}")
    assert e < TOL


def test_moe_ffn_grouped_deterministic(rq, orc):
    a, _, _ = _moe_case(rq, orc, 32, 16, 512, 256, 4, 300)
    b, _, _ = _moe_case(rq, orc, 32, 16, 512, 256, 4, 300)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("tokens", [1, 3])
def test_moe_ffn_grouped_decode_gemv_path(rq, orc, tokens):
    """Up to 4 tokens run every routed pair as GEMVs (activations rounded to f16
    only, no int8 stage): within 1e-3 of the host reference at config 5 shapes."""
    y, ref, routes = _moe_case(rq, orc, tokens, 128, 2048, 768, 8, 400 + tokens)
    assert len(routes) == tokens
    e = orc.rel_err_row_l2(y, ref)
    print(f"decode MoE {tokens} tokens: row-L2 error {e:.2e}")
    assert e < TOL


def test_moe_ffn_grouped_back_to_back(rq, orc):
    """Calls queue on the stream without host synchronisation (tables go
    through a ring of pinned staging buffers): ten calls with different
    routings, then one sync, each equal to the same call run alone."""
    experts, hidden, ffn, top_k = 16, 512, 256, 4
    gate = synth.weights(Q4K, experts * ffn, hidden, 11)
    up = synth.weights(Q4K, experts * ffn, hidden, 12)
    down = synth.weights(Q4K, experts * hidden, ffn, 13)
    W = lambda a, i, o: rq.Weight(rq.GgmlType.Q4K, _dev(a), [i, o, experts])  # noqa: E731
    wg, wu, wd = W(gate, hidden, ffn), W(up, hidden, ffn), W(down, ffn, hidden)
    cases = []
    for i in range(10):
        tokens = [1, 2, 40, 3, 64][i % 5]
        x = _dev(synth.activations(tokens * hidden, 50 + i))
        logits = synth.normals(60 + i, tokens * experts).reshape(tokens, experts)
        cases.append((tokens, x, logits, torch.empty(tokens * hidden, device=DEV)))
    for tokens, x, logits, out in cases:
        rq.moe_ffn_grouped(x, tokens, hidden, logits, experts, top_k, True, 1.0, wg, wu, wd, out)
    torch.cuda.synchronize()
    for tokens, x, logits, out in cases:
        alone = torch.empty_like(out)
        rq.moe_ffn_grouped(x, tokens, hidden, logits, experts, top_k, True, 1.0, wg, wu, wd, alone)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), alone.cpu().numpy())


# ------------------------------------------------------------------ routing on the device

@pytest.mark.parametrize("normalize", [True, False])
def test_moe_route_device_matches_host(rq, normalize):
    """route_top_k_with_norm on the device: the same experts in the same
    order as the host router (moe.rs:47-98) for every token, weights within
    a few ulp (the softmax sum is reduced in another order); ties go to the
    lower index."""
    tokens, experts, k = 512, 128, 8
    logits = synth.normals(700, tokens * experts).reshape(tokens, experts)
    logits[0, :] = 0.25                    # all tied: experts 0..k-1
    logits[1, 5] = logits[1, 9] = 40.0     # a tie at the top
    idx, w = rq.moe_route_device(_dev(logits), tokens, experts, k, normalize, 0.5)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    for t in range(tokens):
        host = rq.route_top_k_with_norm(logits[t], k, normalize)
        assert [e for e, _ in host] == idx[t].tolist(), t
        np.testing.assert_allclose(w[t], np.array([v for _, v in host], np.float32) * 0.5, rtol=1e-6, atol=0)
    assert idx[0].tolist() == list(range(k)) and idx[1][:2].tolist() == [5, 9]


@pytest.mark.parametrize("experts,k", [(130, 8), (6, 6), (3, 2), (1024, 64)])
def test_moe_route_device_shapes(rq, experts, k):
    """Expert counts off the multiple of 4 and at the limits route as the
    host does (same experts, same order)."""
    tokens = 37
    logits = synth.normals(710 + experts, tokens * experts).reshape(tokens, experts)
    logits[3, :] = -1.5  # all tied
    idx, w = rq.moe_route_device(_dev(logits), tokens, experts, k, True, 1.0)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    for t in range(tokens):
        host = rq.route_top_k_with_norm(logits[t], k, True)
        assert [e for e, _ in host] == idx[t].tolist(), t
        np.testing.assert_allclose(w[t], np.array([v for _, v in host], np.float32), rtol=1e-6, atol=0)


def test_moe_route_device_nan_logits_give_valid_experts(rq):
    """A token with NaN logits still selects k distinct valid experts (its
    weights are NaN), so nothing downstream indexes past the expert tensors."""
    tokens, experts, k = 3, 16, 4
    logits = synth.normals(720, tokens * experts).reshape(tokens, experts)
    logits[1, 5] = np.nan
    idx, w = rq.moe_route_device(_dev(logits), tokens, experts, k, True, 1.0)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    assert ((idx >= 0) & (idx < experts)).all()
    assert len(set(idx[1].tolist())) == k and np.isnan(w[1]).all()
    assert np.isfinite(w[[0, 2]]).all()


def _moe_device_case(rq, orc, tokens, experts, hidden, ffn, top_k, seed, ties=False):
    gate = synth.weights(Q4K, experts * ffn, hidden, seed)
    up = synth.weights(Q4K, experts * ffn, hidden, seed + 1)
    down = synth.weights(Q4K, experts * hidden, ffn, seed + 2)
    x = _dev(synth.activations(tokens * hidden, seed + 3))
    logits = synth.normals(seed + 4, tokens * experts).reshape(tokens, experts)
    if ties:  # whole numbers: many experts share each probability
        logits = np.round(logits).astype(np.float32)
    W = lambda a, i, o: rq.Weight(rq.GgmlType.Q4K, _dev(a), [i, o, experts])  # noqa: E731
    ws = (W(gate, hidden, ffn), W(up, hidden, ffn), W(down, ffn, hidden))
    out_d = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped_device(x, tokens, hidden, _dev(logits), experts, top_k, True, 1.0, *ws, out_d)
    out_h = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped(x, tokens, hidden, logits, experts, top_k, True, 1.0, *ws, out_h)
    routes = [orc.route_top_k(logits[t], top_k) for t in range(tokens)]
    ref = orc.moe_ffn_grouped_reference(x.cpu().numpy().reshape(tokens, hidden), routes, gate, up, down, Q4K,
                                        hidden, ffn, experts)
    return (out_d.cpu().numpy().reshape(tokens, hidden), out_h.cpu().numpy().reshape(tokens, hidden), ref, ws, x,
            logits)


@pytest.mark.parametrize("tokens,experts,hidden,ffn,k", [(64, 16, 512, 256, 4), (48, 128, 2048, 768, 8),
                                                         (300, 8, 512, 512, 2), (512, 128, 2048, 768, 8)])
def test_moe_ffn_grouped_device(rq, orc, tokens, experts, hidden, ffn, k):
    """Device routing and grouping give the host-routed pipeline's result
    (same kernels; only last-bit weight differences) and meet the bound
    against the host reference (the last case is BASELINE config 5 in full)."""
    y_d, y_h, ref, _, _, _ = _moe_device_case(rq, orc, tokens, experts, hidden, ffn, k, 800 + tokens)
    assert orc.rel_err_row_l2(y_d, y_h.astype(np.float64)) < 1e-5
    assert orc.rel_err_row_l2(y_d, ref) < TOL


@pytest.mark.parametrize("tokens", [1, 64, 512])
def test_moe_q6k_down_projection(rq, orc, tokens):
    """Q4_K_M-style experts: gate/up Q4_K, down Q6_K at ffn 768 (three
    super-blocks per row, rows 2 bytes past a dword), host and device routing,
    every token against the host reference at the literal 1e-3."""
    experts, hidden, ffn, top_k, seed = 128, 2048, 768, 8, 950 + tokens
    gate = synth.weights(Q4K, experts * ffn, hidden, seed)
    up = synth.weights(Q4K, experts * ffn, hidden, seed + 1)
    down = synth.weights(Q6K, experts * hidden, ffn, seed + 2)
    x = _dev(synth.activations(tokens * hidden, seed + 3))
    logits = synth.normals(seed + 4, tokens * experts).reshape(tokens, experts)
    ws = (rq.Weight(rq.GgmlType.Q4K, _dev(gate), [hidden, ffn, experts]),
          rq.Weight(rq.GgmlType.Q4K, _dev(up), [hidden, ffn, experts]),
          rq.Weight(rq.GgmlType.Q6K, _dev(down), [ffn, hidden, experts]))
    out_h = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped(x, tokens, hidden, logits, experts, top_k, True, 1.0, *ws, out_h)
    out_d = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped_device(x, tokens, hidden, _dev(logits), experts, top_k, True, 1.0, *ws, out_d)
    routes = [orc.route_top_k(logits[t], top_k) for t in range(tokens)]
    ref = orc.moe_ffn_grouped_reference(x.cpu().numpy().reshape(tokens, hidden), routes, gate, up, down, Q4K,
                                        hidden, ffn, experts, down_ty=Q6K)
    for name, o in (("host", out_h), ("device", out_d)):
        e = orc.rel_err_row_l2(o.cpu().numpy().reshape(tokens, hidden), ref)
        print(f"MoE {tokens} tokens, Q6_K down, {name} routing: row-L2 error {e:.2e}")
        assert e < TOL


@pytest.mark.parametrize("tokens,k", [(1, 8), (4, 8), (1, 1), (2, 1), (5, 8), (2, 16), (3, 16)])
def test_moe_ffn_grouped_device_decode(rq, orc, tokens, k):
    """Up to 4 tokens take the two decode launches (device routing in the
    first; host routing of up to 32 pairs in the kernel arguments, 48 pairs
    uploaded); 5 tokens take the grouped MMQ path. Device- and host-routed
    calls agree and meet the bound."""
    y_d, y_h, ref, _, _, _ = _moe_device_case(rq, orc, tokens, 128, 2048, 768, k, 900 + tokens + k)
    assert orc.rel_err_row_l2(y_d, y_h.astype(np.float64)) < 1e-5
    assert orc.rel_err_row_l2(y_d, ref) < TOL


@pytest.mark.parametrize("tokens,experts,k", [(1, 128, 8), (3, 128, 8), (2, 200, 8), (4, 40, 6), (1, 256, 16)])
def test_moe_decode_tied_logits(rq, orc, tokens, experts, k):
    """Decode routing in every workgroup of the gate/up launch with tied
    probabilities (whole-number logits): the k best by probability, then the
    lowest index, as the host router picks them (a different expert among
    the tied ones would change the output by far more than the bound)."""
    y_d, y_h, ref, _, _, _ = _moe_device_case(rq, orc, tokens, experts, 256, 256, k, 990 + experts + tokens,
                                              ties=True)
    assert orc.rel_err_row_l2(y_d, y_h.astype(np.float64)) < 1e-5
    assert orc.rel_err_row_l2(y_d, ref) < TOL


@pytest.mark.parametrize("tokens,experts,k", [(1, 1024, 64), (3, 512, 16), (4, 6, 6)])
def test_moe_decode_wide_routing(rq, orc, tokens, experts, k):
    """Decode with many experts: the plan launch routes each token with all
    1024 threads (one rank count per expert and thread at 1024 experts, up to
    170 threads per expert at 6), the host-routed call plans on the device
    from its own routing; both meet the bound and agree."""
    y_d, y_h, ref, _, _, _ = _moe_device_case(rq, orc, tokens, experts, 256, 256, k, 970 + experts)
    assert orc.rel_err_row_l2(y_d, y_h.astype(np.float64)) < 1e-5
    assert orc.rel_err_row_l2(y_d, ref) < TOL


def test_moe_ffn_grouped_device_decode_in_graph(rq, orc):
    """The GEMV form of the device-routed layer replays from a HIP graph too."""
    tokens, experts, hidden, ffn, k = 2, 32, 1024, 512, 4
    y_d, _, _, ws, x, logits = _moe_device_case(rq, orc, tokens, experts, hidden, ffn, k, 960)
    lg = _dev(logits)
    out = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(tokens, hidden), y_d)
        torch.randn(1024, device=DEV).sum().item()


def test_moe_ffn_grouped_device_in_graph(rq, orc):
    """No host work per call: the whole device-routed MoE layer replays from
    a HIP graph, each replay equal to the eager call."""
    tokens, experts, hidden, ffn, k = 40, 16, 512, 256, 4
    y_d, _, _, ws, x, logits = _moe_device_case(rq, orc, tokens, experts, hidden, ffn, k, 950)
    lg = _dev(logits)
    out = torch.empty(tokens * hidden, device=DEV)
    rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)  # workspace sized
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(tokens, hidden), y_d)
        torch.randn(1024, device=DEV).sum().item()


def test_moe_graph_replays_after_workspace_growth(rq, orc):
    """A captured call keeps its workspace: a later, larger eager call grows
    the library's per-device workspace (the old one is retired, not freed),
    and the graph captured before still replays to the eager result."""
    tokens, experts, hidden, ffn, k = 2, 32, 1024, 512, 4
    y_d, _, _, ws, x, logits = _moe_device_case(rq, orc, tokens, experts, hidden, ffn, k, 970)
    lg = _dev(logits)
    out = torch.empty(tokens * hidden, device=DEV)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)
    torch.cuda.synchronize()
    # a prefill far larger than any other call of the suite (~200 MB of workspace)
    bt, be, bh, bf, bk = 2048, 16, 2048, 2048, 4
    gw = synth.weights(Q4K, be * bf, bh, 980)
    dw = synth.weights(Q4K, be * bh, bf, 981)
    W = lambda a, i, o: rq.Weight(rq.GgmlType.Q4K, _dev(a), [i, o, be])  # noqa: E731
    big = (W(gw, bh, bf), W(gw, bh, bf), W(dw, bf, bh))
    bx = _dev(synth.activations(bt * bh, 982))
    blg = _dev(synth.normals(983, bt * be))
    bout = torch.empty(bt * bh, device=DEV)
    rq.moe_ffn_grouped_device(bx, bt, bh, blg, be, bk, True, 1.0, *big, bout)
    torch.cuda.synchronize()
    assert torch.isfinite(bout).all()
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(tokens, hidden), y_d)


def test_moe_ffn_grouped_device_errors(rq):
    experts, hidden, ffn = 2, 256, 256
    W = lambda n, i, o: rq.Weight(rq.GgmlType.Q4K, torch.zeros(n, dtype=torch.uint8, device=DEV), [i, o, experts])  # noqa: E731
    g = W(experts * ffn * hidden // 256 * 144, hidden, ffn)
    d = W(experts * ffn * hidden // 256 * 144, ffn, hidden)
    x = torch.zeros(hidden, device=DEV)
    lg = torch.zeros(experts, device=DEV)
    with pytest.raises(rq.ReflexError, match="expert_count=2"):
        rq.moe_ffn_grouped_device(x, 1, hidden, lg, experts, 1, True, 1.0, g, g, d, torch.empty(hidden, device=DEV))


def test_moe_device_prefill_bit_stable(rq, orc):
    """The device plan groups each expert's rows in arrival order (LDS
    atomics), which differs between calls; the layer's output does not:
    repeated config 5 prefill calls are equal bit for bit."""
    y_d, _, ref, ws, x, logits = _moe_device_case(rq, orc, 512, 128, 2048, 768, 8, 1400)
    lg = _dev(logits)
    for i in range(4):
        out = torch.empty(512 * 2048, device=DEV)
        rq.moe_ffn_grouped_device(x, 512, 2048, lg, 128, 8, True, 1.0, *ws, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().reshape(512, 2048), y_d), f"call {i}"
    assert orc.rel_err_row_l2(y_d, ref) < TOL


@pytest.mark.parametrize("tokens,experts,hidden,ffn,k,down_ty", [(512, 128, 2048, 768, 8, Q4K), (64, 16, 512, 256, 4, Q4K),
                                                                  (300, 8, 512, 512, 2, Q4K), (512, 128, 2048, 768, 8, Q6K)])
def test_moe_gate_up_pair_matches_separate(rq, orc, tokens, experts, hidden, ffn, k, down_ty):
    """Prefill with Q4_K gate / up, device and host routing: the pair tiles
    (gate and up columns in one workgroup, silu(gate) * up stored from the
    epilogue, then one f16 activation pass) give the separate gate and up
    GEMMs + SiLU·up launch's output bit for bit (RFXQ_MOE_GU_PAIR=0 selects
    the latter), and meet the bound against the host reference."""
    import os
    seed = 1500 + tokens + experts + ffn + down_ty
    gate = synth.weights(Q4K, experts * ffn, hidden, seed)
    up = synth.weights(Q4K, experts * ffn, hidden, seed + 1)
    down = synth.weights(down_ty, experts * hidden, ffn, seed + 2)
    x = _dev(synth.activations(tokens * hidden, seed + 3))
    logits = synth.normals(seed + 4, tokens * experts).reshape(tokens, experts)
    dty = rq.GgmlType.Q4K if down_ty == Q4K else rq.GgmlType.Q6K
    ws = (rq.Weight(rq.GgmlType.Q4K, _dev(gate), [hidden, ffn, experts]),
          rq.Weight(rq.GgmlType.Q4K, _dev(up), [hidden, ffn, experts]),
          rq.Weight(dty, _dev(down), [ffn, hidden, experts]))
    lg = _dev(logits)
    outs = {}
    try:
        for pair in ("1", "0"):
            os.environ["RFXQ_MOE_GU_PAIR"] = pair
            for dev_routing in (True, False):
                out = torch.empty(tokens * hidden, device=DEV)
                if dev_routing:
                    rq.moe_ffn_grouped_device(x, tokens, hidden, lg, experts, k, True, 1.0, *ws, out)
                else:
                    rq.moe_ffn_grouped(x, tokens, hidden, logits, experts, k, True, 1.0, *ws, out)
                torch.cuda.synchronize()
                outs[(pair, dev_routing)] = out.cpu().numpy().reshape(tokens, hidden)
    finally:
        os.environ.pop("RFXQ_MOE_GU_PAIR", None)
    for dev_routing in (True, False):
        assert np.array_equal(outs[("1", dev_routing)], outs[("0", dev_routing)]), f"device routing {dev_routing}"
    outs["1"] = outs[("1", True)]
    routes = [orc.route_top_k(logits[t], k) for t in range(tokens)]
    ref = orc.moe_ffn_grouped_reference(x.cpu().numpy().reshape(tokens, hidden), routes, gate, up, down, Q4K,
                                        hidden, ffn, experts, down_ty=down_ty)
    assert orc.rel_err_row_l2(outs["1"], ref) < TOL
