"""GPU parity of the MoE pieces: gather / scatter-add / SiLU*up against their
definitions (src/kernels_cuda/elementwise.cu:175-222, silu_and_mul.cu:7-23),
expert slicing, and the grouped expert FFN (dense.rs:1509-1559) against the
host reference (per-expert dequant + f64 matmuls, weighted sum)."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q4K = 12
DEV = "cuda:0"


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
    # two int8 quantization stages (x, then SiLU output) -> a looser bound than one GEMM
    assert orc.rel_err_row_l2(y, ref) < 3e-3


def test_moe_ffn_grouped_config5_sampled(rq, orc):
    """BASELINE config 5 shapes (128 experts, hidden 2048, ffn 768, 512 tokens, top-8),
    checked on a 48-token prefix routed with the same logits."""
    y, ref, _ = _moe_case(rq, orc, 48, 128, 2048, 768, 8, 200)
    assert orc.rel_err_row_l2(y, ref) < 3e-3


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
    assert e < 1e-3


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
