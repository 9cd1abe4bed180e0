"""Fused activation producers of the prefill GEMMs: RMSNorm and SiLU·up
that write the quantized activation layouts directly, and GEMMs that read
them. Parity: the producers' f32 outputs are bit-identical to the reference
kernels' (rmsnorm.cu through the oracle restatement; silu_and_mul.cu through
rfxq_silu_and_mul), their activation buffers equal the quantizer's on those
outputs byte for byte, and GEMMs from the buffers equal rfxq_gemm on the f32
activations bit for bit."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4K, Q6K = 8, 12, 14
DEV = "cuda:0"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _a256(n):
    return (n + 255) // 256 * 256


def _layouts(act, rows, k):
    """The written regions of an activation buffer: the int8 layout (xq, xds)
    and the f16 layout (xh, xsx, xrs)."""
    b = act.cpu().numpy()
    sizes = [rows * k, rows * k // 32 * 4, rows * k * 2, rows * (k // 256) * 32, rows * 4]
    out, o = [], 0
    for sz in sizes:
        out.append(b[o:o + sz])
        o += _a256(sz)
    return out


def _same_act(a, b, rows, k):
    for i, (u, v) in enumerate(zip(_layouts(a, rows, k), _layouts(b, rows, k))):
        assert np.array_equal(u, v), f"layout {i}"


@pytest.mark.parametrize("rows,k", [(1, 1024), (7, 4096), (512, 1024), (33, 2048)])
def test_rmsnorm_q8_1(rq, orc, rows, k):
    rng = np.random.default_rng(rows + k)
    x = (rng.standard_normal((rows, k)) * 3.0).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    eps = 1e-6
    act, y = rq.rmsnorm_q8_1(_dev(x), _dev(g), rows, k, eps, want_y=True)
    want = orc.rmsnorm(x, g, rows, k, eps)
    assert np.array_equal(y.cpu().numpy().reshape(rows, k), want)
    _same_act(act, rq.quantize_act_q8_1(_dev(want), rows, k), rows, k)
    act2, none = rq.rmsnorm_q8_1(_dev(x), _dev(g), rows, k, eps)   # without the f32 output
    assert none is None
    _same_act(act2, act, rows, k)


@pytest.mark.parametrize("rows,k", [(1, 3072), (64, 768 * 4), (512, 1024)])
def test_silu_and_mul_q8_1(rq, rows, k):
    rng = np.random.default_rng(rows * 3 + k)
    gate = _dev((rng.standard_normal(rows * k) * 4).astype(np.float32))
    up = _dev(rng.standard_normal(rows * k).astype(np.float32))
    act, y = rq.silu_and_mul_q8_1(gate, up, rows, k, want_y=True)
    ref = rq.silu_and_mul(gate, up)
    assert torch.equal(y, ref)
    _same_act(act, rq.quantize_act_q8_1(ref, rows, k), rows, k)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("rows,n,k", [(512, 1024, 1024), (64, 512, 4096), (300, 136, 2048)])
def test_gemm_from_activation_buffer(rq, opts, ty, rows, n, k):
    """GEMMs from a buffer equal rfxq_gemm on the f32 activation, on the f16
    kernels and on the int8 ones (REFLEX_MMQ_F16=0)."""
    x = _dev(synth.activations(rows * k, 5 + rows))
    w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, 6 + n), k, n, device=DEV)
    act = rq.quantize_act_q8_1(x, rows, k)
    for f16 in (1, 0):
        opts(mmq_f16=f16)
        assert torch.equal(rq.gemm_q8_1(act, w, rows), rq.gemm(x, w, rows)), f"mmq_f16={f16}"


def test_gemm_q8_1_batch(rq, opts):
    opts(quant_mma_splits=1)  # the reference groups unsplit, as the batch
    rows = 200
    shapes = [(Q4K, 768, 1024), (Q6K, 256, 1024), (Q4K, 640, 2048), (Q8_0, 128, 1024)]
    xa, xb = _dev(synth.activations(rows * 1024, 1)), _dev(synth.activations(rows * 2048, 2))
    aa, ab = rq.quantize_act_q8_1(xa, rows, 1024), rq.quantize_act_q8_1(xb, rows, 2048)
    items = []
    for i, (ty, n, k) in enumerate(shapes):
        w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, 20 + i), k, n, device=DEV)
        y = torch.full((rows * n,), float("nan"), device=DEV)
        items.append((aa if k == 1024 else ab, w, y))
    refs = []
    for (act, w, _), (ty, n, k) in zip(items, shapes):
        r = torch.empty(rows * n, device=DEV)
        rq.gemm_batch([(xa if k == 1024 else xb, w, r)], rows)
        refs.append(r)
    rq.gemm_q8_1_batch(items, rows)
    for (_, _, y), r in zip(items, refs):
        assert torch.equal(y, r)


def test_fused_producer_errors(rq):
    x = _dev(np.ones((4, 1000), np.float32))
    with pytest.raises(rq.ReflexError, match="multiple of 256"):
        rq.quantize_act_q8_1(x, 4, 1000)
    w = rq.Weight.from_blocks(Q4K, synth.weights(Q4K, 64, 1024, 3), 1024, 64, device=DEV)
    act = torch.empty(rq.act_q8_1_size(4, 1024) + 256, dtype=torch.uint8, device=DEV)
    with pytest.raises(rq.ReflexError, match="256-byte aligned"):
        rq.gemm_q8_1(act[16:], w, 4)


def test_gemm_q8_1_plan_matches_f32_plan(rq):
    """A plan over activation buffers (rfxq_gemm_q8_1_plan_create: GEMM kernels
    only) gives the f32 plan's results bit for bit (same kernels, tiles and
    split-K), for a 0.6B layer's GEMMs at 512 rows and an 8B layer's at 40."""
    for layer, rows, seed in ((synth.QWEN3_06B_LAYER, 512, 5), (synth.QWEN3_8B_LAYER, 40, 6)):
        group = {"q_proj": "qkv", "k_proj": "qkv", "v_proj": "qkv", "o_proj": "o",
                 "gate_proj": "gu", "up_proj": "gu", "down_proj": "down"}
        xs, acts, f32_items, q_items = {}, {}, [], []
        for pi, (name, ty, n, k) in enumerate(layer):
            g = group[name]
            if g not in xs:
                xs[g] = torch.from_numpy(synth.activations(rows * k, seed * 100 + pi)).to(DEV)
                acts[g] = rq.quantize_act_q8_1(xs[g], rows, k)
            w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, seed * 100 + 50 + pi), k, n, device=DEV)
            f32_items.append((xs[g], w, torch.empty(rows * n, device=DEV)))
            q_items.append((acts[g], w, torch.full((rows * n,), float("nan"), device=DEV)))
        rq.GemmPlan(f32_items, rows).run()
        plan = rq.GemmPlan(q_items, rows, quantized=True)
        for _ in range(2):
            plan.run()
            for (_, _, a), (_, _, b) in zip(f32_items, q_items):
                assert torch.equal(a, b)


@pytest.mark.parametrize("ty", [Q4K, Q6K])
@pytest.mark.parametrize("rows,ffn,k", [(512, 3072, 1024), (64, 768, 2048), (12, 3072, 1024), (300, 1280, 1024),
                                        (512, 14336, 4096)])
def test_gemm_gate_up_silu_q8_1(rq, orc, opts, ty, rows, ffn, k):
    """gemm(gate) + gemm(up) + silu_and_mul fused: y and the activation
    buffer equal the separate GEMMs (for Q4_K with split-K off, as the fused
    tiles never split) followed by rfxq_silu_and_mul_q8_1, bit for bit (Q4_K: one launch
    of gate/up pair tiles at 32-, 64- and 128-row tiles; Q6_K: the separate
    path itself), and y meets the bound against dequant + f64."""
    x = synth.activations(rows * k, 31 + rows)
    gate_np = synth.weights(ty, ffn, k, 32 + ffn)
    up_np = synth.weights(ty, ffn, k, 33 + ffn)
    gate = rq.Weight.from_blocks(ty, gate_np, k, ffn, device=DEV)
    up = rq.Weight.from_blocks(ty, up_np, k, ffn, device=DEV)
    act = rq.quantize_act_q8_1(_dev(x), rows, k)
    opts(quant_mma_splits=1 if ty == Q4K else 0)   # (the separate path keeps the default split policy)
    g = rq.gemm_q8_1(act, gate, rows)
    u = rq.gemm_q8_1(act, up, rows)
    want_act, want_y = rq.silu_and_mul_q8_1(g, u, rows, ffn, want_y=True)
    opts(quant_mma_splits=0)
    got_act, got_y = rq.gemm_gate_up_silu_q8_1(act, rows, gate, up)
    assert torch.equal(got_y, want_y)
    _same_act(got_act, want_act, rows, ffn)
    if rows * ffn * k <= 512 * 3072 * 1024:
        xs = x.reshape(rows, k).astype(np.float64)
        gr = orc.reference_gemm(ty, gate_np, ffn, k, xs)
        ur = orc.reference_gemm(ty, up_np, ffn, k, xs)
        with np.errstate(over="ignore"):
            ref = gr / (1.0 + np.exp(-gr)) * ur
        assert orc.rel_err_row_l2(got_y.cpu().numpy().reshape(rows, ffn), ref) < 1e-3
