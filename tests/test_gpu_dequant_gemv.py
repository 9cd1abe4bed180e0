"""GPU parity: device dequantization (bit-exact with src/dequant.rs) and the
decode GEMV (within tolerance of dequant + f64 host matmul), through the C ABI.

Tolerances: the north star's bound is 1e-3 max error normalised by the output
row's L2 norm; the GEMV (f16-rounded activations, f32 accumulation) is held to
1e-4 on that metric and to the reference's own rel_max_diff < 1e-3
(quant_resident_tests.rs:6-10)."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4K, Q6K = 8, 12, 14
DEV = "cuda:0"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _weight(rq, ty, blocks, n, k, offset=0):
    """A Weight whose blocks sit at `offset` bytes into a fresh device arena."""
    buf = torch.zeros(blocks.size + offset + 64, dtype=torch.uint8, device=DEV)
    buf[offset:offset + blocks.size].copy_(_dev(blocks))
    return rq.Weight(rq.GgmlType(ty), buf, [k, n], offset=offset, len=blocks.size)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("gen", ["reference", "baseline"])
def test_dequant_bit_exact(rq, orc, ty, gen):
    k, n = 1024, 96
    w = orc.synthetic(ty, k, n, 21) if gen == "reference" else synth.weights(ty, n, k, 77)
    want = orc.dequantize(ty, w, n * k)
    blocks = _dev(w)
    got32 = rq.dequantize(ty, blocks, n * k, torch.float32).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want.view(np.uint32))
    got16 = rq.dequantize(ty, blocks, n * k, torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("ty", [Q6K, Q8_0])
def test_dequant_unaligned_blocks(rq, orc, ty):
    """Q6_K / Q8_0 blocks are only 2-byte aligned (gemv_q4k.cu:60-63)."""
    k, n = 512, 7
    w = orc.synthetic(ty, k, n, 5)
    buf = torch.zeros(w.size + 8, dtype=torch.uint8, device=DEV)
    buf[2:2 + w.size].copy_(_dev(w))
    got = rq.dequantize(ty, buf[2:2 + w.size], n * k).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), orc.dequantize(ty, w, n * k).view(np.uint32))


def test_dequant_committed_fixtures(rq):
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz"))
    for ty, name in [(Q4K, "q4k"), (Q6K, "q6k"), (Q8_0, "q8_0")]:
        n, k = f[f"{name}_shape"]
        got = rq.dequantize(ty, _dev(f[f"{name}_w"]), n * k).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), f[f"{name}_deq"].view(np.uint32))


# ------------------------------------------------------------------ GEMV

def _check_gemv(rq, orc, ty, n, k, w_np, x_np, offset=0, tol=1e-4):
    w = _weight(rq, ty, w_np, n, k, offset)
    x = _dev(x_np)
    y = rq.gemv(x, w).cpu().numpy()
    ref = orc.reference_gemm(ty, w_np, n, k, x_np)[0]
    e = orc.rel_err_row_l2(y[None], ref[None])
    assert e < tol, f"type {ty} [{n}x{k}] row-L2 error {e}"
    assert orc.rel_max_diff(y, ref) < 1e-3
    return y


CONFIG2 = [(name, ty, n, k) for name, ty, n, k in synth.QWEN3_06B_LAYER]
CONFIG4 = [(name, ty, n, k) for name, ty, n, k in synth.QWEN3_8B_LAYER] + [synth.LM_HEAD]


@pytest.mark.parametrize("name,ty,n,k", CONFIG2, ids=[c[0] for c in CONFIG2])
def test_gemv_qwen3_06b_shapes(rq, orc, name, ty, n, k):
    seed = synth.seed_for(2, 0, [c[0] for c in CONFIG2].index(name))
    _check_gemv(rq, orc, ty, n, k, synth.weights(ty, n, k, seed), synth.activations(k, seed + 1000))


@pytest.mark.parametrize("name,ty,n,k", CONFIG4, ids=[c[0] for c in CONFIG4])
def test_gemv_8b_shapes(rq, orc, name, ty, n, k):
    seed = synth.seed_for(4, 0, [c[0] for c in CONFIG4].index(name))
    _check_gemv(rq, orc, ty, n, k, synth.weights(ty, n, k, seed), synth.activations(k, seed + 1000))


def test_gemv_config1_q8_0(rq, orc):
    seed = synth.seed_for(1)
    _check_gemv(rq, orc, Q8_0, 1024, 1024, synth.weights(Q8_0, 1024, 1024, seed), synth.activations(1024, seed + 1))


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("n,k", [(1, 256), (3, 256), (5, 768), (37, 512), (130, 1536), (17, 3072), (9, 14336)])
def test_gemv_edge_shapes_reference_generators(rq, orc, ty, n, k):
    """Reference generators: Q6_K d zero / negative, Q8_0 d zero / subnormal / signed.
    With a handful of outputs the row-L2 normalisation is over few values, so the
    f16 activation rounding shows as up to ~2e-4 here (bound: 5e-4; spec: 1e-3)."""
    w = orc.synthetic(ty, k, n, 1000 + n)
    x = orc.activations(k, 7 + n)
    _check_gemv(rq, orc, ty, n, k, w, x, tol=5e-4)


@pytest.mark.parametrize("ty", [Q6K, Q8_0])
def test_gemv_two_byte_aligned_weights(rq, orc, ty):
    n, k = 33, 1024
    w = orc.synthetic(ty, k, n, 99)
    _check_gemv(rq, orc, ty, n, k, w, orc.activations(k, 3), offset=2, tol=5e-4)


def test_gemv_zero_activations_and_one_hot(rq, orc):
    """Closed forms: x = 0 gives y = 0; x = e_j gives column j of the dequantized weight."""
    n, k = 64, 1024
    for ty in (Q4K, Q6K, Q8_0):
        w_np = orc.synthetic(ty, k, n, 4)
        w = _weight(rq, ty, w_np, n, k)
        y0 = rq.gemv(torch.zeros(k, device=DEV), w).cpu().numpy()
        assert np.all(y0 == 0)
        deq = orc.dequant_matrix(ty, w_np, n, k)
        for j in (0, 31, 32, 100, 1023):
            x = torch.zeros(k, device=DEV)
            x[j] = 1.0
            y = rq.gemv(x, w).cpu().numpy()
            # exact weights, but the kernel removes the f16 magic offset (1024 * scale) in f32
            assert np.allclose(y, deq[:, j], rtol=1e-4, atol=1e-4 * np.abs(deq).max()), (ty, j)


def test_gemv_rows_matches_single_row_bitwise(rq, orc):
    n, k = 200, 2048
    for ty in (Q4K, Q6K, Q8_0):
        w_np = orc.synthetic(ty, k, n, 8)
        w = _weight(rq, ty, w_np, n, k)
        xs = orc.activations(13 * k, 3)
        x = _dev(xs)
        y = rq.gemv_q4k(x, w, 13).cpu().numpy().reshape(13, n)
        for r in range(13):
            yr = rq.gemv(_dev(xs[r * k:(r + 1) * k]), w).cpu().numpy()
            assert np.array_equal(y[r], yr)


def test_gemv_batch_and_plan_match_single_calls(rq, orc):
    """A fused launch of mixed types (q/k/v with Q6_K v) equals separate calls bit for bit."""
    items, singles = [], []
    for i, (name, ty, n, k) in enumerate(CONFIG2 * 2):
        w_np = synth.weights(ty, n, k, 500 + i)
        w = _weight(rq, ty, w_np, n, k)
        x = _dev(synth.activations(k, 900 + i))
        items.append((x, w, torch.empty(n, device=DEV)))
        singles.append(rq.gemv(x, w).cpu().numpy())
    rq.gemv_batch(items[:3])
    for (x, w, y), s in zip(items[:3], singles[:3]):
        assert np.array_equal(y.cpu().numpy(), s)
    plan = rq.GemvPlan(items)
    for y in (it[2] for it in items):
        y.fill_(float("nan"))
    plan.run()
    plan.run()
    for (x, w, y), s in zip(items, singles):
        assert np.array_equal(y.cpu().numpy(), s)


def test_gemv_deterministic(rq):
    n, k = 3072, 1024
    w = _weight(rq, Q4K, synth.weights(Q4K, n, k, 3), n, k)
    x = _dev(synth.activations(k, 4))
    a = rq.gemv(x, w).cpu().numpy()
    b = rq.gemv(x, w).cpu().numpy()
    assert np.array_equal(a, b)


def test_gemv_errors_raise(rq):
    w = _weight(rq, Q4K, synth.weights(Q4K, 8, 512, 3), 8, 512)
    with pytest.raises(rq.ReflexError):
        rq.gemv(torch.zeros(511, device=DEV), w)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("scale", [3e4, 1e6])
def test_gemv_activations_beyond_f16_range(rq, orc, ty, scale):
    """x is staged as f16: activations of 3e4..1e6 (MoE SiLU*up outputs reach
    such values) are staged with an exact power-of-two scale that the row
    results undo, so the error bound is the same as for N(0,1) inputs."""
    n, k = 300, 2048
    w_np = orc.synthetic(ty, k, n, 77)
    x = synth.activations(k, 78) * np.float32(scale)
    _check_gemv(rq, orc, ty, n, k, w_np, x)


def test_gemv_batch_table_launch(rq, orc):
    """More GEMVs than fit in the kernel arguments run as one launch over an
    uploaded descriptor table, each equal to its single call bit for bit."""
    items, singles = [], []
    for i in range(9):
        ty = [Q4K, Q6K, Q8_0][i % 3]
        n, k = [(256, 512), (130, 1024), (64, 2048)][i % 3]
        w = _weight(rq, ty, orc.synthetic(ty, k, n, 90 + i), n, k)
        x = _dev(synth.activations(k, 100 + i))
        singles.append(rq.gemv(x, w).cpu().numpy())
        items.append((x, w, torch.full((n,), 7.0, device=DEV)))
    rq.gemv_batch(items)
    for (_, _, y), ref in zip(items, singles):
        assert np.array_equal(y.cpu().numpy(), ref)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_gemv_maximum_in_features(rq, orc, ty):
    """K = 16384 (the largest x staged in LDS) meets the bound; one super-block
    more is rejected with an error, not run."""
    n, k = 48, 16384
    _check_gemv(rq, orc, ty, n, k, orc.synthetic(ty, k, n, 5), orc.activations(k, 6), tol=5e-4)
    k2 = k + 256
    w = _weight(rq, ty, orc.synthetic(ty, k2, 4, 7), 4, k2)
    with pytest.raises(rq.ReflexError, match="exceeds"):
        rq.gemv(torch.zeros(k2, device=DEV), w)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("n,k", [(5, 4352), (33, 8448), (130, 12288), (3, 16128)])
def test_gemv_long_rows(rq, orc, ty, n, k):
    """Rows longer than 4096 run as several passes per lane: K = 4352 has 68
    units per row (4 lanes per row, 17 passes), K = 8448 Q8_0 264; few rows
    leave waves without rows."""
    w = orc.synthetic(ty, k, n, 300 + n)
    x = orc.activations(k, 301 + n)
    _check_gemv(rq, orc, ty, n, k, w, x, tol=5e-4)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_gemv_long_rows_beyond_f16_range(rq, orc, ty):
    """Several-pass rows with |x| beyond 2^15: the staged x is scaled."""
    n, k = 300, 8192
    x = synth.activations(k, 79) * np.float32(2e5)
    _check_gemv(rq, orc, ty, n, k, orc.synthetic(ty, k, n, 78), x)


def test_gemv_mixed_row_lengths_match_single_calls(rq, orc):
    """A launch mixing K = 3072..14336 (one-pass and several-pass rows, x
    staged at the launch's widest size) equals single calls bit for bit."""
    shapes = [(Q4K, 4096, 4096), (Q6K, 1024, 4096), (Q4K, 1024, 3072), (Q6K, 4096, 14336), (Q8_0, 512, 8192)]
    items, singles = [], []
    for i, (ty, n, k) in enumerate(shapes):
        w = _weight(rq, ty, orc.synthetic(ty, k, n, 400 + i), n, k)
        x = _dev(synth.activations(k, 410 + i))
        singles.append(rq.gemv(x, w).cpu().numpy())
        items.append((x, w, torch.full((n,), float("nan"), device=DEV)))
    plan = rq.GemvPlan(items)
    plan.run()
    for (_, _, y), ref in zip(items, singles):
        assert np.array_equal(y.cpu().numpy(), ref)
    rq.gemv_batch(items[:4])
    for (_, _, y), ref in zip(items[:4], singles[:4]):
        assert np.array_equal(y.cpu().numpy(), ref)


def test_gemv_plan_several_waves_of_workgroups(rq):
    """A plan beyond 512 KB per resident workgroup (9 x 33 MB at K = 14336,
    two workgroups per CU) runs as whole waves of workgroups; every output
    equals its single call bit for bit."""
    n, k = 4096, 14336
    w_np = synth.weights(Q4K, n, k, 41)
    buf = _dev(w_np)
    items, singles = [], []
    for i in range(9):
        w = rq.Weight(rq.GgmlType(Q4K), buf, [k, n])
        x = _dev(synth.activations(k, 60 + i))
        singles.append(rq.gemv(x, w).cpu().numpy())
        items.append((x, w, torch.full((n,), float("nan"), device=DEV)))
    rq.GemvPlan(items).run()
    for (_, _, y), ref in zip(items, singles):
        assert np.array_equal(y.cpu().numpy(), ref)


# ------------------------------------------------------------------ gathered rows

@pytest.mark.parametrize("ty,n,k", [(Q6K, 151936, 1024), (Q4K, 3072, 1024), (Q8_0, 1024, 1024)])
def test_gemv_gather_matches_full_gemv(rq, ty, n, k):
    """Model::gemv_gather (system1_tests.rs:16-84 pattern): gathered logits
    equal the full GEMV's at the same rows, bit for bit; first, middle and
    last rows, the argmax, duplicates, and runs of consecutive rows (one
    GEMV per run)."""
    w = _weight(rq, ty, synth.weights(ty, n, k, 44), n, k)
    x = _dev(synth.activations(k, 45))
    full = rq.gemv(x, w).cpu().numpy()
    am = int(np.argmax(full))
    rows = [0, n // 2, n - 1, am, am, 5, 6, 7, 8, 3, n - 2, n - 1]
    got = rq.gemv_gather(x, w, rows).cpu().numpy()
    assert np.array_equal(got, full[rows])
    many = np.random.default_rng(46).integers(0, n, 300).tolist()  # table launch
    assert np.array_equal(rq.gemv_gather(x, w, many).cpu().numpy(), full[many])


def test_gemv_gather_errors(rq):
    n, k = 256, 512
    w = _weight(rq, Q4K, synth.weights(Q4K, n, k, 47), n, k)
    x = _dev(synth.activations(k, 48))
    with pytest.raises(rq.ReflexError, match="row_indices must not be empty"):
        rq.gemv_gather(x, w, [])
    with pytest.raises(rq.ReflexError, match=r"row index 256 out of range \(out_features=256\)"):
        rq.gemv_gather(x, w, [3, 256])
    with pytest.raises(rq.ReflexError, match="x.len"):
        rq.gemv_gather(x[:256], w, [1])


def test_gemv_large_plans_interleaved_repeat(rq):
    """Two plans of tens of MB (one descriptor of 32768 rows; the 8B q, k,
    gate and down shapes), run interleaved three times, each run equal to the
    single calls bit for bit: a plan keeps no state between runs."""
    def big_plan(shapes, seed):
        items, singles = [], []
        for i, (ty, n, k) in enumerate(shapes):
            w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, seed + i), k, n, device=DEV)
            x = _dev(synth.activations(k, seed + 50 + i))
            singles.append(rq.gemv(x, w).cpu().numpy())
            items.append((x, w, torch.empty(n, device=DEV)))
        return rq.GemvPlan(items), items, singles
    a = big_plan([(Q6K, 32768, 1024)], 600)
    b = big_plan([(Q4K, 4096, 4096), (Q6K, 1024, 4096), (Q4K, 14336, 4096), (Q6K, 4096, 14336)], 700)
    for rep in range(3):
        for plan, items, singles in (a, b):
            for _, _, y in items:
                y.fill_(float("nan"))
            plan.run()
            for (_, _, y), ref in zip(items, singles):
                assert np.array_equal(y.cpu().numpy(), ref), f"run {rep}"


@pytest.mark.parametrize("order", [0, 1])
def test_gemv_plan_long_rows_get_their_own_workgroups(rq, orc, order):
    """GEMVs with K > 4096 (several passes per row) start a range segment of
    their own with workgroups in proportion to their cost: a long GEMV with
    only 8 rows (fewer row iterations than its share of workgroups: empty
    ranges), first or between short ones, equals its single call bit for bit
    and meets the bound."""
    shapes = [(Q4K, 64, 4096), (Q6K, 8, 14336), (Q4K, 4096, 1024), (Q8_0, 40, 8192)]
    if order:
        shapes = shapes[1:] + shapes[:1]
    items, singles, refs = [], [], []
    for i, (ty, n, k) in enumerate(shapes):
        w_np = orc.synthetic(ty, k, n, 1200 + i)
        w = _weight(rq, ty, w_np, n, k)
        xs = synth.activations(k, 1210 + i)
        x = _dev(xs)
        singles.append(rq.gemv(x, w).cpu().numpy())
        items.append((x, w, torch.full((n,), float("nan"), device=DEV)))
        refs.append((ty, n, k, w_np, xs))
    plan = rq.GemvPlan(items)
    for _ in range(2):
        plan.run()
        for (_, _, y), s in zip(items, singles):
            assert np.array_equal(y.cpu().numpy(), s)
    ty, n, k, w_np, xs = refs[0 if order else 1]
    want = orc.reference_gemm(ty, w_np, n, k, xs)[0]
    got = items[0 if order else 1][2].cpu().numpy()
    assert orc.rel_err_row_l2(got[None], want[None]) < 5e-4
