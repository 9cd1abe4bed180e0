"""GPU parity of the prefill GEMM path.

Default path (f16 activations; rfxq_act_f16 + rfxq_mmqh_q4k / _q6k / _q8_0):
the activation stage is bit-exact with the oracle's act_f16; every GEMM output
is within the north star's literal 1e-3 (max error over a row normalised by
the row's L2 norm) of dequant.rs + f64 host matmul, at every BASELINE config 3
and config 4 shape (the 8B layer and the tied 151936 x 1024 Q6_K LM head at
M = 512 on sampled rows), and within 2e-5 of an exact-arithmetic model of the
kernel's own operands (oracle.mmqh_model_reference), which isolates the
kernel's f32 accumulation.

int8 path (REFLEX_MMQ_F16=0: Q8_1 activations, per-32 int8 with an f16 scale):
the quantizer and the per-32 int32 block dots are bit-exact with the CPU
emulation, and the GEMM is within 3e-5 of the exact model of that format
(oracle.mmq_model_reference). The format's own quantization error reaches
~1.05e-3 (config 3 k_proj) and ~1.25e-3 (v_proj, Q6_K) on the worst of 512
rows, above the north star's bound, so it is not the default; its tests
check the kernel, not the format."""
import os

import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4K, Q6K = 8, 12, 14
DEV = "cuda:0"
TOL = 1e-3          # the north star's bound, asserted as written
MODEL_TOL = 2e-5    # kernel rounding against the exact model of its operands


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _weight(rq, ty, blocks, n, k):
    return rq.Weight(rq.GgmlType(ty), _dev(blocks), [k, n])


# ------------------------------------------------------------------ int8 path: quantizer and block dots

def test_quantize_q8_1_bit_exact(rq, orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((97, 1024)).astype(np.float32)
    x[0, :32] = 0
    x[1, :64] = np.repeat(np.float32([0.5, -0.5, 1.5, -2.5]), 16)    # exact halves of d*q
    x[2, :32] = np.float32(1e-30)
    x[3, 32:64] = rng.standard_normal(32).astype(np.float32) * 1e4
    xq, xds = rq.quantize_q8_1(_dev(x), 97, 1024)
    qs, ds = orc.quantize_q8_1(x)
    assert np.array_equal(xq.cpu().numpy(), qs)
    d = xds.cpu().numpy().view(np.uint32)
    assert np.array_equal((d & 0xFFFF).astype(np.uint16), ds[..., 0])
    assert np.array_equal((d >> 16).astype(np.uint16), ds[..., 1])


def test_quantize_committed_fixtures(rq):
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz"))
    m, k = f["x"].shape
    xq, xds = rq.quantize_q8_1(_dev(f["x"]), m, k)
    assert np.array_equal(xq.cpu().numpy(), f["xq"])
    d = xds.cpu().numpy().view(np.uint32)
    assert np.array_equal((d & 0xFFFF).astype(np.uint16), f["xds"][..., 0])


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("m,n,k", [(3, 8, 512), (37, 70, 512), (130, 129, 768), (1, 300, 256)])
def test_mmq_block_dots_bit_exact(rq, orc, ty, m, n, k):
    w_np = orc.synthetic(ty, k, n, 31 + m)
    x = orc.activations(m * k, 5 + n).reshape(m, k) * 3
    xq, xds = rq.quantize_q8_1(_dev(x), m, k)
    w = _weight(rq, ty, w_np, n, k)
    got = rq.mmq_block_dots(xq, xds, m, w).cpu().numpy()
    want = orc.block_dots(ty, w_np, n, k, xq.cpu().numpy())
    assert np.array_equal(got, want)


def test_mmq_block_dots_committed_fixtures(rq):
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "fixtures.npz"))
    m, k = f["x"].shape
    xq, xds = rq.quantize_q8_1(_dev(f["x"]), m, k)
    for ty, name in [(Q4K, "q4k"), (Q6K, "q6k"), (Q8_0, "q8_0")]:
        n, kk = f[f"{name}_shape"]
        w = _weight(rq, ty, f[f"{name}_w"], n, kk)
        got = rq.mmq_block_dots(xq, xds, m, w).cpu().numpy()
        assert np.array_equal(got, f[f"{name}_dots"]), name


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("m,n,k", [(7, 200, 1024), (129, 300, 512), (512, 1024, 1024)])
def test_int8_gemm_kernel_matches_format_model(rq, orc, opts, ty, m, n, k):
    """The int8 MMQ kernels against the exact model of the Q8_1 format."""
    opts(mmq_f16=0, fused_max_rows=0)   # the int8 kernel at every row count
    w_np = synth.weights(ty, n, k, 40 + m)
    x = synth.activations(m * k, 41 + m).reshape(m, k)
    y = rq.gemm(_dev(x), _weight(rq, ty, w_np, n, k), m).cpu().numpy().reshape(m, n)
    e = orc.rel_err_row_l2(y, orc.mmq_model_reference(ty, w_np, n, k, x))
    print(f"int8 kernel type {ty} M={m} [{n}x{k}]: {e:.2e} from the format model")
    assert e < 3e-5


# ------------------------------------------------------------------ default path: f16 activations

def _act_regions(rq, act, rows, k):
    """(xh u16 [rows, k], xsx u16 [rows, k/256, 16], xrs f32 [rows]) of an activation buffer."""
    a256 = lambda v: (v + 255) // 256 * 256  # noqa: E731
    b = act.cpu().numpy()
    o = a256(rows * k) + a256(rows * k // 32 * 4)
    xh = b[o:o + rows * k * 2].view(np.uint16).reshape(rows, k)
    o += a256(rows * k * 2)
    xsx = b[o:o + rows * (k // 256) * 32].view(np.uint16).reshape(rows, k // 256, 16)
    o += a256(rows * (k // 256) * 32)
    xrs = b[o:o + rows * 4].view(np.float32)
    return xh, xsx, xrs


def test_act_f16_bit_exact(rq, orc):
    """rfxq_act_f16 (the f16 kernels' input stage) against oracle.act_f16: row
    scales, f16 values in the stored order, and block sums, bit for bit, with
    rows at the edges of the f16 range."""
    rng = np.random.default_rng(3)
    rows, k = 41, 1024
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[0] = 0
    x[1] *= np.float32(1e6)                  # beyond f16 as plain values
    x[2] *= np.float32(1e-30)                # below f16's normal range
    x[3, :] = np.float32(-3.0)               # constant row
    x[4, 5] = np.float32(7e4)                # one large value
    x[5] = rng.standard_normal(k).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 20, k)
    x[6, 100:] = 0
    act = rq.quantize_act_q8_1(_dev(x), rows, k)
    xh, xsx, xrs = _act_regions(rq, act, rows, k)
    wh, wsx, wrs = orc.act_f16(x)
    assert np.array_equal(xrs, wrs)
    assert np.array_equal(xh, wh)
    assert np.array_equal(xsx, wsx)


def _ref_rows(orc, ty, w_np, n, k, xs, chunk=16384):
    """dequant.rs + f64 host matmul for rows xs, in column chunks (bounded memory)."""
    qk, bb = orc.BLOCK_DIMS[ty]
    rb = k // qk * bb
    out = np.empty((xs.shape[0], n), np.float32)
    for c0 in range(0, n, chunk):
        c1 = min(n, c0 + chunk)
        out[:, c0:c1] = orc.reference_gemm(ty, np.ascontiguousarray(w_np[c0 * rb:c1 * rb]), c1 - c0, k, xs)
    return out


def _check_gemm(rq, orc, ty, m, n, k, w_np, x_np, rows_checked=None):
    w = _weight(rq, ty, w_np, n, k)
    y = rq.gemm(_dev(x_np), w, m).cpu().numpy().reshape(m, n)
    rows = np.arange(m) if rows_checked is None else rows_checked
    xs = np.ascontiguousarray(x_np.reshape(m, k)[rows])
    ref = _ref_rows(orc, ty, w_np, n, k, xs)
    e = orc.rel_err_row_l2(y[rows], ref)
    msg = f"type {ty} M={m} [{n}x{k}]: row-L2 error {e:.3e}"
    if rq.gemm_policy(ty, k, n, m)["path"] == rq.PATH_MMQ_F16:   # the f16 kernels: checked against their model
        e_kernel = orc.rel_err_row_l2(y[rows], orc.mmqh_model_reference(ty, w_np, n, k, xs))
        msg += f", kernel {e_kernel:.1e} from its model"
        assert e_kernel < MODEL_TOL, msg
    print(msg)
    assert e < TOL, msg
    return y, e


@pytest.mark.parametrize("name,ty,n,k", synth.QWEN3_06B_LAYER, ids=[c[0] for c in synth.QWEN3_06B_LAYER])
def test_gemm_prefill_qwen3_06b(rq, orc, name, ty, n, k):
    """M = 512, every row checked."""
    seed = synth.seed_for(3, 0, [c[0] for c in synth.QWEN3_06B_LAYER].index(name))
    x = synth.activations(512 * k, seed + 1000).reshape(512, k)
    _check_gemm(rq, orc, ty, 512, n, k, synth.weights(ty, n, k, seed), x)


@pytest.mark.parametrize("name,ty,n,k", synth.QWEN3_8B_LAYER, ids=[c[0] for c in synth.QWEN3_8B_LAYER])
def test_gemm_prefill_8b_sampled_rows(rq, orc, name, ty, n, k):
    """BASELINE config 4 at M = 512: the full GEMM on the GPU, 96 sampled rows checked
    (rows are independent)."""
    seed = synth.seed_for(4, 1, [c[0] for c in synth.QWEN3_8B_LAYER].index(name))
    x = synth.activations(512 * k, seed + 1000).reshape(512, k)
    rows = np.sort(np.random.default_rng(seed).choice(512, 96, replace=False))
    _check_gemm(rq, orc, ty, 512, n, k, synth.weights(ty, n, k, seed), x, rows)


@pytest.mark.parametrize("rows", [3, 4, 5, 12, 29, 48])
@pytest.mark.parametrize("name,ty,n,k", [c for c in synth.QWEN3_8B_LAYER if c[0] in ("q_proj", "down_proj")],
                         ids=["q_proj", "down_proj"])
def test_gemm_few_rows_8b(rq, orc, rows, name, ty, n, k):
    """The few-row paths (GEMVs per row for q_proj at 3-4 rows, 32-row tiles
    for down at 3-4 rows and for both from 5 rows, 64-row tiles; every row
    checked) at the 8B shapes."""
    seed = synth.seed_for(4, 3, rows)
    x = synth.activations(rows * k, seed + 1000).reshape(rows, k)
    _check_gemm(rq, orc, ty, rows, n, k, synth.weights(ty, n, k, seed), x)


def test_gemm_prefill_lm_head_m512(rq, orc):
    """BASELINE config 4's tied LM head, 151936 x 1024 Q6_K, at M = 512: 12 sampled
    rows against the reference over all 151936 columns."""
    _, _, n, k = synth.LM_HEAD
    seed = synth.seed_for(4, 2, 0)
    x = synth.activations(512 * k, seed + 1000).reshape(512, k)
    rows = np.sort(np.random.default_rng(seed).choice(512, 12, replace=False))
    _check_gemm(rq, orc, Q6K, 512, n, k, synth.weights(Q6K, n, k, seed), x, rows)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("m", [2, 5, 7, 12, 29, 32, 33, 48, 64, 65, 129, 513])
def test_gemm_row_counts(rq, orc, ty, m):
    """Every tile height: GEMV rows (2), 32-row (5..32), 64-row (33..64) and
    128-row tiles (65 up), ragged counts of each."""
    n, k = 200, 1024
    w_np = orc.synthetic(ty, k, n, 60 + m)
    x = synth.activations(m * k, 61 + m).reshape(m, k)
    _check_gemm(rq, orc, ty, m, n, k, w_np, x)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("m,n,k", [(33, 200, 256), (129, 1000, 2048), (300, 136, 4096), (64, 130, 768),
                                   (513, 3072, 1024), (200, 520, 1280)])
def test_gemm_ragged_shapes(rq, orc, ty, m, n, k):
    """Ragged M and N, K from one super-block up (Q6_K rows with an odd
    super-block count, k = 256, 768 and 1280, start 2 bytes past a dword),
    held to the literal 1e-3 against dequant + f64 and to the kernel's model."""
    w_np = synth.weights(ty, n, k, 90 + m)
    x = synth.activations(m * k, 91 + m).reshape(m, k)
    _check_gemm(rq, orc, ty, m, n, k, w_np, x)


@pytest.mark.parametrize("k", [256, 768, 1280])
@pytest.mark.parametrize("m", [5, 40, 100, 512])
def test_gemm_q6k_odd_superblocks(rq, orc, m, k):
    """Q6_K with an odd super-block count per row (Q4_K_M MoE down projections:
    ffn 768) on the f16 kernels at every tile height."""
    n = 2048
    assert rq.gemm_policy(Q6K, k, n, m)["path"] == rq.PATH_MMQ_F16
    w_np = synth.weights(Q6K, n, k, 700 + m + k)
    x = synth.activations(m * k, 701 + m + k).reshape(m, k)
    _check_gemm(rq, orc, Q6K, m, n, k, w_np, x)


@pytest.mark.parametrize("m", [2, 5, 32, 512])
def test_gemm_q8_0_config1_matrix(rq, orc, m):
    """Q8_0 prefill on BASELINE config 1's 1024 x 1024 matrix: GEMV rows at 2,
    the f16 tiles from 5 rows."""
    n = k = 1024
    w_np = synth.weights(Q8_0, n, k, 800 + m)
    x = synth.activations(m * k, 801 + m).reshape(m, k)
    _check_gemm(rq, orc, Q8_0, m, n, k, w_np, x)


@pytest.mark.parametrize("ty", [Q6K, Q8_0])
@pytest.mark.parametrize("m", [40, 300])
def test_gemm_weights_two_bytes_past_a_dword(rq, orc, ty, m):
    """Q6_K and Q8_0 weights need only 2-byte alignment: weights starting 2
    bytes past a dword (the Q8_0 tile's unaligned-load form) give the same
    results as the same blocks dword aligned."""
    n, k = 520, 2048
    w_np = synth.weights(ty, n, k, 830 + m)
    buf = torch.zeros(w_np.size + 16, dtype=torch.uint8, device=DEV)
    buf[2:2 + w_np.size] = _dev(w_np)
    w2 = rq.Weight(rq.GgmlType(ty), buf, [k, n], offset=2, len=w_np.size)
    w4 = _weight(rq, ty, w_np, n, k)
    x = _dev(synth.activations(m * k, 831 + m))
    y2 = rq.gemm(x, w2, m)
    assert torch.equal(y2, rq.gemm(x, w4, m))
    e = orc.rel_err_row_l2(y2.cpu().numpy().reshape(m, n),
                           orc.reference_gemm(ty, w_np, n, k, x.cpu().numpy().reshape(m, k)))
    assert e < TOL


def test_gemm_q8_0_large(rq, orc):
    """Q8_0 at an 8B-class shape, M = 512, 64 sampled rows."""
    n, k, m = 4096, 4096, 512
    w_np = synth.weights(Q8_0, n, k, 810)
    x = synth.activations(m * k, 811).reshape(m, k)
    rows = np.sort(np.random.default_rng(812).choice(m, 64, replace=False))
    _check_gemm(rq, orc, Q8_0, m, n, k, w_np, x, rows)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_gemm_weight_past_4gib(rq, orc, ty):
    """A weight whose last columns lie more than 4 GiB past its start (the
    kernels' buffer resources start at each column tile): zero blocks up to
    the last 300 columns, which hold random blocks and are checked against the
    reference; every zero column must come out exactly 0."""
    k, m = 256, 40
    qk, bb = {Q4K: (256, 144), Q6K: (256, 210), Q8_0: (32, 34)}[ty]
    rb = k // qk * bb
    tail = 300
    n = (4 * 2**30 + 64 * 2**20) // rb + tail
    w_tail = synth.weights(ty, tail, k, 820 + ty)
    buf = torch.zeros(n * rb, dtype=torch.uint8, device=DEV)
    buf[(n - tail) * rb:] = _dev(w_tail)
    w = rq.Weight(rq.GgmlType(ty), buf, [k, n])
    assert rq.gemm_policy(ty, k, n, m)["path"] == rq.PATH_MMQ_F16
    x = synth.activations(m * k, 821).reshape(m, k)
    y = rq.gemm(_dev(x), w, m).reshape(m, n)
    assert int(torch.count_nonzero(y[:, :n - tail])) == 0
    yt = y[:, n - tail:].cpu().numpy()
    del y, buf
    e = orc.rel_err_row_l2(yt, orc.reference_gemm(ty, w_tail, tail, k, x))
    print(f"type {ty}: columns past 4 GiB, row-L2 error {e:.2e}")
    assert e < TOL


def test_gemm_rows_independent_and_deterministic(rq, orc, opts):
    """Row r of the output depends only on row r of x, and repeats give identical bits."""
    n, k = 1024, 2048
    w = _weight(rq, Q4K, synth.weights(Q4K, n, k, 9), n, k)
    x = synth.activations(300 * k, 10).reshape(300, k)
    ya = rq.gemm(_dev(x), w, 300).cpu().numpy().reshape(300, n)
    yb = rq.gemm(_dev(x), w, 300).cpu().numpy().reshape(300, n)
    assert np.array_equal(ya, yb)
    opts(quant_mma_splits=1)   # same K decomposition on both sides
    y1 = rq.gemm(_dev(x), w, 300).cpu().numpy().reshape(300, n)
    y2 = rq.gemm(_dev(x[:130]), w, 130).cpu().numpy().reshape(130, n)
    assert np.array_equal(y1[:130], y2)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_gemm_split_k_matches_unsplit(rq, orc, opts, ty):
    n, k, m = 512, 4096, 64
    w_np = synth.weights(ty, n, k, 12)
    w = _weight(rq, ty, w_np, n, k)
    x = _dev(synth.activations(m * k, 13))
    ys = []
    for s in (1, 4, 16):
        opts(quant_mma_splits=s)
        ys.append(rq.gemm(x, w, m).cpu().numpy().reshape(m, n))
    assert np.array_equal(rq.gemm(x, w, m).cpu().numpy().reshape(m, n), ys[-1])   # repeatable
    for y in ys[1:]:
        assert orc.rel_err_row_l2(y, ys[0].astype(np.float64)) < 1e-6


def test_gemm_one_row_is_decode_gemv(rq):
    n, k = 512, 1024
    w = _weight(rq, Q4K, synth.weights(Q4K, n, k, 14), n, k)
    x = _dev(synth.activations(k, 15))
    assert np.array_equal(rq.gemm(x, w, 1).cpu().numpy(), rq.gemv(x, w).cpu().numpy())


def test_gemm_caller_workspace(rq, orc):
    n, k, m = 256, 1024, 40
    w_np = synth.weights(Q6K, n, k, 16)
    w = _weight(rq, Q6K, w_np, n, k)
    x = synth.activations(m * k, 17).reshape(m, k)
    ws = torch.empty(rq.gemm_workspace_size(w, m), dtype=torch.uint8, device=DEV)
    y = rq.gemm(_dev(x), w, m, workspace=ws).cpu().numpy().reshape(m, n)
    assert orc.rel_err_row_l2(y, orc.mmqh_model_reference(Q6K, w_np, n, k, x)) < MODEL_TOL
    with pytest.raises(rq.ReflexError):
        rq.gemm(_dev(x), w, m, workspace=ws[:100])


def test_gemm_plan_few_rows_large_group(rq, orc):
    """A grouped plan of an 8B layer at 3 rows takes one path for all its
    GEMMs (their re-reads together pass 56 MiB: 32-row tiles), and each
    output meets the bound against dequant + f64."""
    rows = 3
    items, refs = [], []
    xs = {}
    for i, (name, ty, n, k) in enumerate(synth.QWEN3_8B_LAYER):
        if k not in xs:
            xs[k] = synth.activations(rows * k, 90 + k % 97).reshape(rows, k)
        w_np = synth.weights(ty, n, k, 120 + i)
        items.append((_dev(xs[k].reshape(-1)), _weight(rq, ty, w_np, n, k), torch.empty(rows * n, device=DEV)))
        refs.append((ty, w_np, n, k, xs[k]))
    rq.GemmPlan(items, rows).run()
    torch.cuda.synchronize()
    for (_, _, y), (ty, w_np, n, k, x) in zip(items, refs):
        ref = orc.reference_gemm(ty, w_np, n, k, x)
        assert orc.rel_err_row_l2(y.cpu().numpy().reshape(rows, n), ref) < TOL


@pytest.mark.parametrize("rows", [300, 12, 29])
def test_gemm_batch_and_plan_match_single_gemms(rq, orc, opts, rows):
    """Grouped GEMMs (each activation brought into its layouts once, one launch
    per weight type; at up to 32 rows Q4_K and Q6_K share one launch of 32-row
    tiles) give the single-GEMM results bit for bit (split-K off on both
    sides; by default a group this small splits K)."""
    shapes = [(Q4K, 768, 1024), (Q4K, 256, 1024), (Q6K, 256, 1024), (Q8_0, 512, 1024), (Q4K, 640, 2048)]
    xa = _dev(synth.activations(rows * 1024, 71))
    xb = _dev(synth.activations(rows * 2048, 72))
    items = []
    for i, (ty, n, k) in enumerate(shapes):
        w = _weight(rq, ty, synth.weights(ty, n, k, 80 + i), n, k)
        items.append((xa if k == 1024 else xb, w, torch.empty(rows * n, device=DEV)))
    opts(quant_mma_splits=1)
    singles = [rq.gemm(x, w, rows).cpu().numpy() for x, w, _ in items]
    rq.gemm_batch(items, rows)
    for (_, _, y), ref in zip(items, singles):
        assert np.array_equal(y.cpu().numpy(), ref)
    for _, _, y in items:
        y.zero_()
    plan = rq.GemmPlan(items, rows)
    for _ in range(2):
        plan.run()
        for (_, _, y), ref in zip(items, singles):
            assert np.array_equal(y.cpu().numpy(), ref)
    opts(quant_mma_splits=0)
    # by default this group splits K: fixed-order partial sums, within f32
    # rounding of the unsplit result, identical between batch and plan
    rq.gemm_batch(items, rows)
    first = [y.cpu().numpy() for _, _, y in items]
    plan = rq.GemmPlan(items, rows)
    plan.run()
    for (_, _, y), a, ref in zip(items, first, singles):
        assert np.array_equal(y.cpu().numpy(), a)
        assert np.abs(a - ref).max() <= 1e-5 * np.abs(ref).max()
    # parity of one grouped result
    n, k = shapes[2][1], shapes[2][2]
    ref = orc.reference_gemm(Q6K, synth.weights(Q6K, n, k, 82), n, k,
                             synth.activations(rows * 1024, 71).reshape(rows, k))
    assert orc.rel_err_row_l2(first[2].reshape(rows, n), ref) < TOL


def test_gemm_plan_long_k_among_short(rq, orc):
    """A launch of many tiles whose GEMMs differ in K (a Q8_0 layer's down
    projection among K = 1024 GEMMs): the long GEMM splits K to about the
    launch's median and its tiles run first. Results stay within f32 rounding
    of the single GEMMs and within the north star's bound of the reference."""
    rows = 512
    shapes = [(Q8_0, 2048, 1024), (Q8_0, 2048, 1024), (Q8_0, 1024, 4096)]
    xa = synth.activations(rows * 1024, 91)
    xb = synth.activations(rows * 4096, 92)
    items, w_nps = [], []
    for i, (ty, n, k) in enumerate(shapes):
        w_nps.append(synth.weights(ty, n, k, 93 + i))
        items.append((_dev(xa if k == 1024 else xb), _weight(rq, ty, w_nps[-1], n, k),
                      torch.empty(rows * n, device=DEV)))
    singles = [rq.gemm(x, w, rows).cpu().numpy() for x, w, _ in items]
    plan = rq.GemmPlan(items, rows)
    for _ in range(2):
        plan.run()
        for (_, _, y), ref in zip(items, singles):
            assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    rq.gemm_batch(items, rows)
    for (_, _, y), ref in zip(items, singles):
        assert np.abs(y.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    sample = np.arange(0, rows, 17)
    ref = orc.reference_gemm(Q8_0, w_nps[2], 1024, 4096, xb.reshape(rows, 4096)[sample])
    y = items[2][2].cpu().numpy().reshape(rows, 1024)[sample]
    assert orc.rel_err_row_l2(y, ref) < TOL


def test_gemm_batch_errors(rq):
    x = _dev(synth.activations(64 * 1024, 3))
    w1 = _weight(rq, Q4K, synth.weights(Q4K, 256, 1024, 1), 256, 1024)
    w2 = _weight(rq, Q4K, synth.weights(Q4K, 256, 512, 2), 256, 512)
    y = torch.empty(64 * 256, device=DEV)
    with pytest.raises(rq.ReflexError):
        rq.gemm_batch([(x, w1, y), (x, w2, y)], 64)   # one x with two in_features


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
@pytest.mark.parametrize("scale,offset", [(3000.0, 2500.0), (1e5, 0.0), (1e-6, 0.0)])
def test_gemm_activation_range(rq, orc, ty, scale, offset):
    """Activations far from N(0,1) (SiLU·up outputs of MoE layers reach 1e5):
    the per-row power-of-two scale keeps them inside f16's range."""
    m, n, k = 64, 256, 1024
    w_np = synth.weights(ty, n, k, 33)
    x = synth.activations(m * k, 34).reshape(m, k) * np.float32(scale) + np.float32(offset)
    _check_gemm(rq, orc, ty, m, n, k, w_np, x)


def test_gemm_q6k_extreme_codes(rq, orc):
    """Q6_K blocks at the limits of the weight operands: scales -128 and 127 with
    codes 0 and 63 (|sc*(q - 32)| = 4096 and 3937), full-scale activations."""
    m, n, k = 96, 256, 1024
    rng = np.random.default_rng(5)
    nb = n * k // 256
    blk = np.zeros((nb, 210), np.uint8)
    blk[:, 0:192] = rng.choice(np.array([0x00, 0xFF], np.uint8), size=(nb, 192))
    blk[:, 192:208] = rng.choice(np.array([0x80, 0x7F], np.uint8), size=(nb, 16))
    blk[:, 208:210] = np.frombuffer(np.float16(1e-3).tobytes(), np.uint8)
    x = np.where(rng.random((m, k)) < 0.5, np.float32(-1.0), np.float32(1.0)).astype(np.float32)
    _check_gemm(rq, orc, Q6K, m, n, k, blk.reshape(-1), x)


def test_gemm_q4k_extreme_scales(rq, orc):
    """Q4_K super-blocks with 6-bit scales and mins at 0 and 63 and codes 0 and 15
    (the weight operand's range ends and a constant part of either sign)."""
    m, n, k = 64, 256, 2048
    rng = np.random.default_rng(6)
    nb = n * k // 256
    blk = synth.weights(Q4K, n, k, 7).reshape(nb, 144).copy()
    blk[:, 4:16] = rng.choice(np.array([0x00, 0xFF], np.uint8), size=(nb, 12))
    blk[:, 16:144] = rng.choice(np.array([0x00, 0xFF, 0x0F, 0xF0], np.uint8), size=(nb, 128))
    x = synth.activations(m * k, 8).reshape(m, k)
    _check_gemm(rq, orc, Q4K, m, n, k, blk.reshape(-1), x)
