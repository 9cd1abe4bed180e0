"""CPU tests pinning the oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against the reference's own known-answer
vectors (src/dequant.rs tests, src/moe.rs tests) and against facts the
mathematics fixes, computed by an independent route (exhaustive f16 tables,
an inverse packer, numpy f64 arithmetic, closed forms), so that a dropped
term, a wrong index or sign, or a transposed operand fails here.
"""
import json
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")
Q8_0, Q8_1, Q4K, Q6K = 8, 9, 12, 14


def f16b(v):
    return np.array([v], dtype=np.float16).view(np.uint8).tolist()


# ------------------------------------------------------------ reference known answers

def test_dequant_hand_vectors(orc):
    """src/dequant.rs:457-653 hand-computed values."""
    data = json.load(open(os.path.join(GOLD, "dequant_hand_vectors.json")))
    for v in data["vectors"]:
        blk = bytearray(v["len"])
        for off, bs in v["set"].items():
            blk[int(off):int(off) + len(bs)] = bytes(bs)
        out = orc.dequantize(v["type"], bytes(blk), v["count"])
        assert out.size == v["count"], v["name"]
        for idx, want in v["expect"].items():
            assert out[int(idx)] == np.float32(want), (v["name"], idx, out[int(idx)], want)


def test_dequant_truncates_and_rejects_unknown(orc):
    """dequant.rs:638-652: unknown types error; output truncates to element_count."""
    with pytest.raises(ValueError):
        orc.dequantize(999, b"", 0)
    assert orc.dequantize(Q8_0, bytes(34), 5).size == 5
    assert orc.dequantize(Q4K, bytes(144 * 2), 300).size == 300


# ------------------------------------------------------------ f16 conversion (half 2.7.1)

def test_f16_to_f32_exhaustive(orc):
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8, 1e-10, 0.5, 1.5, 2049.0,
                  2051.0, 1.00048828125, 1.00146484375], dtype=np.float32),
    ]).astype(np.float32)
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------ get_scale_min_k4 vs an inverse packer

def _pack_scale_min(sc, m):
    """ggml's Q4_K packing of 8 six-bit (scale, min) pairs into 12 bytes: the
    inverse of get_scale_min_k4, written from the bit layout description."""
    q = [0] * 12
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    return bytes(q)


def test_get_scale_min_k4_inverts_packer(orc):
    rng = np.random.default_rng(2)
    for _ in range(300):
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        packed = _pack_scale_min(sc, m)
        for j in range(8):
            assert orc.get_scale_min_k4(j, packed) == (sc[j], m[j])


# ------------------------------------------------------------ dequant closed forms

def _q4k_block(d, dmin, sc, m, nib_lo, nib_hi):
    blk = bytearray(144)
    blk[0:2] = bytes(f16b(d))
    blk[2:4] = bytes(f16b(dmin))
    blk[4:16] = _pack_scale_min(sc, m)
    for g in range(4):
        for l in range(32):
            blk[16 + 32 * g + l] = (nib_lo[64 * g + l] & 15) | ((nib_hi[64 * g + l] & 15) << 4)
    return bytes(blk)


def test_q4k_dequant_closed_form(orc):
    """y[64g+l] = f32(d*sc[2g])*lo - f32(dmin*m[2g]); y[64g+32+l] uses pair 2g+1 and the high nibble."""
    rng = np.random.default_rng(3)
    for _ in range(20):
        d = np.float16(rng.uniform(1e-4, 0.02))
        dmin = np.float16(rng.uniform(1e-4, 0.02))
        sc = rng.integers(0, 64, 8).tolist()
        m = rng.integers(0, 64, 8).tolist()
        lo = rng.integers(0, 16, 256).tolist()
        hi = rng.integers(0, 16, 256).tolist()
        out = orc.dequantize(Q4K, _q4k_block(d, dmin, sc, m, lo, hi), 256)
        for e in range(256):
            g, r = divmod(e, 64)
            j = 2 * g + (r >= 32)
            q = lo[64 * g + r] if r < 32 else hi[64 * g + r - 32]
            want = np.float32(np.float32(d) * np.float32(sc[j])) * np.float32(q) - np.float32(np.float32(dmin) * np.float32(m[j]))
            assert out[e] == want, (e, out[e], want)


def test_q6k_dequant_closed_form(orc):
    """Element 128n+32t+l = (d*sc[8n + l/16 + 2t]) * (q6 - 32) with q6 = 4 low bits | 2 high bits."""
    rng = np.random.default_rng(4)
    for _ in range(20):
        q6 = rng.integers(0, 64, 256)
        sc = rng.integers(-128, 128, 16)
        d = np.float16(rng.uniform(-0.02, 0.02))
        blk = bytearray(210)
        for n in range(2):
            for t in range(4):
                for l in range(32):
                    q = int(q6[128 * n + 32 * t + l])
                    qi = 64 * n + l + (32 if t & 1 else 0)
                    if t & 2:
                        blk[qi] |= (q & 15) << 4
                    else:
                        blk[qi] |= q & 15
                    blk[128 + 32 * n + l] |= (q >> 4) << (2 * t)
        blk[192:208] = sc.astype(np.int8).tobytes()
        blk[208:210] = bytes(f16b(d))
        out = orc.dequantize(Q6K, bytes(blk), 256)
        for e in range(256):
            n, r = divmod(e, 128)
            t, l = divmod(r, 32)
            s = int(sc[8 * n + l // 16 + 2 * t])
            want = np.float32(np.float32(d) * np.float32(s)) * np.float32(int(q6[e]) - 32)
            assert out[e] == want


def test_q8_0_dequant_exact(orc):
    rng = np.random.default_rng(5)
    qs = rng.integers(-128, 128, 32).astype(np.int8)
    d = np.float16(-0.0123)
    out = orc.dequantize(Q8_0, bytes(f16b(d)) + qs.tobytes(), 32)
    assert np.array_equal(out, qs.astype(np.float32) * np.float32(d))


# ------------------------------------------------------------ Q8_1 activation quantizer

def _np_quantize(x):
    """Independent numpy restatement: d = f32(amax)/127 (IEEE), id = 1/d,
    q = roundf(x*id) evaluated exactly in f64 (half away from zero)."""
    xb = x.reshape(x.shape[0], -1, 32).astype(np.float32)
    amax = np.max(np.abs(xb), axis=2)
    d = (amax / np.float32(127.0)).astype(np.float32)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    v = (xb * idv[..., None]).astype(np.float32).astype(np.float64)
    q = (np.trunc(v + np.copysign(0.5, v))).astype(np.int32)
    # exact block sum in f32, in the device kernel's order (8 lane partials, butterfly 4, 2, 1)
    p = ((xb[..., 0::4] + xb[..., 1::4]) + xb[..., 2::4]) + xb[..., 3::4]
    s = ((p[..., 0] + p[..., 4]) + (p[..., 2] + p[..., 6])) + ((p[..., 1] + p[..., 5]) + (p[..., 3] + p[..., 7]))
    s = (s * idv).astype(np.float32)  # in units of d
    return q.astype(np.int8).reshape(x.shape), d.astype(np.float16).view(np.uint16), s.astype(np.float16).view(np.uint16)


def test_quantize_q8_1_matches_independent_restatement(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((37, 256)).astype(np.float32)
    x[0, :32] = 0.0                                    # zero block: d = 0, q = 0
    x[1, :32] = np.arange(32, dtype=np.float32) - 16  # integers
    x[2, 32:64] = 1e-30                               # tiny
    x[3, :32] = np.float32(127.0) * np.float32(0.5) / np.float32(127.0) * np.arange(-16, 16)  # near .5 ties
    qs, ds = orc.quantize_q8_1(x)
    q2, d2, s2 = _np_quantize(x)
    assert np.array_equal(qs, q2)
    assert np.array_equal(ds[..., 0], d2)
    assert np.array_equal(ds[..., 1], s2)
    # invariants: |q| <= 127, the block's max |x| maps to +-127
    assert np.abs(qs.astype(np.int32)).max() <= 127
    xb = np.abs(x.reshape(37, -1, 32))
    qb = np.abs(qs.reshape(37, -1, 32).astype(np.int32))
    nz = xb.max(axis=2) > 0
    am = xb.argmax(axis=2)
    assert np.all(np.take_along_axis(qb, am[..., None], 2)[..., 0][nz] == 127)


# ------------------------------------------------------------ per-32 integer dots

def _codes_via_dequant(orc, ty, w, n, k):
    """Integer weight codes obtained through dequantize() after forcing the
    block scales to 1 and the mins to 0 (an independent route to the codes)."""
    w = w.copy()
    if ty == Q4K:
        b = w.reshape(-1, 144)
        b[:, 0:2] = np.array(f16b(1.0), dtype=np.uint8)
        b[:, 2:4] = 0
        b[:, 4:16] = np.frombuffer(_pack_scale_min([1] * 8, [0] * 8), dtype=np.uint8)
        return orc.dequantize(Q4K, b.reshape(-1), n * k).astype(np.int64).reshape(n, k) - 8  # centered
    if ty == Q6K:
        b = w.reshape(-1, 210)
        sc = b[:, 192:208].view(np.int8).astype(np.int64).copy()
        b[:, 208:210] = np.array(f16b(1.0), dtype=np.uint8)
        b[:, 192:208] = 1
        codes = orc.dequantize(Q6K, b.reshape(-1), n * k).astype(np.int64).reshape(n, k // 256, 256)
        # scale of element e: sc[8n + l/16 + 2t]
        e = np.arange(256)
        sidx = 8 * (e // 128) + (e % 32) // 16 + 2 * ((e % 128) // 32)
        return (codes * sc.reshape(n, k // 256, 16)[:, :, sidx]).reshape(n, k)
    b = w.reshape(-1, 34)
    b[:, 0:2] = np.array(f16b(1.0), dtype=np.uint8)
    return orc.dequantize(Q8_0, b.reshape(-1), n * k).astype(np.int64).reshape(n, k)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_block_dots_brute_force(orc, ty):
    n, k, m = 5, 512, 3
    w = orc.synthetic(ty, k, n, 11)
    rng = np.random.default_rng(7)
    qa = rng.integers(-127, 128, (m, k)).astype(np.int8)
    got = orc.block_dots(ty, w, n, k, qa)
    codes = _codes_via_dequant(orc, ty, w, n, k)
    want = np.einsum("mbj,nbj->mnb", qa.astype(np.int64).reshape(m, k // 32, 32), codes.reshape(n, k // 32, 32))
    assert np.array_equal(got, want)


def test_q4k_scale_min_np_matches_c(orc):
    w = orc.synthetic(Q4K, 512, 6, 17)
    sc, m = orc.q4k_scale_min_np(w, 6, 512)
    b = w.reshape(6, 2, 144)
    for n in range(6):
        for sb in range(2):
            for j in range(8):
                assert orc.get_scale_min_k4(j, bytes(b[n, sb, 4:16])) == (sc[n, 8 * sb + j], m[n, 8 * sb + j])


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_mmq_model_reference_without_quantization(orc, ty):
    """With activations already on the int8 grid of their own block scale
    (x = d*q exactly, d a power of two) the model reference equals the plain
    dequant + f64 matmul: the centered split w = d*sc*(q-8) + c is an identity."""
    n, k = 6, 512
    w = orc.synthetic(ty, k, n, 23)
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, (4, k)).astype(np.float32)
    q[:, ::32] = 127  # block amax = 127 * d exactly
    x = (q * np.float32(2.0 ** -7)).astype(np.float32)
    got = orc.mmq_model_reference(ty, w, n, k, x)
    want = orc.reference_gemm(ty, w, n, k, x)
    # the Q4_K constant part uses the f16-rounded block sum / d, exact here (an integer below 2048)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


# ------------------------------------------------------------ host matmul

def test_host_matmul_matches_f64(orc):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 70)).astype(np.float32)
    w = rng.standard_normal((9, 70)).astype(np.float32)
    want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(orc.host_matmul(x, w), want)


def test_cpu_baseline_matches_reference(orc):
    w = orc.synthetic(Q4K, 512, 40, 3)
    x = orc.activations(512 * 2, 9).reshape(2, 512)
    ref = orc.reference_gemm(Q4K, w, 40, 512, x)
    got = orc.cpu_dequant_matmul(Q4K, w, 40, 512, x, 2)
    assert orc.rel_max_diff(got, ref) < 1e-5


# ------------------------------------------------------------ router (src/moe.rs tests)

def test_route_top_k_hand_values(orc):
    lg = np.log(np.array([1, 2, 3, 4], dtype=np.float32))
    r = orc.route_top_k(lg, 2)
    assert [i for i, _ in r] == [3, 2]
    assert abs(r[0][1] - 4 / 7) < 1e-5 and abs(r[1][1] - 3 / 7) < 1e-5


def test_route_top_k_ties_and_errors(orc):
    r = orc.route_top_k(np.zeros(6, dtype=np.float32), 3)
    assert [i for i, _ in r] == [0, 1, 2]
    assert all(abs(w - 1 / 3) < 1e-6 for _, w in r)
    for lg, k in [([], 1), ([1.0, 2.0], 3), ([1.0, 2.0], 0), ([-np.inf, -np.inf], 1)]:
        with pytest.raises(ValueError):
            orc.route_top_k(np.array(lg, dtype=np.float32), k)


def test_route_top_k_matches_sorting_definition(orc):
    rng = np.random.default_rng(9)
    for _ in range(50):
        lg = rng.standard_normal(128).astype(np.float32)
        r = orc.route_top_k(lg, 8, normalize=False)
        e = np.exp((lg - lg.max()).astype(np.float64))
        p = e / e.sum()
        order = sorted(range(128), key=lambda i: (-p[i], i))[:8]
        assert [i for i, _ in r] == order
        assert np.allclose([w for _, w in r], p[order], rtol=1e-5)


# ------------------------------------------------------------ committed fixtures

def test_committed_fixtures_reproduce(orc):
    """The golden .npz fixtures (tests/golden/make_fixtures.py) still match the oracle."""
    f = np.load(os.path.join(GOLD, "fixtures.npz"))
    for ty, name in [(Q4K, "q4k"), (Q6K, "q6k"), (Q8_0, "q8_0")]:
        w = f[f"{name}_w"]
        n, k = f[f"{name}_shape"]
        assert np.array_equal(orc.dequantize(ty, w, n * k), f[f"{name}_deq"])
        assert np.array_equal(orc.block_dots(ty, w, n, k, f["xq"][:, :k]), f[f"{name}_dots"])
        assert np.array_equal(orc.reference_gemm(ty, w, n, k, f["x"][:, :k]), f[f"{name}_y"])
    qs, ds = orc.quantize_q8_1(f["x"])
    assert np.array_equal(qs, f["xq"]) and np.array_equal(ds, f["xds"])


# ------------------------------------------------------------------ rmsnorm

def _round_f32(q):
    """A Fraction rounded to the nearest float32 (ties to even), exactly."""
    from fractions import Fraction
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)                       # subnormal spacing below 2^-126
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * ulp))


def _rmsnorm_exact(x, w, eps):
    """Independent restatement: the sum of squares as a chain of exactly
    rounded fused multiply-adds (rational arithmetic), then numpy float32
    division, sqrt and products (IEEE, correctly rounded)."""
    from fractions import Fraction
    rows, k = x.shape
    out = np.zeros_like(x)
    for r in range(rows):
        s = np.float32(0.0)
        for v in x[r]:
            s = _round_f32(Fraction(float(v)) * Fraction(float(v)) + Fraction(float(s)))
        inv = np.float32(1.0) / np.sqrt(s / np.float32(k) + np.float32(eps))
        out[r] = (x[r] * inv) * w
    return out


def test_rmsnorm_matches_exact_fma_chain(orc):
    """rmsnorm.cuh:17-41's fused sum order, pinned by exact rational FMAs; a
    plain (separately rounded) sum of squares differs on these inputs."""
    rng = np.random.default_rng(12)
    rows, k, eps = 5, 64, 1e-6
    x = (rng.standard_normal((rows, k)) * np.exp(rng.uniform(-3, 3, (rows, k)))).astype(np.float32)
    w = rng.standard_normal(k).astype(np.float32)
    got = orc.rmsnorm(x, w, rows, k, eps)
    want = _rmsnorm_exact(x, w, eps)
    assert np.array_equal(got, want)
    # the same with a separately rounded v*v: different outputs on some rows
    rows2 = 64
    x2 = (rng.standard_normal((rows2, k)) * np.exp(rng.uniform(-3, 3, (rows2, k)))).astype(np.float32)
    plain = np.zeros(rows2, np.float32)
    for r in range(rows2):
        for v in x2[r]:
            plain[r] = np.float32(plain[r] + np.float32(v * v))
    inv_plain = np.float32(1.0) / np.sqrt(plain / np.float32(k) + np.float32(eps))
    assert not np.array_equal((x2 * inv_plain[:, None]) * w, orc.rmsnorm(x2, w, rows2, k, eps))


def test_rmsnorm_closed_form(orc):
    """Rows of one repeated power of two: the sum of squares is exact, so
    y = w * c / sqrt(c^2 + eps) exactly as numpy computes it in f32."""
    k = 256
    for c, eps in [(1.0, 1e-6), (0.5, 1e-5), (2.0, 0.0)]:
        x = np.full((2, k), c, np.float32)
        w = np.linspace(-2, 2, k, dtype=np.float32)
        got = orc.rmsnorm(x, w, 2, k, eps)
        inv = np.float32(1.0) / np.sqrt(np.float32(c * c) + np.float32(eps))
        assert np.array_equal(got, np.stack([(x[0] * inv) * w] * 2))


# ------------------------------------------------------------ SiLU * up

def test_silu_and_mul_against_f64_and_limits(orc):
    """silu_and_mul.cu:7-23, g / (1 + e^-g) * u in f32 (three roundings plus
    expf's): within 3 ulps of the f64 value (below 1e-35 in magnitude, where
    expf(-g) overflows to inf, within 1e-35); exact zeros at g = 0 and u = 0;
    g * u at large g (e^-g below half an ulp of 1); a vanishing negative tail
    at very negative g; odd symmetry silu(-g) = silu(g) - g checked to
    rounding. A sign error in the exponent, a dropped factor or a swapped
    operand fails one of these."""
    rng = np.random.default_rng(11)
    g = np.concatenate([rng.standard_normal(4000) * 4, rng.uniform(-90, 90, 1000)]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    out = orc.silu_and_mul(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(out - want) <= 3 * ulp + 1e-35)
    z = orc.silu_and_mul(np.zeros(3, np.float32), np.array([1, -2, 3], np.float32))
    assert np.all(z == 0)
    assert np.all(orc.silu_and_mul(g, np.zeros_like(u)) == 0)
    big = np.array([20.0, 40.0, 88.0], np.float32)
    assert np.array_equal(orc.silu_and_mul(big, np.full(3, 3.0, np.float32)), big * np.float32(3.0))
    neg = orc.silu_and_mul(np.array([-90.0, -200.0], np.float32), np.ones(2, np.float32))
    assert np.all(np.abs(neg) < 1e-35) and np.all(neg <= 0)
    a = orc.silu_and_mul(g, np.ones_like(g)).astype(np.float64)
    b = orc.silu_and_mul(-g, np.ones_like(g)).astype(np.float64)
    assert np.all(np.abs((a - b) - g64) <= 8 * np.spacing(np.abs(g)).astype(np.float64) + 1e-30)


# ------------------------------------------------------------ f16 activation format

def test_act_f16_invariants(orc):
    """The f16 activation layout (no reference counterpart beyond the f16
    cast of convert.cu:91): the row scale is a power of two placing the row
    maximum in [256, 512); decoding the stored f16 values times the scale
    gives x back to f16 rounding; the stored order within each group of four
    is (x0, x2, x1, x3) (checked on exactly representable values); block sums
    hi + lo equal the exact sum of the block's 32 f16 values where that sum is
    exact in f32, and agree to f32 rounding elsewhere; an all-zero row has
    scale 1 and zeros."""
    rng = np.random.default_rng(5)
    rows, k = 6, 512
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[1] *= np.float32(3e5)
    x[2] *= np.float32(1e-6)
    x[3] = 0
    x[4] = (np.arange(k) - 250).astype(np.float32)   # max 261: scale 1, exact
    xh, xsx, xrs = orc.act_f16(x)
    for r in (0, 1, 2, 4):
        s = float(xrs[r])
        assert s == 2.0 ** round(np.log2(s))
        mx = np.max(np.abs(x[r])) / s
        assert 256 <= mx < 512
    assert xrs[3] == 1 and np.all(xh[3] == 0)
    h = xh.view(np.float16).astype(np.float64).reshape(rows, k // 4, 4)[:, :, [0, 2, 1, 3]].reshape(rows, k)
    dec = h * xrs[:, None].astype(np.float64)
    assert np.all(np.abs(dec - x) <= np.abs(x) * 2.0 ** -11 + 1e-30)
    # stored order on exact integers: stored[4i + 1] = x[4i + 2], stored[4i + 2] = x[4i + 1]
    st = xh[4].view(np.float16).astype(np.float64).reshape(k // 4, 4)
    xi = x[4].astype(np.float64).reshape(k // 4, 4)
    assert np.array_equal(st, xi[:, [0, 2, 1, 3]])
    sx = xsx.view(np.float16).astype(np.float64)
    tot = (sx[..., :8] + sx[..., 8:]).reshape(rows, k // 32)
    exact = h.reshape(rows, k // 32, 32).sum(axis=2)
    assert np.array_equal(tot[4], exact[4])
    assert np.all(np.abs(tot - exact) <= np.abs(exact) * 2.0 ** -20 + 1e-3 * 2.0 ** -10)


# ------------------------------------------------------------ f16-operand GEMM model

def _q6k_block(d, sc, q):
    """One Q6_K block: ql[128], qh[64], scales[16] (int8), d f16 from 256 six-bit codes
    in element order (dequant.rs:414-445 layout)."""
    blk = bytearray(210)
    for h in range(2):
        for l in range(32):
            q0, q1, q2, q3 = (q[128 * h + l + 32 * j] for j in range(4))
            blk[64 * h + l] = (q0 & 15) | ((q2 & 15) << 4)
            blk[64 * h + 32 + l] = (q1 & 15) | ((q3 & 15) << 4)
            blk[128 + 32 * h + l] = (q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6)
    blk[192:208] = np.asarray(sc, np.int8).tobytes()
    blk[208:210] = bytes(f16b(d))
    return bytes(blk)


@pytest.mark.parametrize("ty", [Q4K, Q6K, Q8_0])
def test_mmqh_model_reference_exact_case(orc, ty):
    """Where every f16 rounding of the f16-operand model is exact (integer
    activations with row maxima in [256, 512): scale 1; power-of-two d and
    dmin with small scales: exact weight operands and constant parts), the
    model equals dequant + f64 matmul bit for bit; a dropped constant part,
    a wrong nibble or qh bit order, or a missing x16 on the high-nibble codes
    breaks the equality."""
    rng = np.random.default_rng(8)
    n, k, rows = 5, 512, 3
    nsb = k // 256
    blocks = []
    for _ in range(n * nsb):
        if ty == Q4K:
            sc = rng.integers(0, 64, 8).tolist()
            m = rng.integers(0, 64, 8).tolist()
            blocks.append(_q4k_block(2.0 ** -4, 2.0 ** -5, sc, m, rng.integers(0, 16, 256).tolist(),
                                     rng.integers(0, 16, 256).tolist()))
        elif ty == Q6K:
            blocks.append(_q6k_block(2.0 ** -6, rng.integers(-15, 16, 16), rng.integers(0, 64, 256).tolist()))
        else:   # eight Q8_0 blocks: power-of-two d (exact f16(q * d)), codes over all of int8
            for _ in range(8):
                d = 2.0 ** int(rng.integers(-9, -3))
                blocks.append(bytes(f16b(d)) + rng.integers(-128, 128, 32).astype(np.int8).tobytes())
    w = np.frombuffer(b"".join(blocks), np.uint8).copy()
    x = rng.integers(-300, 301, (rows, k)).astype(np.float32)
    x[:, 7] = 300
    got = orc.mmqh_model_reference(ty, w, n, k, x)
    want = orc.reference_gemm(ty, w, n, k, x)
    assert np.array_equal(got, want)
    # and on random data the model stays within f16 rounding of the reference
    w2 = orc.synthetic(ty, k, 64, 9)
    x2 = rng.standard_normal((4, k)).astype(np.float32)
    e = orc.rel_err_row_l2(orc.mmqh_model_reference(ty, w2, 64, k, x2), orc.reference_gemm(ty, w2, 64, k, x2))
    assert e < 1e-3
