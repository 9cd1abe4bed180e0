"""TEST INFRASTRUCTURE ONLY: the CPU oracle for the GGUF quantized-matmul path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline). The product package ``reflex_amd`` never imports it.

The numerics live in ``oracle.c`` (a C restatement of the reference's
``src/dequant.rs`` and friends, built with ``-ffp-contract=off``); this module
is a thin numpy/ctypes wrapper. Each function names the reference code it
follows in ``oracle.c``'s header.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

F32, F16, Q8_0, Q8_1, Q4K, Q6K = 0, 1, 8, 9, 12, 14
BLOCK_DIMS = {Q8_0: (32, 34), Q8_1: (32, 36), Q4K: (256, 144), Q6K: (256, 210)}

_lib = None


def build() -> None:
    """Compile liboracle.so from oracle.c (make)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, u64, i32 = ctypes.c_long, ctypes.c_uint64, ctypes.c_int
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_get_scale_min_k4.argtypes = [i32, P, P, P]
        L.oracle_dequantize.argtypes = [i32, P, ctypes.c_size_t, u64, P]
        L.oracle_dequantize.restype = i64
        L.oracle_quantize_q8_1.argtypes = [P, i64, i64, P, P]
        L.oracle_block_dots.argtypes = [i32, P, i64, i64, P, i64, P]
        L.oracle_block_dots.restype = i32
        L.oracle_host_matmul.argtypes = [P, P, i64, i64, i64, P]
        for name in ("oracle_synthetic_q4k", "oracle_synthetic_q6k", "oracle_synthetic_q8_0"):
            getattr(L, name).argtypes = [i64, i64, u64, P]
        L.oracle_activations.argtypes = [i64, u64, P]
        L.oracle_route_top_k.argtypes = [P, i64, i64, i32, P, P]
        L.oracle_route_top_k.restype = i32
        L.oracle_silu_and_mul.argtypes = [P, P, P, i64]
        L.oracle_rmsnorm.argtypes = [P, P, P, i64, i64, ctypes.c_float]
        L.oracle_cpu_dequant_matmul.argtypes = [i32, P, i64, i64, P, i64, P, i32]
        L.oracle_cpu_dequant_matmul.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(bits: int) -> float:
    return lib().oracle_f16_to_f32(bits)


def f32_to_f16(v: float) -> int:
    return lib().oracle_f32_to_f16(v)


def get_scale_min_k4(j: int, scales: bytes) -> tuple[int, int]:
    q = np.frombuffer(bytes(scales), dtype=np.uint8).copy()
    d = ctypes.c_uint8()
    m = ctypes.c_uint8()
    lib().oracle_get_scale_min_k4(j, _p(q), ctypes.byref(d), ctypes.byref(m))
    return d.value, m.value


def dequantize(ty: int, data, element_count: int) -> np.ndarray:
    """dequant.rs:53 ``dequantize``: raw bytes -> f32, truncated to element_count.

    Raises ValueError for a type without a dequantizer (the reference's Err)."""
    buf = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else np.ascontiguousarray(data, dtype=np.uint8)
    if ty in BLOCK_DIMS:
        qk, bb = BLOCK_DIMS[ty]
        cap = (buf.size // bb) * qk
    elif ty == F32:
        cap = buf.size // 4
    elif ty == F16:
        cap = buf.size // 2
    else:
        raise ValueError(f"unknown ggml_type={ty}: no dequantizer known for it")
    out = np.zeros(max(cap, 1), dtype=np.float32)
    n = lib().oracle_dequantize(ty, _p(buf), buf.size, element_count, _p(out))
    if n < 0:
        raise ValueError(f"unknown ggml_type={ty}: no dequantizer known for it")
    return out[:n].copy()


def quantize_q8_1(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-32 Q8_1 activation quantization. Returns (qs int8 [rows,k], ds uint16 [rows,k/32,2])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    qs = np.zeros((rows, k), dtype=np.int8)
    ds = np.zeros((rows, k // 32, 2), dtype=np.uint16)
    lib().oracle_quantize_q8_1(_p(x), rows, k, _p(qs), _p(ds))
    return qs, ds


def block_dots(ty: int, w: np.ndarray, n: int, k: int, qa: np.ndarray) -> np.ndarray:
    """int32 [m, n, k/32] per-32 dots of quantized activations with weight codes."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    m = qa.shape[0]
    out = np.zeros((m, n, k // 32), dtype=np.int32)
    rc = lib().oracle_block_dots(ty, _p(w), n, k, _p(qa), m, _p(out))
    if rc != 0:
        raise ValueError(f"block_dots: unsupported type {ty}")
    return out


def host_matmul(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """quant_resident_tests.rs:709-729: x[rows,in] @ w[out,in]^T in f64, result f32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, in_f = x.shape
    out_f = w.shape[0]
    y = np.zeros((rows, out_f), dtype=np.float32)
    lib().oracle_host_matmul(_p(x), _p(w), rows, in_f, out_f, _p(y))
    return y


def dequant_matrix(ty: int, w: np.ndarray, n: int, k: int) -> np.ndarray:
    return dequantize(ty, w, n * k).reshape(n, k)


def reference_gemm(ty: int, w: np.ndarray, n: int, k: int, x: np.ndarray) -> np.ndarray:
    """The north star's reference: dequant.rs dequantization + f64 host matmul."""
    x2 = x.reshape(-1, k)
    return host_matmul(x2, dequant_matrix(ty, w, n, k))


def synthetic(ty: int, in_f: int, out_f: int, seed: int) -> np.ndarray:
    """The reference tests' xorshift64 weight generators."""
    qk, bb = BLOCK_DIMS[ty]
    out = np.zeros(in_f // qk * out_f * bb, dtype=np.uint8)
    fn = {Q4K: "oracle_synthetic_q4k", Q6K: "oracle_synthetic_q6k", Q8_0: "oracle_synthetic_q8_0"}[ty]
    getattr(lib(), fn)(in_f, out_f, seed, _p(out))
    return out


def activations(n: int, seed: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().oracle_activations(n, seed, _p(out))
    return out


def route_top_k(logits, k: int, normalize: bool = True) -> list[tuple[int, float]]:
    """moe.rs:47-98 route_top_k_with_norm. Raises ValueError on the reference's errors."""
    lg = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    idx = np.zeros(max(k, 1), dtype=np.int32)
    w = np.zeros(max(k, 1), dtype=np.float32)
    rc = lib().oracle_route_top_k(_p(lg) if lg.size else None, lg.size, k, int(normalize), _p(idx), _p(w))
    if rc != 0:
        raise ValueError("route_top_k: invalid logits or k")
    return [(int(i), float(v)) for i, v in zip(idx[:k], w[:k])]


def silu_and_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.zeros_like(g)
    lib().oracle_silu_and_mul(_p(g), _p(u), _p(out), g.size)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, rows: int, k: int, eps: float) -> np.ndarray:
    """rmsnorm.cu:18-55 / rmsnorm.cuh:17-41 (sequential fused sum of squares)."""
    xx = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    ww = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    out = np.zeros(rows * k, dtype=np.float32)
    lib().oracle_rmsnorm(_p(xx), _p(ww), _p(out), rows, k, ctypes.c_float(eps))
    return out.reshape(rows, k)


def moe_ffn_grouped_reference(x, routes, gate_w, up_w, down_w, ty, hidden, ffn, n_experts, down_ty=None):
    """dense.rs:1509-1559 semantics on the host: for each expert, gather its rows,
    gate/up GEMM, silu*up, down GEMM, weighted scatter-add. f64 matmuls on the
    dequantized expert slices (quant_expert_weight: kernels.rs:2656-2694).
    `down_ty` is the down projection's type when it differs (Q4_K_M files
    store it as Q6_K)."""
    rows = x.shape[0]
    out = np.zeros((rows, hidden), dtype=np.float32)
    groups = [[] for _ in range(n_experts)]
    for r, picks in enumerate(routes):
        for e, wgt in picks:
            groups[e].append((r, wgt))
    g_len = gate_w.size // n_experts
    d_len = down_w.size // n_experts
    for e, grp in enumerate(groups):
        if not grp:
            continue
        rr = np.array([r for r, _ in grp])
        ww = np.array([w for _, w in grp], dtype=np.float32)
        xe = x[rr]
        g = reference_gemm(ty, gate_w[e * g_len:(e + 1) * g_len], ffn, hidden, xe)
        u = reference_gemm(ty, up_w[e * g_len:(e + 1) * g_len], ffn, hidden, xe)
        a = silu_and_mul(g, u)
        dn = reference_gemm(ty if down_ty is None else down_ty, down_w[e * d_len:(e + 1) * d_len], hidden, ffn, a)
        out[rr] += ww[:, None] * dn
    return out


def cpu_dequant_matmul(ty: int, w: np.ndarray, n: int, k: int, x: np.ndarray, threads: int) -> np.ndarray:
    """The CPU baseline: dequant restatement + f32 matmul over `threads` OpenMP threads."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x2 = np.ascontiguousarray(x.reshape(-1, k), dtype=np.float32)
    y = np.zeros((x2.shape[0], n), dtype=np.float32)
    rc = lib().oracle_cpu_dequant_matmul(ty, _p(w), n, k, _p(x2), x2.shape[0], _p(y), threads)
    if rc != 0:
        raise ValueError(f"unsupported type {ty}")
    return y


def q4k_scale_min_np(w: np.ndarray, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Vectorised get_scale_min_k4 (dequant.rs:39-47) over every block: (sc, m) as
    int arrays [n, k/32] (checked against the C function in tests)."""
    b = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, k // 256, 144)
    q = b[:, :, 4:16].astype(np.int64)
    sc = np.zeros((n, k // 256, 8), dtype=np.int64)
    m = np.zeros((n, k // 256, 8), dtype=np.int64)
    for j in range(4):
        sc[..., j] = q[..., j] & 63
        m[..., j] = q[..., j + 4] & 63
    for j in range(4, 8):
        sc[..., j] = (q[..., j + 4] & 0xF) | ((q[..., j - 4] >> 6) << 4)
        m[..., j] = (q[..., j + 4] >> 4) | ((q[..., j] >> 6) << 4)
    return sc.reshape(n, k // 32), m.reshape(n, k // 32)


def mmq_model_reference(ty: int, w: np.ndarray, n: int, k: int, x: np.ndarray) -> np.ndarray:
    """The MMQ algorithm in exact (f64) arithmetic on the quantized activations:
    x_hat = f16(d) * q per 32-block (quantize_q8_1); for Q4_K the weights split as
    w = d*sc*(q - 8) + c with c = 8*d*sc - dmin*m, and the constant part c takes
    the block's activation sum d * s (s = f16(sum(x)/d)); Q6_K / Q8_0 use
    x_hat @ W^T. Any difference
    between the kernel and this is the kernel's own rounding."""
    x2 = np.ascontiguousarray(x.reshape(-1, k), dtype=np.float32)
    qs, ds = quantize_q8_1(x2)
    d = ds[..., 0].view(np.float16).astype(np.float64)
    xh = (qs.reshape(x2.shape[0], -1, 32).astype(np.float64) * d[..., None]).reshape(x2.shape[0], k)
    W = dequant_matrix(ty, w, n, k).astype(np.float64)
    if ty != Q4K:
        return (xh @ W.T).astype(np.float32)
    sc, m = q4k_scale_min_np(w, n, k)
    b = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, k // 256, 144)
    dd = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    dm = b[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    dsc = (np.repeat(dd, 8, axis=1) * sc.astype(np.float32)).astype(np.float64)   # f32 product, as dequant.rs
    dmw = (np.repeat(dm, 8, axis=1) * m.astype(np.float32)).astype(np.float64)
    c = 8.0 * dsc - dmw
    # centered part dsc * (q - 8), with the nibbles q read from the block bytes
    qb = b[:, :, 16:144]
    nib = np.empty((n, k // 256, 256), dtype=np.int64)
    for g in range(4):
        nib[:, :, 64 * g:64 * g + 32] = qb[:, :, 32 * g:32 * g + 32] & 15
        nib[:, :, 64 * g + 32:64 * g + 64] = qb[:, :, 32 * g:32 * g + 32] >> 4
    wc = np.repeat(dsc, 32, axis=1) * (nib.reshape(n, k) - 8)
    sx = ds[..., 1].view(np.float16).astype(np.float64) * d  # [rows, k/32]: d * f16(sum(x)/d)
    return (xh @ wc.T + sx @ c.T).astype(np.float32)


def rel_max_diff(a: np.ndarray, b: np.ndarray) -> float:
    """quant_resident_tests.rs:6-10: max|a-b| / max|b|."""
    scale = max(float(np.max(np.abs(b))), 1e-30)
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64)))) / scale


def rel_err_row_l2(y: np.ndarray, ref: np.ndarray) -> float:
    """The north star's metric: max over output rows of max|y - ref| / ||ref_row||_2."""
    y2 = y.reshape(-1, y.shape[-1]).astype(np.float64)
    r2 = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    num = np.max(np.abs(y2 - r2), axis=1)
    den = np.maximum(np.linalg.norm(r2, axis=1), 1e-30)
    return float(np.max(num / den))


# ---------------------------------------------------------------- f16 activation format
#
# The prefill GEMM's activation input (no reference counterpart beyond the f16
# cast of src/kernels_cuda/convert.cu:91, which saturates at 65504 instead of
# scaling): per row, e = ilogb(max|x|) - 8 clamped to [-120, 120] (0 for an
# all-zero or non-finite max), xh = f16_rne(x * 2^-e) stored with each group of
# four as (x0, x2, x1, x3), block sums of the 32 f16 values per 32-block in a
# fixed f32 order (lane partials ((h0+h1)+h2)+h3 over 8 lanes, then
# ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7))) split into f16 hi and lo, and the row
# scale 2^e.

def act_f16(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Returns (xh u16 [rows, k] in the stored order, xsx u16 [rows, k/256, 16], xrs f32 [rows])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    mx = np.max(np.abs(x), axis=1) if k else np.zeros(rows, np.float32)
    ok = (mx > 0) & np.isfinite(mx)
    ex = np.frexp(np.where(ok, mx, 1.0).astype(np.float64))[1] - 1   # ilogb
    e = np.where(ok, np.clip(ex - 8, -120, 120), 0).astype(np.int64)
    scale = np.ldexp(np.float32(1.0), -e).astype(np.float32)
    h = (x * scale[:, None]).astype(np.float32).astype(np.float16)
    xh = h.reshape(rows, k // 4, 4)[:, :, [0, 2, 1, 3]].reshape(rows, k)
    hf = h.astype(np.float32).reshape(rows, k // 32, 8, 4)
    p = ((hf[..., 0] + hf[..., 1]) + hf[..., 2]) + hf[..., 3]           # [rows, blocks, 8] f32
    u = (p[..., 0] + p[..., 1]) + (p[..., 2] + p[..., 3])
    v = (p[..., 4] + p[..., 5]) + (p[..., 6] + p[..., 7])
    s = (u + v).astype(np.float32)
    hi = s.astype(np.float16)
    lo = (s - hi.astype(np.float32)).astype(np.float16)
    xsx = np.concatenate([hi.reshape(rows, k // 256, 8), lo.reshape(rows, k // 256, 8)], axis=2)
    xrs = np.ldexp(np.float32(1.0), e).astype(np.float32)
    return xh.view(np.uint16), xsx.view(np.uint16), xrs


def _f16(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float64)


def mmqh_model_reference(ty: int, w: np.ndarray, n: int, k: int, x: np.ndarray) -> np.ndarray:
    """The f16-activation prefill GEMM's arithmetic in exact (f64) arithmetic on
    its own operands: f16 activations (act_f16) and the f16 weight operands.
    Q4_K: f16((q-8) * f16(d*sc)) for the low-nibble blocks and
    f16(16(q-8) * f16(d*sc/16)) for the high-nibble ones, plus the constant
    part f16(8*d*sc - dmin*m) against the f16 hi + lo block sums. Q6_K:
    f16((q-32) * f16(d*sc)) for codes from low nibbles, f16(16(q-32) *
    f16(d*sc/16)) for codes from high nibbles. Q8_0: f16(q * d). Any
    difference between the kernel and this is the
    kernel's own f32 accumulation."""
    x2 = np.ascontiguousarray(x.reshape(-1, k), dtype=np.float32)
    rows = x2.shape[0]
    xh, xsx, xrs = act_f16(x2)
    hv = xh.view(np.float16).reshape(rows, k // 4, 4)[:, :, [0, 2, 1, 3]].reshape(rows, k).astype(np.float64)
    if ty == Q4K:
        sc, m = q4k_scale_min_np(w, n, k)
        b = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, k // 256, 144)
        dd = np.repeat(b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32), 8, axis=1)
        dm = np.repeat(b[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32), 8, axis=1)
        scf, mf = sc.astype(np.float32), m.astype(np.float32)
        odd = (np.arange(scf.shape[1]) % 2 == 1)[None, :]
        s16 = _f16(dd * scf * np.where(odd, np.float32(0.0625), np.float32(1.0)))   # the block multipliers
        c16 = np.float32(8.0) * dd * scf - dm * mf                        # f32 fma ~ exact here
        c16 = _f16(c16)
        qb = b[:, :, 16:144]
        nib = np.empty((n, k // 256, 256), dtype=np.int64)
        for g in range(4):
            nib[:, :, 64 * g:64 * g + 32] = qb[:, :, 32 * g:32 * g + 32] & 15
            nib[:, :, 64 * g + 32:64 * g + 64] = qb[:, :, 32 * g:32 * g + 32] >> 4
        code = (nib.reshape(n, k) - 8).astype(np.float64) * np.repeat(np.where(odd, 16.0, 1.0), 32, axis=1)
        wop = _f16(code * np.repeat(s16, 32, axis=1))
        sx = (xsx.view(np.float16)[..., :8].astype(np.float64) + xsx.view(np.float16)[..., 8:].astype(np.float64))
        y = hv @ wop.T + sx.reshape(rows, -1) @ c16.T
    elif ty == Q6K:
        b = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, k // 256, 210)
        d = b[:, :, 208:210].copy().view(np.float16)[..., 0].astype(np.float32)
        sc = b[:, :, 192:208].view(np.int8).astype(np.float32)
        # per 16 codes f16(d*sc), applied to 16(q-32) as f16(d*sc/16) in the
        # groups whose codes come from the high nibbles (scales 4-7, 12-15)
        hi = (np.arange(16) % 8 >= 4)[None, None, :]
        s16 = _f16(d[:, :, None] * sc * np.where(hi, np.float32(0.0625), np.float32(1.0)))
        ql, qh = b[:, :, 0:128].astype(np.int64), b[:, :, 128:192].astype(np.int64)
        q = np.empty((n, k // 256, 256), dtype=np.int64)
        for h in range(2):
            L, H = ql[:, :, 64 * h:64 * h + 64], qh[:, :, 32 * h:32 * h + 32]
            q[:, :, 128 * h + 0:128 * h + 32] = (L[:, :, :32] & 15) | ((H & 3) << 4)
            q[:, :, 128 * h + 32:128 * h + 64] = (L[:, :, 32:] & 15) | (((H >> 2) & 3) << 4)
            q[:, :, 128 * h + 64:128 * h + 96] = (L[:, :, :32] >> 4) | (((H >> 4) & 3) << 4)
            q[:, :, 128 * h + 96:128 * h + 128] = (L[:, :, 32:] >> 4) | (((H >> 6) & 3) << 4)
        code = (q - 32).astype(np.float64) * np.repeat(np.where(hi, 16.0, 1.0), 16, axis=2)
        wop = _f16(code.reshape(n, k) * np.repeat(s16.reshape(n, -1), 16, axis=1))
        y = hv @ wop.T
    elif ty == Q8_0:
        # f16(q * d): one rounding of the exact product of the code and the f16 d
        b = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, k // 32, 34)
        d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
        q = b[:, :, 2:34].view(np.int8).astype(np.float64)
        wop = _f16(q * d[:, :, None]).reshape(n, k)
        y = hv @ wop.T
    else:
        raise ValueError("mmqh_model_reference: Q4_K, Q6_K and Q8_0 only")
    return (y * xrs[:, None].astype(np.float64)).astype(np.float32)
