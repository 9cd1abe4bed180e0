"""CPU tests of the product's host side: the C-ABI library loads and exports
every symbol include/rfxq.h declares, host-only logic (router, expert slicing,
block dims) matches the reference semantics, and precondition failures return
the reference's error kinds before anything touches a GPU (kernels.rs:2118-2130).
No compute call runs here."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    import reflex_amd

    if not os.path.exists(reflex_amd.LIB_PATH):
        from reflex_amd import build

        build.build()
    return reflex_amd


def test_exports_every_header_symbol():
    rq = _lib()
    hdr = open(os.path.join(ROOT, "include", "rfxq.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    declared = set(re.findall(r"\b(rfxq_[a-z0-9_]+)\s*\(", hdr))
    assert len(declared) >= 20
    L = rq.lib()
    for name in sorted(declared):
        assert hasattr(L, name), name
    assert declared == set(rq.SIGNATURES), declared ^ set(rq.SIGNATURES)


def test_error_state_resets_on_success():
    """The thread's last error is cleared by the next successful call."""
    rq = _lib()
    with pytest.raises(rq.ReflexError):
        rq.ggml_type_block_dims(99)
    assert rq.lib().rfxq_last_error_code() == 1
    assert rq.ggml_type_block_dims(rq.GgmlType.Q8_0) == (32, 34)
    assert rq.lib().rfxq_last_error_code() == 0


def test_block_dims_and_unknown_type():
    rq = _lib()
    assert rq.ggml_type_block_dims(rq.GgmlType.Q4K) == (256, 144)
    assert rq.ggml_type_block_dims(rq.GgmlType.Q6K) == (256, 210)
    assert rq.ggml_type_block_dims(rq.GgmlType.Q8_0) == (32, 34)
    assert rq.ggml_type_block_dims(rq.GgmlType.Q8_1) == (32, 36)
    with pytest.raises(rq.GgmlError) as e:
        rq.ggml_type_block_dims(999)
    assert "unknown ggml_type=999" in str(e.value)
    assert rq.lib().rfxq_last_error_code() == 1


def _w(rq, ty, k, n, length=None, data=4096, e=0):
    return rq.RfxqWeight(ty, k, n, e, data, length if length is not None else 10**9)


def _call_gemv(rq, w, x_len):
    return rq.lib().rfxq_gemv_to(ctypes.c_void_p(4096), x_len, ctypes.byref(w), ctypes.c_void_p(4096), None)


def test_gemv_preconditions_fail_before_gpu():
    rq = _lib()
    L = rq.lib()
    # K not a multiple of 256 (kernels.rs:2124)
    assert _call_gemv(rq, _w(rq, 12, 300, 8), 300) == 12
    assert "multiple of 256" in L.rfxq_last_error().decode()
    # x.len() != in_features
    assert _call_gemv(rq, _w(rq, 12, 512, 8), 511) == 12
    assert "x.len()=511" in L.rfxq_last_error().decode()
    # a type without a kernel
    assert _call_gemv(rq, _w(rq, 2, 512, 8), 512) == 1
    # too few bytes for the shape
    assert _call_gemv(rq, _w(rq, 12, 512, 8, length=144 * 2 * 8 - 1), 512) == 12
    # Q4_K data must be 16-byte aligned, Q6_K 2-byte aligned
    assert _call_gemv(rq, _w(rq, 12, 512, 8, data=4096 + 8), 512) == 12
    assert _call_gemv(rq, _w(rq, 14, 512, 8, data=4096 + 1), 512) == 12
    # 3-D expert tensors must be sliced first
    assert _call_gemv(rq, _w(rq, 12, 512, 8, e=4), 512) == 12


def test_gemm_preconditions_fail_before_gpu():
    rq = _lib()
    L = rq.lib()
    w = _w(rq, 12, 512, 8)
    rc = L.rfxq_gemm(ctypes.c_void_p(4096), 512 * 3 - 1, ctypes.byref(w), 3, ctypes.c_void_p(4096), None, 0, None)
    assert rc == 12 and "rows*in_features" in L.rfxq_last_error().decode()
    # the MMQ kernels need K % 256 (Q4_K / Q6_K always; Q8_0 on the int8
    # kernels; in f16 mode Q8_0 rows run as GEMVs, which take K % 32)
    w6 = _w(rq, 14, 256, 8)
    w6.in_features = 96
    rc = L.rfxq_gemm(ctypes.c_void_p(4096), 96 * 3, ctypes.byref(w6), 3, ctypes.c_void_p(4096), None, 0, None)
    assert rc == 12 and "multiple of 256" in L.rfxq_last_error().decode()


def test_quant_expert_weight_slices_bytes():
    """kernels.rs:2656-2694: expert e's slice at offset + e*len/E."""
    rq = _lib()
    L = rq.lib()
    w = _w(rq, 12, 2048, 768, length=128 * 768 * 8 * 144, e=128)
    out = rq.RfxqWeight()
    assert L.rfxq_quant_expert_weight(ctypes.byref(w), 5, ctypes.byref(out)) == 0
    assert out.data == 4096 + 5 * 768 * 8 * 144 and out.len == 768 * 8 * 144
    assert (out.in_features, out.out_features, out.expert_count) == (2048, 768, 0)
    assert L.rfxq_quant_expert_weight(ctypes.byref(w), 128, ctypes.byref(out)) == 12
    w2 = _w(rq, 12, 2048, 768)
    assert L.rfxq_quant_expert_weight(ctypes.byref(w2), 0, ctypes.byref(out)) == 12
    assert "3-D" in L.rfxq_last_error().decode()


def test_router_matches_oracle_bitwise(orc):
    rq = _lib()
    rng = np.random.default_rng(12)
    for trial in range(200):
        n = int(rng.integers(1, 160))
        k = int(rng.integers(1, n + 1))
        lg = (rng.standard_normal(n) * rng.uniform(0.1, 8)).astype(np.float32)
        if trial % 7 == 0:
            lg[: n // 2] = lg[0]  # ties
        for norm in (True, False):
            got = rq.route_top_k_with_norm(lg, k, norm)
            want = orc.route_top_k(lg, k, norm)
            assert [i for i, _ in got] == [i for i, _ in want]
            assert np.array_equal(np.float32([w for _, w in got]), np.float32([w for _, w in want]))


def test_router_errors():
    rq = _lib()
    for lg, k in [([], 1), ([1.0, 2.0], 3), ([1.0, 2.0], 0), ([-np.inf, -np.inf], 1)]:
        with pytest.raises(rq.ReflexError):
            rq.route_top_k(np.array(lg, dtype=np.float32), k)
    r = rq.route_top_k(np.log(np.array([1, 2, 3, 4], dtype=np.float32)), 2)
    assert [i for i, _ in r] == [3, 2]


def test_moe_ffn_grouped_shape_errors():
    rq = _lib()
    L = rq.lib()
    g = _w(rq, 12, 2048, 768, e=4)
    d = _w(rq, 12, 768, 1024, e=4)  # wrong hidden
    lg = np.zeros(4 * 2, dtype=np.float32)
    rc = L.rfxq_moe_ffn_grouped(ctypes.c_void_p(4096), 2, 2048, lg.ctypes.data, 4, 2, 1, 1.0, ctypes.byref(g),
                                ctypes.byref(g), ctypes.byref(d), ctypes.c_void_p(4096), None)
    assert rc == 12 and "shapes" in L.rfxq_last_error().decode()


def test_synth_generators_deterministic_and_distributed():
    from reflex_amd import synth

    a = synth.weights(synth.Q4K, 64, 1024, synth.seed_for(2, 3, 1))
    b = synth.weights(synth.Q4K, 64, 1024, synth.seed_for(2, 3, 1))
    c = synth.weights(synth.Q4K, 64, 1024, synth.seed_for(2, 3, 2))
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    blk = a.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.004 < float(d.mean()) < 0.012  # |N(0,1)|*0.01 has mean 0.008
    x = synth.activations(200000, 5)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    q8 = synth.weights(synth.Q8_0, 16, 1024, 7).reshape(-1, 34)[:, 2:].view(np.int8)
    assert q8.min() >= -127 and q8.max() <= 127
    assert synth.weight_bytes(synth.Q4K, 2048, 1024) == 1179648


def test_gate_up_silu_preconditions_fail_before_gpu():
    """rfxq_gemm_gate_up_silu_q8_1 checks its weights and buffers before any
    device work, and asks for no workspace on the fused (Q4_K pair-tile)
    path."""
    rq = _lib()
    L = rq.lib()
    f = L.rfxq_gemm_gate_up_silu_q8_1
    act, y = ctypes.c_void_p(4096), ctypes.c_void_p(8192)
    g4 = _w(rq, 12, 1024, 768)
    u6 = _w(rq, 14, 1024, 768)
    u4n = _w(rq, 12, 1024, 512)
    for up in (u6, u4n):  # another type, another shape
        rc = f(act, 4, ctypes.byref(g4), ctypes.byref(up), act, y, None, 0, None)
        assert rc == 12 and "share a type and shape" in L.rfxq_last_error().decode()
    rc = f(ctypes.c_void_p(4096 + 16), 4, ctypes.byref(g4), ctypes.byref(g4), act, y, None, 0, None)
    assert rc == 12 and "256-byte aligned" in L.rfxq_last_error().decode()
    rc = f(act, 4, ctypes.byref(g4), ctypes.byref(g4), act, ctypes.c_void_p(8192 + 4), None, 0, None)
    assert rc == 11 and "16-byte aligned" in L.rfxq_last_error().decode()
    rc = f(act, 0, ctypes.byref(g4), ctypes.byref(g4), act, y, None, 0, None)
    assert rc == 12
    assert L.rfxq_gemm_gate_up_silu_workspace_size(ctypes.byref(g4), 64) == 0
    # the separate form (Q6_K): the two outputs, then the GEMMs' split-K partials
    assert L.rfxq_gemm_gate_up_silu_workspace_size(ctypes.byref(_w(rq, 14, 1024, 768)), 64) >= 2 * 64 * 768 * 4
