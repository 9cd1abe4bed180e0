"""rfxq_gemm_no_alloc: the GEMM entry point that allocates nothing (its
workspace is the library's fixed per-GPU scratch array). It must give
rfxq_gemm's results bit for bit, call after call, including a second call
with a smaller input that finds the first call's data in the scratch."""
import numpy as np
import pytest
import torch

from reflex_amd import synth

pytestmark = pytest.mark.gpu

Q4K, Q6K, Q8_0 = 12, 14, 8
DEV = "cuda:0"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _pair(rq, x, w, rows):
    want = rq.gemm(x, w, rows)
    got = torch.full((rows * w.out_features,), float("nan"), device=DEV)
    rq.gemm_no_alloc(x, w, rows, got)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("ty,n,k,rows", [
    (Q4K, 4096, 4096, (512, 300)),   # f16 MMQ with split-K (8 splits), then fewer rows
    (Q6K, 1024, 3072, (512, 77)),    # Q6_K f16 MMQ
    (Q4K, 2048, 1024, (12, 5)),      # few rows: 32-row tiles
    (Q8_0, 1024, 1024, (64, 2)),     # Q8_0: f16 MMQ, then GEMV rows
    (Q8_0, 4096, 4096, (512, 9)),    # Q8_0 f16 MMQ, 128- then 32-row tiles
    (Q4K, 2048, 1024, (1, 1)),       # one row: the decode GEMV
    (Q6K, 4096, 14336, (2, 1)),      # long rows (several passes per row) at a few rows, then one
    (Q6K, 4096, 14336, (3, 2)),      # a large matrix at 3 rows (32-row tiles), then GEMV rows
    (Q4K, 1024, 14336, (4, 2)),
])
def test_no_alloc_matches_gemm_two_calls(rq, ty, n, k, rows):
    w = rq.Weight.from_blocks(ty, synth.weights(ty, n, k, 300 + n), k, n, device=DEV)
    for i, m in enumerate(rows):
        x = _dev(synth.activations(m * k, 310 + i))
        got, want = _pair(rq, x, w, m)
        assert torch.equal(got, want), f"call {i}: rows={m}"


def test_no_alloc_int8_path(rq, opts):
    opts(mmq_f16=0)
    n, k = 640, 2048
    w = rq.Weight.from_blocks(Q4K, synth.weights(Q4K, n, k, 320), k, n, device=DEV)
    for i, m in enumerate((257, 40)):
        x = _dev(synth.activations(m * k, 321 + i))
        got, want = _pair(rq, x, w, m)
        assert torch.equal(got, want), f"call {i}: rows={m}"


def test_no_alloc_rejects_beyond_scratch(rq):
    # 4096 rows of in_features 16384: 128 MiB of f16 activations alone
    n, k, m = 256, 16384, 4096
    w = rq.Weight.from_blocks(Q4K, synth.weights(Q4K, n, k, 330), k, n, device=DEV)
    assert rq.gemm_workspace_size(w, m) > 128 << 20
    x = torch.zeros(m * k, device=DEV)
    y = torch.empty(m * n, device=DEV)
    with pytest.raises(rq.InvalidInputError, match="bytes of scratch"):
        rq.gemm_no_alloc(x, w, m, y)
