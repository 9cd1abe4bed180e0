"""Writes tests/golden/fixtures.npz: small golden vectors of the quantized-matmul
path, produced by the CPU oracle (oracle/) after it is pinned by
tests/test_oracle.py. GPU tests compare against these committed values as well
as against the oracle at run time.

Contents (reference test generators, src/model/quant_resident_tests.rs:907-925,
quant_mma_tests.rs:64-84, quant_resident_tests.rs:669-692, activations LCG :40-52):
  {q4k,q6k,q8_0}_w      raw blocks of an [8 x 512] weight
  {..}_deq              dequantized f32 (src/dequant.rs semantics)
  {..}_dots             per-32 int32 dots with the quantized activations
  {..}_y                dequant + f64 host matmul of x (3 rows)
  x, xq, xds            activations and their Q8_1 quantization

Run: python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402

N, K, M = 8, 512, 3


def main():
    out = {}
    x = oracle.activations(M * K, 0xAC7).reshape(M, K)
    xq, xds = oracle.quantize_q8_1(x)
    out.update(x=x, xq=xq, xds=xds)
    for ty, name, seed in [(oracle.Q4K, "q4k", 41), (oracle.Q6K, "q6k", 42), (oracle.Q8_0, "q8_0", 43)]:
        w = oracle.synthetic(ty, K, N, seed)
        out[f"{name}_w"] = w
        out[f"{name}_shape"] = np.array([N, K])
        out[f"{name}_deq"] = oracle.dequantize(ty, w, N * K)
        out[f"{name}_dots"] = oracle.block_dots(ty, w, N, K, xq)
        out[f"{name}_y"] = oracle.reference_gemm(ty, w, N, K, x)
    np.savez_compressed(os.path.join(HERE, "fixtures.npz"), **out)


if __name__ == "__main__":
    main()
