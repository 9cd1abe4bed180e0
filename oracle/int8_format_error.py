"""The per-32 int8 activation format's own error at the BASELINE shapes.

Test infrastructure, not product code: for each config 3 (Qwen3-0.6B layer)
and config 4 (Qwen3-8B layer, LM head) GEMM at M = 512, the exact model of
the int8 MMQ path (oracle.mmq_model_reference: activations quantized per 32
to int8 with an f16 scale, Q8_1; everything else exact) against the north
star's reference (dequant.rs + f64 matmul), as the north star's metric (max
over rows of max |error| / row L2 norm). Rows are sampled at the 8B shapes.
The same for the f16-operand path (oracle.mmqh_model_reference) as the
comparison. Seeded synthetic weights and N(0,1) activations (reflex_amd.synth).

    python -m oracle.int8_format_error
"""
from __future__ import annotations

import numpy as np

import oracle as orc
from reflex_amd import synth


def main() -> None:
    cases = [(3, i, c) for i, c in enumerate(synth.QWEN3_06B_LAYER)]
    cases += [(4, i, c) for i, c in enumerate(synth.QWEN3_8B_LAYER)] + [(4, 9, synth.LM_HEAD)]
    print("| config | GEMM | type | N x K | rows | int8 (Q8_1) format error | f16-operand path error |")
    print("|---|---|---|---|---|---|---|")
    for cfg, i, (name, ty, n, k) in cases:
        seed = synth.seed_for(cfg, 0, i)
        w = synth.weights(ty, n, k, seed)
        rows = 512 if cfg == 3 else 32
        x = synth.activations(rows * k, seed + 1000).reshape(rows, k)
        ref = np.empty((rows, n), np.float64)
        m8 = np.empty((rows, n), np.float64)
        mh = np.empty((rows, n), np.float64)
        qk, bb = orc.BLOCK_DIMS[ty]
        rb = k // qk * bb
        for c0 in range(0, n, 8192):   # column chunks: bounded memory
            c1 = min(n, c0 + 8192)
            wc = np.ascontiguousarray(w[c0 * rb:c1 * rb])
            ref[:, c0:c1] = orc.reference_gemm(ty, wc, c1 - c0, k, x)
            m8[:, c0:c1] = orc.mmq_model_reference(ty, wc, c1 - c0, k, x)
            mh[:, c0:c1] = orc.mmqh_model_reference(ty, wc, c1 - c0, k, x)
        e8, eh = orc.rel_err_row_l2(m8, ref), orc.rel_err_row_l2(mh, ref)
        tn = {synth.Q4K: "Q4_K", synth.Q6K: "Q6_K", synth.Q8_0: "Q8_0"}[ty]
        print(f"| {cfg} | {name} | {tn} | {n} x {k} | {rows} | {e8:.2e} | {eh:.2e} |", flush=True)


if __name__ == "__main__":
    main()
