"""CPU tests of the prefill switches and the GEMM path policy: the
environment is parsed once, strictly, with the reference's messages
(QuantMmaKernels::from_env, src/model/kernels.rs:747-802;
quant_fused_max_rows, :4186-4194), and rfxq_gemm_policy_for makes the
documented choices. No compute call runs here."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
Q8_0, Q4K, Q6K = 8, 12, 14
_ENV_NAMES = ("REFLEX_QUANT_MMA", "REFLEX_QUANT_MMA_SPLITS", "REFLEX_QUANT_MMA_MAX_ROWS", "REFLEX_QUANT_MMA_TILE",
              "REFLEX_MMQ_F16", "REFLEX_QUANT_FUSED_MAX_ROWS")


@pytest.fixture
def rq():
    import reflex_amd

    if not os.path.exists(reflex_amd.LIB_PATH):
        from reflex_amd import build

        build.build()
    prev = reflex_amd.get_options()
    yield reflex_amd
    reflex_amd.set_options(**prev)


_PROBE = r"""
import json, reflex_amd as r
try:
    print(json.dumps({"ok": r.get_options()}))
except r.ReflexError as e:
    print(json.dumps({"err": [e.code, str(e)]}))
"""


def _env_options(**env):
    """get_options() in a fresh process with exactly these REFLEX_* variables."""
    e = {k: v for k, v in os.environ.items() if k not in _ENV_NAMES}
    e.update(env)
    out = subprocess.run([sys.executable, "-c", _PROBE], cwd=ROOT, env=e, capture_output=True, text=True,
                         timeout=120, check=True).stdout
    import json

    return json.loads(out.strip().splitlines()[-1])


def test_env_defaults():
    assert _env_options() == {"ok": {"quant_mma": 1, "quant_mma_splits": 0, "quant_mma_max_rows": 0,
                                     "quant_mma_tile": 0, "mmq_f16": 1, "fused_max_rows": 16}}


def test_env_valid_values():
    got = _env_options(REFLEX_QUANT_MMA="0", REFLEX_QUANT_MMA_SPLITS="+3", REFLEX_QUANT_MMA_MAX_ROWS="0007",
                       REFLEX_QUANT_MMA_TILE="64", REFLEX_MMQ_F16="0", REFLEX_QUANT_FUSED_MAX_ROWS="4")["ok"]
    assert got == {"quant_mma": 0, "quant_mma_splits": 3, "quant_mma_max_rows": 7, "quant_mma_tile": 64,
                   "mmq_f16": 0, "fused_max_rows": 4}
    # empty strings take the defaults, as unset variables do
    assert _env_options(REFLEX_QUANT_MMA="", REFLEX_QUANT_MMA_TILE="")["ok"]["quant_mma"] == 1


@pytest.mark.parametrize("name,value,msg", [
    ("REFLEX_QUANT_MMA", "2", 'REFLEX_QUANT_MMA must be 1 (the default) or 0, got "2"'),
    ("REFLEX_QUANT_MMA", "01", 'REFLEX_QUANT_MMA must be 1 (the default) or 0, got "01"'),
    ("REFLEX_QUANT_MMA", "true", 'REFLEX_QUANT_MMA must be 1 (the default) or 0, got "true"'),
    ("REFLEX_QUANT_MMA_SPLITS", "0", 'REFLEX_QUANT_MMA_SPLITS must be a positive integer, got "0"'),
    ("REFLEX_QUANT_MMA_SPLITS", "-2", 'REFLEX_QUANT_MMA_SPLITS must be a positive integer, got "-2"'),
    ("REFLEX_QUANT_MMA_SPLITS", " 4", 'REFLEX_QUANT_MMA_SPLITS must be a positive integer, got " 4"'),
    ("REFLEX_QUANT_MMA_MAX_ROWS", "x", 'REFLEX_QUANT_MMA_MAX_ROWS must be a non-negative integer, got "x"'),
    ("REFLEX_QUANT_MMA_TILE", "96", 'REFLEX_QUANT_MMA_TILE must be 64 or 128, got "96"'),
    ("REFLEX_QUANT_MMA_TILE", "0", 'REFLEX_QUANT_MMA_TILE must be 64 or 128, got "0"'),
    ("REFLEX_MMQ_F16", "yes", 'REFLEX_MMQ_F16 must be 1 (the default) or 0, got "yes"'),
])
def test_env_invalid_is_invalid_input(name, value, msg):
    assert _env_options(**{name: value}) == {"err": [11, msg]}


def test_fused_max_rows_unparsable_keeps_default():
    """quant_fused_max_rows (kernels.rs:4186-4194) falls back to 16 silently."""
    assert _env_options(REFLEX_QUANT_FUSED_MAX_ROWS="lots")["ok"]["fused_max_rows"] == 16


def test_set_options_round_trip_and_rejects(rq):
    prev = rq.set_options(quant_mma_splits=5, fused_max_rows=2)
    got = rq.get_options()
    assert got["quant_mma_splits"] == 5 and got["fused_max_rows"] == 2
    for bad in ({"quant_mma_tile": 96}, {"quant_mma": 2}, {"mmq_f16": -1}):
        with pytest.raises(rq.InvalidInputError):
            rq.set_options(**bad)
        assert rq.get_options() == got   # a rejected set changes nothing
    with rq.options(mmq_f16=0):
        assert rq.get_options()["mmq_f16"] == 0
    assert rq.get_options() == got
    rq.set_options(**prev)


def test_policy_paths(rq):
    G, I8, F16 = rq.PATH_GEMV_ROWS, rq.PATH_MMQ_INT8, rq.PATH_MMQ_F16
    pol = rq.gemm_policy
    # one row, and up to 4 rows (within fused_max_rows): GEMVs; 5..32 rows:
    # 32 x 256 tiles (the fused few-row form), 33..64: 64 x 256, above: 128 x 256
    assert pol(Q4K, 1024, 2048, 1)["path"] == G
    assert pol(Q4K, 1024, 2048, 4)["path"] == G
    p = pol(Q4K, 1024, 2048, 5)
    assert (p["path"], p["tile_m"], p["tile_n"]) == (F16, 32, 256)
    assert [pol(Q4K, 1024, 2048, m)["tile_m"] for m in (32, 33, 64, 65)] == [32, 64, 64, 128]
    with rq.options(fused_max_rows=2):
        assert pol(Q4K, 1024, 2048, 3)["path"] == F16
    # 3-4 rows of a large matrix read it once on 32-row tiles: (rows - 1) x
    # its bytes of re-reads reach 56 MiB (8B gate 14336 x 4096 Q4_K, 33 MB;
    # down 4096 x 14336 Q6_K, 48 MB); 2 rows stay GEMVs
    assert pol(Q4K, 4096, 14336, 2)["path"] == G
    assert pol(Q4K, 4096, 14336, 3)["path"] == F16
    assert pol(Q6K, 14336, 4096, 3)["path"] == F16
    assert pol(Q4K, 4096, 4096, 4)["path"] == G          # 9.4 MB x 3: GEMVs when alone
    assert pol(Q8_0, 4096, 14336, 3)["path"] == F16
    with rq.options(mmq_f16=0):   # the int8 path keeps GEMVs up to fused_max_rows
        assert pol(Q4K, 1024, 2048, 16)["path"] == G
        assert pol(Q4K, 1024, 2048, 17)["path"] == I8
    # the f16 kernels take Q4_K, Q6_K (any super-block count per row) and Q8_0;
    # the default never picks the int8 format, whose error exceeds 1e-3
    for k in (256, 768, 1024, 1280):
        assert pol(Q6K, k, 1024, 512)["path"] == F16
    assert pol(Q8_0, 1024, 1024, 512)["path"] == F16
    assert pol(Q8_0, 1024, 1024, 5)["path"] == F16
    assert pol(Q8_0, 1024, 1024, 4)["path"] == G
    # weights far past 4 GiB: the kernels' buffers start at each tile
    assert pol(Q4K, 256, 40_000_000, 512)["path"] == F16
    with rq.options(mmq_f16=0):
        p = pol(Q8_0, 1024, 1024, 512)
        assert p["path"] == I8 and (p["tile_m"], p["tile_n"]) == (128, 128)
        assert pol(Q4K, 1024, 2048, 512)["path"] == I8
        with rq.options(quant_mma_tile=64):
            assert pol(Q4K, 1024, 2048, 512)["tile_m"] == 64
    # in_features not a multiple of 256: GEMVs
    assert pol(Q8_0, 1056, 64, 512)["path"] == G
    # the switches
    with rq.options(quant_mma=0):
        assert pol(Q4K, 1024, 2048, 512)["path"] == G
    with rq.options(quant_mma_max_rows=256):
        assert pol(Q4K, 1024, 2048, 512)["path"] == G
        assert pol(Q4K, 1024, 2048, 256)["path"] == F16
    with rq.options(fused_max_rows=0):
        assert pol(Q4K, 1024, 2048, 2)["path"] == F16


def test_policy_tiles_and_splits(rq):
    pol = rq.gemm_policy
    # 0.6B q_proj at M=512 alone: 4 x 8 tiles of 128 x 256 with at most
    # nsb / 2 = 2 splits cover 64 of 256 CUs' 512 places, under half: 64-row
    # tiles (8 x 8 x 2 splits = 128 workgroups)
    p = pol(Q4K, 1024, 2048, 512, 256)
    assert (p["tile_m"], p["tile_n"]) == (64, 256)
    assert (p["splits"], p["sb_per_split"]) == (2, 2)   # capped at nsb / 2 = 2 splits
    # config 1's 1024 x 1024 Q8_0 at M=512: 32-row tiles, one-super-block splits
    p = pol(8, 1024, 1024, 512, 256)
    assert (p["tile_m"], p["splits"], p["sb_per_split"]) == (32, 4, 1)
    # 255 rows keep the tile that holds them
    assert pol(Q4K, 1024, 2048, 255, 256)["tile_m"] == 128
    # 8B q_proj: 4 x 16 = 64 tiles -> ceil(512 / 64) = 8 splits of 2 super-blocks
    p = pol(Q4K, 4096, 4096, 512, 256)
    assert (p["splits"], p["sb_per_split"]) == (8, 2)
    # gate at 8B: 4 x 56 = 224 tiles, half the CUs covered -> no split
    p = pol(Q4K, 4096, 14336, 512, 256)
    assert (p["splits"], p["sb_per_split"]) == (1, 16)
    # fewer CUs: 64 tiles cover half of 128 CUs -> no split; of 160 -> ceil(320 / 64) = 5
    assert pol(Q4K, 4096, 4096, 512, 128)["splits"] == 1
    assert pol(Q4K, 4096, 4096, 512, 160)["splits"] == 4   # 5 splits of ceil(16 / 5) = 4 -> 4 ranges
    # forced splits; the last split may hold fewer super-blocks
    with rq.options(quant_mma_splits=3):
        p = pol(Q4K, 4096, 4096, 512)
        assert (p["splits"], p["sb_per_split"]) == (3, 6)
    with rq.options(quant_mma_splits=100):   # at most one split per super-block
        assert pol(Q4K, 4096, 4096, 512)["splits"] == 16
    # 32-row tiles: splits down to one super-block
    p = pol(Q4K, 4096, 4096, 12, 256)    # 16 tiles -> 32 wanted, 16 super-blocks
    assert (p["splits"], p["sb_per_split"]) == (16, 1)
    p = pol(Q6K, 14336, 4096, 12, 256)   # 16 tiles -> 32 splits of ceil(56 / 32) = 2 -> 28
    assert (p["splits"], p["sb_per_split"]) == (28, 2)
    # 64-row tiles: splits capped at nsb / 2 like the 128-row ones
    p = pol(Q4K, 4096, 4096, 48, 256)    # 16 tiles -> 32 wanted, capped at 16 / 2
    assert (p["tile_m"], p["splits"], p["sb_per_split"]) == (64, 8, 2)
    # Q6_K tiles are 128 x 256 too: down at 8B has 4 x 16 tiles -> 8 splits of 7 super-blocks
    p = pol(Q6K, 14336, 4096, 512, 256)
    assert (p["tile_m"], p["tile_n"], p["splits"], p["sb_per_split"]) == (128, 256, 8, 7)
    # v_proj at 8B: 4 x 4 tiles -> 32 splits, capped at nsb / 2 = 8
    assert pol(Q6K, 4096, 1024, 512, 256)["splits"] == 8


def test_policy_errors(rq):
    with pytest.raises(rq.GgmlError):
        rq.gemm_policy(2, 1024, 1024, 512)
    with pytest.raises(rq.InvalidInputError):
        rq.gemm_policy(Q4K, 1024, 1024, 0)
