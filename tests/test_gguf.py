"""GGUF on-disk path (src/gguf.rs): files written here byte by byte after the
format (and the reference's own synthetic test file, gguf.rs:548-666) are
parsed by the library's reader; tensor bytes come back unchanged, errors
carry the reference's messages. The device upload (QuantArena) and the
kernels on uploaded tensors are checked in the GPU part."""
import os
import struct

import numpy as np
import pytest
import torch

from reflex_amd import synth

MAGIC = 0x46554747


def _s(b: bytearray, s: str) -> None:
    e = s.encode()
    b += struct.pack("<Q", len(e)) + e


def _kv(b: bytearray, key: str, ty: int, payload: bytes) -> None:
    _s(b, key)
    b += struct.pack("<I", ty) + payload


def write_gguf(path, meta, tensors, alignment=None, version=3):
    """meta: list of (key, type id, payload bytes); tensors: list of
    (name, dims, ggml type, raw bytes). Returns the data section start."""
    b = bytearray()
    b += struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta) + (alignment is not None))
    for k, t, p in meta:
        _kv(b, k, t, p)
    if alignment is not None:
        _kv(b, "general.alignment", 4, struct.pack("<I", alignment))
    al = alignment or 32
    offs, off = [], 0
    for _, _, _, raw in tensors:
        offs.append(off)
        off += (len(raw) + al - 1) // al * al
    for (name, dims, ty, _), o in zip(tensors, offs):
        _s(b, name)
        b += struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        b += struct.pack("<IQ", ty, o)
    start = (len(b) + al - 1) // al * al
    b += bytes(start - len(b))
    for (_, _, _, raw), o in zip(tensors, offs):
        b += bytes(start + o - len(b)) + bytes(raw)
    with open(path, "wb") as f:
        f.write(b)
    return start


def _str_payload(s):
    e = s.encode()
    return struct.pack("<Q", len(e)) + e


def test_reference_synthetic_file(rqh, tmp_path):
    """gguf.rs:548-666's synthetic file: version 3, two metadata keys, one F32
    tensor of 4 elements at the default 32-byte alignment."""
    p = tmp_path / "ref.gguf"
    write_gguf(p, [("general.architecture", 8, _str_payload("llama")),
                   ("llama.attention.head_count", 4, struct.pack("<I", 32))],
               [("tok.weight", [4], 0, np.array([1, 2, 3, 4], np.float32).tobytes())])
    f = rqh.GgufFile(p)
    assert f.version == 3 and f.tensor_count == 1
    assert f.meta_str("general.architecture") == "llama"
    assert f.meta_u64("llama.attention.head_count") == 32
    info = f.tensor_info(f.find("tok.weight"))
    assert info["shape"] == [4] and info["ggml_type"] == 0
    assert np.frombuffer(f.tensor_bytes("tok.weight").tobytes(), np.float32).tolist() == [1, 2, 3, 4]


def test_metadata_types_and_arrays(rqh, tmp_path):
    p = tmp_path / "meta.gguf"
    nested = struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2) \
        + struct.pack("<IQ", 4, 1) + struct.pack("<I", 3)
    write_gguf(p, [("arr", 9, struct.pack("<IQ", 4, 3) + struct.pack("<III", 1, 2, 3)),
                   ("nested", 9, nested),
                   ("f", 6, struct.pack("<f", 1.5)), ("d", 12, struct.pack("<d", -2.25)),
                   ("b", 7, b"\x01"), ("neg", 5, struct.pack("<i", -3)), ("u64", 10, struct.pack("<Q", 1 << 40)),
                   ("strs", 9, struct.pack("<IQ", 8, 2) + _str_payload("a") + _str_payload("bc"))], [])
    f = rqh.GgufFile(p)
    assert f.meta_array_len("arr") == 3 and f.meta_array_len("nested") == 2 and f.meta_array_len("strs") == 2
    assert f.meta_f64("f") == 1.5 and f.meta_f64("d") == -2.25
    assert f.meta_u64("u64") == 1 << 40
    with pytest.raises(rqh.GgmlError, match="not an unsigned integer"):
        f.meta_u64("neg")
    with pytest.raises(rqh.GgmlError, match="missing"):
        f.meta_str("absent")


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_quantized_tensors_round_trip(rqh, tmp_path, alignment):
    """Q4_K / Q6_K / Q8_0 / F32 tensors at any alignment: every tensor's bytes
    come back unchanged at the offset the format puts them."""
    ts = []
    for i, (ty, n, k) in enumerate([(12, 96, 512), (14, 64, 1024), (8, 40, 256)]):
        ts.append((f"blk.{i}.w", [k, n], ty, synth.weights(ty, n, k, 10 + i).tobytes()))
    ts.append(("norm", [512], 0, np.arange(512, dtype=np.float32).tobytes()))
    ts.append(("experts", [256, 32, 4], 12, synth.weights(12, 32 * 4, 256, 20).tobytes()))
    p = tmp_path / "q.gguf"
    write_gguf(p, [], ts, alignment=alignment)
    f = rqh.GgufFile(p)
    assert f.tensor_count == len(ts)
    for name, dims, ty, raw in ts:
        info = f.tensor_info(f.find(name))
        assert info["shape"] == dims and info["ggml_type"] == ty
        assert f.tensor_bytes(name).tobytes() == raw


def test_errors(rqh, tmp_path):
    good = tmp_path / "g.gguf"
    write_gguf(good, [], [("w", [256, 4], 12, bytes(4 * 144))])
    raw = good.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"\x00" + raw[1:])
    with pytest.raises(rqh.GgmlError, match="not a GGUF file: magic="):
        rqh.GgufFile(bad)
    trunc = tmp_path / "t.gguf"
    trunc.write_bytes(raw[:30])
    with pytest.raises(rqh.GgmlError, match="unexpected end of file"):
        rqh.GgufFile(trunc)
    short = tmp_path / "s.gguf"
    short.write_bytes(raw[:-100])   # header intact, data cut
    f = rqh.GgufFile(short)
    with pytest.raises(rqh.GgmlError, match="exceeds file length"):
        f.tensor_bytes("w")
    unk = tmp_path / "u.gguf"
    write_gguf(unk, [], [("w", [256], 99, bytes(64))])
    with pytest.raises(rqh.GgmlError, match="unknown ggml_type=99"):
        rqh.GgufFile(unk).tensor_bytes("w")
    with pytest.raises(rqh.IoError, match="opening GGUF file"):
        rqh.GgufFile(tmp_path / "missing.gguf")
    with pytest.raises(rqh.GgmlError, match="not found"):
        rqh.GgufFile(good).find("nope")
    meta = tmp_path / "m.gguf"
    write_gguf(meta, [("x", 13, b"")], [])
    with pytest.raises(rqh.GgmlError, match="unsupported GGUF metadata value type 13"):
        rqh.GgufFile(meta)


@pytest.mark.gpu
def test_upload_and_kernels_on_file_tensors(rq, orc, tmp_path):
    """The arena upload (256-byte aligned offsets) and the kernels on the
    uploaded tensors: device dequant equals the oracle's of the file bytes,
    GEMV / GEMM equal the same calls on directly uploaded blocks."""
    shapes = [("q", 12, 256, 1024), ("v", 14, 128, 1024), ("e", 8, 64, 512)]
    ts = [(n, [k, m], ty, synth.weights(ty, m, k, 30 + i).tobytes()) for i, (n, ty, m, k) in enumerate(shapes)]
    p = tmp_path / "w.gguf"
    write_gguf(p, [], ts, alignment=32)
    f = rq.GgufFile(p)
    ws = f.upload([n for n, *_ in ts], device="cuda:0")
    offs = sorted(w.offset for w in ws.values())
    assert all(o % 256 == 0 for o in offs)
    for (name, dims, ty, raw), (_, _, m, k) in zip(ts, shapes):
        w = ws[name]
        assert w.shape == [k, m] and int(w.ty) == ty
        blocks = np.frombuffer(raw, np.uint8).copy()
        deq = rq.dequantize(ty, w.arena[w.offset:w.offset + w.len], m * k, torch.float32).cpu().numpy()
        assert np.array_equal(deq, orc.dequantize(ty, blocks, m * k))
        x = torch.from_numpy(synth.activations(k, 40)).to("cuda:0")
        direct = rq.Weight.from_blocks(ty, blocks, k, m, device="cuda:0")
        assert torch.equal(rq.gemv(x, w), rq.gemv(x, direct))
        xm = torch.from_numpy(synth.activations(8 * k, 41)).to("cuda:0")
        assert torch.equal(rq.gemm(xm, w, 8), rq.gemm(xm, direct, 8))
