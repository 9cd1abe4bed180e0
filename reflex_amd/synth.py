"""Seeded synthetic GGUF weights and activations at the benchmark shapes.

Every tensor comes from its own SplitMix64 stream (counter form: the i-th
draw is mix(seed + (i+1) * 0x9E3779B97F4A7C15)); normals use Box-Muller in
f64, rounded to f32. Seeds: 0x5EED0000 + config_id * 2**16 + layer * 16 + proj.

  Q4_K block: d, dmin = f16(|N(0,1)| * 0.01); 12 scale bytes and 128 qs bytes
              uniform.
  Q6_K block: ql (128 B) and qh (64 B) uniform; 16 int8 scales uniform;
              d = f16(|N(0,1)| * 0.01).
  Q8_0 block: d = f16(|N(0,1)| * 0.01); 32 int8 quants uniform in [-127, 127].
  activations: N(0,1) f32.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

Q4K, Q6K, Q8_0 = 12, 14, 8
BLOCK = {Q4K: (256, 144), Q6K: (256, 210), Q8_0: (32, 34)}


def seed_for(config_id: int, layer: int = 0, proj: int = 0) -> int:
    return 0x5EED0000 + config_id * (1 << 16) + layer * 16 + proj


def splitmix64(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n uint64 draws of the SplitMix64 sequence seeded with seed ^ (stream << 56)."""
    s = np.uint64((seed ^ (stream << 56)) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        z = s + (np.arange(1, n + 1, dtype=np.uint64) * GAMMA)
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_bytes(seed: int, n: int, stream: int) -> np.ndarray:
    return splitmix64(seed, (n + 7) // 8, stream).view(np.uint8)[:n]


def normals(seed: int, n: int, stream: int = 1) -> np.ndarray:
    """N(0,1) via Box-Muller in f64, rounded to f32."""
    m = (n + 1) // 2
    u = splitmix64(seed, 2 * m, stream)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) / 9007199254740992.0  # (0, 1]
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return z[:n].astype(np.float32)


def _f16_scale(seed: int, n: int, stream: int) -> np.ndarray:
    return (np.abs(normals(seed, n, stream).astype(np.float64)) * 0.01).astype(np.float32).astype(np.float16)


def weights(ty: int, n: int, k: int, seed: int) -> np.ndarray:
    """Raw blocks of an [n, k] (out x in) weight, row-major [n][k/QK]."""
    qk, bb = BLOCK[ty]
    nb = n * (k // qk)
    out = np.empty((nb, bb), dtype=np.uint8)
    if ty == Q4K:
        out[:, 0:2] = _f16_scale(seed, nb, 1).view(np.uint8).reshape(nb, 2)
        out[:, 2:4] = _f16_scale(seed, nb, 2).view(np.uint8).reshape(nb, 2)
        out[:, 4:144] = uniform_bytes(seed, nb * 140, 3).reshape(nb, 140)
    elif ty == Q6K:
        out[:, 0:208] = uniform_bytes(seed, nb * 208, 3).reshape(nb, 208)
        out[:, 208:210] = _f16_scale(seed, nb, 1).view(np.uint8).reshape(nb, 2)
    elif ty == Q8_0:
        out[:, 0:2] = _f16_scale(seed, nb, 1).view(np.uint8).reshape(nb, 2)
        u = splitmix64(seed, (nb * 32 + 1) // 2, 3).view(np.uint32)[: nb * 32]
        out[:, 2:34] = ((u % np.uint32(255)).astype(np.int32) - 127).astype(np.int8).view(np.uint8).reshape(nb, 32)
    else:
        raise ValueError(f"no generator for ggml type {ty}")
    return out.reshape(-1)


def activations(n: int, seed: int) -> np.ndarray:
    return normals(seed, n, 7)


# ---------------------------------------------------------------- benchmark shapes

# (name, ggml type, N (out), K (in)) per layer
QWEN3_06B_LAYER = [
    ("q_proj", Q4K, 2048, 1024),
    ("k_proj", Q4K, 1024, 1024),
    ("v_proj", Q6K, 1024, 1024),
    ("o_proj", Q4K, 1024, 2048),
    ("gate_proj", Q4K, 3072, 1024),
    ("up_proj", Q4K, 3072, 1024),
    ("down_proj", Q4K, 1024, 3072),
]
QWEN3_06B_LAYERS = 28

QWEN3_8B_LAYER = [
    ("q_proj", Q4K, 4096, 4096),
    ("k_proj", Q4K, 1024, 4096),
    ("v_proj", Q6K, 1024, 4096),
    ("o_proj", Q4K, 4096, 4096),
    ("gate_proj", Q4K, 14336, 4096),
    ("up_proj", Q4K, 14336, 4096),
    ("down_proj", Q6K, 4096, 14336),
]
LM_HEAD = ("lm_head", Q6K, 151936, 1024)

MOE = dict(experts=128, hidden=2048, ffn=768, top_k=8, tokens=512, ty=Q4K)


def weight_bytes(ty: int, n: int, k: int) -> int:
    qk, bb = BLOCK[ty]
    return n * (k // qk) * bb
