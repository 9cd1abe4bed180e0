"""Host-side mirror of the reference's quantized-matmul call surface.

Names, argument meaning and errors follow the reference's Rust ``Model``
methods and types for this path (src/model/kernels.rs, src/model/loading.rs,
src/model/dense.rs, src/moe.rs); every call goes through librfxq's C ABI
(include/rfxq.h). Device memory and streams come from PyTorch: tensors are
``torch.cuda`` tensors, launches go on ``torch.cuda.current_stream()``.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field

import numpy as np
import torch

from . import RfxqGemmPolicy, RfxqGemvItem, RfxqOptions, RfxqWeight, lib

__all__ = [
    "ReflexError", "GgmlError", "GpuError", "OutOfMemoryError", "InvalidInputError", "IoError", "GgufFile",
    "GgmlType", "ggml_type_block_dims", "Weight", "QuantArena",
    "dequantize", "gemv", "gemv_to", "gemv_q4k", "gemv_q6k", "gemv_q8_0", "gemv_batch", "GemvPlan",
    "gemv_gather",
    "gemm", "gemm_no_alloc", "gemm_workspace_size", "gemm_batch", "GemmPlan", "quantize_q8_1", "mmq_block_dots",
    "route_top_k", "route_top_k_with_norm", "quant_expert_weight", "expert_gemv", "expert_gemm",
    "moe_gather", "moe_scatter_add", "silu_and_mul", "moe_ffn_grouped", "init",
    "moe_route_device", "moe_ffn_grouped_device",
    "act_q8_1_size", "quantize_act_q8_1", "rmsnorm_q8_1", "silu_and_mul_q8_1", "gemm_q8_1", "gemm_q8_1_batch",
    "gemm_gate_up_silu_q8_1",
    "get_options", "set_options", "options", "gemm_policy", "PATH_GEMV_ROWS", "PATH_MMQ_INT8", "PATH_MMQ_F16",
]


# ------------------------------------------------------------------ errors (src/error.rs)

class ReflexError(Exception):
    """``ReflexError``: ``code`` is the C ABI code (reference ReflexErrorCode values)."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class GgmlError(ReflexError):        # ReflexError::Gguf (unknown / unsupported ggml type)
    pass


class GpuError(ReflexError):         # ReflexError::Cuda
    pass


class OutOfMemoryError(ReflexError):  # ReflexError::OutOfMemory
    pass


class InvalidInputError(ReflexError):  # ReflexError::InvalidInput
    pass


class IoError(ReflexError):           # ReflexError::Io
    pass


_ERR = {1: GgmlError, 3: GpuError, 5: OutOfMemoryError, 10: IoError, 11: InvalidInputError}


def _check(rc: int) -> None:
    if rc != 0:
        msg = lib().rfxq_last_error()
        cls = _ERR.get(rc, ReflexError)
        raise cls(rc, msg.decode() if msg else f"rfxq error {rc}")


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        return t.data_ptr()
    return int(t)


def init(device: int = 0) -> None:
    """Load the embedded gfx950 code object on ``device`` (otherwise lazy)."""
    _check(lib().rfxq_init(device))


# ------------------------------------------------------------------ types (src/gguf.rs)

class GgmlType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q8_1 = 9
    Q4K = 12
    Q6K = 14


def ggml_type_block_dims(ty: int) -> tuple[int, int]:
    """(elements per block, bytes per block): src/gguf.rs:366-400."""
    qk, bb = ctypes.c_uint32(), ctypes.c_uint32()
    _check(lib().rfxq_block_dims(int(ty), ctypes.byref(qk), ctypes.byref(bb)))
    return qk.value, bb.value


# ------------------------------------------------------------------ weights (src/model/loading.rs)

class QuantArena:
    """Raw GGUF blocks of many tensors in one device buffer, 256-byte aligned
    offsets (``QuantArena``, src/model/loading.rs:266-317)."""

    ALIGN = 256

    def __init__(self, sizes: list[int], device: str | torch.device = "cuda"):
        self.offsets = []
        off = 0
        for s in sizes:
            self.offsets.append(off)
            off += (s + self.ALIGN - 1) // self.ALIGN * self.ALIGN
        self.buf = torch.empty(max(off, 1), dtype=torch.uint8, device=device)

    def upload(self, i: int, data: np.ndarray) -> None:
        o = self.offsets[i]
        self.buf[o:o + data.size].copy_(torch.from_numpy(np.ascontiguousarray(data).view(np.uint8)))


@dataclass
class Weight:
    """``Weight { data: WeightData::Quant { ty, arena, offset, len }, shape }``.

    ``shape`` is the reference's ``[in_features, out_features]`` (or
    ``[in, out, expert_count]`` for a stacked expert tensor); ``arena`` a uint8
    device tensor holding the raw blocks at ``offset``.
    """

    ty: GgmlType
    arena: torch.Tensor
    shape: list[int]
    offset: int = 0
    len: int | None = None
    _c: RfxqWeight = field(default=None, repr=False)

    def __post_init__(self):
        if self.len is None:
            self.len = self.arena.numel() - self.offset
        self._c = RfxqWeight(int(self.ty), int(self.shape[0]), int(self.shape[1]),
                             int(self.shape[2]) if len(self.shape) > 2 else 0,
                             self.arena.data_ptr() + self.offset, int(self.len))

    @classmethod
    def from_blocks(cls, ty: int, blocks: np.ndarray, in_features: int, out_features: int,
                    expert_count: int = 0, device="cuda") -> "Weight":
        t = torch.from_numpy(np.ascontiguousarray(blocks).view(np.uint8)).to(device)
        shape = [in_features, out_features] + ([expert_count] if expert_count else [])
        return cls(GgmlType(ty), t, shape)

    def quant_ptr(self) -> int:
        return self.arena.data_ptr() + self.offset

    @property
    def in_features(self) -> int:
        return int(self.shape[0])

    @property
    def out_features(self) -> int:
        return int(self.shape[1])

    def cref(self) -> ctypes.POINTER(RfxqWeight):
        return ctypes.byref(self._c)


def _dev(t: torch.Tensor):
    return torch.cuda.device(t.device)


# ------------------------------------------------------------------ options

PATH_GEMV_ROWS, PATH_MMQ_INT8, PATH_MMQ_F16 = 0, 1, 2
_OPTION_FIELDS = [f for f, _ in RfxqOptions._fields_]


def get_options() -> dict:
    """The library's prefill switches (the environment's ``REFLEX_QUANT_MMA*``,
    ``REFLEX_MMQ_F16``, ``REFLEX_QUANT_FUSED_MAX_ROWS``, read once) as a dict;
    raises InvalidInputError with the reference's message on a bad value."""
    o = RfxqOptions()
    _check(lib().rfxq_get_options(ctypes.byref(o)))
    return {f: getattr(o, f) for f in _OPTION_FIELDS}


def set_options(**changes) -> dict:
    """Change some options (``QuantMmaKernels::set_enabled`` / ``set_splits``,
    kernels.rs:804-830); returns the previous ones, for ``set_options(**prev)``."""
    prev = get_options()
    unknown = set(changes) - set(_OPTION_FIELDS)
    if unknown:
        raise TypeError(f"unknown options {sorted(unknown)}")
    new = dict(prev, **changes)
    _check(lib().rfxq_set_options(ctypes.byref(RfxqOptions(**new))))
    return prev


class options:
    """Context manager: ``with options(mmq_f16=0): ...`` restores the previous options."""

    def __init__(self, **changes):
        self._changes = changes

    def __enter__(self):
        self._prev = set_options(**self._changes)
        return self

    def __exit__(self, *exc):
        set_options(**self._prev)


def gemm_policy(ty: int, in_features: int, out_features: int, rows: int, compute_units: int = 256) -> dict:
    """How ``gemm`` runs a GEMM of this shape on a device with ``compute_units`` CUs."""
    p = RfxqGemmPolicy()
    _check(lib().rfxq_gemm_policy_for(int(ty), in_features, out_features, rows, compute_units, ctypes.byref(p)))
    return {f: getattr(p, f) for f, _ in RfxqGemmPolicy._fields_}


# ------------------------------------------------------------------ dequant

def dequantize(ty: int, blocks: torch.Tensor, element_count: int, dtype=torch.float32) -> torch.Tensor:
    """Device dequantization of raw blocks, truncated to ``element_count``
    (the device twin of src/dequant.rs:53 ``dequantize``)."""
    qk, bb = ggml_type_block_dims(ty)
    nb = blocks.numel() // bb
    out = torch.empty(nb * qk, dtype=dtype, device=blocks.device)
    with _dev(blocks):
        _check(lib().rfxq_dequantize(int(ty), blocks.data_ptr(), nb, out.data_ptr(),
                                     1 if dtype == torch.float16 else 0, _stream()))
    return out[:element_count]


# ------------------------------------------------------------------ GEMV

def gemv_to(x: torch.Tensor, w: Weight, y: torch.Tensor) -> None:
    """``Model::gemv_to`` (kernels.rs:1463): y[out] = W . x into ``y``."""
    with _dev(x):
        _check(lib().rfxq_gemv_to(x.data_ptr(), x.numel(), w.cref(), y.data_ptr(), _stream()))


def gemv(x: torch.Tensor, w: Weight) -> torch.Tensor:
    """``Model::gemv`` (kernels.rs:1826)."""
    y = torch.empty(w.out_features, dtype=torch.float32, device=x.device)
    gemv_to(x, w, y)
    return y


def _gemv_rows(x: torch.Tensor, w: Weight, rows: int) -> torch.Tensor:
    y = torch.empty(rows * w.out_features, dtype=torch.float32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_gemv_rows(x.data_ptr(), x.numel(), w.cref(), rows, y.data_ptr(), _stream()))
    return y


def gemv_q4k(x: torch.Tensor, w: Weight, rows: int) -> torch.Tensor:
    """``Model::gemv_q4k`` (kernels.rs:2110)."""
    return _gemv_rows(x, w, rows)


def gemv_q6k(x: torch.Tensor, w: Weight) -> torch.Tensor:
    """``Model::gemv_q6k`` (kernels.rs:1972)."""
    return _gemv_rows(x, w, 1)


def gemv_q8_0(x: torch.Tensor, w: Weight, rows: int) -> torch.Tensor:
    """``Model::gemv_q8_0`` (kernels.rs:1874)."""
    return _gemv_rows(x, w, rows)


def gemv_gather(x: torch.Tensor, w: Weight, row_indices) -> torch.Tensor:
    """``Model::gemv_gather`` (kernels.rs:2816-2851): the logits of the named
    rows only, as a device tensor (the reference returns host floats)."""
    idx = (ctypes.c_uint32 * len(row_indices))(*[int(r) for r in row_indices])
    y = torch.empty(max(len(row_indices), 1), dtype=torch.float32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_gemv_gather(x.data_ptr(), x.numel(), w.cref(), idx, len(row_indices), y.data_ptr(),
                                      _stream()))
    return y[:len(row_indices)]


def _items(items):
    arr = (RfxqGemvItem * len(items))()
    keep = []
    for i, (x, w, y) in enumerate(items):
        arr[i].x = x.data_ptr()
        arr[i].w = ctypes.pointer(w._c)
        arr[i].y = y.data_ptr()
        keep.append(w)
    return arr, keep


def gemv_batch(items: list[tuple[torch.Tensor, Weight, torch.Tensor]]) -> None:
    """Fused independent GEMVs (``gemv_qkv_to`` / ``gemv_gate_up_to``, kernels.rs:1761-1823)."""
    if not items:
        return
    arr, _keep = _items(items)
    with _dev(items[0][0]):
        _check(lib().rfxq_gemv_batch(arr, len(items), _stream()))


class GemvPlan:
    """A fused GEMV launch whose descriptor table is uploaded once."""

    def __init__(self, items: list[tuple[torch.Tensor, Weight, torch.Tensor]]):
        arr, self._keep = _items(items)
        self._tensors = items
        h = ctypes.c_void_p()
        dev = items[0][0].device.index or 0
        self._lib = lib()  # kept so that __del__ works during interpreter shutdown
        _check(self._lib.rfxq_gemv_plan_create(arr, len(items), dev, ctypes.byref(h)))
        self._h = h

    def run(self) -> None:
        _check(lib().rfxq_gemv_plan_run(self._h, _stream()))

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.rfxq_gemv_plan_destroy(self._h)
            self._h = None


# ------------------------------------------------------------------ GEMM (int8 MMQ)

def quantize_q8_1(x: torch.Tensor, rows: int, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-32 int8 activation quantization: (xq int8 [rows,k], xds int32 [rows,k/32] = d | s<<16)."""
    xq = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    xds = torch.empty((rows, k // 32), dtype=torch.int32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_quantize_q8_1(x.data_ptr(), rows, k, xq.data_ptr(), xds.data_ptr(), _stream()))
    return xq, xds


def gemm_workspace_size(w: Weight, rows: int) -> int:
    return int(lib().rfxq_gemm_workspace_size(w.cref(), rows))


def gemm(x: torch.Tensor, w: Weight, rows: int, workspace: torch.Tensor | None = None,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """``Model::gemm`` (kernels.rs:2197): y[rows, out] = x[rows, in] @ W^T."""
    y = out if out is not None else torch.empty(rows * w.out_features, dtype=torch.float32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_gemm(x.data_ptr(), x.numel(), w.cref(), rows, y.data_ptr(), _ptr(workspace),
                               workspace.numel() if workspace is not None else 0, _stream()))
    return y


def gemm_no_alloc(x: torch.Tensor, w: Weight, rows: int, out: torch.Tensor) -> torch.Tensor:
    """``gemm`` without device allocation (the library's fixed per-GPU scratch;
    ``init`` the device first). Calls that overlap on one GPU race."""
    with _dev(x):
        _check(lib().rfxq_gemm_no_alloc(x.data_ptr(), x.numel(), w.cref(), rows, out.data_ptr(), _stream()))
    return out


def gemm_batch(items: list[tuple[torch.Tensor, Weight, torch.Tensor]], rows: int) -> None:
    """Grouped prefill GEMMs of one row count (the q/k/v and gate/up ``Model::gemm``
    calls on one input, dense.rs:1345-1347, 1476-1477): one quantization per
    distinct x, one MMQ launch per weight type. Items are (x, w, y)."""
    if not items:
        return
    arr, _keep = _items(items)
    with _dev(items[0][0]):
        _check(lib().rfxq_gemm_batch(arr, len(items), rows, _stream()))


# ------------------------------------------------------------------ fused activation producers

def act_q8_1_size(rows: int, k: int) -> int:
    """Bytes of a quantized activation buffer (every MMQ layout) for [rows][k]."""
    return int(lib().rfxq_act_q8_1_size(rows, k))


def _act(rows: int, k: int, device) -> torch.Tensor:
    n = act_q8_1_size(rows, k)
    if n == 0:
        raise InvalidInputError(11, f"activation buffer: rows={rows} k={k} (k must be a multiple of 256)")
    return torch.empty(n, dtype=torch.uint8, device=device)


def quantize_act_q8_1(x: torch.Tensor, rows: int, k: int) -> torch.Tensor:
    """A plain f32 activation [rows][k] quantized into an activation buffer."""
    act = _act(rows, k, x.device)
    with _dev(x):
        _check(lib().rfxq_quantize_act_q8_1(x.data_ptr(), rows, k, act.data_ptr(), _stream()))
    return act


def rmsnorm_q8_1(x: torch.Tensor, weight: torch.Tensor, rows: int, k: int, eps: float, want_y: bool = False):
    """``Model::rmsnorm`` (rmsnorm.cu) fused with quantization: (act, y or None)."""
    act = _act(rows, k, x.device)
    y = torch.empty(rows * k, dtype=torch.float32, device=x.device) if want_y else None
    with _dev(x):
        _check(lib().rfxq_rmsnorm_q8_1(x.data_ptr(), weight.data_ptr(), rows, k, eps, act.data_ptr(),
                                       y.data_ptr() if y is not None else None, _stream()))
    return act, y


def silu_and_mul_q8_1(gate: torch.Tensor, up: torch.Tensor, rows: int, k: int, want_y: bool = False):
    """``Model::silu_and_mul`` (silu_and_mul.cu) fused with quantization: (act, y or None)."""
    act = _act(rows, k, gate.device)
    y = torch.empty(rows * k, dtype=torch.float32, device=gate.device) if want_y else None
    with _dev(gate):
        _check(lib().rfxq_silu_and_mul_q8_1(gate.data_ptr(), up.data_ptr(), rows, k, act.data_ptr(),
                                            y.data_ptr() if y is not None else None, _stream()))
    return act, y


def gemm_q8_1(act: torch.Tensor, w: Weight, rows: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """``Model::gemm`` from a quantized activation buffer."""
    y = out if out is not None else torch.empty(rows * w.out_features, dtype=torch.float32, device=act.device)
    with _dev(act):
        _check(lib().rfxq_gemm_q8_1(act.data_ptr(), rows, w.cref(), y.data_ptr(), None, 0, _stream()))
    return y


def gemm_gate_up_silu_q8_1(act: torch.Tensor, rows: int, gate: Weight, up: Weight):
    """gemm(gate) + gemm(up) + silu_and_mul fused (dense.rs:1476-1478):
    (act_out for the down GEMM, y = silu(gate) * up [rows][ffn] f32)."""
    ffn = gate.out_features
    act_out = _act(rows, ffn, act.device)
    y = torch.empty(rows * ffn, dtype=torch.float32, device=act.device)
    with _dev(act):
        _check(lib().rfxq_gemm_gate_up_silu_q8_1(act.data_ptr(), rows, gate.cref(), up.cref(), act_out.data_ptr(),
                                                 y.data_ptr(), None, 0, _stream()))
    return act_out, y


def gemm_q8_1_batch(items: list[tuple[torch.Tensor, Weight, torch.Tensor]], rows: int) -> None:
    """Grouped GEMMs from activation buffers: items are (act, w, y)."""
    if not items:
        return
    arr, _keep = _items(items)
    with _dev(items[0][0]):
        _check(lib().rfxq_gemm_q8_1_batch(arr, len(items), rows, _stream()))


class GemmPlan:
    """gemm_batch with its tables and activation workspace built once. With
    ``quantized=True`` the items' first members are activation buffers
    (act_q8_1_size layouts, written by a producer) and a run launches only
    the GEMM kernels."""

    def __init__(self, items: list[tuple[torch.Tensor, Weight, torch.Tensor]], rows: int, quantized: bool = False):
        arr, self._keep = _items(items)
        self._tensors = items
        h = ctypes.c_void_p()
        dev = items[0][0].device.index or 0
        self._lib = lib()  # kept so that __del__ works during interpreter shutdown
        create = self._lib.rfxq_gemm_q8_1_plan_create if quantized else self._lib.rfxq_gemm_plan_create
        _check(create(ctypes.cast(arr, ctypes.c_void_p) if quantized else arr, len(items), rows, dev,
                      ctypes.byref(h)))
        self._h = h

    def run(self) -> None:
        _check(lib().rfxq_gemm_plan_run(self._h, _stream()))

    def __del__(self):
        if getattr(self, "_h", None):
            self._lib.rfxq_gemm_plan_destroy(self._h)
            self._h = None


def mmq_block_dots(xq: torch.Tensor, xds: torch.Tensor, rows: int, w: Weight) -> torch.Tensor:
    """The MMQ kernel's int32 per-32 dots: [rows, out, in/32] (test hook)."""
    dots = torch.empty((rows, w.out_features, w.in_features // 32), dtype=torch.int32, device=xq.device)
    with _dev(xq):
        _check(lib().rfxq_mmq_block_dots(xq.data_ptr(), xds.data_ptr(), rows, w.cref(), dots.data_ptr(),
                                         _stream()))
    return dots


# ------------------------------------------------------------------ MoE (src/moe.rs, dense.rs)

def route_top_k_with_norm(logits, k: int, normalize: bool) -> list[tuple[int, float]]:
    """src/moe.rs:47-98 (host)."""
    lg = np.ascontiguousarray(np.asarray(logits, dtype=np.float32))
    idx = np.zeros(max(k, 1), dtype=np.uint32)
    wt = np.zeros(max(k, 1), dtype=np.float32)
    _check(lib().rfxq_route_top_k(lg.ctypes.data if lg.size else None, lg.size, k, int(normalize),
                                  idx.ctypes.data, wt.ctypes.data))
    return [(int(i), float(v)) for i, v in zip(idx[:k], wt[:k])]


def route_top_k(logits, k: int) -> list[tuple[int, float]]:
    """src/moe.rs:35 (renormalised)."""
    return route_top_k_with_norm(logits, k, True)


def quant_expert_weight(w: Weight, expert_idx: int) -> Weight:
    """``Model::quant_expert_weight`` (kernels.rs:2656-2694)."""
    out = RfxqWeight()
    _check(lib().rfxq_quant_expert_weight(w.cref(), expert_idx, ctypes.byref(out)))
    return Weight(w.ty, w.arena, [w.shape[0], w.shape[1]], offset=out.data - w.arena.data_ptr(), len=out.len)


def expert_gemv(x: torch.Tensor, w: Weight, expert_idx: int) -> torch.Tensor:
    """``Model::expert_gemv`` (dense.rs:1086)."""
    y = torch.empty(w.out_features, dtype=torch.float32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_expert_gemv(x.data_ptr(), x.numel(), w.cref(), expert_idx, y.data_ptr(), _stream()))
    return y


def expert_gemm(x: torch.Tensor, w: Weight, expert_idx: int, rows: int) -> torch.Tensor:
    """``Model::expert_gemm`` (dense.rs:1103)."""
    y = torch.empty(rows * w.out_features, dtype=torch.float32, device=x.device)
    with _dev(x):
        _check(lib().rfxq_expert_gemm(x.data_ptr(), x.numel(), w.cref(), expert_idx, rows, y.data_ptr(), None, 0,
                                      _stream()))
    return y


def moe_gather(src: torch.Tensor, perm_row: torch.Tensor, hidden: int) -> torch.Tensor:
    """``Model::moe_gather`` (kernels.rs:2722)."""
    n = perm_row.numel()
    dst = torch.empty(n * hidden, dtype=torch.float32, device=src.device)
    with _dev(src):
        _check(lib().rfxq_moe_gather(src.data_ptr(), perm_row.data_ptr(), dst.data_ptr(), n, hidden, _stream()))
    return dst


def moe_scatter_add(src: torch.Tensor, dest_row: torch.Tensor, weight: torch.Tensor, dst: torch.Tensor,
                    hidden: int) -> None:
    """``Model::moe_scatter_add`` (kernels.rs:2770)."""
    with _dev(src):
        _check(lib().rfxq_moe_scatter_add(src.data_ptr(), dest_row.data_ptr(), weight.data_ptr(), dst.data_ptr(),
                                          dest_row.numel(), hidden, _stream()))


def silu_and_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    out = torch.empty_like(gate)
    with _dev(gate):
        _check(lib().rfxq_silu_and_mul(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(), _stream()))
    return out


def moe_ffn_grouped(x: torch.Tensor, rows: int, hidden: int, router_logits: np.ndarray, expert_count: int,
                    top_k: int, normalize: bool, weight_scale: float, gate: Weight, up: Weight, down: Weight,
                    out: torch.Tensor) -> None:
    """``Model::moe_ffn_grouped`` (dense.rs:1509-1559): out[rows, hidden] is overwritten."""
    lg = np.ascontiguousarray(router_logits, dtype=np.float32)
    with _dev(x):
        _check(lib().rfxq_moe_ffn_grouped(x.data_ptr(), rows, hidden, lg.ctypes.data, expert_count, top_k,
                                          int(normalize), float(weight_scale), gate.cref(), up.cref(), down.cref(),
                                          out.data_ptr(), _stream()))


def moe_route_device(logits: torch.Tensor, tokens: int, expert_count: int, top_k: int, normalize: bool,
                     weight_scale: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """``route_top_k_with_norm`` (moe.rs:47-98) on device logits: (expert ids, weights), [tokens, top_k]."""
    idx = torch.empty((tokens, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((tokens, top_k), dtype=torch.float32, device=logits.device)
    with _dev(logits):
        _check(lib().rfxq_moe_route_device(logits.data_ptr(), tokens, expert_count, top_k, int(normalize),
                                           float(weight_scale), idx.data_ptr(), w.data_ptr(), _stream()))
    return idx, w


def moe_ffn_grouped_device(x: torch.Tensor, rows: int, hidden: int, router_logits: torch.Tensor, expert_count: int,
                           top_k: int, normalize: bool, weight_scale: float, gate: Weight, up: Weight, down: Weight,
                           out: torch.Tensor) -> None:
    """``moe_ffn_grouped`` with routing on the device (logits stay in device memory)."""
    with _dev(x):
        _check(lib().rfxq_moe_ffn_grouped_device(x.data_ptr(), rows, hidden, router_logits.data_ptr(), expert_count,
                                                 top_k, int(normalize), float(weight_scale), gate.cref(), up.cref(),
                                                 down.cref(), out.data_ptr(), _stream()))


# ------------------------------------------------------------------ GGUF files

class GgufFile:
    """``GgufFile`` (src/gguf.rs:183-334): a memory-mapped, parsed GGUF file."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        self._lib = lib()
        _check(self._lib.rfxq_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rfxq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return int(lib().rfxq_gguf_version(self._h))

    @property
    def tensor_count(self) -> int:
        return int(lib().rfxq_gguf_tensor_count(self._h))

    def find(self, name: str) -> int:
        i = ctypes.c_uint64()
        _check(lib().rfxq_gguf_find_tensor(self._h, name.encode(), ctypes.byref(i)))
        return i.value

    def tensor_info(self, index: int) -> dict:
        name, nd, ty, off = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        _check(lib().rfxq_gguf_tensor_info(self._h, index, ctypes.byref(name), ctypes.byref(nd), dims,
                                           ctypes.byref(ty), ctypes.byref(off)))
        return {"name": name.value.decode(), "shape": list(dims[:nd.value]), "ggml_type": ty.value,
                "offset": off.value}

    def tensor_bytes(self, name_or_index) -> np.ndarray:
        """The tensor's raw bytes (a copy out of the mapping)."""
        i = self.find(name_or_index) if isinstance(name_or_index, str) else int(name_or_index)
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(lib().rfxq_gguf_tensor_data(self._h, i, ctypes.byref(p), ctypes.byref(n)))
        return np.frombuffer(ctypes.string_at(p.value, n.value), dtype=np.uint8).copy()

    def meta_u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        _check(lib().rfxq_gguf_meta_u64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_f64(self, key: str) -> float:
        v = ctypes.c_double()
        _check(lib().rfxq_gguf_meta_f64(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str:
        v = ctypes.c_char_p()
        _check(lib().rfxq_gguf_meta_str(self._h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def meta_array_len(self, key: str) -> int:
        v = ctypes.c_uint64()
        _check(lib().rfxq_gguf_meta_array_len(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def upload(self, names: list[str], device="cuda") -> dict:
        """QuantArena (loading.rs:266-317): the named tensors in one device
        allocation at 256-byte aligned offsets; returns name -> Weight."""
        idx = (ctypes.c_uint64 * len(names))(*[self.find(n) for n in names])
        size = int(lib().rfxq_gguf_arena_size(self._h, idx, len(names)))
        if size == 0 and names:
            raise GgmlError(1, "gguf upload: a tensor's byte range is invalid")
        arena = torch.empty(max(size, 256), dtype=torch.uint8, device=device)
        ws = (RfxqWeight * max(len(names), 1))()
        with _dev(arena):
            _check(lib().rfxq_gguf_upload(self._h, idx, len(names), arena.data_ptr(), arena.numel(), ws, _stream()))
        torch.cuda.synchronize(arena.device)  # the copies read the mapping
        out = {}
        for j, n in enumerate(names):
            w = ws[j]
            shape = [w.in_features, w.out_features] + ([w.expert_count] if w.expert_count else [])
            ty = GgmlType(w.ggml_type) if w.ggml_type in GgmlType._value2member_map_ else w.ggml_type
            out[n] = Weight(ty, arena, shape,
                            offset=w.data - arena.data_ptr(), len=w.len)
        return out
